/*
 * TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).
 *
 * Independent float64 restatement of multi-scale deformable attention as
 * explicit loops over the closed form, used to pin oracle/msda_torch.py:
 *
 *   out[b,q,m,c] = sum_{l,p} attn[b,q,m,l,p] * bilinear(value_l[b,:,:,m,c], x, y)
 *   x = loc[...,0] * W_l - 0.5,  y = loc[...,1] * H_l - 0.5
 *
 * with corners outside [0,W-1]x[0,H-1] read as zero (grid_sample zero padding,
 * the reference path /root/reference/mu_space/ops/multi_scale_deformable_attn.py:42-48;
 * same coordinate as the reference kernel, ms_deform_attn_musa_kernel.muh:286-287).
 * Gradients are the analytic derivatives of that closed form
 * (ms_deform_attn_musa_kernel.muh:93-166): for top gradient g and
 * tg = g * attn,
 *   grad_value[corner] += w_corner * tg
 *   grad_attn          += g * bilinear
 *   grad_loc_x         += W * tg * d bilinear / dx
 *   grad_loc_y         += H * tg * d bilinear / dy
 * grad_value is accumulated into (zero it first); grad_loc and grad_attn are
 * overwritten. Layouts are the operator's (value [bs,nv,M,C],
 * loc [bs,nq,M,L,P,2], attn [bs,nq,M,L,P], out [bs,nq,M*C]).
 */
#include <math.h>
#include <stdint.h>

typedef struct {
  int64_t x0, y0;
  double wx1, wy1;
  int ok[4]; /* (y0,x0) (y0,x1) (y1,x0) (y1,x1) inside the level */
} tap_t;

static tap_t make_tap(double lx, double ly, int64_t h, int64_t w) {
  tap_t t;
  const double x = lx * (double)w - 0.5, y = ly * (double)h - 0.5;
  const double fx = floor(x), fy = floor(y);
  t.x0 = (int64_t)fx;
  t.y0 = (int64_t)fy;
  t.wx1 = x - fx;
  t.wy1 = y - fy;
  const int x0in = t.x0 >= 0 && t.x0 < w, x1in = t.x0 + 1 >= 0 && t.x0 + 1 < w;
  const int y0in = t.y0 >= 0 && t.y0 < h, y1in = t.y0 + 1 >= 0 && t.y0 + 1 < h;
  t.ok[0] = y0in && x0in;
  t.ok[1] = y0in && x1in;
  t.ok[2] = y1in && x0in;
  t.ok[3] = y1in && x1in;
  return t;
}

static int64_t corner_cell(const tap_t *t, int corner, int64_t start, int64_t w) {
  const int64_t dy = corner >> 1, dx = corner & 1;
  return start + (t->y0 + dy) * w + (t->x0 + dx);
}

void msda_direct_forward(const double *value, const int64_t *shapes, const int64_t *starts,
                         const double *loc, const double *attn, double *out, int64_t bs,
                         int64_t nv, int64_t heads, int64_t channels, int64_t levels,
                         int64_t nq, int64_t points) {
  for (int64_t b = 0; b < bs; ++b)
    for (int64_t q = 0; q < nq; ++q)
      for (int64_t m = 0; m < heads; ++m) {
        const int64_t si = (b * nq + q) * heads + m;
        double *o = out + si * channels;
        for (int64_t c = 0; c < channels; ++c) o[c] = 0.0;
        for (int64_t l = 0; l < levels; ++l) {
          const int64_t h = shapes[2 * l], w = shapes[2 * l + 1], start = starts[l];
          for (int64_t p = 0; p < points; ++p) {
            const int64_t s = (si * levels + l) * points + p;
            const tap_t t = make_tap(loc[2 * s], loc[2 * s + 1], h, w);
            const double cw[4] = {(1 - t.wy1) * (1 - t.wx1), (1 - t.wy1) * t.wx1,
                                  t.wy1 * (1 - t.wx1), t.wy1 * t.wx1};
            for (int k = 0; k < 4; ++k) {
              if (!t.ok[k]) continue;
              const double *v =
                  value + ((b * nv + corner_cell(&t, k, start, w)) * heads + m) * channels;
              for (int64_t c = 0; c < channels; ++c) o[c] += attn[s] * cw[k] * v[c];
            }
          }
        }
      }
}

void msda_direct_backward(const double *value, const int64_t *shapes, const int64_t *starts,
                          const double *loc, const double *attn, const double *grad_out,
                          double *grad_value, double *grad_loc, double *grad_attn, int64_t bs,
                          int64_t nv, int64_t heads, int64_t channels, int64_t levels,
                          int64_t nq, int64_t points) {
  for (int64_t b = 0; b < bs; ++b)
    for (int64_t q = 0; q < nq; ++q)
      for (int64_t m = 0; m < heads; ++m) {
        const int64_t si = (b * nq + q) * heads + m;
        const double *g = grad_out + si * channels;
        for (int64_t l = 0; l < levels; ++l) {
          const int64_t h = shapes[2 * l], w = shapes[2 * l + 1], start = starts[l];
          for (int64_t p = 0; p < points; ++p) {
            const int64_t s = (si * levels + l) * points + p;
            const tap_t t = make_tap(loc[2 * s], loc[2 * s + 1], h, w);
            const double wx0 = 1 - t.wx1, wy0 = 1 - t.wy1;
            const double cw[4] = {wy0 * wx0, wy0 * t.wx1, t.wy1 * wx0, t.wy1 * t.wx1};
            /* d cw / dx and d cw / dy */
            const double dx[4] = {-wy0, wy0, -t.wy1, t.wy1};
            const double dy[4] = {-wx0, -t.wx1, wx0, t.wx1};
            double ga = 0.0, gx = 0.0, gy = 0.0;
            for (int k = 0; k < 4; ++k) {
              if (!t.ok[k]) continue;
              const int64_t row = ((b * nv + corner_cell(&t, k, start, w)) * heads + m) * channels;
              for (int64_t c = 0; c < channels; ++c) {
                const double tg = g[c] * attn[s];
                ga += g[c] * cw[k] * value[row + c];
                gx += tg * dx[k] * value[row + c];
                gy += tg * dy[k] * value[row + c];
                grad_value[row + c] += cw[k] * tg;
              }
            }
            grad_attn[s] = ga;
            grad_loc[2 * s] = gx * (double)w;
            grad_loc[2 * s + 1] = gy * (double)h;
          }
        }
      }
}
