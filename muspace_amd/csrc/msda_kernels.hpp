// MSDA forward and backward kernels for MI355X (gfx950, wave64).
//
// Work unit = one (batch b, query q, head m) triple; its output row is C
// channels. Units are enumerated head-major, u = (b*M + m)*nq + q, and blocks
// are remapped so that each XCD owns a contiguous range of units: the value
// rows a block gathers from then belong to one (b, m) slab (at the BEVFormer
// SCA shape 30825 cells x 128 B = 3.9 MB, one XCD's L2).
//
// Fast kernels ("row" kernels, C = 16, 32 or 64): a lane holds 16 bytes of
// channels (CPL = 4 fp32 or 8 fp16/bf16 channels), KQ = C/CPL lanes hold one
// corner row, and the NG = 64/KQ lane groups of a wavefront work on NG
// different samples at once. One 16-byte load instruction therefore gathers
// NG full corner rows (8 rows of 128 B for fp32 C=32). GU groups share a unit;
// group gi takes the unit's samples gi, gi+GU, gi+2GU, ...
//
// Generic kernels: any C, one thread per output element (forward) or per
// sample (backward); they exist for shape coverage, not speed.
//
// Reference semantics: ms_deformable_im2col_gpu_kernel* and
// ms_deformable_col2im_gpu_kernel_warp_broadcast_multi_warp_channels32
// (/root/reference/csrc/ms_deformable_attn/ms_deform_attn_musa_kernel.muh:243-417,625-733),
// with the sampling arithmetic of the PyTorch path (see msda_device.hpp).
#pragma once

#include "msda_device.hpp"

namespace msda {

constexpr int kBlock = 256;  // 4 wavefronts

// Launch geometry of the row kernels, computed on the host.
struct RowPlan {
  int gu_log2;  // log2(groups per unit)
  int iters;    // wave iterations per wavefront
};

template <typename VT>
struct RowTraits {
  static constexpr int kCpl = 16 / sizeof(VT);
};

// Decoded unit: flat sampling index si = (b*nq + q)*M + m and its batch/head.
struct Unit {
  int b, m, si;
};

__device__ __forceinline__ Unit decode_unit(int u, const Shape &s) {
  const int q = u % s.queries;
  const int t = u / s.queries;
  Unit r;
  r.m = t % s.heads;
  r.b = t / s.heads;
  r.si = (r.b * s.queries + q) * s.heads + r.m;
  return r;
}

// ------------------------------------------------------------- forward ---

template <typename VT, typename GT, int C, int NS>
__global__ void __launch_bounds__(kBlock)
    msda_forward_rows(const VT *__restrict__ value, const int64_t *__restrict__ shapes,
                      const int64_t *__restrict__ starts, const GT *__restrict__ loc,
                      const GT *__restrict__ attn, VT *__restrict__ out, Shape s, RowPlan plan) {
  constexpr int CPL = RowTraits<VT>::kCpl;
  constexpr int KQ = C / CPL;
  constexpr int NG = kWave / KQ;
  static_assert(C % CPL == 0 && (KQ & (KQ - 1)) == 0 && KQ <= kWave, "bad row layout");

  __shared__ Level lv[kMaxLevels];
  stage_levels(lv, shapes, starts, s);

  const int lane = threadIdx.x % kWave;
  const int wave = threadIdx.x / kWave;
  const int grp = lane / KQ, k = lane % KQ;
  const int GU = 1 << plan.gu_log2;
  const int UW = NG >> plan.gu_log2;  // units per wave iteration
  const int gi = grp & (GU - 1);
  const int slot = grp >> plan.gu_log2;
  const int MC = s.heads * C;

  const int lb = xcd_logical_block(blockIdx.x, gridDim.x);
  const int64_t wave_id = static_cast<int64_t>(lb) * (kBlock / kWave) + wave;

  for (int it = 0; it < plan.iters; ++it) {
    const int64_t u64 = (wave_id * plan.iters + it) * UW + slot;
    const bool live = u64 < s.units;
    const Unit U = decode_unit(live ? static_cast<int>(u64) : 0, s);
    const VT *vbase = value + static_cast<size_t>(U.b) * s.spatial * MC + U.m * C + k * CPL;
    const GT *lbase = loc + static_cast<size_t>(U.si) * s.lp * 2;
    const GT *abase = attn + static_cast<size_t>(U.si) * s.lp;

    float acc[CPL];
#pragma unroll
    for (int j = 0; j < CPL; ++j) acc[j] = 0.0f;

    for (int s0 = 0; s0 < s.lp; s0 += GU * NS) {
      float w[NS][4];
      float v[NS][4][CPL];
#pragma unroll
      for (int i = 0; i < NS; ++i) {
        const int smp = s0 + gi + GU * i;
        const bool ok = live && smp < s.lp;
        const int sm = ok ? smp : 0;
        const Level L = lv[level_of_sample(sm, s)];
        const float a = ok ? to_float(abase[sm]) : 0.0f;
        const Tap t = make_tap(to_float(lbase[2 * sm]), to_float(lbase[2 * sm + 1]), L, ok);
        w[i][0] = a * (t.wy0 * t.wx0);
        w[i][1] = a * (t.wy0 * t.wx1);
        w[i][2] = a * (t.wy1 * t.wx0);
        w[i][3] = a * (t.wy1 * t.wx1);
        const int c00 = (L.start + t.cell00) * MC;
        const int c10 = c00 + L.w * MC;
        const bool ok4[4] = {t.y0ok && t.x0ok, t.y0ok && t.x1ok, t.y1ok && t.x0ok,
                             t.y1ok && t.x1ok};
        const int off4[4] = {c00, c00 + MC, c10, c10 + MC};
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          if (ok4[c]) {
            load16(vbase + off4[c], v[i][c]);
          } else {
#pragma unroll
            for (int j = 0; j < CPL; ++j) v[i][c][j] = 0.0f;
          }
        }
      }
#pragma unroll
      for (int i = 0; i < NS; ++i) {
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
          acc[j] += w[i][0] * v[i][0][j] + w[i][1] * v[i][1][j] + w[i][2] * v[i][2][j] +
                    w[i][3] * v[i][3][j];
        }
      }
    }
    // sum the GU groups of the unit (lane distance KQ, 2KQ, ...)
    for (int off = KQ; off < KQ * GU; off <<= 1) {
#pragma unroll
      for (int j = 0; j < CPL; ++j) acc[j] += __shfl_xor(acc[j], off, kWave);
    }
    if (live && gi == 0) store16(out + static_cast<size_t>(U.si) * C + k * CPL, acc);
  }
}

// ------------------------------------------------------------ backward ---

template <typename VT, typename GT, int C, int NS>
__global__ void __launch_bounds__(kBlock)
    msda_backward_rows(const VT *__restrict__ value, const int64_t *__restrict__ shapes,
                       const int64_t *__restrict__ starts, const GT *__restrict__ loc,
                       const GT *__restrict__ attn, const VT *__restrict__ grad_out,
                       float *__restrict__ grad_value, float *__restrict__ grad_loc,
                       float *__restrict__ grad_attn, Shape s, RowPlan plan) {
  constexpr int CPL = RowTraits<VT>::kCpl;
  constexpr int KQ = C / CPL;
  constexpr int NG = kWave / KQ;
  static_assert(C % CPL == 0 && (KQ & (KQ - 1)) == 0 && KQ <= kWave, "bad row layout");

  __shared__ Level lv[kMaxLevels];
  stage_levels(lv, shapes, starts, s);

  const int lane = threadIdx.x % kWave;
  const int wave = threadIdx.x / kWave;
  const int grp = lane / KQ, k = lane % KQ;
  const int GU = 1 << plan.gu_log2;
  const int UW = NG >> plan.gu_log2;
  const int gi = grp & (GU - 1);
  const int slot = grp >> plan.gu_log2;
  const int MC = s.heads * C;

  const int lb = xcd_logical_block(blockIdx.x, gridDim.x);
  const int64_t wave_id = static_cast<int64_t>(lb) * (kBlock / kWave) + wave;

  for (int it = 0; it < plan.iters; ++it) {
    const int64_t u64 = (wave_id * plan.iters + it) * UW + slot;
    const bool live = u64 < s.units;
    const Unit U = decode_unit(live ? static_cast<int>(u64) : 0, s);
    const size_t row0 = static_cast<size_t>(U.b) * s.spatial * MC + U.m * C + k * CPL;
    const VT *vbase = value + row0;
    float *gvbase = grad_value + row0;
    const GT *lbase = loc + static_cast<size_t>(U.si) * s.lp * 2;
    const GT *abase = attn + static_cast<size_t>(U.si) * s.lp;
    float *glbase = grad_loc + static_cast<size_t>(U.si) * s.lp * 2;
    float *gabase = grad_attn + static_cast<size_t>(U.si) * s.lp;

    float g[CPL];
    if (live) {
      load16(grad_out + static_cast<size_t>(U.si) * C + k * CPL, g);
    } else {
#pragma unroll
      for (int j = 0; j < CPL; ++j) g[j] = 0.0f;
    }

    for (int s0 = 0; s0 < s.lp; s0 += GU * NS) {
      Tap t[NS];
      float a[NS], fw[NS], fh[NS];
      int off[NS][4];
      bool okc[NS][4];
      float v[NS][4][CPL];
#pragma unroll
      for (int i = 0; i < NS; ++i) {
        const int smp = s0 + gi + GU * i;
        const bool ok = live && smp < s.lp;
        const int sm = ok ? smp : 0;
        const Level L = lv[level_of_sample(sm, s)];
        a[i] = ok ? to_float(abase[sm]) : 0.0f;
        fw[i] = L.fw;
        fh[i] = L.fh;
        t[i] = make_tap(to_float(lbase[2 * sm]), to_float(lbase[2 * sm + 1]), L, ok);
        const int c00 = (L.start + t[i].cell00) * MC;
        const int c10 = c00 + L.w * MC;
        off[i][0] = c00;
        off[i][1] = c00 + MC;
        off[i][2] = c10;
        off[i][3] = c10 + MC;
        okc[i][0] = t[i].y0ok && t[i].x0ok;
        okc[i][1] = t[i].y0ok && t[i].x1ok;
        okc[i][2] = t[i].y1ok && t[i].x0ok;
        okc[i][3] = t[i].y1ok && t[i].x1ok;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          if (okc[i][c]) {
            load16(vbase + off[i][c], v[i][c]);
          } else {
#pragma unroll
            for (int j = 0; j < CPL; ++j) v[i][c][j] = 0.0f;
          }
        }
      }
#pragma unroll
      for (int i = 0; i < NS; ++i) {
        const float wx0 = t[i].wx0, wx1 = t[i].wx1, wy0 = t[i].wy0, wy1 = t[i].wy1;
        const float cw[4] = {wy0 * wx0, wy0 * wx1, wy1 * wx0, wy1 * wx1};
        float ga = 0.0f, gx = 0.0f, gy = 0.0f;
        float tg[CPL];
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
          tg[j] = g[j] * a[i];
          const float v00 = v[i][0][j], v01 = v[i][1][j], v10 = v[i][2][j], v11 = v[i][3][j];
          const float val = cw[0] * v00 + cw[1] * v01 + cw[2] * v10 + cw[3] * v11;
          ga += g[j] * val;
          gx += tg[j] * (wy0 * (v01 - v00) + wy1 * (v11 - v10));
          gy += tg[j] * (wx0 * (v10 - v00) + wx1 * (v11 - v01));
        }
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          if (okc[i][c]) {
            float *p = gvbase + off[i][c];
#pragma unroll
            for (int j = 0; j < CPL; ++j) unsafeAtomicAdd(p + j, cw[c] * tg[j]);
          }
        }
        ga = group_sum<KQ>(ga);
        gx = group_sum<KQ>(gx);
        gy = group_sum<KQ>(gy);
        const int smp = s0 + gi + GU * i;
        if (live && smp < s.lp && k == 0) {
          gabase[smp] = ga;
          *reinterpret_cast<float2 *>(glbase + 2 * smp) = make_float2(gx * fw[i], gy * fh[i]);
        }
      }
    }
  }
}

// ------------------------------------------------------- generic (any C) ---

template <typename VT, typename GT>
__global__ void __launch_bounds__(kBlock)
    msda_forward_generic(const VT *__restrict__ value, const int64_t *__restrict__ shapes,
                         const int64_t *__restrict__ starts, const GT *__restrict__ loc,
                         const GT *__restrict__ attn, VT *__restrict__ out, Shape s) {
  __shared__ Level lv[kMaxLevels];
  stage_levels(lv, shapes, starts, s);
  const int C = s.channels, MC = s.heads * C;
  const int64_t total = static_cast<int64_t>(s.units) * C;
  for (int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; idx < total;
       idx += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int c = static_cast<int>(idx % C);
    const int si = static_cast<int>(idx / C);
    const int m = si % s.heads;
    const int b = si / (s.heads * s.queries);
    const VT *vbase = value + static_cast<size_t>(b) * s.spatial * MC + m * C + c;
    const GT *lbase = loc + static_cast<size_t>(si) * s.lp * 2;
    const GT *abase = attn + static_cast<size_t>(si) * s.lp;
    float acc = 0.0f;
    for (int smp = 0; smp < s.lp; ++smp) {
      const Level L = lv[smp / s.points];
      const float a = to_float(abase[smp]);
      const Tap t = make_tap(to_float(lbase[2 * smp]), to_float(lbase[2 * smp + 1]), L, true);
      const int c00 = (L.start + t.cell00) * MC, c10 = c00 + L.w * MC;
      const float v00 = (t.y0ok && t.x0ok) ? to_float(vbase[c00]) : 0.0f;
      const float v01 = (t.y0ok && t.x1ok) ? to_float(vbase[c00 + MC]) : 0.0f;
      const float v10 = (t.y1ok && t.x0ok) ? to_float(vbase[c10]) : 0.0f;
      const float v11 = (t.y1ok && t.x1ok) ? to_float(vbase[c10 + MC]) : 0.0f;
      acc += a * (t.wy0 * t.wx0) * v00 + a * (t.wy0 * t.wx1) * v01 +
             a * (t.wy1 * t.wx0) * v10 + a * (t.wy1 * t.wx1) * v11;
    }
    out[idx] = from_float<VT>(acc);
  }
}

template <typename VT, typename GT>
__global__ void __launch_bounds__(kBlock)
    msda_backward_generic(const VT *__restrict__ value, const int64_t *__restrict__ shapes,
                          const int64_t *__restrict__ starts, const GT *__restrict__ loc,
                          const GT *__restrict__ attn, const VT *__restrict__ grad_out,
                          float *__restrict__ grad_value, float *__restrict__ grad_loc,
                          float *__restrict__ grad_attn, Shape s) {
  __shared__ Level lv[kMaxLevels];
  stage_levels(lv, shapes, starts, s);
  const int C = s.channels, MC = s.heads * C;
  const int64_t total = static_cast<int64_t>(s.units) * s.lp;
  for (int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; idx < total;
       idx += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int smp = static_cast<int>(idx % s.lp);
    const int si = static_cast<int>(idx / s.lp);
    const int m = si % s.heads;
    const int b = si / (s.heads * s.queries);
    const size_t row0 = static_cast<size_t>(b) * s.spatial * MC + m * C;
    const Level L = lv[smp / s.points];
    const float a = to_float(attn[idx]);
    const Tap t = make_tap(to_float(loc[2 * idx]), to_float(loc[2 * idx + 1]), L, true);
    const int c00 = (L.start + t.cell00) * MC, c10 = c00 + L.w * MC;
    const int off4[4] = {c00, c00 + MC, c10, c10 + MC};
    const bool ok4[4] = {t.y0ok && t.x0ok, t.y0ok && t.x1ok, t.y1ok && t.x0ok, t.y1ok && t.x1ok};
    const float cw[4] = {t.wy0 * t.wx0, t.wy0 * t.wx1, t.wy1 * t.wx0, t.wy1 * t.wx1};
    float ga = 0.0f, gx = 0.0f, gy = 0.0f;
    for (int c = 0; c < C; ++c) {
      const float gc = to_float(grad_out[static_cast<size_t>(si) * C + c]);
      const float tg = gc * a;
      float v[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = ok4[e] ? to_float(value[row0 + off4[e] + c]) : 0.0f;
      const float val = cw[0] * v[0] + cw[1] * v[1] + cw[2] * v[2] + cw[3] * v[3];
      ga += gc * val;
      gx += tg * (t.wy0 * (v[1] - v[0]) + t.wy1 * (v[3] - v[2]));
      gy += tg * (t.wx0 * (v[2] - v[0]) + t.wx1 * (v[3] - v[1]));
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if (ok4[e]) unsafeAtomicAdd(grad_value + row0 + off4[e] + c, cw[e] * tg);
      }
    }
    grad_attn[idx] = ga;
    grad_loc[2 * idx] = gx * L.fw;
    grad_loc[2 * idx + 1] = gy * L.fh;
  }
}

// Fill with zeros (used before the atomic fallback backward; a kernel rather
// than a memset so that the launch sequence is graph-capture friendly).
__global__ void __launch_bounds__(kBlock) zero_kernel(float *x, int64_t n) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    x[i] = 0.0f;
  }
}

// ---------------------------------------------------------------- smoke ---

__global__ void __launch_bounds__(kBlock) add_one_kernel(const float *x, float *y, int64_t n) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    y[i] = x[i] + 1.0f;
  }
}

}  // namespace msda
