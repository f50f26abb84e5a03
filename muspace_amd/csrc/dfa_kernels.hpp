// Deformable aggregation (SparseDrive's multi-camera, multi-scale feature
// aggregation) for MI355X (gfx950, wave64).
//
// Tensors (float32, row-major):
//   mc_ms_feat         [batch, num_feat, C]   every (camera, scale) map of a batch entry, H*W
//                                              rows of C channels starting at scale_start_index
//   spatial_shape      [cams, scales, 2]  int32 (H, W)
//   scale_start_index  [cams, scales]     int32
//   sampling_location  [batch, anchors, pts, cams, 2]   (x along W, y along H, in [0, 1])
//   weights            [batch, anchors, pts, cams, scales, groups]
//   output             [batch, anchors, C]
// output[b, a, c] = sum over (pt, cam) with 0 < x < 1 and 0 < y < 1 (strictly; other
// points are skipped), over scales s, of
//   weights[b, a, pt, cam, s, c / (C / groups)] * bilinear(map(b, cam, s), y*H - 0.5, x*W - 0.5)[c]
// with corners outside [0, H-1] x [0, W-1] dropped. Reference semantics:
// deformable_aggregation_kernel_opt / deformable_aggregation_grad_kernel_opt
// (/root/reference/csrc/deformable_aggregation/deformable_aggregation_musa.mu:39-160,304-430)
// and the PyTorch reference (/root/reference/mu_space/ops/deformable_aggregation.py:88-158).
//
// Row kernels (C = 64*NT channels, NT <= 4): one wavefront per (batch, anchor);
// lane i owns channels i, i+64, ... so every gather, atomic and store of a
// corner row is a contiguous 256-byte access. The lanes load the locations of
// 64 (pt, cam) pairs at once and ballot the active ones; the wavefront then
// walks only the active pairs, whose geometry is uniform (read from the owning
// lane). Corner loads are unconditional raw buffer loads: a corner outside its
// map gets an out-of-range offset, which reads zero.
//
// Generic kernels (any C and groups) exist for shape coverage, not speed.
#pragma once

#include "msda_device.hpp"

namespace dfa {

using msda::kOobOffset;
using msda::kWave;

constexpr int kBlock = 256;     // four (batch, anchor) rows per workgroup
constexpr int kMaxViews = 256;  // cameras x scales, staged in LDS
constexpr int kMaxGroups = 8;

struct Dims {
  int batch, cams, feat, embeds, scales, anchors, pts, groups;
};

// One (camera, scale) feature map; h = w = 0 marks a map that would reach
// outside [0, num_feat) and is skipped instead of read out of bounds.
struct View {
  int h, w, start;
};

__device__ __forceinline__ void stage_views(View *v, const int32_t *shape, const int32_t *start,
                                            const Dims &d) {
  const int n = d.cams * d.scales;
  for (int i = threadIdx.x; i < n; i += blockDim.x) {
    const int h = shape[2 * i], w = shape[2 * i + 1], s0 = start[i];
    const bool ok = h > 0 && w > 0 && s0 >= 0 &&
                    static_cast<int64_t>(s0) + static_cast<int64_t>(h) * w <= d.feat;
    v[i] = ok ? View{h, w, s0} : View{0, 0, 0};
  }
  __syncthreads();
}

// Bilinear tap of one sample in one map: the four corner rows (cell index in
// the map, -1 when the corner is outside) and their weights, plus the
// quantities the location gradient needs.
struct Tap {
  int cell[4];
  float w[4];
  float lh, lw, hh, hw;
};

__device__ __forceinline__ Tap make_tap(float x, float y, const View &v) {
  const float h_im = y * static_cast<float>(v.h) - 0.5f;
  const float w_im = x * static_cast<float>(v.w) - 0.5f;
  const int h0 = static_cast<int>(floorf(h_im)), w0 = static_cast<int>(floorf(w_im));
  const int h1 = h0 + 1, w1 = w0 + 1;
  Tap t;
  t.lh = h_im - static_cast<float>(h0);
  t.lw = w_im - static_cast<float>(w0);
  t.hh = 1.0f - t.lh;
  t.hw = 1.0f - t.lw;
  t.w[0] = t.hh * t.hw;
  t.w[1] = t.hh * t.lw;
  t.w[2] = t.lh * t.hw;
  t.w[3] = t.lh * t.lw;
  t.cell[0] = h0 >= 0 && w0 >= 0 ? h0 * v.w + w0 : -1;
  t.cell[1] = h0 >= 0 && w1 <= v.w - 1 ? h0 * v.w + w1 : -1;
  t.cell[2] = h1 <= v.h - 1 && w0 >= 0 ? h1 * v.w + w0 : -1;
  t.cell[3] = h1 <= v.h - 1 && w1 <= v.w - 1 ? h1 * v.w + w1 : -1;
  return t;
}

__device__ __forceinline__ bool active(float x, float y) {
  return x > 0.0f && x < 1.0f && y > 0.0f && y < 1.0f;  // NaN is inactive
}

__device__ __forceinline__ float buffer_load4(__amdgpu_buffer_rsrc_t r, uint32_t offset) {
  return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, offset, 0, 0));
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = kWave / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

// Sum over aligned runs of `width` lanes (a power of two <= 64).
__device__ __forceinline__ float segment_sum(float v, int width) {
  for (int off = 1; off < width; off <<= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

template <int NT>
__global__ void __launch_bounds__(kBlock)
    dfa_forward_rows(const float *__restrict__ feat, uint32_t feat_bytes,
                     const int32_t *__restrict__ shape, const int32_t *__restrict__ start,
                     const float *__restrict__ loc, const float *__restrict__ weights,
                     float *__restrict__ out, Dims d) {
  constexpr int C = NT * kWave;
  __shared__ View views[kMaxViews];
  stage_views(views, shape, start, d);
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int row = msda::xcd_logical_block(blockIdx.x, gridDim.x) * (kBlock / kWave) + wave;
  if (row >= d.batch * d.anchors) return;  // no barrier follows
  const int b = row / d.anchors;
  const int cpg = C / d.groups;
  const __amdgpu_buffer_rsrc_t rf = msda::make_rsrc(feat, feat_bytes);
  int grp[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) grp[t] = (t * kWave + lane) / cpg;
  float acc[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) acc[t] = 0.0f;

  const int pairs = d.pts * d.cams, sg = d.scales * d.groups;
  const float *loc_row = loc + static_cast<size_t>(row) * pairs * 2;
  const float *w_row = weights + static_cast<size_t>(row) * pairs * sg;
  const uint32_t batch_base = static_cast<uint32_t>(b) * static_cast<uint32_t>(d.feat);
  for (int base = 0; base < pairs; base += kWave) {
    const int pi = min(base + lane, pairs - 1);
    const float lx = loc_row[2 * pi], ly = loc_row[2 * pi + 1];
    uint64_t mask = __ballot(base + lane < pairs && active(lx, ly));
    while (mask) {
      const int l = __builtin_ctzll(mask);
      mask &= mask - 1;
      const float x = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(lx), l));
      const float y = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ly), l));
      const int pair = base + l, cam = pair % d.cams;
      const float *wp = w_row + static_cast<size_t>(pair) * sg;
#pragma unroll 2
      for (int s = 0; s < d.scales; ++s) {
        const View v = views[cam * d.scales + s];
        const Tap tp = make_tap(x, y, v);
        float val[4][NT];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const bool ok = v.h > 0 && tp.cell[k] >= 0;
          const uint32_t row_off =
              ok ? (batch_base + static_cast<uint32_t>(v.start + tp.cell[k])) * (C * 4u)
                 : kOobOffset;
#pragma unroll
          for (int t = 0; t < NT; ++t) val[k][t] = buffer_load4(rf, row_off + (t * kWave + lane) * 4u);
        }
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          const float wg = wp[s * d.groups + grp[t]];
          acc[t] += (tp.w[0] * val[0][t] + tp.w[1] * val[1][t] + tp.w[2] * val[2][t] +
                     tp.w[3] * val[3][t]) * wg;
        }
      }
    }
  }
  float *o = out + static_cast<size_t>(row) * C + lane;
#pragma unroll
  for (int t = 0; t < NT; ++t) o[t * kWave] += acc[t];
}

template <int NT>
__global__ void __launch_bounds__(kBlock)
    dfa_backward_rows(const float *__restrict__ feat, uint32_t feat_bytes,
                      const int32_t *__restrict__ shape, const int32_t *__restrict__ start,
                      const float *__restrict__ loc, const float *__restrict__ weights,
                      const float *__restrict__ grad_out, float *__restrict__ grad_feat,
                      float *__restrict__ grad_loc, float *__restrict__ grad_weights, Dims d) {
  constexpr int C = NT * kWave;
  __shared__ View views[kMaxViews];
  stage_views(views, shape, start, d);
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int row = msda::xcd_logical_block(blockIdx.x, gridDim.x) * (kBlock / kWave) + wave;
  if (row >= d.batch * d.anchors) return;  // no barrier follows
  const int b = row / d.anchors;
  const int cpg = C / d.groups;
  const int seg = cpg < kWave ? cpg : kWave;  // lanes summed for one group's weight gradient
  const int tpg = cpg / seg;                  // channel slots per group (cpg > 64)
  const __amdgpu_buffer_rsrc_t rf = msda::make_rsrc(feat, feat_bytes);
  int grp[NT];
  float g[NT];
  const float *go = grad_out + static_cast<size_t>(row) * C + lane;
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    grp[t] = (t * kWave + lane) / cpg;
    g[t] = go[t * kWave];
  }

  const int pairs = d.pts * d.cams, sg = d.scales * d.groups;
  const float *loc_row = loc + static_cast<size_t>(row) * pairs * 2;
  const float *w_row = weights + static_cast<size_t>(row) * pairs * sg;
  float *gl_row = grad_loc + static_cast<size_t>(row) * pairs * 2;
  float *gw_row = grad_weights + static_cast<size_t>(row) * pairs * sg;
  const size_t batch_elem = static_cast<size_t>(b) * d.feat * C;
  for (int base = 0; base < pairs; base += kWave) {
    const int n = min(kWave, pairs - base);
    const int pi = base + min(lane, n - 1);
    const float lx = loc_row[2 * pi], ly = loc_row[2 * pi + 1];
    const uint64_t act = __ballot(lane < n && active(lx, ly));
    // weight gradients of skipped pairs are zero
    for (int e = lane; e < n * sg; e += kWave) {
      if (!((act >> (e / sg)) & 1)) gw_row[static_cast<size_t>(base) * sg + e] = 0.0f;
    }
    float my_gx = 0.0f, my_gy = 0.0f;  // location gradient of this lane's pair
    uint64_t mask = act;
    while (mask) {
      const int l = __builtin_ctzll(mask);
      mask &= mask - 1;
      const float x = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(lx), l));
      const float y = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ly), l));
      const int pair = base + l, cam = pair % d.cams;
      const float *wp = w_row + static_cast<size_t>(pair) * sg;
      float *gwp = gw_row + static_cast<size_t>(pair) * sg;
      float gx = 0.0f, gy = 0.0f;
      for (int s = 0; s < d.scales; ++s) {
        const View v = views[cam * d.scales + s];
        const Tap tp = make_tap(x, y, v);
        float val[4][NT];
        bool ok[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          ok[k] = v.h > 0 && tp.cell[k] >= 0;
          const uint32_t row_off =
              ok[k] ? (static_cast<uint32_t>(b) * static_cast<uint32_t>(d.feat) +
                       static_cast<uint32_t>(v.start + tp.cell[k])) * (C * 4u)
                    : kOobOffset;
#pragma unroll
          for (int t = 0; t < NT; ++t) val[k][t] = buffer_load4(rf, row_off + (t * kWave + lane) * 4u);
        }
        float gwt[NT];
        float top[NT];
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          const float wg = wp[s * d.groups + grp[t]];
          top[t] = g[t] * wg;
          const float sampled = tp.w[0] * val[0][t] + tp.w[1] * val[1][t] +
                                tp.w[2] * val[2][t] + tp.w[3] * val[3][t];
          gwt[t] = g[t] * sampled;
          const float dh = -tp.hw * val[0][t] - tp.lw * val[1][t] + tp.hw * val[2][t] +
                           tp.lw * val[3][t];
          const float dw = -tp.hh * val[0][t] + tp.hh * val[1][t] - tp.lh * val[2][t] +
                           tp.lh * val[3][t];
          gx += static_cast<float>(v.w) * dw * top[t];
          gy += static_cast<float>(v.h) * dh * top[t];
        }
        // feature gradient: one contiguous 256-byte atomic per corner and slot
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          if (ok[k]) {  // uniform across the wavefront
            float *dst = grad_feat + batch_elem + static_cast<size_t>(v.start + tp.cell[k]) * C + lane;
#pragma unroll
            for (int t = 0; t < NT; ++t) unsafeAtomicAdd(dst + t * kWave, tp.w[k] * top[t]);
          }
        }
        // weight gradient of each group: sum over its channels
        if (tpg == 1) {
#pragma unroll
          for (int t = 0; t < NT; ++t) {
            const float sum = segment_sum(gwt[t], seg);
            if ((lane & (seg - 1)) == 0) gwp[s * d.groups + grp[t]] = sum;
          }
        } else {
#pragma unroll
          for (int t = 0; t < NT; ++t) gwt[t] = wave_sum(gwt[t]);
          if (lane == 0) {
            for (int gi = 0; gi < d.groups; ++gi) {
              float sum = 0.0f;
#pragma unroll
              for (int t = 0; t < NT; ++t) sum += t / tpg == gi ? gwt[t] : 0.0f;
              gwp[s * d.groups + gi] = sum;
            }
          }
        }
      }
      gx = wave_sum(gx);
      gy = wave_sum(gy);
      if (lane == l) {
        my_gx = gx;
        my_gy = gy;
      }
    }
    if (lane < n) {
      gl_row[2 * (base + lane)] = my_gx;
      gl_row[2 * (base + lane) + 1] = my_gy;
    }
  }
}

// ------------------------------------------------------------- generic ---

// One thread per (batch, anchor, channel): the whole sum, no atomics.
__global__ void __launch_bounds__(kBlock)
    dfa_forward_generic(const float *__restrict__ feat, const int32_t *__restrict__ shape,
                        const int32_t *__restrict__ start, const float *__restrict__ loc,
                        const float *__restrict__ weights, float *__restrict__ out, Dims d) {
  __shared__ View views[kMaxViews];
  stage_views(views, shape, start, d);
  const int C = d.embeds, cpg = C / d.groups;
  const int pairs = d.pts * d.cams, sg = d.scales * d.groups;
  const int64_t total = static_cast<int64_t>(d.batch) * d.anchors * C;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int c = static_cast<int>(i % C);
    const int64_t row = i / C;
    const int64_t b = row / d.anchors;
    const float *loc_row = loc + row * pairs * 2;
    const float *w_row = weights + row * pairs * sg;
    float acc = 0.0f;
    for (int pair = 0; pair < pairs; ++pair) {
      const float x = loc_row[2 * pair], y = loc_row[2 * pair + 1];
      if (!active(x, y)) continue;
      const int cam = pair % d.cams;
      for (int s = 0; s < d.scales; ++s) {
        const View v = views[cam * d.scales + s];
        if (v.h == 0) continue;
        const Tap tp = make_tap(x, y, v);
        float sampled = 0.0f;
        for (int k = 0; k < 4; ++k) {
          if (tp.cell[k] >= 0) {
            sampled += tp.w[k] * feat[(b * d.feat + v.start + tp.cell[k]) * C + c];
          }
        }
        acc += sampled * w_row[static_cast<int64_t>(pair) * sg + s * d.groups + c / cpg];
      }
    }
    out[i] += acc;
  }
}

// One thread per (batch, anchor, pt, cam): loops over scales and channels;
// feature gradients with atomics, location and weight gradients written
// (zero for a skipped pair).
__global__ void __launch_bounds__(kBlock)
    dfa_backward_generic(const float *__restrict__ feat, const int32_t *__restrict__ shape,
                         const int32_t *__restrict__ start, const float *__restrict__ loc,
                         const float *__restrict__ weights, const float *__restrict__ grad_out,
                         float *__restrict__ grad_feat, float *__restrict__ grad_loc,
                         float *__restrict__ grad_weights, Dims d) {
  __shared__ View views[kMaxViews];
  stage_views(views, shape, start, d);
  const int C = d.embeds, cpg = C / d.groups;
  const int pairs = d.pts * d.cams, sg = d.scales * d.groups;
  const int64_t total = static_cast<int64_t>(d.batch) * d.anchors * pairs;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int pair = static_cast<int>(i % pairs);
    const int64_t row = i / pairs;
    const int64_t b = row / d.anchors;
    const int cam = pair % d.cams;
    const float x = loc[2 * i], y = loc[2 * i + 1];
    float *gw = grad_weights + i * sg;
    if (!active(x, y)) {
      for (int e = 0; e < sg; ++e) gw[e] = 0.0f;
      grad_loc[2 * i] = 0.0f;
      grad_loc[2 * i + 1] = 0.0f;
      continue;
    }
    const float *w = weights + i * sg;
    const float *go = grad_out + row * C;
    float gx = 0.0f, gy = 0.0f;
    for (int s = 0; s < d.scales; ++s) {
      const View v = views[cam * d.scales + s];
      float gsum[kMaxGroups];
      for (int gi = 0; gi < kMaxGroups; ++gi) gsum[gi] = 0.0f;
      if (v.h > 0) {
        const Tap tp = make_tap(x, y, v);
        const int64_t base = (b * d.feat + v.start) * C;
        for (int c = 0; c < C; ++c) {
          const int gi = c / cpg;
          const float top = go[c] * w[s * d.groups + gi];
          float vals[4];
          for (int k = 0; k < 4; ++k) {
            vals[k] = tp.cell[k] >= 0 ? feat[base + static_cast<int64_t>(tp.cell[k]) * C + c] : 0.0f;
            if (tp.cell[k] >= 0) {
              unsafeAtomicAdd(grad_feat + base + static_cast<int64_t>(tp.cell[k]) * C + c,
                              tp.w[k] * top);
            }
          }
          gsum[gi] += go[c] * (tp.w[0] * vals[0] + tp.w[1] * vals[1] + tp.w[2] * vals[2] +
                               tp.w[3] * vals[3]);
          const float dh = -tp.hw * vals[0] - tp.lw * vals[1] + tp.hw * vals[2] + tp.lw * vals[3];
          const float dw = -tp.hh * vals[0] + tp.hh * vals[1] - tp.lh * vals[2] + tp.lh * vals[3];
          gx += static_cast<float>(v.w) * dw * top;
          gy += static_cast<float>(v.h) * dh * top;
        }
      }
      for (int gi = 0; gi < d.groups; ++gi) gw[s * d.groups + gi] = gsum[gi];
    }
    grad_loc[2 * i] = gx;
    grad_loc[2 * i + 1] = gy;
  }
}

}  // namespace dfa
