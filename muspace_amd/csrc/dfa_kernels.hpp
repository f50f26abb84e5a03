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
// Row kernels (C = 64*NT channels, NT <= 4): one to four wavefronts per
// (batch, anchor) row; lane i owns channels i, i+64, ... so every gather,
// atomic and store of a corner row is a contiguous 256-byte access. The lanes
// load the locations of 64 (pt, cam) pairs at once and ballot the active ones;
// each wavefront then walks only its share of the active pairs, whose geometry
// is uniform (read from the owning lane). Corner loads are unconditional raw buffer loads: a corner outside its
// map gets an out-of-range offset, which reads zero.
//
// Generic kernels (any C and groups) exist for shape coverage, not speed.
#pragma once

#include <cfloat>

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
// outside [0, num_feat) and is skipped instead of read out of bounds. lds:
// the map's first accumulator cell in dfa_backward_coarse, or -1 when the
// row kernel adds its feature gradients with device atomics.
struct View {
  int h, w, start, lds;
};

__device__ __forceinline__ void stage_views(View *v, const int32_t *shape, const int32_t *start,
                                            const Dims &d) {
  const int n = d.cams * d.scales;
  for (int i = threadIdx.x; i < n; i += blockDim.x) {
    const int h = shape[2 * i], w = shape[2 * i + 1], s0 = start[i];
    const bool ok = h > 0 && w > 0 && s0 >= 0 &&
                    static_cast<int64_t>(s0) + static_cast<int64_t>(h) * w <= d.feat;
    v[i] = ok ? View{h, w, s0, -1} : View{0, 0, 0, -1};
  }
  __syncthreads();
}

// Maps of one camera whose feature gradients dfa_backward_coarse sums in LDS:
// the smallest maps first (ties: the lower scale) while their cells fit
// `budget` in total. Sets View::lds of each chosen map and returns the cells
// used. Both feature-gradient kernels run it on the same views, so they agree
// on which maps the LDS kernel owns.
__device__ inline int select_coarse(View *v, int scales, int budget) {
  int used = 0;
  for (;;) {
    int best = -1, best_cells = 0;
    for (int s = 0; s < scales; ++s) {
      const int cells = v[s].h * v[s].w;  // 0 for a skipped map
      if (v[s].lds < 0 && cells > 0 && (best < 0 || cells < best_cells)) {
        best = s;
        best_cells = cells;
      }
    }
    if (best < 0 || best_cells > budget - used) break;
    v[best].lds = used;
    used += best_cells;
  }
  return used;
}

// select_coarse for every camera (budget 0: none), then a barrier.
__device__ inline void mark_coarse(View *views, const Dims &d, int budget) {
  if (budget > 0) {
    for (int cam = threadIdx.x; cam < d.cams; cam += blockDim.x) {
      select_coarse(views + cam * d.scales, d.scales, budget);
    }
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

// Sum over the wavefront, every lane receiving it (DPP inside the 16-lane
// rows, readlane across them: no LDS-routed shuffles). Whole wavefront active.
__device__ __forceinline__ float wave_sum(float v) { return msda::group_sum_sel(v, kWave); }

// Sum over aligned runs of `width` lanes (a power of two <= 64, uniform),
// every lane of the run receiving it; whole wavefront active.
__device__ __forceinline__ float segment_sum(float v, int width) {
  return msda::group_sum_sel(v, width);
}

// Forward, one (batch, anchor) row over `parts` (1, 2 or 4) wavefronts of one
// workgroup: the row's active pairs are dealt round-robin by their rank among
// the active pairs, and the parts' partial rows are summed through LDS by
// part 0, which adds the row to `out`.
template <int NT>
__global__ void __launch_bounds__(kBlock)
    dfa_forward_rows(const float *__restrict__ feat, uint32_t feat_bytes,
                     const int32_t *__restrict__ shape, const int32_t *__restrict__ start,
                     const float *__restrict__ loc, const float *__restrict__ weights,
                     float *__restrict__ out, Dims d, int parts) {
  constexpr int C = NT * kWave;
  __shared__ View views[kMaxViews];
  __shared__ float partial[kBlock / kWave][C];
  stage_views(views, shape, start, d);
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int unit = msda::xcd_logical_block(blockIdx.x, gridDim.x) * (kBlock / kWave) + wave;
  const int row = unit / parts, part = unit & (parts - 1);  // parts: 1, 2 or 4
  const bool live = row < d.batch * d.anchors;  // every wavefront reaches the barrier below
  const int b = live ? row / d.anchors : 0;
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
  const uint64_t below = (uint64_t{1} << lane) - 1;
  int seen = 0;  // active pairs of the row before this run of 64
  for (int base = 0; live && base < pairs; base += kWave) {
    const int pi = min(base + lane, pairs - 1);
    const float lx = loc_row[2 * pi], ly = loc_row[2 * pi + 1];
    const bool on = base + lane < pairs && active(lx, ly);
    const uint64_t act = __ballot(on);
    const bool mine = on && ((seen + __builtin_popcountll(act & below)) & (parts - 1)) == part;
    seen += __builtin_popcountll(act);
    uint64_t mask = __ballot(mine);
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
  if (parts > 1) {  // uniform over the workgroup
    if (part > 0) {
#pragma unroll
      for (int t = 0; t < NT; ++t) partial[wave][t * kWave + lane] = acc[t];
    }
    __syncthreads();
    if (part > 0) return;
    for (int w = wave + 1; w < wave + parts; ++w) {
#pragma unroll
      for (int t = 0; t < NT; ++t) acc[t] += partial[w][t * kWave + lane];
    }
  }
  if (!live) return;
  float *o = out + static_cast<size_t>(row) * C + lane;
#pragma unroll
  for (int t = 0; t < NT; ++t) o[t * kWave] += acc[t];
}

// Backward, one (batch, anchor) row split over `parts` wavefronts: the row's
// active pairs are dealt round-robin (by their rank among the active pairs)
// so that every wavefront of the row gets a near-equal share; a skipped
// pair's zero gradients go to the wavefront `pair % parts`. Location and
// weight gradients are per pair and feature gradients are atomics, so the
// parts need no reduction. A pair's corner rows and weights are loaded two
// scales at a time before either is used, so one memory latency covers two
// scales (four scales at once cost registers and occupancy: slower).
constexpr int kScaleRun = 2;

template <int NT>
__global__ void __launch_bounds__(kBlock)
    dfa_backward_rows(const float *__restrict__ feat, uint32_t feat_bytes,
                      const int32_t *__restrict__ shape, const int32_t *__restrict__ start,
                      const float *__restrict__ loc, const float *__restrict__ weights,
                      const float *__restrict__ grad_out, float *__restrict__ grad_feat,
                      float *__restrict__ grad_loc, float *__restrict__ grad_weights, Dims d,
                      int coarse_budget, int parts) {
  constexpr int C = NT * kWave;
  __shared__ View views[kMaxViews];
  stage_views(views, shape, start, d);
  mark_coarse(views, d, coarse_budget);  // maps whose feature gradients another kernel sums
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int unit = msda::xcd_logical_block(blockIdx.x, gridDim.x) * (kBlock / kWave) + wave;
  const int row = unit / parts, part = unit & (parts - 1);  // parts: 1, 2 or 4
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
  const uint32_t batch_row = static_cast<uint32_t>(b) * static_cast<uint32_t>(d.feat);
  const uint64_t below = (uint64_t{1} << lane) - 1;
  const int sgd = sg > 0 ? sg : 1;  // no scales: nothing is zeroed
  const int lane_p = lane / sgd, lane_j = lane - lane_p * sgd;  // element `lane` of a run
  const int step_p = kWave / sgd, step_j = kWave - step_p * sgd;
  int seen = 0;  // active pairs of the row before this run of 64
  for (int base = 0; base < pairs; base += kWave) {
    const int n = min(kWave, pairs - base);
    const int pi = base + min(lane, n - 1);
    const float lx = loc_row[2 * pi], ly = loc_row[2 * pi + 1];
    const bool on = lane < n && active(lx, ly);
    const uint64_t act = __ballot(on);
    const int owner = (on ? seen + __builtin_popcountll(act & below) : pi) & (parts - 1);
    const uint64_t own = __ballot(lane < n && owner == part);
    seen += __builtin_popcountll(act);
    // weight gradients of skipped pairs are zero: element e = p * sg + j of
    // the run, (p, j) stepped by kWave elements per pass (no division inside)
    for (int e = lane, p = lane_p, j = lane_j; e < n * sg; e += kWave) {
      if (!((act >> p) & 1) && ((base + p) & (parts - 1)) == part) {
        gw_row[static_cast<size_t>(base) * sg + e] = 0.0f;
      }
      p += step_p;
      j += step_j;
      if (j >= sg) {
        j -= sg;
        ++p;
      }
    }
    float my_gx = 0.0f, my_gy = 0.0f;  // location gradient of this lane's pair
    uint64_t mask = act & own;
    while (mask) {
      const int l = __builtin_ctzll(mask);
      mask &= mask - 1;
      const float x = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(lx), l));
      const float y = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ly), l));
      const int pair = base + l, cam = pair % d.cams;
      const float *wp = w_row + static_cast<size_t>(pair) * sg;
      float *gwp = gw_row + static_cast<size_t>(pair) * sg;
      const View *cv = views + cam * d.scales;
      float gx = 0.0f, gy = 0.0f;
      for (int s0 = 0; s0 < d.scales; s0 += kScaleRun) {
        // every load of the run first (scales past the last read nothing)
        float val[kScaleRun][4][NT];
        float wv[kScaleRun][NT];
#pragma unroll
        for (int j = 0; j < kScaleRun; ++j) {
          const int s = min(s0 + j, d.scales - 1);
          const View v = cv[s];
          const Tap tp = make_tap(x, y, v);
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            const bool ok = s0 + j < d.scales && v.h > 0 && tp.cell[k] >= 0;
            const uint32_t row_off =
                ok ? (batch_row + static_cast<uint32_t>(v.start + tp.cell[k])) * (C * 4u)
                   : kOobOffset;
#pragma unroll
            for (int t = 0; t < NT; ++t) {
              val[j][k][t] = buffer_load4(rf, row_off + (t * kWave + lane) * 4u);
            }
          }
#pragma unroll
          for (int t = 0; t < NT; ++t) wv[j][t] = wp[s * d.groups + grp[t]];
        }
#pragma unroll
        for (int j = 0; j < kScaleRun; ++j) {
          const int s = s0 + j;
          if (s >= d.scales) break;  // uniform
          const View v = cv[s];
          const Tap tp = make_tap(x, y, v);
          float gwt[NT];
          float top[NT];
#pragma unroll
          for (int t = 0; t < NT; ++t) {
            top[t] = g[t] * wv[j][t];
            const float q0 = val[j][0][t], q1 = val[j][1][t], q2 = val[j][2][t],
                        q3 = val[j][3][t];
            gwt[t] = g[t] * (tp.w[0] * q0 + tp.w[1] * q1 + tp.w[2] * q2 + tp.w[3] * q3);
            const float dh = -tp.hw * q0 - tp.lw * q1 + tp.hw * q2 + tp.lw * q3;
            const float dw = -tp.hh * q0 + tp.hh * q1 - tp.lh * q2 + tp.lh * q3;
            gx += static_cast<float>(v.w) * dw * top[t];
            gy += static_cast<float>(v.h) * dh * top[t];
          }
          // feature gradient: one contiguous 256-byte atomic per corner and slot
          // (maps summed by dfa_backward_coarse are left to it)
          if (v.lds < 0 && v.h > 0) {  // uniform across the wavefront
#pragma unroll
            for (int k = 0; k < 4; ++k) {
              if (tp.cell[k] >= 0) {
                float *dst =
                    grad_feat + batch_elem + static_cast<size_t>(v.start + tp.cell[k]) * C + lane;
#pragma unroll
                for (int t = 0; t < NT; ++t) unsafeAtomicAdd(dst + t * kWave, tp.w[k] * top[t]);
              }
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
      }
      gx = wave_sum(gx);
      gy = wave_sum(gy);
      if (lane == l) {
        my_gx = gx;
        my_gy = gy;
      }
    }
    if ((own >> lane) & 1) {
      gl_row[2 * (base + lane)] = my_gx;
      gl_row[2 * (base + lane) + 1] = my_gy;
    }
  }
}

// ------------------------------------------------------ coarse maps ---
//
// Feature gradients of a camera's small maps, summed in LDS. The row kernel
// adds every corner contribution with an fp32 device atomic, and those
// atomics bound it (all of them reach the memory side, ~330 G dwords/s). The
// small maps take as many contributions as the large ones on far fewer cells,
// so a workgroup per (batch entry, camera, run of channels) sums them in LDS,
// CS channels at a time, and adds each cell once. fp32 LDS atomics cost ~194
// clocks per wavefront instruction on gfx950 and 64-bit integer ones 8-14, so
// the sums are fixed point: contribution x = w_corner * (grad_out * weight)
// becomes the integer nearest x * 2^S (an exact float64 product rounded once
// by a fused multiply-add against 1.5 * 2^52, whose low mantissa bits then
// hold the integer). S is chosen per workgroup from a bound on |x| (the
// largest |grad_out| of its channels times the largest weight of its maps,
// both over its active pairs; bilinear weights are at most 1) so that no sum
// of at most 2^pair_log2 contributions passes 2^50: |x| < 2^e gives
// S = 50 - pair_log2 - e. The integer sums are exact and independent of
// order; each contribution is rounded by at most 2^-(S+1), about
// 2^-(51 - pair_log2) of the bound. A workgroup that meets a non-finite
// grad_out or weight adds with fp32 device atomics instead, as the row kernel
// would.

constexpr int kCoarseBlock = 1024;
constexpr int kCoarseLdsBytes = 128 * 1024;  // accumulators of one workgroup
constexpr int kCoarseList = 4096;            // active pairs listed in LDS
constexpr int kCoarseUnroll = 4;             // locations per thread per listing step

// Grid: batch * cams * (C / (CS * ns)) workgroups (runs of ns slices of CS
// channels inside one weight group; run fastest, XCD-contiguous, so an XCD
// serves whole batch entries from its L2); dynamic LDS: budget * CS 64-bit
// sums, channel-major (acc[c * cells + cell]: the lanes of one add, each on a
// random cell, then spread over the banks). The workgroup lists its active
// (anchor, pt) pairs in LDS and holds their locations and weights in
// registers (up to kPer a thread); then, per slice, one thread per pair adds
// every LDS map, corner and channel, and the workgroup adds the sums to
// grad_feat.
template <int CS>
__global__ void __launch_bounds__(kCoarseBlock)
    dfa_backward_coarse(const int32_t *__restrict__ shape, const int32_t *__restrict__ start,
                        const float *__restrict__ loc, const float *__restrict__ weights,
                        const float *__restrict__ grad_out, float *__restrict__ grad_feat,
                        Dims d, int budget, int pair_log2, int ns) {
  static_assert(CS == 4 || CS == 8 || CS == 16, "slices of 4, 8 or 16 channels");
  extern __shared__ unsigned long long acc[];
  __shared__ View views[kMaxViews];
  __shared__ int coarse[kMaxViews];      // the camera's LDS maps (scale indices), by View::lds
  __shared__ int shared_map[kMaxViews];  // 1: the map overlaps another map (atomic adds)
  __shared__ int list[kCoarseList];      // active pairs
  __shared__ int n_coarse, n_used, n_list;
  __shared__ uint32_t max_w_bits, max_g_bits;
  __shared__ int any_bad;
  stage_views(views, shape, start, d);
  mark_coarse(views, d, budget);
  const int C = d.embeds, runs = C / (CS * ns);
  const int lb = msda::xcd_logical_block(static_cast<int>(blockIdx.x), static_cast<int>(gridDim.x));
  const int run = lb % runs, cam = (lb / runs) % d.cams, b = lb / (runs * d.cams);
  const View *cv = views + cam * d.scales;
  const int tid = threadIdx.x, lane = tid % kWave;
  if (tid == 0) {  // the LDS maps in accumulator order
    int n = 0, used = 0;
    for (int s = 0; s < d.scales; ++s) {
      if (cv[s].lds < 0) continue;
      int at = n++;
      for (; at > 0 && cv[coarse[at - 1]].lds > cv[s].lds; --at) coarse[at] = coarse[at - 1];
      coarse[at] = s;
      used += cv[s].h * cv[s].w;
    }
    for (int i = 0; i < n; ++i) shared_map[i] = 0;
    for (int s = n; s < 4; ++s) coarse[s] = 0;  // read (not used) by the unrolled weight loads
    n_coarse = n;
    n_used = used;
    n_list = 0;
    max_w_bits = 0u;
    max_g_bits = 0u;
    any_bad = 0;
  }
  __syncthreads();
  const int nsc = n_coarse, used = n_used;
  if (nsc == 0) return;  // uniform: the camera has no LDS map
  // an LDS map that overlaps another map is added to grad_feat atomically
  const int nviews = d.cams * d.scales;
  for (int t = tid; t < nsc * nviews; t += blockDim.x) {
    const int i = t / nviews, j = t - i * nviews;
    const View &m = cv[coarse[i]];
    const int64_t lo = m.start, hi = lo + static_cast<int64_t>(m.h) * m.w;
    const int64_t olo = views[j].start, ohi = olo + static_cast<int64_t>(views[j].h) * views[j].w;
    if (j != cam * d.scales + coarse[i] && ohi > olo && olo < hi && lo < ohi) shared_map[i] = 1;
  }
  for (int i = tid; i < used * CS; i += blockDim.x) acc[i] = 0ull;

  const int ch0 = run * ns * CS;  // first channel of the run
  const int group = ch0 / (C / d.groups);
  const int sg = d.scales * d.groups;
  const int pairs = d.anchors * d.pts;  // (anchor, pt) pairs of this (batch entry, camera)
  const size_t row0 = static_cast<size_t>(b) * d.anchors;
  auto pair_index = [&](int p) {  // index of (b, anchor, pt, cam) in loc and weights
    const int a = p / d.pts;
    return ((row0 + a) * d.pts + (p - a * d.pts)) * d.cams + cam;
  };
  auto grad_at = [&](int p, int ch) {  // grad_out of the pair's anchor from channel ch
    return reinterpret_cast<const float4 *>(grad_out + (row0 + p / d.pts) * C + ch);
  };
  auto load_weights = [&](int p, float (&w)[4]) {
    const float *wp = weights + pair_index(p) * sg + group;
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = i < nsc ? wp[coarse[i] * d.groups] : 0.0f;
  };
  float mw = 0.0f, mg = 0.0f;
  bool bad = false;
  auto bound_pair = [&](int p, const float (&w)[4]) {  // weights, then the run's grad_out
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float a = fabsf(w[i]);
      bad |= !(a <= FLT_MAX);
      mw = fmaxf(mw, a);
    }
    for (int i = 4; i < nsc; ++i) {  // more than four LDS maps: the rest from memory
      const float a = fabsf(weights[pair_index(p) * sg + group + coarse[i] * d.groups]);
      bad |= !(a <= FLT_MAX);
      mw = fmaxf(mw, a);
    }
    const float4 *go = grad_at(p, ch0);
    for (int q = 0; q < ns * CS / 4; ++q) {
      const float4 g = go[q];
      const float a = fmaxf(fmaxf(fabsf(g.x), fabsf(g.y)), fmaxf(fabsf(g.z), fabsf(g.w)));
      // fmaxf drops NaN (an inf stays in a); a NaN component makes the sum NaN
      const float sum = (g.x + g.y) + (g.z + g.w);
      bad |= !(a <= FLT_MAX) || sum != sum;
      mg = fmaxf(mg, a);
    }
  };

  // 1. list the active pairs (locations only)
  for (int p0 = 0; p0 < pairs; p0 += kCoarseUnroll * kCoarseBlock) {
    float2 xy[kCoarseUnroll];
#pragma unroll
    for (int j = 0; j < kCoarseUnroll; ++j) {
      const int p = min(p0 + j * kCoarseBlock + tid, pairs - 1);
      xy[j] = *reinterpret_cast<const float2 *>(loc + 2 * pair_index(p));
    }
#pragma unroll
    for (int j = 0; j < kCoarseUnroll; ++j) {
      const int p = p0 + j * kCoarseBlock + tid;
      const bool act = p < pairs && active(xy[j].x, xy[j].y);
      const uint64_t m = __ballot(act);
      int base = 0;
      if (lane == 0 && m != 0) base = atomicAdd(&n_list, __popcll(m));
      base = __shfl(base, 0, kWave);
      const int slot =
          base + __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(m >> 32),
                                           __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(m), 0));
      if (act && slot < kCoarseList) list[slot] = p;
    }
  }
  __syncthreads();
  const int listed = n_list;

  // 2. the listed pairs' locations and weights into registers (when they fit)
  // and the bound over them; past that, over every active pair from memory
  constexpr int kPer = CS == 4 ? 3 : CS == 8 ? 2 : 1;
  static_assert(kPer * kCoarseBlock <= kCoarseList, "held pairs come from the list");
  const bool in_regs = listed <= kPer * kCoarseBlock;
  int pp[kPer];
  float2 pxy[kPer];
  float pw[kPer][4];
  if (in_regs) {
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int i = tid + j * kCoarseBlock;
      pp[j] = i < listed ? list[i] : -1;
      if (pp[j] >= 0) {
        pxy[j] = *reinterpret_cast<const float2 *>(loc + 2 * pair_index(pp[j]));
        load_weights(pp[j], pw[j]);
      }
    }
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      if (pp[j] >= 0) bound_pair(pp[j], pw[j]);
    }
  } else {
    for (int p = tid; p < pairs; p += blockDim.x) {
      const float2 xy = *reinterpret_cast<const float2 *>(loc + 2 * pair_index(p));
      if (!active(xy.x, xy.y)) continue;
      float w[4];
      load_weights(p, w);
      bound_pair(p, w);
    }
  }
#pragma unroll
  for (int off = kWave / 2; off > 0; off >>= 1) {
    mw = fmaxf(mw, __shfl_xor(mw, off, kWave));
    mg = fmaxf(mg, __shfl_xor(mg, off, kWave));
  }
  const bool wave_bad = __ballot(bad) != 0;
  if (lane == 0) {  // non-negative floats order as their bit patterns
    atomicMax(&max_w_bits, __float_as_uint(mw));
    atomicMax(&max_g_bits, __float_as_uint(mg));
    if (wave_bad) any_bad = 1;
  }
  __syncthreads();
  const float bound = __uint_as_float(max_g_bits) * __uint_as_float(max_w_bits);
  const bool slow = any_bad != 0 || !(bound <= FLT_MAX);
  if (!slow && bound == 0.0f) return;  // uniform: every contribution is zero
  int e2 = 0;
  (void)frexpf(bound, &e2);  // bound < 2^e2
  const int shift = 50 - pair_log2 - e2;
  const double scale = ldexp(1.0, shift), inv_scale = ldexp(1.0, -shift);
  constexpr double kMagic = 6755399441055744.0;  // 1.5 * 2^52
  const long long magic_bits = __double_as_longlong(kMagic);
  const size_t feat_b = static_cast<size_t>(b) * d.feat;
  int map_end[4];  // accumulator ends of the first four maps
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    map_end[i] = i < nsc ? (cv[coarse[i]].lds + cv[coarse[i]].h * cv[coarse[i]].w) * CS : INT_MAX;
  }

  // 3. every LDS map, corner and channel of one active pair in slice `ch`
  auto add_pair = [&](int p, float2 xy, const float (&g)[CS], const float (&w)[4], int ch) {
    for (int si = 0; si < nsc; ++si) {
      const View v = cv[coarse[si]];
      const float wg = si == 0   ? w[0]
                       : si == 1 ? w[1]
                       : si == 2 ? w[2]
                       : si == 3 ? w[3]
                                 : weights[pair_index(p) * sg + group + coarse[si] * d.groups];
      const Tap tp = make_tap(xy.x, xy.y, v);
      if (slow) {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          if (tp.cell[k] < 0) continue;
          float *dst = grad_feat + (feat_b + v.start + tp.cell[k]) * C + ch;
#pragma unroll
          for (int c = 0; c < CS; ++c) unsafeAtomicAdd(dst + c, tp.w[k] * (g[c] * wg));
        }
        continue;
      }
      double wk[4];
      int at[4];  // accumulator cell of the corner, -1 outside the map
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        wk[k] = tp.w[k];
        at[k] = tp.cell[k] >= 0 ? v.lds + tp.cell[k] : -1;
      }
#pragma unroll
      for (int c = 0; c < CS; ++c) {
        const double tc = static_cast<double>(g[c] * wg) * scale;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          if (at[k] < 0) continue;
          const long long q = __double_as_longlong(fma(wk[k], tc, kMagic)) - magic_bits;
          atomicAdd(acc + c * used + at[k], static_cast<unsigned long long>(q));
        }
      }
    }
  };
  auto load_grad = [&](int p, int ch, float (&g)[CS]) {
    const float4 *go = grad_at(p, ch);
#pragma unroll
    for (int q = 0; q < CS / 4; ++q) {
      const float4 v = go[q];
      g[4 * q] = v.x;
      g[4 * q + 1] = v.y;
      g[4 * q + 2] = v.z;
      g[4 * q + 3] = v.w;
    }
  };

  for (int sl = 0; sl < ns; ++sl) {
    const int ch = ch0 + sl * CS;
    if (in_regs) {
      float pg[kPer][CS];
#pragma unroll
      for (int j = 0; j < kPer; ++j) {
        if (pp[j] >= 0) load_grad(pp[j], ch, pg[j]);
      }
#pragma unroll
      for (int j = 0; j < kPer; ++j) {
        if (pp[j] >= 0) add_pair(pp[j], pxy[j], pg[j], pw[j], ch);
      }
    } else {
      for (int p = tid; p < pairs; p += blockDim.x) {
        const float2 xy = *reinterpret_cast<const float2 *>(loc + 2 * pair_index(p));
        if (!active(xy.x, xy.y)) continue;
        float g[CS], w[4];
        load_weights(p, w);
        load_grad(p, ch, g);
        add_pair(p, xy, g, w, ch);
      }
    }
    if (slow) continue;  // uniform
    __syncthreads();
    // 4. the sums into grad_feat; each accumulator is cleared for the next
    // slice once read. The accumulators are the LDS maps' cells back to back;
    // a thread reads kFlush of them together, so their grad_feat reads
    // overlap. Element offsets fit 32 bits: the row kernels address the
    // feature tensor with 32-bit byte offsets.
    constexpr int kFlush = 8;
    for (int i0 = 0; i0 < used * CS; i0 += kFlush * kCoarseBlock) {
      float old[kFlush], add[kFlush];
      uint32_t off[kFlush];
      uint32_t own = 0u;  // bit j: no other map shares element j's row
#pragma unroll
      for (int j = 0; j < kFlush; ++j) {
        const int i = i0 + j * kCoarseBlock + tid;
        long long q = 0;
        if (i < used * CS) {  // channel-major in LDS: acc[c * used + cell]
          const int a = (i % CS) * used + i / CS;
          q = static_cast<long long>(acc[a]);
          acc[a] = 0ull;
        }
        add[j] = static_cast<float>(static_cast<double>(q) * inv_scale);
        int si = 0;  // the map of accumulator i
        if (nsc > 4) {
          while (si + 1 < nsc &&
                 i >= (cv[coarse[si]].lds + cv[coarse[si]].h * cv[coarse[si]].w) * CS) {
            ++si;
          }
        } else {
          si = (i >= map_end[0]) + (i >= map_end[1]) + (i >= map_end[2]);
        }
        const View &v = cv[coarse[si]];
        off[j] = static_cast<uint32_t>((feat_b + v.start + (i / CS - v.lds)) * C + ch + i % CS);
        const bool mine = shared_map[si] == 0;
        own |= mine ? 1u << j : 0u;
        old[j] = mine && q != 0 ? grad_feat[off[j]] : 0.0f;
      }
#pragma unroll
      for (int j = 0; j < kFlush; ++j) {
        if (add[j] == 0.0f) continue;
        if ((own >> j) & 1u) {
          grad_feat[off[j]] = old[j] + add[j];  // the only writer of this element in this kernel
        } else {
          unsafeAtomicAdd(grad_feat + off[j], add[j]);
        }
      }
    }
    __syncthreads();
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
