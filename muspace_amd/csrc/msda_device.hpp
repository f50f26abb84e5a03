// Device-side building blocks of the MI355X (gfx950) MSDA kernels.
//
// Sampling semantics are those of the reference PyTorch path
// (/root/reference/mu_space/ops/multi_scale_deformable_attn.py:26-58): bilinear
// grid_sample with zero padding and align_corners=False on grid = 2*loc - 1.
// The pixel coordinate is evaluated with the exact operation sequence of
// PyTorch's CPU grid_sample, ix = fma(x + 1, W/2, -0.5) with x = 2*loc - 1, so
// that floor(ix) and therefore every corner choice agrees bit-for-bit with
// that path; the reference's MUSA kernel uses loc*W - 0.5 instead
// (/root/reference/csrc/ms_deformable_attn/ms_deform_attn_musa_kernel.muh:286-287),
// which differs in the last bit for about 15% of coordinates.
//
// Corners outside [0,W-1]x[0,H-1] read as zero (grid_sample "zeros" padding).
// The reference kernel additionally skips a whole sample unless
// -1 < h < H and -1 < w < W (…kernel.muh:289); that agrees with per-corner
// padding everywhere except exactly at h == -1 or w == -1, where this code
// follows grid_sample.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#include <climits>

namespace msda {

constexpr int kWave = 64;
constexpr int kMaxLevels = 64;

// Per-level metadata staged in LDS once per workgroup.
struct Level {
  int h, w, start;
  float fh, fw;          // H and W as float (bounds tests, gradient scale)
  float half_h, half_w;  // H/2 and W/2 (grid_sample's unnormalise factor)
};

struct Shape {
  int batch, spatial, heads, channels, levels, queries, points;
  int lp;     // levels * points
  int units;  // batch * queries * heads
  float inv_points;
};

// ---------------------------------------------------------------- dtypes ---

struct bf16_t {
  uint16_t bits;
};

__device__ __forceinline__ float to_float(float v) { return v; }
__device__ __forceinline__ float to_float(__half v) { return __half2float(v); }
__device__ __forceinline__ float to_float(bf16_t v) {
  return __uint_as_float(static_cast<uint32_t>(v.bits) << 16);
}

template <typename T>
__device__ __forceinline__ T from_float(float v);
template <>
__device__ __forceinline__ float from_float<float>(float v) {
  return v;
}
template <>
__device__ __forceinline__ __half from_float<__half>(float v) {
  return __float2half(v);  // round to nearest even
}
template <>
__device__ __forceinline__ bf16_t from_float<bf16_t>(float v) {
  // Round to nearest even; every NaN becomes the canonical quiet NaN 0x7FC0,
  // as torch's float -> bfloat16 conversion does.
  const uint32_t u = __float_as_uint(v);
  bf16_t r;
  if ((u & 0x7fffffffu) > 0x7f800000u) {
    r.bits = 0x7fc0;
  } else {
    r.bits = static_cast<uint16_t>((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
  }
  return r;
}

// 16-byte vector access: 16 / sizeof(T) channels per lane.
__device__ __forceinline__ void load16(const float *p, float (&o)[4]) {
  const float4 v = *reinterpret_cast<const float4 *>(p);
  o[0] = v.x;
  o[1] = v.y;
  o[2] = v.z;
  o[3] = v.w;
}
__device__ __forceinline__ void load16(const bf16_t *p, float (&o)[8]) {
  const uint4 v = *reinterpret_cast<const uint4 *>(p);
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    o[2 * i] = __uint_as_float(w[i] << 16);
    o[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
  }
}
__device__ __forceinline__ void load16(const __half *p, float (&o)[8]) {
  const uint4 v = *reinterpret_cast<const uint4 *>(p);
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    o[2 * i] = __half2float(__ushort_as_half(static_cast<unsigned short>(w[i] & 0xffffu)));
    o[2 * i + 1] = __half2float(__ushort_as_half(static_cast<unsigned short>(w[i] >> 16)));
  }
}

// Four channels per lane: 16 bytes of fp32 or 8 bytes of fp16/bf16.
__device__ __forceinline__ void load4ch(const float *p, float (&o)[4]) { load16(p, o); }
__device__ __forceinline__ void load4ch(const bf16_t *p, float (&o)[4]) {
  const uint2 v = *reinterpret_cast<const uint2 *>(p);
  o[0] = __uint_as_float(v.x << 16);
  o[1] = __uint_as_float(v.x & 0xffff0000u);
  o[2] = __uint_as_float(v.y << 16);
  o[3] = __uint_as_float(v.y & 0xffff0000u);
}
__device__ __forceinline__ void load4ch(const __half *p, float (&o)[4]) {
  const uint2 v = *reinterpret_cast<const uint2 *>(p);
  o[0] = __half2float(__ushort_as_half(static_cast<unsigned short>(v.x & 0xffffu)));
  o[1] = __half2float(__ushort_as_half(static_cast<unsigned short>(v.x >> 16)));
  o[2] = __half2float(__ushort_as_half(static_cast<unsigned short>(v.y & 0xffffu)));
  o[3] = __half2float(__ushort_as_half(static_cast<unsigned short>(v.y >> 16)));
}

__device__ __forceinline__ void store16(float *p, const float (&v)[4]) {
  *reinterpret_cast<float4 *>(p) = make_float4(v[0], v[1], v[2], v[3]);
}
template <typename T>
__device__ __forceinline__ uint16_t bits16(T v);
template <>
__device__ __forceinline__ uint16_t bits16<bf16_t>(bf16_t v) {
  return v.bits;
}
template <>
__device__ __forceinline__ uint16_t bits16<__half>(__half v) {
  return __half_as_ushort(v);
}
template <typename T>
__device__ __forceinline__ void store16(T *p, const float (&v)[8]) {
  uint32_t w[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    w[i] = static_cast<uint32_t>(bits16(from_float<T>(v[2 * i]))) |
           (static_cast<uint32_t>(bits16(from_float<T>(v[2 * i + 1]))) << 16);
  }
  *reinterpret_cast<uint4 *>(p) = make_uint4(w[0], w[1], w[2], w[3]);
}

// Streaming accesses: data read or written once per launch is marked
// non-temporal, so that it does not displace the lines a kernel reuses (the
// gathered value rows) from L2. Measured at c2: forward 424 -> 381 us;
// backward 884 -> 865 us (tile records, results and write-back; bin_count's
// locations). bin_scatter's and grad_gather's streams measured slower marked
// and are left as they are.
typedef uint32_t nt_u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float load_nt(const float *p) { return __builtin_nontemporal_load(p); }
__device__ __forceinline__ float load_nt(const bf16_t *p) {
  const unsigned short b = __builtin_nontemporal_load(reinterpret_cast<const unsigned short *>(p));
  return __uint_as_float(static_cast<uint32_t>(b) << 16);
}
__device__ __forceinline__ float load_nt(const __half *p) {
  const unsigned short b = __builtin_nontemporal_load(reinterpret_cast<const unsigned short *>(p));
  return __half2float(__ushort_as_half(b));
}

__device__ __forceinline__ uint4 load_nt(const uint4 *p) {
  const nt_u32x4 w = __builtin_nontemporal_load(reinterpret_cast<const nt_u32x4 *>(p));
  return make_uint4(w[0], w[1], w[2], w[3]);
}
__device__ __forceinline__ void store_nt(uint4 *p, const uint4 v) {
  const nt_u32x4 w = {v.x, v.y, v.z, v.w};
  __builtin_nontemporal_store(w, reinterpret_cast<nt_u32x4 *>(p));
}

__device__ __forceinline__ void store16_nt(float *p, const float (&v)[4]) {
  const nt_u32x4 w = {__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]),
                      __float_as_uint(v[3])};
  __builtin_nontemporal_store(w, reinterpret_cast<nt_u32x4 *>(p));
}
template <typename T>
__device__ __forceinline__ void store16_nt(T *p, const float (&v)[8]) {
  nt_u32x4 w;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    w[i] = static_cast<uint32_t>(bits16(from_float<T>(v[2 * i]))) |
           (static_cast<uint32_t>(bits16(from_float<T>(v[2 * i + 1]))) << 16);
  }
  __builtin_nontemporal_store(w, reinterpret_cast<nt_u32x4 *>(p));
}

// ------------------------------------------------------- cross-lane sums ---

#define MSDA_DPP(v, ctrl)                                                            \
  __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), (ctrl), 0xF, 0xF, \
                                             false))

// Inclusive prefix sum over the 64 lanes of a wavefront, all in DPP: a
// Kogge-Stone scan inside each 16-lane row (row_shr 1, 2, 4, 8; lanes
// shifted in from outside the row read 0), then row 0's total added to rows
// 1 and 3 and row 1's running total to rows 2 and 3 (row_bcast 15 and 31, a
// row mask picking the rows that receive it). Six VALU instructions instead
// of six LDS-routed shuffles. Must be called with the whole wavefront active.
__device__ __forceinline__ uint32_t wave_inclusive_sum(uint32_t v) {
#define MSDA_DPP_U32(x, ctrl, rows)                                                      \
  static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(x), (ctrl), (rows), \
                                                    0xF, true))
  v += MSDA_DPP_U32(v, 0x111, 0xF);  // row_shr:1
  v += MSDA_DPP_U32(v, 0x112, 0xF);  // row_shr:2
  v += MSDA_DPP_U32(v, 0x114, 0xF);  // row_shr:4
  v += MSDA_DPP_U32(v, 0x118, 0xF);  // row_shr:8
  v += MSDA_DPP_U32(v, 0x142, 0xA);  // row_bcast:15 -> rows 1, 3
  v += MSDA_DPP_U32(v, 0x143, 0xC);  // row_bcast:31 -> rows 2, 3
#undef MSDA_DPP_U32
  return v;
}

// Sum over aligned groups of N consecutive lanes (N a power of two <= 64);
// every lane of the group receives the total. Must be called with the whole
// wavefront active.
template <int N>
__device__ __forceinline__ float group_sum(float v) {
  if constexpr (N >= 2) v += MSDA_DPP(v, 0xB1);   // quad_perm [1,0,3,2]: lane ^ 1
  if constexpr (N >= 4) v += MSDA_DPP(v, 0x4E);   // quad_perm [2,3,0,1]: lane ^ 2
  if constexpr (N >= 8) v += MSDA_DPP(v, 0x141);  // row_half_mirror: other quad of 8
  if constexpr (N >= 16) v += MSDA_DPP(v, 0x140); // row_mirror: other half of 16
  if constexpr (N >= 32) v += __shfl_xor(v, 16, kWave);
  if constexpr (N >= 64) v += __shfl_xor(v, 32, kWave);
  return v;
}

// Max over aligned groups of N consecutive lanes, like group_sum.
template <int N>
__device__ __forceinline__ float group_max(float v) {
  if constexpr (N >= 2) v = fmaxf(v, MSDA_DPP(v, 0xB1));
  if constexpr (N >= 4) v = fmaxf(v, MSDA_DPP(v, 0x4E));
  if constexpr (N >= 8) v = fmaxf(v, MSDA_DPP(v, 0x141));
  if constexpr (N >= 16) v = fmaxf(v, MSDA_DPP(v, 0x140));
  if constexpr (N >= 32) v = fmaxf(v, __shfl_xor(v, 16, kWave));
  if constexpr (N >= 64) v = fmaxf(v, __shfl_xor(v, 32, kWave));
  return v;
}

// The same with the group width n (a power of two <= 64) known at run time;
// n must be uniform across the wavefront. Groups of 32 and 64 combine the
// four 16-lane row totals through readlane (VALU) instead of an LDS-routed
// shuffle.
template <typename Op>
__device__ __forceinline__ float combine_rows(float v, int n, Op op) {
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  const float lo = op(r0, r1), hi = op(r2, r3);
  if (n == 64) return op(lo, hi);
  return (threadIdx.x % kWave) < 32 ? lo : hi;
}

// Branch-free forms for a run-time width n >= 1 (uniform): every DPP step is
// computed and a uniform select keeps it only where n asks for it, so the
// reduction is straight-line code the scheduler can interleave with other work.
template <typename Op>
__device__ __forceinline__ float group_reduce_sel(float v, int n, Op op) {
  float w = op(v, MSDA_DPP(v, 0xB1));
  v = n >= 2 ? w : v;
  w = op(v, MSDA_DPP(v, 0x4E));
  v = n >= 4 ? w : v;
  w = op(v, MSDA_DPP(v, 0x141));
  v = n >= 8 ? w : v;
  w = op(v, MSDA_DPP(v, 0x140));
  v = n >= 16 ? w : v;
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  const float lo = op(r0, r1), hi = op(r2, r3);
  const float wide = n >= 64 ? op(lo, hi) : ((threadIdx.x % kWave) < 32 ? lo : hi);
  return n >= 32 ? wide : v;
}

__device__ __forceinline__ float group_sum_sel(float v, int n) {
  return group_reduce_sel(v, n, [](float x, float y) { return x + y; });
}

__device__ __forceinline__ float group_max_sel(float v, int n) {
  return group_reduce_sel(v, n, [](float x, float y) { return fmaxf(x, y); });
}

__device__ __forceinline__ float group_sum_n(float v, int n) {
  switch (n) {
    case 1: return v;
    case 2: return group_sum<2>(v);
    case 4: return group_sum<4>(v);
    case 8: return group_sum<8>(v);
    case 16: return group_sum<16>(v);
    default:
      return combine_rows(group_sum<16>(v), n, [](float x, float y) { return x + y; });
  }
}

__device__ __forceinline__ float group_max_n(float v, int n) {
  switch (n) {
    case 1: return v;
    case 2: return group_max<2>(v);
    case 4: return group_max<4>(v);
    case 8: return group_max<8>(v);
    case 16: return group_max<16>(v);
    default:
      return combine_rows(group_max<16>(v), n, [](float x, float y) { return fmaxf(x, y); });
  }
}

// ------------------------------------------------------- buffer loads ---

// Raw buffer loads over a tensor of `bytes` bytes: a 16-byte load at an
// offset past the end returns zeros (hardware range check), which the row
// kernels use for bilinear corners outside their level.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));  // an MFMA accumulator
constexpr uint32_t kOobOffset = 0x80000000u;  // past the end of every buffer used here (< 2 GiB)
constexpr uint32_t kBufferWord3 = 0x00020000u;  // raw, untyped 32-bit data

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), static_cast<short>(0),
                                           static_cast<int>(bytes), static_cast<int>(kBufferWord3));
}

__device__ __forceinline__ u32x4 buffer_load16(__amdgpu_buffer_rsrc_t r, uint32_t offset) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, offset, 0, 0);
}

// 16 raw bytes of channels -> floats
__device__ __forceinline__ void decode16(float, u32x4 v, float (&o)[4]) {
  o[0] = __uint_as_float(v.x);
  o[1] = __uint_as_float(v.y);
  o[2] = __uint_as_float(v.z);
  o[3] = __uint_as_float(v.w);
}
__device__ __forceinline__ void decode16(bf16_t, u32x4 v, float (&o)[8]) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    o[2 * i] = __uint_as_float(w[i] << 16);
    o[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
  }
}
__device__ __forceinline__ void decode16(__half, u32x4 v, float (&o)[8]) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    o[2 * i] = __half2float(__ushort_as_half(static_cast<unsigned short>(w[i] & 0xffffu)));
    o[2 * i + 1] = __half2float(__ushort_as_half(static_cast<unsigned short>(w[i] >> 16)));
  }
}

// --------------------------------------------------------------- staging ---

// Copy level metadata into LDS. A level whose cells would fall outside
// [0, spatial), or overlap the cells of an earlier in-range level, is made
// empty (contributes nothing): no kernel reads out of bounds, and every value
// cell belongs to at most one level, which the tile-owned backward relies on.
__device__ __forceinline__ void stage_levels(Level *lv, const int64_t *shapes,
                                             const int64_t *starts, const Shape &s) {
  // [start, end) of each in-range level; end = -1 marks an out-of-range level
  __shared__ int64_t range[kMaxLevels][2];
  for (int l = threadIdx.x; l < s.levels; l += blockDim.x) {
    const int64_t h = shapes[2 * l], w = shapes[2 * l + 1], st = starts[l];
    const bool ok = h >= 0 && w >= 0 && h <= s.spatial && w <= s.spatial && st >= 0 &&
                    st + h * w <= s.spatial;
    range[l][0] = st;
    range[l][1] = ok ? st + h * w : -1;
  }
  __syncthreads();
  for (int l = threadIdx.x; l < s.levels; l += blockDim.x) {
    const int64_t a0 = range[l][0], a1 = range[l][1];
    bool ok = a1 >= 0;
    for (int j = 0; j < l && ok; ++j) {
      const int64_t b0 = range[j][0], b1 = range[j][1];
      ok = !(b1 > b0 && a1 > a0 && a0 < b1 && b0 < a1);  // no cell shared with an earlier level
    }
    Level L;
    L.h = ok ? static_cast<int>(shapes[2 * l]) : 0;
    L.w = ok ? static_cast<int>(shapes[2 * l + 1]) : 0;
    L.start = ok ? static_cast<int>(a0) : 0;
    L.fh = static_cast<float>(L.h);
    L.fw = static_cast<float>(L.w);
    L.half_h = L.fh * 0.5f;
    L.half_w = L.fw * 0.5f;
    lv[l] = L;
  }
  __syncthreads();
}

// ------------------------------------------------------------- geometry ---

// One bilinear sample: corner offsets (in cells, relative to the level's first
// cell) and the four bilinear weights with their validity masks.
struct Tap {
  int x0, y0;              // top-left corner (may be -1); meaningless unless `in`
  int cell00;              // cell index of the top-left corner inside the level
  float wx0, wx1, wy0, wy1;
  bool in;                 // at least one corner inside the level
  bool x0ok, x1ok, y0ok, y1ok;
};

// grid_sample coordinate and corner selection for one sample. `live` false
// makes every corner invalid.
__device__ __forceinline__ Tap make_tap(float loc_x, float loc_y, const Level &L, bool live) {
  // grid = 2*loc - 1 (one rounding, 2*loc is exact), then
  // ix = fma(grid + 1, W/2, -0.5), the sequence PyTorch's CPU grid_sample uses.
  const float gx = 2.0f * loc_x - 1.0f;
  const float gy = 2.0f * loc_y - 1.0f;
  const float ix = __builtin_fmaf(gx + 1.0f, L.half_w, -0.5f);
  const float iy = __builtin_fmaf(gy + 1.0f, L.half_h, -0.5f);
  // Samples with no in-bounds corner (and NaN) are dropped before the float ->
  // int conversion, which keeps the integer corner coordinates small.
  const bool in = live && ix >= -1.0f && ix < L.fw && iy >= -1.0f && iy < L.fh;
  const float fx = floorf(ix), fy = floorf(iy);
  const int x0 = in ? static_cast<int>(fx) : -2;
  const int y0 = in ? static_cast<int>(fy) : -2;
  Tap t;
  t.x0 = x0;
  t.y0 = y0;
  t.in = in;
  // a dropped sample's fractions are 0: its corners all read zero, and a NaN
  // or infinite coordinate (ix - floor(ix) = NaN) would otherwise turn those
  // zeros into NaN (NaN * 0); the reference kernel skips such a sample
  t.wx1 = in ? ix - fx : 0.0f;
  t.wx0 = 1.0f - t.wx1;
  t.wy1 = in ? iy - fy : 0.0f;
  t.wy0 = 1.0f - t.wy1;
  t.x0ok = in && x0 >= 0;
  t.x1ok = in && x0 + 1 < L.w;
  t.y0ok = in && y0 >= 0;
  t.y1ok = in && y0 + 1 < L.h;
  t.cell00 = y0 * L.w + x0;
  return t;
}

// Level of flat sample index smp = l * P + p. Exact for smp < 2^20: (smp + 0.5)/P
// is at least 0.5/P away from an integer.
__device__ __forceinline__ int level_of_sample(int smp, const Shape &s) {
  return static_cast<int>((static_cast<float>(smp) + 0.5f) * s.inv_points);
}

// Workgroup barrier for LDS traffic only: waits for this wavefront's LDS
// operations (lgkmcnt) and meets the other wavefronts, but leaves its global
// loads, stores, atomics and buffer-to-LDS loads in flight. __syncthreads()
// also drains those (vmcnt(0)), which would turn every prefetch issued before
// a barrier into a stall at it. Valid where the wavefronts of a workgroup
// exchange data through LDS only; a buffer-to-LDS load must be waited for
// (vmcnt) by the wavefront that issued it before this barrier publishes it.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0); vmcnt and expcnt left as they are
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Logical block index that gives each XCD a contiguous range of blocks.
// Workgroups are handed to the 8 XCDs round-robin, so physical block i runs
// on XCD i % 8; this bijection on [0, nblk) maps XCD x onto the x-th
// contiguous slice, keeping neighbouring work (same batch and head) inside
// one XCD's L2.
__device__ __forceinline__ int xcd_logical_block(int bid, int nblk) {
  constexpr int kXcd = 8;
  const int x = bid % kXcd, j = bid / kXcd;
  const int q = nblk / kXcd, r = nblk % kXcd;
  return x * q + (x < r ? x : r) + j;
}

}  // namespace msda
