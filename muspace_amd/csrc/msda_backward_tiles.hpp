// Tile-owned MSDA backward for MI355X (gfx950): no global atomics.
//
// grad_value[b, cell, m, :] = sum over samples s of (b, m) with a bilinear
// corner at `cell` of  w_corner(s) * attn(s) * grad_out[b, q(s), m, :].
// The reference scatters this with one fp32 global atomic per corner and
// channel (ms_deform_attn_musa_kernel.muh:93-166, 625-733). On MI355X, fp32
// atomics to device memory resolve past the per-XCD L2 (measured ~80-330 G
// dwords/s) and fp32 LDS atomics run at ~0.3 dword/clk/CU, so this path
// instead makes every output cell the property of one workgroup:
//
//   1. bin_count   per (b, m, query chunk): which 16x16 cell tiles each sample
//                  touches (up to 4), per-tile histogram in LDS; also the
//                  per-(b,q,m) max |grad_out| and zero location/weight
//                  gradients for samples that touch no cell.
//   2. bin_scan    per (b, m): exclusive scan of the histograms -> per-chunk
//                  write cursors and per-tile record ranges; zeroes value rows
//                  that belong to no level.
//   3. bin_scatter per chunk: record id (q << lp_log2 | sample) into its tiles.
//   4. tile        per tile (persistent, XCD-ordered): stage the value tile
//                  plus a one-cell halo in LDS, then
//                  pass 1: per owned cell, count and max |contribution| of
//                          its records (LDS u32 add / max, which are fast);
//                  pass 2: contributions rounded to per-cell fixed point
//                          (scale 2^(30 - ceil(log2(count * max)))) and summed
//                          with LDS int32 atomics -- exact, so the result does
//                          not depend on the order of the records; the record
//                          whose top-left corner lies in the tile also computes
//                          grad_attn and grad_sampling_loc from the LDS value
//                          tile (no value gathers from HBM/L2);
//                  write-back: int32 -> float per cell, plain stores.
// grad_value and the two other gradients are fully written (no zero-fill).
#pragma once

#include "msda_device.hpp"

namespace msda {

constexpr int kTileBlock = 512;      // tile kernel workgroup (8 wavefronts)
constexpr int kBinBlock = 256;       // count/scatter workgroup, one query per thread
constexpr int kMaxTilesPerSlab = 16384;  // LDS histogram of the binning kernels

// Host-computed sizes of the binning scratch.
struct BinPlan {
  int chunks;      // query chunks per (b, m)
  int chunk_q;     // queries per chunk (== kBinBlock)
  int tile_bound;  // stride of the per-(b, m) tile arrays (>= tiles per slab)
  int lp_log2;     // record = (q << lp_log2) | sample
  int64_t rec_cap; // record capacity per (b, m) = 4 * queries * lp
};

// Per-level tile table in LDS: level l owns tiles [base[l], base[l+1]).
template <int T>
__device__ __forceinline__ void stage_tiles(const Level *lv, int levels, int *ntc, int *base) {
  if (threadIdx.x == 0) {
    base[0] = 0;
    for (int l = 0; l < levels; ++l) {
      const int nr = (lv[l].h + T - 1) / T, nc = (lv[l].w + T - 1) / T;
      ntc[l] = nc;
      base[l + 1] = base[l] + nr * nc;
    }
  }
  __syncthreads();
}

// Tiles (within the (b, m) slab) holding a valid corner of `t`; the first is
// the primary tile, which holds corner (max(y0,0), max(x0,0)) and with its
// halo all four corners. Returns the number of tiles (0 if no valid corner).
template <int T>
__device__ __forceinline__ int sample_tiles(const Tap &t, int ntc, int base, int (&tiles)[4]) {
  if (!t.in) return 0;
  const int py = t.y0 < 0 ? 0 : t.y0, px = t.x0 < 0 ? 0 : t.x0;
  int n = 0;
  tiles[n++] = base + (py / T) * ntc + px / T;
  const bool ok[4] = {t.y0ok && t.x0ok, t.y0ok && t.x1ok, t.y1ok && t.x0ok, t.y1ok && t.x1ok};
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    if (!ok[c]) continue;
    const int y = t.y0 + (c >> 1), x = t.x0 + (c & 1);
    const int tile = base + (y / T) * ntc + x / T;
    bool seen = false;
    for (int i = 0; i < n; ++i) seen |= tiles[i] == tile;
    if (!seen) tiles[n++] = tile;
  }
  return n;
}

// ------------------------------------------------------------ 1. count ---

template <typename VT, typename GT, int C, int T>
__global__ void __launch_bounds__(kBinBlock)
    msda_bin_count(const int64_t *__restrict__ shapes, const int64_t *__restrict__ starts,
                   const GT *__restrict__ loc, const VT *__restrict__ grad_out, Shape s,
                   BinPlan p, uint32_t *__restrict__ counts, float *__restrict__ gmax,
                   float *__restrict__ grad_loc, float *__restrict__ grad_attn) {
  __shared__ Level lv[kMaxLevels];
  __shared__ int ntc[kMaxLevels], base[kMaxLevels + 1];
  extern __shared__ uint32_t hist[];
  stage_levels(lv, shapes, starts, s);
  stage_tiles<T>(lv, s.levels, ntc, base);
  const int nt = base[s.levels];
  for (int i = threadIdx.x; i < nt; i += blockDim.x) hist[i] = 0;
  __syncthreads();

  const int bm = blockIdx.x / p.chunks, ch = blockIdx.x % p.chunks;
  const int b = bm / s.heads, m = bm % s.heads;
  const int q = ch * p.chunk_q + threadIdx.x;
  if (q < s.queries) {
    const int si = (b * s.queries + q) * s.heads + m;
    float mx = 0.0f;
    const VT *g = grad_out + static_cast<size_t>(si) * C;
    for (int c = 0; c < C; ++c) mx = fmaxf(mx, fabsf(to_float(g[c])));
    gmax[si] = mx;
    const GT *lc = loc + static_cast<size_t>(si) * s.lp * 2;
    for (int smp = 0; smp < s.lp; ++smp) {
      const int l = level_of_sample(smp, s);
      const Tap t = make_tap(to_float(lc[2 * smp]), to_float(lc[2 * smp + 1]), lv[l], true);
      int tiles[4];
      const int n = sample_tiles<T>(t, ntc[l], base[l], tiles);
      if (n == 0) {
        const size_t o = static_cast<size_t>(si) * s.lp + smp;
        grad_attn[o] = 0.0f;
        grad_loc[2 * o] = 0.0f;
        grad_loc[2 * o + 1] = 0.0f;
      }
      for (int i = 0; i < n; ++i) atomicAdd(&hist[tiles[i]], 1u);
    }
  }
  __syncthreads();
  uint32_t *row = counts + static_cast<size_t>(blockIdx.x) * p.tile_bound;
  for (int i = threadIdx.x; i < nt; i += blockDim.x) row[i] = hist[i];
}

// ------------------------------------------------------------- 2. scan ---

template <int C, int T>
__global__ void __launch_bounds__(kBinBlock)
    msda_bin_scan(const int64_t *__restrict__ shapes, const int64_t *__restrict__ starts,
                  Shape s, BinPlan p, uint32_t *__restrict__ counts,
                  uint32_t *__restrict__ tile_start, float *__restrict__ grad_value) {
  __shared__ Level lv[kMaxLevels];
  __shared__ int ntc[kMaxLevels], base[kMaxLevels + 1];
  __shared__ uint32_t part[kBinBlock];
  stage_levels(lv, shapes, starts, s);
  stage_tiles<T>(lv, s.levels, ntc, base);
  const int nt = base[s.levels];
  const int bm = blockIdx.x;
  uint32_t *cnt = counts + static_cast<size_t>(bm) * p.chunks * p.tile_bound;
  uint32_t *ts = tile_start + static_cast<size_t>(bm) * (p.tile_bound + 1);

  // each thread owns a contiguous run of tiles: totals, then a block scan
  const int per = (nt + kBinBlock - 1) / kBinBlock;
  const int t0 = threadIdx.x * per, t1 = min(nt, t0 + per);
  uint32_t run = 0;
  for (int t = t0; t < t1; ++t) {
    uint32_t tot = 0;
    for (int c = 0; c < p.chunks; ++c) tot += cnt[static_cast<size_t>(c) * p.tile_bound + t];
    ts[t] = tot;  // temporarily the total
    run += tot;
  }
  part[threadIdx.x] = run;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t acc = 0;
    for (int i = 0; i < kBinBlock; ++i) {
      const uint32_t v = part[i];
      part[i] = acc;
      acc += v;
    }
    ts[nt] = acc;
  }
  __syncthreads();
  uint32_t off = part[threadIdx.x];
  for (int t = t0; t < t1; ++t) {
    const uint32_t tot = ts[t];
    ts[t] = off;
    uint32_t cur = off;
    for (int c = 0; c < p.chunks; ++c) {
      uint32_t *x = &cnt[static_cast<size_t>(c) * p.tile_bound + t];
      const uint32_t v = *x;
      *x = cur;
      cur += v;
    }
    off += tot;
  }

  // value rows of this (b, m) that belong to no level get a zero gradient
  const int b = bm / s.heads, m = bm % s.heads;
  for (int cell = threadIdx.x; cell < s.spatial; cell += blockDim.x) {
    bool covered = false;
    for (int l = 0; l < s.levels && !covered; ++l) {
      covered = cell >= lv[l].start && cell < lv[l].start + lv[l].h * lv[l].w;
    }
    if (!covered) {
      float *row = grad_value + (static_cast<size_t>(b) * s.spatial + cell) * s.heads * C + m * C;
      for (int c = 0; c < C; ++c) row[c] = 0.0f;
    }
  }
}

// ---------------------------------------------------------- 3. scatter ---

template <typename GT, int T>
__global__ void __launch_bounds__(kBinBlock)
    msda_bin_scatter(const int64_t *__restrict__ shapes, const int64_t *__restrict__ starts,
                     const GT *__restrict__ loc, Shape s, BinPlan p,
                     const uint32_t *__restrict__ counts, uint32_t *__restrict__ records) {
  __shared__ Level lv[kMaxLevels];
  __shared__ int ntc[kMaxLevels], base[kMaxLevels + 1];
  extern __shared__ uint32_t cursor[];
  stage_levels(lv, shapes, starts, s);
  stage_tiles<T>(lv, s.levels, ntc, base);
  const int nt = base[s.levels];
  const uint32_t *row = counts + static_cast<size_t>(blockIdx.x) * p.tile_bound;
  for (int i = threadIdx.x; i < nt; i += blockDim.x) cursor[i] = row[i];
  __syncthreads();

  const int bm = blockIdx.x / p.chunks, ch = blockIdx.x % p.chunks;
  const int b = bm / s.heads, m = bm % s.heads;
  const int q = ch * p.chunk_q + threadIdx.x;
  if (q >= s.queries) return;
  uint32_t *rec = records + static_cast<size_t>(bm) * p.rec_cap;
  const int si = (b * s.queries + q) * s.heads + m;
  const GT *lc = loc + static_cast<size_t>(si) * s.lp * 2;
  for (int smp = 0; smp < s.lp; ++smp) {
    const int l = level_of_sample(smp, s);
    const Tap t = make_tap(to_float(lc[2 * smp]), to_float(lc[2 * smp + 1]), lv[l], true);
    int tiles[4];
    const int n = sample_tiles<T>(t, ntc[l], base[l], tiles);
    const uint32_t id = (static_cast<uint32_t>(q) << p.lp_log2) | static_cast<uint32_t>(smp);
    for (int i = 0; i < n; ++i) rec[atomicAdd(&cursor[tiles[i]], 1u)] = id;
  }
}

// ------------------------------------------------------------- 4. tile ---

template <typename VT, int C>
struct TileLayout {
  static constexpr int kCpl = 16 / sizeof(VT);  // channels per 16-byte lane chunk
  static constexpr int kKq = C / kCpl;          // lanes per record (one cell row)
  // int32 gradient row of a cell, rotated by cell so that the lanes of
  // different records in one instruction spread over the LDS banks
  __device__ static __forceinline__ int gpos(int cell, int ch) {
    return cell * C + ((ch + 4 * (cell & (C / 4 - 1))) & (C - 1));
  }
};

template <int T>
__host__ __device__ constexpr size_t tile_lds_bytes(int c, int value_bytes) {
  return static_cast<size_t>((T + 1) * (T + 1)) * c * value_bytes +  // value tile + halo
         static_cast<size_t>(T * T) * c * 4 +                       // int32 gradient tile
         static_cast<size_t>(T * T) * 12;                           // count, max, exponent
}

template <typename VT, typename GT, int C, int T>
__global__ void __launch_bounds__(kTileBlock)
    msda_tile_backward(const VT *__restrict__ value, const int64_t *__restrict__ shapes,
                       const int64_t *__restrict__ starts, const GT *__restrict__ loc,
                       const GT *__restrict__ attn, const VT *__restrict__ grad_out,
                       const float *__restrict__ gmax, const uint32_t *__restrict__ records,
                       const uint32_t *__restrict__ tile_start, Shape s, BinPlan p,
                       float *__restrict__ grad_value, float *__restrict__ grad_loc,
                       float *__restrict__ grad_attn) {
  using Lay = TileLayout<VT, C>;
  constexpr int CPL = Lay::kCpl, KQ = Lay::kKq, TV = T + 1;
  static_assert(C % CPL == 0 && (KQ & (KQ - 1)) == 0 && KQ <= kWave, "bad tile layout");
  __shared__ Level lv[kMaxLevels];
  __shared__ int ntc[kMaxLevels], base[kMaxLevels + 1];
  extern __shared__ __align__(16) unsigned char lds[];
  VT *vt = reinterpret_cast<VT *>(lds);
  int *gt = reinterpret_cast<int *>(lds + static_cast<size_t>(TV * TV) * C * sizeof(VT));
  uint32_t *ccount = reinterpret_cast<uint32_t *>(gt + T * T * C);
  uint32_t *cmax = ccount + T * T;
  int *cexp = reinterpret_cast<int *>(cmax + T * T);

  stage_levels(lv, shapes, starts, s);
  stage_tiles<T>(lv, s.levels, ntc, base);
  const int nt = base[s.levels];
  const int64_t total = static_cast<int64_t>(s.batch) * s.heads * nt;
  const int MC = s.heads * C;

  // XCD-ordered persistent loop: XCD x walks the x-th eighth of the tiles
  constexpr int kXcd = 8;
  const int x = blockIdx.x % kXcd, per_xcd = gridDim.x / kXcd;
  const int64_t lo = total * x / kXcd, hi = total * (x + 1) / kXcd;
  const int lane = threadIdx.x % kWave;
  const int grp = threadIdx.x / KQ, k = threadIdx.x % KQ;
  const int ngroups = kTileBlock / KQ;

  for (int64_t tid = lo + blockIdx.x / kXcd; tid < hi; tid += per_xcd) {
    const int bm = static_cast<int>(tid / nt), tl = static_cast<int>(tid % nt);
    const int b = bm / s.heads, m = bm % s.heads;
    int l = 0;
    while (base[l + 1] <= tl) ++l;
    const Level L = lv[l];
    const int ty = (tl - base[l]) / ntc[l], tx = (tl - base[l]) % ntc[l];
    const int y_lo = ty * T, x_lo = tx * T;
    const size_t slab = static_cast<size_t>(b) * s.spatial * MC + m * C;

    // stage the value tile (rows y_lo..y_lo+T, cols x_lo..x_lo+T) and clear
    for (int i = threadIdx.x; i < TV * TV * KQ; i += kTileBlock) {
      const int cell = i / KQ, kk = i % KQ;
      const int r = cell / TV, c = cell % TV;
      if (y_lo + r < L.h && x_lo + c < L.w) {
        const VT *src = value + slab +
                        static_cast<size_t>(L.start + (y_lo + r) * L.w + x_lo + c) * MC + kk * CPL;
        *reinterpret_cast<uint4 *>(vt + cell * C + kk * CPL) =
            *reinterpret_cast<const uint4 *>(src);
      }
    }
    for (int i = threadIdx.x; i < T * T * C; i += kTileBlock) gt[i] = 0;
    for (int i = threadIdx.x; i < T * T; i += kTileBlock) {
      ccount[i] = 0;
      cmax[i] = 0;
    }
    __syncthreads();

    const uint32_t r0 = tile_start[static_cast<size_t>(bm) * (p.tile_bound + 1) + tl];
    const uint32_t r1 = tile_start[static_cast<size_t>(bm) * (p.tile_bound + 1) + tl + 1];
    const uint32_t *rec = records + static_cast<size_t>(bm) * p.rec_cap;
    const uint32_t smask = (1u << p.lp_log2) - 1u;

    // pass 1: per owned cell, record count and max |contribution|
    for (uint32_t i = r0 + threadIdx.x; i < r1; i += kTileBlock) {
      const uint32_t id = rec[i];
      const int q = static_cast<int>(id >> p.lp_log2), smp = static_cast<int>(id & smask);
      if (q >= s.queries || smp >= s.lp) continue;  // never true for records bin_scatter wrote
      const size_t si = (static_cast<size_t>(b) * s.queries + q) * s.heads + m;
      const size_t o = si * s.lp + smp;
      const Tap t = make_tap(to_float(loc[2 * o]), to_float(loc[2 * o + 1]), L, true);
      const float mag = fabsf(to_float(attn[o])) * gmax[si];
      const float cw[4] = {t.wy0 * t.wx0, t.wy0 * t.wx1, t.wy1 * t.wx0, t.wy1 * t.wx1};
      const bool ok[4] = {t.y0ok && t.x0ok, t.y0ok && t.x1ok, t.y1ok && t.x0ok, t.y1ok && t.x1ok};
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int yy = t.y0 + (c >> 1) - y_lo, xx = t.x0 + (c & 1) - x_lo;
        if (ok[c] && yy >= 0 && yy < T && xx >= 0 && xx < T) {
          const int cell = yy * T + xx;
          atomicAdd(&ccount[cell], 1u);
          atomicMax(&cmax[cell], __float_as_uint(cw[c] * mag));
        }
      }
    }
    __syncthreads();
    // per-cell fixed-point exponent: count * max * 2^e <= 2^30
    for (int i = threadIdx.x; i < T * T; i += kTileBlock) {
      const float bound = static_cast<float>(ccount[i]) * __uint_as_float(cmax[i]);
      int e = 0;
      if (!(bound <= 3.0e38f)) {
        e = INT_MIN;  // non-finite contributions: the cell's gradient is NaN
      } else if (bound > 0.0f) {
        int ex;
        frexpf(bound, &ex);
        e = 30 - ex;
      }
      cexp[i] = e;
    }
    __syncthreads();

    // pass 2: fixed-point accumulation; the primary record also produces
    // the attention-weight and location gradients from the LDS value tile
    for (uint32_t i0 = r0; i0 < r1; i0 += ngroups) {
      const uint32_t i = i0 + grp;
      const uint32_t raw_id = i < r1 ? rec[i] : rec[r0];
      const int raw_q = static_cast<int>(raw_id >> p.lp_log2);
      const int raw_smp = static_cast<int>(raw_id & smask);
      // the range test never fails for records bin_scatter wrote
      const bool live = i < r1 && raw_q < s.queries && raw_smp < s.lp;
      const int q = live ? raw_q : 0, smp = live ? raw_smp : 0;
      const size_t si = (static_cast<size_t>(b) * s.queries + q) * s.heads + m;
      const size_t o = si * s.lp + smp;
      const Tap t = make_tap(to_float(loc[2 * o]), to_float(loc[2 * o + 1]), L, live);
      const float a = to_float(attn[o]);
      float g[CPL];
      load16(grad_out + si * C + k * CPL, g);
      const float cw[4] = {t.wy0 * t.wx0, t.wy0 * t.wx1, t.wy1 * t.wx0, t.wy1 * t.wx1};
      const bool ok[4] = {t.y0ok && t.x0ok, t.y0ok && t.x1ok, t.y1ok && t.x0ok, t.y1ok && t.x1ok};
      const int py = t.y0 < 0 ? 0 : t.y0, px = t.x0 < 0 ? 0 : t.x0;
      const bool primary = live && t.in && py >= y_lo && py < y_lo + T && px >= x_lo &&
                           px < x_lo + T;
      float ga = 0.0f, gx = 0.0f, gy = 0.0f;
      if (primary) {
        float v[4][CPL];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const int yy = t.y0 + (c >> 1) - y_lo, xx = t.x0 + (c & 1) - x_lo;
          if (ok[c]) {
            load16(vt + (yy * TV + xx) * C + k * CPL, v[c]);
          } else {
#pragma unroll
            for (int j = 0; j < CPL; ++j) v[c][j] = 0.0f;
          }
        }
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
          const float tg = g[j] * a;
          const float val = cw[0] * v[0][j] + cw[1] * v[1][j] + cw[2] * v[2][j] + cw[3] * v[3][j];
          ga += g[j] * val;
          gx += tg * (t.wy0 * (v[1][j] - v[0][j]) + t.wy1 * (v[3][j] - v[2][j]));
          gy += tg * (t.wx0 * (v[2][j] - v[0][j]) + t.wx1 * (v[3][j] - v[1][j]));
        }
      }
      ga = group_sum<KQ>(ga);
      gx = group_sum<KQ>(gx);
      gy = group_sum<KQ>(gy);
      if (primary && k == 0) {
        grad_attn[o] = ga;
        *reinterpret_cast<float2 *>(grad_loc + 2 * o) = make_float2(gx * L.fw, gy * L.fh);
      }
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int yy = t.y0 + (c >> 1) - y_lo, xx = t.x0 + (c & 1) - x_lo;
        if (live && ok[c] && yy >= 0 && yy < T && xx >= 0 && xx < T) {
          const int cell = yy * T + xx;
          const int e = cexp[cell];
          if (e != INT_MIN) {
#pragma unroll
            for (int j = 0; j < CPL; ++j) {
              const int iv = __float2int_rn(ldexpf(cw[c] * (g[j] * a), e));
              atomicAdd(&gt[Lay::gpos(cell, k * CPL + j)], iv);
            }
          }
        }
      }
    }
    __syncthreads();

    // write-back: every owned cell of the level, 4 fp32 channels per lane chunk
    for (int i = threadIdx.x; i < T * T * (C / 4); i += kTileBlock) {
      const int cell = i / (C / 4), c4 = (i % (C / 4)) * 4;
      const int yy = cell / T, xx = cell % T;
      if (y_lo + yy < L.h && x_lo + xx < L.w) {
        const int e = cexp[cell];
        float4 r;
        if (e == INT_MIN) {
          r = make_float4(__int_as_float(0x7fc00000), __int_as_float(0x7fc00000),
                          __int_as_float(0x7fc00000), __int_as_float(0x7fc00000));
        } else {
          r.x = ldexpf(static_cast<float>(gt[Lay::gpos(cell, c4 + 0)]), -e);
          r.y = ldexpf(static_cast<float>(gt[Lay::gpos(cell, c4 + 1)]), -e);
          r.z = ldexpf(static_cast<float>(gt[Lay::gpos(cell, c4 + 2)]), -e);
          r.w = ldexpf(static_cast<float>(gt[Lay::gpos(cell, c4 + 3)]), -e);
        }
        float *dst = grad_value + slab +
                     static_cast<size_t>(L.start + (y_lo + yy) * L.w + x_lo + xx) * MC + c4;
        *reinterpret_cast<float4 *>(dst) = r;
      }
    }
    __syncthreads();
  }
  (void)lane;
}

}  // namespace msda
