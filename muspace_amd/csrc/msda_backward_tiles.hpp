// Tile-owned MSDA backward for MI355X (gfx950).
//
// grad_value[b, cell, m, :] = sum over samples s of (b, m) with a bilinear
// corner at `cell` of  w_corner(s) * attn(s) * grad_out[b, q(s), m, :].
// The reference scatters this with one fp32 global atomic per corner and
// channel (ms_deform_attn_musa_kernel.muh:93-166, 625-733). On MI355X, fp32
// atomics to device memory resolve past the per-XCD L2 (measured ~80-330 G
// dwords/s) and fp32 LDS atomics run at ~0.3 dword/clk/CU, so this path makes
// each value cell the property of one T x T cell tile and accumulates in
// registers and plain LDS read-modify-writes:
//
//   1. bin_count   per (b, m, query chunk): the primary tile of every sample
//                  (the tile holding its clamped top-left corner), per-tile
//                  histogram in LDS. Also zeroes the gradients of samples
//                  with no corner inside their level and the tile-boundary
//                  cells of grad_value (see below).
//   2. bin_scan    per (b, m): exclusive scan of the histograms -> per-chunk
//                  write cursors and per-tile record ranges; one work item
//                  per tile, or several of at most `rmax` records for a tile
//                  holding more ("split"); items appended, coarsest level
//                  first, to one compact list; zeroes the cells of empty and
//                  split tiles and the value rows that belong to no level.
//   3. bin_scatter per chunk: 16-byte records {query<<lp_log2 | sample,
//                  location x, location y, attention weight} into their tile.
//   4. tile        persistent, one 1024-thread workgroup per CU, items taken
//                  round-robin inside an XCD's share of the list: stage the
//                  value tile in LDS, then for each batch of K records:
//                  counting sort by top-left corner position in LDS, stage
//                  the grad_out rows, and let lane groups own positions and
//                  accumulate in registers. Records, grad_out rows and the
//                  next value tile are prefetched one or two batches ahead.
//
// Ownership of cells: a record's top-left corner lies on one of the
// (T+1)^2 positions [-1, T-1]^2 of its primary tile, so its corners cover the
// cells [0, T]^2 of that tile's frame: the tile's own T x T cells plus a
// one-cell halo (row T and column T) that belongs to the tiles below and to
// the right. Cells of a tile's first row (column) also receive halo
// contributions from the tile above (to the left) unless the tile touches the
// level's top (left) edge. Those "boundary" cells are zeroed in step 1 and
// every contribution to them, and to all cells of split tiles, is a line-wide
// fp32 global atomic add; every other cell gets one plain store.
// grad_value, grad_sampling_loc and grad_attention_weight are fully written.
#pragma once

#include <type_traits>

#include "msda_device.hpp"

namespace msda {

constexpr int kTileBlock = 1024;         // tile kernel workgroup (16 wavefronts)
constexpr int kBinBlock = 256;           // binning workgroup
constexpr int kMaxTilesPerSlab = 16384;  // LDS histogram of the binning kernels
constexpr int kZeroList = 2048;          // tiles listed for zeroing per slab
constexpr size_t kTileLdsLimit = 160 * 1024;

// Host-computed sizes of the binning scratch (all per (b, m) slab).
struct BinPlan {
  int chunks;       // query chunks per slab
  int chunk_q;      // queries per chunk
  int tile_bound;   // stride of the per-slab tile arrays (>= tiles per slab)
  int lp_log2;      // record id = (q << lp_log2) | sample
  int rmax;         // records per work item (a multiple of the batch size)
  int item_cap;     // capacity of the compact work-item list (all slabs)
  int64_t rec_cap;  // records per slab = queries * lp (one per sample)
};

// One work item: records [r0, r1) of one tile of the (b, m) slab. `tile`
// packs the slab-local tile index (bits 0-15), its level (bits 16-21) and
// the split flag (bit 31: all cells of the tile are added atomically);
// (y_lo, x_lo) is the tile origin in its level.
struct Item {
  uint32_t b, m, tile, r0;
  uint32_t r1, y_lo, x_lo, pad;
};
constexpr uint32_t kSplitBit = 0x80000000u;
constexpr uint32_t kNoRecord = 0xffffffffu;  // sample with no corner inside its level
constexpr uint32_t kTileIndexMask = 0xffffu;

// Tile-kernel configuration per (value type, channels): tile edge T, batch
// size K (records sorted together) and channels per lane CPL. The LDS holds
// the value tile with its halo, four fp32 corner planes, K staged grad_out
// rows, K sorted records, two id buffers and the position counts.
template <typename VT, int C>
struct TileCfg;
template <> struct TileCfg<float, 16> { static constexpr int T = 14, K = 512, CPL = 4; };
template <> struct TileCfg<float, 32> { static constexpr int T = 10, K = 512, CPL = 4; };
template <> struct TileCfg<float, 64> { static constexpr int T = 7, K = 256, CPL = 4; };
template <> struct TileCfg<bf16_t, 16> { static constexpr int T = 14, K = 512, CPL = 4; };
template <> struct TileCfg<bf16_t, 32> { static constexpr int T = 12, K = 512, CPL = 4; };
template <> struct TileCfg<bf16_t, 64> { static constexpr int T = 7, K = 512, CPL = 4; };
template <> struct TileCfg<__half, 16> : TileCfg<bf16_t, 16> {};
template <> struct TileCfg<__half, 32> : TileCfg<bf16_t, 32> {};
template <> struct TileCfg<__half, 64> : TileCfg<bf16_t, 64> {};

template <typename VT, int C>
__host__ __device__ constexpr size_t tile_lds_bytes() {
  constexpr int T = TileCfg<VT, C>::T, K = TileCfg<VT, C>::K, NPOS = (T + 1) * (T + 1);
  return static_cast<size_t>(NPOS + 1) * C * sizeof(VT) +  // value tile + halo, zero row
         static_cast<size_t>(4 * NPOS) * C * 4 +           // corner planes
         static_cast<size_t>(K) * C * sizeof(VT) +         // staged grad_out rows
         static_cast<size_t>(K) * 16 +                     // sorted records
         static_cast<size_t>(2 * K) * 4 +                  // record ids, two batches
         static_cast<size_t>(3 * NPOS) * 4 +               // position count, offset, order
         64 * 4 +                                          // count buckets
         static_cast<size_t>(C) * 4;                       // zero slot
}

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

// Primary tile (slab-local index) of a sample with a corner in its level:
// the tile holding (max(y0, 0), max(x0, 0)).
template <int T>
__device__ __forceinline__ int primary_tile(const Tap &t, int ntc, int base) {
  const int py = t.y0 < 0 ? 0 : t.y0, px = t.x0 < 0 ? 0 : t.x0;
  return base + (py / T) * ntc + px / T;
}

// Tile geometry of slab-local tile index tl.
struct TileGeom {
  int l, y_lo, x_lo;
};

__device__ __forceinline__ TileGeom tile_geom(int tl, int T, const int *ntc, const int *base) {
  TileGeom g;
  g.l = 0;
  while (base[g.l + 1] <= tl) ++g.l;
  const int r = tl - base[g.l];
  g.y_lo = (r / ntc[g.l]) * T;
  g.x_lo = (r % ntc[g.l]) * T;
  return g;
}

__device__ __forceinline__ TileGeom item_geom(const Item &d) {
  return TileGeom{static_cast<int>((d.tile >> 16) & 63u), static_cast<int>(d.y_lo),
                  static_cast<int>(d.x_lo)};
}

// Cell (r, c) of a tile frame (0 <= r, c < T) receives halo contributions
// from a neighbouring tile.
__device__ __forceinline__ bool boundary_cell(int r, int c, const TileGeom &g) {
  return (r == 0 && g.y_lo > 0) || (c == 0 && g.x_lo > 0);
}

// Zero the C floats of each cell (r, c) in [0, T)^2 of tile g that lies
// inside the level and satisfies pick(r, c), with `nthreads` threads.
template <int C, int T, typename Pick>
__device__ __forceinline__ void zero_tile_cells(float *grad_value, size_t slab, int MC,
                                                const Level &L, const TileGeom &g, int tid,
                                                int nthreads, Pick pick) {
  constexpr int C4 = C / 4;
  for (int i = tid; i < T * T * C4; i += nthreads) {
    const int cell = i / C4, c4 = (i % C4) * 4;
    const int r = cell / T, c = cell % T;
    const int y = g.y_lo + r, x = g.x_lo + c;
    if (y >= L.h || x >= L.w || !pick(r, c)) continue;
    *reinterpret_cast<float4 *>(grad_value + slab +
                                static_cast<size_t>(L.start + y * L.w + x) * MC + c4) =
        make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  }
}

// Block-wide exclusive scan of per-thread run totals (kBinBlock threads);
// returns this thread's offset, writes the grand total to *total.
__device__ __forceinline__ uint32_t block_exclusive(uint32_t run, uint32_t *part, uint32_t *total) {
  const int lane = threadIdx.x % kWave, wid = threadIdx.x / kWave;
  uint32_t incl = run;
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    const uint32_t up = __shfl_up(incl, d, kWave);
    if (lane >= d) incl += up;
  }
  if (lane == kWave - 1) part[wid] = incl;
  __syncthreads();
  uint32_t before = 0, all = 0;
  for (int w = 0; w < kBinBlock / kWave; ++w) {
    const uint32_t v = part[w];
    before += w < wid ? v : 0u;
    all += v;
  }
  __syncthreads();
  *total = all;
  return before + incl - run;
}

// ------------------------------------------------------------ 1. count ---

template <typename GT, int C, int T>
__global__ void __launch_bounds__(kBinBlock)
    msda_bin_count(const int64_t *__restrict__ shapes, const int64_t *__restrict__ starts,
                   const GT *__restrict__ loc, Shape s, BinPlan p,
                   uint32_t *__restrict__ counts, uint32_t *__restrict__ item_total,
                   float *__restrict__ grad_value) {
  __shared__ Level lv[kMaxLevels];
  __shared__ int ntc[kMaxLevels], base[kMaxLevels + 1];
  extern __shared__ uint32_t hist[];
  stage_levels(lv, shapes, starts, s);
  stage_tiles<T>(lv, s.levels, ntc, base);
  const int nt = base[s.levels];
  for (int i = threadIdx.x; i < nt; i += blockDim.x) hist[i] = 0;
  if (blockIdx.x == 0 && threadIdx.x == 0) *item_total = 0;
  __syncthreads();

  const int bm = blockIdx.x / p.chunks, ch = blockIdx.x % p.chunks;
  const int b = bm / s.heads, m = bm % s.heads;
  const int q0 = ch * p.chunk_q;
  const int nq = min(p.chunk_q, s.queries - q0);

  // samples: consecutive threads read consecutive locations of a query
  const int lpp = 1 << p.lp_log2;
  for (int i = threadIdx.x; i < nq * lpp; i += blockDim.x) {
    const int q = q0 + (i >> p.lp_log2), smp = i & (lpp - 1);
    if (smp >= s.lp) continue;
    const size_t o = (static_cast<size_t>(b * s.queries + q) * s.heads + m) * s.lp + smp;
    const int l = level_of_sample(smp, s);
    const Tap t = make_tap(to_float(loc[2 * o]), to_float(loc[2 * o + 1]), lv[l], true);
    if (t.in) atomicAdd(&hist[primary_tile<T>(t, ntc[l], base[l])], 1u);
  }

  // boundary cells of the slab's tiles ch, ch + chunks, ...
  const int MC = s.heads * C;
  const size_t slab = static_cast<size_t>(b) * s.spatial * MC + m * C;
  for (int tl = ch; tl < nt; tl += p.chunks) {
    const TileGeom g = tile_geom(tl, T, ntc, base);
    zero_tile_cells<C, T>(grad_value, slab, MC, lv[g.l], g, threadIdx.x, blockDim.x,
                          [&](int r, int c) { return boundary_cell(r, c, g); });
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
                  uint32_t *__restrict__ tile_start, uint32_t *__restrict__ item_total,
                  Item *__restrict__ items, float *__restrict__ grad_value) {
  __shared__ Level lv[kMaxLevels];
  __shared__ int ntc[kMaxLevels], base[kMaxLevels + 1];
  __shared__ uint32_t part[kBinBlock / kWave];
  __shared__ uint32_t item_base, zero_count;
  __shared__ uint32_t zero_list[kZeroList];
  stage_levels(lv, shapes, starts, s);
  stage_tiles<T>(lv, s.levels, ntc, base);
  const int nt = base[s.levels];
  const int bm = blockIdx.x;
  const int b = bm / s.heads, m = bm % s.heads;
  uint32_t *cnt = counts + static_cast<size_t>(bm) * p.chunks * p.tile_bound;
  uint32_t *ts = tile_start + static_cast<size_t>(bm) * (p.tile_bound + 1);
  if (threadIdx.x == 0) zero_count = 0;

  // each thread owns a contiguous run of tiles
  const int per = (nt + kBinBlock - 1) / kBinBlock;
  const int t0 = min(nt, static_cast<int>(threadIdx.x) * per), t1 = min(nt, t0 + per);
  uint32_t run = 0;
  for (int t = t0; t < t1; ++t) {
    uint32_t tot = 0;
    for (int c = 0; c < p.chunks; ++c) tot += cnt[static_cast<size_t>(c) * p.tile_bound + t];
    ts[t] = tot;  // the tile's record count until it is replaced by its offset
    run += tot;
  }
  uint32_t total;
  uint32_t off = block_exclusive(run, part, &total);
  if (threadIdx.x == 0) ts[nt] = total;
  for (int t = t0; t < t1; ++t) {
    const uint32_t n = ts[t];
    ts[t] = off;
    uint32_t cur = off;
    for (int c = 0; c < p.chunks; ++c) {
      uint32_t *x = &cnt[static_cast<size_t>(c) * p.tile_bound + t];
      const uint32_t v = *x;
      *x = cur;
      cur += v;
    }
    off += n;
  }
  __syncthreads();

  // items, tiles in reverse order (coarse, densely sampled levels first);
  // thread i owns reversed positions [u0, u1)
  const uint32_t rmax = static_cast<uint32_t>(p.rmax);
  const int u0 = t0, u1 = t1;
  uint32_t r_items = 0;
  for (int u = u0; u < u1; ++u) {
    const int t = nt - 1 - u;
    r_items += (ts[t + 1] - ts[t] + rmax - 1) / rmax;
  }
  uint32_t slab_items;
  uint32_t item_off = block_exclusive(r_items, part, &slab_items);
  if (threadIdx.x == 0) item_base = atomicAdd(item_total, slab_items);
  __syncthreads();
  item_off += item_base;
  for (int u = u0; u < u1; ++u) {
    const int t = nt - 1 - u;
    const uint32_t a = ts[t], e = ts[t + 1], n = e - a;
    const uint32_t k = (n + rmax - 1) / rmax;
    if (k != 1) {
      const uint32_t z = atomicAdd(&zero_count, 1u);
      if (z < static_cast<uint32_t>(kZeroList)) zero_list[z] = static_cast<uint32_t>(t);
    }
    const TileGeom g = k > 0 ? tile_geom(t, T, ntc, base) : TileGeom{0, 0, 0};
    for (uint32_t j = 0; j < k; ++j) {
      Item it;
      it.b = static_cast<uint32_t>(b);
      it.m = static_cast<uint32_t>(m);
      it.tile = static_cast<uint32_t>(t) | (static_cast<uint32_t>(g.l) << 16) |
                (k > 1 ? kSplitBit : 0u);
      it.r0 = a + j * rmax;
      it.r1 = min(e, it.r0 + rmax);
      it.y_lo = static_cast<uint32_t>(g.y_lo);
      it.x_lo = static_cast<uint32_t>(g.x_lo);
      it.pad = 0;
      if (item_off < static_cast<uint32_t>(p.item_cap)) items[item_off] = it;
      ++item_off;
    }
  }
  __syncthreads();

  // non-boundary cells of empty and split tiles (boundary cells: bin_count)
  const int MC = s.heads * C;
  const size_t slab = static_cast<size_t>(b) * s.spatial * MC + m * C;
  const uint32_t nz = zero_count;
  const bool listed = nz <= static_cast<uint32_t>(kZeroList);
  for (uint32_t i = 0; i < (listed ? nz : static_cast<uint32_t>(nt)); ++i) {
    const int t = listed ? static_cast<int>(zero_list[i]) : static_cast<int>(i);
    if (!listed) {
      const uint32_t n = ts[t + 1] - ts[t];
      if (n != 0 && n <= rmax) continue;
    }
    const TileGeom g = tile_geom(t, T, ntc, base);
    zero_tile_cells<C, T>(grad_value, slab, MC, lv[g.l], g, threadIdx.x, blockDim.x,
                          [&](int r, int c) { return !boundary_cell(r, c, g); });
  }

  // value rows of this (b, m) that belong to no level get a zero gradient
  for (int cell = threadIdx.x; cell < s.spatial; cell += blockDim.x) {
    bool covered = false;
    for (int l = 0; l < s.levels && !covered; ++l) {
      covered = cell >= lv[l].start && cell < lv[l].start + lv[l].h * lv[l].w;
    }
    if (!covered) {
      float *row = grad_value + slab + static_cast<size_t>(cell) * MC;
      for (int c = 0; c < C; c += 4) {
        *reinterpret_cast<float4 *>(row + c) = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      }
    }
  }
}

// ---------------------------------------------------------- 3. scatter ---

template <typename GT, int T>
__global__ void __launch_bounds__(kBinBlock)
    msda_bin_scatter(const int64_t *__restrict__ shapes, const int64_t *__restrict__ starts,
                     const GT *__restrict__ loc, const GT *__restrict__ attn, Shape s, BinPlan p,
                     const uint32_t *__restrict__ counts, uint4 *__restrict__ records,
                     uint32_t *__restrict__ rec_of_sample) {
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
  const int q0 = ch * p.chunk_q;
  const int nq = min(p.chunk_q, s.queries - q0);
  uint4 *rec = records + static_cast<size_t>(bm) * p.rec_cap;
  const int lpp = 1 << p.lp_log2;
  for (int i = threadIdx.x; i < nq * lpp; i += blockDim.x) {
    const int q = q0 + (i >> p.lp_log2), smp = i & (lpp - 1);
    if (smp >= s.lp) continue;
    const size_t o = (static_cast<size_t>(b * s.queries + q) * s.heads + m) * s.lp + smp;
    const int l = level_of_sample(smp, s);
    const float lx = to_float(loc[2 * o]), ly = to_float(loc[2 * o + 1]);
    const Tap t = make_tap(lx, ly, lv[l], true);
    if (!t.in) {
      rec_of_sample[o] = kNoRecord;
      continue;
    }
    const uint32_t id = (static_cast<uint32_t>(q) << p.lp_log2) | static_cast<uint32_t>(smp);
    const uint32_t at = atomicAdd(&cursor[primary_tile<T>(t, ntc[l], base[l])], 1u);
    rec[at] = make_uint4(id, __float_as_uint(lx), __float_as_uint(ly),
                         __float_as_uint(to_float(attn[o])));
    rec_of_sample[o] = at;
  }
}

// ------------------------------------------------------------- 4. tile ---

// Position in one workgroup's batch sequence: item n of its round-robin
// share, batch k of that item, and the item's descriptor.
struct BatchCursor {
  int n;
  uint32_t k;
  Item d;
  bool valid;
};

template <int K>
__device__ __forceinline__ uint32_t item_batches(const Item &d) {
  return (d.r1 - d.r0 + K - 1) / K;
}

// One work item = records [r0, r1) of a tile of T x T value cells. The
// records are processed in batches of K: counting-sorted by top-left corner
// position ((T+1)^2 positions, [-1, T-1]^2 in the tile frame), then lane
// group g owns positions g, g + NG, ... and accumulates, in registers, the
// four corner sums S_p[d] = sum_r w_d(r) * attn(r) * grad_out[q(r)] of each
// of them; S_p[d] is added to slot p of corner plane d (no other group writes
// it). At the end of the item, cell (r, c) sums slot (r - dy, c - dx) of
// plane (dy, dx). Per record, the owner group also produces the attention
// and location gradients from the LDS value tile:
//   D_d = grad_out . v_d (corner value rows), grad_attn = sum_d w_d D_d,
//   grad_ix = attn * (wy0 (D1 - D0) + wy1 (D3 - D2)),
//   grad_iy = attn * (wx0 (D2 - D0) + wx1 (D3 - D1)),
//   grad_loc = (grad_ix * W, grad_iy * H)   (d ix / d loc_x = W)
// which is grid_sample's bilinear backward (zeros padding) regrouped by
// corner.
template <typename VT, int C>
__global__ void __launch_bounds__(kTileBlock)
    msda_tile_backward(const VT *__restrict__ value, const int64_t *__restrict__ shapes,
                       const int64_t *__restrict__ starts, const VT *__restrict__ grad_out,
                       uint4 *__restrict__ records, const Item *__restrict__ items,
                       const uint32_t *__restrict__ item_total, Shape s, BinPlan p,
                       float *__restrict__ grad_value) {
  using Cfg = TileCfg<VT, C>;
  constexpr int T = Cfg::T, K = Cfg::K, CPL = Cfg::CPL;
  constexpr int TV = T + 1, NPOS = TV * TV;
  constexpr int KQ = C / CPL;          // lanes per group
  constexpr int NG = kTileBlock / KQ;  // lane groups
  constexpr int GROWS = K / NG;        // grad_out rows staged per group and batch
  constexpr int VB = static_cast<int>(sizeof(VT));
  constexpr int UPV = C * VB / 16;     // 16-byte units per value row
  constexpr int LANE_B = CPL * VB;     // bytes per lane and grad_out row
  // native vector types (HIP's uint4 is a union wrapper that keeps arrays of
  // it in scratch memory)
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
  using LaneUnit = typename std::conditional<LANE_B == 16, u32x4, u32x2>::type;
  static_assert(CPL == 4 && (KQ & (KQ - 1)) == 0 && KQ <= kWave, "bad lane layout");
  static_assert(NPOS * UPV <= kTileBlock, "value tile: one 16-byte unit per thread");
  static_assert(K <= kTileBlock && K % NG == 0 && NPOS <= kTileBlock, "bad batch size");
  static_assert(tile_lds_bytes<VT, C>() + 3400 <= kTileLdsLimit, "tile LDS budget");

  __shared__ Level lv[kMaxLevels];
  __shared__ int ntc[kMaxLevels], base[kMaxLevels + 1];
  extern __shared__ __align__(16) unsigned char lds[];
  VT *vt = reinterpret_cast<VT *>(lds);  // NPOS cells + one zero row
  float *planes = reinterpret_cast<float *>(lds + static_cast<size_t>(NPOS + 1) * C * VB);
  VT *gst = reinterpret_cast<VT *>(planes + 4 * NPOS * C);
  uint4 *stash = reinterpret_cast<uint4 *>(gst + K * C);
  uint32_t *ids = reinterpret_cast<uint32_t *>(stash + K);  // [2][K]
  uint32_t *pcount = ids + 2 * K;
  uint32_t *poff = pcount + NPOS;
  uint32_t *order = poff + NPOS;
  uint32_t *bucket = order + NPOS;                         // [64]
  float *dummy = reinterpret_cast<float *>(bucket + 64);  // [C], always zero

  stage_levels(lv, shapes, starts, s);
  stage_tiles<T>(lv, s.levels, ntc, base);
  const int MC = s.heads * C;
  const int tid = threadIdx.x;
  const int grp = tid / KQ, k = tid % KQ;

  // this workgroup's items: lo + wid, lo + wid + nw, ... below hi
  constexpr int kXcd = 8;
  const uint32_t n_items = min(*item_total, static_cast<uint32_t>(p.item_cap));
  const int xcd = blockIdx.x % kXcd, wid = blockIdx.x / kXcd, nw = gridDim.x / kXcd;
  const uint32_t lo = static_cast<uint32_t>(static_cast<uint64_t>(n_items) * xcd / kXcd);
  const uint32_t hi = static_cast<uint32_t>(static_cast<uint64_t>(n_items) * (xcd + 1) / kXcd);
  auto item_at = [&](int n, bool &ok) {
    const uint64_t idx = static_cast<uint64_t>(lo) + wid + static_cast<uint64_t>(n) * nw;
    ok = idx < hi;
    Item d{0u, 0u, 0u, 0u, 0u, 0u, 0u, 0u};
    if (ok) d = items[idx];
    return d;
  };

  // cursors of batches b (c0), b + 1 (c1) and b + 2 (c2); `pre` is the
  // descriptor of the item after c2's
  BatchCursor c0;
  c0.n = 0;
  c0.k = 0;
  c0.d = item_at(0, c0.valid);
  if (!c0.valid) return;  // uniform: no item for this workgroup
  bool pre_ok;
  Item pre = item_at(1, pre_ok);
  auto advance = [&](const BatchCursor &c) {
    BatchCursor r = c;
    if (!c.valid) return r;
    if (c.k + 1 < item_batches<K>(c.d)) {
      r.k = c.k + 1;
    } else {
      r.n = c.n + 1;
      r.k = 0;
      r.d = pre;
      r.valid = pre_ok;
      pre = item_at(r.n + 1, pre_ok);
    }
    return r;
  };
  BatchCursor c1 = advance(c0);
  BatchCursor c2 = advance(c1);

  auto batch_range = [&](const BatchCursor &c, uint32_t &s0, uint32_t &s1) {
    s0 = c.d.r0 + c.k * K;
    s1 = min(c.d.r1, s0 + K);
  };
  // Loads below are issued unconditionally (a clamped, always valid address
  // when there is nothing to load) so that no branch separates a prefetch
  // from the code that consumes it a batch later.
  auto load_record = [&](const BatchCursor &c) {
    uint32_t s0, s1;
    batch_range(c, s0, s1);
    const bool ok = c.valid && tid < K && s0 + tid < s1;
    const size_t at =
        ok ? static_cast<size_t>(c.d.b * s.heads + c.d.m) * p.rec_cap + s0 + tid : 0;
    return records[at];
  };
  auto geom = [&](const BatchCursor &c) {
    return item_geom(c.d);
  };
  auto slab_offset = [&](const Item &d) {
    return static_cast<size_t>(d.b) * s.spatial * MC + d.m * C;
  };
  // source of this thread's 16-byte unit of the value tile (cells [0, T]^2)
  // of c's item; `ok` false for cells outside the level (stored as zeros)
  auto value_unit_src = [&](const BatchCursor &c, bool &ok) {
    const TileGeom g = geom(c);
    const Level L = lv[g.l];
    const int u = tid < NPOS * UPV ? tid : 0;
    const int cell = u / UPV, kk = u % UPV;
    const int y = g.y_lo + cell / TV, x = g.x_lo + cell % TV;
    ok = c.valid && tid < NPOS * UPV && y < L.h && x < L.w;
    const size_t at =
        ok ? slab_offset(c.d) + static_cast<size_t>(L.start + y * L.w + x) * MC : 0;
    return reinterpret_cast<const uint4 *>(value + at) + (ok ? kk : 0);
  };
  // source of row grp + j * NG of c's batch of grad_out rows, in record
  // order (record ids read from bid; rows past the batch read row 0)
  auto grow_src = [&](const BatchCursor &c, const uint32_t *bid, int j) {
    uint32_t s0, s1;
    batch_range(c, s0, s1);
    const int ns = c.valid ? static_cast<int>(s1 - s0) : 0;
    const int b = static_cast<int>(c.d.b), m = static_cast<int>(c.d.m);
    const int t = grp + j * NG;
    const int q = t < ns ? static_cast<int>(bid[t] >> p.lp_log2) : 0;
    return reinterpret_cast<const LaneUnit *>(
        grad_out + ((static_cast<size_t>(b) * s.queries + q) * s.heads + m) * C + k * CPL);
  };
  const uint32_t smask = (1u << p.lp_log2) - 1u;
  // location and weight gradients of record t (batch order) of a finished
  // batch, from its sorted slot (stash[slot] = {t, wx1, wy1, attn}) and the
  // D_0..D_3 the owner left at the start of grad_out row t
  auto finish_record = [&](int t, uint32_t slot, const Level &Lf, float &ga, float &gx,
                           float &gy) {
    const uint4 e = stash[slot];
    const float4 D = *reinterpret_cast<const float4 *>(gst + t * C);
    const float wx1 = __uint_as_float(e.y), wy1 = __uint_as_float(e.z);
    const float a = __uint_as_float(e.w);
    const float wx0 = 1.0f - wx1, wy0 = 1.0f - wy1;
    ga = wy0 * (wx0 * D.x + wx1 * D.y) + wy1 * (wx0 * D.z + wx1 * D.w);
    gx = a * (wy0 * (D.y - D.x) + wy1 * (D.w - D.z)) * Lf.fw;
    gy = a * (wx0 * (D.z - D.x) + wx1 * (D.w - D.y)) * Lf.fh;
  };
  // cell sums of a finished item's corner planes to grad_value; every plane
  // slot that maps to a cell of [0, T]^2 is read once and zeroed (slots that
  // map to row or column -1 only ever hold contributions of invalid corners)
  auto write_back = [&](const Item &d) {
    const TileGeom g = item_geom(d);
    const Level Lw = lv[g.l];
    const bool split = (d.tile & kSplitBit) != 0;
    const size_t slab = slab_offset(d);
    for (int i = tid; i < NPOS * C; i += kTileBlock) {
      const int cell = i / C, ch = i % C;
      const int r = cell / TV, c = cell % TV;  // cell (r, c) of [0, T]^2
      float sum = 0.0f;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int pr = r - (q >> 1), pc = c - (q & 1);  // position, >= -1
        float *pl = pr < T && pc < T ? planes + (q * NPOS + (pr + 1) * TV + pc + 1) * C + ch
                                     : dummy + ch;  // always zero
        sum += *pl;
        *pl = 0.0f;
      }
      const int y = g.y_lo + r, x = g.x_lo + c;
      if (y >= Lw.h || x >= Lw.w) continue;
      float *dst = grad_value + slab + static_cast<size_t>(Lw.start + y * Lw.w + x) * MC + ch;
      if (!split && r < T && c < T && !boundary_cell(r, c, g)) {
        *dst = sum;
      } else {
        unsafeAtomicAdd(dst, sum);
      }
    }
  };

  // prologue: batch 0's records, value tile and grad_out rows
  uint4 r_cur = load_record(c0);
  uint4 r_next = load_record(c1);
  {
    bool ok0;
    const uint4 u = *value_unit_src(c0, ok0);
    if (tid < NPOS * UPV) {
      reinterpret_cast<uint4 *>(vt)[tid] = ok0 ? u : make_uint4(0u, 0u, 0u, 0u);
    }
  }
  if (tid < UPV) reinterpret_cast<uint4 *>(vt + NPOS * C)[tid] = make_uint4(0u, 0u, 0u, 0u);
  if (tid < C) dummy[tid] = 0.0f;
  for (int i = tid; i < NPOS * C; i += kTileBlock) {
    reinterpret_cast<float4 *>(planes)[i] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  }
  if (tid < NPOS) pcount[tid] = 0;
  if (tid < K) ids[tid] = r_cur.x;
  __syncthreads();
  LaneUnit gregs[GROWS];
#pragma unroll
  for (int j = 0; j < GROWS; ++j) gregs[j] = *grow_src(c0, ids, j);

  // the previous batch's location/weight gradients of this thread's record,
  // stored over that (consumed) record during the next batch
  int ns_prev = 0;
  size_t f_at = 0;
  float f_ga = 0.0f, f_gx = 0.0f, f_gy = 0.0f;
  bool wb_pending = false;  // the previous batch finished an item
  Item wb_item{0u, 0u, 0u, 0u, 0u, 0u, 0u, 0u};
  for (uint32_t bi = 0; c0.valid; ++bi) {
    const uint32_t *ids_cur = ids + (bi & 1) * K;
    uint32_t *ids_nxt = ids + ((bi + 1) & 1) * K;
    const TileGeom g0 = geom(c0);
    const Level L = lv[g0.l];
    uint32_t s0, s1;
    batch_range(c0, s0, s1);
    const int ns = static_cast<int>(s1 - s0);
    const bool last_of_item = c0.k + 1 == item_batches<K>(c0.d);
    const bool next_new_item = c1.valid && c1.k == 0;

    // A. sort keys of this batch; its grad_out rows into LDS; the next
    // batch's ids; prefetch the batch after next and the next value tile;
    // then the previous batch's gradient stores (after the waits above)
    int pos = -1;
    uint32_t rank = 0;
    uint4 entry = make_uint4(0u, 0u, 0u, 0u);
    if (tid < ns) {
      const Tap t = make_tap(__uint_as_float(r_cur.y), __uint_as_float(r_cur.z), L, true);
      const int py = t.y0 - g0.y_lo + 1, px = t.x0 - g0.x_lo + 1;
      if (t.in && py >= 0 && py < TV && px >= 0 && px < TV) {  // always, for binned records
        pos = py * TV + px;
        entry = make_uint4(static_cast<uint32_t>(tid), __float_as_uint(t.wx1),
                           __float_as_uint(t.wy1), r_cur.w);
        rank = atomicAdd(&pcount[pos], 1u);
      }
    }
#pragma unroll
    for (int j = 0; j < GROWS; ++j) {
      *reinterpret_cast<LaneUnit *>(gst + (grp + j * NG) * C + k * CPL) = gregs[j];
    }
    if (tid < K) ids_nxt[tid] = r_next.x;
    const uint4 r_after = load_record(c2);
    bool v_ok;
    const uint4 v_next = *value_unit_src(c1, v_ok);
    if (tid < ns_prev) {
      records[f_at] = make_uint4(__float_as_uint(f_ga), __float_as_uint(f_gx),
                                 __float_as_uint(f_gy), 0u);
    }
    __syncthreads();

    // B. (one wavefront) exclusive scan of the position counts, then the
    // positions in order of decreasing count (counting sort on min(n, 63))
    if (tid < kWave) {
      uint32_t carry = 0;
      for (int c = 0; c < NPOS; c += kWave) {
        const int i = c + tid;
        const uint32_t v = i < NPOS ? pcount[i] : 0u;
        uint32_t incl = v;
#pragma unroll
        for (int d = 1; d < kWave; d <<= 1) {
          const uint32_t up = __shfl_up(incl, d, kWave);
          if (tid >= d) incl += up;
        }
        if (i < NPOS) poff[i] = carry + incl - v;
        carry += __shfl(incl, kWave - 1, kWave);
      }
      bucket[tid] = 0;
      for (int i = tid; i < NPOS; i += kWave) atomicAdd(&bucket[63 - min(pcount[i], 63u)], 1u);
      const uint32_t v = bucket[tid];
      uint32_t incl = v;
#pragma unroll
      for (int d = 1; d < kWave; d <<= 1) {
        const uint32_t up = __shfl_up(incl, d, kWave);
        if (tid >= d) incl += up;
      }
      bucket[tid] = incl - v;
      for (int i = tid; i < NPOS; i += kWave) {
        order[atomicAdd(&bucket[63 - min(pcount[i], 63u)], 1u)] = static_cast<uint32_t>(i);
      }
    }
    __syncthreads();

    // C. records in position order
    uint32_t my_slot = 0;
    if (pos >= 0) {
      my_slot = poff[pos] + rank;
      stash[my_slot] = entry;
    }
    __syncthreads();

    // D. next batch's grad_out rows in flight; write back the item the
    // previous batch finished; then reduce this batch
#pragma unroll
    for (int j = 0; j < GROWS; ++j) gregs[j] = *grow_src(c1, ids_nxt, j);
    if (wb_pending) {
      write_back(wb_item);
      __syncthreads();
    }
#pragma unroll 1
    for (int i = grp; i < NPOS; i += NG) {
      const int p_id = static_cast<int>(order[i]);
      const uint32_t n = pcount[p_id];
      if (n == 0) break;  // positions are in order of decreasing count
      const uint32_t first = poff[p_id];
      const int py = p_id / TV - 1, px = p_id % TV - 1;  // tile frame, >= -1
      // corner value rows (row -1 or column -1: the zero row after the tile)
      const VT *vrow[4];
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        const int cy = py + (d >> 1), cx = px + (d & 1);
        vrow[d] = vt + ((cy >= 0 && cx >= 0) ? (cy * TV + cx) * C : NPOS * C) + k * CPL;
      }
      float v[4][CPL];
#pragma unroll
      for (int d = 0; d < 4; ++d) load4ch(vrow[d], v[d]);
      float acc[4][CPL];
#pragma unroll
      for (int d = 0; d < 4; ++d)
#pragma unroll
        for (int j = 0; j < CPL; ++j) acc[d][j] = 0.0f;
      uint4 e = stash[first];
      for (uint32_t r = 0; r < n; ++r) {
        const uint4 e_next = stash[first + min(r + 1, n - 1)];
        const int t = static_cast<int>(e.x);
        const float wx1 = __uint_as_float(e.y), wy1 = __uint_as_float(e.z);
        const float a = __uint_as_float(e.w);
        const float wx0 = 1.0f - wx1, wy0 = 1.0f - wy1;
        const float wa[4] = {wy0 * wx0 * a, wy0 * wx1 * a, wy1 * wx0 * a, wy1 * wx1 * a};
        float gv[CPL];
        load4ch(gst + t * C + k * CPL, gv);
        float D[4];
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          float dd = 0.0f;
#pragma unroll
          for (int j = 0; j < CPL; ++j) {
            acc[d][j] += wa[d] * gv[j];
            dd += gv[j] * v[d][j];
          }
          D[d] = group_sum<KQ>(dd);
        }
        // D_0..D_3 replace the start of grad_out row t (read by this group
        // alone, above); the gradients are finished per record in E
        if (k == 0) *reinterpret_cast<float4 *>(gst + t * C) = make_float4(D[0], D[1], D[2], D[3]);
        e = e_next;
      }
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        float4 *dst = reinterpret_cast<float4 *>(planes + (d * NPOS + p_id) * C + k * CPL);
        float4 cur = *dst;
        cur.x += acc[d][0];
        cur.y += acc[d][1];
        cur.z += acc[d][2];
        cur.w += acc[d][3];
        *dst = cur;
      }
    }
    __syncthreads();

    // E. this batch's location/weight gradients (stored in the next A),
    // position counts reset, next value tile staged
    if (tid < ns) {
      finish_record(tid, my_slot, L, f_ga, f_gx, f_gy);
      f_at = static_cast<size_t>(c0.d.b * s.heads + c0.d.m) * p.rec_cap + s0 + tid;
    }
    if (tid < NPOS) pcount[tid] = 0;
    if (next_new_item && tid < NPOS * UPV) {
      reinterpret_cast<uint4 *>(vt)[tid] = v_ok ? v_next : make_uint4(0u, 0u, 0u, 0u);
    }
    ns_prev = ns;
    wb_pending = last_of_item;
    wb_item = c0.d;
    r_cur = r_next;
    r_next = r_after;
    c0 = c1;
    c1 = c2;
    c2 = advance(c2);
    __syncthreads();
  }
  if (tid < ns_prev) {
    records[f_at] = make_uint4(__float_as_uint(f_ga), __float_as_uint(f_gx),
                               __float_as_uint(f_gy), 0u);
  }
  if (wb_pending) write_back(wb_item);
}

// -------------------------------------------------------------- 5. gather ---

// Location and attention-weight gradients in sample order: sample o's
// record slot holds {grad_attn, grad_loc_x, grad_loc_y} after the tile
// kernel. Blocks walk the samples slab by slab (XCD-contiguous), so the
// record reads of one block stay inside one slab's record range and the
// stores are whole lines.
__global__ void __launch_bounds__(kBinBlock)
    msda_grad_gather(const uint32_t *__restrict__ rec_of_sample, const uint4 *__restrict__ records,
                     Shape s, BinPlan p, int blocks_per_slab, float *__restrict__ grad_loc,
                     float *__restrict__ grad_attn) {
  const int lb = xcd_logical_block(static_cast<int>(blockIdx.x), static_cast<int>(gridDim.x));
  const int bm = lb / blocks_per_slab;
  const int j = (lb % blocks_per_slab) * kBinBlock + static_cast<int>(threadIdx.x);
  if (j >= s.queries * s.lp) return;
  const int q = j / s.lp, smp = j % s.lp;
  const int b = bm / s.heads, m = bm % s.heads;
  const size_t o = ((static_cast<size_t>(b) * s.queries + q) * s.heads + m) * s.lp + smp;
  const uint32_t r = rec_of_sample[o];
  float ga = 0.0f, gx = 0.0f, gy = 0.0f;
  if (r != kNoRecord) {
    const uint4 v = records[static_cast<size_t>(bm) * p.rec_cap + r];
    ga = __uint_as_float(v.x);
    gx = __uint_as_float(v.y);
    gy = __uint_as_float(v.z);
  }
  grad_attn[o] = ga;
  *reinterpret_cast<float2 *>(grad_loc + 2 * o) = make_float2(gx, gy);
}

}  // namespace msda
