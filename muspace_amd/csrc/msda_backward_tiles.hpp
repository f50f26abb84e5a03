// Tile-owned MSDA backward for MI355X (gfx950): no global atomics.
//
// grad_value[b, cell, m, :] = sum over samples s of (b, m) with a bilinear
// corner at `cell` of  w_corner(s) * attn(s) * grad_out[b, q(s), m, :].
// The reference scatters this with one fp32 global atomic per corner and
// channel (ms_deform_attn_musa_kernel.muh:93-166, 625-733). On MI355X, fp32
// atomics to device memory resolve past the per-XCD L2 (measured ~80-330 G
// dwords/s), fp32 LDS atomics run at ~0.3 dword/clk/CU and integer LDS
// atomics stall on bank conflicts, so this path instead makes every output
// cell the property of one workgroup and accumulates in registers:
//
//   1. bin_count   per (b, m, query chunk): which T x T cell tiles each sample
//                  touches (up to 4), per-tile histogram in LDS; zero
//                  location/weight gradients for samples that touch no cell.
//   2. bin_scan    per (b, m): exclusive scan of the histograms -> per-chunk
//                  write cursors and per-tile record ranges; splits tiles
//                  with more than `rmax` records into chunks (work items) so
//                  that a heavily sampled small level is spread over many
//                  CUs, `rmax` adapted to the partial-tile pool; zeroes value
//                  rows that belong to no level.
//   3. bin_scatter per chunk: record id (q << lp_log2 | sample) into its tiles.
//   4. tile        per work item (persistent, XCD-ordered): stage the value
//                  tile plus a one-cell halo in LDS, then
//                  counting-sort its records by top-left corner in LDS and
//                  let each lane group accumulate, in registers, the four
//                  corner sums of the positions it owns (no atomics on the
//                  gradient, see msda_tile_backward); the record whose
//                  top-left corner lies in the tile also computes grad_attn
//                  and grad_sampling_loc from the LDS value tile (no value
//                  gathers from HBM/L2); plain stores to grad_value, or to a
//                  partial tile when the tile was split.
//   5. combine     per split tile: sum its partial tiles in chunk order.
// grad_value and the two other gradients are fully written (no zero-fill).
#pragma once

#include "msda_device.hpp"

namespace msda {

constexpr int kTileBlock = 512;          // tile kernel workgroup (8 wavefronts)
constexpr int kBinBlock = 256;           // binning workgroup
constexpr int kMaxTilesPerSlab = 16384;  // LDS histogram of the binning kernels
constexpr int kCombineBlocksPerSlab = 16;

// Host-computed sizes of the binning scratch (all per (b, m) slab).
struct BinPlan {
  int chunks;      // query chunks per slab
  int chunk_q;     // queries per chunk
  int tile_bound;  // stride of the per-slab tile arrays (>= tiles per slab)
  int lp_log2;     // record = (q << lp_log2) | sample
  int rmax0;       // preferred records per work item
  int slot_cap;    // partial tiles per slab
  int item_cap;    // work items per slab (tile_bound + slot_cap)
  int64_t rec_cap; // record capacity = 4 * queries * lp
};

// Per-slab bookkeeping written by bin_scan.
struct SlabMeta {
  uint32_t rmax, nitems, nmulti, pad;
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

// Block-wide exclusive scan of per-thread run totals (kBinBlock threads);
// returns this thread's offset, writes the grand total to *total.
__device__ __forceinline__ uint32_t block_exclusive(uint32_t run, uint32_t *part, uint32_t *total) {
  part[threadIdx.x] = run;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t acc = 0;
    for (int i = 0; i < kBinBlock; ++i) {
      const uint32_t v = part[i];
      part[i] = acc;
      acc += v;
    }
    *total = acc;
  }
  __syncthreads();
  const uint32_t off = part[threadIdx.x];
  __syncthreads();
  return off;
}

// ------------------------------------------------------------ 1. count ---

template <typename GT, int T>
__global__ void __launch_bounds__(kBinBlock)
    msda_bin_count(const int64_t *__restrict__ shapes, const int64_t *__restrict__ starts,
                   const GT *__restrict__ loc, Shape s, BinPlan p,
                   uint32_t *__restrict__ counts, float *__restrict__ grad_loc,
                   float *__restrict__ grad_attn) {
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
    int tiles[4];
    const int n = sample_tiles<T>(t, ntc[l], base[l], tiles);
    if (n == 0) {
      grad_attn[o] = 0.0f;
      grad_loc[2 * o] = 0.0f;
      grad_loc[2 * o + 1] = 0.0f;
    }
    for (int j = 0; j < n; ++j) atomicAdd(&hist[tiles[j]], 1u);
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
                  uint32_t *__restrict__ tile_start, SlabMeta *__restrict__ meta,
                  uint2 *__restrict__ items, uint32_t *__restrict__ slot_base,
                  uint32_t *__restrict__ multi, float *__restrict__ grad_value) {
  __shared__ Level lv[kMaxLevels];
  __shared__ int ntc[kMaxLevels], base[kMaxLevels + 1];
  __shared__ uint32_t part[kBinBlock];
  __shared__ uint32_t total;
  stage_levels(lv, shapes, starts, s);
  stage_tiles<T>(lv, s.levels, ntc, base);
  const int nt = base[s.levels];
  const int bm = blockIdx.x;
  uint32_t *cnt = counts + static_cast<size_t>(bm) * p.chunks * p.tile_bound;
  uint32_t *ts = tile_start + static_cast<size_t>(bm) * (p.tile_bound + 1);
  uint2 *it = items + static_cast<size_t>(bm) * p.item_cap;
  uint32_t *sb = slot_base + static_cast<size_t>(bm) * p.tile_bound;
  uint32_t *mu = multi + static_cast<size_t>(bm) * p.tile_bound;

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
  uint32_t off = block_exclusive(run, part, &total);
  if (threadIdx.x == 0) ts[nt] = total;
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
  __syncthreads();

  // records per work item: the smallest rmax >= rmax0 whose split tiles fit
  // the slab's partial-tile pool
  uint32_t rmax = static_cast<uint32_t>(p.rmax0);
  for (;;) {
    uint32_t need = 0;
    for (int t = t0; t < t1; ++t) {
      const uint32_t n = ts[t + 1] - ts[t];
      if (n > rmax) need += (n + rmax - 1) / rmax;
    }
    uint32_t slots;
    block_exclusive(need, part, &total);
    slots = total;
    __syncthreads();
    if (slots <= static_cast<uint32_t>(p.slot_cap) || rmax >= (1u << 31)) break;
    rmax *= 2;
  }

  // work items, partial slots and the list of split tiles
  uint32_t n_items = 0, n_slots = 0, n_multi = 0;
  for (int t = t0; t < t1; ++t) {
    const uint32_t n = ts[t + 1] - ts[t];
    const uint32_t c = n > rmax ? (n + rmax - 1) / rmax : 1;
    n_items += c;
    if (c > 1) {
      n_slots += c;
      n_multi += 1;
    }
  }
  uint32_t item_off = block_exclusive(n_items, part, &total);
  const uint32_t items_total = total;
  uint32_t slot_off = block_exclusive(n_slots, part, &total);
  uint32_t multi_off = block_exclusive(n_multi, part, &total);
  const uint32_t multi_total = total;
  for (int t = t0; t < t1; ++t) {
    const uint32_t n = ts[t + 1] - ts[t];
    const uint32_t c = n > rmax ? (n + rmax - 1) / rmax : 1;
    for (uint32_t k = 0; k < c; ++k) it[item_off + k] = make_uint2(t, k);
    item_off += c;
    if (c > 1) {
      sb[t] = slot_off;
      slot_off += c;
      mu[multi_off++] = t;
    }
  }
  if (threadIdx.x == 0) {
    SlabMeta mt;
    mt.rmax = rmax;
    mt.nitems = items_total;
    mt.nmulti = multi_total;
    mt.pad = 0;
    meta[bm] = mt;
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
  const int q0 = ch * p.chunk_q;
  const int nq = min(p.chunk_q, s.queries - q0);
  uint32_t *rec = records + static_cast<size_t>(bm) * p.rec_cap;
  const int lpp = 1 << p.lp_log2;
  for (int i = threadIdx.x; i < nq * lpp; i += blockDim.x) {
    const int q = q0 + (i >> p.lp_log2), smp = i & (lpp - 1);
    if (smp >= s.lp) continue;
    const size_t o = (static_cast<size_t>(b * s.queries + q) * s.heads + m) * s.lp + smp;
    const int l = level_of_sample(smp, s);
    const Tap t = make_tap(to_float(loc[2 * o]), to_float(loc[2 * o + 1]), lv[l], true);
    int tiles[4];
    const int n = sample_tiles<T>(t, ntc[l], base[l], tiles);
    const uint32_t id = (static_cast<uint32_t>(q) << p.lp_log2) | static_cast<uint32_t>(smp);
    for (int j = 0; j < n; ++j) rec[atomicAdd(&cursor[tiles[j]], 1u)] = id;
  }
}

// ------------------------------------------------------------- 4. tile ---

// Tile edge per channel count: four fp32 corner planes of T*T cells, the
// value tile with its halo and the record stash fill about 150 KB of LDS.
template <int C>
struct TileEdge {
  static constexpr int value = C == 16 ? 15 : (C == 32 ? 14 : 10);
};

constexpr int kStash = 1024;  // records sorted per sub-batch

template <int T>
__host__ __device__ constexpr size_t tile_lds_bytes(int c, int value_bytes) {
  return static_cast<size_t>((T + 1) * (T + 1)) * c * value_bytes +  // value tile + halo
         static_cast<size_t>(4 * T * T) * c * 4 +                   // corner planes (fp32)
         static_cast<size_t>(kStash) * 16 +                         // sorted record stash
         static_cast<size_t>((T + 1) * (T + 1)) * 8;                // position count, offset
}

// One work item = a tile of T x T value cells and a range of its records.
// Every record's top-left corner lies on one of the (T+1)^2 positions
// [-1, T-1]^2 around the tile. Records are counting-sorted by position in
// LDS; a lane group owns positions and accumulates, in registers, the four
// corner sums S_p[d] = sum_r w_d(r) * attn(r) * grad_out[q(r)] of its
// positions; each S_p[d] then lands on cell p + d of corner plane d, a cell
// that no other position writes, and the planes are summed per cell. No
// atomic touches the gradient. A record whose top-left corner (clamped to the
// level) is inside the tile is its primary record and also produces the
// attention-weight and location gradients from the LDS value tile.
template <typename VT, typename GT, int C, int T>
__global__ void __launch_bounds__(kTileBlock)
    msda_tile_backward(const VT *__restrict__ value, const int64_t *__restrict__ shapes,
                       const int64_t *__restrict__ starts, const GT *__restrict__ loc,
                       const GT *__restrict__ attn, const VT *__restrict__ grad_out,
                       const uint32_t *__restrict__ records,
                       const uint32_t *__restrict__ tile_start,
                       const SlabMeta *__restrict__ meta, const uint2 *__restrict__ items,
                       const uint32_t *__restrict__ slot_base, Shape s, BinPlan p,
                       float *__restrict__ grad_value, float *__restrict__ partials,
                       float *__restrict__ grad_loc, float *__restrict__ grad_attn) {
  // four channels per lane whatever the storage type, so that the per-lane
  // accumulators fit the register budget of 1024-thread workgroups
  constexpr int CPL = 4, KQ = C / CPL, TV = T + 1, NPOS = TV * TV;
  constexpr int UPC = C * static_cast<int>(sizeof(VT)) / 16;  // 16-byte units per value row
  constexpr int NGROUPS = kTileBlock / KQ;
  constexpr int PPG = (NPOS + NGROUPS - 1) / NGROUPS;  // positions per lane group
  static_assert(C % CPL == 0 && (KQ & (KQ - 1)) == 0 && KQ <= kWave, "bad tile layout");
  __shared__ Level lv[kMaxLevels];
  __shared__ int ntc[kMaxLevels], base[kMaxLevels + 1];
  extern __shared__ __align__(16) unsigned char lds[];
  VT *vt = reinterpret_cast<VT *>(lds);
  float *planes = reinterpret_cast<float *>(lds + static_cast<size_t>(NPOS) * C * sizeof(VT));
  uint4 *stash = reinterpret_cast<uint4 *>(planes + 4 * T * T * C);
  uint32_t *pcount = reinterpret_cast<uint32_t *>(stash + kStash);
  uint32_t *poff = pcount + NPOS;

  stage_levels(lv, shapes, starts, s);
  stage_tiles<T>(lv, s.levels, ntc, base);
  const int MC = s.heads * C;

  constexpr int kXcd = 8;
  const int xcd = blockIdx.x % kXcd, per_xcd = gridDim.x / kXcd;
  const int64_t total = static_cast<int64_t>(s.batch) * s.heads * p.item_cap;
  const int64_t lo = total * xcd / kXcd, hi = total * (xcd + 1) / kXcd;
  const int grp = threadIdx.x / KQ, k = threadIdx.x % KQ;
  const uint32_t smask = (1u << p.lp_log2) - 1u;

  for (int64_t flat = lo + blockIdx.x / kXcd; flat < hi; flat += per_xcd) {
    const int bm = static_cast<int>(flat / p.item_cap);
    const int j = static_cast<int>(flat % p.item_cap);
    const SlabMeta mt = meta[bm];
    if (static_cast<uint32_t>(j) >= mt.nitems) continue;  // uniform across the block
    const uint2 item = items[static_cast<size_t>(bm) * p.item_cap + j];
    const int tl = static_cast<int>(item.x);
    const int b = bm / s.heads, m = bm % s.heads;
    const TileGeom tg = tile_geom(tl, T, ntc, base);
    const Level L = lv[tg.l];
    const int y_lo = tg.y_lo, x_lo = tg.x_lo;
    const size_t slab = static_cast<size_t>(b) * s.spatial * MC + m * C;
    const uint32_t *ts = tile_start + static_cast<size_t>(bm) * (p.tile_bound + 1);
    const uint32_t t_r0 = ts[tl], t_r1 = ts[tl + 1];
    const bool split = t_r1 - t_r0 > mt.rmax;
    const uint32_t r0 = t_r0 + item.y * mt.rmax;
    const uint32_t r1 = min(t_r1, r0 + mt.rmax);
    const uint32_t *rec = records + static_cast<size_t>(bm) * p.rec_cap;

    // stage the value tile (rows y_lo..y_lo+T, cols x_lo..x_lo+T)
    for (int i = threadIdx.x; i < NPOS * UPC; i += kTileBlock) {
      const int cell = i / UPC, kk = i % UPC;
      const int r = cell / TV, c = cell % TV;
      if (y_lo + r < L.h && x_lo + c < L.w) {
        const VT *src = value + slab +
                        static_cast<size_t>(L.start + (y_lo + r) * L.w + x_lo + c) * MC;
        reinterpret_cast<uint4 *>(vt + cell * C)[kk] = reinterpret_cast<const uint4 *>(src)[kk];
      }
    }

    for (int i = threadIdx.x; i < T * T * C; i += kTileBlock) {
      *reinterpret_cast<float4 *>(planes + 4 * i) = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }

    for (uint32_t sb0 = r0; sb0 < r1; sb0 += kStash) {
      const uint32_t sb1 = min(r1, sb0 + kStash);
      for (int i = threadIdx.x; i < NPOS; i += kTileBlock) pcount[i] = 0;
      __syncthreads();
      // sort phase: position and rank of each record of the sub-batch
      uint4 entry[kStash / kTileBlock];
      int pos[kStash / kTileBlock];
      uint32_t rank[kStash / kTileBlock];
#pragma unroll
      for (int u = 0; u < kStash / kTileBlock; ++u) {
        const uint32_t i = sb0 + u * kTileBlock + threadIdx.x;
        pos[u] = -1;
        if (i >= sb1) continue;
        const uint32_t id = rec[i];
        const int q = static_cast<int>(id >> p.lp_log2), smp = static_cast<int>(id & smask);
        if (q >= s.queries || smp >= s.lp) continue;  // never true for records bin_scatter wrote
        const size_t si = (static_cast<size_t>(b) * s.queries + q) * s.heads + m;
        const size_t o = si * s.lp + smp;
        const Tap t = make_tap(to_float(loc[2 * o]), to_float(loc[2 * o + 1]), L, true);
        const int py = t.y0 - y_lo + 1, px = t.x0 - x_lo + 1;
        if (!t.in || py < 0 || py >= TV || px < 0 || px >= TV) continue;  // likewise never
        pos[u] = py * TV + px;
        entry[u] = make_uint4(id, __float_as_uint(t.wx1), __float_as_uint(t.wy1),
                              __float_as_uint(to_float(attn[o])));
        rank[u] = atomicAdd(&pcount[pos[u]], 1u);
      }
      __syncthreads();
      if (threadIdx.x < kWave) {
        // exclusive scan of the position counts by one wavefront
        uint32_t carry = 0;
        for (int c0 = 0; c0 < NPOS; c0 += kWave) {
          const int c = c0 + static_cast<int>(threadIdx.x);
          const uint32_t v = c < NPOS ? pcount[c] : 0u;
          uint32_t incl = v;
#pragma unroll
          for (int d = 1; d < kWave; d <<= 1) {
            const uint32_t up = __shfl_up(incl, d, kWave);
            if (static_cast<int>(threadIdx.x) >= d) incl += up;
          }
          if (c < NPOS) poff[c] = carry + incl - v;
          carry += __shfl(incl, kWave - 1, kWave);
        }
      }
      __syncthreads();
#pragma unroll
      for (int u = 0; u < kStash / kTileBlock; ++u) {
        if (pos[u] >= 0) stash[poff[pos[u]] + rank[u]] = entry[u];
      }
      __syncthreads();

      // owner phase: lane group grp owns positions grp, grp + NGROUPS, ...
#pragma unroll 1
      for (int pp = 0; pp < PPG; ++pp) {
        const int pos_id = grp + pp * NGROUPS;
        const uint32_t n = pos_id < NPOS ? pcount[pos_id] : 0u;
        const uint32_t first = pos_id < NPOS ? poff[pos_id] : 0u;
        const int py = pos_id / TV - 1, px = pos_id % TV - 1;  // tile-local top-left corner
        const int y0 = y_lo + py, x0 = x_lo + px;              // level coordinates
        const bool primary = (y0 < 0 ? 0 : y0) >= y_lo && (y0 < 0 ? 0 : y0) < y_lo + T &&
                             (x0 < 0 ? 0 : x0) >= x_lo && (x0 < 0 ? 0 : x0) < x_lo + T;
        const bool ok[4] = {y0 >= 0 && x0 >= 0, y0 >= 0 && x0 + 1 < L.w,
                            y0 + 1 < L.h && x0 >= 0, y0 + 1 < L.h && x0 + 1 < L.w};
        // the value rows of the four corners (tile-local), when primary
        float v[4][CPL];
        if (primary) {
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            if (ok[c]) {
              load4ch(vt + ((py + (c >> 1)) * TV + px + (c & 1)) * C + k * CPL, v[c]);
            } else {
#pragma unroll
              for (int jj = 0; jj < CPL; ++jj) v[c][jj] = 0.0f;
            }
          }
        }
        // the group's positions hold different record counts: loop to the
        // wave's longest list so the cross-lane sums below see a full wave
        uint32_t n_wave = n;
        for (int d = KQ; d < kWave; d <<= 1) n_wave = max(n_wave, __shfl_xor(n_wave, d, kWave));
        float acc[4][CPL];
#pragma unroll
        for (int d = 0; d < 4; ++d)
#pragma unroll
          for (int jj = 0; jj < CPL; ++jj) acc[d][jj] = 0.0f;
        constexpr int kUnroll = 4;  // records of one position in flight together
        for (uint32_t r0i = 0; r0i < n_wave; r0i += kUnroll) {
          uint4 e[kUnroll];
          float g[kUnroll][CPL];
#pragma unroll
          for (int u = 0; u < kUnroll; ++u) {
            const uint32_t r = r0i + u;
            e[u] = stash[r < n ? first + r : 0u];
            if (r >= n) e[u].w = 0u;  // attention 0: contributes nothing
            const int q = r < n ? static_cast<int>(e[u].x >> p.lp_log2) : 0;
            const size_t si = (static_cast<size_t>(b) * s.queries + q) * s.heads + m;
            load4ch(grad_out + si * C + k * CPL, g[u]);
          }
#pragma unroll
          for (int u = 0; u < kUnroll; ++u) {
            const bool live = r0i + u < n;
            const int q = static_cast<int>(e[u].x >> p.lp_log2);
            const int smp = static_cast<int>(e[u].x & smask);
            const float wx1 = __uint_as_float(e[u].y), wy1 = __uint_as_float(e[u].z);
            const float a = __uint_as_float(e[u].w);
            const float wx0 = 1.0f - wx1, wy0 = 1.0f - wy1;
            const float cw[4] = {wy0 * wx0, wy0 * wx1, wy1 * wx0, wy1 * wx1};
#pragma unroll
            for (int jj = 0; jj < CPL; ++jj) {
              const float tgv = g[u][jj] * a;
#pragma unroll
              for (int d = 0; d < 4; ++d) acc[d][jj] += cw[d] * tgv;
            }
            if (primary) {  // uniform per lane group
              float ga = 0.0f, gx = 0.0f, gy = 0.0f;
#pragma unroll
              for (int jj = 0; jj < CPL; ++jj) {
                const float tgv = g[u][jj] * a;
                const float val = cw[0] * v[0][jj] + cw[1] * v[1][jj] + cw[2] * v[2][jj] +
                                  cw[3] * v[3][jj];
                ga += g[u][jj] * val;
                gx += tgv * (wy0 * (v[1][jj] - v[0][jj]) + wy1 * (v[3][jj] - v[2][jj]));
                gy += tgv * (wx0 * (v[2][jj] - v[0][jj]) + wx1 * (v[3][jj] - v[1][jj]));
              }
              ga = group_sum<KQ>(ga);
              gx = group_sum<KQ>(gx);
              gy = group_sum<KQ>(gy);
              if (live && k == 0) {
                const size_t o =
                    ((static_cast<size_t>(b) * s.queries + q) * s.heads + m) * s.lp + smp;
                // the reference path's gradient of grid_sample w.r.t. a
                // sampling location, for tgv = grad_out * attn
                grad_attn[o] = ga;
                *reinterpret_cast<float2 *>(grad_loc + 2 * o) =
                    make_float2(gx * L.fw, gy * L.fh);
              }
            }
          }
        }
        // add the position's corner sums to its cells of the four planes;
        // cell p + d of plane d belongs to position p alone
        if (n > 0) {
#pragma unroll
          for (int d = 0; d < 4; ++d) {
            const int cy = py + (d >> 1), cx = px + (d & 1);
            if (cy < 0 || cy >= T || cx < 0 || cx >= T) continue;
            float *dst = planes + (d * T * T + cy * T + cx) * C + k * CPL;
#pragma unroll
            for (int jj = 0; jj < CPL; jj += 4) {
              float4 cur = *reinterpret_cast<float4 *>(dst + jj);
              cur.x += acc[d][jj];
              cur.y += acc[d][jj + 1];
              cur.z += acc[d][jj + 2];
              cur.w += acc[d][jj + 3];
              *reinterpret_cast<float4 *>(dst + jj) = cur;
            }
          }
        }
      }
      __syncthreads();
    }

    __syncthreads();

    // write-back: cell sum of the four planes, to grad_value or (split tile)
    // to this chunk's partial tile
    float *part = split ? partials + (static_cast<size_t>(bm) * p.slot_cap +
                                      slot_base[static_cast<size_t>(bm) * p.tile_bound + tl] +
                                      item.y) *
                                         (T * T * C)
                        : nullptr;
    for (int i = threadIdx.x; i < T * T * (C / 4); i += kTileBlock) {
      const int cell = i / (C / 4), c4 = (i % (C / 4)) * 4;
      const int yy = cell / T, xx = cell % T;
      if (y_lo + yy < L.h && x_lo + xx < L.w) {
        float4 r = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          const float4 v = *reinterpret_cast<const float4 *>(planes + (d * T * T + cell) * C + c4);
          r.x += v.x;
          r.y += v.y;
          r.z += v.z;
          r.w += v.w;
        }
        float *dst = split ? part + cell * C + c4
                           : grad_value + slab +
                                 static_cast<size_t>(L.start + (y_lo + yy) * L.w + x_lo + xx) * MC +
                                 c4;
        *reinterpret_cast<float4 *>(dst) = r;
      }
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------- 5. combine ---

// Sum the partial tiles of every split tile in chunk order (deterministic for
// a given split) and store the cells' gradients.
template <int C, int T>
__global__ void __launch_bounds__(kBinBlock)
    msda_tile_combine(const int64_t *__restrict__ shapes, const int64_t *__restrict__ starts,
                      Shape s, BinPlan p, const uint32_t *__restrict__ tile_start,
                      const SlabMeta *__restrict__ meta, const uint32_t *__restrict__ slot_base,
                      const uint32_t *__restrict__ multi, const float *__restrict__ partials,
                      float *__restrict__ grad_value) {
  __shared__ Level lv[kMaxLevels];
  __shared__ int ntc[kMaxLevels], base[kMaxLevels + 1];
  stage_levels(lv, shapes, starts, s);
  stage_tiles<T>(lv, s.levels, ntc, base);
  const int bm = blockIdx.x / kCombineBlocksPerSlab, r = blockIdx.x % kCombineBlocksPerSlab;
  const SlabMeta mt = meta[bm];
  const int b = bm / s.heads, m = bm % s.heads;
  const int MC = s.heads * C;
  const size_t slab = static_cast<size_t>(b) * s.spatial * MC + m * C;
  const uint32_t *ts = tile_start + static_cast<size_t>(bm) * (p.tile_bound + 1);
  for (uint32_t i = 0; i < mt.nmulti; ++i) {
    const int tl = static_cast<int>(multi[static_cast<size_t>(bm) * p.tile_bound + i]);
    const uint32_t n = ts[tl + 1] - ts[tl];
    const uint32_t chunks = (n + mt.rmax - 1) / mt.rmax;
    const float *part0 = partials + (static_cast<size_t>(bm) * p.slot_cap +
                                     slot_base[static_cast<size_t>(bm) * p.tile_bound + tl]) *
                                        (T * T * C);
    const TileGeom tg = tile_geom(tl, T, ntc, base);
    const Level L = lv[tg.l];
    // the slab's blocks split each tile's cells between them
    for (int e = r * blockDim.x + threadIdx.x; e < T * T * (C / 4);
         e += kCombineBlocksPerSlab * blockDim.x) {
      const int cell = e / (C / 4), c4 = (e % (C / 4)) * 4;
      const int yy = cell / T, xx = cell % T;
      if (tg.y_lo + yy >= L.h || tg.x_lo + xx >= L.w) continue;
      float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      for (uint32_t k = 0; k < chunks; ++k) {
        const float4 v =
            *reinterpret_cast<const float4 *>(part0 + static_cast<size_t>(k) * (T * T * C) +
                                              cell * C + c4);
        acc.x += v.x;
        acc.y += v.y;
        acc.z += v.z;
        acc.w += v.w;
      }
      float *dst = grad_value + slab +
                   static_cast<size_t>(L.start + (tg.y_lo + yy) * L.w + tg.x_lo + xx) * MC + c4;
      *reinterpret_cast<float4 *>(dst) = acc;
    }
  }
}

}  // namespace msda
