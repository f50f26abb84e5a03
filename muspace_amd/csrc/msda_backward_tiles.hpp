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
//   2. bin_cursors per (b, m) and group of tiles: each tile's histogram
//                  entries -> per-chunk write cursors relative to the tile's
//                  first record, and the tile's record count;
//      bin_scan    per (b, m): exclusive scan of the tile counts -> per-tile
//                  record ranges (writers add a tile's start to its chunk
//                  cursor); one work item
//                  per tile, or several of at most `rmax` records for a tile
//                  holding more ("split"); items appended, coarsest level
//                  first, to one compact list; zeroes the cells of empty and
//                  split tiles and the value rows that belong to no level.
//   3. bin_scatter per chunk: 16-byte records {position << 23 | query <<
//                  lp_log2 | sample, wx1, wy1, attention weight} into their
//                  tile (position: the top-left corner in the tile frame;
//                  wx1, wy1: the bilinear fractions of the sample's tap).
//   4. tile        persistent, one 768-thread workgroup per CU, items taken
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

// Tile kernel workgroup: 12 wavefronts, 3 per SIMD (at most 168 VGPRs; 512
// threads, 2 per SIMD, left the VALU idle half the time: c2 tile kernel
// 652 -> 622 us, c4 bf16 step 3419 -> 3236 us with K = 2304; 1024 threads
// spill to scratch).
constexpr int kTileBlock = 768;
constexpr int kBinBlock = 256;           // binning workgroup
constexpr int kMaxTilesPerSlab = 16384;  // LDS histogram of the binning kernels
constexpr int kZeroList = 2048;          // tiles listed for zeroing per slab
constexpr size_t kTileLdsLimit = 160 * 1024;
constexpr int kXcdQueues = 8;            // item queues of the tile kernel (one per XCD)
constexpr int kPosShift = 23;            // record id bits [23, 32): position in the tile frame
constexpr uint32_t kSampleMask = (1u << kPosShift) - 1u;  // (q << lp_log2) | sample
constexpr uint32_t kNoItem = 0xffffffffu;

// Host-computed sizes of the binning scratch (all per (b, m) slab).
struct BinPlan {
  int chunks;       // query chunks per slab
  int chunk_q;      // queries per chunk (a power of two)
  int count_sub;    // chunks counted by one bin_count block (one histogram row each)
  int tile_bound;   // stride of the per-slab tile arrays (>= tiles per slab)
  int lp_log2;      // record id = (position << kPosShift) | (q << lp_log2) | sample
  int rmax;         // records per work item (a multiple of the batch size)
  int item_cap;     // capacity of the compact work-item list (all slabs)
  int64_t rec_cap;  // records per slab = queries * lp (one per sample)
  // 1: the tile kernel writes each record's location and weight gradients
  // straight to the sample's place (and bin_scatter zeroes samples without a
  // record); 0: it stores them over the record and msda_grad_gather copies
  // them into sample order through rec_of_sample.
  int direct;
  // 1: bin_count keeps its LDS histograms as two 16-bit counters per word
  // (a chunk has fewer than 65536 samples), half the LDS, twice the blocks
  // per CU where the histograms limit them
  int hist16;
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

// Tile-kernel configuration per (value type, channels): tile edge T and
// batch size K (records sorted together); CPL channels per lane. The LDS
// holds the value tile with its halo plus a zero row, four fp32 corner
// planes, K sorted records and the position counts, offsets and order.
template <typename VT, int C>
struct TileCfg;
template <> struct TileCfg<float, 16> { static constexpr int T = 16, K = 2304, CPL = 8; };
template <> struct TileCfg<float, 32> { static constexpr int T = 13, K = 1536, CPL = 8; };
template <> struct TileCfg<float, 64> { static constexpr int T = 8, K = 2304, CPL = 8; };
template <> struct TileCfg<bf16_t, 16> { static constexpr int T = 16, K = 2304, CPL = 8; };
template <> struct TileCfg<bf16_t, 32> { static constexpr int T = 13, K = 2304, CPL = 8; };
template <> struct TileCfg<bf16_t, 64> { static constexpr int T = 9, K = 2304, CPL = 8; };
template <> struct TileCfg<__half, 16> : TileCfg<bf16_t, 16> {};
template <> struct TileCfg<__half, 32> : TileCfg<bf16_t, 32> {};
template <> struct TileCfg<__half, 64> : TileCfg<bf16_t, 64> {};

// Padding after each value-tile cell in LDS (one 16-byte unit): a cell's row
// is 128 bytes in fp32 (64 in 16-bit), a multiple of the bank width, so
// without it the owner groups' reads of 16 different cells started on two
// bank offsets only.
constexpr int kVtPad = 16;

template <typename VT, int C>
__host__ __device__ constexpr size_t tile_lds_bytes() {
  constexpr int T = TileCfg<VT, C>::T, K = TileCfg<VT, C>::K, NPOS = (T + 1) * (T + 1);
  return static_cast<size_t>(NPOS + 1) * (C * sizeof(VT) + kVtPad) +  // value tile, zero row
         static_cast<size_t>(4 * NPOS) * C * 4 +           // corner planes
         static_cast<size_t>(K) * 16 +                     // sorted records
         static_cast<size_t>(4 * NPOS) * 4 +               // position count, offset, rank table
         2 * 64 * 4 +                                      // count buckets, bucket starts
         16 * 4;                                           // per-wavefront count totals
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
  // unsigned division by the constant T (py, px >= 0): a multiply-high and
  // a shift, without the signed form's sign fix-up
  const unsigned py = t.y0 < 0 ? 0u : static_cast<unsigned>(t.y0);
  const unsigned px = t.x0 < 0 ? 0u : static_cast<unsigned>(t.x0);
  return base + static_cast<int>(py / T) * ntc + static_cast<int>(px / T);
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

// Zero the C floats of each boundary cell of tile g (boundary_cell: its
// first row when the tile is not at the level's top, its first column when
// not at the left) inside the level, with `nthreads` threads. The cells are
// enumerated (row 0, then column 0 below it) rather than filtered out of all
// T * T (c4 bf16 step 2754 -> 2742 us).
template <int C, int T>
__device__ __forceinline__ void zero_boundary_cells(float *grad_value, size_t slab, int MC,
                                                    const Level &L, const TileGeom &g, int tid,
                                                    int nthreads) {
  constexpr int C4 = C / 4;
  const int top = g.y_lo > 0 ? 1 : 0, left = g.x_lo > 0 ? 1 : 0;
  const int n_row = top * T, n_col = left * (T - top);
  for (int i = tid; i < (n_row + n_col) * C4; i += nthreads) {
    const int k = i / C4, c4 = (i % C4) * 4;
    const int r = k < n_row ? 0 : top + (k - n_row);
    const int c = k < n_row ? k : 0;
    const int y = g.y_lo + r, x = g.x_lo + c;
    if (y >= L.h || x >= L.w) continue;
    *reinterpret_cast<float4 *>(grad_value + slab +
                                static_cast<size_t>(L.start + y * L.w + x) * MC + c4) =
        make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  }
}

// Block-wide exclusive scan of per-thread run totals (kBinBlock threads);
// returns this thread's offset, writes the grand total to *total. Only LDS
// is exchanged, so the barriers leave global memory operations in flight.
__device__ __forceinline__ uint32_t block_exclusive(uint32_t run, uint32_t *part, uint32_t *total) {
  const int lane = threadIdx.x % kWave, wid = threadIdx.x / kWave;
  const uint32_t incl = wave_inclusive_sum(run);
  if (lane == kWave - 1) part[wid] = incl;
  lds_barrier();
  uint32_t before = 0, all = 0;
  for (int w = 0; w < kBinBlock / kWave; ++w) {
    const uint32_t v = part[w];
    before += w < wid ? v : 0u;
    all += v;
  }
  lds_barrier();
  *total = all;
  return before + incl - run;
}

// ------------------------------------------------------------ 1. count ---

// One block per (b, m) slab and group of count_sub consecutive query chunks:
// a histogram row per chunk (samples per primary tile), written to
// counts[(slab * chunks + chunk) * tile_bound + tile].
template <typename GT, int C, int T>
__global__ void __launch_bounds__(kBinBlock)
    msda_bin_count(const int64_t *__restrict__ shapes, const int64_t *__restrict__ starts,
                   const GT *__restrict__ loc, Shape s, BinPlan p,
                   uint32_t *__restrict__ counts, uint32_t *__restrict__ item_total,
                   float *__restrict__ grad_value) {
  __shared__ Level lv[kMaxLevels];
  __shared__ int ntc[kMaxLevels], base[kMaxLevels + 1];
  // [count_sub][nt] counters: one per word, or (hist16) counter i in the
  // 16-bit half i & 1 of word i >> 1
  extern __shared__ uint32_t hist[];
  stage_levels(lv, shapes, starts, s);
  stage_tiles<T>(lv, s.levels, ntc, base);
  const int nt = base[s.levels];
  const int groups = (p.chunks + p.count_sub - 1) / p.count_sub;
  const int bm = blockIdx.x / groups, grp = blockIdx.x % groups;
  const int ch0 = grp * p.count_sub;
  const int nsub = min(p.count_sub, p.chunks - ch0);
  const bool h16 = p.hist16 != 0;
  const int hwords = h16 ? (nsub * nt + 1) >> 1 : nsub * nt;
  for (int i = threadIdx.x; i < hwords; i += blockDim.x) hist[i] = 0;
  auto count_one = [&](int i) {
    if (h16) {
      atomicAdd(&hist[i >> 1], 1u << ((i & 1) << 4));
    } else {
      atomicAdd(&hist[i], 1u);
    }
  };
  // the item counter and the tile kernel's per-XCD take counters
  if (blockIdx.x == 0 && threadIdx.x <= kXcdQueues) item_total[threadIdx.x] = 0;
  __syncthreads();

  const int b = bm / s.heads, m = bm % s.heads;
  const int q0 = ch0 * p.chunk_q;
  const int nq = min(nsub * p.chunk_q, s.queries - q0);
  const int cq_log2 = __builtin_ctz(static_cast<unsigned>(p.chunk_q));

  // samples: consecutive threads read consecutive locations of a query; U
  // samples per thread in flight (every load unconditional, clamped index)
  const int lpp = 1 << p.lp_log2;
  const int total = nq * lpp;
  constexpr int U = 8;  // 16 measured slower (c2 bin_count 40.5 -> 44.6 us)
  if (lpp <= kBinBlock) {
    // a thread's samples are kBinBlock apart, a multiple of lpp: all have
    // sample index smp = tid % lpp, so its level, level table entries and
    // tile base are loaded once, and a sample's location is a 32-bit offset
    // (queries of the group x floats per query) from the group's first one
    const int smp = static_cast<int>(threadIdx.x) & (lpp - 1);
    const bool smp_ok = smp < s.lp;
    const int l = level_of_sample(smp_ok ? smp : 0, s);
    const Level L = lv[l];
    const int tnc = ntc[l], tbase = base[l];
    const GT *loc_g =
        loc + 2 * ((static_cast<size_t>(b * s.queries + q0) * s.heads + m) * s.lp);
    const uint32_t q_floats = 2u * static_cast<uint32_t>(s.heads * s.lp);
    for (int i0 = threadIdx.x; i0 < total; i0 += kBinBlock * U) {
      float lx[U], ly[U];
      bool live[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int i = i0 + u * kBinBlock;
        live[u] = i < total && smp_ok;
        const uint32_t off = live[u] ? static_cast<uint32_t>(i >> p.lp_log2) * q_floats +
                                           2u * static_cast<uint32_t>(smp)
                                     : 0u;
        lx[u] = load_nt(&loc_g[off]);
        ly[u] = load_nt(&loc_g[off + 1]);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int i = i0 + u * kBinBlock;
        const Tap t = make_tap(lx[u], ly[u], L, live[u]);
        const int row = (i >> p.lp_log2) >> cq_log2;  // chunk of the group
        if (t.in) count_one(row * nt + primary_tile<T>(t, tnc, tbase));
      }
    }
  } else {
    for (int i0 = threadIdx.x; i0 < total; i0 += kBinBlock * U) {
      float lx[U], ly[U];
      bool live[U];
      int smp[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int i = i0 + u * kBinBlock;
        const int q = q0 + (i >> p.lp_log2);
        smp[u] = i & (lpp - 1);
        live[u] = i < total && smp[u] < s.lp;
        const size_t o =
            live[u] ? (static_cast<size_t>(b * s.queries + q) * s.heads + m) * s.lp + smp[u] : 0;
        lx[u] = load_nt(&loc[2 * o]);
        ly[u] = load_nt(&loc[2 * o + 1]);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int i = i0 + u * kBinBlock;
        const int l = level_of_sample(live[u] ? smp[u] : 0, s);
        const Tap t = make_tap(lx[u], ly[u], lv[l], live[u]);
        const int row = (i >> p.lp_log2) >> cq_log2;  // chunk of the group
        if (t.in) count_one(row * nt + primary_tile<T>(t, ntc[l], base[l]));
      }
    }
  }

  // boundary cells of the slab's tiles grp, grp + groups, ...
  const int MC = s.heads * C;
  const size_t slab = static_cast<size_t>(b) * s.spatial * MC + m * C;
  for (int tl = grp; tl < nt; tl += groups) {
    const TileGeom g = tile_geom(tl, T, ntc, base);
    zero_boundary_cells<C, T>(grad_value, slab, MC, lv[g.l], g, threadIdx.x, blockDim.x);
  }
  __syncthreads();
  for (int j = 0; j < nsub; ++j) {
    uint32_t *row = counts + (static_cast<size_t>(bm) * p.chunks + ch0 + j) * p.tile_bound;
    for (int i = threadIdx.x; i < nt; i += blockDim.x) {
      const int k = j * nt + i;
      row[i] = h16 ? (hist[k >> 1] >> ((k & 1) << 4)) & 0xffffu : hist[k];
    }
  }
}

// ---------------------------------------------------------- 2. cursors ---

constexpr int kCurBlockLog2 = 8;
constexpr int kCurBlock = 1 << kCurBlockLog2;  // bin_cursors workgroup

// Per tile of a slab, the per-chunk counts -> each chunk's write cursor
// relative to the tile's first record (exclusive prefix over chunks, in
// place), and the tile's record count to tile_start[slab][tile] (bin_scan
// then turns the counts into the tiles' offsets; the records' writers add
// the tile's offset to its chunk cursor). Grid: slabs x gridDim.y blocks; a
// block takes groups of kCurBlock / S consecutive tiles (group blockIdx.y,
// blockIdx.y + gridDim.y, ...), S threads a tile (S = 1 << seg_log2): thread
// (seg, t) sums and rewrites chunks [seg * per, (seg + 1) * per) of tile t,
// consecutive lanes on consecutive tiles, so each chunk's counts are read
// as one run. One block a slab, a thread a tile, took 18-33 us at the
// benchmark shapes: a slab's counts (chunks x tiles words, up to 160 k at c3)
// went through one CU.
template <int T>
__global__ void __launch_bounds__(kCurBlock)
    msda_bin_cursors(const int64_t *__restrict__ shapes, const int64_t *__restrict__ starts,
                     Shape s, BinPlan p, int seg_log2, uint32_t *__restrict__ counts,
                     uint32_t *__restrict__ tile_start) {
  __shared__ Level lv[kMaxLevels];
  __shared__ int ntc[kMaxLevels], base[kMaxLevels + 1];
  __shared__ uint32_t segsum[kCurBlock];
  stage_levels(lv, shapes, starts, s);
  stage_tiles<T>(lv, s.levels, ntc, base);
  const int nt = base[s.levels];
  const int bm = blockIdx.x;
  const int S = 1 << seg_log2, tpb = kCurBlock >> seg_log2;
  const int tl = static_cast<int>(threadIdx.x) & (tpb - 1);
  const int seg = static_cast<int>(threadIdx.x) >> (kCurBlockLog2 - seg_log2);
  const int per = (p.chunks + S - 1) >> seg_log2;
  const int c0 = seg * per, c1 = min(p.chunks, c0 + per);
  uint32_t *cnt = counts + static_cast<size_t>(bm) * p.chunks * p.tile_bound;
  uint32_t *ts = tile_start + static_cast<size_t>(bm) * (p.tile_bound + 1);
  constexpr int kRound = 16;  // counts in flight per thread
  for (int g = blockIdx.y; g * tpb < nt; g += gridDim.y) {
    const int t = g * tpb + tl;
    const bool ok = t < nt;
    const int tc = ok ? t : nt - 1;  // clamped: every load is issued
    uint32_t sum = 0;
    for (int cb = c0; cb < c1; cb += kRound) {
      uint32_t v[kRound];
#pragma unroll
      for (int j = 0; j < kRound; ++j) {
        v[j] = cnt[static_cast<size_t>(min(cb + j, p.chunks - 1)) * p.tile_bound + tc];
      }
#pragma unroll
      for (int j = 0; j < kRound; ++j) sum += cb + j < c1 ? v[j] : 0u;
    }
    segsum[threadIdx.x] = sum;
    lds_barrier();
    uint32_t before = 0, total = 0;
    for (int k = 0; k < S; ++k) {
      const uint32_t v = segsum[k * tpb + tl];
      before += k < seg ? v : 0u;
      total += v;
    }
    if (ok && seg == 0) ts[t] = total;
    uint32_t cur = before;
    for (int cb = c0; cb < c1; cb += kRound) {
      uint32_t v[kRound];
#pragma unroll
      for (int j = 0; j < kRound; ++j) {
        v[j] = cnt[static_cast<size_t>(min(cb + j, p.chunks - 1)) * p.tile_bound + tc];
      }
#pragma unroll
      for (int j = 0; j < kRound; ++j) {
        if (ok && cb + j < c1) {
          cnt[static_cast<size_t>(cb + j) * p.tile_bound + t] = cur;
          cur += v[j];
        }
      }
    }
    lds_barrier();  // segsum is rewritten by the next group
  }
}

// ------------------------------------------------------------- 2. scan ---

template <int C, int T>
__global__ void __launch_bounds__(kBinBlock)
    msda_bin_scan(const int64_t *__restrict__ shapes, const int64_t *__restrict__ starts,
                  Shape s, BinPlan p, uint32_t *__restrict__ tile_start,
                  uint32_t *__restrict__ item_total,
                  Item *__restrict__ items, uint32_t *__restrict__ zero_tiles,
                  float *__restrict__ grad_value) {
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
  uint32_t *ts = tile_start + static_cast<size_t>(bm) * (p.tile_bound + 1);
  if (threadIdx.x == 0) zero_count = 0;

  // each thread owns a contiguous run of tiles: their record counts
  // (bin_cursors) -> their offsets in the slab's records
  const int per = (nt + kBinBlock - 1) / kBinBlock;
  const int t0 = min(nt, static_cast<int>(threadIdx.x) * per), t1 = min(nt, t0 + per);
  uint32_t run = 0;
  for (int t = t0; t < t1; ++t) run += ts[t];
  uint32_t total;
  uint32_t off = block_exclusive(run, part, &total);
  if (threadIdx.x == 0) ts[nt] = total;
  for (int t = t0; t < t1; ++t) {
    const uint32_t n = ts[t];
    ts[t] = off;
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

  // empty and split tiles, whose non-boundary cells bin_scatter zeroes
  // (boundary cells: bin_count); zero_tiles[slab] = {count, tile...}
  uint32_t *zl = zero_tiles + static_cast<size_t>(bm) * (p.tile_bound + 1);
  const uint32_t nz = zero_count;
  if (nz <= static_cast<uint32_t>(kZeroList)) {
    for (uint32_t i = threadIdx.x; i < nz; i += blockDim.x) zl[1 + i] = zero_list[i];
    if (threadIdx.x == 0) zl[0] = nz;
  } else if (threadIdx.x == 0) {
    uint32_t n = 0;
    for (int t = 0; t < nt; ++t) {
      const uint32_t c = ts[t + 1] - ts[t];
      if (c == 0 || c > rmax) zl[1 + n++] = static_cast<uint32_t>(t);
    }
    zl[0] = n;
  }

  const int MC = s.heads * C;
  const size_t slab = static_cast<size_t>(b) * s.spatial * MC + m * C;
  // value rows of this (b, m) that belong to no level get a zero gradient
  // (none when the levels tile [0, spatial), the usual case: valid levels
  // do not overlap, so covering `spatial` cells means covering them all)
  int64_t covered_cells = 0;
  for (int l = 0; l < s.levels; ++l) covered_cells += static_cast<int64_t>(lv[l].h) * lv[l].w;
  if (covered_cells == s.spatial) return;
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

// Samples per sub-chunk of bin_scatter (a power of two; the chunk's queries
// are processed kScatterSlots >> lp_log2 at a time).
constexpr int kScatterSlots = 2048;
constexpr int kScatterPerThread = kScatterSlots / kBinBlock;

__host__ __device__ constexpr size_t scatter_lds_bytes(int tile_bound) {
  return static_cast<size_t>(kScatterSlots) * 16 +       // records in arrival order
         static_cast<size_t>(kScatterSlots) * 4 +        // tile-sorted slot list
         static_cast<size_t>(2 * (tile_bound + 1)) * 4;  // write cursors, local offsets
}

// Writes each sample's 16-byte record into its tile's range and its record
// index into the sample -> record map. A sub-chunk's records are first
// ranked per tile and staged in LDS in arrival order, then written out in
// tile order, so consecutive threads store consecutive records of one
// tile's run (whole lines instead of one scattered 16-byte piece per lane).
template <typename GT, int C, int T>
__global__ void __launch_bounds__(kBinBlock)
    msda_bin_scatter(const int64_t *__restrict__ shapes, const int64_t *__restrict__ starts,
                     const GT *__restrict__ loc, const GT *__restrict__ attn, Shape s, BinPlan p,
                     const uint32_t *__restrict__ counts,
                     const uint32_t *__restrict__ tile_start,
                     const uint32_t *__restrict__ zero_tiles,
                     uint4 *__restrict__ records, uint32_t *__restrict__ rec_of_sample,
                     float *__restrict__ grad_loc, float *__restrict__ grad_attn,
                     float *__restrict__ grad_value) {
  __shared__ Level lv[kMaxLevels];
  __shared__ int ntc[kMaxLevels], base[kMaxLevels + 1];
  __shared__ uint32_t part[kBinBlock / kWave];
  extern __shared__ __align__(16) unsigned char dyn[];
  uint4 *stage = reinterpret_cast<uint4 *>(dyn);                       // [kScatterSlots]
  uint32_t *sorted = reinterpret_cast<uint32_t *>(stage + kScatterSlots);  // [kScatterSlots]
  uint32_t *cursor = sorted + kScatterSlots;                         // [tile_bound + 1]
  uint32_t *loff = cursor + (p.tile_bound + 1);                      // [tile_bound + 1]
  stage_levels(lv, shapes, starts, s);
  stage_tiles<T>(lv, s.levels, ntc, base);
  const int nt = base[s.levels];
  const uint32_t *row = counts + static_cast<size_t>(blockIdx.x) * p.tile_bound;
  const uint32_t *ts_row = tile_start + static_cast<size_t>(blockIdx.x / p.chunks) * (p.tile_bound + 1);
  for (int i = threadIdx.x; i < nt; i += blockDim.x) cursor[i] = ts_row[i] + row[i];

  const int bm = blockIdx.x / p.chunks, ch = blockIdx.x % p.chunks;
  const int b = bm / s.heads, m = bm % s.heads;
  const int q0 = ch * p.chunk_q;
  const int nq = min(p.chunk_q, s.queries - q0);
  uint4 *rec = records + static_cast<size_t>(bm) * p.rec_cap;
  const int lpp = 1 << p.lp_log2;
  const int sub_q = kScatterSlots >> p.lp_log2;  // >= 1 (lpp <= kScatterSlots, checked on the host)
  // each thread owns a contiguous run of tiles in the scans below
  const int per = (nt + kBinBlock - 1) / kBinBlock;
  const int t0 = min(nt, static_cast<int>(threadIdx.x) * per), t1 = min(nt, t0 + per);

  for (int qs = 0; qs < nq; qs += sub_q) {
    const int nsq = min(sub_q, nq - qs);
    for (int i = threadIdx.x; i < nt; i += blockDim.x) loff[i] = 0;
    lds_barrier();
    // 1. loads first (every one unconditional, clamped index), then the tap,
    // the rank inside its tile (LDS counter) and the record in arrival order
    float lx[kScatterPerThread], ly[kScatterPerThread], aw[kScatterPerThread];
    uint32_t key[kScatterPerThread];  // tile << 12 | slot, or kNoRecord
    uint32_t rk[kScatterPerThread];   // rank inside the tile
#pragma unroll
    for (int u = 0; u < kScatterPerThread; ++u) {
      const int j = threadIdx.x + u * kBinBlock;  // slot: query j >> lp_log2, sample j & (lpp - 1)
      const int q = q0 + qs + (j >> p.lp_log2), smp = j & (lpp - 1);
      const bool live = (j >> p.lp_log2) < nsq && smp < s.lp;
      const size_t o =
          live ? (static_cast<size_t>(b * s.queries + q) * s.heads + m) * s.lp + smp : 0;
      lx[u] = to_float(loc[2 * o]);
      ly[u] = to_float(loc[2 * o + 1]);
      aw[u] = to_float(attn[o]);
    }
#pragma unroll
    for (int u = 0; u < kScatterPerThread; ++u) {
      const int j = threadIdx.x + u * kBinBlock;
      const int q = q0 + qs + (j >> p.lp_log2), smp = j & (lpp - 1);
      const bool live = (j >> p.lp_log2) < nsq && smp < s.lp;
      const int l = level_of_sample(live ? smp : 0, s);
      const Tap t = make_tap(lx[u], ly[u], lv[l], live);
      key[u] = kNoRecord;
      rk[u] = 0;
      uint32_t at = kNoRecord;
      if (t.in) {
        const int tile = primary_tile<T>(t, ntc[l], base[l]);
        const uint32_t rank = atomicAdd(&loff[tile], 1u);
        key[u] = (static_cast<uint32_t>(tile) << 12) | static_cast<uint32_t>(j);
        at = cursor[tile] + rank;
        // top-left corner in the frame of its primary tile: [-1, T-1]^2 -> [0, T]^2
        const int ty = t.y0 < 0 ? 0 : t.y0, tx = t.x0 < 0 ? 0 : t.x0;
        const int pos = (t.y0 - (ty / T) * T + 1) * (T + 1) + (t.x0 - (tx / T) * T + 1);
        stage[j] = make_uint4((static_cast<uint32_t>(pos) << kPosShift) |
                                  (static_cast<uint32_t>(q) << p.lp_log2) |
                                  static_cast<uint32_t>(smp),
                              __float_as_uint(t.wx1), __float_as_uint(t.wy1),
                              __float_as_uint(aw[u]));
        rk[u] = rank;
      }
      if (live) {
        const size_t o = (static_cast<size_t>(b * s.queries + q) * s.heads + m) * s.lp + smp;
        if (!p.direct) {
          rec_of_sample[o] = at;
        } else if (at == kNoRecord) {  // no record: its gradients are zero
          grad_attn[o] = 0.0f;
          *reinterpret_cast<float2 *>(grad_loc + 2 * o) = make_float2(0.0f, 0.0f);
        }
      }
    }
    lds_barrier();
    // 2. tile counts -> exclusive offsets (in place); the counts are kept as
    // differences of consecutive offsets (loff[nt] = the sub-chunk's total)
    uint32_t run = 0;
    for (int t = t0; t < t1; ++t) run += loff[t];
    uint32_t total;
    uint32_t off = block_exclusive(run, part, &total);
    for (int t = t0; t < t1; ++t) {
      const uint32_t n = loff[t];
      loff[t] = off;
      off += n;
    }
    if (threadIdx.x == 0) loff[nt] = total;
    lds_barrier();
    // 3. tile-sorted list of slots
#pragma unroll
    for (int u = 0; u < kScatterPerThread; ++u) {
      if (key[u] != kNoRecord) sorted[loff[key[u] >> 12] + rk[u]] = key[u];
    }
    lds_barrier();
    // 4. records out in tile order: consecutive i of one tile are consecutive
    // records of its global range
    for (int i = threadIdx.x; i < static_cast<int>(total); i += kBinBlock) {
      const uint32_t e = sorted[i];
      const uint32_t tile = e >> 12, j = e & 0xfffu;
      rec[cursor[tile] + (static_cast<uint32_t>(i) - loff[tile])] = stage[j];
    }
    lds_barrier();
    // 5. cursors past this sub-chunk's records
    for (int t = threadIdx.x; t < nt; t += blockDim.x) cursor[t] += loff[t + 1] - loff[t];
    lds_barrier();
  }

  // non-boundary cells of the slab's empty and split tiles listed by
  // bin_scan: tiles ch, ch + chunks, ... of the list
  const uint32_t *zl = zero_tiles + static_cast<size_t>(bm) * (p.tile_bound + 1);
  const uint32_t nz = zl[0];
  const int MC = s.heads * C;
  const size_t slab = static_cast<size_t>(b) * s.spatial * MC + m * C;
  for (uint32_t z = ch; z < nz; z += p.chunks) {
    const TileGeom g = tile_geom(static_cast<int>(zl[1 + z]), T, ntc, base);
    zero_tile_cells<C, T>(grad_value, slab, MC, lv[g.l], g, threadIdx.x, blockDim.x,
                          [&](int r, int c) { return !boundary_cell(r, c, g); });
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

// One lane's eight channels of a value or grad_out row in the owner loop:
// fp32 as floats; fp16/bf16 kept packed (16 bytes), so that the corner dot
// products take one v_dot2 (two products, fp32 sum) per channel pair and
// only the corner sums need the channels as floats (c4 tile kernel: bf16
// 1468 -> 1445 us, fp16 1512 -> 1451 us against decoded rows and FMAs).
template <typename VT>
struct Row8 {
  float f[8];
};
template <>
struct Row8<bf16_t> {
  u32x4 w;
};
template <>
struct Row8<__half> {
  u32x4 w;
};

// row from LDS (16-byte aligned)
__device__ __forceinline__ void lds_row8(const float *p, Row8<float> &o) {
  const float4 a = reinterpret_cast<const float4 *>(p)[0];
  const float4 b = reinterpret_cast<const float4 *>(p)[1];
  o.f[0] = a.x; o.f[1] = a.y; o.f[2] = a.z; o.f[3] = a.w;
  o.f[4] = b.x; o.f[5] = b.y; o.f[6] = b.z; o.f[7] = b.w;
}
template <typename VT>
__device__ __forceinline__ void lds_row8(const VT *p, Row8<VT> &o) {
  o.w = *reinterpret_cast<const u32x4 *>(p);
}

// row at byte offset `off` of a buffer (32-bit offsets: fewer address
// instructions than 64-bit pointers)
__device__ __forceinline__ void buf_row8(__amdgpu_buffer_rsrc_t r, uint32_t off, Row8<float> &o) {
  float a[4], b[4];
  decode16(float(), buffer_load16(r, off), a);
  decode16(float(), buffer_load16(r, off + 16), b);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    o.f[j] = a[j];
    o.f[4 + j] = b[j];
  }
}
template <typename VT>
__device__ __forceinline__ void buf_row8(__amdgpu_buffer_rsrc_t r, uint32_t off, Row8<VT> &o) {
  o.w = buffer_load16(r, off);
}

// sum over the eight channels of a[j] * b[j]
__device__ __forceinline__ float dot8(const Row8<float> &a, const Row8<float> &b) {
  float d = 0.0f;
#pragma unroll
  for (int j = 0; j < 8; ++j) d += a.f[j] * b.f[j];
  return d;
}
__device__ __forceinline__ float dot8(const Row8<bf16_t> &a, const Row8<bf16_t> &b) {
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  const uint32_t x[4] = {a.w.x, a.w.y, a.w.z, a.w.w}, y[4] = {b.w.x, b.w.y, b.w.z, b.w.w};
  float d = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i)
    d = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, x[i]),
                                        __builtin_bit_cast(bf16x2, y[i]), d, false);
  return d;
}
__device__ __forceinline__ float dot8(const Row8<__half> &a, const Row8<__half> &b) {
  typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
  const uint32_t x[4] = {a.w.x, a.w.y, a.w.z, a.w.w}, y[4] = {b.w.x, b.w.y, b.w.z, b.w.w};
  float d = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i)
    d = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, x[i]), __builtin_bit_cast(f16x2, y[i]),
                               d, false);
  return d;
}

// the eight channels as floats (channel j of the lane -> o[j])
__device__ __forceinline__ void floats8(const Row8<float> &a, float (&o)[8]) {
#pragma unroll
  for (int j = 0; j < 8; ++j) o[j] = a.f[j];
}
template <typename VT>
__device__ __forceinline__ void floats8(const Row8<VT> &a, float (&o)[8]) {
  decode16(VT(), a.w, o);
}

// The four corner dot products of one record, D_d = sum over the group's KQ
// lanes of dd[d], by a reduce-scatter across the group (each step halves the
// values a lane carries), stored to the record's slot d4[0..3]. KQ = 4: lane k
// ends with D_k; KQ = 2: lane k with D_k and D_k+2; KQ = 8: lanes 4 + k of
// the group with D_k (row_ror by 4 brings the other quad's sums).
template <int KQ>
__device__ __forceinline__ void store_corner_dots(const float (&dd)[4], int k, float *d4) {
  const bool b0 = (k & 1) != 0;
  // lanes k and k ^ 1: an even lane keeps corners 0 and 2, an odd lane 1 and 3
  const float s0 = b0 ? dd[0] : dd[1], s1 = b0 ? dd[2] : dd[3];
  const float k0 = (b0 ? dd[1] : dd[0]) + MSDA_DPP(s0, 0xB1);
  const float k1 = (b0 ? dd[3] : dd[2]) + MSDA_DPP(s1, 0xB1);
  if constexpr (KQ == 2) {
    d4[k] = k0;
    d4[k + 2] = k1;
  } else {
    // lanes k and k ^ 2: lanes 0, 1 keep corners 0, 1; lanes 2, 3 keep 2, 3
    const bool b1 = (k & 2) != 0;
    const float s = b1 ? k0 : k1;
    float kk = (b1 ? k1 : k0) + MSDA_DPP(s, 0x4E);
    if constexpr (KQ == 4) {
      d4[k] = kk;
    } else {
      kk += MSDA_DPP(kk, 0x124);  // row_ror:4 -> lane i gets lane i - 4 of its row
      if (k >= 4) d4[k - 4] = kk;
    }
  }
}

// One work item = records [r0, r1) of a tile of T x T value cells. The
// records are processed in batches of K: counting-sorted by top-left corner
// position ((T+1)^2 positions, [-1, T-1]^2 in the tile frame) in LDS; lane
// group g (KQ lanes of 8 channels) then owns positions of rank g,
// 2 NG - 1 - g, 2 NG + g, ... (ranks in decreasing-count order) and
// accumulates, in registers, the four corner sums
// S_p[d] = sum_r w_d(r) * attn(r) * grad_out[q(r)] of each; S_p[d] goes to
// slot p of corner plane d (no other group writes it): stored by the item's
// first batch, which visits every position, added by its later batches. At
// the end of the item, cell (r, c) sums slot (r - dy, c - dx) of plane
// (dy, dx). Per record the owner group also computes the four corner dot
// products D_d = grad_out . v_d from the LDS value tile, from which one
// thread per record forms the attention and location gradients:
//   grad_attn = sum_d w_d D_d,
//   grad_ix = attn * (wy0 (D1 - D0) + wy1 (D3 - D2)),
//   grad_iy = attn * (wx0 (D2 - D0) + wx1 (D3 - D1)),
//   grad_loc = (grad_ix * W, grad_iy * H)   (d ix / d loc_x = W),
// grid_sample's bilinear backward (zeros padding) regrouped by corner; they
// are stored over the record's own (consumed) slot for msda_grad_gather.
//
// Memory order: gfx950 counts loads and stores in one in-order vmcnt, so a
// wait for one load also waits for everything issued before it. The next
// batch's records are loaded first thing in a batch (into registers); the
// next item's value tile is loaded into registers at the end of phase E of
// the previous batch and written to LDS in phase C; the owner loop keeps NR
// grad_out rows in flight per group. No buffer-to-LDS loads: after one, the
// compiler makes every LDS access wait for it (and so for all earlier loads
// and stores).
template <typename VT, int C>
__global__ void __launch_bounds__(kTileBlock)
    msda_tile_backward(const VT *__restrict__ value, uint32_t value_bytes,
                       const int64_t *__restrict__ shapes, const int64_t *__restrict__ starts,
                       const VT *__restrict__ grad_out, uint32_t grad_bytes,
                       uint4 *__restrict__ records,
                       const Item *__restrict__ items, uint32_t *__restrict__ item_total,
                       Shape s, BinPlan p, float *__restrict__ grad_value,
                       float *__restrict__ grad_loc, float *__restrict__ grad_attn) {
  using Cfg = TileCfg<VT, C>;
  constexpr int T = Cfg::T, K = Cfg::K, CPL = Cfg::CPL;
  constexpr int TV = T + 1, NPOS = TV * TV;
  constexpr int KQ = C / CPL;          // lanes per group
  constexpr int NG = kTileBlock / KQ;  // lane groups
  constexpr int VB = static_cast<int>(sizeof(VT));
  constexpr int UPV = C * VB / 16;     // 16-byte units per value row
  constexpr int VPT = (NPOS * UPV + kTileBlock - 1) / kTileBlock;  // value units per thread
  constexpr int RPT = K / kTileBlock;  // records per thread
  constexpr int NR = 2;                // grad_out rows in flight per group
  // owners' corner sums as MFMA outer products (needs whole 4-lane groups):
  // for 16-bit values, whose owner loop also decodes each grad_out row
  // (c4 tile kernel: bf16 1515 -> 1469 us, fp16 1650 -> 1511 us, before the
  // packed dots and the request order below); fp32 values keep the vector
  // FMAs, which measured faster there (c2 536 against 547 us, c1 191
  // against 196 us)
  constexpr bool kMfmaSums = KQ >= 4 && sizeof(VT) == 2;
  // teams of up to 4 groups inside one 16-lane DPP row
  constexpr int kMaxTeamShift = KQ <= 4 ? 2 : 1;
  static_assert(CPL == 8 && (KQ == 2 || KQ == 4 || KQ == 8), "bad lane layout");
  static_assert(K % kTileBlock == 0 && NPOS <= kTileBlock, "bad batch size");
  static_assert(K < 65536 && NPOS < 65536, "rank table packs count and position in 16 bits");
  static_assert(tile_lds_bytes<VT, C>() + 3400 <= kTileLdsLimit, "tile LDS budget");

  __shared__ Level lv[kMaxLevels];
  __shared__ int ntc[kMaxLevels], base[kMaxLevels + 1];
  __shared__ int team_shift_s;  // log2 of the owner team size of the current batch
  extern __shared__ __align__(16) unsigned char lds[];
  constexpr int CS = C + kVtPad / VB;  // elements per value-tile cell, with its padding
  VT *vt = reinterpret_cast<VT *>(lds);  // NPOS cells + one zero row, CS elements apart
  float *planes = reinterpret_cast<float *>(lds + static_cast<size_t>(NPOS + 1) * CS * VB);
  uint4 *stash = reinterpret_cast<uint4 *>(planes + 4 * NPOS * C);
  uint32_t *pcount = reinterpret_cast<uint32_t *>(stash + K);
  uint32_t *poff = pcount + NPOS;
  // rank table: rank r -> {count << 16 | position, first slot}
  uint2 *rtab = reinterpret_cast<uint2 *>(poff + NPOS);
  uint32_t *bucket = reinterpret_cast<uint32_t *>(rtab + NPOS);  // [64] positions per count bucket
  uint32_t *bstart = bucket + 64;   // [64] first rank of each bucket
  uint32_t *wsum = bstart + 64;     // [16] counts per wavefront of positions

  stage_levels(lv, shapes, starts, s);
  stage_tiles<T>(lv, s.levels, ntc, base);
  const int MC = s.heads * C;
  const int tid = threadIdx.x;
  const int lane = tid % kWave, wave = tid / kWave;
  const int grp = tid / KQ, k = tid % KQ;
  const __amdgpu_buffer_rsrc_t vrsrc = make_rsrc(value, value_bytes);
  const __amdgpu_buffer_rsrc_t grsrc = make_rsrc(grad_out, grad_bytes);

  // Items are taken dynamically: the list is cut into one contiguous share
  // per XCD (workgroups are dispatched to the XCDs round-robin, so block
  // i % 8 runs on XCD i % 8 and a slab's items stay in one XCD's L2), and
  // the workgroups of an XCD take items of its share in list order through
  // an atomic counter (zeroed by bin_count). Thread 0 takes the next item one
  // item ahead and publishes its index through LDS.
  const uint32_t n_items = min(*item_total, static_cast<uint32_t>(p.item_cap));
  const int xcd = static_cast<int>(blockIdx.x % kXcdQueues);
  const uint32_t lo = static_cast<uint32_t>(static_cast<uint64_t>(n_items) * xcd / kXcdQueues);
  const uint32_t hi =
      static_cast<uint32_t>(static_cast<uint64_t>(n_items) * (xcd + 1) / kXcdQueues);
  uint32_t *queue = item_total + 1 + xcd;
  __shared__ uint32_t taken[2];
  __shared__ Item taken_item;  // descriptor of taken[0], fetched by wavefront 0
  auto take_item = [&]() -> uint32_t {  // thread 0 only
    const uint32_t i = lo < hi ? atomicAdd(queue, 1u) : 0u;
    return lo + i < hi ? lo + i : kNoItem;
  };
  auto item_of = [&](uint32_t idx, bool &ok) {
    ok = idx != kNoItem;
    Item d{0u, 0u, 0u, 0u, 0u, 0u, 0u, 0u};
    if (ok) d = items[idx];
    return d;
  };

  // cursors of batches b (c0) and b + 1 (c1); `pre` is the descriptor of the
  // item after c1's. advance() hands `pre` over when a cursor moves to a new
  // item; the caller then refills `pre` from a freshly taken item.
  if (tid == 0) {
    taken[0] = take_item();
    taken[1] = take_item();
  }
  __syncthreads();
  BatchCursor c0;
  c0.n = 0;
  c0.k = 0;
  c0.d = item_of(taken[0], c0.valid);
  if (!c0.valid) return;  // uniform: no item for this workgroup
  bool pre_ok;
  Item pre = item_of(taken[1], pre_ok);
  auto moves_on = [&](const BatchCursor &c) {
    return c.valid && c.k + 1 >= item_batches<K>(c.d);
  };
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
    }
    return r;
  };
  const bool refill0 = moves_on(c0);
  __syncthreads();  // taken[] read by every thread
  if (refill0 && tid == 0) taken[0] = take_item();
  BatchCursor c1 = advance(c0);
  __syncthreads();
  if (refill0) pre = item_of(taken[0], pre_ok);

  auto batch_range = [&](const BatchCursor &c, uint32_t &s0, uint32_t &s1) {
    s0 = c.d.r0 + c.k * K;
    s1 = min(c.d.r1, s0 + K);
  };
  auto rec_base = [&](const Item &d) {
    return static_cast<size_t>(d.b * s.heads + d.m) * p.rec_cap;
  };
  // loads are issued unconditionally (clamped, always valid addresses): a
  // load inside a branch is waited for before the branch joins
  auto load_record = [&](const BatchCursor &c, int u) {
    uint32_t s0, s1;
    batch_range(c, s0, s1);
    const uint32_t i = s0 + tid + u * kTileBlock;
    const size_t at = c.valid && i < s1 ? rec_base(c.d) + i : 0;
    return load_nt(records + at);  // each record is read once
  };
  auto slab_offset = [&](const Item &d) {
    return static_cast<size_t>(d.b) * s.spatial * MC + d.m * C;
  };
  // Value tile (cells [0, T]^2 of the item's frame) of d: 16-byte unit u =
  // tid + v * kTileBlock of the tile goes to vt + 16 u. The next item's tile
  // is loaded into registers at the end of phase E of the batch before its
  // first one and written to LDS in that first batch's phase C (vt is read
  // only in phase D). Every load is issued (an out-of-range offset, which
  // reads zeros, for units past the tile, cells outside the level and
  // batches that start no item). Buffer-to-LDS loads held no registers, but
  // every LDS access after one waits for it -- and, vmcnt counting in issue
  // order, for every store issued before it -- so each batch's first LDS
  // access waited for the previous batch's scattered gradient stores to
  // drain. value_bytes < 2^31 is checked on the host.
  uint4 vt_next[VPT];
  auto load_value_tile = [&](const Item &d, bool want) {
    const TileGeom g = item_geom(d);
    const Level L = lv[g.l];
    const size_t slab = slab_offset(d);
#pragma unroll
    for (int v = 0; v < VPT; ++v) {
      const int unit = tid + v * kTileBlock;
      const int cell = unit / UPV, kk = unit % UPV;
      const int y = g.y_lo + cell / TV, x = g.x_lo + cell % TV;
      const uint32_t off =
          want && unit < NPOS * UPV && y < L.h && x < L.w
              ? static_cast<uint32_t>(
                    (slab + static_cast<size_t>(L.start + y * L.w + x) * MC) * VB) +
                    static_cast<uint32_t>(kk * 16)
              : kOobOffset;
      // cache policy 2 = non-temporal: a tile's value rows are staged once
      const u32x4 w = __builtin_amdgcn_raw_buffer_load_b128(vrsrc, off, 0, 2);
      vt_next[v] = make_uint4(w[0], w[1], w[2], w[3]);
    }
  };
  auto store_value_tile = [&]() {
    // the thread index through an empty asm: the slot addresses are
    // recomputed here (a few instructions) rather than hoisted out of the
    // batch loop, where they were held in registers through phase D
    int me = tid;
    asm volatile("" : "+v"(me));
#pragma unroll
    for (int v = 0; v < VPT; ++v) {
      const int unit = me + v * kTileBlock;
      // unit kk of cell c -> 16-byte slot c * (UPV + 1) + kk (the padding)
      if (unit < NPOS * UPV) reinterpret_cast<uint4 *>(vt)[unit + unit / UPV] = vt_next[v];
    }
  };
  // cell sums of a finished item's corner planes to grad_value: cell (r, c)
  // of [0, T]^2 sums slot (r - dy, c - dx) of plane (dy, dx) (slots that map
  // to row or column -1 only ever hold contributions of invalid corners and
  // are not read). Cells the item owns alone get one 16-byte store per four
  // channels; cells it shares with a neighbouring tile's items (the halo row
  // and column, the first row and column away from the level's edge, every
  // cell of a split tile) are added with fp32 atomics, one channel per lane,
  // so that one atomic instruction covers whole 128-byte lines (four channels
  // per lane put a lane every 16 bytes and took four instructions per line).
  auto write_back = [&](const Item &d) {
    constexpr int C4 = C / 4;
    const TileGeom g = item_geom(d);
    const Level Lw = lv[g.l];
    const bool split = (d.tile & kSplitBit) != 0;
    const size_t slab = slab_offset(d);
    auto cell_ptr = [&](int r, int c) {
      return grad_value + slab +
             static_cast<size_t>(Lw.start + (g.y_lo + r) * Lw.w + g.x_lo + c) * MC;
    };
    // Position (r - dy, c - dx) of plane q = 2 dy + dx lies a fixed distance
    // from position (r, c) of plane 0 (kQ1, kQ2, kQ3 floats for q = 1, 2, 3),
    // so the four reads of a cell come off one address. They are issued before any is waited for:
    // the empty asm takes all their values at once (scheduled freely, the
    // compiler waited for each read before issuing the next, four LDS round
    // trips per cell). Every cell (r, c) of [0, T]^2 gives addresses inside
    // the four planes; a slot that is not the cell's is read and not added.
    constexpr int kQ1 = NPOS * C - C, kQ2 = 2 * NPOS * C - TV * C;
    constexpr int kQ3 = 3 * NPOS * C - (TV + 1) * C;
    auto plane_base = [&](int r, int c, int ch) {
      return planes + ((r + 1) * TV + c + 1) * C + ch;
    };
    if (!split) {
      for (int i = tid; i < T * T * C4; i += kTileBlock) {
        const int cell = i / C4, ch = (i % C4) * 4;
        const int r = cell / T, c = cell % T;
        const float *pl = plane_base(r, c, ch);
        float4 v[4];
        v[0] = *reinterpret_cast<const float4 *>(pl);
        v[1] = *reinterpret_cast<const float4 *>(pl + kQ1);
        v[2] = *reinterpret_cast<const float4 *>(pl + kQ2);
        v[3] = *reinterpret_cast<const float4 *>(pl + kQ3);
#pragma unroll
        for (int q = 0; q < 4; ++q)
          asm volatile("" : "+v"(v[q].x), "+v"(v[q].y), "+v"(v[q].z), "+v"(v[q].w));
        if (g.y_lo + r >= Lw.h || g.x_lo + c >= Lw.w || boundary_cell(r, c, g)) continue;
        const float sv[4] = {v[0].x + v[1].x + v[2].x + v[3].x, v[0].y + v[1].y + v[2].y + v[3].y,
                             v[0].z + v[1].z + v[2].z + v[3].z, v[0].w + v[1].w + v[2].w + v[3].w};
        store16_nt(cell_ptr(r, c) + ch, sv);
      }
    }
    // shared cells, enumerated: split tiles all of [0, T]^2; otherwise row T
    // (T + 1 cells), column T above it (T), then row 0 if the tile is not at
    // the level's top (T) and column 0 below that row if not at its left
    const int top = g.y_lo > 0 ? 1 : 0, left = g.x_lo > 0 ? 1 : 0;
    const int n_shared = split ? NPOS : TV + T + top * T + left * (T - top);
    for (int i = tid; i < n_shared * C; i += kTileBlock) {
      const int k = i / C, ch = i % C;
      int r, c;
      if (split) {
        r = k / TV;
        c = k % TV;
      } else if (k < TV) {
        r = T;
        c = k;
      } else if (k < TV + T) {
        r = k - TV;
        c = T;
      } else if (top && k < TV + 2 * T) {
        r = 0;
        c = k - TV - T;
      } else {
        r = top + (k - TV - T - top * T);
        c = 0;
      }
      const float *pl = plane_base(r, c, ch);
      float v0 = pl[0], v1 = pl[kQ1], v2 = pl[kQ2], v3 = pl[kQ3];
      asm volatile("" : "+v"(v0), "+v"(v1), "+v"(v2), "+v"(v3));
      if (g.y_lo + r >= Lw.h || g.x_lo + c >= Lw.w) continue;
      // plane q holds a position of the tile (row and column < T) for
      // q = 0 when r, c < T, q = 1 when r < T, q = 2 when c < T, q = 3 always
      const float sum =
          (r < T && c < T ? v0 : 0.0f) + (r < T ? v1 : 0.0f) + (c < T ? v2 : 0.0f) + v3;
      unsafeAtomicAdd(cell_ptr(r, c) + ch, sum);
    }
  };

  // prologue: batch 0's records and value tile
  uint4 r_cur[RPT];
#pragma unroll
  for (int u = 0; u < RPT; ++u) r_cur[u] = load_record(c0, u);
  load_value_tile(c0.d, true);
  store_value_tile();
  if (tid < UPV) reinterpret_cast<uint4 *>(vt + NPOS * CS)[tid] = make_uint4(0u, 0u, 0u, 0u);
  if (tid < NPOS) pcount[tid] = 0;
  if (tid < kWave) bucket[tid] = 0;
  __syncthreads();

  for (;;) {
    const TileGeom g0 = item_geom(c0.d);
    const Level L = lv[g0.l];
    uint32_t s0, s1;
    batch_range(c0, s0, s1);
    const int ns = static_cast<int>(s1 - s0);
    const bool first_of_item = c0.k == 0;
    const bool last_of_item = c0.k + 1 == item_batches<K>(c0.d);
    const bool next_new_item = c1.valid && c1.k == 0;
    const int b0 = static_cast<int>(c0.d.b), m0 = static_cast<int>(c0.d.m);

    // c1 moves on to a new item at the end of this batch: thread 0 takes
    // the item after it now and publishes it in phase E, so the atomic's
    // round trip overlaps the batch
    const bool refill = moves_on(c1);
    uint32_t took = 0;
    // (mbcnt_lo(~0, 0) is 0 for thread 0; it makes the address look
    // lane-dependent, so the compiler's atomic optimizer leaves this one-
    // thread atomic alone instead of broadcasting its result -- and waiting
    // for it, and for every earlier memory operation -- right here)
    if (refill && tid == 0 && lo < hi) {
      took = atomicAdd(queue + __builtin_amdgcn_mbcnt_lo(~0u, 0u), 1u);
    }

    // A. next batch's records; this batch's sort keys. Record slots are
    // u * kTileBlock + tid; a wavefront whose first slot is past the batch
    // skips the per-record work.
    uint4 r_next[RPT];
#pragma unroll
    for (int u = 0; u < RPT; ++u) r_next[u] = load_record(c1, u);
    const int wave_slot = tid & ~(kWave - 1);
    int pos[RPT];
    uint32_t rank[RPT];
    float my_wx1[RPT], my_wy1[RPT], my_a[RPT];
    uint32_t my_id[RPT];  // query << lp_log2 | sample
#pragma unroll
    for (int u = 0; u < RPT; ++u) {
      const int i = tid + u * kTileBlock;
      my_id[u] = r_cur[u].x & kSampleMask;
      pos[u] = -1;
      rank[u] = 0;
      my_wx1[u] = my_wy1[u] = 0.0f;
      my_a[u] = __uint_as_float(r_cur[u].w);
      // the record carries its tap (bin_scatter): position, wx1, wy1
      if (wave_slot + u * kTileBlock < ns && i < ns) {
        my_wx1[u] = __uint_as_float(r_cur[u].y);
        my_wy1[u] = __uint_as_float(r_cur[u].z);
        pos[u] = static_cast<int>(min(r_cur[u].x >> kPosShift, static_cast<uint32_t>(NPOS - 1)));
        rank[u] = atomicAdd(&pcount[pos[u]], 1u);
      }
    }
    lds_barrier();

    // B. positions in order of decreasing count (counting sort on
    // min(n, 63)) and the exclusive scan of the counts, one thread per
    // position: B1 scans within wavefronts and ranks each position in its
    // count bucket, B2 adds the wavefront totals and scans the buckets, B3
    // places each position.
    constexpr int kPosWaves = (NPOS + kWave - 1) / kWave;
    uint32_t p_cnt = 0, p_incl = 0, p_brank = 0;
    int p_bk = 0;
    if (tid < kPosWaves * kWave) {
      p_cnt = tid < NPOS ? pcount[tid] : 0u;
      p_incl = wave_inclusive_sum(p_cnt);
      if (lane == kWave - 1) wsum[wave] = p_incl;
      if (tid < NPOS) {
        p_bk = 63 - static_cast<int>(min(p_cnt, 63u));
        p_brank = atomicAdd(&bucket[p_bk], 1u);
      }
    }
    lds_barrier();
    uint32_t p_off = 0;
    if (tid < NPOS) {
      uint32_t before = 0;
      for (int w = 0; w < wave; ++w) before += wsum[w];
      p_off = before + p_incl - p_cnt;
      poff[tid] = p_off;
    }
    if (tid < kWave) {
      const uint32_t v = bucket[tid];
      const uint32_t incl = wave_inclusive_sum(v);
      bstart[tid] = incl - v;
      // owner team size: positions used = NPOS - (positions with count 0)
      if (tid == kWave - 1) {
        const int used = NPOS - static_cast<int>(v);
        int shift = 0;
        if (kMaxTeamShift >= 1 && used <= NG / 2) shift = 1;
        if (kMaxTeamShift >= 2 && used <= NG / 4) shift = 2;
        team_shift_s = shift;
      }
    }
    lds_barrier();
    if (tid < NPOS) {
      rtab[bstart[p_bk] + p_brank] = make_uint2((p_cnt << 16) | static_cast<uint32_t>(tid), p_off);
    }

    // C. records in position order; a new item's value tile (loaded into
    // registers in the previous batch) into LDS
    uint32_t my_slot[RPT];
#pragma unroll
    for (int u = 0; u < RPT; ++u) {
      my_slot[u] = 0;
      if (wave_slot + u * kTileBlock < ns && pos[u] >= 0) {
        my_slot[u] = poff[pos[u]] + rank[u];
        // the owners take the row weights with the attention weight folded
        // in: {id, wx1, (1 - wy1) a, wy1 a}
        stash[my_slot[u]] = make_uint4(r_cur[u].x, __float_as_uint(my_wx1[u]),
                                       __float_as_uint((1.0f - my_wy1[u]) * my_a[u]),
                                       __float_as_uint(my_wy1[u] * my_a[u]));
      }
    }
    if (first_of_item) store_value_tile();
    lds_barrier();

    // D. owners: teams of S = 1, 2 or 4 lane groups (inside one 16-lane DPP
    // row; S grows when the batch uses few positions, as in the thin tiles at
    // a level's edge); team t takes ranks t, 2 NT - 1 - t, 2 NT + t, ...
    // (snake order: the owners of the largest positions of one round get the
    // smallest of the next). Group `sub` of a team takes the position's
    // records sub, sub + S, ...; the S register sums are added across the
    // team (row_ror) and its last group writes the planes. The first batch of
    // an item visits every position (zero-count ones store zero sums); later
    // batches stop at the first empty position and add.
    // When the batch uses single-group teams, wavefront 0 -- which holds the
    // largest positions, and whose chain of grad_out loads bounds the phase --
    // works in teams of two instead (its 8 teams take ranks 0-7 of a round,
    // the other wavefronts' groups the ranks after them). Wavefront-uniform,
    // so the team sum stays one DPP pass per wavefront. Measured against
    // single groups everywhere: c2 tile kernel 616 -> 588 us, c4 bf16 1600
    // -> 1543 us; a first wavefront of 4-group teams, or two wavefronts of
    // 2-group teams, gained less.
    // grad_out rows through a buffer resource: byte offsets below 2^31
    // (checked on the host), q < 2^24 and the row stride below 2^24 (24-bit
    // multiply)
    const uint32_t gbase = static_cast<uint32_t>(
        ((static_cast<size_t>(b0) * s.queries * s.heads + m0) * C + k * CPL) * VB);
    const uint32_t q_stride = static_cast<uint32_t>(s.heads * C * VB);  // grad_out row bytes
    const u32x4 *vstash = reinterpret_cast<const u32x4 *>(stash);
    float *stash_f = reinterpret_cast<float *>(stash);
    auto grow = [&](uint32_t id) {
      const uint32_t q =
          min((id & kSampleMask) >> p.lp_log2, static_cast<uint32_t>(s.queries - 1));
      return gbase + __umul24(q, q_stride);
    };
    int tshift = team_shift_s;
    int NT = NG >> tshift, team = grp >> tshift;
    if (tshift == 0) {
      constexpr int GPW = kWave / KQ;  // lane groups per wavefront
      if (__builtin_amdgcn_readfirstlane(wave) == 0) {
        tshift = 1;
        team = grp >> 1;
      } else {
        team = grp - GPW / 2;
      }
      NT = NG - GPW / 2;
    }
    const int S = 1 << tshift;
    const int sub = grp & (S - 1);
#pragma unroll 1
    for (int rnd = 0; rnd * NT < NPOS; ++rnd) {
      const int i = rnd * NT + ((rnd & 1) ? NT - 1 - team : team);
      if (i >= NPOS) break;  // later rounds start further out
      const uint2 rt = rtab[i];  // one LDS read: position, its count and first slot
      const int p_id = static_cast<int>(rt.x & 0xffffu);
      const uint32_t n = rt.x >> 16;
      if (n == 0 && !first_of_item) break;  // positions are in order of decreasing count
      // acc[j][d]: corner d's sum of this lane's channel k * CPL + j (an
      // MFMA accumulator per j; packing separate floats into one per MFMA
      // measured 10% slower for 16-bit values)
      f32x4 acc[CPL];
#pragma unroll
      for (int j = 0; j < CPL; ++j) acc[j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      // this group's records of the position: sub, sub + S, ...
      const uint32_t cnt = n > static_cast<uint32_t>(sub)
                               ? (n - static_cast<uint32_t>(sub) + S - 1) >> tshift
                               : 0u;
      if (cnt > 0) {
        const uint32_t first = rt.y + static_cast<uint32_t>(sub);
        const uint32_t stride = static_cast<uint32_t>(S);
        const int py = p_id / TV - 1, px = p_id % TV - 1;  // tile frame, >= -1
        // corner value rows (row -1 or column -1: the zero row after the tile)
        Row8<VT> v[4];
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          const int cy = py + (d >> 1), cx = px + (d & 1);
          lds_row8(vt + ((cy >= 0 && cx >= 0) ? (cy * TV + cx) * CS : NPOS * CS) + k * CPL, v[d]);
        }
        // One record: its four corner dot products (stored over its stash
        // slot) and, except where the MFMA sums run, its corner sums. With
        // MFMA sums the record's decoded row and its corner weight for this
        // lane are returned in gv, wk for the caller's sums, which come
        // after the group's next row is requested.
        auto one_record = [&](const u32x4 &e, const Row8<VT> &gr, uint32_t slot,
                              float (&gv)[CPL], float &wk) {
          const float wx1 = __uint_as_float(e.y);
          const float ay0 = __uint_as_float(e.z), ay1 = __uint_as_float(e.w);
          const float wx0 = 1.0f - wx1;
          float dd[4];
          if constexpr (sizeof(VT) == 4) {
            // fp32 rows: corner sums and dots in one pass over the row (at
            // the kernel's register limit: a copy of the row, to request the
            // next one before the sums, spills)
            const float wa[4] = {ay0 * wx0, ay0 * wx1, ay1 * wx0, ay1 * wx1};
#pragma unroll
            for (int d = 0; d < 4; ++d) {
              dd[d] = 0.0f;
#pragma unroll
              for (int j = 0; j < CPL; ++j) {
                acc[j][d] += wa[d] * gr.f[j];
                dd[d] += gr.f[j] * v[d].f[j];
              }
            }
          } else {
#pragma unroll
            for (int d = 0; d < 4; ++d) dd[d] = dot8(gr, v[d]);
            floats8(gr, gv);
            if constexpr (kMfmaSums) {
              wk = ((k & 2) ? ay1 : ay0) * ((k & 1) ? wx1 : wx0);
            } else {
              const float wa[4] = {ay0 * wx0, ay0 * wx1, ay1 * wx0, ay1 * wx1};
#pragma unroll
              for (int j = 0; j < CPL; ++j)
#pragma unroll
                for (int d = 0; d < 4; ++d) acc[j][d] += wa[d] * gv[j];
            }
          }
          // D_0..D_3 replace the consumed record (read by this group alone)
          store_corner_dots<KQ>(dd, k, stash_f + slot * 4);
        };
        // NR records in flight: register set j holds this group's record
        // r + j and, once the record's row has been used, is refilled with
        // record r + j + NR (stash entry read, row requested). The MFMA sums
        // of record r + j come after that request: the chain of a
        // position's rows is what the phase waits on (c4 bf16 tile kernel
        // 1446 -> 1382 us against sums before the request; requesting before
        // the dots, from a copy of the row, measured 4% slower than after
        // them). Past the end of the list a set keeps its record: a
        // processed slot holds D values, not a record id.
        u32x4 e[NR];
        Row8<VT> g[NR];
#pragma unroll
        for (int j = 0; j < NR; ++j) {
          e[j] = vstash[first + stride * min(static_cast<uint32_t>(j), cnt - 1)];
          buf_row8(grsrc, grow(e[j].x), g[j]);
          // requests in set order: the loop waits for set j's row by its
          // place in the in-order vmcnt, which holds only if set 0's row
          // went out first (the compiler issued set 1's first, and every
          // record then waited for both rows: c4 bf16 tile kernel 1378 ->
          // 1330 us with the order kept, c2 fp32 556 -> 533 us)
          __builtin_amdgcn_sched_barrier(0);
        }
        for (uint32_t r = 0; r < cnt; r += NR) {
#pragma unroll
          for (int j = 0; j < NR; ++j) {
            const bool live = r + j < cnt;
            float gv[CPL];
            float wk = 0.0f;
            if (live) one_record(e[j], g[j], first + stride * (r + j), gv, wk);
            const uint32_t nx = r + j + NR;
            const u32x4 t = vstash[first + stride * min(nx, cnt - 1)];
            e[j] = nx < cnt ? t : e[j];
            buf_row8(grsrc, grow(e[j].x), g[j]);
            if constexpr (kMfmaSums) {
              // corner sums on the matrix cores: v_mfma_f32_4x4x1f32 is 16
              // independent 4 x 4 outer products, block b on lanes
              // 4b..4b+3 (A[i] from lane 4b + i, B[j] from lane 4b + j,
              // D[i][j] in register i of lane 4b + j). A lane group of
              // KQ >= 4 lanes is KQ / 4 whole blocks: lane k gives corner
              // (k & 3)'s weight as A and its channel k * CPL + j as B, so
              // register d of lane k gets w_d * g[k * CPL + j] -- acc[j][d]
              // -- at twice the rate of the vector FMAs and off the vector
              // pipe. A block is one group's lanes only, and the result is
              // written under EXEC, so a group that has run out of records
              // keeps its sums.
              if (live) {
#pragma unroll
                for (int jj = 0; jj < CPL; ++jj)
                  acc[jj] = __builtin_amdgcn_mfma_f32_4x4x1f32(wk, gv[jj], acc[jj], 0, 0, 0);
              }
            }
          }
        }
      }
      // team sum: group g of a row receives group g - 1 (then g - 2), so the
      // team's last group ends with the sum over the team
      if (S >= 2) {
#pragma unroll
        for (int d = 0; d < 4; ++d)
#pragma unroll
          for (int j = 0; j < CPL; ++j) acc[j][d] += MSDA_DPP(acc[j][d], 0x120 + KQ);
      }
      if constexpr (kMaxTeamShift >= 2) {
        if (S >= 4) {
#pragma unroll
          for (int d = 0; d < 4; ++d)
#pragma unroll
            for (int j = 0; j < CPL; ++j) acc[j][d] += MSDA_DPP(acc[j][d], 0x120 + 2 * KQ);
        }
      }
      if (sub == S - 1) {
        float *pb = planes + p_id * C + k * CPL;  // slot p_id of plane d at pb + d * NPOS * C
        if (!first_of_item) {
          // the item's earlier batches' sums: all reads issued before any is
          // waited for (the empty asm takes them together; scheduled freely,
          // each read was waited for before the next was issued)
          float4 old[4][CPL / 4];
#pragma unroll
          for (int d = 0; d < 4; ++d)
#pragma unroll
            for (int h = 0; h < CPL / 4; ++h)
              old[d][h] = reinterpret_cast<const float4 *>(pb + d * NPOS * C)[h];
#pragma unroll
          for (int d = 0; d < 4; ++d)
#pragma unroll
            for (int h = 0; h < CPL / 4; ++h)
              asm volatile("" : "+v"(old[d][h].x), "+v"(old[d][h].y), "+v"(old[d][h].z),
                           "+v"(old[d][h].w));
#pragma unroll
          for (int d = 0; d < 4; ++d)
#pragma unroll
            for (int h = 0; h < CPL / 4; ++h) {
              acc[4 * h][d] += old[d][h].x;
              acc[4 * h + 1][d] += old[d][h].y;
              acc[4 * h + 2][d] += old[d][h].z;
              acc[4 * h + 3][d] += old[d][h].w;
            }
        }
#pragma unroll
        for (int d = 0; d < 4; ++d)
#pragma unroll
          for (int h = 0; h < CPL / 4; ++h)
            reinterpret_cast<float4 *>(pb + d * NPOS * C)[h] = make_float4(
                acc[4 * h][d], acc[4 * h + 1][d], acc[4 * h + 2][d], acc[4 * h + 3][d]);
      }
    }
    lds_barrier();

    // E. the next batch's records move into place first (the empty asm
    // pins the wait for their loads here, before this phase's stores are
    // issued); then this batch's location/weight gradients, the position
    // counts reset, a finished item written back and, when the next batch
    // starts an item, its value tile requested (into registers, waited for
    // in that batch's phase C)
#pragma unroll
    for (int u = 0; u < RPT; ++u) {
      r_cur[u] = r_next[u];
      asm volatile("" : "+v"(r_cur[u].x), "+v"(r_cur[u].y), "+v"(r_cur[u].z), "+v"(r_cur[u].w));
    }
    const size_t rb = rec_base(c0.d) + s0;
    const size_t sb = (static_cast<size_t>(c0.d.b) * s.queries * s.heads + c0.d.m) * s.lp;
#pragma unroll
    for (int u = 0; u < RPT; ++u) {
      const int i = tid + u * kTileBlock;
      if (wave_slot + u * kTileBlock < ns && i < ns) {
        const uint4 Dr = stash[my_slot[u]];
        const float D0 = __uint_as_float(Dr.x), D1 = __uint_as_float(Dr.y);
        const float D2 = __uint_as_float(Dr.z), D3 = __uint_as_float(Dr.w);
        const float wx1 = my_wx1[u], wy1 = my_wy1[u], a = my_a[u];
        const float wx0 = 1.0f - wx1, wy0 = 1.0f - wy1;
        const float ga = wy0 * (wx0 * D0 + wx1 * D1) + wy1 * (wx0 * D2 + wx1 * D3);
        const float gx = a * (wy0 * (D1 - D0) + wy1 * (D3 - D2)) * L.fw;
        const float gy = a * (wx0 * (D2 - D0) + wx1 * (D3 - D1)) * L.fh;
        if (p.direct) {  // straight to the sample's place: o = ((b*Q + q)*M + m)*lp + smp
          const uint32_t q = my_id[u] >> p.lp_log2, smp = my_id[u] & ((1u << p.lp_log2) - 1u);
          const size_t o = sb + static_cast<size_t>(q) * s.heads * s.lp + smp;
          grad_attn[o] = ga;
          *reinterpret_cast<float2 *>(grad_loc + 2 * o) = make_float2(gx, gy);
        } else {
          store_nt(records + rb + i, make_uint4(__float_as_uint(ga), __float_as_uint(gx),
                                                __float_as_uint(gy), 0u));
        }
      }
    }
    if (tid < NPOS) pcount[tid] = 0;
    if (tid < kWave) bucket[tid] = 0;
    if (last_of_item) write_back(c0.d);
    load_value_tile(c1.d, next_new_item);
    if (refill && wave == 0) {
      // wavefront 0 fetches the taken item's descriptor (scalar loads) and
      // hands it over through LDS: it has slack before the barrier (the other
      // wavefronts finish phase E later), where every workgroup loading it
      // after the barrier waited a scalar memory round trip in the next
      // batch's first phase
      const uint32_t t = __builtin_amdgcn_readfirstlane(took);
      const uint32_t idx = lo + t < hi ? lo + t : kNoItem;
      bool ok;
      const Item d = item_of(idx, ok);
      if (lane == 0) {
        taken[0] = idx;
        taken_item = d;
      }
    }
    c0 = c1;
    c1 = advance(c1);
    lds_barrier();
    if (refill) {
      pre_ok = taken[0] != kNoItem;
      pre = taken_item;
    }
    if (!c0.valid) break;
  }
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
