// MSDA forward with the backward's record scatter fused in (gfx950).
//
// The tile-owned backward (msda_backward_tiles.hpp) needs every sample's
// 16-byte record {position << 23 | query << lp_log2 | sample, wx1, wy1, attn}
// in its primary tile's record range. Binning it as three kernels
// (bin_count -> bin_scan -> bin_scatter) reads the geometry twice and, on a
// second stream beside the forward, gains nothing: the forward row kernel
// holds 242 VGPRs per wavefront, so no binning wavefront fits next to it and
// the binning runs after it. Here bin_count, bin_cursors and bin_scan run first, with
// query chunks that are exactly the forward's blocks, and the forward block
// that computes a chunk's taps also writes the chunk's records:
//
//   sample(): a live sample's tap -> primary tile, its rank in the tile
//             (integer LDS counter), the record staged in LDS at the sample's
//             place in the block's tap order; a sample with no corner in its
//             level gets zero location/weight gradients (or no record);
//   finish(): the block's tile counts scanned, the staged records sorted by
//             tile in LDS and stored in tile order at the binning's cursors
//             (consecutive threads, consecutive records of one tile), then
//             the cells of the slab's empty and split tiles zeroed
//             (bin_scatter's duties).
//
// Storing each record straight from its lane at an LDS-atomic slot (no
// staging, no sort) measured slower: c2 forward + binning 630 against 525
// us, c4 bf16 1791 against 1510 us.
//
// The records, tile ranges and work items are those of the three-kernel
// binning, so msda_tile_backward runs on them unchanged. The host takes this
// path only where the tile kernel writes the location and weight gradients
// straight to sample order (BinPlan::direct), so no sample -> record index
// is written here.
#pragma once

#include "msda_backward_tiles.hpp"
#include "msda_kernels.hpp"

namespace msda {

// Bounds of the fused path (checked on the host): the block's staged samples
// (tap slots), and the dynamic LDS, which holds the staged records, a key per
// slot, the tile-sorted slot list and one word per tile of the slab. The
// budget keeps two forward blocks (8 wavefronts, the forward's register
// limit) on a CU beside their static LDS (at most 24 KB).
constexpr int kFwdBinSlots = 2048;
constexpr size_t kFwdBinDynLds = 56 * 1024;

__host__ __device__ constexpr size_t fwd_bin_lds_bytes(int slots, int tile_bound) {
  return static_cast<size_t>(slots) * 16 +               // staged records
         static_cast<size_t>(slots) * 4 +                // tile << 16 | rank per slot
         static_cast<size_t>((slots + 1) / 2) * 4 +      // tile-sorted slot list (16-bit)
         static_cast<size_t>(tile_bound + 1) * 4;        // tile counts, then offsets
}

// Host-built arguments of the fused binning.
struct FwdBinArgs {
  const uint32_t *cursors;     // bin_cursors' per-(chunk, tile) cursors, relative to the tile
  const uint32_t *tile_start;  // bin_scan's per-slab tile offsets
  const uint32_t *zero_tiles;  // per slab {count, tile...}: empty and split tiles
  uint4 *records;
  float *grad_loc, *grad_attn, *grad_value;
  BinPlan p;                   // chunk_q = the forward block's units
  int slots;                   // tap slots per block: 4 wavefronts x steps x taps per step
  void *probs;                 // PT != void: each sample's softmax probability, [.., L*P]
};

// PT: void, or the type in which the softmax probabilities are stored (the
// forward with logits, msda_forward_softmax_bin_rows): sample() then takes
// the sample's probability, stores it at the sample's place in `probs` (the
// softmax backward reads it) and records it rounded to PT, the weight the
// backward's tile kernel uses -- what binning the stored probabilities gives.
template <int C, int T, typename PT = void>
struct TileBinner {
  static constexpr bool kActive = true;
  static constexpr bool kProbs = !std::is_void<PT>::value;
  FwdBinArgs a;
  int bm, ch, b, m, nt;
  const Level *lv;
  int *ntc, *base;
  uint32_t *part;
  uint4 *stage;
  uint32_t *keys;
  uint16_t *sorted;
  uint32_t *loff;  // per tile: the block's count, then its exclusive offset; [nt] = total

  __device__ __forceinline__ TileBinner(const FwdBinArgs &args, unsigned char *dyn, int *ntc_s,
                                        int *base_s, uint32_t *part_s, int lb, const Shape &s)
      : a(args), ntc(ntc_s), base(base_s), part(part_s) {
    bm = lb / a.p.chunks;
    ch = lb % a.p.chunks;
    b = bm / s.heads;
    m = bm % s.heads;
    stage = reinterpret_cast<uint4 *>(dyn);
    keys = reinterpret_cast<uint32_t *>(stage + a.slots);
    sorted = reinterpret_cast<uint16_t *>(keys + a.slots);
    loff = reinterpret_cast<uint32_t *>(dyn + static_cast<size_t>(a.slots) * 20 +
                                        static_cast<size_t>((a.slots + 1) / 2) * 4);
  }

  // units of chunk ch of slab bm: queries [ch * chunk_q, (ch + 1) * chunk_q)
  __device__ __forceinline__ int64_t first_unit(int, int64_t, const Shape &s) const {
    return static_cast<int64_t>(bm) * s.queries + static_cast<int64_t>(ch) * a.p.chunk_q;
  }
  __device__ __forceinline__ int64_t end_unit(int, int64_t, const Shape &s) const {
    const int q1 = min(s.queries, (ch + 1) * a.p.chunk_q);
    return static_cast<int64_t>(bm) * s.queries + q1;
  }

  // Tile tables, cleared counters and slots.
  __device__ __forceinline__ void begin(const Level *levels, const Shape &s) {
    lv = levels;
    stage_tiles<T>(lv, s.levels, ntc, base);
    nt = base[s.levels];
    for (int i = threadIdx.x; i < nt; i += kBlock) loff[i] = 0;
    for (int i = threadIdx.x; i < a.slots; i += kBlock) keys[i] = kNoRecord;
    lds_barrier();
  }

  // One live sample (ok) of the block; slot < a.slots.
  __device__ __forceinline__ void sample(const Tap &t, int l, int q, int smp, float attn, bool ok,
                                         int slot, const Shape &s) {
    if (!ok) return;
    const size_t o = (static_cast<size_t>(b * s.queries + q) * s.heads + m) * s.lp + smp;
    if constexpr (kProbs) {
      const PT pr = from_float<PT>(attn);
      static_cast<PT *>(a.probs)[o] = pr;
      attn = to_float(pr);
    }
    if (!t.in) {  // no corner inside the level: zero gradients, no record
      a.grad_attn[o] = 0.0f;
      *reinterpret_cast<float2 *>(a.grad_loc + 2 * o) = make_float2(0.0f, 0.0f);
      return;
    }
    const int tile = primary_tile<T>(t, ntc[l], base[l]);
    const uint32_t rank = atomicAdd(&loff[tile], 1u);
    // top-left corner in the frame of its primary tile: [-1, T-1]^2 -> [0, T]^2
    const int ty = t.y0 < 0 ? 0 : t.y0, tx = t.x0 < 0 ? 0 : t.x0;
    const int pos = (t.y0 - (ty / T) * T + 1) * (T + 1) + (t.x0 - (tx / T) * T + 1);
    keys[slot] = (static_cast<uint32_t>(tile) << 16) | rank;
    stage[slot] = make_uint4((static_cast<uint32_t>(pos) << kPosShift) |
                                 (static_cast<uint32_t>(q) << a.p.lp_log2) |
                                 static_cast<uint32_t>(smp),
                             __float_as_uint(t.wx1), __float_as_uint(t.wy1),
                             __float_as_uint(attn));
  }

  __device__ __forceinline__ int lb_row() const { return bm * a.p.chunks + ch; }

  __device__ __forceinline__ void finish(const Shape &s) {
    lds_barrier();  // every tap staged and counted
    // tile counts -> block-local exclusive offsets, in place (each thread a
    // contiguous run of tiles)
    const int per = (nt + kBlock - 1) / kBlock;
    const int t0 = min(nt, static_cast<int>(threadIdx.x) * per), t1 = min(nt, t0 + per);
    uint32_t run = 0;
    for (int t = t0; t < t1; ++t) run += loff[t];
    uint32_t total;
    uint32_t off = block_exclusive(run, part, &total);
    for (int t = t0; t < t1; ++t) {
      const uint32_t n = loff[t];
      loff[t] = off;
      off += n;
    }
    lds_barrier();
    // slots in tile order
    for (int i = threadIdx.x; i < a.slots; i += kBlock) {
      const uint32_t key = keys[i];
      if (key != kNoRecord) sorted[loff[key >> 16] + (key & 0xffffu)] = static_cast<uint16_t>(i);
    }
    lds_barrier();
    // records out in tile order: consecutive i of one tile are consecutive
    // records of this chunk's range in that tile (the tile's start plus the
    // chunk's cursor). The cursors and starts (L2-resident) are loaded for
    // all of a thread's records first.
    constexpr int U = kFwdBinSlots / kBlock;
    const uint32_t *cur_row = a.cursors + static_cast<size_t>(lb_row()) * a.p.tile_bound;
    const uint32_t *ts_row = a.tile_start + static_cast<size_t>(bm) * (a.p.tile_bound + 1);
    uint4 *rec = a.records + static_cast<size_t>(bm) * a.p.rec_cap;
    uint32_t slot[U], at[U], cur[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int i = static_cast<int>(threadIdx.x) + u * kBlock;
      slot[u] = i < static_cast<int>(total) ? sorted[i] : 0u;
      const uint32_t tile = i < static_cast<int>(total) ? keys[slot[u]] >> 16 : 0u;
      at[u] = static_cast<uint32_t>(i) - loff[tile];
      cur[u] = ts_row[tile] + cur_row[tile];
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int i = static_cast<int>(threadIdx.x) + u * kBlock;
      if (i >= static_cast<int>(total)) break;
      const uint32_t r = cur[u] + at[u];
      // non-temporal: a chunk's run in a tile is a few records at the finest
      // level, written long before or after its neighbours' (other chunks),
      // so the L2 cannot merge the partial lines; plain stores measured
      // slower (c2 forward + binning 525 -> 577 us, c4 bf16 1510 -> 1590 us)
      store_nt(rec + r, stage[slot[u]]);  // read once, by the tile kernel
    }
    // non-boundary cells of the slab's empty and split tiles listed by
    // bin_scan: tiles ch, ch + chunks, ... of the list
    const uint32_t *zl = a.zero_tiles + static_cast<size_t>(bm) * (a.p.tile_bound + 1);
    const uint32_t nz = zl[0];
    const int MC = s.heads * C;
    const size_t slab = static_cast<size_t>(b) * s.spatial * MC + m * C;
    for (uint32_t z = ch; z < nz; z += a.p.chunks) {
      const TileGeom g = tile_geom(static_cast<int>(zl[1 + z]), T, ntc, base);
      zero_tile_cells<C, T>(a.grad_value, slab, MC, lv[g.l], g, threadIdx.x, kBlock,
                            [&](int r, int c) { return !boundary_cell(r, c, g); });
    }
  }
};

// The forward row kernel over chunk (lb % chunks) of slab (lb / chunks),
// binning the chunk's samples as it goes (TileBinner). Grid: slabs x chunks
// blocks, logical blocks contiguous per XCD.
template <typename VT, typename GT, int C, int NS, int T>
__global__ void __launch_bounds__(kBlock, kRowWavesPerSimd)
    msda_forward_bin_rows(const VT *__restrict__ value, uint32_t value_bytes,
                          const int64_t *__restrict__ shapes, const int64_t *__restrict__ starts,
                          const GT *__restrict__ loc, const GT *__restrict__ attn,
                          VT *__restrict__ out, Shape s, RowPlan plan, FwdBinArgs args) {
  extern __shared__ __align__(16) unsigned char fwd_bin_dyn[];
  __shared__ int ntc[kMaxLevels], base[kMaxLevels + 1];
  __shared__ uint32_t part[kBlock / kWave];
  const int lb = xcd_logical_block(blockIdx.x, gridDim.x);
  TileBinner<C, T> bin(args, fwd_bin_dyn, ntc, base, part, lb, s);
  forward_rows<VT, GT, C, NS, DenseRows<VT>, false, TileBinner<C, T>>(
      value, value_bytes, shapes, starts, loc, attn, DenseRows<VT>{out}, s, plan, lb, bin);
}

// The same with the attention weights given as logits (the softmax over each
// unit's L*P samples fused into the prologue, forward_rows kSoftmax): every
// sample's probability goes to args.probs (GT) and into its record. Only for
// plans whose units are one step each (the host checks), where a sample's
// probability is final when its tap is computed.
template <typename VT, typename GT, int C, int NS, int T>
__global__ void __launch_bounds__(kBlock, kRowWavesPerSimd)
    msda_forward_softmax_bin_rows(const VT *__restrict__ value, uint32_t value_bytes,
                                  const int64_t *__restrict__ shapes,
                                  const int64_t *__restrict__ starts, const GT *__restrict__ loc,
                                  const GT *__restrict__ logits, VT *__restrict__ out, Shape s,
                                  RowPlan plan, FwdBinArgs args) {
  extern __shared__ __align__(16) unsigned char fwd_bin_dyn[];
  __shared__ int ntc[kMaxLevels], base[kMaxLevels + 1];
  __shared__ uint32_t part[kBlock / kWave];
  const int lb = xcd_logical_block(blockIdx.x, gridDim.x);
  TileBinner<C, T, GT> bin(args, fwd_bin_dyn, ntc, base, part, lb, s);
  forward_rows<VT, GT, C, NS, DenseRows<VT>, true, TileBinner<C, T, GT>>(
      value, value_bytes, shapes, starts, loc, logits, DenseRows<VT>{out}, s, plan, lb, bin);
}

}  // namespace msda
