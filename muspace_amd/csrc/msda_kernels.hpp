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
// The forward row kernels are built for two of their blocks per CU (two
// wavefronts per SIMD), so at most 256 registers a lane: past that (even one
// register kept in an AGPR) gfx950 allocates the next granule and a SIMD holds
// one wavefront. The launch bound makes the compiler keep to it.
constexpr int kRowWavesPerSimd = 2;

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

// Unit u, advanced in steps of `stride` units without divisions.
struct UnitIter {
  int b, m, q;
  __device__ __forceinline__ void init(int64_t u, const Shape &s) {
    q = static_cast<int>(u % s.queries);
    const int64_t t = u / s.queries;
    m = static_cast<int>(t % s.heads);
    b = static_cast<int>(t / s.heads);
  }
  __device__ __forceinline__ void advance(int stride, const Shape &s) {
    q += stride;
    while (q >= s.queries) {  // at most stride / queries + 1 times
      q -= s.queries;
      if (++m == s.heads) {
        m = 0;
        ++b;
      }
    }
  }
  __device__ __forceinline__ int si(const Shape &s) const { return (b * s.queries + q) * s.heads + m; }
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

// Where a forward unit (b, q, m) reads its geometry and value, and what it does
// with its C sums.
//
// DenseRows: the operator's output, out[(b*nq + q)*M + m][C]; geometry row
// (b, q, m) of [batch, nq, M, L*P]; value slab b of [batch, spatial, M, C].
template <typename VT>
struct DenseRows {
  VT *out;
  // geometry row of (b, q, m) and first value row of its slab
  __device__ __forceinline__ void locate(int b, int q, int m, const Shape &s, int &row,
                                         size_t &slab) const {
    row = (b * s.queries + q) * s.heads + m;
    slab = static_cast<size_t>(b) * s.spatial;
  }
  // what the epilogue of a unit loads ahead of time (nothing here)
  static constexpr bool kLoadsAhead = false;
  struct Ticket {};
  __device__ __forceinline__ void fetch_index(Ticket &, int) const {}
  __device__ __forceinline__ void fetch_count(Ticket &, int, const Shape &) const {}
  template <int C, int CPL>
  __device__ __forceinline__ void put(int b, int q, int m, int k, const float (&acc)[CPL],
                                      const Ticket &, const Shape &s) const {
    store16_nt(out + static_cast<size_t>((b * s.queries + q) * s.heads + m) * C + k * CPL, acc);
  }
  __device__ __forceinline__ void put1(int b, int q, int m, int c, float acc,
                                       const Shape &s) const {
    out[static_cast<size_t>((b * s.queries + q) * s.heads + m) * s.channels + c] =
        from_float<VT>(acc);
  }
};

constexpr int kMaxCams = 16;  // cameras per scatter-average launch

// CameraSlots: BEVFormer spatial cross-attention's epilogue, fused into the
// forward (reference sketch: ms_deformable_im2col_scatter_div_*,
// /root/reference/csrc/ms_deformable_attn/ms_deform_attn_musa_kernel.muh:419-486).
// Value and geometry are camera-rebatched, [batch*cams, spatial, M, C] and
// [batch*cams, max_len, M, L*P]. A launch covers cameras cam0 .. cam0+ncam-1;
// their valid rows are numbered back to back, q = off[j] + r for row
// r < off[j+1] - off[j] of camera cam0 + j, and index[q] is that row's BEV
// query. Unit (b, q, m) adds its sums to slot (b, index[q], m):
//   slots[b, index[q], m*C + c] += sum_c * (1 / count[b, index[q]]).
// kAtomic: the launch holds several cameras, which may share a slot, and adds
// with fp32 global atomics (float slots only). Otherwise the launch holds one
// camera, whose indices are distinct, and a plain read-modify-write suffices;
// cameras are then launched in order. An index outside [0, num_query) adds
// nothing. The row kernels cut the launch's blocks into one segment per
// camera (blk[]), so that every block works on one camera (segment()).
template <typename VT, typename GT, bool kAtomic>
struct CameraSlots {
  VT *slots;             // [batch, num_query, M*C]
  const int64_t *index;  // [off[ncam]] BEV query of each valid row
  const GT *count;       // [batch, num_query], cameras that see the query
  int cams, cam0, ncam, max_len, num_query;
  int off[kMaxCams + 1];  // first q of each camera of the launch; off[ncam] = valid rows
  int blk[kMaxCams + 1];  // row kernels: first logical block of each camera's segment
  static_assert(!kAtomic || std::is_same<VT, float>::value, "atomic slots are float32");

  // The camera of logical block lb (uniform across the block: scalar code).
  // Returns this policy narrowed to that camera, turns lb into the block's
  // index inside the camera's segment and s into the camera's shape
  // (s.queries = its valid rows).
  __device__ __forceinline__ CameraSlots segment(int &lb, Shape &s) const {
    int j = 0;
#pragma unroll
    for (int c = 1; c < kMaxCams; ++c) j = c < ncam && lb >= blk[c] ? c : j;
    int first = 0, len = 0, b0 = 0;  // constant indices only
#pragma unroll
    for (int c = 0; c < kMaxCams; ++c) {
      if (c == j) {
        first = off[c];
        len = off[c + 1] - off[c];
        b0 = blk[c];
      }
    }
    CameraSlots o = *this;
    o.index = index + first;
    o.cam0 = cam0 + j;
    o.ncam = 1;
    o.off[0] = 0;
    o.off[1] = len;
    s.queries = len;
    s.units = s.batch * len * s.heads;
    lb -= b0;
    return o;
  }

  __device__ __forceinline__ void locate(int b, int q, int m, const Shape &s, int &row,
                                         size_t &slab) const {
    int j = 0, first = 0;  // constant indices only: off[] stays in scalar registers
    if (ncam > 1) {
#pragma unroll
      for (int c = 1; c < kMaxCams; ++c) {
        if (c < ncam && q >= off[c]) {
          j = c;
          first = off[c];
        }
      }
    }
    const int cam = cam0 + j;
    row = ((b * cams + cam) * max_len + (q - first)) * s.heads + m;
    slab = static_cast<size_t>(b * cams + cam) * s.spatial;
  }
  // slot row of (b, q, m) and the factor 1/count, or nullptr outside the grid
  __device__ __forceinline__ VT *slot(int b, int q, int m, const Shape &s, float &inv) const {
    const int64_t bev = index[q];
    if (bev < 0 || bev >= num_query) return nullptr;
    const int64_t bq = static_cast<int64_t>(b) * num_query + bev;
    inv = 1.0f / to_float(count[bq]);
    return slots + (bq * s.heads + m) * s.channels;
  }
  // A unit's BEV query and count, loaded ahead of its epilogue: the index one
  // unit early, the count when the unit starts (before its gathers, so the
  // in-order wait for the gathers covers it). Loads are unconditional with
  // clamped offsets (q < s.queries always; count[0] exists: num_query > 0).
  static constexpr bool kLoadsAhead = true;
  struct Ticket {
    int64_t bev;
    float count;
  };
  __device__ __forceinline__ void fetch_index(Ticket &tk, int q) const { tk.bev = index[q]; }
  __device__ __forceinline__ void fetch_count(Ticket &tk, int b, const Shape &s) const {
    const bool ok = b < s.batch && tk.bev >= 0 && tk.bev < num_query;
    tk.count = to_float(count[ok ? static_cast<int64_t>(b) * num_query + tk.bev : 0]);
  }
  template <int C, int CPL>
  __device__ __forceinline__ void put(int b, int q, int m, int k, const float (&acc)[CPL],
                                      const Ticket &tk, const Shape &s) const {
    if (tk.bev < 0 || tk.bev >= num_query) return;
    const float inv = 1.0f / tk.count;
    VT *row = slots + ((static_cast<int64_t>(b) * num_query + tk.bev) * s.heads + m) * C;
    if constexpr (kAtomic) {
#pragma unroll
      for (int c = 0; c < CPL; ++c) unsafeAtomicAdd(row + k * CPL + c, acc[c] * inv);
    } else {
      float cur[CPL];
      load16(row + k * CPL, cur);
#pragma unroll
      for (int c = 0; c < CPL; ++c) cur[c] += acc[c] * inv;
      store16(row + k * CPL, cur);
    }
  }
  __device__ __forceinline__ void put1(int b, int q, int m, int c, float acc,
                                       const Shape &s) const {
    float inv;
    VT *row = slot(b, q, m, s, inv);
    if (row == nullptr) return;
    if constexpr (kAtomic) {
      unsafeAtomicAdd(row + c, acc * inv);
    } else {
      row[c] = from_float<VT>(to_float(row[c]) + acc * inv);
    }
  }
};

// Hooks of forward_rows that also fix a block's units. NoBin: blocks of
// per_block consecutive units (in the order u = (b*M + m)*nq + q), no
// binning. A binning hook (TileBinner, msda_backward_tiles.hpp) sees each live
// sample's tap as the forward computes it.
struct NoBin {
  static constexpr bool kActive = false;
  __device__ __forceinline__ int64_t first_unit(int lb, int64_t per_block, const Shape &) const {
    return static_cast<int64_t>(lb) * per_block;
  }
  __device__ __forceinline__ int64_t end_unit(int, int64_t, const Shape &s) const {
    return s.units;
  }
  __device__ __forceinline__ void begin(const Level *, const Shape &) {}
  __device__ __forceinline__ void sample(const Tap &, int, int, int, float, bool, int,
                                         const Shape &) {}
  __device__ __forceinline__ void finish(const Shape &) {}
};

// Forward row kernel. Per step (a chunk of NS samples for each lane group),
// lane i < NG*NS computes one sample's bilinear tap -- the four corner byte
// offsets (kOobOffset for a corner outside the level) and the four weights
// with the attention weight folded in -- into a wavefront-private LDS table;
// lane group g then gathers the corner rows of its NS samples with 16-byte
// buffer loads (out-of-range offsets read zeros) and accumulates.
//
// Software pipeline (NS >= 4): a step's gathers are issued in two halves and
// the loop always keeps one half in flight while it consumes the other --
// issue H1(st), consume H0(st), tap of step st+1, issue H0(st+1), consume
// H1(st) -- so a wavefront never waits for all of a step's corner rows with
// nothing else outstanding (with two wavefronts per SIMD that wait left the
// memory pipe idle: c2 forward 382 -> 366 us). NS <= 2 issues and consumes
// a step in place. The next step's
// geometry is loaded right after its first stage is issued (vmcnt counts in
// issue order), and every load is unconditional (clamped indices; a load
// inside a branch is waited for before the branch joins). The tap tables are
// double-buffered by step parity and padded by one entry per lane group, so
// the NG groups' reads of one sample slot fall in different LDS banks.
// value_bytes < 2^31 (checked on the host) keeps every offset in 32 bits.
//
// kSoftmax: `attn` holds logits, and each unit's weights are their softmax
// over its L*P samples. A unit's tap lanes are one aligned block of GU*NS
// lanes, so the softmax is a running max and sum over that block (DPP and
// readlane reductions) per step, the online form: a step that raises the
// unit's max rescales the accumulators by exp(old max - new max), and the
// unit's row is scaled by 1/sum before it is stored. When a unit fits one
// step (the common case, L*P <= GU*NS) that is the plain exp(x - max) / sum.
// The reductions are branch-free (every step computed, uniform selects), so
// they schedule with the tap's own arithmetic.
template <typename VT, typename GT, int C, int NS, typename Out, bool kSoftmax = false,
          typename Bin = NoBin>
__device__ __forceinline__ void forward_rows(const VT *__restrict__ value, uint32_t value_bytes,
                                             const int64_t *__restrict__ shapes,
                                             const int64_t *__restrict__ starts,
                                             const GT *__restrict__ loc,
                                             const GT *__restrict__ attn, const Out &out,
                                             const Shape &s, const RowPlan &plan, int lb,
                                             Bin &bin) {
  constexpr int CPL = RowTraits<VT>::kCpl;
  constexpr int VB = static_cast<int>(sizeof(VT));
  constexpr int KQ = C / CPL;
  constexpr int NG = kWave / KQ;
  // stages per step: NS >= 4 gathers a step in two halves; NS <= 2 in one
  constexpr int NSPLIT = NS >= 4 ? 2 : 1;
  constexpr int NH = NS / NSPLIT;  // samples per stage
  // tap table: one padding entry per lane group when NS >= 4, so the groups'
  // reads of one sample slot fall in different LDS banks (NS = 1 is
  // conflict-free as it is; NS = 2 measured no gain)
  constexpr int PAD = NSPLIT == 2 ? 1 : 0;
  static_assert(NSPLIT == 1 || NS % 2 == 0, "two equal halves");
  constexpr int TW = kWave + PAD * (kWave / NS);  // table entries per wavefront
  static_assert(C % CPL == 0 && (KQ & (KQ - 1)) == 0 && KQ <= kWave, "bad row layout");
  static_assert(NG * NS <= kWave, "one tap per lane");

  __shared__ Level lv[kMaxLevels];
  // double-buffered by step parity when a step's tap is written while the
  // previous step is still being consumed (NSPLIT == 2)
  __shared__ u32x4 tap_off[NSPLIT][(kBlock / kWave) * TW];
  __shared__ float4 tap_w[NSPLIT][(kBlock / kWave) * TW];
  // kSoftmax, per step parity and unit slot: the step's rescale and 1/sum
  __shared__ float2 unit_norm[2][kSoftmax ? kBlock : 1];
  stage_levels(lv, shapes, starts, s);
  bin.begin(lv, s);
  const __amdgpu_buffer_rsrc_t vr = make_rsrc(value, value_bytes);

  const int lane = threadIdx.x % kWave;
  const int wave = threadIdx.x / kWave;
  const int grp = lane / KQ, k = lane % KQ;
  const int GU = 1 << plan.gu_log2;
  const int UW = NG >> plan.gu_log2;  // units per wave iteration
  const int gi = grp & (GU - 1);
  const int slot = grp >> plan.gu_log2;
  const int MC = s.heads * C;
  // the sample this lane computes the tap of: sample tj of lane group tg
  const int tg = min(lane / NS, NG - 1), tj = lane % NS;
  const int tgi = tg & (GU - 1), tslot = tg >> plan.gu_log2;
  // table entry of lane group g's sample j: g * (NS + PAD) + j
  const int my_entry = wave * TW + tg * (NS + PAD) + tj;
  const int grp_entry = wave * TW + grp * (NS + PAD);

  const int chunks = (s.lp + GU * NS - 1) / (GU * NS);
  const int steps = plan.iters * chunks;

  // geometry of this lane's tap sample in step st; the tap unit and the
  // output unit advance by UW units per wave iteration. The block's units
  // are [first_unit, end_unit) (the hook object decides; NoBin: blocks of
  // per_block consecutive units up to s.units)
  const int64_t per_block = static_cast<int64_t>(kBlock / kWave) * plan.iters * UW;
  const int64_t u_first = bin.first_unit(lb, per_block, s) +
                          static_cast<int64_t>(wave) * plan.iters * UW;
  const int64_t u_end = bin.end_unit(lb, per_block, s);
  UnitIter tu, ou, on;  // on: the output unit after ou
  tu.init(u_first + tslot, s);
  ou.init(u_first + slot, s);
  typename Out::Ticket tk_cur, tk_next;  // epilogue data of ou and on
  if constexpr (Out::kLoadsAhead) {
    on = ou;
    on.advance(UW, s);
    out.fetch_index(tk_cur, ou.q);
    out.fetch_index(tk_next, on.q);
  }
  float lx, ly, a;
  bool ok;
  int sm;
  uint32_t unit_base;  // byte offset of the tap unit's (b, head m) in value
  // kSoftmax: the tap unit's running max and sum, and this lane's weight
  // exp(x - max) for the current step
  float m_run = 0.0f, s_run = 0.0f, e_cur = 0.0f;
  auto softmax_step = [&](int st) {  // the logit of step st is `a`
    const int tb = GU * NS;  // the unit's tap lanes: an aligned block
    const float x = ok ? a : -INFINITY;
    const float mx = group_max_sel(x, tb);
    if (st % chunks == 0) {
      m_run = -INFINITY;
      s_run = 0.0f;
    }
    const float m_new = fmaxf(m_run, mx);
    const bool none = m_new == -INFINITY;  // no finite logit yet
    const float sc = none ? 1.0f : __expf(m_run - m_new);
    e_cur = ok && !none ? __expf(x - m_new) : 0.0f;
    const float es = group_sum_sel(e_cur, tb);
    s_run = s_run * sc + es;
    m_run = m_new;
    if (lane < NG * NS && (lane & (tb - 1)) == 0) {
      // hardware reciprocal (1 ulp); 1/0 = inf keeps an all -inf unit NaN
      unit_norm[st & 1][wave * kWave + tslot] = make_float2(sc, __builtin_amdgcn_rcpf(s_run));
    }
  };
  auto load_geometry = [&](int st) {
    const int it = st / chunks, s0 = (st % chunks) * GU * NS;
    if (st > 0 && st % chunks == 0) tu.advance(UW, s);
    const int64_t u64 = u_first + static_cast<int64_t>(it) * UW + tslot;
    const bool live = st < steps && u64 < u_end && lane < NG * NS;
    const int smp = s0 + tgi + GU * tj;
    ok = live && smp < s.lp;
    sm = ok ? smp : 0;
    int grow = 0;
    size_t slab = 0;
    if (live) out.locate(tu.b, tu.q, tu.m, s, grow, slab);
    const size_t o = static_cast<size_t>(grow) * s.lp + sm;
    lx = load_nt(&loc[2 * o]);  // geometry streams through once
    ly = load_nt(&loc[2 * o + 1]);
    a = load_nt(&attn[o]);
    unit_base = static_cast<uint32_t>((slab * MC + tu.m * C) * VB);
  };
  // A. this lane's tap of step st (geometry loaded) into table st & 1
  auto tap = [&](int st) {
    const int l = level_of_sample(sm, s);
    const Level L = lv[l];
    const Tap t = make_tap(lx, ly, L, ok);
    // the binning hook sees every live sample once: slot = its place in the
    // block's tap order (st < steps whenever ok)
    [[maybe_unused]] const int bin_slot = (wave * steps + st) * (NG * NS) + lane;
    if constexpr (Bin::kActive && !kSoftmax) {
      bin.sample(t, l, tu.q, sm, ok ? a : 0.0f, ok, bin_slot, s);
    }
    float ai = ok ? a : 0.0f;
    if constexpr (kSoftmax) {
      softmax_step(st);
      ai = e_cur;  // 0 unless ok
      if constexpr (Bin::kActive) {
        // the sample's probability exp(x - max) / sum, final here because
        // the host fuses the binning only where a unit is one step (chunks
        // == 1: the max and sum cover all of the unit's logits); the same
        // 1/sum scales the unit's output row in end_step
        bin.sample(t, l, tu.q, sm, ai * __builtin_amdgcn_rcpf(s_run), ok, bin_slot, s);
      }
    }
    const uint32_t row = static_cast<uint32_t>(MC * VB);
    const uint32_t c00 = unit_base + static_cast<uint32_t>(L.start + t.cell00) * row;
    const uint32_t c10 = c00 + static_cast<uint32_t>(L.w) * row;
    u32x4 off;
    off.x = t.y0ok && t.x0ok ? c00 : kOobOffset;
    off.y = t.y0ok && t.x1ok ? c00 + row : kOobOffset;
    off.z = t.y1ok && t.x0ok ? c10 : kOobOffset;
    off.w = t.y1ok && t.x1ok ? c10 + row : kOobOffset;
    if (lane < NG * NS) {  // lanes past the taps would alias group NG-1's entries
      const int tb = st & (NSPLIT - 1);
      tap_off[tb][my_entry] = off;
      tap_w[tb][my_entry] = make_float4(ai * (t.wy0 * t.wx0), ai * (t.wy0 * t.wx1),
                                        ai * (t.wy1 * t.wx0), ai * (t.wy1 * t.wx1));
    }
  };
  // B. gathers of stage h of step st (this lane group's samples h*NH ..
  // h*NH + NH - 1)
  const uint32_t ch = static_cast<uint32_t>(k * 16);
  auto issue = [&](int st, int h, u32x4 (&raw)[NH][4]) {
#pragma unroll
    for (int j = 0; j < NH; ++j) {
      const u32x4 off = tap_off[st & (NSPLIT - 1)][grp_entry + h * NH + j];
      raw[j][0] = buffer_load16(vr, off.x + ch);
      raw[j][1] = buffer_load16(vr, off.y + ch);
      raw[j][2] = buffer_load16(vr, off.z + ch);
      raw[j][3] = buffer_load16(vr, off.w + ch);
    }
  };
  // C. accumulate half h of step st
  float acc[CPL];
#pragma unroll
  for (int j = 0; j < CPL; ++j) acc[j] = 0.0f;
  auto consume = [&](int st, int h, const u32x4 (&raw)[NH][4]) {
#pragma unroll
    for (int j = 0; j < NH; ++j) {
      const float4 w = tap_w[st & (NSPLIT - 1)][grp_entry + h * NH + j];
      float v0[CPL], v1[CPL], v2[CPL], v3[CPL];
      decode16(VT(), raw[j][0], v0);
      decode16(VT(), raw[j][1], v1);
      decode16(VT(), raw[j][2], v2);
      decode16(VT(), raw[j][3], v3);
#pragma unroll
      for (int c = 0; c < CPL; ++c) {
        acc[c] += w.x * v0[c] + w.y * v1[c] + w.z * v2[c] + w.w * v3[c];
      }
    }
  };

  // the start of step st: its unit's epilogue data; kSoftmax with a unit of
  // several steps: rescale to the step's running max, which tap(st) wrote
  // (so tap(st) must come first)
  auto begin_step = [&](int st) {
    if (st % chunks == 0) out.fetch_count(tk_cur, ou.b, s);
    if constexpr (kSoftmax) {
      if (chunks > 1) {
        const float sc = unit_norm[st & 1][wave * kWave + slot].x;
#pragma unroll
        for (int j = 0; j < CPL; ++j) acc[j] *= sc;
      }
    }
  };
  // D. the end of step st; at the end of a unit sum the GU groups (lane
  // distance KQ, 2KQ, ...) and store. Steps past the last one (the step
  // pipeline rounds up to pairs) end nothing.
  auto end_step = [&](int st) {
    if (st >= steps || st % chunks != chunks - 1) return;
    for (int off = KQ; off < KQ * GU; off <<= 1) {
#pragma unroll
      for (int j = 0; j < CPL; ++j) acc[j] += __shfl_xor(acc[j], off, kWave);
    }
    if constexpr (kSoftmax) {
      const float inv = unit_norm[st & 1][wave * kWave + slot].y;
#pragma unroll
      for (int j = 0; j < CPL; ++j) acc[j] *= inv;
    }
    const int64_t u64 = u_first + static_cast<int64_t>(st / chunks) * UW + slot;
    if (u64 < u_end && gi == 0) {
      out.template put<C, CPL>(ou.b, ou.q, ou.m, k, acc, tk_cur, s);
    }
    if constexpr (Out::kLoadsAhead) {
      ou = on;
      tk_cur = tk_next;
      on.advance(UW, s);
      out.fetch_index(tk_next, on.q);
    } else {
      ou.advance(UW, s);
    }
#pragma unroll
    for (int j = 0; j < CPL; ++j) acc[j] = 0.0f;
  };
  // Past the last step the taps have zero weights and out-of-range offsets
  // (which read zeros), so the pipeline's look-ahead is harmless.
  u32x4 raw0[NH][4], raw1[NH][4];
  load_geometry(0);
  if constexpr (NSPLIT == 2) {
    tap(0);
    issue(0, 0, raw0);
    load_geometry(1);
    for (int st = 0; st < steps; ++st) {
      begin_step(st);
      issue(st, 1, raw1);
      consume(st, 0, raw0);
      // the next step's tap and first half, then its successor's geometry
      tap(st + 1);
      issue(st + 1, 0, raw0);
      load_geometry(st + 2);
      consume(st, 1, raw1);
      end_step(st);
    }
  } else {
    // one or two samples per group: a step's few gathers are issued and
    // consumed in place (double-buffering whole steps measured slower here:
    // c1 179 -> 201 us, c3 133 -> 137 us)
    (void)raw1;
    for (int st = 0; st < steps; ++st) {
      // the tap first: with kSoftmax it writes the step's rescale, which
      // begin_step applies
      tap(st);
      begin_step(st);
      issue(st, 0, raw0);
      load_geometry(st + 1);
      consume(st, 0, raw0);
      end_step(st);
    }
  }
  bin.finish(s);
}

template <typename VT, typename GT, int C, int NS>
__global__ void __launch_bounds__(kBlock, kRowWavesPerSimd)
    msda_forward_rows(const VT *__restrict__ value, uint32_t value_bytes,
                      const int64_t *__restrict__ shapes, const int64_t *__restrict__ starts,
                      const GT *__restrict__ loc, const GT *__restrict__ attn,
                      VT *__restrict__ out, Shape s, RowPlan plan) {
  NoBin nb;
  forward_rows<VT, GT, C, NS>(value, value_bytes, shapes, starts, loc, attn, DenseRows<VT>{out},
                              s, plan, xcd_logical_block(blockIdx.x, gridDim.x), nb);
}

// Forward with the attention weights given as logits: softmax over each
// unit's L*P samples fused into the prologue (forward_rows, kSoftmax).
template <typename VT, typename GT, int C, int NS>
__global__ void __launch_bounds__(kBlock, kRowWavesPerSimd)
    msda_forward_softmax_rows(const VT *__restrict__ value, uint32_t value_bytes,
                              const int64_t *__restrict__ shapes,
                              const int64_t *__restrict__ starts, const GT *__restrict__ loc,
                              const GT *__restrict__ logits, VT *__restrict__ out, Shape s,
                              RowPlan plan) {
  NoBin nb;
  forward_rows<VT, GT, C, NS, DenseRows<VT>, true>(value, value_bytes, shapes, starts, loc,
                                                   logits, DenseRows<VT>{out}, s, plan,
                                                   xcd_logical_block(blockIdx.x, gridDim.x), nb);
}

// Cameras of the spatial cross-attention, summed into the BEV slots
// (CameraSlots above); s.batch is the batch. Each camera's units take the
// logical blocks [out.blk[j], out.blk[j+1]).
template <typename VT, typename GT, int C, int NS, bool kAtomic>
__global__ void __launch_bounds__(kBlock, kRowWavesPerSimd)
    msda_forward_scatter_div_rows(const VT *__restrict__ value, uint32_t value_bytes,
                                  const int64_t *__restrict__ shapes,
                                  const int64_t *__restrict__ starts, const GT *__restrict__ loc,
                                  const GT *__restrict__ attn, CameraSlots<VT, GT, kAtomic> out,
                                  Shape s, RowPlan plan) {
  int lb = xcd_logical_block(blockIdx.x, gridDim.x);
  Shape sc = s;
  const CameraSlots<VT, GT, kAtomic> cam = out.segment(lb, sc);
  NoBin nb;
  forward_rows<VT, GT, C, NS>(value, value_bytes, shapes, starts, loc, attn, cam, sc, plan, lb, nb);
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

template <typename VT, typename GT, typename Out>
__device__ __forceinline__ void forward_generic(const VT *__restrict__ value,
                                                const int64_t *__restrict__ shapes,
                                                const int64_t *__restrict__ starts,
                                                const GT *__restrict__ loc,
                                                const GT *__restrict__ attn, const Out &out,
                                                const Shape &s) {
  __shared__ Level lv[kMaxLevels];
  stage_levels(lv, shapes, starts, s);
  const int C = s.channels, MC = s.heads * C;
  const int64_t total = static_cast<int64_t>(s.units) * C;
  for (int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; idx < total;
       idx += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int c = static_cast<int>(idx % C);
    const int si = static_cast<int>(idx / C);  // (b*nq + q)*M + m
    const int m = si % s.heads;
    const int q = (si / s.heads) % s.queries;
    const int b = si / (s.heads * s.queries);
    int row;
    size_t slab;
    out.locate(b, q, m, s, row, slab);
    const VT *vbase = value + slab * MC + m * C + c;
    const GT *lbase = loc + static_cast<size_t>(row) * s.lp * 2;
    const GT *abase = attn + static_cast<size_t>(row) * s.lp;
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
    out.put1(b, q, m, c, acc, s);
  }
}

template <typename VT, typename GT>
__global__ void __launch_bounds__(kBlock, kRowWavesPerSimd)
    msda_forward_generic(const VT *__restrict__ value, const int64_t *__restrict__ shapes,
                         const int64_t *__restrict__ starts, const GT *__restrict__ loc,
                         const GT *__restrict__ attn, VT *__restrict__ out, Shape s) {
  forward_generic<VT, GT>(value, shapes, starts, loc, attn, DenseRows<VT>{out}, s);
}

template <typename VT, typename GT, bool kAtomic>
__global__ void __launch_bounds__(kBlock, kRowWavesPerSimd)
    msda_forward_scatter_div_generic(const VT *__restrict__ value,
                                     const int64_t *__restrict__ shapes,
                                     const int64_t *__restrict__ starts,
                                     const GT *__restrict__ loc, const GT *__restrict__ attn,
                                     CameraSlots<VT, GT, kAtomic> out, Shape s) {
  forward_generic<VT, GT>(value, shapes, starts, loc, attn, out, s);
}

// Valid rows of each camera: camera c's rows r < len[c] are q = off[c] + r of
// the concatenated index.
struct CameraRows {
  int off[kMaxCams], len[kMaxCams];
};

// Backward of the scatter-average: the gradient of the cameras' MSDA output
// rows, grad_out[(b*cams + cam)*max_len + r][row] =
// grad_slots[b, index[off[cam] + r]][row] / count[b, index[off[cam] + r]] for
// r < len[cam]; rows past len[cam] (the rebatch padding) and indices outside
// [0, num_query) get zeros. Grid row blockIdx.y handles camera cam0 +
// blockIdx.y, so the table lookup is uniform across a block; W = 16 /
// sizeof(VT) elements per thread (16-byte rows) or 1.
template <typename VT, typename GT, int W>
__global__ void __launch_bounds__(kBlock)
    msda_scatter_div_grad(const VT *__restrict__ grad_slots, const int64_t *__restrict__ index,
                          const GT *__restrict__ count, VT *__restrict__ grad_out, int batch,
                          int cams, int cam0, CameraRows rows, int max_len, int num_query,
                          int row) {
  static_assert(W == 1 || W * sizeof(VT) == 16, "one element or one 16-byte chunk per thread");
  const int j = blockIdx.y;
  int off = 0, valid = 0;
#pragma unroll
  for (int c = 0; c < kMaxCams; ++c) {
    if (c == j) {
      off = rows.off[c];
      valid = rows.len[c];
    }
  }
  const int cam = cam0 + j;
  const int per_row = row / W;
  const int64_t total = static_cast<int64_t>(batch) * max_len * per_row;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int e0 = static_cast<int>(i % per_row);
    const int64_t br = i / per_row;
    const int r = static_cast<int>(br % max_len);
    const int b = static_cast<int>(br / max_len);
    float v[W];
#pragma unroll
    for (int e = 0; e < W; ++e) v[e] = 0.0f;
    if (r < valid) {
      const int64_t bev = index[off + r];
      if (bev >= 0 && bev < num_query) {
        const int64_t bq = static_cast<int64_t>(b) * num_query + bev;
        const float inv = 1.0f / to_float(count[bq]);
        const VT *src = grad_slots + bq * row + static_cast<int64_t>(e0) * W;
        if constexpr (W == 1) {
          v[0] = to_float(src[0]);
        } else {
          load16(src, v);
        }
#pragma unroll
        for (int e = 0; e < W; ++e) v[e] *= inv;
      }
    }
    VT *dst = grad_out + (static_cast<int64_t>(b * cams + cam) * max_len + r) * row +
              static_cast<int64_t>(e0) * W;
    if constexpr (W == 1) {
      dst[0] = from_float<VT>(v[0]);
    } else {
      store16(dst, v);
    }
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
// ------------------------------------------------------------ softmax ---

// Softmax of each unit's L*P logits and its backward, for the paths that do
// not fuse it (the binning of the backward, the generic and atomic kernels).
// A unit is W <= 16 consecutive lanes (W = pow2 >= L*P / 4, so about four
// samples per lane; the reductions stay in DPP); a lane takes the unit's
// samples i, i + W, ... (contiguous across the unit's lanes).
template <typename GT>
__global__ void __launch_bounds__(kBlock)
    msda_softmax_units(const GT *__restrict__ logits, GT *__restrict__ probs, Shape s,
                       int w_log2) {
  const int W = 1 << w_log2;
  const int64_t unit =
      (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) >> w_log2;
  const int i = threadIdx.x & (W - 1);
  const bool live = unit < s.units;
  const GT *x = logits + (live ? unit : 0) * s.lp;
  float mx = -INFINITY;
  for (int j = i; j < s.lp; j += W) mx = fmaxf(mx, to_float(x[j]));
  mx = group_max_n(mx, W);
  const bool none = mx == -INFINITY;
  float sum = 0.0f;
  for (int j = i; j < s.lp; j += W) sum += none ? 0.0f : expf(to_float(x[j]) - mx);
  sum = group_sum_n(sum, W);
  if (!live) return;
  const float inv = 1.0f / sum;
  GT *p = probs + unit * s.lp;
  for (int j = i; j < s.lp; j += W) {
    p[j] = from_float<GT>(none ? 0.0f * inv : expf(to_float(x[j]) - mx) * inv);
  }
}

// grad (in place) = p * (grad - sum_j p_j grad_j) over each unit's samples:
// the weight gradient becomes the logit gradient.
template <typename GT>
__global__ void __launch_bounds__(kBlock)
    msda_softmax_backward_units(const GT *__restrict__ probs, float *__restrict__ grad, Shape s,
                                int w_log2) {
  const int W = 1 << w_log2;
  const int64_t unit =
      (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) >> w_log2;
  const int i = threadIdx.x & (W - 1);
  const bool live = unit < s.units;
  const GT *p = probs + (live ? unit : 0) * s.lp;
  float *g = grad + (live ? unit : 0) * s.lp;
  float dot = 0.0f;
  for (int j = i; j < s.lp; j += W) dot += to_float(p[j]) * g[j];
  dot = group_sum_n(dot, W);
  if (!live) return;
  for (int j = i; j < s.lp; j += W) g[j] = to_float(p[j]) * (g[j] - dot);
}

// Four consecutive elements as one 16-byte (fp32) or 8-byte (16-bit) access.
__device__ __forceinline__ void load4f(const float *p, float (&v)[4]) {
  const float4 q = *reinterpret_cast<const float4 *>(p);
  v[0] = q.x; v[1] = q.y; v[2] = q.z; v[3] = q.w;
}
template <typename T>
__device__ __forceinline__ void load4f(const T *p, float (&v)[4]) {
  const uint2 q = *reinterpret_cast<const uint2 *>(p);
  const T *h = reinterpret_cast<const T *>(&q);
#pragma unroll
  for (int k = 0; k < 4; ++k) v[k] = to_float(h[k]);
}
__device__ __forceinline__ void store4f(float *p, const float (&v)[4]) {
  *reinterpret_cast<float4 *>(p) = make_float4(v[0], v[1], v[2], v[3]);
}
template <typename T>
__device__ __forceinline__ void store4f(T *p, const float (&v)[4]) {
  uint2 q;
  T *h = reinterpret_cast<T *>(&q);
#pragma unroll
  for (int k = 0; k < 4; ++k) h[k] = from_float<T>(v[k]);
  *reinterpret_cast<uint2 *>(p) = q;
}

// The same two kernels when L*P is a multiple of 4 and at most 64: lane i of
// a unit's W = pow2 >= L*P/4 lanes holds samples [4i, 4i + 4) in registers
// (one access each way); lanes past L*P/4 idle.
template <typename GT>
__global__ void __launch_bounds__(kBlock)
    msda_softmax_units4(const GT *__restrict__ logits, GT *__restrict__ probs, Shape s,
                        int w_log2) {
  const int64_t unit =
      (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) >> w_log2;
  const int i = threadIdx.x & ((1 << w_log2) - 1);
  const bool live = unit < s.units, has = live && 4 * i < s.lp;
  const size_t at = has ? static_cast<size_t>(unit) * s.lp + 4 * i : 0;
  float v[4];
  load4f(logits + at, v);
  float mx = has ? fmaxf(fmaxf(v[0], v[1]), fmaxf(v[2], v[3])) : -INFINITY;
  mx = group_max_n(mx, 1 << w_log2);
  const bool none = mx == -INFINITY;
  float sum = 0.0f;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    v[k] = none ? 0.0f : expf(v[k] - mx);
    sum += v[k];
  }
  sum = group_sum_n(has ? sum : 0.0f, 1 << w_log2);
  if (!has) return;
  const float inv = 1.0f / sum;
#pragma unroll
  for (int k = 0; k < 4; ++k) v[k] *= inv;  // an all -inf unit: 0 * inf = NaN
  store4f(probs + at, v);
}

template <typename GT>
__global__ void __launch_bounds__(kBlock)
    msda_softmax_backward_units4(const GT *__restrict__ probs, float *__restrict__ grad, Shape s,
                                 int w_log2) {
  const int64_t unit =
      (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) >> w_log2;
  const int i = threadIdx.x & ((1 << w_log2) - 1);
  const bool live = unit < s.units, has = live && 4 * i < s.lp;
  const size_t at = has ? static_cast<size_t>(unit) * s.lp + 4 * i : 0;
  float p[4], g[4];
  load4f(probs + at, p);
  load4f(grad + at, g);
  float dot = has ? p[0] * g[0] + p[1] * g[1] + p[2] * g[2] + p[3] * g[3] : 0.0f;
  dot = group_sum_n(dot, 1 << w_log2);
  if (!has) return;
#pragma unroll
  for (int k = 0; k < 4; ++k) g[k] = p[k] * (g[k] - dot);
  store4f(grad + at, g);
}

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
