// C-ABI entry points of libmuspace_msda.so (declared in include/muspace_msda.h).
//
// Host-side validation and kernel selection. Mirrors the checks of the
// reference's TVM-FFI launchers ms_deform_attn_forward / ms_deform_attn_backward
// (/root/reference/csrc/ms_deformable_attn/ms_deform_attn_musa.mu:507-628):
// dtype and pointer checks, dims, im2col_step > 0 and batch % step == 0.
// Errors are returned as codes with a thread-local message instead of C++
// exceptions, and the whole batch is one launch (the reference's per-chunk
// loop has no numeric effect).
#include <hip/hip_runtime.h>

#include <climits>
#include <cstdint>
#include <initializer_list>
#include <mutex>
#include <type_traits>
#include <cstdarg>
#include <cstdio>

#include "../../include/muspace_msda.h"
#include "capi_errors.hpp"
#include "msda_backward_tiles.hpp"
#include "msda_forward_bin.hpp"
#include "msda_kernels.hpp"

namespace {

using capi::check_launch;
using capi::fail;
using capi::ok;

struct Args {
  int64_t batch, spatial, heads, channels, levels, queries, points, step;
};

const char *dtype_name(int d) {
  switch (d) {
    case MUSPACE_DTYPE_F32: return "float32";
    case MUSPACE_DTYPE_F16: return "float16";
    case MUSPACE_DTYPE_BF16: return "bfloat16";
    default: return "unknown";
  }
}

// Shared validation of both directions; fills `s` on success.
int validate(const char *fn, const Args &a, int value_dtype, int geometry_dtype,
             msda::Shape &s) {
  if (value_dtype != MUSPACE_DTYPE_F32 && value_dtype != MUSPACE_DTYPE_F16 &&
      value_dtype != MUSPACE_DTYPE_BF16) {
    return fail(MUSPACE_EINVAL, "%s: value must be float32, float16 or bfloat16 (dtype code %d)",
                fn, value_dtype);
  }
  if (geometry_dtype != MUSPACE_DTYPE_F32 && geometry_dtype != value_dtype) {
    return fail(MUSPACE_EINVAL,
                "%s: sampling_locations/attention_weights must be float32 or %s, got %s", fn,
                dtype_name(value_dtype), dtype_name(geometry_dtype));
  }
  if (a.batch < 0 || a.spatial < 0 || a.heads <= 0 || a.channels <= 0 || a.levels < 0 ||
      a.queries < 0 || a.points < 0) {
    return fail(MUSPACE_EINVAL,
                "%s: invalid dims batch=%lld spatial_size=%lld heads=%lld channels=%lld "
                "levels=%lld queries=%lld points=%lld",
                fn, (long long)a.batch, (long long)a.spatial, (long long)a.heads,
                (long long)a.channels, (long long)a.levels, (long long)a.queries,
                (long long)a.points);
  }
  const int64_t step = a.batch < a.step ? a.batch : a.step;
  if (a.batch > 0 && step <= 0) {
    return fail(MUSPACE_EINVAL, "%s: im2col_step must be positive, got %lld", fn,
                (long long)a.step);
  }
  if (a.batch > 0 && a.batch % step != 0) {
    return fail(MUSPACE_EINVAL, "%s: batch %lld is not divisible by im2col_step %lld", fn,
                (long long)a.batch, (long long)step);
  }
  if (a.levels > msda::kMaxLevels) {
    return fail(MUSPACE_EINVAL, "%s: at most %d levels are supported, got %lld", fn,
                msda::kMaxLevels, (long long)a.levels);
  }
  const int64_t lp = a.levels * a.points;
  const int64_t mc = a.heads * a.channels;
  if (lp > (1 << 20) || mc > INT_MAX || a.spatial * mc > INT_MAX ||
      a.queries * a.heads * lp * 2 > INT_MAX || a.batch * a.queries * a.heads > INT_MAX ||
      a.queries * mc > INT_MAX) {
    return fail(MUSPACE_ERANGE,
                "%s: shape exceeds 32-bit per-batch indexing (spatial_size*heads*channels, "
                "queries*heads*levels*points*2 and batch*queries*heads must each fit in int32)",
                fn);
  }
  s.batch = static_cast<int>(a.batch);
  s.spatial = static_cast<int>(a.spatial);
  s.heads = static_cast<int>(a.heads);
  s.channels = static_cast<int>(a.channels);
  s.levels = static_cast<int>(a.levels);
  s.queries = static_cast<int>(a.queries);
  s.points = static_cast<int>(a.points);
  s.lp = static_cast<int>(lp);
  s.units = static_cast<int>(a.batch * a.queries * a.heads);
  s.inv_points = a.points > 0 ? 1.0f / static_cast<float>(a.points) : 0.0f;
  return ok();
}

int pow2_ceil(int v) {
  int p = 1;
  while (p < v) p <<= 1;
  return p;
}

int log2_int(int v) {
  int l = 0;
  while ((1 << l) < v) ++l;
  return l;
}

// Row-kernel launch plan: groups per unit, samples per group per pass, grid.
struct Launch {
  msda::RowPlan plan;
  int ns;
  int blocks;
};

Launch plan_rows(const msda::Shape &s, int kq, int max_ns, bool forward) {
  const int ng = msda::kWave / kq;
  int gu = pow2_ceil(s.lp > 0 ? s.lp : 1);
  if (gu > ng) gu = ng;
  const int need = (s.lp + gu - 1) / gu;
  Launch L;
  L.ns = need <= 1 ? 1 : (need <= 2 ? 2 : 4);
  if (forward) {
    // forward: as many samples per lane group and step as the lane group has
    // lanes for taps, up to 8 (4 * NS corner gathers in flight per group and
    // fewer groups to reduce over per unit). Measured against the smallest NS
    // that covers a unit with at most 64/KQ groups: NS 8 for L*P >= 16 and
    // 4 for L*P >= 4 took the forward at c1 from 178 to 140 us, c3 from 133
    // to 105 us and c4 bf16 (KQ = 4) from 1058 to 882 us; at c2 (L*P = 32)
    // 8 was already chosen.
    const int ns = (kq >= 8 && max_ns >= 8 && s.lp >= 16) ? 8 : (kq >= 4 && s.lp >= 4) ? 4 : 0;
    if (ns > L.ns) {
      L.ns = ns;
      gu = pow2_ceil((s.lp + ns - 1) / ns);
      if (gu > ng) gu = ng;
    }
  }
  if (L.ns > kq) L.ns = kq;  // the forward computes one tap per lane: ng * ns <= 64
  if (L.ns > max_ns) L.ns = max_ns;
  L.plan.gu_log2 = log2_int(gu);
  L.plan.iters = 8;  // units per lane group: the next unit's geometry loads overlap the gathers
  const int64_t units_per_wave_iter = ng / gu;
  const int64_t wave_iters = (s.units + units_per_wave_iter - 1) / units_per_wave_iter;
  const int64_t waves = (wave_iters + L.plan.iters - 1) / L.plan.iters;
  const int64_t per_block = msda::kBlock / msda::kWave;
  L.blocks = static_cast<int>((waves + per_block - 1) / per_block);
  return L;
}

int generic_blocks(int64_t work) {
  int64_t b = (work + msda::kBlock - 1) / msda::kBlock;
  if (b > 65536) b = 65536;
  if (b < 1) b = 1;
  return static_cast<int>(b);
}

bool needs_data(const msda::Shape &s) { return s.units > 0; }

size_t value_bytes(const msda::Shape &s, size_t elem) {
  return static_cast<size_t>(s.batch) * s.spatial * s.heads * s.channels * elem;
}

bool aligned(const void *p, uintptr_t bytes) {
  return (reinterpret_cast<uintptr_t>(p) & (bytes - 1)) == 0;
}

// The row kernels move 16 bytes per lane (value, output, grad_output,
// grad_value) and 8 bytes per location gradient; views with an odd storage
// offset take the element-wise generic kernels instead.
bool rows_aligned(std::initializer_list<const void *> ptrs16, const void *ptr8 = nullptr) {
  for (const void *p : ptrs16) {
    if (!aligned(p, 16)) return false;
  }
  return ptr8 == nullptr || aligned(ptr8, 8);
}


// ---------------------------------------------------------------- forward ---

// Runs go(NS, launch) with NS the samples per lane group that plan_rows chose
// for the forward row kernels (1, 2, 4 or 8, at most KQ).
template <typename VT, int C, typename Go>
void forward_rows_ns(const msda::Shape &s, Go &&go) {
  constexpr int KQ = C / msda::RowTraits<VT>::kCpl;
  // 16-bit C = 64 rows at NS = 8 need more than 256 VGPRs (one wavefront per
  // SIMD and AGPR spills): four samples per step there
  const Launch L = plan_rows(s, KQ, sizeof(VT) == 2 && C >= 64 ? 4 : 8, true);
  switch (L.ns) {
    case 1:
      go(std::integral_constant<int, 1>(), L);
      break;
    case 2:
      if constexpr (KQ >= 2) go(std::integral_constant<int, 2>(), L);
      break;
    case 8:
      if constexpr (KQ >= 8) go(std::integral_constant<int, 8>(), L);
      break;
    default:
      if constexpr (KQ >= 4) go(std::integral_constant<int, 4>(), L);
      break;
  }
}

template <typename VT, typename GT, int C>
void launch_forward_rows(const void *value, const int64_t *shapes, const int64_t *starts,
                         const void *loc, const void *attn, void *out, const msda::Shape &s,
                         hipStream_t st) {
  const VT *v = static_cast<const VT *>(value);
  const GT *lc = static_cast<const GT *>(loc);
  const GT *aw = static_cast<const GT *>(attn);
  VT *o = static_cast<VT *>(out);
  const uint32_t vbytes = static_cast<uint32_t>(value_bytes(s, sizeof(VT)));
  forward_rows_ns<VT, C>(s, [&](auto ns, const Launch &L) {
    msda::msda_forward_rows<VT, GT, C, decltype(ns)::value>
        <<<L.blocks, msda::kBlock, 0, st>>>(v, vbytes, shapes, starts, lc, aw, o, s, L.plan);
  });
}

template <typename VT, typename GT>
void launch_forward(const void *value, const int64_t *shapes, const int64_t *starts,
                    const void *loc, const void *attn, void *out, const msda::Shape &s,
                    hipStream_t st) {
  // the row kernel addresses value with 32-bit byte offsets below kOobOffset
  const bool small = value_bytes(s, sizeof(VT)) + 64 <= msda::kOobOffset;
  const int rows = rows_aligned({value, out}) && small ? s.channels : 0;
  switch (rows) {
    case 16:
      launch_forward_rows<VT, GT, 16>(value, shapes, starts, loc, attn, out, s, st);
      return;
    case 32:
      launch_forward_rows<VT, GT, 32>(value, shapes, starts, loc, attn, out, s, st);
      return;
    case 64:
      launch_forward_rows<VT, GT, 64>(value, shapes, starts, loc, attn, out, s, st);
      return;
    default:
      msda::msda_forward_generic<VT, GT>
          <<<generic_blocks(static_cast<int64_t>(s.units) * s.channels), msda::kBlock, 0, st>>>(
              static_cast<const VT *>(value), shapes, starts, static_cast<const GT *>(loc),
              static_cast<const GT *>(attn), static_cast<VT *>(out), s);
      return;
  }
}

// ------------------------------------------------- softmax over L*P (fused) ---

// The standalone softmax kernels: four samples per lane in registers when
// L*P is a multiple of 4 up to 64 (rows of 16 or 8 bytes per lane), else a
// strided loop. Lanes per unit: pow2 >= L*P / 4, at most 16.
bool softmax_by_four(const msda::Shape &s) { return s.lp % 4 == 0 && s.lp <= 64; }

int softmax_lanes_log2(const msda::Shape &s) {
  int w = pow2_ceil(s.lp > 0 ? (s.lp + 3) / 4 : 1);
  if (w > 16) w = 16;
  return log2_int(w);
}

int softmax_blocks(const msda::Shape &s) {
  const int64_t lanes = static_cast<int64_t>(s.units) << softmax_lanes_log2(s);
  return static_cast<int>((lanes + msda::kBlock - 1) / msda::kBlock);
}

template <typename GT>
void launch_softmax(const void *logits, void *probs, const msda::Shape &s, hipStream_t st) {
  const GT *x = static_cast<const GT *>(logits);
  GT *p = static_cast<GT *>(probs);
  if (softmax_by_four(s) && aligned(logits, 4 * sizeof(GT))) {
    msda::msda_softmax_units4<GT><<<softmax_blocks(s), msda::kBlock, 0, st>>>(
        x, p, s, softmax_lanes_log2(s));
  } else {
    msda::msda_softmax_units<GT><<<softmax_blocks(s), msda::kBlock, 0, st>>>(
        x, p, s, softmax_lanes_log2(s));
  }
}

template <typename GT>
void launch_softmax_backward(const void *probs, float *grad, const msda::Shape &s,
                             hipStream_t st) {
  const GT *p = static_cast<const GT *>(probs);
  if (softmax_by_four(s) && aligned(grad, 16)) {
    msda::msda_softmax_backward_units4<GT><<<softmax_blocks(s), msda::kBlock, 0, st>>>(
        p, grad, s, softmax_lanes_log2(s));
  } else {
    msda::msda_softmax_backward_units<GT><<<softmax_blocks(s), msda::kBlock, 0, st>>>(
        p, grad, s, softmax_lanes_log2(s));
  }
}

size_t probs_bytes(const msda::Shape &s, int geometry_dtype) {
  const size_t gb = geometry_dtype == MUSPACE_DTYPE_F32 ? 4 : 2;
  return (static_cast<size_t>(s.units) * s.lp * gb + 255) & ~static_cast<size_t>(255);
}

template <typename VT, typename GT, int C>
void launch_forward_softmax_rows(const void *value, const int64_t *shapes, const int64_t *starts,
                                 const void *loc, const void *logits, void *out,
                                 const msda::Shape &s, hipStream_t st) {
  const uint32_t vbytes = static_cast<uint32_t>(value_bytes(s, sizeof(VT)));
  forward_rows_ns<VT, C>(s, [&](auto ns, const Launch &L) {
    msda::msda_forward_softmax_rows<VT, GT, C, decltype(ns)::value>
        <<<L.blocks, msda::kBlock, 0, st>>>(static_cast<const VT *>(value), vbytes, shapes,
                                            starts, static_cast<const GT *>(loc),
                                            static_cast<const GT *>(logits),
                                            static_cast<VT *>(out), s, L.plan);
  });
}

// Forward with logits: the row kernels fuse the softmax; other shapes take the
// standalone softmax into stream-ordered scratch, then the generic kernel.
// Returns false when that scratch cannot be allocated.
template <typename VT, typename GT>
bool launch_forward_softmax(const void *value, const int64_t *shapes, const int64_t *starts,
                            const void *loc, const void *logits, void *out,
                            const msda::Shape &s, int geometry_dtype, hipStream_t st) {
  const bool small = value_bytes(s, sizeof(VT)) + 64 <= msda::kOobOffset;
  const int rows = rows_aligned({value, out}) && small ? s.channels : 0;
  switch (rows) {
    case 16:
      launch_forward_softmax_rows<VT, GT, 16>(value, shapes, starts, loc, logits, out, s, st);
      return true;
    case 32:
      launch_forward_softmax_rows<VT, GT, 32>(value, shapes, starts, loc, logits, out, s, st);
      return true;
    case 64:
      launch_forward_softmax_rows<VT, GT, 64>(value, shapes, starts, loc, logits, out, s, st);
      return true;
    default: {
      void *probs = nullptr;
      if (hipMallocAsync(&probs, probs_bytes(s, geometry_dtype), st) != hipSuccess) {
        (void)hipGetLastError();
        return false;
      }
      launch_softmax<GT>(logits, probs, s, st);
      launch_forward<VT, GT>(value, shapes, starts, loc, probs, out, s, st);
      (void)hipFreeAsync(probs, st);
      return true;
    }
  }
}

// ------------------------------------------ spatial cross-attention epilogue ---

// Camera-rebatched dims of the scatter-average entry points.
struct CamDims {
  int64_t batch, cams, max_len, num_query;
};

// Checks the camera dims and the dense geometry they imply; `full` describes
// the whole rebatched value and geometry ([batch*cams, ...]).
int validate_cameras(const char *fn, const Args &a, const CamDims &c, int value_dtype,
                     int geometry_dtype, msda::Shape &full) {
  if (c.batch < 0 || c.cams <= 0 || c.max_len < 0 || c.num_query < 0) {
    return fail(MUSPACE_EINVAL,
                "%s: invalid dims batch=%lld num_cams=%lld max_len=%lld num_query=%lld", fn,
                (long long)c.batch, (long long)c.cams, (long long)c.max_len,
                (long long)c.num_query);
  }
  if (c.batch * c.cams > INT_MAX || c.num_query > INT_MAX) {
    return fail(MUSPACE_ERANGE, "%s: batch*num_cams or num_query exceeds int32", fn);
  }
  return validate(fn, a, value_dtype, geometry_dtype, full);
}

// Checks 0 <= valid_lens[i] <= max_len (host array) and sums them.
int check_lengths(const char *fn, const int64_t *valid_lens, int64_t cams, int64_t max_len,
                  int64_t &total) {
  if (!valid_lens) return fail(MUSPACE_EINVAL, "%s: null valid_lens", fn);
  total = 0;
  for (int64_t i = 0; i < cams; ++i) {
    if (valid_lens[i] < 0 || valid_lens[i] > max_len) {
      return fail(MUSPACE_EINVAL, "%s: valid_lens[%lld] = %lld is outside [0, max_len=%lld]", fn,
                  (long long)i, (long long)valid_lens[i], (long long)max_len);
    }
    total += valid_lens[i];
  }
  return ok();
}

// One launch of cameras out.cam0 .. out.cam0 + out.ncam - 1 (out.off[out.ncam]
// valid rows); `full` is the whole rebatched value.
template <typename VT, typename GT, bool kAtomic>
void launch_scatter_div(const void *value, const int64_t *shapes, const int64_t *starts,
                        const void *loc, const void *attn,
                        const msda::CameraSlots<VT, GT, kAtomic> &out, const msda::Shape &full,
                        int batch, void *slots, hipStream_t st) {
  msda::Shape s = full;
  s.batch = batch;
  s.queries = out.off[out.ncam];
  s.units = batch * s.queries * s.heads;
  if (s.units == 0) return;
  const VT *v = static_cast<const VT *>(value);
  const GT *lc = static_cast<const GT *>(loc);
  const GT *aw = static_cast<const GT *>(attn);
  // the row kernel addresses all cameras' value with 32-bit byte offsets
  const size_t vb = value_bytes(full, sizeof(VT));
  const bool small = vb + 64 <= msda::kOobOffset;
  const int rows = rows_aligned({value, slots}) && small ? s.channels : 0;
  const uint32_t vbytes = static_cast<uint32_t>(vb);
  auto go = [&](auto cc) {
    constexpr int C = decltype(cc)::value;
    constexpr int KQ = C / msda::RowTraits<VT>::kCpl;
    forward_rows_ns<VT, C>(s, [&](auto ns, const Launch &L) {
      // one segment of whole blocks per camera (the plan depends on L*P only)
      msda::CameraSlots<VT, GT, kAtomic> seg = out;
      const int64_t per_wave = static_cast<int64_t>((msda::kWave / KQ) >> L.plan.gu_log2) *
                               L.plan.iters;
      const int64_t per_block = per_wave * (msda::kBlock / msda::kWave);
      int64_t blocks = 0;
      for (int j = 0; j < seg.ncam; ++j) {
        seg.blk[j] = static_cast<int>(blocks);
        const int64_t units = static_cast<int64_t>(s.batch) * s.heads *
                              (seg.off[j + 1] - seg.off[j]);
        blocks += (units + per_block - 1) / per_block;
      }
      seg.blk[seg.ncam] = static_cast<int>(blocks);
      msda::msda_forward_scatter_div_rows<VT, GT, C, decltype(ns)::value, kAtomic>
          <<<static_cast<int>(blocks), msda::kBlock, 0, st>>>(v, vbytes, shapes, starts, lc, aw,
                                                              seg, s, L.plan);
    });
  };
  switch (rows) {
    case 16: go(std::integral_constant<int, 16>()); return;
    case 32: go(std::integral_constant<int, 32>()); return;
    case 64: go(std::integral_constant<int, 64>()); return;
    default:
      msda::msda_forward_scatter_div_generic<VT, GT, kAtomic>
          <<<generic_blocks(static_cast<int64_t>(s.units) * s.channels), msda::kBlock, 0, st>>>(
              v, shapes, starts, lc, aw, out, s);
      return;
  }
}

// Cameras [cam0, cam0 + ncam) of `valid_lens`, numbered back to back from
// index + first; returns the camera table of one launch.
template <typename Table>
void fill_camera_table(Table &tb, const int64_t *valid_lens, int cam0, int ncam) {
  int q = 0;
  for (int j = 0; j < ncam; ++j) {
    tb.off[j] = q;
    q += static_cast<int>(valid_lens[cam0 + j]);
  }
  tb.off[ncam] = q;
}

template <typename VT, typename GT>
void launch_scatter_div_grad(const void *grad_slots, const int64_t *index,
                             const int64_t *valid_lens, const void *count, void *grad_out,
                             const CamDims &c, int row, hipStream_t st) {
  constexpr int W = 16 / static_cast<int>(sizeof(VT));
  const VT *g = static_cast<const VT *>(grad_slots);
  const GT *cnt = static_cast<const GT *>(count);
  VT *o = static_cast<VT *>(grad_out);
  const bool vec = row % W == 0 && aligned(grad_slots, 16) && aligned(grad_out, 16);
  const int64_t work = c.batch * c.max_len * (vec ? row / W : row);
  const int B = static_cast<int>(c.batch), NC = static_cast<int>(c.cams),
            ML = static_cast<int>(c.max_len), NQ = static_cast<int>(c.num_query);
  int64_t first = 0;
  for (int cam0 = 0; cam0 < NC; cam0 += msda::kMaxCams) {
    const int ncam = NC - cam0 < msda::kMaxCams ? NC - cam0 : msda::kMaxCams;
    msda::CameraRows tb{};
    int q = 0;
    for (int j = 0; j < ncam; ++j) {
      tb.off[j] = q;
      tb.len[j] = static_cast<int>(valid_lens[cam0 + j]);
      q += tb.len[j];
    }
    const dim3 grid(generic_blocks(work), ncam);
    if (vec) {
      msda::msda_scatter_div_grad<VT, GT, W><<<grid, msda::kBlock, 0, st>>>(
          g, index + first, cnt, o, B, NC, cam0, tb, ML, NQ, row);
    } else {
      msda::msda_scatter_div_grad<VT, GT, 1><<<grid, msda::kBlock, 0, st>>>(
          g, index + first, cnt, o, B, NC, cam0, tb, ML, NQ, row);
    }
    first += q;
  }
}

// Calls f(VT(), GT()) for the value dtype and the geometry (loc, attn, count)
// dtype: float32 or the value dtype.
template <typename F>
void with_dtypes(int value_dtype, int geometry_dtype, F &&f) {
  using msda::bf16_t;
  switch (value_dtype) {
    case MUSPACE_DTYPE_F32:
      f(float(), float());
      return;
    case MUSPACE_DTYPE_F16:
      if (geometry_dtype == MUSPACE_DTYPE_F32) {
        f(__half(), float());
      } else {
        f(__half(), __half());
      }
      return;
    default:
      if (geometry_dtype == MUSPACE_DTYPE_F32) {
        f(bf16_t(), float());
      } else {
        f(bf16_t(), bf16_t());
      }
      return;
  }
}

// --------------------------------------------------------------- backward ---

// Atomic fallback (shapes the tile path does not take): grad_value is zeroed
// here, then accumulated with fp32 global atomics.
template <typename VT, typename GT, int C>
void launch_backward_rows(const void *value, const int64_t *shapes, const int64_t *starts,
                          const void *loc, const void *attn, const void *grad_out, float *gv,
                          float *gl, float *ga, const msda::Shape &s, hipStream_t st) {
  constexpr int KQ = C / msda::RowTraits<VT>::kCpl;
  const Launch L = plan_rows(s, KQ, 4, false);
  const VT *v = static_cast<const VT *>(value);
  const GT *lc = static_cast<const GT *>(loc);
  const GT *aw = static_cast<const GT *>(attn);
  const VT *go = static_cast<const VT *>(grad_out);
  switch (L.ns) {
    case 1:
      msda::msda_backward_rows<VT, GT, C, 1><<<L.blocks, msda::kBlock, 0, st>>>(
          v, shapes, starts, lc, aw, go, gv, gl, ga, s, L.plan);
      break;
    case 2:
      msda::msda_backward_rows<VT, GT, C, 2><<<L.blocks, msda::kBlock, 0, st>>>(
          v, shapes, starts, lc, aw, go, gv, gl, ga, s, L.plan);
      break;
    default:
      msda::msda_backward_rows<VT, GT, C, 4><<<L.blocks, msda::kBlock, 0, st>>>(
          v, shapes, starts, lc, aw, go, gv, gl, ga, s, L.plan);
      break;
  }
}

template <typename VT, typename GT>
void launch_backward_atomic(const void *value, const int64_t *shapes, const int64_t *starts,
                            const void *loc, const void *attn, const void *grad_out, float *gv,
                            float *gl, float *ga, const msda::Shape &s, hipStream_t st) {
  const int64_t n = static_cast<int64_t>(s.batch) * s.spatial * s.heads * s.channels;
  if (n > 0) msda::zero_kernel<<<generic_blocks(n), msda::kBlock, 0, st>>>(gv, n);
  const int rows = rows_aligned({value, grad_out, gv}, gl) ? s.channels : 0;
  switch (rows) {
    case 16:
      launch_backward_rows<VT, GT, 16>(value, shapes, starts, loc, attn, grad_out, gv, gl, ga,
                                       s, st);
      return;
    case 32:
      launch_backward_rows<VT, GT, 32>(value, shapes, starts, loc, attn, grad_out, gv, gl, ga,
                                       s, st);
      return;
    case 64:
      launch_backward_rows<VT, GT, 64>(value, shapes, starts, loc, attn, grad_out, gv, gl, ga,
                                       s, st);
      return;
    default:
      msda::msda_backward_generic<VT, GT>
          <<<generic_blocks(static_cast<int64_t>(s.units) * s.lp), msda::kBlock, 0, st>>>(
              static_cast<const VT *>(value), shapes, starts, static_cast<const GT *>(loc),
              static_cast<const GT *>(attn), static_cast<const VT *>(grad_out), gv, gl, ga, s);
      return;
  }
}

size_t align256(size_t v) { return (v + 255) & ~static_cast<size_t>(255); }

// Tile edge and batch size of the tile-owned backward per value dtype and
// channel count (0 when the tile path does not cover the channel count).
template <typename VT>
int tile_edge_for(int channels) {
  switch (channels) {
    case 16: return msda::TileCfg<VT, 16>::T;
    case 32: return msda::TileCfg<VT, 32>::T;
    case 64: return msda::TileCfg<VT, 64>::T;
    default: return 0;
  }
}

template <typename VT>
int tile_batch_for(int channels) {
  switch (channels) {
    case 16: return msda::TileCfg<VT, 16>::K;
    case 32: return msda::TileCfg<VT, 32>::K;
    default: return msda::TileCfg<VT, 64>::K;
  }
}

int tile_batch(int value_dtype, int channels) {
  return value_dtype == MUSPACE_DTYPE_F32 ? tile_batch_for<float>(channels)
                                          : tile_batch_for<msda::bf16_t>(channels);
}

int tile_edge(int value_dtype, int channels) {
  return value_dtype == MUSPACE_DTYPE_F32 ? tile_edge_for<float>(channels)
                                          : tile_edge_for<msda::bf16_t>(channels);  // fp16: same
}

// Persistent grid of the tile kernel: one workgroup per CU, a multiple of 8
// (the XCD count) so that every XCD gets the same number of workgroups.
int tile_grid() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        cus <= 0) {
      cus = 256;
    }
    cached[dev] = ((cus + 7) / 8) * 8;
  }
  return cached[dev];
}

// The forward row kernel's units (queries of one slab) and tap slots per
// block: the query chunk of the binning fused into the forward. False where
// no row kernel serves the channel count.
bool fwd_bin_chunk(const msda::Shape &s, int value_dtype, int &units, int &slots,
                   int *unit_steps = nullptr) {
  if (s.channels != 16 && s.channels != 32 && s.channels != 64) return false;
  const int vb = value_dtype == MUSPACE_DTYPE_F32 ? 4 : 2;
  const int kq = s.channels / (16 / vb);
  const Launch L = plan_rows(s, kq, vb == 2 && s.channels >= 64 ? 4 : 8, true);
  const int ng = msda::kWave / kq, gu = 1 << L.plan.gu_log2;
  const int lchunks = (s.lp + gu * L.ns - 1) / (gu * L.ns);
  const int waves = msda::kBlock / msda::kWave;
  units = waves * L.plan.iters * (ng / gu);
  slots = waves * L.plan.iters * lchunks * ng * L.ns;  // ng * ns <= 64 taps per step
  if (unit_steps) *unit_steps = lchunks;
  return units > 0;
}

// bin_count blocks per slab: groups of count_sub chunks.
int count_groups(const msda::BinPlan &p) { return (p.chunks + p.count_sub - 1) / p.count_sub; }

// bin_count's LDS histograms (count_sub rows of tile_bound counters), with
// 16-bit counters where a chunk has fewer than 65536 samples.
size_t count_hist_bytes(msda::BinPlan &p) {
  p.hist16 = (static_cast<int64_t>(p.chunk_q) << p.lp_log2) < 65536 ? 1 : 0;
  const size_t counters = static_cast<size_t>(p.tile_bound) * p.count_sub;
  return p.hist16 ? (counters + 1) / 2 * 4 : counters * 4;
}

// bin_cursors over the counts bin_count wrote: S = 1 << seg_log2 threads a
// tile, so that a thread takes at most 32 chunks (S <= 16), and about 512
// blocks in all (at most 32 a slab).
template <int T>
void launch_bin_cursors(const int64_t *shapes, const int64_t *starts, const msda::Shape &s,
                        const msda::BinPlan &p, int bm, uint32_t *counts, uint32_t *tile_start,
                        hipStream_t st) {
  int seg_log2 = 0;
  while (seg_log2 < 4 && ((p.chunks + (1 << seg_log2) - 1) >> seg_log2) > 32) ++seg_log2;
  int gy = 512 / (bm > 0 ? bm : 1);
  gy = gy < 1 ? 1 : (gy > 32 ? 32 : gy);
  msda::msda_bin_cursors<T><<<dim3(bm, gy), msda::kCurBlock, 0, st>>>(shapes, starts, s, p,
                                                                      seg_log2, counts,
                                                                      tile_start);
}

// Scratch layout of the tile-owned backward.
struct TileWorkspace {
  msda::BinPlan plan;
  size_t counts, tile_start, zero_tiles, records, rec_of_sample, items, item_total, bytes;
};

bool plan_tile_workspace(const msda::Shape &s, int value_dtype, TileWorkspace &w) {
  const int T = tile_edge(value_dtype, s.channels);
  if (T == 0) return false;
  msda::BinPlan &p = w.plan;
  // binning chunks of about 4096 sample slots (at least kBinBlock queries): a
  // binning block's cost has a part per tile of the slab (histogram, scans),
  // so few samples per query (c3: L*P = 4) want more queries per block
  // (c3 binning 135 -> 89 us; c2, 32 samples per query, keeps 256 queries)
  const int per_q = 4096 >> log2_int(s.lp > 0 ? s.lp : 1);
  p.chunk_q = per_q > msda::kBinBlock ? per_q : msda::kBinBlock;
  p.chunks = (s.queries + p.chunk_q - 1) / p.chunk_q;
  p.count_sub = 1;
  p.hist16 = 0;  // set per launch (count_hist_bytes)
  // a level of n cells has ceil(h/T)*ceil(w/T) <= n/T + 1 tiles
  const int64_t bound = static_cast<int64_t>(s.spatial) / T + s.levels + 1;
  if (bound > msda::kMaxTilesPerSlab) return false;
  p.tile_bound = static_cast<int>(bound);
  // bin_scatter stages a sub-chunk of records and two tile arrays in LDS
  if (msda::scatter_lds_bytes(p.tile_bound) + 4096 > msda::kTileLdsLimit) return false;
  p.lp_log2 = log2_int(s.lp > 0 ? s.lp : 1);
  if ((1 << p.lp_log2) > msda::kScatterSlots) return false;
  // record ids pack (q << lp_log2) | sample below bit kPosShift and the tap's
  // position in the tile frame above it
  if ((static_cast<int64_t>(s.queries) << p.lp_log2) > (int64_t{1} << msda::kPosShift)) return false;
  if ((T + 1) * (T + 1) > (1 << (32 - msda::kPosShift))) return false;
  // the tile kernel addresses grad_out rows with a 24-bit multiply (q < 2^24)
  // and a 32-bit element offset inside one batch entry
  if (s.queries >= (1 << 24)) return false;
  // the tile kernel stages value tiles with 32-bit buffer offsets below kOobOffset
  const size_t vb = value_dtype == MUSPACE_DTYPE_F32 ? 4 : 2;
  if (value_bytes(s, vb) + 64 > msda::kOobOffset) return false;
  // ... and reads grad_out rows with 32-bit buffer offsets below kOobOffset
  if (static_cast<size_t>(s.batch) * s.queries * s.heads * s.channels * vb + 64 >
      msda::kOobOffset) {
    return false;
  }
  if (static_cast<int64_t>(s.queries) * s.heads * s.channels >= (int64_t{1} << 32)) return false;
  p.rec_cap = static_cast<int64_t>(s.queries) * s.lp;
  // Direct gradient writes scatter 12 bytes per sample over the slab's span of
  // queries * lp samples; the records path instead stores them over the
  // records and msda_grad_gather un-sorts them, one random 16-byte read per
  // sample. Measured with the current kernels (full steps, direct writes also
  // taking the fused forward): c2 (3.8 MB) and c3 (1.9 MB) 5% and 11% faster
  // direct, c1 (4.3 MB) 1.4% and c4 (5.8 MB) 1.2% faster direct. Spans past
  // 8 MB keep the records path (not measured there).
  p.direct = p.rec_cap * 12 <= (8 << 20) ? 1 : 0;
  if (p.rec_cap >= (int64_t{1} << 31)) return false;
  const int64_t bm = static_cast<int64_t>(s.batch) * s.heads;
  // records per work item (a tile with more is split into items whose cells
  // are all added atomically): about 4 items' worth per workgroup, 4 to 8
  // batches, in whole batches. Measured at the benchmark shapes: single-
  // batch items (splitting nearly every tile) cost c1 55 us; items of more
  // than 8 batches leave the largest ones running alone at the end (c4).
  const int K = tile_batch(value_dtype, s.channels);
  const int64_t total = bm * p.rec_cap;
  if (total >= (int64_t{1} << 32)) return false;  // sample indices are 32-bit in the tile kernel
  int64_t mult = (total + int64_t{4} * tile_grid() * K - 1) / (int64_t{4} * tile_grid() * K);
  mult = mult < 4 ? 4 : (mult > 8 ? 8 : mult);
  p.rmax = static_cast<int>(mult * K);
  const int64_t item_cap = bm * (p.tile_bound + (p.rec_cap + p.rmax - 1) / p.rmax + 1);
  if (item_cap >= (int64_t{1} << 31)) return false;
  p.item_cap = static_cast<int>(item_cap);
  size_t off = 0;
  auto take = [&off](size_t bytes) {
    const size_t at = off;
    off = align256(off + bytes);
    return at;
  };
  // the histograms of either chunking: bin_count's own, or the forward
  // blocks' when the binning is fused into the forward
  int fwd_units = 0, fwd_slots = 0;
  const int fwd_chunks = fwd_bin_chunk(s, value_dtype, fwd_units, fwd_slots)
                             ? (s.queries + fwd_units - 1) / fwd_units
                             : 0;
  const int count_chunks = fwd_chunks > p.chunks ? fwd_chunks : p.chunks;
  w.counts = take(static_cast<size_t>(bm) * count_chunks * p.tile_bound * 4);
  w.tile_start = take(static_cast<size_t>(bm) * (p.tile_bound + 1) * 4);
  w.zero_tiles = take(static_cast<size_t>(bm) * (p.tile_bound + 1) * 4);
  w.records = take(static_cast<size_t>(bm) * p.rec_cap * 16);
  w.rec_of_sample = take(p.direct ? 0 : static_cast<size_t>(bm) * p.rec_cap * 4);
  w.items = take(static_cast<size_t>(p.item_cap) * sizeof(msda::Item));
  w.item_total = take(4 * (1 + msda::kXcdQueues));  // item count, per-XCD take counters
  w.bytes = off;
  return true;
}

// Parts of the backward: binning (bin_count, bin_scan, bin_scatter) reads only
// the geometry and may run before grad_output exists, e.g. on a second stream
// during the forward; the rest needs grad_output and the binned workspace.
enum class Phase { kAll, kBin, kRest };

template <typename VT, typename GT, int C>
void launch_backward_tiles(const void *value, const int64_t *shapes, const int64_t *starts,
                           const void *loc, const void *attn, const void *grad_out, float *gv,
                           float *gl, float *ga, const msda::Shape &s, const TileWorkspace &w,
                           void *workspace, Phase phase, hipStream_t st) {
  constexpr int T = msda::TileCfg<VT, C>::T;
  unsigned char *ws = static_cast<unsigned char *>(workspace);
  uint32_t *counts = reinterpret_cast<uint32_t *>(ws + w.counts);
  uint32_t *tile_start = reinterpret_cast<uint32_t *>(ws + w.tile_start);
  uint32_t *zero_tiles = reinterpret_cast<uint32_t *>(ws + w.zero_tiles);
  uint4 *records = reinterpret_cast<uint4 *>(ws + w.records);
  uint32_t *rec_of_sample = reinterpret_cast<uint32_t *>(ws + w.rec_of_sample);
  msda::Item *items = reinterpret_cast<msda::Item *>(ws + w.items);
  uint32_t *item_total = reinterpret_cast<uint32_t *>(ws + w.item_total);
  msda::BinPlan p = w.plan;
  const int bm = s.batch * s.heads;
  const VT *v = static_cast<const VT *>(value);
  const GT *lc = static_cast<const GT *>(loc);
  const GT *aw = static_cast<const GT *>(attn);
  const VT *go = static_cast<const VT *>(grad_out);
  const size_t hist_bytes = count_hist_bytes(p);

  auto count = msda::msda_bin_count<GT, C, T>;
  auto scatter = msda::msda_bin_scatter<GT, C, T>;
  auto tile = msda::msda_tile_backward<VT, C>;
  constexpr size_t tile_bytes = msda::tile_lds_bytes<VT, C>();
  (void)hipFuncSetAttribute(reinterpret_cast<const void *>(count),
                            hipFuncAttributeMaxDynamicSharedMemorySize, hist_bytes);
  const size_t scatter_bytes = msda::scatter_lds_bytes(p.tile_bound);
  (void)hipFuncSetAttribute(reinterpret_cast<const void *>(scatter),
                            hipFuncAttributeMaxDynamicSharedMemorySize, scatter_bytes);
  (void)hipFuncSetAttribute(reinterpret_cast<const void *>(tile),
                            hipFuncAttributeMaxDynamicSharedMemorySize, tile_bytes);

  if (phase != Phase::kRest) {
    count<<<bm * count_groups(p), msda::kBinBlock, hist_bytes, st>>>(shapes, starts, lc, s, p,
                                                                     counts, item_total, gv);
    launch_bin_cursors<T>(shapes, starts, s, p, bm, counts, tile_start, st);
    msda::msda_bin_scan<C, T><<<bm, msda::kBinBlock, 0, st>>>(
        shapes, starts, s, p, tile_start, item_total, items, zero_tiles, gv);
    scatter<<<bm * p.chunks, msda::kBinBlock, scatter_bytes, st>>>(
        shapes, starts, lc, aw, s, p, counts, tile_start, zero_tiles, records, rec_of_sample, gl,
        ga, gv);
  }
  if (phase == Phase::kBin) return;
  const uint32_t vbytes = static_cast<uint32_t>(value_bytes(s, sizeof(VT)));
  const uint32_t gbytes = static_cast<uint32_t>(static_cast<size_t>(s.batch) * s.queries *
                                                s.heads * C * sizeof(VT));
  tile<<<tile_grid(), msda::kTileBlock, tile_bytes, st>>>(v, vbytes, shapes, starts, go, gbytes,
                                                          records, items, item_total, s, p, gv,
                                                          gl, ga);
  if (!p.direct) {
    const int per_slab = static_cast<int>((p.rec_cap + msda::kBinBlock - 1) / msda::kBinBlock);
    msda::msda_grad_gather<<<bm * per_slab, msda::kBinBlock, 0, st>>>(rec_of_sample, records, s,
                                                                      p, per_slab, gl, ga);
  }
}

// Whether ms_deform_attn_forward_bin stores the records from the forward
// kernel for shape s (given a planned tile workspace w): only where the tile
// kernel writes the location and weight gradients straight to sample order
// (the records-plus-gather path would also need the sample -> record index,
// which the fused forward measured slower to store than bin_scatter does),
// within the block's tap slots and its LDS budget. units, slots: the
// forward block's queries and tap slots.
// softmax: the forward takes logits (msda_forward_softmax_bin_rows), which
// needs units of one step each, so that a sample's probability is final when
// its tap is computed.
bool fwd_bin_fuses(const msda::Shape &s, int value_dtype, const TileWorkspace &w, int &units,
                   int &slots, bool softmax = false) {
  if (!w.plan.direct) return false;
  int unit_steps = 0;
  if (!fwd_bin_chunk(s, value_dtype, units, slots, &unit_steps)) return false;
  if (softmax && unit_steps != 1) return false;
  return slots <= msda::kFwdBinSlots &&
         msda::fwd_bin_lds_bytes(slots, w.plan.tile_bound) <= msda::kFwdBinDynLds;
}

// The forward with the backward's binning fused in (msda_forward_bin.hpp):
// bin_count and bin_scan over the forward blocks' query chunks, then the
// forward row kernel, which also stores every chunk's records. With `probs`
// non-null, `attn` holds logits: the kernel is the softmax-fused forward,
// which also writes every sample's probability (GT) to `probs` and records
// it. Launches nothing and returns false where that does not apply.
template <typename VT, typename GT, int C>
bool launch_forward_bin_tiles(const void *value, const int64_t *shapes, const int64_t *starts,
                              const void *loc, const void *attn, void *out, float *gv, float *gl,
                              float *ga, const msda::Shape &s, const TileWorkspace &w,
                              void *workspace, hipStream_t st, void *probs = nullptr) {
  constexpr int T = msda::TileCfg<VT, C>::T;
  constexpr int value_dtype = std::is_same<VT, float>::value ? MUSPACE_DTYPE_F32
                                                             : MUSPACE_DTYPE_F16;
  int units = 0, slots = 0;
  if (!fwd_bin_fuses(s, value_dtype, w, units, slots, probs != nullptr)) return false;
  unsigned char *ws = static_cast<unsigned char *>(workspace);
  uint32_t *counts = reinterpret_cast<uint32_t *>(ws + w.counts);
  uint32_t *tile_start = reinterpret_cast<uint32_t *>(ws + w.tile_start);
  uint32_t *zero_tiles = reinterpret_cast<uint32_t *>(ws + w.zero_tiles);
  uint4 *records = reinterpret_cast<uint4 *>(ws + w.records);
  msda::Item *items = reinterpret_cast<msda::Item *>(ws + w.items);
  uint32_t *item_total = reinterpret_cast<uint32_t *>(ws + w.item_total);
  msda::BinPlan p = w.plan;
  const int bm = s.batch * s.heads;
  p.chunk_q = units;
  p.chunks = (s.queries + units - 1) / units;
  // bin_count blocks count several forward chunks each (a histogram row per
  // chunk) when there would be more than about 4096 blocks, up to 8192
  // sample slots and 64 KB of LDS histograms per block: its cost per block
  // (level tables, histogram clear and flush) dominated at c4 (22560 chunks;
  // count and scan 250 -> 166 us), while at c2 (7536 chunks) four per block
  // left too few blocks (42 -> 60 us)
  const int per_chunk = units << p.lp_log2;
  int sub = bm * p.chunks / 4096;
  const int by_slots = 8192 / per_chunk, by_lds = 16384 / p.tile_bound;
  sub = sub < by_slots ? sub : by_slots;
  sub = sub < by_lds ? sub : by_lds;
  p.count_sub = sub > 1 ? sub : 1;
  const GT *lc = static_cast<const GT *>(loc);
  const GT *aw = static_cast<const GT *>(attn);
  const size_t hist_bytes = count_hist_bytes(p);
  auto count = msda::msda_bin_count<GT, C, T>;
  (void)hipFuncSetAttribute(reinterpret_cast<const void *>(count),
                            hipFuncAttributeMaxDynamicSharedMemorySize, hist_bytes);
  count<<<bm * count_groups(p), msda::kBinBlock, hist_bytes, st>>>(shapes, starts, lc, s, p,
                                                                   counts, item_total, gv);
  launch_bin_cursors<T>(shapes, starts, s, p, bm, counts, tile_start, st);
  msda::msda_bin_scan<C, T><<<bm, msda::kBinBlock, 0, st>>>(
      shapes, starts, s, p, tile_start, item_total, items, zero_tiles, gv);
  const msda::FwdBinArgs args{counts, tile_start, zero_tiles, records, gl, ga,
                              gv,     p,          slots,      probs};
  const size_t lds = msda::fwd_bin_lds_bytes(slots, p.tile_bound);
  const uint32_t vbytes = static_cast<uint32_t>(value_bytes(s, sizeof(VT)));
  forward_rows_ns<VT, C>(s, [&](auto ns, const Launch &L) {
    auto k = probs ? msda::msda_forward_softmax_bin_rows<VT, GT, C, decltype(ns)::value, T>
                   : msda::msda_forward_bin_rows<VT, GT, C, decltype(ns)::value, T>;
    (void)hipFuncSetAttribute(reinterpret_cast<const void *>(k),
                              hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    k<<<bm * p.chunks, msda::kBlock, lds, st>>>(static_cast<const VT *>(value), vbytes, shapes,
                                                 starts, lc, aw, static_cast<VT *>(out), s,
                                                 L.plan, args);
  });
  return true;
}

template <typename VT, typename GT>
bool launch_forward_bin(const void *value, const int64_t *shapes, const int64_t *starts,
                        const void *loc, const void *attn, void *out, float *gv, float *gl,
                        float *ga, const msda::Shape &s, void *workspace, size_t workspace_bytes,
                        hipStream_t st, void *probs = nullptr) {
  constexpr int value_dtype = std::is_same<VT, float>::value ? MUSPACE_DTYPE_F32
                                                             : MUSPACE_DTYPE_F16;
  TileWorkspace w;
  const bool fits = plan_tile_workspace(s, value_dtype, w) && workspace != nullptr &&
                    workspace_bytes >= w.bytes && rows_aligned({value, out, gv}, gl) &&
                    aligned(workspace, 256);
  if (!fits) return false;
  switch (s.channels) {
    case 16:
      return launch_forward_bin_tiles<VT, GT, 16>(value, shapes, starts, loc, attn, out, gv, gl,
                                                  ga, s, w, workspace, st, probs);
    case 32:
      return launch_forward_bin_tiles<VT, GT, 32>(value, shapes, starts, loc, attn, out, gv, gl,
                                                  ga, s, w, workspace, st, probs);
    case 64:
      return launch_forward_bin_tiles<VT, GT, 64>(value, shapes, starts, loc, attn, out, gv, gl,
                                                  ga, s, w, workspace, st, probs);
    default:
      return false;
  }
}

template <typename VT, typename GT>
void launch_backward(const void *value, const int64_t *shapes, const int64_t *starts,
                     const void *loc, const void *attn, const void *grad_out, float *gv,
                     float *gl, float *ga, const msda::Shape &s, void *workspace,
                     size_t workspace_bytes, Phase phase, hipStream_t st) {
  constexpr int value_dtype = std::is_same<VT, float>::value ? MUSPACE_DTYPE_F32
                                                             : MUSPACE_DTYPE_F16;
  TileWorkspace w;
  const bool tiles = plan_tile_workspace(s, value_dtype, w) && workspace != nullptr &&
                     workspace_bytes >= w.bytes && rows_aligned({value, grad_out, gv}, gl) &&
                     aligned(workspace, 256);
  if (!tiles) {  // the atomic fallback has no binning: all of it is the second part
    if (phase != Phase::kBin) {
      launch_backward_atomic<VT, GT>(value, shapes, starts, loc, attn, grad_out, gv, gl, ga, s,
                                     st);
    }
    return;
  }
  switch (s.channels) {
    case 16:
      launch_backward_tiles<VT, GT, 16>(value, shapes, starts, loc, attn, grad_out, gv, gl, ga,
                                        s, w, workspace, phase, st);
      return;
    case 32:
      launch_backward_tiles<VT, GT, 32>(value, shapes, starts, loc, attn, grad_out, gv, gl, ga,
                                        s, w, workspace, phase, st);
      return;
    default:
      launch_backward_tiles<VT, GT, 64>(value, shapes, starts, loc, attn, grad_out, gv, gl, ga,
                                        s, w, workspace, phase, st);
      return;
  }
}

int backward_impl(const char *fn, const void *value, int value_dtype,
                  const int64_t *spatial_shapes, const int64_t *level_start_index,
                  const void *sampling_locations, const void *attention_weights,
                  int geometry_dtype, const void *grad_output, float *grad_value,
                  float *grad_sampling_locations, float *grad_attention_weights, const Args &a,
                  void *workspace, size_t workspace_bytes, hipStream_t st,
                  Phase phase = Phase::kAll, bool softmax = false) {
  msda::Shape s;
  if (int rc = validate(fn, a, value_dtype, geometry_dtype, s)) return rc;
  const int64_t nvalue = a.batch * a.spatial * a.heads * a.channels;
  if (nvalue > 0 && !grad_value) return fail(MUSPACE_EINVAL, "%s: null tensor pointer", fn);
  if (!needs_data(s) || s.lp == 0) {
    // nothing samples the value: its gradient is zero
    if (nvalue > 0 && phase != Phase::kBin) {
      msda::zero_kernel<<<generic_blocks(nvalue), msda::kBlock, 0, st>>>(grad_value, nvalue);
      return check_launch(fn);
    }
    return ok();
  }
  // the binning part does not read grad_output, which may not exist yet
  if (!value || !spatial_shapes || !level_start_index || !sampling_locations ||
      !attention_weights || (!grad_output && phase != Phase::kBin) || !grad_sampling_locations ||
      !grad_attention_weights) {
    return fail(MUSPACE_EINVAL, "%s: null tensor pointer", fn);
  }
  if (!softmax) {
    with_dtypes(value_dtype, geometry_dtype, [&](auto vt, auto gt) {
      launch_backward<decltype(vt), decltype(gt)>(
          value, spatial_shapes, level_start_index, sampling_locations, attention_weights,
          grad_output, grad_value, grad_sampling_locations, grad_attention_weights, s, workspace,
          workspace_bytes, phase, st);
    });
    return check_launch(fn);
  }
  // attention_weights are logits: the binning part writes their softmax to the
  // head of the workspace and bins with it; the rest turns the weight gradient
  // into the logit gradient in place
  const size_t pb = probs_bytes(s, geometry_dtype);
  if (!workspace || workspace_bytes < pb || !aligned(workspace, 256)) {
    return fail(MUSPACE_EINVAL, "%s: workspace of %zu bytes (256-byte aligned) required, got %zu",
                fn, pb, workspace_bytes);
  }
  void *probs = workspace;
  void *tiles = static_cast<unsigned char *>(workspace) + pb;
  with_dtypes(value_dtype, geometry_dtype, [&](auto vt, auto gt) {
    using VT = decltype(vt);
    using GT = decltype(gt);
    if (phase != Phase::kRest) launch_softmax<GT>(attention_weights, probs, s, st);
    launch_backward<VT, GT>(value, spatial_shapes, level_start_index, sampling_locations, probs,
                            grad_output, grad_value, grad_sampling_locations,
                            grad_attention_weights, s, tiles, workspace_bytes - pb, phase, st);
    if (phase != Phase::kBin) launch_softmax_backward<GT>(probs, grad_attention_weights, s, st);
  });
  return check_launch(fn);
}

// Scratch of the softmax backward: the probabilities, then the tile path's
// workspace when it applies.
size_t softmax_workspace_bytes(const msda::Shape &s, int value_dtype, int geometry_dtype) {
  TileWorkspace w;
  const size_t tiles = plan_tile_workspace(s, value_dtype, w) ? w.bytes : 0;
  return probs_bytes(s, geometry_dtype) + tiles;
}

// Scratch of ms_deform_attn_backward_noalloc: one array per GPU, in the code
// object's zero-initialised data, held until the process ends. In host code
// `scratch` is a host-side stand-in for the symbol; the device address comes
// from hipGetSymbolAddress, once per device.
constexpr size_t kNoAllocScratchBytes = MUSPACE_NOALLOC_SCRATCH_BYTES;
constexpr int kMaxDevices = 64;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];
std::mutex g_scratch_mutex;
void *g_scratch_ptr[kMaxDevices] = {};

// The current device's address of `scratch` into *out.
int scratch_on_current_device(const char *fn, void **out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    (void)hipGetLastError();
    return fail(MUSPACE_EINVAL, "%s: no current HIP device (or device index >= %d)", fn,
                kMaxDevices);
  }
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[dev] == nullptr) {
    void *p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
      (void)hipGetLastError();
      return fail(MUSPACE_ELAUNCH, "%s: hipGetSymbolAddress(scratch) failed on device %d: %s",
                  fn, dev, hipGetErrorString(e));
    }
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return ok();
}

// Batch entries per pass of the no-allocation backward: the largest count
// whose tile workspace fits the scratch (0 if one entry does not fit).
int64_t noalloc_batch_step(const msda::Shape &s, int value_dtype, size_t *one_entry_bytes) {
  int64_t nb = s.batch;
  *one_entry_bytes = 0;
  while (nb >= 1) {
    msda::Shape sc = s;
    sc.batch = static_cast<int>(nb);
    sc.units = static_cast<int>(nb * s.queries * s.heads);
    TileWorkspace w;
    if (!plan_tile_workspace(sc, value_dtype, w)) return 0;
    if (nb == 1) *one_entry_bytes = w.bytes;
    if (w.bytes <= kNoAllocScratchBytes) return nb;
    // the workspace grows about linearly with the batch entries; the next
    // count is at least 1, so that one entry's size is always planned (and
    // reported when even that does not fit)
    const int64_t scaled = static_cast<int64_t>(
        static_cast<double>(nb) * static_cast<double>(kNoAllocScratchBytes) /
        static_cast<double>(w.bytes));
    const int64_t next = scaled < nb ? scaled : nb - 1;
    if (nb == 1) break;
    nb = next < 1 ? 1 : next;
  }
  return 0;
}

}  // namespace

extern "C" {

int ms_deform_attn_forward(const void *value, int value_dtype, const int64_t *spatial_shapes,
                           const int64_t *level_start_index, const void *sampling_locations,
                           const void *attention_weights, int geometry_dtype, void *output,
                           int64_t batch, int64_t spatial_size, int64_t num_heads,
                           int64_t channels, int64_t num_levels, int64_t num_query,
                           int64_t num_point, int64_t im2col_step, void *stream) {
  static const char *fn = "ms_deform_attn_forward";
  const Args a{batch, spatial_size, num_heads, channels, num_levels, num_query, num_point,
               im2col_step};
  msda::Shape s;
  if (int rc = validate(fn, a, value_dtype, geometry_dtype, s)) return rc;
  if (!needs_data(s)) return ok();
  if (!output || ((!value || !spatial_shapes || !level_start_index || !sampling_locations ||
                   !attention_weights) &&
                  s.lp > 0)) {
    return fail(MUSPACE_EINVAL, "%s: null tensor pointer", fn);
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  using msda::bf16_t;
  switch (value_dtype) {
    case MUSPACE_DTYPE_F32:
      launch_forward<float, float>(value, spatial_shapes, level_start_index, sampling_locations,
                                   attention_weights, output, s, st);
      break;
    case MUSPACE_DTYPE_F16:
      if (geometry_dtype == MUSPACE_DTYPE_F32) {
        launch_forward<__half, float>(value, spatial_shapes, level_start_index,
                                      sampling_locations, attention_weights, output, s, st);
      } else {
        launch_forward<__half, __half>(value, spatial_shapes, level_start_index,
                                       sampling_locations, attention_weights, output, s, st);
      }
      break;
    default:
      if (geometry_dtype == MUSPACE_DTYPE_F32) {
        launch_forward<bf16_t, float>(value, spatial_shapes, level_start_index,
                                      sampling_locations, attention_weights, output, s, st);
      } else {
        launch_forward<bf16_t, bf16_t>(value, spatial_shapes, level_start_index,
                                       sampling_locations, attention_weights, output, s, st);
      }
      break;
  }
  return check_launch(fn);
}

int ms_deform_attn_forward_scatter_div(
    const void *value, int value_dtype, const int64_t *spatial_shapes,
    const int64_t *level_start_index, const void *sampling_locations,
    const void *attention_weights, int geometry_dtype, const int64_t *index, const void *count,
    void *slots, int64_t batch, int64_t num_cams, int64_t cam_id, int64_t valid_len,
    int64_t spatial_size, int64_t num_heads, int64_t channels, int64_t num_levels,
    int64_t max_len, int64_t num_point, int64_t num_query, void *stream) {
  static const char *fn = "ms_deform_attn_forward_scatter_div";
  const int64_t rows = batch * num_cams;
  const Args a{rows, spatial_size, num_heads, channels, num_levels, max_len, num_point,
               rows > 0 ? rows : 1};
  const CamDims c{batch, num_cams, max_len, num_query};
  msda::Shape full;
  if (int rc = validate_cameras(fn, a, c, value_dtype, geometry_dtype, full)) return rc;
  if (cam_id < 0 || cam_id >= num_cams || valid_len < 0 || valid_len > max_len) {
    return fail(MUSPACE_EINVAL,
                "%s: need 0 <= cam_id < num_cams and 0 <= valid_len <= max_len (cam_id=%lld "
                "num_cams=%lld valid_len=%lld max_len=%lld)",
                fn, (long long)cam_id, (long long)num_cams, (long long)valid_len,
                (long long)max_len);
  }
  // nothing is added (with num_query == 0 every index is skipped)
  if (batch == 0 || valid_len == 0 || full.lp == 0 || num_query == 0) return ok();
  if (!value || !spatial_shapes || !level_start_index || !sampling_locations ||
      !attention_weights || !index || !count || !slots) {
    return fail(MUSPACE_EINVAL, "%s: null tensor pointer", fn);
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  with_dtypes(value_dtype, geometry_dtype, [&](auto vt, auto gt) {
    using VT = decltype(vt);
    using GT = decltype(gt);
    msda::CameraSlots<VT, GT, false> out{};
    out.slots = static_cast<VT *>(slots);
    out.index = index;
    out.count = static_cast<const GT *>(count);
    out.cams = static_cast<int>(num_cams);
    out.cam0 = static_cast<int>(cam_id);
    out.ncam = 1;
    out.max_len = static_cast<int>(max_len);
    out.num_query = static_cast<int>(num_query);
    out.off[0] = 0;
    out.off[1] = static_cast<int>(valid_len);
    launch_scatter_div<VT, GT, false>(value, spatial_shapes, level_start_index,
                                      sampling_locations, attention_weights, out, full,
                                      static_cast<int>(batch), slots, st);
  });
  return check_launch(fn);
}

int ms_deform_attn_forward_scatter_div_cams(
    const void *value, int value_dtype, const int64_t *spatial_shapes,
    const int64_t *level_start_index, const void *sampling_locations,
    const void *attention_weights, int geometry_dtype, const int64_t *index,
    const int64_t *valid_lens, const void *count, void *slots, int64_t batch, int64_t num_cams,
    int64_t spatial_size, int64_t num_heads, int64_t channels, int64_t num_levels,
    int64_t max_len, int64_t num_point, int64_t num_query, void *stream) {
  static const char *fn = "ms_deform_attn_forward_scatter_div_cams";
  const int64_t rows = batch * num_cams;
  const Args a{rows, spatial_size, num_heads, channels, num_levels, max_len, num_point,
               rows > 0 ? rows : 1};
  const CamDims c{batch, num_cams, max_len, num_query};
  msda::Shape full;
  if (int rc = validate_cameras(fn, a, c, value_dtype, geometry_dtype, full)) return rc;
  int64_t total = 0;
  if (int rc = check_lengths(fn, valid_lens, num_cams, max_len, total)) return rc;
  // nothing is added (with num_query == 0 every index is skipped)
  if (batch == 0 || total == 0 || full.lp == 0 || num_query == 0) return ok();
  if (!value || !spatial_shapes || !level_start_index || !sampling_locations ||
      !attention_weights || !index || !count || !slots) {
    return fail(MUSPACE_EINVAL, "%s: null tensor pointer", fn);
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int cams = static_cast<int>(num_cams);
  with_dtypes(value_dtype, geometry_dtype, [&](auto vt, auto gt) {
    using VT = decltype(vt);
    using GT = decltype(gt);
    auto fill = [&](auto &out, int cam0, int ncam) {
      out.slots = static_cast<VT *>(slots);
      out.count = static_cast<const GT *>(count);
      out.cams = cams;
      out.cam0 = cam0;
      out.ncam = ncam;
      out.max_len = static_cast<int>(max_len);
      out.num_query = static_cast<int>(num_query);
      fill_camera_table(out, valid_lens, cam0, ncam);
    };
    int64_t first = 0;  // index entry of the launch's first row
    if constexpr (std::is_same<VT, float>::value) {
      // float32 slots: up to kMaxCams cameras per launch, added with atomics
      for (int cam0 = 0; cam0 < cams; cam0 += msda::kMaxCams) {
        msda::CameraSlots<float, GT, true> out{};
        fill(out, cam0, cams - cam0 < msda::kMaxCams ? cams - cam0 : msda::kMaxCams);
        out.index = index + first;
        launch_scatter_div<float, GT, true>(value, spatial_shapes, level_start_index,
                                            sampling_locations, attention_weights, out, full,
                                            static_cast<int>(batch), slots, st);
        first += out.off[out.ncam];
      }
    } else {
      // 16-bit slots: one camera per launch, in order, plain read-modify-write
      for (int cam = 0; cam < cams; ++cam) {
        msda::CameraSlots<VT, GT, false> out{};
        fill(out, cam, 1);
        out.index = index + first;
        launch_scatter_div<VT, GT, false>(value, spatial_shapes, level_start_index,
                                          sampling_locations, attention_weights, out, full,
                                          static_cast<int>(batch), slots, st);
        first += out.off[1];
      }
    }
  });
  return check_launch(fn);
}

int ms_deform_attn_scatter_div_grad(const void *grad_slots, int value_dtype,
                                    const int64_t *index, const int64_t *valid_lens,
                                    const void *count, int count_dtype, void *grad_output,
                                    int64_t batch, int64_t num_cams, int64_t max_len,
                                    int64_t num_query, int64_t row, void *stream) {
  static const char *fn = "ms_deform_attn_scatter_div_grad";
  if (value_dtype != MUSPACE_DTYPE_F32 && value_dtype != MUSPACE_DTYPE_F16 &&
      value_dtype != MUSPACE_DTYPE_BF16) {
    return fail(MUSPACE_EINVAL, "%s: grad must be float32, float16 or bfloat16 (dtype code %d)",
                fn, value_dtype);
  }
  if (count_dtype != MUSPACE_DTYPE_F32 && count_dtype != value_dtype) {
    return fail(MUSPACE_EINVAL, "%s: count must be float32 or %s, got %s", fn,
                dtype_name(value_dtype), dtype_name(count_dtype));
  }
  if (batch < 0 || num_cams <= 0 || max_len < 0 || num_query < 0 || row <= 0) {
    return fail(MUSPACE_EINVAL,
                "%s: invalid dims batch=%lld num_cams=%lld max_len=%lld num_query=%lld row=%lld",
                fn, (long long)batch, (long long)num_cams, (long long)max_len,
                (long long)num_query, (long long)row);
  }
  if (batch * num_cams > INT_MAX || max_len > INT_MAX || num_query > INT_MAX || row > INT_MAX) {
    return fail(MUSPACE_ERANGE, "%s: dims exceed int32", fn);
  }
  int64_t total = 0;
  if (int rc = check_lengths(fn, valid_lens, num_cams, max_len, total)) return rc;
  if (batch == 0 || max_len == 0) return ok();
  if (!grad_output || (total > 0 && (!grad_slots || !index || !count))) {
    return fail(MUSPACE_EINVAL, "%s: null tensor pointer", fn);
  }
  const CamDims c{batch, num_cams, max_len, num_query};
  hipStream_t st = static_cast<hipStream_t>(stream);
  with_dtypes(value_dtype, count_dtype, [&](auto vt, auto gt) {
    launch_scatter_div_grad<decltype(vt), decltype(gt)>(grad_slots, index, valid_lens, count,
                                                        grad_output, c, static_cast<int>(row),
                                                        st);
  });
  return check_launch(fn);
}

size_t ms_deform_attn_backward_workspace_size(int value_dtype, int64_t batch,
                                              int64_t spatial_size, int64_t num_heads,
                                              int64_t channels, int64_t num_levels,
                                              int64_t num_query, int64_t num_point) {
  const Args a{batch, spatial_size, num_heads, channels, num_levels, num_query, num_point,
               batch > 0 ? batch : 1};
  msda::Shape s;
  if (validate("ms_deform_attn_backward_workspace_size", a, value_dtype, value_dtype, s)) {
    return 0;
  }
  ok();
  TileWorkspace w;
  if (!needs_data(s) || s.lp == 0 || !plan_tile_workspace(s, value_dtype, w)) return 0;
  return w.bytes;
}

int ms_deform_attn_forward_bin_fused(int value_dtype, int64_t batch, int64_t spatial_size,
                                     int64_t num_heads, int64_t channels, int64_t num_levels,
                                     int64_t num_query, int64_t num_point) {
  const Args a{batch, spatial_size, num_heads, channels, num_levels, num_query, num_point,
               batch > 0 ? batch : 1};
  msda::Shape s;
  if (validate("ms_deform_attn_forward_bin_fused", a, value_dtype, value_dtype, s)) return 0;
  ok();
  TileWorkspace w;
  int units = 0, slots = 0;
  return needs_data(s) && s.lp > 0 && plan_tile_workspace(s, value_dtype, w) &&
                 fwd_bin_fuses(s, value_dtype, w, units, slots)
             ? 1
             : 0;
}

int ms_deform_attn_backward_ws(const void *value, int value_dtype, const int64_t *spatial_shapes,
                               const int64_t *level_start_index, const void *sampling_locations,
                               const void *attention_weights, int geometry_dtype,
                               const void *grad_output, float *grad_value,
                               float *grad_sampling_locations, float *grad_attention_weights,
                               int64_t batch, int64_t spatial_size, int64_t num_heads,
                               int64_t channels, int64_t num_levels, int64_t num_query,
                               int64_t num_point, int64_t im2col_step, void *workspace,
                               size_t workspace_bytes, void *stream) {
  const Args a{batch, spatial_size, num_heads, channels, num_levels, num_query, num_point,
               im2col_step};
  return backward_impl("ms_deform_attn_backward_ws", value, value_dtype, spatial_shapes,
                       level_start_index, sampling_locations, attention_weights, geometry_dtype,
                       grad_output, grad_value, grad_sampling_locations, grad_attention_weights,
                       a, workspace, workspace_bytes, static_cast<hipStream_t>(stream));
}

int ms_deform_attn_backward_bin(const void *value, int value_dtype,
                                const int64_t *spatial_shapes, const int64_t *level_start_index,
                                const void *sampling_locations, const void *attention_weights,
                                int geometry_dtype, const void *grad_output, float *grad_value,
                                float *grad_sampling_locations, float *grad_attention_weights,
                                int64_t batch, int64_t spatial_size, int64_t num_heads,
                                int64_t channels, int64_t num_levels, int64_t num_query,
                                int64_t num_point, int64_t im2col_step, void *workspace,
                                size_t workspace_bytes, void *stream) {
  const Args a{batch, spatial_size, num_heads, channels, num_levels, num_query, num_point,
               im2col_step};
  return backward_impl("ms_deform_attn_backward_bin", value, value_dtype, spatial_shapes,
                       level_start_index, sampling_locations, attention_weights, geometry_dtype,
                       grad_output, grad_value, grad_sampling_locations, grad_attention_weights,
                       a, workspace, workspace_bytes, static_cast<hipStream_t>(stream),
                       Phase::kBin);
}

int ms_deform_attn_backward_rest(const void *value, int value_dtype,
                                 const int64_t *spatial_shapes, const int64_t *level_start_index,
                                 const void *sampling_locations, const void *attention_weights,
                                 int geometry_dtype, const void *grad_output, float *grad_value,
                                 float *grad_sampling_locations, float *grad_attention_weights,
                                 int64_t batch, int64_t spatial_size, int64_t num_heads,
                                 int64_t channels, int64_t num_levels, int64_t num_query,
                                 int64_t num_point, int64_t im2col_step, void *workspace,
                                 size_t workspace_bytes, void *stream) {
  const Args a{batch, spatial_size, num_heads, channels, num_levels, num_query, num_point,
               im2col_step};
  return backward_impl("ms_deform_attn_backward_rest", value, value_dtype, spatial_shapes,
                       level_start_index, sampling_locations, attention_weights, geometry_dtype,
                       grad_output, grad_value, grad_sampling_locations, grad_attention_weights,
                       a, workspace, workspace_bytes, static_cast<hipStream_t>(stream),
                       Phase::kRest);
}

int ms_deform_attn_forward_bin(const void *value, int value_dtype, const int64_t *spatial_shapes,
                               const int64_t *level_start_index, const void *sampling_locations,
                               const void *attention_weights, int geometry_dtype, void *output,
                               float *grad_value, float *grad_sampling_locations,
                               float *grad_attention_weights, int64_t batch,
                               int64_t spatial_size, int64_t num_heads, int64_t channels,
                               int64_t num_levels, int64_t num_query, int64_t num_point,
                               int64_t im2col_step, void *workspace, size_t workspace_bytes,
                               void *stream) {
  static const char *fn = "ms_deform_attn_forward_bin";
  const Args a{batch, spatial_size, num_heads, channels, num_levels, num_query, num_point,
               im2col_step};
  msda::Shape s;
  if (int rc = validate(fn, a, value_dtype, geometry_dtype, s)) return rc;
  hipStream_t st = static_cast<hipStream_t>(stream);
  bool fused = false;
  if (needs_data(s) && s.lp > 0) {
    if (!value || !spatial_shapes || !level_start_index || !sampling_locations ||
        !attention_weights || !output || !grad_value || !grad_sampling_locations ||
        !grad_attention_weights) {
      return fail(MUSPACE_EINVAL, "%s: null tensor pointer", fn);
    }
    with_dtypes(value_dtype, geometry_dtype, [&](auto vt, auto gt) {
      fused = launch_forward_bin<decltype(vt), decltype(gt)>(
          value, spatial_shapes, level_start_index, sampling_locations, attention_weights,
          output, grad_value, grad_sampling_locations, grad_attention_weights, s, workspace,
          workspace_bytes, st);
    });
    if (fused) return check_launch(fn);
  }
  // the two calls this one stands for
  if (int rc = ms_deform_attn_forward(value, value_dtype, spatial_shapes, level_start_index,
                                      sampling_locations, attention_weights, geometry_dtype,
                                      output, batch, spatial_size, num_heads, channels,
                                      num_levels, num_query, num_point, im2col_step, stream)) {
    return rc;
  }
  return ms_deform_attn_backward_bin(value, value_dtype, spatial_shapes, level_start_index,
                                     sampling_locations, attention_weights, geometry_dtype,
                                     nullptr, grad_value, grad_sampling_locations,
                                     grad_attention_weights, batch, spatial_size, num_heads,
                                     channels, num_levels, num_query, num_point, im2col_step,
                                     workspace, workspace_bytes, stream);
}

int ms_deform_attn_backward(const void *value, int value_dtype, const int64_t *spatial_shapes,
                            const int64_t *level_start_index, const void *sampling_locations,
                            const void *attention_weights, int geometry_dtype,
                            const void *grad_output, float *grad_value,
                            float *grad_sampling_locations, float *grad_attention_weights,
                            int64_t batch, int64_t spatial_size, int64_t num_heads,
                            int64_t channels, int64_t num_levels, int64_t num_query,
                            int64_t num_point, int64_t im2col_step, void *stream) {
  static const char *fn = "ms_deform_attn_backward";
  const Args a{batch, spatial_size, num_heads, channels, num_levels, num_query, num_point,
               im2col_step};
  hipStream_t st = static_cast<hipStream_t>(stream);
  msda::Shape s;
  if (int rc = validate(fn, a, value_dtype, geometry_dtype, s)) return rc;
  if (needs_data(s) && s.lp > 0 &&
      (!value || !spatial_shapes || !level_start_index || !sampling_locations ||
       !attention_weights || !grad_output || !grad_value || !grad_sampling_locations ||
       !grad_attention_weights)) {
    return fail(MUSPACE_EINVAL, "%s: null tensor pointer", fn);
  }
  // stream-ordered scratch of the tile-owned path; freed in stream order
  size_t bytes = 0;
  TileWorkspace w;
  if (needs_data(s) && s.lp > 0 && plan_tile_workspace(s, value_dtype, w)) bytes = w.bytes;
  void *workspace = nullptr;
  if (bytes > 0 && hipMallocAsync(&workspace, bytes, st) != hipSuccess) {
    (void)hipGetLastError();
    workspace = nullptr;  // the atomic fallback needs no scratch
    bytes = 0;
  }
  const int rc = backward_impl(fn, value, value_dtype, spatial_shapes, level_start_index,
                               sampling_locations, attention_weights, geometry_dtype, grad_output,
                               grad_value, grad_sampling_locations, grad_attention_weights, a,
                               workspace, bytes, st);
  if (workspace) (void)hipFreeAsync(workspace, st);
  return rc;
}

int ms_deform_attn_backward_noalloc(const void *value, int value_dtype,
                                    const int64_t *spatial_shapes,
                                    const int64_t *level_start_index,
                                    const void *sampling_locations,
                                    const void *attention_weights, int geometry_dtype,
                                    const void *grad_output, float *grad_value,
                                    float *grad_sampling_locations,
                                    float *grad_attention_weights, int64_t batch,
                                    int64_t spatial_size, int64_t num_heads, int64_t channels,
                                    int64_t num_levels, int64_t num_query, int64_t num_point,
                                    int64_t im2col_step, void *stream) {
  static const char *fn = "ms_deform_attn_backward_noalloc";
  const Args a{batch, spatial_size, num_heads, channels, num_levels, num_query, num_point,
               im2col_step};
  hipStream_t st = static_cast<hipStream_t>(stream);
  msda::Shape s;
  if (int rc = validate(fn, a, value_dtype, geometry_dtype, s)) return rc;
  TileWorkspace w;
  const bool tiles = needs_data(s) && s.lp > 0 && plan_tile_workspace(s, value_dtype, w);
  if (!tiles) {  // zero gradients or the atomic fallback: no scratch at all
    return backward_impl(fn, value, value_dtype, spatial_shapes, level_start_index,
                         sampling_locations, attention_weights, geometry_dtype, grad_output,
                         grad_value, grad_sampling_locations, grad_attention_weights, a, nullptr,
                         0, st);
  }
  if (!value || !spatial_shapes || !level_start_index || !sampling_locations ||
      !attention_weights || !grad_output || !grad_value || !grad_sampling_locations ||
      !grad_attention_weights) {
    return fail(MUSPACE_EINVAL, "%s: null tensor pointer", fn);
  }
  size_t one_entry = 0;
  const int64_t step = noalloc_batch_step(s, value_dtype, &one_entry);
  if (step <= 0) {
    return fail(MUSPACE_ERANGE,
                "%s: one batch entry of this shape needs %zu bytes of scratch; the "
                "no-allocation scratch holds %zu (use ms_deform_attn_backward or _ws)",
                fn, one_entry, kNoAllocScratchBytes);
  }
  void *ws = nullptr;
  if (int rc = scratch_on_current_device(fn, &ws)) return rc;
  const size_t vb = value_dtype == MUSPACE_DTYPE_F32 ? 4 : 2;
  const size_t gb = geometry_dtype == MUSPACE_DTYPE_F32 ? 4 : 2;
  const size_t per_value = static_cast<size_t>(spatial_size) * num_heads * channels;
  const size_t per_sample = static_cast<size_t>(num_query) * num_heads * num_levels * num_point;
  const size_t per_out = static_cast<size_t>(num_query) * num_heads * channels;
  for (int64_t b0 = 0; b0 < batch; b0 += step) {
    const int64_t nb = batch - b0 < step ? batch - b0 : step;
    const Args ab{nb, spatial_size, num_heads, channels, num_levels, num_query, num_point, nb};
    const size_t b = static_cast<size_t>(b0);
    const int rc = backward_impl(
        fn, static_cast<const unsigned char *>(value) + b * per_value * vb, value_dtype,
        spatial_shapes, level_start_index,
        static_cast<const unsigned char *>(sampling_locations) + b * per_sample * 2 * gb,
        static_cast<const unsigned char *>(attention_weights) + b * per_sample * gb,
        geometry_dtype, static_cast<const unsigned char *>(grad_output) + b * per_out * vb,
        grad_value + b * per_value, grad_sampling_locations + b * per_sample * 2,
        grad_attention_weights + b * per_sample, ab, ws, kNoAllocScratchBytes, st);
    if (rc != MUSPACE_OK) return rc;
  }
  return ok();
}

int ms_deform_attn_forward_softmax(const void *value, int value_dtype,
                                   const int64_t *spatial_shapes,
                                   const int64_t *level_start_index,
                                   const void *sampling_locations, const void *attention_logits,
                                   int geometry_dtype, void *output, int64_t batch,
                                   int64_t spatial_size, int64_t num_heads, int64_t channels,
                                   int64_t num_levels, int64_t num_query, int64_t num_point,
                                   int64_t im2col_step, void *stream) {
  static const char *fn = "ms_deform_attn_forward_softmax";
  const Args a{batch, spatial_size, num_heads, channels, num_levels, num_query, num_point,
               im2col_step};
  msda::Shape s;
  if (int rc = validate(fn, a, value_dtype, geometry_dtype, s)) return rc;
  if (!needs_data(s)) return ok();
  if (!output || ((!value || !spatial_shapes || !level_start_index || !sampling_locations ||
                   !attention_logits) &&
                  s.lp > 0)) {
    return fail(MUSPACE_EINVAL, "%s: null tensor pointer", fn);
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  bool launched = true;
  with_dtypes(value_dtype, geometry_dtype, [&](auto vt, auto gt) {
    launched = launch_forward_softmax<decltype(vt), decltype(gt)>(
        value, spatial_shapes, level_start_index, sampling_locations, attention_logits, output, s,
        geometry_dtype, st);
  });
  if (!launched) return fail(MUSPACE_ENOMEM, "%s: scratch allocation failed", fn);
  return check_launch(fn);
}

size_t ms_deform_attn_backward_softmax_workspace_size(int value_dtype, int geometry_dtype,
                                                      int64_t batch, int64_t spatial_size,
                                                      int64_t num_heads, int64_t channels,
                                                      int64_t num_levels, int64_t num_query,
                                                      int64_t num_point) {
  const Args a{batch, spatial_size, num_heads, channels, num_levels, num_query, num_point,
               batch > 0 ? batch : 1};
  msda::Shape s;
  if (validate("ms_deform_attn_backward_softmax_workspace_size", a, value_dtype, geometry_dtype,
               s)) {
    return 0;
  }
  ok();
  if (!needs_data(s) || s.lp == 0) return 0;
  return softmax_workspace_bytes(s, value_dtype, geometry_dtype);
}

int ms_deform_attn_backward_softmax_bin(
    const void *value, int value_dtype, const int64_t *spatial_shapes,
    const int64_t *level_start_index, const void *sampling_locations,
    const void *attention_logits, int geometry_dtype, const void *grad_output, float *grad_value,
    float *grad_sampling_locations, float *grad_attention_logits, int64_t batch,
    int64_t spatial_size, int64_t num_heads, int64_t channels, int64_t num_levels,
    int64_t num_query, int64_t num_point, int64_t im2col_step, void *workspace,
    size_t workspace_bytes, void *stream) {
  const Args a{batch, spatial_size, num_heads, channels, num_levels, num_query, num_point,
               im2col_step};
  return backward_impl("ms_deform_attn_backward_softmax_bin", value, value_dtype, spatial_shapes,
                       level_start_index, sampling_locations, attention_logits, geometry_dtype,
                       grad_output, grad_value, grad_sampling_locations, grad_attention_logits,
                       a, workspace, workspace_bytes, static_cast<hipStream_t>(stream),
                       Phase::kBin, true);
}

int ms_deform_attn_forward_softmax_bin(
    const void *value, int value_dtype, const int64_t *spatial_shapes,
    const int64_t *level_start_index, const void *sampling_locations,
    const void *attention_logits, int geometry_dtype, void *output, float *grad_value,
    float *grad_sampling_locations, float *grad_attention_logits, int64_t batch,
    int64_t spatial_size, int64_t num_heads, int64_t channels, int64_t num_levels,
    int64_t num_query, int64_t num_point, int64_t im2col_step, void *workspace,
    size_t workspace_bytes, void *stream) {
  static const char *fn = "ms_deform_attn_forward_softmax_bin";
  const Args a{batch, spatial_size, num_heads, channels, num_levels, num_query, num_point,
               im2col_step};
  msda::Shape s;
  if (int rc = validate(fn, a, value_dtype, geometry_dtype, s)) return rc;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (needs_data(s) && s.lp > 0) {
    if (!value || !spatial_shapes || !level_start_index || !sampling_locations ||
        !attention_logits || !output || !grad_value || !grad_sampling_locations ||
        !grad_attention_logits) {
      return fail(MUSPACE_EINVAL, "%s: null tensor pointer", fn);
    }
    // the probabilities head the workspace, as in the softmax backward
    const size_t pb = probs_bytes(s, geometry_dtype);
    if (!workspace || workspace_bytes < pb || !aligned(workspace, 256)) {
      return fail(MUSPACE_EINVAL,
                  "%s: workspace of %zu bytes (256-byte aligned) required, got %zu", fn, pb,
                  workspace_bytes);
    }
    unsigned char *tiles = static_cast<unsigned char *>(workspace) + pb;
    bool fused = false;
    with_dtypes(value_dtype, geometry_dtype, [&](auto vt, auto gt) {
      fused = launch_forward_bin<decltype(vt), decltype(gt)>(
          value, spatial_shapes, level_start_index, sampling_locations, attention_logits, output,
          grad_value, grad_sampling_locations, grad_attention_logits, s, tiles,
          workspace_bytes - pb, st, workspace);
    });
    if (fused) return check_launch(fn);
  }
  // the two calls this one stands for
  if (int rc = ms_deform_attn_forward_softmax(value, value_dtype, spatial_shapes,
                                              level_start_index, sampling_locations,
                                              attention_logits, geometry_dtype, output, batch,
                                              spatial_size, num_heads, channels, num_levels,
                                              num_query, num_point, im2col_step, stream)) {
    return rc;
  }
  return ms_deform_attn_backward_softmax_bin(
      value, value_dtype, spatial_shapes, level_start_index, sampling_locations,
      attention_logits, geometry_dtype, nullptr, grad_value, grad_sampling_locations,
      grad_attention_logits, batch, spatial_size, num_heads, channels, num_levels, num_query,
      num_point, im2col_step, workspace, workspace_bytes, stream);
}

int ms_deform_attn_forward_softmax_bin_fused(int value_dtype, int64_t batch,
                                             int64_t spatial_size, int64_t num_heads,
                                             int64_t channels, int64_t num_levels,
                                             int64_t num_query, int64_t num_point) {
  const Args a{batch, spatial_size, num_heads, channels, num_levels, num_query, num_point,
               batch > 0 ? batch : 1};
  msda::Shape s;
  if (validate("ms_deform_attn_forward_softmax_bin_fused", a, value_dtype, value_dtype, s)) {
    return 0;
  }
  ok();
  TileWorkspace w;
  int units = 0, slots = 0;
  return needs_data(s) && s.lp > 0 && plan_tile_workspace(s, value_dtype, w) &&
                 fwd_bin_fuses(s, value_dtype, w, units, slots, true)
             ? 1
             : 0;
}

int ms_deform_attn_backward_softmax_rest(
    const void *value, int value_dtype, const int64_t *spatial_shapes,
    const int64_t *level_start_index, const void *sampling_locations,
    const void *attention_logits, int geometry_dtype, const void *grad_output, float *grad_value,
    float *grad_sampling_locations, float *grad_attention_logits, int64_t batch,
    int64_t spatial_size, int64_t num_heads, int64_t channels, int64_t num_levels,
    int64_t num_query, int64_t num_point, int64_t im2col_step, void *workspace,
    size_t workspace_bytes, void *stream) {
  const Args a{batch, spatial_size, num_heads, channels, num_levels, num_query, num_point,
               im2col_step};
  return backward_impl("ms_deform_attn_backward_softmax_rest", value, value_dtype, spatial_shapes,
                       level_start_index, sampling_locations, attention_logits, geometry_dtype,
                       grad_output, grad_value, grad_sampling_locations, grad_attention_logits,
                       a, workspace, workspace_bytes, static_cast<hipStream_t>(stream),
                       Phase::kRest, true);
}

int ms_deform_attn_backward_softmax(
    const void *value, int value_dtype, const int64_t *spatial_shapes,
    const int64_t *level_start_index, const void *sampling_locations,
    const void *attention_logits, int geometry_dtype, const void *grad_output, float *grad_value,
    float *grad_sampling_locations, float *grad_attention_logits, int64_t batch,
    int64_t spatial_size, int64_t num_heads, int64_t channels, int64_t num_levels,
    int64_t num_query, int64_t num_point, int64_t im2col_step, void *stream) {
  static const char *fn = "ms_deform_attn_backward_softmax";
  const Args a{batch, spatial_size, num_heads, channels, num_levels, num_query, num_point,
               im2col_step};
  hipStream_t st = static_cast<hipStream_t>(stream);
  msda::Shape s;
  if (int rc = validate(fn, a, value_dtype, geometry_dtype, s)) return rc;
  // stream-ordered scratch (probabilities and binning); freed in stream order
  const size_t bytes =
      needs_data(s) && s.lp > 0 ? softmax_workspace_bytes(s, value_dtype, geometry_dtype) : 0;
  void *workspace = nullptr;
  if (bytes > 0 && hipMallocAsync(&workspace, bytes, st) != hipSuccess) {
    (void)hipGetLastError();
    return fail(MUSPACE_ENOMEM, "%s: scratch allocation of %zu bytes failed", fn, bytes);
  }
  const int rc = backward_impl(fn, value, value_dtype, spatial_shapes, level_start_index,
                               sampling_locations, attention_logits, geometry_dtype, grad_output,
                               grad_value, grad_sampling_locations, grad_attention_logits, a,
                               workspace, bytes, st, Phase::kAll, true);
  if (workspace) (void)hipFreeAsync(workspace, st);
  return rc;
}

int add_one(const float *x, float *y, int64_t n, void *stream) {
  if (n < 0) return fail(MUSPACE_EINVAL, "add_one: negative size %lld", (long long)n);
  if (n == 0) return ok();
  if (!x || !y) return fail(MUSPACE_EINVAL, "add_one: null tensor pointer");
  msda::add_one_kernel<<<generic_blocks(n), msda::kBlock, 0, static_cast<hipStream_t>(stream)>>>(
      x, y, n);
  return check_launch("add_one");
}

const char *muspace_last_error(void) { return capi::g_error; }

int muspace_abi_version(void) { return MUSPACE_MSDA_ABI_VERSION; }

}  // extern "C"
