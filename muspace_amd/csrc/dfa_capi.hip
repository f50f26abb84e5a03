// C-ABI entry points of deformable aggregation (declared in include/muspace_dfa.h).
//
// Replaces the reference's four TVM-FFI exports
// deformable_aggregation_{forward,backward}_{opt,base}
// (/root/reference/csrc/deformable_aggregation/deformable_aggregation_musa.mu:683-751),
// keeping their argument order (feature maps, spatial_shape, scale_start_index,
// sampling_location, weights, outputs) and their accumulate semantics: the
// forward adds into `output` and the backward adds into `grad_mc_ms_feat`
// (callers zero them, as the reference's autograd function does), while the
// location and weight gradients are written. "opt" takes the wavefront-per-
// anchor row kernels when the channel layout allows it; "base" always takes
// the generic kernels.
#include <hip/hip_runtime.h>

#include <climits>
#include <cstdint>

#include "../../include/muspace_dfa.h"
#include "capi_errors.hpp"
#include "dfa_kernels.hpp"

namespace {

using capi::check_launch;
using capi::fail;
using capi::ok;

struct DfaArgs {
  int64_t batch, cams, feat, embeds, scales, anchors, pts, groups;
};

int validate(const char *fn, const DfaArgs &a, dfa::Dims &d) {
  if (a.batch < 0 || a.cams < 0 || a.feat < 0 || a.embeds <= 0 || a.scales < 0 ||
      a.anchors < 0 || a.pts < 0) {
    return fail(MUSPACE_EINVAL,
                "%s: invalid dims batch=%lld num_cams=%lld num_feat=%lld num_embeds=%lld "
                "num_scale=%lld num_anchors=%lld num_pts=%lld",
                fn, (long long)a.batch, (long long)a.cams, (long long)a.feat,
                (long long)a.embeds, (long long)a.scales, (long long)a.anchors,
                (long long)a.pts);
  }
  if (a.groups <= 0 || a.groups > dfa::kMaxGroups) {
    return fail(MUSPACE_EINVAL, "%s: num_groups must be in [1, %d], got %lld", fn,
                dfa::kMaxGroups, (long long)a.groups);
  }
  if (a.embeds % a.groups != 0) {
    return fail(MUSPACE_EINVAL, "%s: num_embeds %lld must be divisible by num_groups %lld", fn,
                (long long)a.embeds, (long long)a.groups);
  }
  if (a.cams * a.scales > dfa::kMaxViews) {
    return fail(MUSPACE_EINVAL, "%s: num_cams * num_scale must be at most %d, got %lld", fn,
                dfa::kMaxViews, (long long)(a.cams * a.scales));
  }
  if (a.batch * a.anchors > INT_MAX || a.feat > INT_MAX || a.embeds > INT_MAX ||
      a.pts * a.cams > INT_MAX / 2) {
    return fail(MUSPACE_ERANGE, "%s: dims exceed the kernels' 32-bit indexing", fn);
  }
  d.batch = static_cast<int>(a.batch);
  d.cams = static_cast<int>(a.cams);
  d.feat = static_cast<int>(a.feat);
  d.embeds = static_cast<int>(a.embeds);
  d.scales = static_cast<int>(a.scales);
  d.anchors = static_cast<int>(a.anchors);
  d.pts = static_cast<int>(a.pts);
  d.groups = static_cast<int>(a.groups);
  return ok();
}

int generic_blocks(int64_t work) {
  int64_t b = (work + dfa::kBlock - 1) / dfa::kBlock;
  if (b > 65536) b = 65536;
  if (b < 1) b = 1;
  return static_cast<int>(b);
}

// Channel slots per lane of the row kernels (C = 64 * NT), or 0 when the
// layout needs the generic kernels: C a multiple of 64 up to 256, each group
// a power-of-two run of lanes or a whole number of 64-channel slots, and the
// features addressable with 32-bit byte offsets.
int row_slots(const dfa::Dims &d) {
  const int C = d.embeds;
  if (C % dfa::kWave != 0 || C / dfa::kWave > 4) return 0;
  const int cpg = C / d.groups;
  const bool pow2 = (cpg & (cpg - 1)) == 0;
  if (!(cpg % dfa::kWave == 0 || (cpg < dfa::kWave && pow2))) return 0;
  const uint64_t bytes = static_cast<uint64_t>(d.batch) * d.feat * C * 4u;
  if (bytes + 64 > dfa::kOobOffset) return 0;
  return C / dfa::kWave;
}

// Channel slice of dfa_backward_coarse (0: every map is left to the row
// kernel's atomics), with its accumulator budget in cells and the bound on
// contributions per sum (2^pair_log2 >= anchors * pts). The host does not see
// the map sizes (device tensors), so it sizes the slice for the maps below the
// finest of a pyramid that halves each scale, about a quarter of a camera's
// rows: the widest slice whose accumulators hold that many cells. The kernels
// choose the maps that fit on the device. The kernel reads grad_output in
// 16-byte pieces and locations in 8-byte pieces, so it needs pointers aligned
// to those.
int coarse_slice(const dfa::Dims &d, const float *loc, const float *grad_out, int &budget,
                 int &pair_log2) {
  const int64_t pairs = static_cast<int64_t>(d.anchors) * d.pts;
  if (d.scales == 0 || d.cams == 0 || pairs > (int64_t{1} << 20) ||
      reinterpret_cast<uintptr_t>(grad_out) % 16 != 0 || reinterpret_cast<uintptr_t>(loc) % 8 != 0) {
    return 0;
  }
  pair_log2 = 0;
  while ((int64_t{1} << pair_log2) < pairs) ++pair_log2;
  const int cpg = d.embeds / d.groups;
  const int64_t want = static_cast<int64_t>(d.feat) / d.cams / 4;
  for (int cs : {16, 8, 4}) {
    if (cpg % cs != 0) continue;
    budget = dfa::kCoarseLdsBytes / (8 * cs);
    if (budget >= want || cs == 4) return cs;
  }
  return 0;
}

template <int CS>
void launch_coarse(const int32_t *shape, const int32_t *start, const float *loc,
                   const float *weights, const float *grad_out, float *grad_feat,
                   const dfa::Dims &d, int budget, int pair_log2, hipStream_t st) {
  const size_t lds = static_cast<size_t>(budget) * CS * sizeof(unsigned long long);
  (void)hipFuncSetAttribute(reinterpret_cast<const void *>(dfa::dfa_backward_coarse<CS>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
  // a workgroup takes up to four slices of one weight group
  const int per_group = d.embeds / d.groups / CS;
  int ns = 4;
  while (per_group % ns != 0) --ns;
  const int blocks = d.batch * d.cams * (d.embeds / (CS * ns));
  dfa::dfa_backward_coarse<CS><<<blocks, dfa::kCoarseBlock, lds, st>>>(
      shape, start, loc, weights, grad_out, grad_feat, d, budget, pair_log2, ns);
}

int forward_impl(const char *fn, bool optimized, const float *feat, const int32_t *shape,
                 const int32_t *start, const float *loc, const float *weights, float *out,
                 const DfaArgs &a, void *stream) {
  dfa::Dims d;
  if (int rc = validate(fn, a, d)) return rc;
  if (static_cast<int64_t>(d.batch) * d.anchors == 0) return ok();
  if (!out || ((!feat || !shape || !start || !loc || !weights) && d.pts * d.cams > 0)) {
    return fail(MUSPACE_EINVAL, "%s: null tensor pointer", fn);
  }
  if (d.pts * d.cams == 0 || d.scales == 0) return ok();  // nothing is added
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int nt = optimized ? row_slots(d) : 0;
  const int rows = d.batch * d.anchors;
  // wavefronts per row of dfa_forward_rows (1, 2 or 4: one workgroup holds a
  // row's parts): few rows give each SIMD few wavefronts with long serial
  // pair walks, so a row's pairs are shared
  const int parts = rows >= 8192 * 4 ? 1 : rows >= 8192 * 2 ? 2 : 4;
  const int units = nt > 0 ? rows * parts : rows;
  const int blocks = (units + dfa::kBlock / dfa::kWave - 1) / (dfa::kBlock / dfa::kWave);
  const uint32_t bytes = static_cast<uint32_t>(static_cast<uint64_t>(d.batch) * d.feat *
                                               d.embeds * 4u);
  switch (nt) {
    case 1:
      dfa::dfa_forward_rows<1><<<blocks, dfa::kBlock, 0, st>>>(feat, bytes, shape, start, loc,
                                                               weights, out, d, parts);
      break;
    case 2:
      dfa::dfa_forward_rows<2><<<blocks, dfa::kBlock, 0, st>>>(feat, bytes, shape, start, loc,
                                                               weights, out, d, parts);
      break;
    case 3:
      dfa::dfa_forward_rows<3><<<blocks, dfa::kBlock, 0, st>>>(feat, bytes, shape, start, loc,
                                                               weights, out, d, parts);
      break;
    case 4:
      dfa::dfa_forward_rows<4><<<blocks, dfa::kBlock, 0, st>>>(feat, bytes, shape, start, loc,
                                                               weights, out, d, parts);
      break;
    default:
      dfa::dfa_forward_generic<<<generic_blocks(static_cast<int64_t>(rows) * d.embeds),
                                 dfa::kBlock, 0, st>>>(feat, shape, start, loc, weights, out, d);
      break;
  }
  return check_launch(fn);
}

int backward_impl(const char *fn, bool optimized, const float *feat, const int32_t *shape,
                  const int32_t *start, const float *loc, const float *weights,
                  const float *grad_out, float *grad_feat, float *grad_loc, float *grad_weights,
                  const DfaArgs &a, void *stream) {
  dfa::Dims d;
  if (int rc = validate(fn, a, d)) return rc;
  if (static_cast<int64_t>(d.batch) * d.anchors * d.pts * d.cams == 0) return ok();
  if (!feat || !shape || !start || !loc || !grad_out || !grad_feat || !grad_loc ||
      (!weights && d.scales > 0) || (!grad_weights && d.scales > 0)) {
    return fail(MUSPACE_EINVAL, "%s: null tensor pointer", fn);
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int nt = optimized ? row_slots(d) : 0;
  const int rows = d.batch * d.anchors;
  // wavefronts per row of dfa_backward_rows: few rows give each of the 1024
  // SIMDs few wavefronts with long serial pair walks, so a row's pairs are
  // shared (SparseDrive's 7,200 rows: backward call 929 -> 842 us at four)
  const int parts = rows >= 8192 * 4 ? 1 : rows >= 8192 * 2 ? 2 : 4;
  const int units = nt > 0 ? rows * parts : rows;
  const int blocks = (units + dfa::kBlock / dfa::kWave - 1) / (dfa::kBlock / dfa::kWave);
  const uint32_t bytes = static_cast<uint32_t>(static_cast<uint64_t>(d.batch) * d.feat *
                                               d.embeds * 4u);
  // the small maps' feature gradients summed in LDS first (they only add)
  int budget = 0, pair_log2 = 0;
  const int cs = nt > 0 ? coarse_slice(d, loc, grad_out, budget, pair_log2) : 0;
  switch (cs) {
    case 16:
      launch_coarse<16>(shape, start, loc, weights, grad_out, grad_feat, d, budget, pair_log2,
                        st);
      break;
    case 8:
      launch_coarse<8>(shape, start, loc, weights, grad_out, grad_feat, d, budget, pair_log2, st);
      break;
    case 4:
      launch_coarse<4>(shape, start, loc, weights, grad_out, grad_feat, d, budget, pair_log2, st);
      break;
    default:
      budget = 0;
      break;
  }
  switch (nt) {
    case 1:
      dfa::dfa_backward_rows<1><<<blocks, dfa::kBlock, 0, st>>>(feat, bytes, shape, start, loc,
                                                                weights, grad_out, grad_feat,
                                                                grad_loc, grad_weights, d, budget,
                                                                parts);
      break;
    case 2:
      dfa::dfa_backward_rows<2><<<blocks, dfa::kBlock, 0, st>>>(feat, bytes, shape, start, loc,
                                                                weights, grad_out, grad_feat,
                                                                grad_loc, grad_weights, d, budget,
                                                                parts);
      break;
    case 3:
      dfa::dfa_backward_rows<3><<<blocks, dfa::kBlock, 0, st>>>(feat, bytes, shape, start, loc,
                                                                weights, grad_out, grad_feat,
                                                                grad_loc, grad_weights, d, budget,
                                                                parts);
      break;
    case 4:
      dfa::dfa_backward_rows<4><<<blocks, dfa::kBlock, 0, st>>>(feat, bytes, shape, start, loc,
                                                                weights, grad_out, grad_feat,
                                                                grad_loc, grad_weights, d, budget,
                                                                parts);
      break;
    default:
      dfa::dfa_backward_generic<<<generic_blocks(static_cast<int64_t>(rows) * d.pts * d.cams),
                                  dfa::kBlock, 0, st>>>(feat, shape, start, loc, weights,
                                                        grad_out, grad_feat, grad_loc,
                                                        grad_weights, d);
      break;
  }
  return check_launch(fn);
}

}  // namespace

extern "C" {

int deformable_aggregation_forward_opt(const float *mc_ms_feat, const int32_t *spatial_shape,
                                       const int32_t *scale_start_index,
                                       const float *sampling_location, const float *weights,
                                       float *output, int64_t batch, int64_t num_cams,
                                       int64_t num_feat, int64_t num_embeds, int64_t num_scale,
                                       int64_t num_anchors, int64_t num_pts, int64_t num_groups,
                                       void *stream) {
  const DfaArgs a{batch, num_cams, num_feat, num_embeds, num_scale, num_anchors, num_pts,
                  num_groups};
  return forward_impl("deformable_aggregation_forward_opt", true, mc_ms_feat, spatial_shape,
                      scale_start_index, sampling_location, weights, output, a, stream);
}

int deformable_aggregation_forward_base(const float *mc_ms_feat, const int32_t *spatial_shape,
                                        const int32_t *scale_start_index,
                                        const float *sampling_location, const float *weights,
                                        float *output, int64_t batch, int64_t num_cams,
                                        int64_t num_feat, int64_t num_embeds, int64_t num_scale,
                                        int64_t num_anchors, int64_t num_pts, int64_t num_groups,
                                        void *stream) {
  const DfaArgs a{batch, num_cams, num_feat, num_embeds, num_scale, num_anchors, num_pts,
                  num_groups};
  return forward_impl("deformable_aggregation_forward_base", false, mc_ms_feat, spatial_shape,
                      scale_start_index, sampling_location, weights, output, a, stream);
}

int deformable_aggregation_backward_opt(
    const float *mc_ms_feat, const int32_t *spatial_shape, const int32_t *scale_start_index,
    const float *sampling_location, const float *weights, const float *grad_output,
    float *grad_mc_ms_feat, float *grad_sampling_location, float *grad_weights, int64_t batch,
    int64_t num_cams, int64_t num_feat, int64_t num_embeds, int64_t num_scale,
    int64_t num_anchors, int64_t num_pts, int64_t num_groups, void *stream) {
  const DfaArgs a{batch, num_cams, num_feat, num_embeds, num_scale, num_anchors, num_pts,
                  num_groups};
  return backward_impl("deformable_aggregation_backward_opt", true, mc_ms_feat, spatial_shape,
                       scale_start_index, sampling_location, weights, grad_output,
                       grad_mc_ms_feat, grad_sampling_location, grad_weights, a, stream);
}

int deformable_aggregation_backward_base(
    const float *mc_ms_feat, const int32_t *spatial_shape, const int32_t *scale_start_index,
    const float *sampling_location, const float *weights, const float *grad_output,
    float *grad_mc_ms_feat, float *grad_sampling_location, float *grad_weights, int64_t batch,
    int64_t num_cams, int64_t num_feat, int64_t num_embeds, int64_t num_scale,
    int64_t num_anchors, int64_t num_pts, int64_t num_groups, void *stream) {
  const DfaArgs a{batch, num_cams, num_feat, num_embeds, num_scale, num_anchors, num_pts,
                  num_groups};
  return backward_impl("deformable_aggregation_backward_base", false, mc_ms_feat, spatial_shape,
                       scale_start_index, sampling_location, weights, grad_output,
                       grad_mc_ms_feat, grad_sampling_location, grad_weights, a, stream);
}

}  // extern "C"
