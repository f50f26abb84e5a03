/*
 * C-ABI of deformable aggregation (SparseDrive's multi-camera, multi-scale
 * deformable feature aggregation) in `libmuspace_msda.so`, MI355X (gfx950).
 *
 * These entry points replace the reference's four TVM-FFI typed exports
 *   deformable_aggregation_forward_opt   /root/reference/csrc/deformable_aggregation/deformable_aggregation_musa.mu:717-720,748
 *   deformable_aggregation_forward_base  .../deformable_aggregation_musa.mu:721-724,749
 *   deformable_aggregation_backward_opt  .../deformable_aggregation_musa.mu:725-735,750
 *   deformable_aggregation_backward_base .../deformable_aggregation_musa.mu:736-746,751
 * with the same argument order, followed by the dimensions the reference
 * reads from the tensors (deformable_aggregation_musa.mu:660-668) and the
 * stream.
 *
 * Tensors (device pointers, dense, row-major, float32 unless noted):
 *   mc_ms_feat          [batch, num_feat, num_embeds]
 *   spatial_shape       [num_cams, num_scale, 2] int32 (H, W), device-resident
 *   scale_start_index   [num_cams, num_scale] int32, device-resident
 *   sampling_location   [batch, num_anchors, num_pts, num_cams, 2] (x along W, y along H)
 *   weights             [batch, num_anchors, num_pts, num_cams, num_scale, num_groups]
 *   output / grad_output [batch, num_anchors, num_embeds]
 *   grad_mc_ms_feat, grad_sampling_location, grad_weights: like their inputs
 *
 * output[b, a, c] += sum over (pt, cam) with 0 < x < 1 and 0 < y < 1 (other
 * points, NaN included, are skipped) and over scales s of
 *   weights[b, a, pt, cam, s, c / (num_embeds / num_groups)]
 *   * bilinear(map (b, cam, s), h = y*H - 0.5, w = x*W - 0.5)[c],
 * corners outside [0, H-1] x [0, W-1] dropped.
 *
 * Conventions (those of the reference kernels):
 *  - The forward ADDS into output and the backward ADDS into grad_mc_ms_feat;
 *    the caller zero-fills them (the reference's autograd function does).
 *    grad_sampling_location and grad_weights are written for every point (zero
 *    for a skipped point), so they need no zero-fill.
 *  - 1 <= num_groups <= 8 and num_embeds % num_groups == 0 (the reference's
 *    operator checks, mu_space/ops/deformable_aggregation.py:66-70);
 *    num_cams * num_scale <= 256.
 *  - A (camera, scale) map whose start + H*W would pass num_feat contributes
 *    zero instead of being read out of bounds.
 *  - Launches are ordered on `stream`; nothing synchronises. Return 0 or a
 *    MUSPACE_E* code with muspace_last_error() set (muspace_msda.h).
 *  - _opt runs one wavefront per (batch, anchor) when num_embeds is a
 *    multiple of 64 up to 256 with power-of-two group widths, else the generic
 *    kernels; _base always runs the generic kernels (one thread per output
 *    element forward, per (batch, anchor, pt, cam) backward).
 *  - backward_opt (row-kernel layout, num_anchors * num_pts <= 2^20, 16-byte
 *    aligned grad_output, 8-byte aligned sampling_location) first sums the
 *    feature gradients of each camera's smallest maps in LDS as 64-bit
 *    fixed-point integers scaled from a bound on the contributions, then adds
 *    them once per cell; those sums are deterministic. A non-finite
 *    grad_output or weight sends the affected workgroup to fp32 atomics.
 */
#ifndef MUSPACE_DFA_H_
#define MUSPACE_DFA_H_

#include <stdint.h>

#include "muspace_msda.h"

#ifdef __cplusplus
extern "C" {
#endif

MUSPACE_API int deformable_aggregation_forward_opt(
    const float *mc_ms_feat, const int32_t *spatial_shape, const int32_t *scale_start_index,
    const float *sampling_location, const float *weights, float *output, int64_t batch,
    int64_t num_cams, int64_t num_feat, int64_t num_embeds, int64_t num_scale,
    int64_t num_anchors, int64_t num_pts, int64_t num_groups, void *stream);

MUSPACE_API int deformable_aggregation_forward_base(
    const float *mc_ms_feat, const int32_t *spatial_shape, const int32_t *scale_start_index,
    const float *sampling_location, const float *weights, float *output, int64_t batch,
    int64_t num_cams, int64_t num_feat, int64_t num_embeds, int64_t num_scale,
    int64_t num_anchors, int64_t num_pts, int64_t num_groups, void *stream);

MUSPACE_API int deformable_aggregation_backward_opt(
    const float *mc_ms_feat, const int32_t *spatial_shape, const int32_t *scale_start_index,
    const float *sampling_location, const float *weights, const float *grad_output,
    float *grad_mc_ms_feat, float *grad_sampling_location, float *grad_weights, int64_t batch,
    int64_t num_cams, int64_t num_feat, int64_t num_embeds, int64_t num_scale,
    int64_t num_anchors, int64_t num_pts, int64_t num_groups, void *stream);

MUSPACE_API int deformable_aggregation_backward_base(
    const float *mc_ms_feat, const int32_t *spatial_shape, const int32_t *scale_start_index,
    const float *sampling_location, const float *weights, const float *grad_output,
    float *grad_mc_ms_feat, float *grad_sampling_location, float *grad_weights, int64_t batch,
    int64_t num_cams, int64_t num_feat, int64_t num_embeds, int64_t num_scale,
    int64_t num_anchors, int64_t num_pts, int64_t num_groups, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* MUSPACE_DFA_H_ */
