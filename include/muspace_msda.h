/*
 * C-ABI of the MI355X (gfx950) multi-scale deformable attention library
 * `libmuspace_msda.so`.
 *
 * These entry points replace the two TVM-FFI typed exports of the reference's
 * native MSDA library:
 *   ms_deform_attn_forward   /root/reference/csrc/ms_deformable_attn/ms_deform_attn_musa.mu:507-560,627
 *   ms_deform_attn_backward  /root/reference/csrc/ms_deformable_attn/ms_deform_attn_musa.mu:561-626,628
 * and the build smoke export
 *   add_one                  /root/reference/csrc/ffi/muspace_ops.mu:40-55
 * The reference's Python loader (/root/reference/mu_space/runtime/native.py:20-77)
 * resolves those names through TVM-FFI; here they are plain C symbols resolved
 * through ctypes (muspace_amd/runtime/native.py).
 *
 * Conventions (same ownership and stream rules as the reference boundary):
 *  - Every pointer is a device pointer. The caller allocates every input and
 *    output; the library keeps no state. ms_deform_attn_backward takes
 *    stream-ordered scratch (hipMallocAsync / hipFreeAsync on `stream`);
 *    ms_deform_attn_backward_ws takes it from the caller instead.
 *  - All tensors are dense and row-major ("contiguous"):
 *      value               [batch, spatial_size, num_heads, channels]      value_dtype
 *      spatial_shapes      [num_levels, 2] int64 (H, W), device-resident
 *      level_start_index   [num_levels] int64, device-resident
 *      sampling_locations  [batch, num_query, num_heads, num_levels, num_point, 2]  geometry_dtype
 *                          ([..., 0] = x along W, [..., 1] = y along H, normalised to [0, 1])
 *      attention_weights   [batch, num_query, num_heads, num_levels, num_point]     geometry_dtype
 *      output              [batch, num_query, num_heads * channels]        value_dtype
 *      grad_output         like output                                     value_dtype
 *      grad_value          like value, float32, fully OVERWRITTEN (cells outside every
 *                          level get zero)
 *      grad_sampling_locations  like sampling_locations, float32, fully OVERWRITTEN
 *      grad_attention_weights   like attention_weights, float32, fully OVERWRITTEN
 *  - geometry_dtype is MUSPACE_DTYPE_F32 or equal to value_dtype.
 *  - Launches are ordered on `stream` (a hipStream_t; NULL = the null stream).
 *    Nothing synchronises; asynchronous device faults are not reported here.
 *  - Return 0 on success. On failure return a non-zero MUSPACE_E* code and set
 *    a thread-local message readable through muspace_last_error(); no kernel
 *    was launched in that case.
 *  - `im2col_step` keeps the reference's validation: step = min(batch,
 *    im2col_step) must be > 0 and divide batch (ms_deform_attn_musa.mu:523-524).
 *    Batch chunking has no numeric effect, so the whole batch runs in one launch.
 *  - Sampling follows torch.nn.functional.grid_sample(mode="bilinear",
 *    padding_mode="zeros", align_corners=False) on grid = 2*loc - 1, which is
 *    the reference PyTorch path (/root/reference/mu_space/ops/multi_scale_deformable_attn.py:26-58).
 *  - Level metadata is read on the device. A level whose (start, H, W) would
 *    address outside [0, spatial_size) is treated as empty (contributes zero)
 *    instead of being read out of bounds.
 */
#ifndef MUSPACE_MSDA_H_
#define MUSPACE_MSDA_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MUSPACE_MSDA_ABI_VERSION 6

/* the library is built with -fvisibility=hidden; only these symbols export */
#if defined(__GNUC__)
#define MUSPACE_API __attribute__((visibility("default")))
#else
#define MUSPACE_API
#endif

/* dtype codes for value / output / grad_output and for the sampling geometry */
#define MUSPACE_DTYPE_F32 0
#define MUSPACE_DTYPE_F16 1
#define MUSPACE_DTYPE_BF16 2

/* return codes */
#define MUSPACE_OK 0
#define MUSPACE_EINVAL 1  /* bad argument: null pointer, negative size, dtype, im2col_step */
#define MUSPACE_ERANGE 2  /* shape too large for the kernels' 32-bit intra-batch indexing */
#define MUSPACE_ELAUNCH 3 /* the HIP runtime rejected a launch */
#define MUSPACE_ENOMEM 4  /* stream-ordered scratch could not be allocated */

/* Forward: output = MSDA(value, geometry). Replaces ms_deform_attn_forward
 * (/root/reference/csrc/ms_deformable_attn/ms_deform_attn_musa.mu:507-560). */
MUSPACE_API int ms_deform_attn_forward(const void *value, int value_dtype, const int64_t *spatial_shapes,
                           const int64_t *level_start_index, const void *sampling_locations,
                           const void *attention_weights, int geometry_dtype, void *output,
                           int64_t batch, int64_t spatial_size, int64_t num_heads,
                           int64_t channels, int64_t num_levels, int64_t num_query,
                           int64_t num_point, int64_t im2col_step, void *stream);

/* Backward: overwrites grad_value, grad_sampling_locations and
 * grad_attention_weights. Replaces ms_deform_attn_backward
 * (/root/reference/csrc/ms_deformable_attn/ms_deform_attn_musa.mu:561-626). */
MUSPACE_API int ms_deform_attn_backward(const void *value, int value_dtype, const int64_t *spatial_shapes,
                            const int64_t *level_start_index, const void *sampling_locations,
                            const void *attention_weights, int geometry_dtype,
                            const void *grad_output, float *grad_value,
                            float *grad_sampling_locations, float *grad_attention_weights,
                            int64_t batch, int64_t spatial_size, int64_t num_heads,
                            int64_t channels, int64_t num_levels, int64_t num_query,
                            int64_t num_point, int64_t im2col_step, void *stream);

/* ms_deform_attn_backward that allocates nothing: no hipMalloc, hipFree or
 * allocating library call, for callers that cannot allocate (code under HIP
 * graph capture, tight serving loops, harnesses that forbid it). No reference
 * counterpart. Same arguments and results as ms_deform_attn_backward. Its
 * scratch is one file-scope device array of MUSPACE_NOALLOC_SCRATCH_BYTES per
 * GPU, held until the process ends; the batch is processed in passes of as
 * many batch entries as fit it (each pass is exact: a batch entry's gradients
 * depend on that entry alone). A shape whose single batch entry needs more
 * scratch than that is rejected with MUSPACE_ERANGE before anything runs.
 * Every call on one GPU uses that GPU's array, so calls that overlap on one
 * GPU (concurrent streams, or threads without stream ordering) race; calls
 * ordered on one stream are safe. */
#define MUSPACE_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)
MUSPACE_API int ms_deform_attn_backward_noalloc(
    const void *value, int value_dtype, const int64_t *spatial_shapes,
    const int64_t *level_start_index, const void *sampling_locations,
    const void *attention_weights, int geometry_dtype, const void *grad_output,
    float *grad_value, float *grad_sampling_locations, float *grad_attention_weights,
    int64_t batch, int64_t spatial_size, int64_t num_heads, int64_t channels, int64_t num_levels,
    int64_t num_query, int64_t num_point, int64_t im2col_step, void *stream);

/* Scratch bytes ms_deform_attn_backward_ws needs for these dims (0: the shape
 * takes the atomic fallback and needs none). No reference counterpart: the
 * reference backward scatters with global atomics and needs no scratch. */
MUSPACE_API size_t ms_deform_attn_backward_workspace_size(int value_dtype, int64_t batch,
                                                          int64_t spatial_size, int64_t num_heads,
                                                          int64_t channels, int64_t num_levels,
                                                          int64_t num_query, int64_t num_point);

/* ms_deform_attn_backward with caller-provided scratch (256-byte aligned, at
 * least ms_deform_attn_backward_workspace_size bytes), so that it allocates
 * nothing. Same results; replaces ms_deform_attn_backward
 * (/root/reference/csrc/ms_deformable_attn/ms_deform_attn_musa.mu:561-626)
 * for callers that manage memory themselves (the Python operator does). */
MUSPACE_API int ms_deform_attn_backward_ws(
    const void *value, int value_dtype, const int64_t *spatial_shapes,
    const int64_t *level_start_index, const void *sampling_locations,
    const void *attention_weights, int geometry_dtype, const void *grad_output,
    float *grad_value, float *grad_sampling_locations, float *grad_attention_weights,
    int64_t batch, int64_t spatial_size, int64_t num_heads, int64_t channels, int64_t num_levels,
    int64_t num_query, int64_t num_point, int64_t im2col_step, void *workspace,
    size_t workspace_bytes, void *stream);

/* ms_deform_attn_backward_ws in two calls on the same workspace and the same
 * arguments: _bin runs the binning of the tile-owned path (it reads only the
 * geometry -- sampling_locations, attention_weights and the level metadata --
 * and already writes parts of the three gradient buffers), _rest the rest
 * (it reads value and grad_output). _bin may therefore be issued before
 * grad_output exists, e.g. on a second stream during the forward; the caller
 * orders _rest after it (same stream or an event), keeps the workspace and the
 * gradient buffers alive in between and passes identical arguments to both,
 * except that grad_output may be NULL in _bin. Each _bin serves one _rest
 * (the rest consumes the binned work list). Shapes the tile path does not
 * take do nothing in _bin and everything in _rest. No reference counterpart
 * (the reference backward is one launch). */
MUSPACE_API int ms_deform_attn_backward_bin(
    const void *value, int value_dtype, const int64_t *spatial_shapes,
    const int64_t *level_start_index, const void *sampling_locations,
    const void *attention_weights, int geometry_dtype, const void *grad_output,
    float *grad_value, float *grad_sampling_locations, float *grad_attention_weights,
    int64_t batch, int64_t spatial_size, int64_t num_heads, int64_t channels, int64_t num_levels,
    int64_t num_query, int64_t num_point, int64_t im2col_step, void *workspace,
    size_t workspace_bytes, void *stream);
MUSPACE_API int ms_deform_attn_backward_rest(
    const void *value, int value_dtype, const int64_t *spatial_shapes,
    const int64_t *level_start_index, const void *sampling_locations,
    const void *attention_weights, int geometry_dtype, const void *grad_output,
    float *grad_value, float *grad_sampling_locations, float *grad_attention_weights,
    int64_t batch, int64_t spatial_size, int64_t num_heads, int64_t channels, int64_t num_levels,
    int64_t num_query, int64_t num_point, int64_t im2col_step, void *workspace,
    size_t workspace_bytes, void *stream);

/* ms_deform_attn_forward followed by ms_deform_attn_backward_bin on the same
 * arguments, workspace and stream, in one call: the forward's output plus the
 * binned workspace (and the parts of the three gradient buffers the binning
 * writes) that ms_deform_attn_backward_rest then consumes. Where the tile
 * path applies, the forward kernel itself stores the backward's records
 * (bin_count and bin_scan run first, over the forward blocks' query chunks),
 * so the geometry is read once for both and nothing runs beside the forward;
 * elsewhere it makes exactly those two calls. Same results as the two calls.
 * No reference counterpart: the reference forward
 * (/root/reference/csrc/ms_deformable_attn/ms_deform_attn_musa.mu:507-560)
 * prepares nothing for its backward. */
MUSPACE_API int ms_deform_attn_forward_bin(
    const void *value, int value_dtype, const int64_t *spatial_shapes,
    const int64_t *level_start_index, const void *sampling_locations,
    const void *attention_weights, int geometry_dtype, void *output, float *grad_value,
    float *grad_sampling_locations, float *grad_attention_weights, int64_t batch,
    int64_t spatial_size, int64_t num_heads, int64_t channels, int64_t num_levels,
    int64_t num_query, int64_t num_point, int64_t im2col_step, void *workspace,
    size_t workspace_bytes, void *stream);

/* 1 if ms_deform_attn_forward_bin, given 16-byte-aligned tensors and a
 * 256-byte-aligned workspace of ms_deform_attn_backward_workspace_size bytes,
 * stores the backward's records from the forward kernel for these dims; 0 if
 * it runs ms_deform_attn_forward and the binning kernels instead (or the
 * shape takes the atomic backward). Results are the same either way. No
 * reference counterpart. */
MUSPACE_API int ms_deform_attn_forward_bin_fused(int value_dtype, int64_t batch,
                                                 int64_t spatial_size, int64_t num_heads,
                                                 int64_t channels, int64_t num_levels,
                                                 int64_t num_query, int64_t num_point);

/* BEVFormer spatial cross-attention, one camera, with the scatter-average
 * fused into the forward: for the camera-rebatched
 *   value               [batch*num_cams, spatial_size, num_heads, channels]  value_dtype
 *   sampling_locations  [batch*num_cams, max_len, num_heads, num_levels, num_point, 2]
 *   attention_weights   [batch*num_cams, max_len, num_heads, num_levels, num_point]
 * (row b*num_cams + cam_id holds camera cam_id of batch b; geometry_dtype), the
 * BEV query of each of the camera's rows
 *   index               [valid_len] int64 (distinct; entries outside
 *                       [0, num_query) are skipped)
 * and the per-query camera count
 *   count               [batch, num_query] geometry_dtype (>= 1)
 * it adds, for every b, r < valid_len, head m and channel c,
 *   slots[b, index[r], m*channels + c] += MSDA(b*num_cams + cam_id, r, m, c) / count[b, index[r]]
 * to slots [batch, num_query, num_heads*channels] value_dtype, in place.
 * Rows r >= valid_len (the rebatch padding) are not read. Calls for different
 * cameras of the same slots must be ordered (same stream): a camera's rows
 * are added without atomics. Replaces the reference's unexported
 * ms_deformable_im2col_scatter_div_musa
 * (/root/reference/csrc/ms_deformable_attn/ms_deform_attn_musa.mu:455-505, kernel
 * ms_deform_attn_musa_kernel.muh:419-486), same arguments and order plus the
 * dtype codes; any channel count (the reference's supports 32 only). */
MUSPACE_API int ms_deform_attn_forward_scatter_div(
    const void *value, int value_dtype, const int64_t *spatial_shapes,
    const int64_t *level_start_index, const void *sampling_locations,
    const void *attention_weights, int geometry_dtype, const int64_t *index, const void *count,
    void *slots, int64_t batch, int64_t num_cams, int64_t cam_id, int64_t valid_len,
    int64_t spatial_size, int64_t num_heads, int64_t channels, int64_t num_levels,
    int64_t max_len, int64_t num_point, int64_t num_query, void *stream);

/* All cameras of ms_deform_attn_forward_scatter_div in one call: the same sum
 * for cameras 0 .. num_cams-1, where camera c's valid_lens[c] rows take their
 * BEV queries from the concatenated
 *   index               [sum(valid_lens)] int64 (camera 0's entries, then
 *                       camera 1's, ...; distinct within a camera)
 * and valid_lens is a HOST array [num_cams]. float32 slots: up to 16 cameras
 * per launch, added with fp32 global atomics (the order in which two cameras
 * reach one slot is not fixed; from zero-initialised slots a sum of two is
 * exact either way). 16-bit slots: one launch per camera, in order. No
 * reference counterpart (the reference's sketch launches per camera); same
 * result as calling ms_deform_attn_forward_scatter_div for each camera in
 * order. */
MUSPACE_API int ms_deform_attn_forward_scatter_div_cams(
    const void *value, int value_dtype, const int64_t *spatial_shapes,
    const int64_t *level_start_index, const void *sampling_locations,
    const void *attention_weights, int geometry_dtype, const int64_t *index,
    const int64_t *valid_lens, const void *count, void *slots, int64_t batch, int64_t num_cams,
    int64_t spatial_size, int64_t num_heads, int64_t channels, int64_t num_levels,
    int64_t max_len, int64_t num_point, int64_t num_query, void *stream);

/* Gradient of the cameras' MSDA output rows under the scatter-average:
 * grad_output[b*num_cams + c, r, :] = grad_slots[b, q, :] / count[b, q] with
 * q = the BEV query of camera c's row r (concatenated index and host
 * valid_lens as in ms_deform_attn_forward_scatter_div_cams) for
 * r < valid_lens[c], zero for valid_lens[c] <= r < max_len and for skipped
 * indices. grad_slots [batch, num_query, row] and grad_output
 * [batch*num_cams, max_len, row] are value_dtype; count is float32 or
 * value_dtype. ms_deform_attn_backward on grad_output then gives the value,
 * location and weight gradients. No reference counterpart (the reference's
 * fused path is forward-only); it is the chain rule of the same sum. */
MUSPACE_API int ms_deform_attn_scatter_div_grad(const void *grad_slots, int value_dtype,
                                                const int64_t *index, const int64_t *valid_lens,
                                                const void *count, int count_dtype,
                                                void *grad_output, int64_t batch,
                                                int64_t num_cams, int64_t max_len,
                                                int64_t num_query, int64_t row, void *stream);

/* Softmax over L*P fused into the operator (producer side of the path:
 * BEVFormer's MSDeformableAttention3D and friends apply
 *   attention_weights = logits.view(bs, nq, M, L*P).softmax(-1)
 * before calling the reference's ms_deform_attn_forward; no reference
 * counterpart). `attention_logits` has the shape and dtype of
 * attention_weights; each (b, q, m) unit's L*P weights are the softmax of its
 * logits (an all -inf unit gives NaN, as torch.softmax does). Otherwise the
 * contract of ms_deform_attn_forward. The row kernels fuse the softmax into
 * their prologue; other shapes run a standalone softmax into stream-ordered
 * scratch (MUSPACE_ENOMEM if it cannot be allocated). */
MUSPACE_API int ms_deform_attn_forward_softmax(
    const void *value, int value_dtype, const int64_t *spatial_shapes,
    const int64_t *level_start_index, const void *sampling_locations,
    const void *attention_logits, int geometry_dtype, void *output, int64_t batch,
    int64_t spatial_size, int64_t num_heads, int64_t channels, int64_t num_levels,
    int64_t num_query, int64_t num_point, int64_t im2col_step, void *stream);

/* Scratch bytes of the softmax backward (the probabilities, then the
 * binning scratch of ms_deform_attn_backward_workspace_size when the tile path
 * applies); 0 when nothing is sampled or the dims are invalid. */
MUSPACE_API size_t ms_deform_attn_backward_softmax_workspace_size(
    int value_dtype, int geometry_dtype, int64_t batch, int64_t spatial_size, int64_t num_heads,
    int64_t channels, int64_t num_levels, int64_t num_query, int64_t num_point);

/* Backward of ms_deform_attn_forward_softmax in two calls on one workspace
 * (256-byte aligned, at least the size above; MUSPACE_EINVAL otherwise), as
 * ms_deform_attn_backward_bin / _rest: _bin reads the geometry and logits only
 * (grad_output may be NULL) and writes the probabilities and the binning into
 * the workspace; _rest writes grad_value, grad_sampling_locations and
 * grad_attention_logits = p * (g - sum_j p_j g_j) per unit, g being the
 * gradient of the softmax weights. */
MUSPACE_API int ms_deform_attn_backward_softmax_bin(
    const void *value, int value_dtype, const int64_t *spatial_shapes,
    const int64_t *level_start_index, const void *sampling_locations,
    const void *attention_logits, int geometry_dtype, const void *grad_output, float *grad_value,
    float *grad_sampling_locations, float *grad_attention_logits, int64_t batch,
    int64_t spatial_size, int64_t num_heads, int64_t channels, int64_t num_levels,
    int64_t num_query, int64_t num_point, int64_t im2col_step, void *workspace,
    size_t workspace_bytes, void *stream);

MUSPACE_API int ms_deform_attn_backward_softmax_rest(
    const void *value, int value_dtype, const int64_t *spatial_shapes,
    const int64_t *level_start_index, const void *sampling_locations,
    const void *attention_logits, int geometry_dtype, const void *grad_output, float *grad_value,
    float *grad_sampling_locations, float *grad_attention_logits, int64_t batch,
    int64_t spatial_size, int64_t num_heads, int64_t channels, int64_t num_levels,
    int64_t num_query, int64_t num_point, int64_t im2col_step, void *workspace,
    size_t workspace_bytes, void *stream);

/* ms_deform_attn_forward_softmax followed by ms_deform_attn_backward_softmax_bin
 * on the same arguments, workspace (as sized above) and stream, in one call:
 * the output plus the probabilities and the binned workspace that
 * ms_deform_attn_backward_softmax_rest then consumes. Where the tile path
 * applies and each unit's L*P logits fit one step of the forward row kernel,
 * the softmax-fused forward kernel itself writes the probabilities and stores
 * the backward's records (weighted by the probabilities), as
 * ms_deform_attn_forward_bin does; elsewhere it makes exactly those two calls.
 * Same contract as the two calls. No reference counterpart (the reference's
 * callers apply the softmax in torch before its forward). */
MUSPACE_API int ms_deform_attn_forward_softmax_bin(
    const void *value, int value_dtype, const int64_t *spatial_shapes,
    const int64_t *level_start_index, const void *sampling_locations,
    const void *attention_logits, int geometry_dtype, void *output, float *grad_value,
    float *grad_sampling_locations, float *grad_attention_logits, int64_t batch,
    int64_t spatial_size, int64_t num_heads, int64_t channels, int64_t num_levels,
    int64_t num_query, int64_t num_point, int64_t im2col_step, void *workspace,
    size_t workspace_bytes, void *stream);

/* 1 if ms_deform_attn_forward_softmax_bin (aligned tensors, a workspace as
 * above) fuses the probabilities and the record stores into the forward kernel
 * for these dims; 0 if it makes the two calls. No reference counterpart. */
MUSPACE_API int ms_deform_attn_forward_softmax_bin_fused(int value_dtype, int64_t batch,
                                                         int64_t spatial_size,
                                                         int64_t num_heads, int64_t channels,
                                                         int64_t num_levels, int64_t num_query,
                                                         int64_t num_point);

/* Both parts in one call with stream-ordered scratch (MUSPACE_ENOMEM if it
 * cannot be allocated). */
MUSPACE_API int ms_deform_attn_backward_softmax(
    const void *value, int value_dtype, const int64_t *spatial_shapes,
    const int64_t *level_start_index, const void *sampling_locations,
    const void *attention_logits, int geometry_dtype, const void *grad_output, float *grad_value,
    float *grad_sampling_locations, float *grad_attention_logits, int64_t batch,
    int64_t spatial_size, int64_t num_heads, int64_t channels, int64_t num_levels,
    int64_t num_query, int64_t num_point, int64_t im2col_step, void *stream);

/* Build smoke: y[i] = x[i] + 1 for i < n (float32). Mirrors add_one
 * (/root/reference/csrc/ffi/muspace_ops.mu:40-55). */
MUSPACE_API int add_one(const float *x, float *y, int64_t n, void *stream);

/* Message of the last failed call on this thread ("" if none). Replaces the
 * TVM_FFI_ICHECK exception text of the reference boundary
 * (/root/reference/csrc/ffi/tensor_utils.hpp:13-38). */
MUSPACE_API const char *muspace_last_error(void);

/* MUSPACE_MSDA_ABI_VERSION of the loaded library. No reference counterpart:
 * lets the Python loader refuse a stale library. */
MUSPACE_API int muspace_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* MUSPACE_MSDA_H_ */
