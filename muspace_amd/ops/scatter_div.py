"""BEVFormer spatial cross-attention with the scatter-average fused into MSDA.

The step after the MSDA path in BEVFormer's ``SpatialCrossAttention``: each
camera attends its rebatched BEV queries, and every BEV query's slot receives
the average over the cameras that see it. Unfused, that is one MSDA call over
``[bs*num_cams, max_len]`` rows, a ``[bs*num_cams, max_len, M*C]`` output,
then per camera ``slots[b, index] += queries[b, cam, :len(index)]`` and
``slots / count``. The reference sketches the fusion as the unexported
``ms_deformable_im2col_scatter_div_gpu_kernel_channels32_runtime``
(/root/reference/csrc/ms_deformable_attn/ms_deform_attn_musa_kernel.muh:419-486)
with its host wrapper ``ms_deformable_im2col_scatter_div_musa``
(/root/reference/csrc/ms_deformable_attn/ms_deform_attn_musa.mu:455-505): one
launch per camera adds ``MSDA(row) * (1 / count[bev])`` straight into
``slots[bev]``, so the per-camera output never reaches memory. This operator
keeps that arithmetic (each camera's sum is scaled by ``1/count`` and then
added) but runs all cameras in one launch (``ms_deform_attn_forward_scatter_div_cams``):
float32 slots take the cameras' adds as fp32 atomics, so one launch fills the
GPU where six per-camera launches each leave a tail; 16-bit slots keep one
ordered launch per camera. It also adds the backward the reference lacks: the
gradient of a camera's output row is ``grad_slots[b, bev] / count[b, bev]``
(``ms_deform_attn_scatter_div_grad``), after which the MSDA backward gives
the value, location and weight gradients.

HIP only: ROCm tensors and the native library are required, there is no CPU
path.
"""

from __future__ import annotations

from typing import Sequence

import torch

from ..runtime.kernel_dispatch import is_rocm_tensor
from .multi_scale_deformable_attn import (
    _native_extension,
    _native_geometry_dtype,
    _validate_inputs,
)


class _ScatterDivFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, value, spatial_shapes, level_start_index, sampling_locations,
                attention_weights, count, slots, *indexes):
        ext = _native_extension()
        if ext is None:
            raise RuntimeError("muSPACE HIP native library is unavailable")
        geometry = _native_geometry_dtype(value, sampling_locations, attention_weights)
        value_arg = value.contiguous()
        sampling_arg = sampling_locations.to(geometry).contiguous()
        attn_arg = attention_weights.to(geometry).contiguous()
        count_arg = count.to(geometry).contiguous()
        spatial_arg = spatial_shapes.contiguous()
        start_arg = level_start_index.contiguous()
        lens = [int(index.numel()) for index in indexes]
        index_arg = torch.cat([index.reshape(-1) for index in indexes])
        ext.ms_deform_attn_forward_scatter_div_cams(
            value_arg, spatial_arg, start_arg, sampling_arg, attn_arg, index_arg, lens, count_arg,
            slots,
        )
        ctx.mark_dirty(slots)
        ctx.lens = lens
        ctx.dtypes = (value.dtype, sampling_locations.dtype, attention_weights.dtype)
        ctx.save_for_backward(value_arg, spatial_arg, start_arg, sampling_arg, attn_arg, count_arg,
                              index_arg)
        return slots

    @staticmethod
    def backward(ctx, grad_slots):
        ext = _native_extension()
        if ext is None:
            raise RuntimeError("muSPACE HIP native library is unavailable")
        value, spatial_shapes, level_start_index, sampling, attention, count, index = (
            ctx.saved_tensors
        )
        rows, max_len = sampling.shape[0], sampling.shape[1]
        row = value.shape[2] * value.shape[3]
        grad = grad_slots.to(value.dtype).contiguous()
        # every row of every camera is written (zeros past each camera's valid rows)
        grad_rows = torch.empty((rows, max_len, row), dtype=value.dtype, device=value.device)
        ext.ms_deform_attn_scatter_div_grad(grad, index, ctx.lens, count, grad_rows)
        grad_value = torch.empty(value.shape, dtype=torch.float32, device=value.device)
        grad_sampling = torch.empty(sampling.shape, dtype=torch.float32, device=value.device)
        grad_attention = torch.empty(attention.shape, dtype=torch.float32, device=value.device)
        ext.ms_deform_attn_backward(value, spatial_shapes, level_start_index, sampling, attention,
                                    grad_rows, grad_value, grad_sampling, grad_attention,
                                    max(rows, 1))
        value_dtype, sampling_dtype, attention_dtype = ctx.dtypes
        return (
            grad_value.to(value_dtype),
            None,
            None,
            grad_sampling.to(sampling_dtype),
            grad_attention.to(attention_dtype),
            None,
            grad_slots,
            *([None] * len(ctx.lens)),
        )


def multi_scale_deformable_attn_scatter_div(
    value: torch.Tensor,
    spatial_shapes: torch.Tensor,
    level_start_index: torch.Tensor,
    sampling_locations: torch.Tensor,
    attention_weights: torch.Tensor,
    indexes: Sequence[torch.Tensor],
    count: torch.Tensor,
    slots: torch.Tensor | None = None,
) -> torch.Tensor:
    """Per-camera MSDA summed into BEV slots as ``slots[b, bev] += out / count[b, bev]``.

    Args:
        value: ``[bs*num_cams, nv, M, C]``; row ``b*num_cams + cam`` is camera
            ``cam`` of batch entry ``b`` (BEVFormer's key/value rebatch).
        spatial_shapes, level_start_index: int64 level metadata, as for
            :func:`multi_scale_deformable_attn`.
        sampling_locations: ``[bs*num_cams, max_len, M, L, P, 2]``.
        attention_weights: ``[bs*num_cams, max_len, M, L, P]``.
        indexes: ``num_cams`` int64 tensors; ``indexes[cam][r]`` is the BEV
            query of the camera's rebatched row ``r``. Entries of one camera must
            be distinct (BEVFormer takes them from ``nonzero``); entries outside
            ``[0, num_query)`` are skipped. ``len(indexes[cam]) <= max_len``;
            rows past it are padding and are not read.
        count: ``[bs, num_query]``, the number of cameras that see each query
            (BEVFormer clamps it to at least 1).
        slots: ``[bs, num_query, M*C]`` in the value dtype, added to in place;
            zeros when ``None``.

    Returns:
        ``slots`` (a new zero-initialised tensor when none was given).
    """
    _validate_inputs(value, spatial_shapes, level_start_index)
    if len(indexes) == 0:
        raise ValueError("indexes must hold one index tensor per camera")
    tensors = (value, spatial_shapes, level_start_index, sampling_locations, attention_weights,
               count, *indexes) + (() if slots is None else (slots,))
    if not all(is_rocm_tensor(t) for t in tensors):
        raise RuntimeError(
            "multi_scale_deformable_attn_scatter_div runs on ROCm tensors only "
            "(no CPU implementation)"
        )
    if any(index.dtype != torch.int64 or index.dim() != 1 for index in indexes):
        raise TypeError("indexes must be 1-D int64 tensors")
    num_cams = len(indexes)
    if value.dim() != 4 or value.shape[0] % num_cams != 0:
        raise RuntimeError(
            f"value must be [bs*num_cams, nv, M, C] with num_cams={num_cams}, "
            f"got {list(value.shape)}"
        )
    max_len = sampling_locations.shape[1]
    for cam, index in enumerate(indexes):
        if index.numel() > max_len:
            raise RuntimeError(
                f"indexes[{cam}] has {index.numel()} entries, more than max_len={max_len}"
            )
    if count.dim() != 2:
        raise RuntimeError("count must be [bs, num_query]")
    if slots is None:
        batch = value.shape[0] // num_cams
        slots = torch.zeros((batch, count.shape[1], value.shape[2] * value.shape[3]),
                            dtype=value.dtype, device=value.device)
    return _ScatterDivFunction.apply(value, spatial_shapes, level_start_index,
                                     sampling_locations, attention_weights, count, slots,
                                     *indexes)
