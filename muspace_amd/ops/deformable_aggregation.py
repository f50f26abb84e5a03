"""Deformable aggregation: SparseDrive's multi-camera, multi-scale feature aggregation.

Mirrors the reference operator module
(/root/reference/mu_space/ops/deformable_aggregation.py:1-433): the canonical
``deformable_aggregation`` with backends ``auto`` / ``hip`` (alias ``musa``) /
``reference``, the SparseDrive-compatible ``deformable_aggregation_function``,
the PyTorch ``deformable_aggregation_reference`` and the ``feature_maps_format``
helper. The native backend calls the HIP kernels of ``libmuspace_msda.so``
(``deformable_aggregation_{forward,backward}_opt``, include/muspace_dfa.h).

Semantics (reference ops:88-158 and the kernels it mirrors): for every
(batch b, anchor a), over sample points p and cameras c whose normalised
location (x, y) lies strictly inside (0, 1) -- other points are skipped -- and
over scales s,
    out[b, a, ch] += weights[b, a, p, c, s, ch // (C/groups)]
                     * bilinear(map(b, c, s), y*H - 0.5, x*W - 0.5)[ch]
with bilinear corners outside the map dropped.
"""

from __future__ import annotations

import torch

from ..runtime.kernel_dispatch import (
    NATIVE_BACKEND,
    DispatchDecision,
    DispatchReport,
    explain_dispatch as _explain_dispatch,
    is_rocm_tensor,
    record_dispatch_report,
)
from ..runtime.native import NativeModuleUnavailable, native_error, native_module_proxy

OPERATOR_NAME = "deformable_aggregation"
MAX_GROUPS = 8


def _native_extension():
    try:
        return native_module_proxy()
    except NativeModuleUnavailable:
        return None


def _normalize_inputs(mc_ms_feat, spatial_shape, scale_start_index, sampling_location, weights):
    """Dtype and rank checks with the reference's messages (ops:34-78)."""
    if mc_ms_feat.dtype != torch.float32:
        raise TypeError("mc_ms_feat must use float32")
    if sampling_location.dtype != torch.float32:
        raise TypeError("sampling_location must use float32")
    if weights.dtype != torch.float32:
        raise TypeError("weights must use float32")
    if spatial_shape.dtype != torch.int32:
        raise TypeError("spatial_shape must use int32")
    if scale_start_index.dtype != torch.int32:
        raise TypeError("scale_start_index must use int32")
    if mc_ms_feat.dim() != 3:
        raise ValueError("mc_ms_feat must have shape [B, num_feat, C]")
    if spatial_shape.dim() != 3 or spatial_shape.size(-1) != 2:
        raise ValueError("spatial_shape must have shape [num_cams, num_scale, 2]")
    if scale_start_index.dim() != 2:
        raise ValueError("scale_start_index must have shape [num_cams, num_scale]")
    if sampling_location.dim() != 5 or sampling_location.size(-1) != 2:
        raise ValueError("sampling_location must have shape [B, anchors, pts, cams, 2]")
    if weights.dim() != 6:
        raise ValueError("weights must have shape [B, anchors, pts, cams, scale, groups]")
    num_groups = weights.size(-1)
    if num_groups <= 0 or num_groups > MAX_GROUPS:
        raise ValueError(f"num_groups must be in [1, {MAX_GROUPS}]")
    if mc_ms_feat.size(-1) % num_groups != 0:
        raise ValueError("num_embeds must be divisible by num_groups")
    return (
        mc_ms_feat.contiguous(),
        spatial_shape.contiguous(),
        scale_start_index.contiguous(),
        sampling_location.contiguous(),
        weights.contiguous(),
    )


def deformable_aggregation_reference(
    mc_ms_feat: torch.Tensor,
    spatial_shape: torch.Tensor,
    scale_start_index: torch.Tensor,
    sampling_location: torch.Tensor,
    weights: torch.Tensor,
) -> torch.Tensor:
    """PyTorch formulation of the same sum, differentiable, on any device.

    Same arithmetic as the reference's per-sample loop (ops:88-158), batched:
    one gather per (camera, scale) and corner over all (batch, anchor, point).
    """
    batch, _, channels = mc_ms_feat.shape
    anchors, pts = sampling_location.shape[1], sampling_location.shape[2]
    groups = weights.shape[-1]
    x = sampling_location[..., 0]  # [B, A, P, cams]
    y = sampling_location[..., 1]
    active = (x > 0) & (x < 1) & (y > 0) & (y < 1)
    out = mc_ms_feat.new_zeros((batch, anchors, channels))
    for cam, (cam_shapes, cam_starts) in enumerate(
        zip(spatial_shape.tolist(), scale_start_index.tolist())
    ):
        for scale, ((height, width), start) in enumerate(zip(cam_shapes, cam_starts)):
            fmap = mc_ms_feat[:, start: start + height * width]  # [B, H*W, C]
            h_im = y[..., cam] * height - 0.5
            w_im = x[..., cam] * width - 0.5
            h0, w0 = torch.floor(h_im), torch.floor(w_im)
            lh, lw = h_im - h0, w_im - w0
            hh, hw = 1.0 - lh, 1.0 - lw
            sampled = mc_ms_feat.new_zeros((batch, anchors, pts, channels))
            for dh, dw, wgt in ((0, 0, hh * hw), (0, 1, hh * lw), (1, 0, lh * hw),
                                (1, 1, lh * lw)):
                hc, wc = h0 + dh, w0 + dw
                keep = (hc >= 0) & (hc <= height - 1) & (wc >= 0) & (wc <= width - 1)
                keep = keep & active[..., cam]
                cell = (hc.clamp(0, height - 1) * width + wc.clamp(0, width - 1)).long()
                rows = torch.gather(
                    fmap, 1, cell.reshape(batch, anchors * pts, 1).expand(-1, -1, channels)
                ).view(batch, anchors, pts, channels)
                sampled = sampled + torch.where(keep, wgt, torch.zeros_like(wgt))[..., None] * rows
            group_w = weights[:, :, :, cam, scale, :].repeat_interleave(channels // groups, dim=-1)
            out = out + (sampled * group_w).sum(dim=2)
    return out


class _NativeDeformableAggregationFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, mc_ms_feat, spatial_shape, scale_start_index, sampling_location, weights):
        ext = _native_extension()
        if ext is None:
            raise RuntimeError("muSPACE HIP native library is unavailable")
        # the kernels add into the output (reference accumulate semantics)
        output = mc_ms_feat.new_zeros(
            (mc_ms_feat.size(0), sampling_location.size(1), mc_ms_feat.size(2))
        )
        ext.deformable_aggregation_forward_opt(
            mc_ms_feat, spatial_shape, scale_start_index, sampling_location, weights, output
        )
        ctx.save_for_backward(mc_ms_feat, spatial_shape, scale_start_index, sampling_location,
                              weights)
        return output

    @staticmethod
    def backward(ctx, grad_output):
        ext = _native_extension()
        if ext is None:
            raise RuntimeError("muSPACE HIP native library is unavailable")
        mc_ms_feat, spatial_shape, scale_start_index, sampling_location, weights = (
            ctx.saved_tensors
        )
        # feature gradients accumulate (atomics); the other two are written in full
        grad_mc_ms_feat = torch.zeros_like(mc_ms_feat)
        grad_sampling_location = torch.empty_like(sampling_location)
        grad_weights = torch.empty_like(weights)
        ext.deformable_aggregation_backward_opt(
            mc_ms_feat, spatial_shape, scale_start_index, sampling_location, weights,
            grad_output.float().contiguous(), grad_mc_ms_feat, grad_sampling_location,
            grad_weights,
        )
        return grad_mc_ms_feat, None, None, grad_sampling_location, grad_weights


def _report(backend, selected, decision, native_available, reason=None, **extra) -> None:
    record_dispatch_report(
        DispatchReport(
            operator=OPERATOR_NAME,
            requested_backend=backend,
            selected_backend=selected,
            device=decision.device,
            reason=decision.reason if reason is None else reason,
            native_available=native_available,
            **extra,
        )
    )


def deformable_aggregation(
    mc_ms_feat: torch.Tensor,
    spatial_shape: torch.Tensor,
    scale_start_index: torch.Tensor,
    sampling_location: torch.Tensor,
    weights: torch.Tensor,
    *,
    backend: str = "auto",
) -> torch.Tensor:
    """Aggregated features ``[B, anchors, C]`` (reference ops:259-373).

    ``backend``: ``"auto"`` (HIP kernels on ROCm tensors, the PyTorch
    formulation elsewhere), ``"hip"`` (alias ``"musa"``: native kernels or an
    error) or ``"reference"``.
    """
    tensors = _normalize_inputs(mc_ms_feat, spatial_shape, scale_start_index, sampling_location,
                                weights)
    mc_ms_feat, spatial_shape, scale_start_index, sampling_location, weights = tensors
    native_available = _native_extension() is not None
    decision = _explain_dispatch(mc_ms_feat, backend=backend, native_available=native_available)
    if decision.backend == "error":
        _report(backend, "error", decision, native_available)
        detail = native_error() if not native_available and is_rocm_tensor(mc_ms_feat) else None
        raise RuntimeError(f"{decision.reason}: {detail}" if detail else decision.reason)
    if decision.backend == "reference":
        _report(backend, "reference", decision, native_available)
        return deformable_aggregation_reference(*tensors)
    if sampling_location.size(1) == 0:
        # no anchors: an empty output that still ties every input into the graph
        _report(backend, NATIVE_BACKEND, decision, native_available)
        output = mc_ms_feat.new_zeros((mc_ms_feat.size(0), 0, mc_ms_feat.size(2)))
        return output + mc_ms_feat.sum() * 0 + sampling_location.sum() * 0 + weights.sum() * 0
    try:
        output = _NativeDeformableAggregationFunction.apply(*tensors)
    except RuntimeError as exc:
        if backend != "auto":
            _report(backend, "error", decision, native_available, str(exc))
            raise
        # reference recovery policy (ops:344-373): auto falls back, recorded
        fallback = DispatchDecision(
            "reference", decision.device,
            "native backend failed; falling back to PyTorch reference",
        )
        _report(backend, "reference", fallback, native_available, native_fallback=True,
                fallback_reason=str(exc))
        return deformable_aggregation_reference(*tensors)
    _report(backend, NATIVE_BACKEND, decision, native_available)
    return output


def deformable_aggregation_function(
    feature_maps: torch.Tensor,
    spatial_shape: torch.Tensor,
    scale_start_index: torch.Tensor,
    sampling_location: torch.Tensor,
    weights: torch.Tensor,
    *,
    backend: str = "auto",
) -> torch.Tensor:
    """SparseDrive-compatible alias (reference ops:376-393): casts to the
    operator's dtypes, then :func:`deformable_aggregation`."""
    return deformable_aggregation(
        feature_maps.contiguous().float(),
        spatial_shape.contiguous().to(dtype=torch.int32),
        scale_start_index.contiguous().to(dtype=torch.int32),
        sampling_location.contiguous().float(),
        weights.contiguous().float(),
        backend=backend,
    )


def feature_maps_format(feature_maps, inverse: bool = False):
    """Pack per-scale camera maps into the operator's layout, or unpack it.

    Forward: ``feature_maps`` is a list over scales of ``[bs, cams, C, H, W]``
    tensors (or a list of such lists, packed one after another). Returns
    ``[col_feats [bs, cams * sum(H*W), C], spatial_shape [cams, scales, 2],
    scale_start_index [cams, scales]]``: camera-major, scales in order inside a
    camera, each map row-major. A list of lists packs each inner list and
    concatenates the results; as in the reference, the start indices of later
    lists are not offset. ``inverse=True`` walks the packed features in that
    order and returns per-scale ``[bs, n, C, H, W]`` tensors, one list per run
    of consecutive cameras with identical shapes. SparseDrive's helper of the
    same name (reference ops:396-427) defines the layout.
    """
    if inverse:
        col_feats, spatial_shape, scale_start_index = feature_maps
        shapes = [[(int(h), int(w)) for h, w in cam] for cam in spatial_shape.tolist()]
        runs: list[list[int]] = []  # consecutive cameras with identical shapes
        for cam, cam_shapes in enumerate(shapes):
            if runs and shapes[runs[-1][0]] == cam_shapes:
                runs[-1].append(cam)
            else:
                runs.append([cam])
        bs, channels = col_feats.shape[0], col_feats.shape[-1]
        result, first = [], 0
        for run in runs:
            sizes = [h * w for h, w in shapes[run[0]]]
            span = len(run) * sum(sizes)
            block = col_feats[:, first: first + span].view(bs, len(run), sum(sizes), channels)
            first += span
            per_scale = []
            for part, (h, w) in zip(block.split(sizes, dim=2), shapes[run[0]]):
                per_scale.append(part.reshape(bs, len(run), h, w, channels).permute(0, 1, 4, 2, 3))
            result.append(per_scale)
        return result

    if isinstance(feature_maps[0], (list, tuple)):
        packed = [feature_maps_format(group) for group in feature_maps]
        col_feats = torch.cat([p[0] for p in packed], dim=1)
        spatial_shape = torch.cat([p[1] for p in packed], dim=0)
        scale_start_index = torch.cat([p[2] for p in packed], dim=0)
        return [col_feats, spatial_shape, scale_start_index]

    bs, cams, channels = feature_maps[0].shape[:3]
    sizes = [(int(f.shape[-2]), int(f.shape[-1])) for f in feature_maps]
    # [bs, cams, sum(H*W), C], camera-major then scale
    flat = torch.cat([f.flatten(3) for f in feature_maps], dim=-1).transpose(2, 3)
    col_feats = flat.reshape(bs, cams * flat.shape[2], channels)
    device = col_feats.device
    spatial_shape = torch.tensor([sizes] * cams, dtype=torch.int64, device=device)
    per_cam = sum(h * w for h, w in sizes)
    level_offsets = [0]
    for h, w in sizes[:-1]:
        level_offsets.append(level_offsets[-1] + h * w)
    scale_start_index = torch.tensor(
        [[cam * per_cam + off for off in level_offsets] for cam in range(cams)],
        dtype=torch.int64, device=device,
    )
    return [col_feats, spatial_shape, scale_start_index]


__all__ = [
    "deformable_aggregation",
    "deformable_aggregation_function",
    "deformable_aggregation_reference",
    "feature_maps_format",
]

