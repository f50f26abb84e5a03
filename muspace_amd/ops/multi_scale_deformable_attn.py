"""Canonical multi-scale deformable attention (MSDA) operator.

Public contract of /root/reference/mu_space/ops/multi_scale_deformable_attn.py:
  * ``multi_scale_deformable_attn(value, spatial_shapes, level_start_index,
    sampling_locations, attention_weights, *, im2col_step=64, backend="auto")``
    (reference :215-338), recording one dispatch report per call;
  * ``multi_scale_deformable_attn_pytorch`` -- the grid_sample formulation used
    by the ``reference`` backend and by CPU tensors (reference :26-58);
  * ``multi_scale_deformable_attn_pytorch_compat`` -- the 4-argument mmcv
    signature that derives ``level_start_index`` (reference :61-75);
  * ``explain_dispatch`` (reference :341-348).

On ROCm tensors the work runs in the hand-written gfx950 HIP kernels of
``libmuspace_msda.so``. Autograd contract of ``_NativeMSDAFunction``
(reference :101-190): gradients for value, sampling_locations and
attention_weights, ``None`` for the metadata and ``im2col_step``; returned
gradients take the dtypes of the inputs the function received.

Dtype policy of the native path (differs from the reference on purpose):
  * float16 and bfloat16 ``value`` are storage dtypes of the kernels; every
    sampling coordinate, bilinear weight and accumulator is float32 (the
    reference upcasts float16 to float32 in Python, :120-130);
  * float32 ``sampling_locations`` / ``attention_weights`` stay float32 next to
    a 16-bit ``value`` instead of being narrowed to it (:206-209): narrowing
    the sampling geometry to 8 mantissa bits moves samples by up to W/256
    pixels. 16-bit geometry of the value's own dtype is read as is.
The ``reference`` backend keeps the reference's behaviour exactly (geometry
cast to the value dtype before grid_sample).
"""

from __future__ import annotations

import os
import threading
import warnings
import weakref

import torch
import torch.nn.functional as F

from ..runtime.kernel_dispatch import (
    NATIVE_BACKEND,
    DispatchDecision,
    DispatchReport,
    explain_dispatch as _explain_dispatch,
    is_rocm_tensor,
    record_dispatch_report,
)
from ..runtime.native import NativeModuleUnavailable, native_error, native_module_proxy

OPERATOR_NAME = "multi_scale_deformable_attn"
_VALUE_DTYPES = (torch.float16, torch.bfloat16, torch.float32)


def _native_extension():
    try:
        return native_module_proxy()
    except NativeModuleUnavailable:
        return None


def multi_scale_deformable_attn_pytorch(
    value: torch.Tensor,
    value_spatial_shapes: torch.Tensor,
    sampling_locations: torch.Tensor,
    attention_weights: torch.Tensor,
) -> torch.Tensor:
    """MSDA as per-level ``F.grid_sample`` calls (bilinear, zeros, align_corners=False).

    Same formulation as the reference path (ops:26-58): value is split into
    levels in order (``level_start_index`` is implied), ``grid = 2*loc - 1``,
    each level is sampled for all heads at once as a ``[bs*M, C, H, W]`` image,
    and the ``L*P`` samples are weighted by ``attention_weights`` and summed.
    """
    bs, _, heads, channels = value.shape
    _, queries, _, levels, points, _ = sampling_locations.shape
    shapes = [(int(h), int(w)) for h, w in value_spatial_shapes.tolist()]
    grids = 2 * sampling_locations - 1
    per_level = []
    for level, (feat, (h, w)) in enumerate(zip(value.split([h * w for h, w in shapes], 1), shapes)):
        image = feat.flatten(2).transpose(1, 2).reshape(bs * heads, channels, h, w)
        grid = grids[:, :, :, level].transpose(1, 2).flatten(0, 1)
        per_level.append(
            F.grid_sample(image, grid, mode="bilinear", padding_mode="zeros", align_corners=False)
        )
    weights = attention_weights.transpose(1, 2).reshape(bs * heads, 1, queries, levels * points)
    sampled = torch.stack(per_level, dim=-2).flatten(-2)  # [bs*M, C, nq, L*P]
    out = (sampled * weights).sum(-1).view(bs, heads * channels, queries)
    return out.transpose(1, 2).contiguous()


def level_start_index_from_shapes(value_spatial_shapes: torch.Tensor) -> torch.Tensor:
    """``[0, cumsum(H*W)[:-1]]`` (reference ops:67-68, patcher runtime.py:389-395)."""
    sizes = value_spatial_shapes[:, 0] * value_spatial_shapes[:, 1]
    if sizes.numel() == 0:
        return sizes.new_empty(0)
    return torch.cat([sizes.new_zeros(1), sizes.cumsum(0)[:-1]])


def multi_scale_deformable_attn_pytorch_compat(
    value: torch.Tensor,
    value_spatial_shapes: torch.Tensor,
    sampling_locations: torch.Tensor,
    attention_weights: torch.Tensor,
) -> torch.Tensor:
    """mmcv's 4-argument helper signature, routed through the canonical op."""
    return multi_scale_deformable_attn(
        value,
        value_spatial_shapes,
        level_start_index_from_shapes(value_spatial_shapes),
        sampling_locations,
        attention_weights,
    )


def _requires_native_backend(
    value: torch.Tensor,
    spatial_shapes: torch.Tensor,
    level_start_index: torch.Tensor,
    sampling_locations: torch.Tensor,
    attention_weights: torch.Tensor,
) -> bool:
    return any(
        is_rocm_tensor(t)
        for t in (value, spatial_shapes, level_start_index, sampling_locations, attention_weights)
    )


def _native_geometry_dtype(value: torch.Tensor, *geometry: torch.Tensor) -> torch.dtype:
    if value.dtype != torch.float32 and all(t.dtype == value.dtype for t in geometry):
        return value.dtype
    return torch.float32


# Early binning: the tile-owned backward's binning reads only the geometry, so
# the forward does it. ms_deform_attn_forward_bin runs the forward and the
# binning as one call, in which the forward kernel itself stores the
# backward's records (the geometry is read once for both; a binning on a second
# stream beside the forward kernel could not overlap it, the forward's
# registers leaving no room on its SIMDs). The backward's buffers (its scratch
# and the three float32 gradients) then live from the forward to the
# backward; MUSPACE_EARLY_BINNING=0 turns this off, and a per-device byte
# budget bounds what all forwards awaiting their backward may hold
# (MUSPACE_EARLY_BINNING_BUDGET bytes, default 1/32 of the device's memory):
# a forward that would exceed it does not bin early. The softmax operator
# (msda_softmax.py) does the same through ms_deform_attn_forward_softmax_bin.
EARLY_BINNING_ENV = "MUSPACE_EARLY_BINNING"
EARLY_BINNING_BUDGET_ENV = "MUSPACE_EARLY_BINNING_BUDGET"


class BinningBudget:
    """Bytes held by early binning per device, against a limit.

    A forward reserves its buffers' bytes before allocating them and the
    reservation is returned when its scratch tensor is freed (after the
    backward consumed it, or when the graph is dropped without a backward).
    """

    def __init__(self, limit_of=None) -> None:
        self._held: dict[int, int] = {}
        self._limits: dict[int, int] = {}
        self._lock = threading.Lock()
        self._limit_of = limit_of or self._device_limit

    @staticmethod
    def _device_limit(index: int) -> int:
        raw = os.environ.get(EARLY_BINNING_BUDGET_ENV, "").strip()
        if raw:
            return int(raw)
        return torch.cuda.get_device_properties(index).total_memory // 32

    def held(self, index: int) -> int:
        with self._lock:
            return self._held.get(index, 0)

    def try_reserve(self, index: int, nbytes: int) -> bool:
        with self._lock:
            limit = self._limits.get(index)
            if limit is None:
                limit = self._limits[index] = self._limit_of(index)
            held = self._held.get(index, 0)
            if held + nbytes > limit:
                return False
            self._held[index] = held + nbytes
            return True

    def release(self, index: int, nbytes: int) -> None:
        with self._lock:
            self._held[index] = self._held.get(index, 0) - nbytes


binning_budget = BinningBudget()


def _device_index(device: torch.device) -> int:
    return device.index if device.index is not None else torch.cuda.current_device()


def _reserve_early_buffers(workspace_bytes: int, *like: torch.Tensor):
    """Reserve the budget for a workspace of `workspace_bytes` and float32
    gradients shaped like `like`; returns a release callback or None."""
    device = like[0].device
    nbytes = workspace_bytes + 4 * sum(t.numel() for t in like)
    index = _device_index(device)
    if not binning_budget.try_reserve(index, nbytes):
        return None
    return lambda: binning_budget.release(index, nbytes)


def _early_binning_enabled() -> bool:
    return os.environ.get(EARLY_BINNING_ENV, "1").strip().lower() not in {"0", "false", "no", "off"}


def _bins_early(*tensors: torch.Tensor) -> bool:
    """Whether a forward should start its backward's binning: a graph will be
    recorded (grad mode on, which Function.forward itself cannot see) and an
    input needs a gradient."""
    return (_early_binning_enabled() and torch.is_grad_enabled()
            and any(t.requires_grad for t in tensors))


def _binning_buffers(ext, value, sampling, attn):
    """The backward's workspace and float32 gradients, allocated in the
    forward for a binning there; None when the shape takes the atomic
    backward (nothing to bin) or the early-binning budget is spent."""
    nbytes = ext.backward_workspace_bytes(value, sampling)
    if nbytes <= 1:
        return None
    release = _reserve_early_buffers(nbytes, value, sampling, attn)
    if release is None:
        return None
    try:
        workspace = ext.backward_workspace(value, sampling)
    except BaseException:
        release()  # nothing was allocated: the reservation goes back now
        raise
    # from here on the workspace's finalizer returns the reservation, also
    # when an allocation below raises and drops the workspace
    weakref.finalize(workspace, release)
    device = value.device
    grads = (
        torch.empty(value.shape, dtype=torch.float32, device=device),
        torch.empty(sampling.shape, dtype=torch.float32, device=device),
        torch.empty(attn.shape, dtype=torch.float32, device=device),
    )
    return workspace, grads


class _NativeMSDAFunction(torch.autograd.Function):
    @staticmethod
    def forward(
        ctx,
        value: torch.Tensor,
        spatial_shapes: torch.Tensor,
        level_start_index: torch.Tensor,
        sampling_locations: torch.Tensor,
        attention_weights: torch.Tensor,
        im2col_step: int,
        early_binning: bool = False,
    ) -> torch.Tensor:
        ext = _native_extension()
        if ext is None:
            raise RuntimeError("muSPACE HIP native library is unavailable")
        ctx.im2col_step = im2col_step
        ctx.value_dtype = value.dtype
        ctx.sampling_dtype = sampling_locations.dtype
        ctx.attention_dtype = attention_weights.dtype
        geometry = _native_geometry_dtype(value, sampling_locations, attention_weights)
        value_arg = value.contiguous()
        sampling_arg = sampling_locations.to(geometry).contiguous()
        attn_arg = attention_weights.to(geometry).contiguous()
        spatial_arg = spatial_shapes.contiguous()
        start_arg = level_start_index.contiguous()
        output = value_arg.new_empty(
            (value_arg.size(0), sampling_arg.size(1), value_arg.size(2) * value_arg.size(3))
        )
        # every tensor is checked before anything is allocated or launched
        ext.check_forward(value_arg, spatial_arg, start_arg, sampling_arg, attn_arg, output)
        ctx.binned = None
        if early_binning and any(ctx.needs_input_grad[i] for i in (0, 3, 4)):
            ctx.binned = _binning_buffers(ext, value_arg, sampling_arg, attn_arg)
        if ctx.binned is not None:
            workspace, grads = ctx.binned
            ext.ms_deform_attn_forward_bin(value_arg, spatial_arg, start_arg, sampling_arg,
                                           attn_arg, output, *grads, im2col_step, workspace)
        else:
            ext.ms_deform_attn_forward(
                value_arg, spatial_arg, start_arg, sampling_arg, attn_arg, output, im2col_step
            )
        ctx.save_for_backward(value_arg, spatial_arg, start_arg, sampling_arg, attn_arg)
        return output

    @staticmethod
    def backward(ctx, grad_output: torch.Tensor) -> tuple[torch.Tensor | None, ...]:
        ext = _native_extension()
        if ext is None:
            raise RuntimeError("muSPACE HIP native library is unavailable")
        value, spatial_shapes, level_start_index, sampling_locations, attention_weights = (
            ctx.saved_tensors
        )
        grad = grad_output.to(value.dtype).contiguous()
        binned, ctx.binned = ctx.binned, None  # one backward per binning
        if binned is not None:
            # the binning ran in the forward's call, on the stream autograd
            # runs this backward on
            workspace, (grad_value, grad_sampling, grad_attention) = binned
            ext.ms_deform_attn_backward_rest(
                value, spatial_shapes, level_start_index, sampling_locations, attention_weights,
                grad, grad_value, grad_sampling, grad_attention, ctx.im2col_step, workspace,
            )
        else:
            # gradients are float32 whatever the storage dtype; the kernels write
            # every element of all three, so none needs zero-filling
            grad_value = torch.empty(value.shape, dtype=torch.float32, device=value.device)
            grad_sampling = torch.empty(
                sampling_locations.shape, dtype=torch.float32, device=value.device
            )
            grad_attention = torch.empty(
                attention_weights.shape, dtype=torch.float32, device=value.device
            )
            ext.ms_deform_attn_backward(
                value,
                spatial_shapes,
                level_start_index,
                sampling_locations,
                attention_weights,
                grad,
                grad_value,
                grad_sampling,
                grad_attention,
                ctx.im2col_step,
            )
        return (
            grad_value.to(dtype=ctx.value_dtype),
            None,
            None,
            grad_sampling.to(dtype=ctx.sampling_dtype),
            grad_attention.to(dtype=ctx.attention_dtype),
            None,
            None,
        )


def _validate_inputs(
    value: torch.Tensor,
    spatial_shapes: torch.Tensor,
    level_start_index: torch.Tensor,
) -> None:
    # messages and exception types of the reference (ops:200-205)
    if spatial_shapes.dtype != torch.int64:
        raise TypeError("spatial_shapes must be int64")
    if level_start_index.dtype != torch.int64:
        raise TypeError("level_start_index must be int64")
    if value.dtype not in _VALUE_DTYPES:
        raise TypeError("value must be float16, bfloat16 or float32")


def _reference_inputs(value, spatial_shapes, sampling_locations, attention_weights):
    """The reference's normalisation (ops:206-212): geometry in the value dtype."""
    return (
        value.contiguous(),
        spatial_shapes.contiguous(),
        sampling_locations.to(dtype=value.dtype).contiguous(),
        attention_weights.to(dtype=value.dtype).contiguous(),
    )


def _report(backend: str, selected: str, decision: DispatchDecision, native_available: bool,
            reason: str | None = None, **extra) -> None:
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


def multi_scale_deformable_attn(
    value: torch.Tensor,
    spatial_shapes: torch.Tensor,
    level_start_index: torch.Tensor,
    sampling_locations: torch.Tensor,
    attention_weights: torch.Tensor,
    *,
    im2col_step: int = 64,
    backend: str = "auto",
) -> torch.Tensor:
    """Multi-scale deformable attention, ``[bs, nq, M*C]`` in ``value.dtype``.

    ``backend``: ``"auto"`` (HIP kernels on ROCm tensors, the PyTorch path
    elsewhere), ``"hip"`` (alias ``"musa"``: native kernels or an error) or
    ``"reference"`` (the grid_sample path on any device).
    """
    _validate_inputs(value, spatial_shapes, level_start_index)
    native_available = _native_extension() is not None
    decision = _explain_dispatch(value, backend=backend, native_available=native_available)
    if decision.backend == "error":
        _report(backend, "error", decision, native_available)
        detail = native_error() if not native_available and is_rocm_tensor(value) else None
        raise RuntimeError(f"{decision.reason}: {detail}" if detail else decision.reason)
    if decision.backend == "reference" or not _requires_native_backend(
        value, spatial_shapes, level_start_index, sampling_locations, attention_weights
    ):
        reason = None if decision.backend == "reference" else "inputs do not require the native backend"
        _report(backend, "reference", decision, native_available, reason)
        return multi_scale_deformable_attn_pytorch(
            *_reference_inputs(value, spatial_shapes, sampling_locations, attention_weights)
        )
    if sampling_locations.size(1) == 0:
        # no queries: an empty output that still ties every input into the graph
        output = value.new_zeros((value.size(0), 0, value.size(2) * value.size(3)))
        _report(backend, NATIVE_BACKEND, decision, native_available)
        return (
            output
            + value.sum() * 0
            + sampling_locations.sum().to(value.dtype) * 0
            + attention_weights.sum().to(value.dtype) * 0
        )
    try:
        output = _NativeMSDAFunction.apply(
            value,
            spatial_shapes,
            level_start_index,
            sampling_locations,
            attention_weights,
            im2col_step,
            _bins_early(value, sampling_locations, attention_weights),
        )
    except RuntimeError as exc:
        if backend != "auto":
            _report(backend, "error", decision, native_available, str(exc))
            raise
        # reference recovery policy (ops:311-338): auto falls back, recorded
        _report(
            backend,
            "reference",
            decision,
            native_available,
            "native backend failed; falling back to PyTorch reference",
            native_fallback=True,
            fallback_reason=str(exc),
        )
        warnings.warn(
            f"muSPACE HIP MSDA failed ({exc}); falling back to the PyTorch reference",
            RuntimeWarning,
            stacklevel=2,
        )
        return multi_scale_deformable_attn_pytorch(
            *_reference_inputs(value, spatial_shapes, sampling_locations, attention_weights)
        )
    _report(backend, NATIVE_BACKEND, decision, native_available)
    return output


def explain_dispatch(value: torch.Tensor, *, backend: str = "auto") -> DispatchDecision:
    return _explain_dispatch(
        value, backend=backend, native_available=_native_extension() is not None
    )
