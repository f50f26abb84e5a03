"""MSDA with the attention softmax fused in: the producer side of the path.

BEVFormer-style modules turn their attention projection into weights with a
softmax over each query's L*P samples per head and then call the operator:

    weights = logits.view(bs, nq, M, L * P).softmax(-1).view(bs, nq, M, L, P)
    out = multi_scale_deformable_attn(value, shapes, starts, loc, weights)

(the composition the reference's own tests and model scripts use:
/root/reference/tests/ops/test_multi_scale_deformable_attn.py:62,
/root/reference/model_examples/BEVFormer/scripts/smoke_openmmlab.py:31-32).
``multi_scale_deformable_attn_softmax`` takes the logits instead. On ROCm
tensors the forward row kernels compute the softmax in their prologue, so the
weights are never read back from HBM. Its backward's last step turns the
weight gradient into the logit gradient, p * (g - sum_j p_j g_j). In training
(a graph is recorded and an input needs a gradient) the forward also bins for
the backward, as ``multi_scale_deformable_attn`` does: one call
(ms_deform_attn_forward_softmax_bin) in which, where each query's L*P logits
fit one step of the forward row kernel, the forward kernel writes every
sample's probability to the backward's scratch and stores its records weighted
by it; the backward then runs its second part only. Without a graph the
forward writes nothing but the output, and the backward (if any) recomputes
the probabilities. Gradients and dtypes follow ``multi_scale_deformable_attn``.
"""

from __future__ import annotations

import weakref

import torch

from ..runtime.kernel_dispatch import (
    NATIVE_BACKEND,
    DispatchReport,
    explain_dispatch as _explain_dispatch,
    is_rocm_tensor,
    record_dispatch_report,
)
from ..runtime.native import native_error
from .multi_scale_deformable_attn import (
    _bins_early,
    _native_extension,
    _reserve_early_buffers,
    _native_geometry_dtype,
    _validate_inputs,
    multi_scale_deformable_attn_pytorch,
)

OPERATOR_NAME = "multi_scale_deformable_attn_softmax"


def attention_softmax(attention_logits: torch.Tensor) -> torch.Tensor:
    """Softmax over each (b, q, m) unit's L*P logits, shape kept."""
    bs, nq, heads, levels, points = attention_logits.shape
    return attention_logits.reshape(bs, nq, heads, levels * points).softmax(-1).reshape(
        bs, nq, heads, levels, points
    )


def _binning_buffers(ext, value, sampling, logits):
    """Workspace (probabilities first, then the binning scratch) and float32
    gradients for a forward that bins for its backward; None when the
    early-binning budget is spent (the backward then runs in one call)."""
    release = _reserve_early_buffers(ext.backward_softmax_workspace_bytes(value, sampling),
                                     value, sampling, logits)
    if release is None:
        return None
    try:
        workspace = ext.backward_softmax_workspace(value, sampling)
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
        torch.empty(logits.shape, dtype=torch.float32, device=device),
    )
    return workspace, grads


class _NativeMSDASoftmaxFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, value, spatial_shapes, level_start_index, sampling_locations,
                attention_logits, im2col_step, early_binning=False):
        ext = _native_extension()
        if ext is None:
            raise RuntimeError("muSPACE HIP native library is unavailable")
        ctx.im2col_step = im2col_step
        ctx.value_dtype = value.dtype
        ctx.sampling_dtype = sampling_locations.dtype
        ctx.logits_dtype = attention_logits.dtype
        geometry = _native_geometry_dtype(value, sampling_locations, attention_logits)
        value_arg = value.contiguous()
        sampling_arg = sampling_locations.to(geometry).contiguous()
        logits_arg = attention_logits.to(geometry).contiguous()
        spatial_arg = spatial_shapes.contiguous()
        start_arg = level_start_index.contiguous()
        output = value_arg.new_empty(
            (value_arg.size(0), sampling_arg.size(1), value_arg.size(2) * value_arg.size(3))
        )
        # every tensor is checked before the first launch (the binning below
        # runs before the forward's own launch)
        ext.check_forward(value_arg, spatial_arg, start_arg, sampling_arg, logits_arg, output)
        ctx.binned = None
        if early_binning and any(ctx.needs_input_grad[i] for i in (0, 3, 4)):
            ctx.binned = _binning_buffers(ext, value_arg, sampling_arg, logits_arg)
        if ctx.binned is not None:
            # the forward and the backward's first part in one call: where the
            # shape allows, the softmax-fused forward kernel itself writes the
            # probabilities and stores the backward's records
            workspace, grads = ctx.binned
            ext.ms_deform_attn_forward_softmax_bin(value_arg, spatial_arg, start_arg,
                                                   sampling_arg, logits_arg, output, *grads,
                                                   im2col_step, workspace)
        else:
            ext.ms_deform_attn_forward_softmax(value_arg, spatial_arg, start_arg, sampling_arg,
                                               logits_arg, output, im2col_step)
        ctx.save_for_backward(value_arg, spatial_arg, start_arg, sampling_arg, logits_arg)
        return output

    @staticmethod
    def backward(ctx, grad_output):
        ext = _native_extension()
        if ext is None:
            raise RuntimeError("muSPACE HIP native library is unavailable")
        value, spatial_shapes, level_start_index, sampling_locations, logits = ctx.saved_tensors
        grad = grad_output.to(value.dtype).contiguous()
        binned, ctx.binned = ctx.binned, None  # one backward per binning
        if binned is not None:
            workspace, (grad_value, grad_sampling, grad_logits) = binned
            ext.ms_deform_attn_backward_softmax_rest(
                value, spatial_shapes, level_start_index, sampling_locations, logits, grad,
                grad_value, grad_sampling, grad_logits, ctx.im2col_step, workspace,
            )
        else:
            grad_value = torch.empty(value.shape, dtype=torch.float32, device=value.device)
            grad_sampling = torch.empty(sampling_locations.shape, dtype=torch.float32,
                                        device=value.device)
            grad_logits = torch.empty(logits.shape, dtype=torch.float32, device=value.device)
            ext.ms_deform_attn_backward_softmax(
                value, spatial_shapes, level_start_index, sampling_locations, logits, grad,
                grad_value, grad_sampling, grad_logits, ctx.im2col_step,
            )
        return (
            grad_value.to(dtype=ctx.value_dtype),
            None,
            None,
            grad_sampling.to(dtype=ctx.sampling_dtype),
            grad_logits.to(dtype=ctx.logits_dtype),
            None,
            None,
        )


def _report(backend, selected, decision, native_available, reason=None):
    record_dispatch_report(
        DispatchReport(
            operator=OPERATOR_NAME,
            requested_backend=backend,
            selected_backend=selected,
            device=decision.device,
            reason=decision.reason if reason is None else reason,
            native_available=native_available,
        )
    )


def multi_scale_deformable_attn_softmax(
    value: torch.Tensor,
    spatial_shapes: torch.Tensor,
    level_start_index: torch.Tensor,
    sampling_locations: torch.Tensor,
    attention_logits: torch.Tensor,
    *,
    im2col_step: int = 64,
    backend: str = "auto",
) -> torch.Tensor:
    """``multi_scale_deformable_attn`` with ``attention_weights =
    attention_softmax(attention_logits)``, ``[bs, nq, M*C]`` in ``value.dtype``.

    ``backend``: ``"auto"`` (HIP kernels on ROCm tensors, the PyTorch path
    elsewhere), ``"hip"`` (native kernels or an error) or ``"reference"``
    (softmax, then the grid_sample path, on any device). A native failure is
    raised, not hidden behind the PyTorch path.
    """
    _validate_inputs(value, spatial_shapes, level_start_index)
    if attention_logits.dim() != 5:
        raise ValueError("attention_logits must be [bs, num_query, num_heads, num_levels, "
                         "num_points]")
    native_available = _native_extension() is not None
    decision = _explain_dispatch(value, backend=backend, native_available=native_available)
    if decision.backend == "error":
        _report(backend, "error", decision, native_available)
        detail = native_error() if not native_available and is_rocm_tensor(value) else None
        raise RuntimeError(f"{decision.reason}: {detail}" if detail else decision.reason)
    if decision.backend == "reference":
        _report(backend, "reference", decision, native_available)
        return multi_scale_deformable_attn_pytorch(
            value, spatial_shapes,
            sampling_locations.to(value.dtype),
            attention_softmax(attention_logits).to(value.dtype),
        )
    if sampling_locations.size(1) == 0:
        output = value.new_zeros((value.size(0), 0, value.size(2) * value.size(3)))
        _report(backend, NATIVE_BACKEND, decision, native_available)
        return (
            output
            + value.sum() * 0
            + sampling_locations.sum().to(value.dtype) * 0
            + attention_logits.sum().to(value.dtype) * 0
        )
    output = _NativeMSDASoftmaxFunction.apply(
        value, spatial_shapes, level_start_index, sampling_locations, attention_logits,
        im2col_step, _bins_early(value, sampling_locations, attention_logits),
    )
    _report(backend, NATIVE_BACKEND, decision, native_available)
    return output
