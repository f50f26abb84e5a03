"""TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

CPU restatement of MSDA with its attention weights produced by a softmax over
each (batch, query, head) unit's L*P logits, the composition BEVFormer-style
modules use and the reference's tests and model scripts call
(/root/reference/tests/ops/test_multi_scale_deformable_attn.py:62 softmax,
then the operator; /root/reference/model_examples/BEVFormer/scripts/smoke_openmmlab.py:31-32
``multi_scale_deformable_attn_pytorch(value, shapes, sampling, weights_raw.softmax(-1))``).

``forward`` is torch.softmax over the flattened L*P axis followed by the
grid_sample restatement of msda_torch.py; autograd of it is the backward
oracle (``forward_backward``). ``logit_grad`` states the softmax backward in
closed form, g_logit = p * (g - sum_j p_j g_j), on the operator's weight
gradient: an independent route to the same numbers that pins the autograd one.
"""

from __future__ import annotations

import torch

from .msda_torch import msda_forward, msda_forward_backward


def softmax_weights(logits: torch.Tensor) -> torch.Tensor:
    bs, nq, heads, levels, points = logits.shape
    flat = logits.reshape(bs, nq, heads, levels * points)
    return torch.softmax(flat, dim=-1).reshape(bs, nq, heads, levels, points)


def forward(value, spatial_shapes, sampling_locations, logits):
    return msda_forward(value, spatial_shapes, sampling_locations, softmax_weights(logits))


def forward_backward(value, spatial_shapes, sampling_locations, logits, grad_output):
    """(output, grad_value, grad_sampling_locations, grad_logits) by autograd."""
    v = value.detach().clone().requires_grad_(True)
    loc = sampling_locations.detach().clone().requires_grad_(True)
    lg = logits.detach().clone().requires_grad_(True)
    out = forward(v, spatial_shapes, loc, lg)
    out.backward(grad_output)
    return out.detach(), v.grad, loc.grad, lg.grad


def logit_grad(value, spatial_shapes, sampling_locations, logits, grad_output):
    """Logit gradient in closed form from the operator's weight gradient."""
    p = softmax_weights(logits.detach())
    _, _, _, g = msda_forward_backward(value, spatial_shapes, sampling_locations, p, grad_output)
    bs, nq, heads, levels, points = logits.shape
    pf = p.reshape(bs, nq, heads, -1)
    gf = g.reshape(bs, nq, heads, -1)
    dot = (pf * gf).sum(-1, keepdim=True)
    return (pf * (gf - dot)).reshape(logits.shape)
