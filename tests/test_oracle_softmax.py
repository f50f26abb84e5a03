"""Pins of the fused-softmax oracle (oracle/msda_softmax.py) on the CPU.

The softmax is torch's; what these tests fix is its axis (each (b, q, m) unit's
L*P logits jointly, not each level's P), its composition with the operator and
the closed-form logit gradient the backward kernels implement.
"""

from __future__ import annotations

import torch

from msda_testlib import random_case
from oracle import msda_softmax
from oracle.msda_torch import msda_forward


def _case(seed, **kw):
    value, shapes, _, loc, _, grad = random_case(seed, **kw)
    g = torch.Generator().manual_seed(seed + 100)
    logits = torch.randn(loc.shape[:-1], generator=g, dtype=value.dtype) * 2.0
    return value, shapes, loc, logits, grad


def test_equal_logits_give_uniform_weights_over_levels_and_points():
    """Constant logits per unit: every weight is 1/(L*P). A softmax over each
    level's P points alone (a plausible slip: the reference test's dim=-1 on
    [.., L, P] weights) gives 1/P and an output L times larger."""
    value, shapes, loc, logits, _ = _case(1)
    logits = torch.full_like(logits, 0.7)
    levels, points = loc.shape[3], loc.shape[4]
    uniform = torch.full(logits.shape, 1.0 / (levels * points), dtype=logits.dtype)
    expected = msda_forward(value, shapes, loc, uniform)
    torch.testing.assert_close(msda_softmax.forward(value, shapes, loc, logits), expected,
                               rtol=1e-12, atol=1e-12)
    per_level = msda_forward(value, shapes, loc, torch.softmax(logits, dim=-1))
    torch.testing.assert_close(per_level, expected * levels, rtol=1e-12, atol=1e-12)


def test_shift_of_a_unit_leaves_the_output_unchanged():
    value, shapes, loc, logits, _ = _case(2)
    shift = torch.randn(logits.shape[:3], dtype=logits.dtype)[..., None, None] * 5
    torch.testing.assert_close(msda_softmax.forward(value, shapes, loc, logits + shift),
                               msda_softmax.forward(value, shapes, loc, logits),
                               rtol=1e-12, atol=1e-12)


def test_autograd_logit_gradient_equals_the_closed_form():
    """Two routes to grad_logits: autograd through torch.softmax, and
    p * (g - <p, g>) on the operator's weight gradient."""
    value, shapes, loc, logits, grad = _case(3)
    _, _, _, auto = msda_softmax.forward_backward(value, shapes, loc, logits, grad)
    closed = msda_softmax.logit_grad(value, shapes, loc, logits, grad)
    torch.testing.assert_close(auto, closed, rtol=1e-10, atol=1e-12)
    # softmax is shift invariant per unit, so each unit's logit gradient sums to zero
    sums = auto.reshape(*auto.shape[:3], -1).sum(-1)
    torch.testing.assert_close(sums, torch.zeros_like(sums), rtol=0, atol=1e-12)
    assert auto.abs().max() > 1e-3


def test_minus_infinity_logits_get_zero_weight():
    value, shapes, loc, logits, _ = _case(4)
    masked = logits.clone()
    masked[0, 1, 2, 0, :] = float("-inf")
    weights = msda_softmax.softmax_weights(masked)
    assert torch.all(weights[0, 1, 2, 0] == 0)
    torch.testing.assert_close(weights.reshape(*weights.shape[:3], -1).sum(-1),
                               torch.ones(weights.shape[:3], dtype=weights.dtype))


def test_gradcheck_of_the_oracle():
    value, shapes, loc, logits, _ = _case(5, batch=1, queries=2, heads=2, channels=2,
                                          levels=((3, 4), (2, 2)), points=2)
    loc = loc.clamp(0.05, 0.95)  # away from cell edges, where the gradient is continuous
    args = [t.detach().clone().requires_grad_(True) for t in (value, loc, logits)]
    assert torch.autograd.gradcheck(
        lambda v, lc, lg: msda_softmax.forward(v, shapes, lc, lg), args, eps=1e-6, atol=1e-6
    )


def test_operator_on_cpu_tensors_takes_the_reference_path():
    from muspace_amd import clear_dispatch_report, get_last_dispatch_report
    from muspace_amd.ops import level_start_index_from_shapes, multi_scale_deformable_attn_softmax

    value, shapes, loc, logits, _ = _case(6, dtype=torch.float32)
    clear_dispatch_report()
    out = multi_scale_deformable_attn_softmax(value, shapes, level_start_index_from_shapes(shapes),
                                              loc, logits)
    report = get_last_dispatch_report()
    assert report.operator == "multi_scale_deformable_attn_softmax"
    assert report.selected_backend == "reference"
    torch.testing.assert_close(out, msda_softmax.forward(value, shapes, loc, logits),
                               rtol=1e-6, atol=1e-6)
