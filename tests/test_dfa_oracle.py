"""Deformable aggregation: the oracle pinned, and the CPU-side API.

The oracle (oracle/dfa_torch.py) has two independent formulations. They are
pinned by the reference tests' small case (values worked out by hand below;
/root/reference/tests/ops/test_deformable_aggregation.py:83-99,134-147), by
closed forms (a constant field, a linear field and its location gradient),
by gradcheck, and by a planted mistake that must fail. The operator's own
PyTorch backend and its validation follow
/root/reference/tests/ops/test_deformable_aggregation.py:134-168.
"""

from __future__ import annotations

import sys
import types

import pytest
import torch

from muspace_amd.ops import (
    deformable_aggregation,
    deformable_aggregation_reference,
    feature_maps_format,
)
from oracle import dfa_torch


def small_case(dtype=torch.float32, requires_grad=False):
    """The reference tests' small case: one camera, maps 2x2 and 1x1, 4 channels
    in 2 groups; anchor 1 sits on the open-interval boundary x = 1."""
    mc = torch.arange(20, dtype=dtype).view(1, 5, 4)
    spatial = torch.tensor([[[2, 2], [1, 1]]], dtype=torch.int32)
    start = torch.tensor([[0, 4]], dtype=torch.int32)
    loc = torch.tensor([[[[[0.5, 0.5]]], [[[1.0, 0.5]]]]], dtype=dtype)
    weights = torch.tensor([[[[[[0.25, 0.5], [0.75, 1.0]]]], [[[[0.5, 0.25], [1.0, 0.75]]]]]],
                           dtype=dtype)
    if requires_grad:
        for t in (mc, loc, weights):
            t.requires_grad_(True)
    return mc, spatial, start, loc, weights


# anchor 0: scale 0 samples the 2x2 map at its centre (mean of cells 0-3 =
# [6, 7, 8, 9]) times group weights (0.25, 0.25, 0.5, 0.5); scale 1 samples
# the single cell [16..19] times (0.75, 0.75, 1, 1). Anchor 1 is skipped.
SMALL_EXPECTED = torch.tensor([[[13.5, 14.5, 22.0, 23.5], [0.0, 0.0, 0.0, 0.0]]])


def random_case(seed, *, batch=2, anchors=3, pts=2, shapes=((3, 4), (2, 2)), cams=2,
                channels=8, groups=2, dtype=torch.float64, boundary=True):
    g = torch.Generator().manual_seed(seed)
    spatial = torch.tensor([[list(s) for s in shapes]] * cams, dtype=torch.int32)
    # cameras may differ: the second camera's first map is one row taller
    if cams > 1:
        spatial[1, 0, 0] += 1
    sizes = (spatial[..., 0] * spatial[..., 1]).flatten()
    start = torch.cat([torch.zeros(1, dtype=torch.int64), sizes.cumsum(0)[:-1]])
    start = start.view(cams, len(shapes)).to(torch.int32)
    num_feat = int(sizes.sum())
    mc = torch.randn(batch, num_feat, channels, generator=g, dtype=dtype)
    loc = torch.rand(batch, anchors, pts, cams, 2, generator=g, dtype=dtype) * 1.2 - 0.1
    if boundary:  # exact boundaries are skipped
        loc[0, 0, 0, 0, 0] = 0.0
        loc[0, 0, 1, 0, 1] = 1.0
    weights = torch.rand(batch, anchors, pts, cams, len(shapes), groups, generator=g, dtype=dtype)
    return mc, spatial, start, loc, weights


@pytest.mark.parametrize("form", [dfa_torch.aggregate_loops, dfa_torch.aggregate_batched])
def test_oracle_small_case_known_answer(form):
    out = form(*small_case(torch.float64))
    torch.testing.assert_close(out, SMALL_EXPECTED.double(), rtol=0, atol=1e-12)


@pytest.mark.parametrize("seed", [0, 1, 2, 3])
def test_oracle_forms_agree(seed):
    case = random_case(seed)
    loops = dfa_torch.aggregate_loops(*case)
    batched = dfa_torch.aggregate_batched(*case)
    torch.testing.assert_close(batched, loops, rtol=1e-12, atol=1e-12)
    assert loops.abs().sum() > 0


def test_oracle_forms_agree_on_nan_locations_and_gradients():
    """A NaN location is skipped by both forms, in the output and in every gradient
    (reference kernel: deformable_aggregation_musa.mu:376, the open-interval test is false
    for NaN)."""
    case = [t.requires_grad_(t.is_floating_point()) for t in random_case(7)]
    with torch.no_grad():
        case[3][1, 2, 0, 1, 0] = float("nan")
        case[3][0, 1, 1, 0, 1] = float("nan")
    twin = [t.detach().clone().requires_grad_(t.is_floating_point()) for t in case]
    loops = dfa_torch.aggregate_loops(*case)
    batched = dfa_torch.aggregate_batched(*twin)
    assert torch.isfinite(batched).all()
    torch.testing.assert_close(batched, loops, rtol=1e-12, atol=1e-12)
    grad = torch.randn(loops.shape, generator=torch.Generator().manual_seed(1), dtype=loops.dtype)
    (loops * grad).sum().backward()
    (batched * grad).sum().backward()
    for i in (0, 3, 4):
        assert torch.isfinite(twin[i].grad).all()
        torch.testing.assert_close(twin[i].grad, case[i].grad, rtol=1e-12, atol=1e-12)


def test_oracle_constant_field():
    """Feature 3 everywhere and every corner inside its map: each active
    (point, camera, scale) adds 3 * its group weight."""
    mc, spatial, start, loc, weights = random_case(4, boundary=False)
    mc = torch.full_like(mc, 3.0)
    loc = 0.3 + 0.4 * loc.clamp(0, 1)  # inside [0.5/W, 1 - 0.5/W] for W, H >= 2
    out = dfa_torch.aggregate_batched(mc, spatial, start, loc, weights)
    per_group = mc.shape[-1] // weights.shape[-1]
    expected = 3.0 * weights.sum(dim=(2, 3, 4)).repeat_interleave(per_group, dim=-1)
    torch.testing.assert_close(out, expected, rtol=1e-12, atol=1e-12)


def test_oracle_linear_field_and_location_gradient():
    """Feature = alpha*row + beta*col in every map: bilinear sampling is exact,
    so out = sum w * (alpha*(y*H - 0.5) + beta*(x*W - 0.5)) and d out/dx =
    sum w * beta * W (the location gradient's x W, H factors)."""
    mc, spatial, start, loc, weights = random_case(5, boundary=False)
    alpha, beta = 0.7, -1.3
    field = torch.zeros_like(mc)
    for c in range(spatial.shape[0]):
        for s in range(spatial.shape[1]):
            h, w = spatial[c, s].tolist()
            rows = torch.arange(h, dtype=mc.dtype).repeat_interleave(w)
            cols = torch.arange(w, dtype=mc.dtype).repeat(h)
            st = int(start[c, s])
            field[:, st: st + h * w] = (alpha * rows + beta * cols)[None, :, None]
    loc = (0.3 + 0.4 * loc.clamp(0, 1)).requires_grad_(True)
    out = dfa_torch.aggregate_batched(field, spatial, start, loc, weights)
    per_group = mc.shape[-1] // weights.shape[-1]
    hs = spatial[..., 0].to(mc.dtype)  # [cams, scales]
    ws = spatial[..., 1].to(mc.dtype)
    x, y = loc[..., 0:1], loc[..., 1:2]  # [B, A, P, cams, 1]
    value = alpha * (y * hs - 0.5) + beta * (x * ws - 0.5)  # [B, A, P, cams, scales]
    expected = (weights * value[..., None]).sum(dim=(2, 3, 4)).repeat_interleave(per_group, -1)
    torch.testing.assert_close(out, expected.detach(), rtol=1e-12, atol=1e-12)
    out.sum().backward()
    grad_x = (weights.sum(-1) * per_group * beta * ws).sum(-1)  # [B, A, P, cams]
    grad_y = (weights.sum(-1) * per_group * alpha * hs).sum(-1)
    torch.testing.assert_close(loc.grad[..., 0], grad_x, rtol=1e-10, atol=1e-10)
    torch.testing.assert_close(loc.grad[..., 1], grad_y, rtol=1e-10, atol=1e-10)


def test_oracle_gradcheck():
    mc, spatial, start, loc, weights = random_case(6, batch=1, anchors=2, pts=1, channels=4,
                                                   boundary=False)
    loc = 0.05 + 0.9 * loc.clamp(0, 1)
    args = [t.clone().requires_grad_(True) for t in (mc, loc, weights)]
    assert torch.autograd.gradcheck(
        lambda m, l, w: dfa_torch.aggregate_batched(m, spatial, start, l, w), args,
        eps=1e-6, atol=1e-6)


def test_planted_xy_swap_is_caught():
    """A mutant that reads (y, x) for (x, y) fails the two-form check on
    non-square maps."""
    case = list(random_case(7, boundary=False))
    mutant = dfa_torch.aggregate_batched(case[0], case[1], case[2], case[3].flip(-1), case[4])
    assert not torch.allclose(mutant, dfa_torch.aggregate_loops(*case), rtol=1e-6, atol=1e-6)


# ------------------------------------------------------------ the operator ---


def test_reference_backend_matches_the_oracle():
    for seed in (8, 9):
        case = [t.float() if t.is_floating_point() else t for t in random_case(seed)]
        out = deformable_aggregation(*case, backend="reference")
        torch.testing.assert_close(out, dfa_torch.aggregate_loops(*case), rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(deformable_aggregation_reference(*small_case()), SMALL_EXPECTED)


def test_reference_handles_boundary_and_invalid_locations():
    """Reference test :134-147: the boundary anchor contributes nothing and
    gradients are finite."""
    tensors = small_case(requires_grad=True)
    output = deformable_aggregation(*tensors, backend="reference")
    torch.testing.assert_close(output[:, 1], torch.zeros_like(output[:, 1]))
    output.square().sum().backward()
    for tensor in (tensors[0], tensors[3], tensors[4]):
        assert tensor.grad is not None and torch.isfinite(tensor.grad).all()


def test_validation_messages_follow_the_reference():
    """Reference test :150-159."""
    tensors = list(small_case())
    tensors[-1] = torch.ones((1, 2, 1, 1, 2, 3), dtype=torch.float32)
    with pytest.raises(ValueError, match="divisible by num_groups"):
        deformable_aggregation(*tensors, backend="reference")
    tensors = list(small_case())
    tensors[1] = tensors[1].to(torch.int64)
    with pytest.raises(TypeError, match="spatial_shape must use int32"):
        deformable_aggregation(*tensors, backend="reference")
    tensors = list(small_case())
    tensors[0] = tensors[0].double()
    with pytest.raises(TypeError, match="mc_ms_feat must use float32"):
        deformable_aggregation(*tensors, backend="reference")


def test_feature_maps_format_round_trip_preserves_values():
    """Reference test :162-171."""
    levels = [
        torch.arange(1 * 2 * 4 * 2 * 3, dtype=torch.float32).view(1, 2, 4, 2, 3),
        torch.arange(1 * 2 * 4 * 1 * 2, dtype=torch.float32).view(1, 2, 4, 1, 2),
    ]
    formatted = feature_maps_format(levels)
    assert formatted[1].tolist() == [[[2, 3], [1, 2]], [[2, 3], [1, 2]]]
    assert formatted[2].tolist() == [[0, 6], [8, 14]]
    restored = feature_maps_format(formatted, inverse=True)
    assert len(restored) == 1
    for got, expected in zip(restored[0], levels):
        torch.testing.assert_close(got, expected)


def test_feature_maps_format_packs_what_the_operator_reads():
    """A packed map read back at its scale start is the camera's map."""
    levels = [torch.randn(2, 3, 8, 4, 5), torch.randn(2, 3, 8, 2, 3)]
    col, spatial, start = feature_maps_format(levels)
    for cam in range(3):
        for scale, lv in enumerate(levels):
            h, w = spatial[cam, scale].tolist()
            st = int(start[cam, scale])
            got = col[:, st: st + h * w].view(2, h, w, 8).permute(0, 3, 1, 2)
            torch.testing.assert_close(got, lv[:, cam])
