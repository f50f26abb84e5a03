"""Deformable aggregation on the GPU: the HIP kernels against the oracle.

Mirrors the reference's device tests
(/root/reference/tests/ops/test_deformable_aggregation.py:174-227): the small
case forward and backward, zero anchors, and the optimised kernels against
the baseline ones at SparseDrive's production shape. Expected values come from
oracle/dfa_torch.py; at the production shape the oracle's batched form runs on
the GPU (it is plain torch). Tolerances: forward 1e-5 (the reference tests
use 1e-4), gradients 1e-4 relative (1e-3 there).
"""

from __future__ import annotations

import pytest
import torch

from conftest import gpu_available
from muspace_amd import clear_dispatch_report, get_last_dispatch_report
from muspace_amd.ops import deformable_aggregation
from muspace_amd.runtime.native import load_native_module
from muspace_amd.workloads import make_dfa_inputs
from oracle import dfa_torch
from test_dfa_oracle import SMALL_EXPECTED, random_case, small_case

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not gpu_available(), reason="AMD GPU required"),
]

DEV = "cuda"


def _to_device(case, requires_grad=True):
    out = []
    for t in case:
        d = t.detach().to(DEV)
        if d.is_floating_point():
            d = d.float()
            if requires_grad:
                d.requires_grad_(True)
        out.append(d)
    return out


def _reference_copy(case):
    return [t.detach().cpu().double().requires_grad_(True) if t.is_floating_point()
            else t.detach().cpu() for t in case]


def test_small_case_forward_and_backward():
    native = _to_device(small_case())
    ref = _reference_copy(native)
    clear_dispatch_report()
    actual = deformable_aggregation(*native, backend="hip")
    report = get_last_dispatch_report()
    assert report.operator == "deformable_aggregation" and report.selected_backend == "hip"
    torch.testing.assert_close(actual.cpu(), SMALL_EXPECTED, rtol=1e-5, atol=1e-5)
    expected = dfa_torch.aggregate_loops(*ref)
    actual.square().sum().backward()
    expected.square().sum().backward()
    for a, e in zip((native[0], native[3], native[4]), (ref[0], ref[3], ref[4])):
        torch.testing.assert_close(a.grad.cpu().double(), e.grad, rtol=1e-4, atol=1e-4)


def test_zero_anchors_returns_empty_output_and_zero_gradients():
    mc, spatial, start, loc, weights = _to_device(small_case(), requires_grad=False)
    mc.requires_grad_(True)
    loc = loc[:, :0].detach().requires_grad_()
    weights = weights[:, :0].detach().requires_grad_()
    output = deformable_aggregation(mc, spatial, start, loc, weights, backend="hip")
    assert output.shape == (1, 0, 4)
    output.sum().backward()
    for tensor in (mc, loc, weights):
        torch.testing.assert_close(tensor.grad, torch.zeros_like(tensor.grad))


@pytest.mark.parametrize(
    "channels,groups",
    [(256, 8), (64, 8), (128, 1), (192, 3), (256, 2), (48, 4), (96, 3)],
)
def test_random_cases_match_the_oracle(channels, groups):
    """Row kernels for C = 64, 128, 192, 256 with group widths from 8 lanes to
    two 64-channel slots; the generic kernels for C = 48 and 96."""
    case = random_case(11, batch=2, anchors=9, pts=3, cams=3, shapes=((7, 9), (4, 5), (2, 3)),
                       channels=channels, groups=groups)
    native = _to_device(case)
    ref = _reference_copy(native)
    actual = deformable_aggregation(*native, backend="hip")
    expected = dfa_torch.aggregate_batched(*ref)
    torch.testing.assert_close(actual.cpu().double(), expected.detach(), rtol=1e-5, atol=1e-5)
    grad = torch.randn(actual.shape, generator=torch.Generator().manual_seed(2))
    (actual * grad.to(DEV)).sum().backward()
    (expected * grad.double()).sum().backward()
    for a, e in zip((native[0], native[3], native[4]), (ref[0], ref[3], ref[4])):
        torch.testing.assert_close(a.grad.cpu().double(), e.grad, rtol=1e-4, atol=1e-4)


def _production(seed):
    t = make_dfa_inputs(seed=seed, device=DEV)
    return (t["mc_ms_feat"], t["spatial_shape"], t["scale_start_index"], t["sampling_location"],
            t["weights"], t["grad_output"])


def test_opt_matches_base_at_the_production_shape():
    """Reference test :194-227 (opt against base; 1e-4 forward, 1e-3 gradients)."""
    lib = load_native_module()
    mc, spatial, start, loc, weights, grad_out = _production(2333)
    outs = []
    for name in ("opt", "base"):
        out = torch.zeros((mc.shape[0], loc.shape[1], mc.shape[2]), device=DEV)
        getattr(lib, f"deformable_aggregation_forward_{name}")(mc, spatial, start, loc, weights,
                                                               out)
        gf, gl, gw = torch.zeros_like(mc), torch.zeros_like(loc), torch.zeros_like(weights)
        getattr(lib, f"deformable_aggregation_backward_{name}")(mc, spatial, start, loc, weights,
                                                                grad_out, gf, gl, gw)
        outs.append((out, gf, gl, gw))
    for a, b in zip(*outs):
        torch.testing.assert_close(a, b, rtol=1e-4, atol=1e-4)


def test_production_shape_matches_the_oracle():
    """Full SparseDrive shape (8 x 900 anchors, 13 points, 6 cameras x 4
    scales, 256 channels in 8 groups) against the oracle's batched form run
    on the GPU, forward and backward."""
    mc, spatial, start, loc, weights, grad_out = _production(7)
    native = [t.clone().requires_grad_(t.is_floating_point()) for t in (mc, spatial, start, loc,
                                                                          weights)]
    oracle_in = [t.clone().requires_grad_(t.is_floating_point()) for t in (mc, spatial, start,
                                                                             loc, weights)]
    actual = deformable_aggregation(*native)
    expected = dfa_torch.aggregate_batched(*oracle_in)
    torch.testing.assert_close(actual, expected.detach(), rtol=1e-5, atol=1e-5)
    actual.backward(grad_out)
    expected.backward(grad_out)
    for a, e in zip((native[0], native[3], native[4]), (oracle_in[0], oracle_in[3], oracle_in[4])):
        torch.testing.assert_close(a.grad, e.grad, rtol=1e-4, atol=1e-4)


def test_sparsedrive_patched_entry_runs_the_hip_kernels(monkeypatch):
    import sys
    import types

    from muspace_amd.patcher import SparseDrivePatcher

    ops = types.ModuleType("projects.mmdet3d_plugin.ops")
    ops.deformable_aggregation_function = lambda *a: None
    monkeypatch.setitem(sys.modules, ops.__name__, ops)
    patcher = SparseDrivePatcher()
    patcher.apply(strict=True)
    try:
        clear_dispatch_report()
        mc, spatial, start, loc, weights = _to_device(small_case(), requires_grad=False)
        out = ops.deformable_aggregation_function(mc, spatial.long(), start.long(), loc, weights)
        assert get_last_dispatch_report().selected_backend == "hip"
        torch.testing.assert_close(out.cpu(), SMALL_EXPECTED, rtol=1e-5, atol=1e-5)
    finally:
        patcher.restore()


# --- backward contract at medium shapes ------------------------------------------------------

def _oracle_grads(case, grad_out):
    """Expected (grad_mc_ms_feat, grad_sampling_location, grad_weights) in float64 on the CPU."""
    ref = _reference_copy(case)
    out = dfa_torch.aggregate_batched(*ref)
    (out * grad_out.cpu().double()).sum().backward()
    return ref[0].grad, ref[3].grad, ref[4].grad


def _backward_opt(case, grad_out, init_feat=None, init_other=None):
    """deformable_aggregation_backward_opt through the C-ABI on buffers that start at
    init_feat (grad_mc_ms_feat) and init_other (the location and weight gradients)."""
    lib = load_native_module()
    mc, spatial, start, loc, weights = _to_device(case, requires_grad=False)
    gf = torch.zeros_like(mc) if init_feat is None else init_feat.clone()
    gl = torch.zeros_like(loc) if init_other is None else torch.full_like(loc, init_other)
    gw = torch.zeros_like(weights) if init_other is None else torch.full_like(weights, init_other)
    lib.deformable_aggregation_backward_opt(mc, spatial, start, loc, weights,
                                            grad_out.to(DEV).float(), gf, gl, gw)
    torch.cuda.synchronize()
    return gf, gl, gw


# Location gradients at these shapes sum about 1000 fp32 products of size up to ~W = 30 per
# element, so fp32 rounding alone leaves ~1e-4 absolute: they are held to the reference tests'
# gradient bar (tests/ops/test_deformable_aggregation.py:194-227, 1e-3), the feature and weight
# gradients to 1e-4.
LOC_TOL = dict(rtol=1e-4, atol=1e-3)


def _medium_case(seed, channels, groups, anchors=300):
    """Locations on a 1/4096 grid: x * W - 0.5 is then exact in float32, so the kernels'
    cell coordinates equal the float64 oracle's. (Off the grid, one float32 ulp of a
    coordinate near 30 moves a location gradient by about a * W^2 * |D| * 2e-6, up to
    1e-3 here: a second-order effect of the input rounding, not of the kernels.)"""
    case = list(random_case(seed, batch=2, anchors=anchors, pts=5, cams=3,
                            shapes=((20, 30), (10, 15), (5, 8), (3, 4)), channels=channels,
                            groups=groups))
    loc = case[3]
    loc.copy_(torch.round(loc * 4096) / 4096)
    loc[1, 7, 2, 1] = float("nan")  # a NaN location is skipped
    loc[1, 8, 0, 2] = torch.tensor([1 / 4096, 1 - 1 / 4096], dtype=loc.dtype)  # edge corners
    return case


@pytest.mark.parametrize("channels,groups", [(128, 8), (256, 8), (256, 4), (96, 3)])
def test_medium_backward_matches_the_oracle(channels, groups):
    """Groups of 16, 32, 64 (row kernels) and 32 channels (generic kernel, C = 96): 300
    anchors, 12 (camera, scale) maps of up to 20 x 30 cells; NaN and near-edge locations."""
    case = _medium_case(5, channels, groups)
    grad_out = torch.randn(2, 300, channels, generator=torch.Generator().manual_seed(6))
    gf, gl, gw = _backward_opt(case, grad_out)
    ef, el, ew = _oracle_grads(case, grad_out)
    torch.testing.assert_close(gf.cpu().double(), ef, rtol=1e-4, atol=1e-4)
    torch.testing.assert_close(gl.cpu().double(), el, **LOC_TOL)
    torch.testing.assert_close(gw.cpu().double(), ew, rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("channels,groups", [(256, 8), (64, 8)])
def test_backward_adds_into_grad_feat_and_writes_the_others(channels, groups):
    """The reference's contract (deformable_aggregation_musa.mu:411-428): grad_mc_ms_feat
    is added into, the location and weight gradients are stored (groups of 32 and of 8)."""
    case = _medium_case(8, channels, groups, anchors=40)
    grad_out = torch.randn(2, 40, channels, generator=torch.Generator().manual_seed(9))
    init = torch.randn(case[0].shape, generator=torch.Generator().manual_seed(10))
    gf, gl, gw = _backward_opt(case, grad_out, init_feat=init.to(DEV).float(), init_other=7.0)
    ef, el, ew = _oracle_grads(case, grad_out)
    torch.testing.assert_close(gf.cpu().double(), ef + init.double(), rtol=1e-4, atol=1e-4)
    torch.testing.assert_close(gl.cpu().double(), el, **LOC_TOL)
    torch.testing.assert_close(gw.cpu().double(), ew, rtol=1e-4, atol=1e-4)


def test_overlapping_maps_add_both_contributions():
    """Maps that share cells (start indexes are inputs: the reference's nested
    feature_maps_format, mu_space/ops/deformable_aggregation.py:399-404, restarts them at 0
    per group): both maps' contributions reach the shared rows."""
    case = _medium_case(11, 256, 8, anchors=60)
    spatial, start = case[1], case[2]
    spatial[1] = spatial[0]
    start[1] = start[0]  # camera 1 reads camera 0's maps
    grad_out = torch.randn(2, 60, 256, generator=torch.Generator().manual_seed(12))
    gf, gl, gw = _backward_opt(case, grad_out)
    ef, el, ew = _oracle_grads(case, grad_out)
    torch.testing.assert_close(gf.cpu().double(), ef, rtol=1e-4, atol=1e-4)
    torch.testing.assert_close(gl.cpu().double(), el, **LOC_TOL)
    torch.testing.assert_close(gw.cpu().double(), ew, rtol=1e-4, atol=1e-4)


def test_backward_twice_with_a_smaller_case():
    """Two calls in a row, the second smaller: nothing of the first call leaks into it."""
    for anchors in (300, 37):
        case = _medium_case(13, 256, 8, anchors=anchors)
        grad_out = torch.randn(2, anchors, 256, generator=torch.Generator().manual_seed(14))
        gf, gl, gw = _backward_opt(case, grad_out)
        ef, el, ew = _oracle_grads(case, grad_out)
        torch.testing.assert_close(gf.cpu().double(), ef, rtol=1e-4, atol=1e-4)
        torch.testing.assert_close(gl.cpu().double(), el, **LOC_TOL)
        torch.testing.assert_close(gw.cpu().double(), ew, rtol=1e-4, atol=1e-4)


# --- the coarse maps' LDS sums (dfa_backward_coarse) -------------------------------------------
# The optimised backward sums the feature gradients of each camera's small maps in LDS as
# fixed-point integers, with a scale chosen per workgroup from the largest contribution; a
# workgroup that meets a non-finite grad_output or weight falls back to fp32 device atomics.


@pytest.mark.parametrize("scale", [1e-30, 1e30])
def test_coarse_sums_keep_their_precision_at_any_gradient_scale(scale):
    """grad_output scaled by 1e-30 and 1e30: the fixed-point scale follows, so the feature
    and weight gradients keep the 1e-4 relative bar."""
    case = _medium_case(21, 256, 8, anchors=120)
    grad_out = torch.randn(2, 120, 256, generator=torch.Generator().manual_seed(22)) * scale
    gf, gl, gw = _backward_opt(case, grad_out)
    ef, el, ew = _oracle_grads(case, grad_out)
    assert torch.isfinite(gf).all()
    torch.testing.assert_close(gf.cpu().double(), ef, rtol=1e-4, atol=1e-4 * scale)
    torch.testing.assert_close(gw.cpu().double(), ew, rtol=1e-4, atol=1e-4 * scale)


def test_non_finite_grad_output_matches_the_base_kernels():
    """An inf and a NaN in grad_output: the workgroups that see them add with fp32 atomics,
    so every gradient equals the base kernels' (non-finite entries included)."""
    lib = load_native_module()
    case = _medium_case(23, 256, 8, anchors=80)
    grad_out = torch.randn(2, 80, 256, generator=torch.Generator().manual_seed(24))
    grad_out[0, 5, 40] = float("inf")
    grad_out[1, 9, 3] = float("nan")
    mc, spatial, start, loc, weights = _to_device(case, requires_grad=False)
    results = []
    for name in ("opt", "base"):
        gf, gl, gw = torch.zeros_like(mc), torch.zeros_like(loc), torch.zeros_like(weights)
        getattr(lib, f"deformable_aggregation_backward_{name}")(mc, spatial, start, loc, weights,
                                                                grad_out.to(DEV), gf, gl, gw)
        results.append((gf, gl, gw))
    assert not torch.isfinite(results[0][0]).all()
    for a, b, tol in zip(*results, (dict(rtol=1e-4, atol=1e-4), LOC_TOL,
                                    dict(rtol=1e-4, atol=1e-4))):
        torch.testing.assert_close(a, b, equal_nan=True, **tol)


def test_every_point_active_matches_the_base_kernels():
    """SparseDrive's shape with every (anchor, point, camera) inside its image: 11,700 active
    pairs per (batch entry, camera), more than a workgroup lists or holds, so the coarse
    kernel reads its pairs from memory."""
    lib = load_native_module()
    t = make_dfa_inputs(seed=31, device=DEV, active_frac=1.0)
    mc, spatial, start, loc, weights = (t[k] for k in ("mc_ms_feat", "spatial_shape",
                                                        "scale_start_index",
                                                        "sampling_location", "weights"))
    results = []
    for name in ("opt", "base"):
        gf, gl, gw = torch.zeros_like(mc), torch.zeros_like(loc), torch.zeros_like(weights)
        getattr(lib, f"deformable_aggregation_backward_{name}")(mc, spatial, start, loc, weights,
                                                                t["grad_output"], gf, gl, gw)
        results.append((gf, gl, gw))
    for a, b, tol in zip(*results, (dict(rtol=1e-4, atol=1e-4), LOC_TOL,
                                    dict(rtol=1e-4, atol=1e-4))):
        torch.testing.assert_close(a, b, **tol)


def test_more_than_four_small_maps():
    """Six maps per camera, all small enough for LDS: the maps past the fourth take their
    weights from memory."""
    case = list(random_case(25, batch=2, anchors=70, pts=4, cams=2,
                            shapes=((12, 16), (8, 10), (6, 8), (4, 5), (3, 3), (2, 2)),
                            channels=128, groups=4))
    case[3].copy_(torch.round(case[3] * 4096) / 4096)
    grad_out = torch.randn(2, 70, 128, generator=torch.Generator().manual_seed(26))
    gf, gl, gw = _backward_opt(case, grad_out)
    ef, el, ew = _oracle_grads(case, grad_out)
    torch.testing.assert_close(gf.cpu().double(), ef, rtol=1e-4, atol=1e-4)
    torch.testing.assert_close(gl.cpu().double(), el, **LOC_TOL)
    torch.testing.assert_close(gw.cpu().double(), ew, rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("rows", [16384, 16385, 32768])
def test_row_counts_past_the_split_thresholds_match_the_base_kernels(rows):
    """The row kernels share a row's pairs among four wavefronts below 16,384 (batch, anchor)
    rows, two below 32,768 and one from there on; every other test stays below 16,384. At the
    two larger counts, forward and backward against the base kernels; an odd count leaves the
    last workgroup of the two-wavefront split with a row and two idle wavefronts."""
    lib = load_native_module()
    batch = 2 if rows % 2 == 0 else 1
    anchors = rows // batch
    case = list(random_case(rows, batch=batch, anchors=anchors, pts=3, cams=3,
                            shapes=((12, 20), (6, 10), (3, 5)), channels=256, groups=8,
                            dtype=torch.float32))
    case[3].copy_(torch.round(case[3] * 4096) / 4096)
    grad_out = torch.randn(batch, anchors, 256, generator=torch.Generator().manual_seed(rows))
    mc, spatial, start, loc, weights = _to_device(case, requires_grad=False)
    outs = []
    for name in ("opt", "base"):
        out = torch.zeros((batch, anchors, 256), device=DEV)
        getattr(lib, f"deformable_aggregation_forward_{name}")(mc, spatial, start, loc, weights,
                                                               out)
        gf, gl, gw = torch.zeros_like(mc), torch.zeros_like(loc), torch.zeros_like(weights)
        getattr(lib, f"deformable_aggregation_backward_{name}")(mc, spatial, start, loc, weights,
                                                                grad_out.to(DEV), gf, gl, gw)
        outs.append((out, gf, gl, gw))
    assert outs[1][0].abs().max() > 0 and outs[1][1].abs().max() > 0
    for a, b, tol in zip(*outs, (dict(rtol=1e-5, atol=1e-5), dict(rtol=1e-4, atol=1e-4),
                                 LOC_TOL, dict(rtol=1e-4, atol=1e-4))):
        torch.testing.assert_close(a, b, **tol)


def test_misaligned_grad_output_and_locations_skip_the_coarse_kernel():
    """grad_output 4 bytes past a 16-byte boundary and locations 4 bytes past an 8-byte one:
    the backward leaves the coarse kernel out (it reads them in 16- and 8-byte pieces) and
    every map takes the row kernel's atomics; the gradients are the aligned call's."""
    lib = load_native_module()
    case = _medium_case(27, 256, 8, anchors=50)
    mc, spatial, start, loc, weights = _to_device(case, requires_grad=False)
    grad_out = torch.randn(2, 50, 256, generator=torch.Generator().manual_seed(28)).to(DEV)
    shifted_go = torch.empty(grad_out.numel() + 1, device=DEV)[1:].view_as(grad_out)
    shifted_go.copy_(grad_out)
    shifted_loc = torch.empty(loc.numel() + 1, device=DEV)[1:].view_as(loc)
    shifted_loc.copy_(loc)
    assert shifted_go.data_ptr() % 16 == 4 and shifted_loc.data_ptr() % 8 == 4
    results = []
    for go, lc in ((grad_out, loc), (shifted_go, loc), (grad_out, shifted_loc)):
        gf, gl, gw = torch.zeros_like(mc), torch.zeros_like(loc), torch.zeros_like(weights)
        lib.deformable_aggregation_backward_opt(mc, spatial, start, lc, weights, go, gf, gl, gw)
        results.append((gf, gl, gw))
    for other in results[1:]:
        for a, b, tol in zip(results[0], other, (dict(rtol=1e-4, atol=1e-4), LOC_TOL,
                                                 dict(rtol=1e-4, atol=1e-4))):
            torch.testing.assert_close(b, a, **tol)


@pytest.mark.parametrize("seed", range(12))
def test_random_shapes_backward_matches_the_oracle(seed):
    """Seeded random channels (64-256), group widths (8 lanes to two 64-channel slots), 1-5
    maps of up to 40 x 40 per camera, 1-6 cameras, up to 300 anchors and 13 points, grad_output
    scaled by 1e-3 to 1e3 (the coarse kernel's fixed-point scale follows it), every third seed
    with 10% NaN locations."""
    r = torch.Generator().manual_seed(11000 + seed)
    pick = lambda lo, hi: int(torch.randint(lo, hi + 1, (1,), generator=r))  # noqa: E731
    channels = (64, 128, 192, 256)[pick(0, 3)]
    widths = [c for c in (8, 16, 32, 64, 128)
              if channels % c == 0 and channels // c <= 8 and (c < 64 or c % 64 == 0)]
    groups = channels // widths[pick(0, len(widths) - 1)]
    shapes = tuple((pick(1, 40), pick(1, 40)) for _ in range(pick(1, 5)))
    cams, anchors, pts = pick(1, 6), pick(1, 300), pick(2, 13)
    case = list(random_case(seed, batch=pick(1, 3), anchors=anchors, pts=pts, cams=cams,
                            shapes=shapes, channels=channels, groups=groups))
    loc = case[3]
    loc.copy_(torch.round(loc * 4096) / 4096)
    if seed % 3 == 0:
        drop = torch.rand(loc.shape[:-1], generator=r) < 0.1
        loc[..., 0] = torch.where(drop, torch.nan, loc[..., 0])
    scale = 10.0 ** pick(-3, 3)
    grad_out = torch.randn(case[0].shape[0], anchors, channels,
                           generator=torch.Generator().manual_seed(seed)) * scale
    gf, gl, gw = _backward_opt(case, grad_out)
    ef, el, ew = _oracle_grads(case, grad_out)
    torch.testing.assert_close(gf.cpu().double(), ef, rtol=1e-4, atol=1e-4 * scale)
    torch.testing.assert_close(gl.cpu().double(), el, rtol=1e-4, atol=1e-3 * scale)
    torch.testing.assert_close(gw.cpu().double(), ew, rtol=1e-4, atol=1e-4 * scale)
