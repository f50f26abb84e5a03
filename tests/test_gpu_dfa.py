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
