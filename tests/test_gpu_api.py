"""The operator API on ROCm tensors: the reference's device tests, HIP backend.

Mirrors /root/reference/tests/ops/test_multi_scale_deformable_attn.py:256-468
(skipped there without MUSA) with the native backend ``"hip"``; the expected
values come from the CPU oracle rather than the device's own reference path.
"""

from importlib import import_module

import pytest
import torch

from conftest import gpu_available
from msda_testlib import reference_fixture as _fixture
from muspace_amd import clear_dispatch_report, get_last_dispatch_report, multi_scale_deformable_attn
from oracle import msda_torch

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not gpu_available(), reason="AMD GPU required"),
]

msda_module = import_module("muspace_amd.ops.multi_scale_deformable_attn")
DEV = "cuda"


def _cpu_copy(tensors, dtype=None):
    out = []
    for t in tensors:
        if t.dtype.is_floating_point:
            c = t.detach().cpu()
            c = c.float() if dtype is None else c.to(dtype)
            out.append(c.requires_grad_(t.requires_grad))
        else:
            out.append(t.detach().cpu())
    return tuple(out)


class _NativeCallSpy:
    """Record the dtype of every tensor handed to a native MSDA entry point."""

    def __init__(self, inner):
        self._inner = inner
        self.calls = []

    def __getattr__(self, name):
        target = getattr(self._inner, name)

        def recorded(*args, **kwargs):
            # size queries and argument checks are not kernel entry points
            if name not in {"backward_workspace", "backward_workspace_bytes",
                            "backward_softmax_workspace_bytes", "check_forward",
                            "check_backward"}:
                self.calls.append((name, [getattr(arg, "dtype", None) for arg in args]))
            return target(*args, **kwargs)

        return recorded


@pytest.mark.parametrize("backend", ["hip", "musa", "auto"])
def test_native_matches_reference_forward(backend):
    clear_dispatch_report()
    tensors = _fixture(device=DEV)
    expected = msda_torch.msda_forward(*[t for i, t in enumerate(_cpu_copy(tensors)) if i != 2])
    actual = multi_scale_deformable_attn(*tensors, backend=backend)
    torch.testing.assert_close(actual.cpu(), expected.detach(), rtol=1e-5, atol=1e-5)
    report = get_last_dispatch_report()
    assert report.selected_backend == "hip"
    assert report.native_fallback is False


def test_native_zero_queries_returns_empty_output_and_zero_gradients():
    value, spatial_shapes, level_start_index, locations, weights = _fixture(device=DEV, queries=0)
    output = multi_scale_deformable_attn(value, spatial_shapes, level_start_index, locations,
                                         weights, backend="hip")
    assert output.shape == (1, 0, 6)
    output.sum().backward()
    for tensor in (value, locations, weights):
        torch.testing.assert_close(tensor.grad, torch.zeros_like(tensor.grad))


@pytest.mark.parametrize("embed_dims", [2, 32])
def test_native_matches_reference_backward_on_multiple_levels(embed_dims):
    native = _fixture(device=DEV, batch=1, queries=3, heads=2, embed_dims=embed_dims,
                      levels=((1, 2), (2, 1)), points=2)
    reference = _cpu_copy(native)
    actual = multi_scale_deformable_attn(*native, backend="hip")
    expected = msda_torch.msda_forward(reference[0], reference[1], reference[3], reference[4])
    grad = torch.linspace(0.1, 1.0, actual.numel(), device=DEV).view_as(actual)
    (actual * grad).sum().backward()
    (expected * grad.cpu()).sum().backward()
    for a, e in zip((native[0], native[3], native[4]), (reference[0], reference[3], reference[4])):
        torch.testing.assert_close(a.grad.cpu(), e.grad, rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_native_shape_and_dtype_coverage(dtype):
    tensors = _fixture(device=DEV, dtype=dtype, batch=1, queries=4, heads=2, embed_dims=4,
                       levels=((1, 2), (2, 1)), points=2)
    reference = _cpu_copy(tensors)
    expected = msda_torch.msda_forward(reference[0], reference[1], reference[3], reference[4])
    actual = multi_scale_deformable_attn(*tensors, backend="hip")
    assert actual.dtype == dtype
    tolerance = 1e-2 if dtype != torch.float32 else 1e-5
    torch.testing.assert_close(actual.float().cpu(), expected.detach(), rtol=tolerance,
                               atol=tolerance)


def test_native_bf16_reaches_the_kernel_as_bfloat16(monkeypatch):
    """The storage dtype survives to the C-ABI; gradient buffers are float32."""
    inner = msda_module._native_extension()
    assert inner is not None
    spy = _NativeCallSpy(inner)
    monkeypatch.setattr(msda_module, "_native_extension", lambda: spy)
    tensors = _fixture(device=DEV, dtype=torch.bfloat16, batch=1, queries=4, heads=2,
                       embed_dims=4, levels=((1, 2), (2, 1)), points=2)
    output = multi_scale_deformable_attn(*tensors, backend="hip")
    output.float().sum().backward()
    # this shape (4 channels) takes the atomic backward: no early binning
    assert [name for name, _ in spy.calls] == ["ms_deform_attn_forward", "ms_deform_attn_backward"]
    assert spy.calls[0][1][:6] == [torch.bfloat16, torch.int64, torch.int64, torch.bfloat16,
                                   torch.bfloat16, torch.bfloat16]
    assert spy.calls[1][1][5:9] == [torch.bfloat16, torch.float32, torch.float32, torch.float32]


def test_native_bf16_value_keeps_float32_geometry(monkeypatch):
    """float32 locations next to a bfloat16 value are not narrowed."""
    inner = msda_module._native_extension()
    spy = _NativeCallSpy(inner)
    monkeypatch.setattr(msda_module, "_native_extension", lambda: spy)
    value, shapes, starts, loc, attn = _fixture(device=DEV, batch=1, queries=4, heads=2,
                                                embed_dims=32, levels=((3, 5),), points=4)
    out = multi_scale_deformable_attn(value.detach().bfloat16(), shapes, starts, loc, attn,
                                      backend="hip")
    assert spy.calls[0][1][3:5] == [torch.float32, torch.float32]
    expected = msda_torch.msda_forward(value.detach().bfloat16().float().cpu(), shapes.cpu(),
                                       loc.detach().cpu(), attn.detach().cpu())
    torch.testing.assert_close(out.float().cpu(), expected, rtol=1e-2, atol=1e-2)


def test_native_bf16_matches_the_fp32_reference_forward_and_backward():
    clear_dispatch_report()
    native = _fixture(device=DEV, dtype=torch.bfloat16, batch=1, queries=4, heads=2,
                      embed_dims=4, levels=((1, 2), (2, 1)), points=2)
    reference = _cpu_copy(native)
    expected = msda_torch.msda_forward(reference[0], reference[1], reference[3], reference[4])
    actual = multi_scale_deformable_attn(*native, backend="hip")
    assert actual.dtype == torch.bfloat16
    report = get_last_dispatch_report()
    assert report.selected_backend == "hip"
    assert report.native_fallback is False
    grad = torch.linspace(0.1, 1.0, actual.numel(), device=DEV).view_as(actual)
    (actual.float() * grad).sum().backward()
    (expected * grad.cpu()).sum().backward()
    tolerance = 2e-2
    torch.testing.assert_close(actual.float().cpu(), expected.detach(), rtol=tolerance,
                               atol=tolerance)
    for index in (0, 3, 4):
        torch.testing.assert_close(native[index].grad.float().cpu(), reference[index].grad,
                                   rtol=tolerance, atol=tolerance)


def test_native_bf16_keeps_sampling_geometry_in_fp32():
    """Reference KAT: width 1000, loc 0.5 in bfloat16 -> exactly 2048, not 4096."""
    width, step = 1000, 4096.0
    value = torch.zeros(1, width, 1, 1, dtype=torch.bfloat16, device=DEV)
    value[:, width // 2:] = step
    value.requires_grad_(True)
    spatial_shapes = torch.tensor([[1, width]], dtype=torch.int64, device=DEV)
    level_start_index = torch.zeros(1, dtype=torch.int64, device=DEV)
    locations = torch.full((1, 1, 1, 1, 1, 2), 0.5, dtype=torch.bfloat16, device=DEV)
    weights = torch.ones(1, 1, 1, 1, 1, dtype=torch.bfloat16, device=DEV)
    actual = multi_scale_deformable_attn(value, spatial_shapes, level_start_index, locations,
                                         weights, backend="hip")
    assert actual.float().cpu().item() == 2048.0


def test_autograd_end_to_end_fp32_full_channel_layout():
    """Default C=32 / 8-head layout through autograd, against the oracle."""
    value, shapes, starts, loc, attn = _fixture(device=DEV, batch=2, queries=33, heads=8,
                                                embed_dims=32, levels=((6, 9), (3, 5), (2, 2)),
                                                points=4)
    ref = _cpu_copy((value, shapes, starts, loc, attn))
    out = multi_scale_deformable_attn(value, shapes, starts, loc, attn)
    expected = msda_torch.msda_forward(ref[0], ref[1], ref[3], ref[4])
    g = torch.randn(out.shape, generator=torch.Generator().manual_seed(1))
    (out * g.to(DEV)).sum().backward()
    (expected * g).sum().backward()
    torch.testing.assert_close(out.detach().cpu(), expected.detach(), rtol=1e-5, atol=1e-5)
    for a, e in zip((value, loc, attn), (ref[0], ref[3], ref[4])):
        torch.testing.assert_close(a.grad.cpu(), e.grad, rtol=1e-4, atol=1e-4)


def test_early_binning_matches_the_one_call_backward(monkeypatch):
    """The autograd function bins in its forward call (the forward kernel
    stores the backward's records); the result equals the one-call backward
    (MUSPACE_EARLY_BINNING=0), and a second backward (retain_graph) takes the
    one-call path."""
    def grads(early):
        monkeypatch.setenv("MUSPACE_EARLY_BINNING", "1" if early else "0")
        value, shapes, starts, loc, attn = _fixture(device=DEV, batch=2, queries=300, heads=8,
                                                    embed_dims=32, levels=((20, 30), (10, 15)),
                                                    points=4)
        out = multi_scale_deformable_attn(value, shapes, starts, loc, attn)
        g = torch.randn(out.shape, generator=torch.Generator().manual_seed(3)).to(DEV)
        (out * g).sum().backward(retain_graph=True)
        first = [t.grad.clone() for t in (value, loc, attn)]
        for t in (value, loc, attn):
            t.grad = None
        (out * g).sum().backward()
        second = [t.grad.clone() for t in (value, loc, attn)]
        return first, second

    early_first, early_second = grads(True)
    late_first, _ = grads(False)
    for a, b, c in zip(early_first, early_second, late_first):
        torch.testing.assert_close(a, c, rtol=1e-6, atol=1e-6)
        torch.testing.assert_close(b, c, rtol=1e-6, atol=1e-6)


def test_no_binning_when_no_graph_is_recorded(monkeypatch):
    """Under torch.no_grad() no backward can follow, so the forward starts no
    binning even though its inputs require gradients (a tile-path shape)."""
    monkeypatch.setenv("MUSPACE_EARLY_BINNING", "1")
    inner = msda_module._native_extension()
    spy = _NativeCallSpy(inner)
    monkeypatch.setattr(msda_module, "_native_extension", lambda: spy)
    tensors = _fixture(device=DEV, batch=1, queries=64, heads=2, embed_dims=32,
                       levels=((8, 12),), points=4)
    with torch.no_grad():
        multi_scale_deformable_attn(*tensors, backend="hip")
    assert [name for name, _ in spy.calls] == ["ms_deform_attn_forward"]
    spy.calls.clear()
    multi_scale_deformable_attn(*tensors, backend="hip")
    assert [name for name, _ in spy.calls] == ["ms_deform_attn_forward_bin"]


@pytest.mark.parametrize("embed_dims", [32, 3])
def test_split_backward_entry_points_match_the_one_call(embed_dims):
    """ms_deform_attn_backward_bin on a second stream, then _rest on the main
    stream, against ms_deform_attn_backward_ws (C = 3 takes the atomic path:
    nothing to bin, all of it in _rest)."""
    from muspace_amd.runtime.native import load_native_module

    lib = load_native_module()
    value, shapes, starts, loc, attn = _fixture(device=DEV, batch=2, queries=200, heads=4,
                                                embed_dims=embed_dims, levels=((16, 24), (8, 12)),
                                                points=4, requires_grad=False)
    grad = torch.randn((2, 200, 4 * embed_dims), generator=torch.Generator().manual_seed(4))
    grad = grad.to(DEV)

    def buffers():
        return (torch.empty(value.shape, device=DEV), torch.empty(loc.shape, device=DEV),
                torch.empty(attn.shape, device=DEV))

    ref = buffers()
    lib.ms_deform_attn_backward(value, shapes, starts, loc, attn, grad, *ref, 64)
    got = buffers()
    ws = lib.backward_workspace(value, loc)
    side = torch.cuda.Stream()
    ready = torch.cuda.Event()
    ready.record(torch.cuda.current_stream())
    side.wait_event(ready)
    lib.ms_deform_attn_backward_bin(value, shapes, starts, loc, attn, *got, 64, ws, stream=side)
    done = torch.cuda.Event()
    done.record(side)
    torch.cuda.current_stream().wait_event(done)
    lib.ms_deform_attn_backward_rest(value, shapes, starts, loc, attn, grad, *got, 64, ws)
    for a, b in zip(got, ref):
        torch.testing.assert_close(a, b, rtol=1e-6, atol=1e-6)


def test_early_binning_reservation_is_returned_after_the_backward(monkeypatch):
    """The bytes a forward reserves for its early-binned backward buffers are
    returned once the backward has consumed them, and a forward over the
    budget runs without early binning and still gets the same gradients."""
    monkeypatch.setenv("MUSPACE_EARLY_BINNING", "1")
    budget = msda_module.binning_budget
    index = torch.cuda.current_device()
    before = budget.held(index)
    tensors = _fixture(device=DEV, batch=2, queries=96, heads=2, embed_dims=32,
                       levels=((8, 12), (4, 6)), points=4)
    out = multi_scale_deformable_attn(*tensors, backend="hip")
    assert budget.held(index) > before  # the backward's buffers are held
    g = torch.randn(out.shape, generator=torch.Generator().manual_seed(5)).to(DEV)
    out.backward(g)
    del out
    assert budget.held(index) == before
    early = [t.grad.clone() for t in (tensors[0], tensors[3], tensors[4])]
    for t in (tensors[0], tensors[3], tensors[4]):
        t.grad = None
    tight = msda_module.BinningBudget(limit_of=lambda i: 0)
    monkeypatch.setattr(msda_module, "binning_budget", tight)
    out = multi_scale_deformable_attn(*tensors, backend="hip")
    assert tight.held(index) == 0
    out.backward(g)
    for a, t in zip(early, (tensors[0], tensors[3], tensors[4])):
        torch.testing.assert_close(t.grad, a, rtol=1e-6, atol=1e-6)
