"""MSDA with the attention softmax fused in (ms_deform_attn_forward_softmax and
its backward) on the GPU, against oracle/msda_softmax.py in float64 on the CPU.

Cases: one step per unit (L*P <= the unit's tap lanes) and several steps (the
online max/sum with rescaling), L*P not a power of two, channel counts 16, 32
and 64 (row kernels, tile backward) and 8 (the standalone softmax with the
generic forward and the atomic backward), 16-bit value storage, -inf logits,
and the operator with its early binning on and off. Every gradient buffer
starts as NaN, so an element the kernels fail to write fails the test.
Tolerances: fp32 forward 1e-5, gradients 1e-4; 16-bit storage 2e-2.
"""

from __future__ import annotations

import pytest
import torch

from conftest import gpu_available
from msda_testlib import level_starts
from muspace_amd.runtime.native import load_native_module
from oracle import msda_softmax

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not gpu_available(), reason="AMD GPU required"),
]

DEV = "cuda"
LEVELS = ((20, 30), (10, 15), (5, 8), (3, 4))


def _case(seed, *, batch=2, queries=70, heads=4, channels=32, levels=LEVELS, points=8):
    g = torch.Generator().manual_seed(seed)
    nv = sum(h * w for h, w in levels)
    value = torch.randn(batch, nv, heads, channels, generator=g)
    loc = torch.rand(batch, queries, heads, len(levels), points, 2, generator=g) * 1.2 - 0.1
    logits = torch.randn(batch, queries, heads, len(levels), points, generator=g) * 2.0
    grad = torch.randn(batch, queries, heads * channels, generator=g)
    shapes = torch.tensor(levels, dtype=torch.int64)
    return value, shapes, level_starts(levels), loc, logits, grad


def _native(value, shapes, starts, loc, logits, grad, vdt=torch.float32, gdt=torch.float32):
    lib = load_native_module()
    v = value.to(DEV, vdt).contiguous()
    lc, lg = loc.to(DEV, gdt).contiguous(), logits.to(DEV, gdt).contiguous()
    sh, st = shapes.to(DEV), starts.to(DEV)
    out = torch.empty((v.shape[0], lc.shape[1], v.shape[2] * v.shape[3]), dtype=vdt, device=DEV)
    lib.ms_deform_attn_forward_softmax(v, sh, st, lc, lg, out, 64)
    gv = torch.full(v.shape, float("nan"), device=DEV)
    gl = torch.full(lc.shape, float("nan"), device=DEV)
    glg = torch.full(lg.shape, float("nan"), device=DEV)
    lib.ms_deform_attn_backward_softmax(v, sh, st, lc, lg, grad.to(DEV, vdt).contiguous(), gv,
                                        gl, glg, 64)
    torch.cuda.synchronize()
    return [t.cpu().double() for t in (out, gv, gl, glg)]


def _oracle(value, shapes, loc, logits, grad, vdt=torch.float32, gdt=torch.float32):
    """The oracle on the inputs the kernels saw (rounded to their storage dtypes)."""
    as_seen = lambda t, dt: t.to(dt).double()  # noqa: E731
    out, gv, gl, glg = msda_softmax.forward_backward(
        as_seen(value, vdt), shapes, as_seen(loc, gdt), as_seen(logits, gdt), as_seen(grad, vdt)
    )
    return [out, gv, gl, glg]


def _assert_all(actual, expected, fwd_tol, bwd_tol, names=("out", "grad_value", "grad_loc",
                                                           "grad_logits")):
    for a, e, n in zip(actual, expected, names):
        if a is None:
            continue
        tol = fwd_tol if n == "out" else bwd_tol
        torch.testing.assert_close(a, e, rtol=tol, atol=tol, msg=lambda m, n=n: f"{n}: {m}")


@pytest.mark.parametrize(
    "channels,levels,points",
    [
        (32, LEVELS, 8),        # one step per unit (L*P = 32)
        (32, LEVELS, 32),       # two steps per unit: the online softmax rescales
        (16, LEVELS, 8),
        (64, LEVELS, 8),
        (32, LEVELS[:3], 5),    # L*P = 15, not a power of two
        (8, LEVELS, 4),         # standalone softmax, generic forward, atomic backward
    ],
)
def test_fp32_forward_and_backward_match_the_oracle(channels, levels, points):
    case = _case(channels * 100 + points, channels=channels, levels=levels, points=points)
    value, shapes, starts, loc, logits, grad = case
    _assert_all(_native(*case), _oracle(value, shapes, loc, logits, grad), 1e-5, 1e-4)


@pytest.mark.parametrize("vdt,gdt", [(torch.bfloat16, torch.float32),
                                     (torch.bfloat16, torch.bfloat16),
                                     (torch.float16, torch.float16)])
def test_16bit_storage_matches_the_oracle(vdt, gdt):
    case = _case(7)
    value, shapes, starts, loc, logits, grad = case
    _assert_all(_native(*case, vdt=vdt, gdt=gdt),
                _oracle(value, shapes, loc, logits, grad, vdt, gdt), 2e-2, 2e-2)


@pytest.mark.parametrize("vdt", [torch.bfloat16, torch.float16])
def test_16bit_c16_two_steps_per_unit(vdt):
    """16-bit values with C = 16 run two lanes per row (two samples per lane
    group and step), so L*P = 128 takes two steps per unit in the one-stage
    loop: the second step's online-softmax rescale must be the one its own
    tap computed (applying it before the tap used the step-before-last's)."""
    case = _case(8, channels=16, points=32)
    value, shapes, starts, loc, logits, grad = case
    _assert_all(_native(*case, vdt=vdt, gdt=torch.float32),
                _oracle(value, shapes, loc, logits, grad, vdt, torch.float32), 2e-2, 2e-2)


@pytest.mark.parametrize("early", [False, True], ids=["one-call", "forward-binning"])
def test_minus_infinity_logits(early):
    """Masked samples get weight zero; a unit whose logits are all -inf gives
    NaN, as torch.softmax does (its output row and its logit gradients);
    through the plain entries and through the forward that bins (whose records
    carry the probabilities)."""
    case = list(_case(9))
    logits = case[4]
    logits[0, 3, 1, 0, :] = float("-inf")       # one level masked
    logits[1, 5, 2, :, ::2] = float("-inf")     # every other point masked
    logits[1, 6, 0] = float("-inf")             # the whole unit
    value, shapes, starts, loc, logits, grad = case
    if early:
        (out, gv, gl, glg), fused = _native_early(*case)
        assert fused
    else:
        out, gv, gl, glg = _native(*case)
    e_out, e_gv, e_gl, e_glg = _oracle(value, shapes, loc, logits, grad)
    torch.testing.assert_close(out, e_out, rtol=1e-5, atol=1e-5, equal_nan=True)
    assert torch.isnan(out[1, 6, 0:32]).all() and torch.isfinite(out[1, 6, 32:]).all()
    keep = torch.ones(logits.shape[:3], dtype=torch.bool)
    keep[1, 6, 0] = False
    torch.testing.assert_close(glg[keep], e_glg[keep], rtol=1e-4, atol=1e-4)
    assert torch.isnan(glg[1, 6, 0]).all()


@pytest.mark.parametrize("early", ["1", "0"])
def test_operator_autograd_matches_the_oracle(early, monkeypatch):
    from muspace_amd import clear_dispatch_report, get_last_dispatch_report
    from muspace_amd.ops import multi_scale_deformable_attn_softmax

    monkeypatch.setenv("MUSPACE_EARLY_BINNING", early)
    value, shapes, starts, loc, logits, grad = _case(11)
    v, lc, lg = (t.to(DEV).requires_grad_(True) for t in (value, loc, logits))
    clear_dispatch_report()
    out = multi_scale_deformable_attn_softmax(v, shapes.to(DEV), starts.to(DEV), lc, lg)
    assert get_last_dispatch_report().selected_backend == "hip"
    out.backward(grad.to(DEV))
    expected = _oracle(value, shapes, loc, logits, grad)
    actual = [out.detach().cpu().double()] + [t.grad.cpu().double() for t in (v, lc, lg)]
    _assert_all(actual, expected, 1e-5, 1e-4)


def test_fused_equals_softmax_then_operator():
    """The fused forward against torch.softmax followed by the plain operator,
    both on the GPU: only the order of float32 roundings differs."""
    from muspace_amd.ops import (attention_softmax, multi_scale_deformable_attn,
                                 multi_scale_deformable_attn_softmax)

    value, shapes, starts, loc, logits, _ = _case(13, queries=300)
    args = [t.to(DEV) for t in (value, shapes, starts, loc)]
    fused = multi_scale_deformable_attn_softmax(*args, logits.to(DEV))
    plain = multi_scale_deformable_attn(*args, attention_softmax(logits.to(DEV)))
    torch.testing.assert_close(fused, plain, rtol=1e-5, atol=1e-6)


def _raw_backward_args(lib, value, shapes, starts, loc, logits, grad, gv, gl, glg):
    from muspace_amd.runtime.native import DTYPE_F32

    batch, spatial, heads, channels = value.shape
    return [value.data_ptr(), DTYPE_F32, shapes.data_ptr(), starts.data_ptr(), loc.data_ptr(),
            logits.data_ptr(), DTYPE_F32, grad.data_ptr(), gv.data_ptr(), gl.data_ptr(),
            glg.data_ptr(), batch, spatial, heads, channels, shapes.shape[0], loc.shape[1],
            loc.shape[4], 64]


def test_allocating_backward_export_matches_the_workspace_calls():
    """ms_deform_attn_backward_softmax (stream-ordered scratch) through the raw C-ABI
    against _bin + _rest on a caller workspace, on the tile path (C = 32) and the
    atomic path (C = 8)."""
    lib = load_native_module()
    for channels in (32, 8):
        value, shapes, starts, loc, logits, grad = (t.to(DEV) for t in _case(21, channels=channels))
        ref = [torch.empty(t.shape, device=DEV) for t in (value, loc, logits)]
        lib.ms_deform_attn_backward_softmax(value, shapes, starts, loc, logits, grad, *ref, 64)
        got = [torch.full(t.shape, float("nan"), device=DEV) for t in (value, loc, logits)]
        args = _raw_backward_args(lib, value, shapes, starts, loc, logits, grad, *got)
        rc = lib._raw["ms_deform_attn_backward_softmax"](
            *args, torch.cuda.current_stream().cuda_stream)
        assert rc == 0, lib._raw["muspace_last_error"]()
        torch.cuda.synchronize()
        for a, b in zip(got, ref):
            torch.testing.assert_close(a, b, rtol=1e-6, atol=1e-6)


def test_softmax_backward_parts_need_a_workspace():
    """The probabilities live in the workspace: _bin without one is MUSPACE_EINVAL
    (checked on the host; nothing is launched)."""
    lib = load_native_module()
    value, shapes, starts, loc, logits, grad = (t.to(DEV) for t in _case(22))
    bufs = [torch.empty(t.shape, device=DEV) for t in (value, loc, logits)]
    args = _raw_backward_args(lib, value, shapes, starts, loc, logits, grad, *bufs)
    rc = lib._raw["ms_deform_attn_backward_softmax_bin"](
        *args, None, 0, torch.cuda.current_stream().cuda_stream)
    assert rc == 1  # MUSPACE_EINVAL
    assert b"workspace" in lib._raw["muspace_last_error"]()


def _native_early(value, shapes, starts, loc, logits, grad, vdt=torch.float32,
                  gdt=torch.float32):
    """ms_deform_attn_forward_softmax_bin, then ms_deform_attn_backward_softmax_rest
    on its workspace (the operator's training path); also returns whether the
    forward kernel did the binning itself."""
    lib = load_native_module()
    v = value.to(DEV, vdt).contiguous()
    lc, lg = loc.to(DEV, gdt).contiguous(), logits.to(DEV, gdt).contiguous()
    sh, st = shapes.to(DEV), starts.to(DEV)
    out = torch.empty((v.shape[0], lc.shape[1], v.shape[2] * v.shape[3]), dtype=vdt, device=DEV)
    gv = torch.full(v.shape, float("nan"), device=DEV)
    gl = torch.full(lc.shape, float("nan"), device=DEV)
    glg = torch.full(lg.shape, float("nan"), device=DEV)
    ws = lib.backward_softmax_workspace(v, lc)
    lib.ms_deform_attn_forward_softmax_bin(v, sh, st, lc, lg, out, gv, gl, glg, 64, ws)
    lib.ms_deform_attn_backward_softmax_rest(v, sh, st, lc, lg, grad.to(DEV, vdt).contiguous(),
                                             gv, gl, glg, 64, ws)
    torch.cuda.synchronize()
    return [t.cpu().double() for t in (out, gv, gl, glg)], lib.forward_softmax_bin_fuses(v, lc)


EARLY = [
    # (channels, points, value dtype, geometry dtype, fused into the forward kernel)
    (32, 8, torch.float32, torch.float32, True),     # one step per unit
    (16, 8, torch.float32, torch.float32, True),
    (64, 8, torch.float32, torch.float32, True),
    (32, 8, torch.bfloat16, torch.float32, True),
    (32, 8, torch.bfloat16, torch.bfloat16, True),   # probabilities stored in bf16
    (32, 8, torch.float16, torch.float16, True),
    (32, 32, torch.float32, torch.float32, False),   # two steps per unit: the two calls
]


@pytest.mark.parametrize("channels,points,vdt,gdt,fused", EARLY,
                         ids=[f"c{c}-p{p}-{str(v)[6:]}-{str(g)[6:]}" for c, p, v, g, _ in EARLY])
def test_forward_softmax_bin_then_rest_matches_the_oracle(channels, points, vdt, gdt, fused):
    case = _case(31 + channels + points, channels=channels, points=points)
    value, shapes, starts, loc, logits, grad = case
    actual, did_fuse = _native_early(*case, vdt=vdt, gdt=gdt)
    assert did_fuse == fused
    tol = (1e-5, 1e-4) if vdt == torch.float32 else (2e-2, 2e-2)
    _assert_all(actual, _oracle(value, shapes, loc, logits, grad, vdt, gdt), *tol)


def test_forward_softmax_bin_at_c2_matches_the_oracle():
    """The BASELINE c2 shape with logits (the bench's softmax leg), through the
    fused forward-binning call and the rest of the backward: output and the
    location and logit gradients on 48 seeded queries against the float32 oracle,
    grad_value through the adjoint identity <grad_out, out> = <value, grad_value>
    at full size, and every gradient element written."""
    from muspace_amd.workloads import CONFIGS, make_inputs

    cfg = CONFIGS["c2"]
    t = make_inputs(cfg, value_dtype=torch.float32)
    g = torch.Generator().manual_seed(5)
    logits = torch.randn(t["attention_weights"].shape, generator=g)
    grad = t["grad_output"]
    lib = load_native_module()
    v = t["value"].to(DEV)
    lc, lg = t["sampling_locations"].to(DEV), logits.to(DEV)
    assert lib.forward_softmax_bin_fuses(v, lc)
    sh, st = t["spatial_shapes"].to(DEV), t["level_start_index"].to(DEV)
    out = torch.empty((cfg.batch, cfg.queries, cfg.heads * cfg.channels), device=DEV)
    gv, gl, glg = (torch.full(x.shape, float("nan"), device=DEV) for x in (v, lc, lg))
    ws = lib.backward_softmax_workspace(v, lc)
    print("[softmax] c2 forward_softmax_bin + rest", flush=True)
    lib.ms_deform_attn_forward_softmax_bin(v, sh, st, lc, lg, out, gv, gl, glg, 64, ws)
    gd = grad.to(DEV)
    lib.ms_deform_attn_backward_softmax_rest(v, sh, st, lc, lg, gd, gv, gl, glg, 64, ws)
    torch.cuda.synchronize()
    assert torch.isfinite(gv).all() and torch.isfinite(gl).all() and torch.isfinite(glg).all()
    idx = torch.randperm(cfg.queries, generator=torch.Generator().manual_seed(7))[:48]
    idx = idx.sort().values
    # the oracle in float32, as the kernels compute the sampling coordinates:
    # they follow grid_sample's float32 arithmetic, and against float64 the
    # rounding of a bilinear fraction (about 1e-5 at W = 200) exceeds the
    # 1e-4 absolute tolerance wherever a location gradient nearly cancels
    e_out, _, e_gl, e_glg = msda_softmax.forward_backward(
        t["value"], t["spatial_shapes"], t["sampling_locations"][:, idx], logits[:, idx],
        grad[:, idx])
    e_out, e_gl, e_glg = (x.double() for x in (e_out, e_gl, e_glg))
    _assert_all([out.cpu()[:, idx].double(), None, gl.cpu()[:, idx].double(),
                 glg.cpu()[:, idx].double()], [e_out, None, e_gl, e_glg], 1e-5, 1e-4,
                names=("out", "skip", "grad_loc", "grad_logits"))
    lhs = float((out.double() * gd.double()).sum())
    rhs = float((v.double() * gv.double()).sum())
    scale = float((out.double().abs() * gd.double().abs()).sum())
    assert abs(lhs - rhs) <= 1e-5 * scale, (lhs, rhs, scale)
