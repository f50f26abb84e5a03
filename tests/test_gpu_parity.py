"""Parity of the HIP kernels with the oracle, called through the C-ABI.

Tolerances (torch.testing.assert_close semantics, |a-e| <= atol + rtol*|e|):
  float32 forward 1e-5, float32 backward 1e-4 (atomic accumulation order is
  nondeterministic), float16/bfloat16 value 1e-2 against the float32 oracle
  evaluated on the same 16-bit-quantised value.

Full BASELINE shapes are checked on a seeded subset of queries (every query's
output and location/weight gradients depend only on that query, so the oracle
on the subset is exact), grad_value with grad_output masked to that subset,
and at full size through the adjoint identities <g, out> = <value, dvalue> =
<attn, dattn>, which hold because MSDA is linear in value and in attention.
"""

from __future__ import annotations

import pytest
import torch

from conftest import gpu_available
from msda_testlib import level_starts, max_violation
from muspace_amd.workloads import CONFIGS, make_inputs
from oracle import msda_torch

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not gpu_available(), reason="AMD GPU required"),
]

DEV = "cuda"
TOL = {torch.float32: (1e-5, 1e-4), torch.float16: (1e-2, 1e-2), torch.bfloat16: (1e-2, 1e-2)}


def _assert_close(actual, expected, tol, what):
    actual = actual.detach().double().cpu()
    expected = expected.detach().double().cpu()
    viol = max_violation(actual.numpy(), expected.numpy(), tol, tol)
    assert viol <= 0, (
        f"{what}: max |diff| {float((actual - expected).abs().max()):.3e} exceeds tolerance {tol}"
    )


def run_forward(lib, t, value_dtype, geometry_dtype, im2col_step=64):
    value = t["value"].to(value_dtype).to(DEV).contiguous()
    loc = t["sampling_locations"].to(geometry_dtype).to(DEV).contiguous()
    attn = t["attention_weights"].to(geometry_dtype).to(DEV).contiguous()
    shapes, starts = t["spatial_shapes"].to(DEV), t["level_start_index"].to(DEV)
    out = torch.empty((value.shape[0], loc.shape[1], value.shape[2] * value.shape[3]),
                      dtype=value_dtype, device=DEV)
    lib.ms_deform_attn_forward(value, shapes, starts, loc, attn, out, im2col_step)
    return out


def run_backward(lib, t, grad, value_dtype, geometry_dtype, im2col_step=64):
    value = t["value"].to(value_dtype).to(DEV).contiguous()
    loc = t["sampling_locations"].to(geometry_dtype).to(DEV).contiguous()
    attn = t["attention_weights"].to(geometry_dtype).to(DEV).contiguous()
    shapes, starts = t["spatial_shapes"].to(DEV), t["level_start_index"].to(DEV)
    # poisoned: every element of all three gradients must be overwritten
    gv = torch.full(value.shape, float("nan"), dtype=torch.float32, device=DEV)
    gl = torch.full(loc.shape, float("nan"), dtype=torch.float32, device=DEV)
    ga = torch.full(attn.shape, float("nan"), dtype=torch.float32, device=DEV)
    lib.ms_deform_attn_backward(value, shapes, starts, loc, attn,
                                grad.to(value_dtype).to(DEV).contiguous(), gv, gl, ga,
                                im2col_step)
    return gv, gl, ga


def run_fused(lib, t, grad, value_dtype, geometry_dtype, im2col_step=64):
    """ms_deform_attn_forward_bin (the forward kernel stores the backward's
    records), then ms_deform_attn_backward_rest: output and gradients."""
    value = t["value"].to(value_dtype).to(DEV).contiguous()
    loc = t["sampling_locations"].to(geometry_dtype).to(DEV).contiguous()
    attn = t["attention_weights"].to(geometry_dtype).to(DEV).contiguous()
    shapes, starts = t["spatial_shapes"].to(DEV), t["level_start_index"].to(DEV)
    # poisoned: every element of the output and all three gradients must be
    # overwritten
    out = torch.full((value.shape[0], loc.shape[1], value.shape[2] * value.shape[3]),
                     float("nan"), dtype=value_dtype, device=DEV)
    gv = torch.full(value.shape, float("nan"), dtype=torch.float32, device=DEV)
    gl = torch.full(loc.shape, float("nan"), dtype=torch.float32, device=DEV)
    ga = torch.full(attn.shape, float("nan"), dtype=torch.float32, device=DEV)
    ws = lib.backward_workspace(value, loc)
    lib.ms_deform_attn_forward_bin(value, shapes, starts, loc, attn, out, gv, gl, ga,
                                   im2col_step, ws)
    lib.ms_deform_attn_backward_rest(value, shapes, starts, loc, attn,
                                     grad.to(value_dtype).to(DEV).contiguous(), gv, gl, ga,
                                     im2col_step, ws)
    return out, gv, gl, ga


def oracle_inputs(t, value_dtype, geometry_dtype):
    """The oracle sees exactly what the kernel reads, upcast to float32."""
    return (
        t["value"].to(value_dtype).float().cpu(),
        t["spatial_shapes"].cpu(),
        t["sampling_locations"].to(geometry_dtype).float().cpu(),
        t["attention_weights"].to(geometry_dtype).float().cpu(),
    )


def small_case(seed, batch, queries, heads, channels, levels, points, lo=-0.1, hi=1.1):
    g = torch.Generator().manual_seed(seed)
    L, nv = len(levels), sum(h * w for h, w in levels)
    logits = torch.randn(batch, queries, heads, L * points, generator=g)
    t = {
        "value": torch.randn(batch, nv, heads, channels, generator=g),
        "spatial_shapes": torch.tensor(levels, dtype=torch.int64),
        "level_start_index": level_starts(levels),
        "sampling_locations": torch.rand(batch, queries, heads, L, points, 2, generator=g)
        * (hi - lo) + lo,
        "attention_weights": torch.softmax(logits, -1).view(batch, queries, heads, L, points),
    }
    grad = torch.randn(batch, queries, heads * channels, generator=g)
    return t, grad


# (batch, queries, heads, channels, levels, points): reference test shapes
# (odd channels, generic kernels) and row-kernel shapes covering every
# samples-per-query layout (L*P = 1, 2, 3, 4, 5, 8, 12, 16, 32, 40, 64), and
# L*P = 256, where a binning chunk (256 queries) holds 65536 samples, past
# bin_count's 16-bit histogram counters.
SMALL = [
    (1, 5, 2, 3, ((2, 2),), 4),
    (2, 3, 4, 2, ((1, 3), (2, 1)), 2),
    (1, 7, 1, 8, ((1, 1), (1, 2), (2, 2)), 3),
    (1, 4, 2, 4, ((1, 2), (2, 1)), 2),
    (2, 37, 8, 32, ((9, 13),), 1),
    (2, 29, 8, 32, ((9, 13),), 2),
    (1, 31, 3, 32, ((5, 4), (3, 3), (2, 2)), 1),
    (2, 23, 8, 32, ((17, 11),), 4),
    (1, 19, 5, 32, ((6, 7),), 5),
    (3, 17, 8, 32, ((8, 9), (4, 5)), 4),
    (1, 13, 8, 32, ((12, 7), (6, 4), (3, 2)), 4),
    (2, 11, 8, 32, ((10, 12), (5, 6), (3, 3), (2, 2)), 4),
    (2, 9, 8, 32, ((10, 12), (5, 6), (3, 3), (2, 2)), 8),
    (1, 7, 4, 32, ((10, 12), (5, 6), (3, 3), (2, 2), (1, 1)), 8),
    (1, 5, 2, 32, ((10, 12), (5, 6), (3, 3), (2, 2)), 16),
    (2, 21, 8, 16, ((9, 10), (4, 5)), 4),
    (2, 21, 4, 64, ((9, 10), (4, 5)), 4),
    (1, 15, 8, 12, ((9, 10), (4, 5)), 4),
    (1, 300, 2, 32, ((10, 12), (5, 6), (3, 3), (2, 2)), 64),
]
DTYPES = [
    (torch.float32, torch.float32),
    (torch.bfloat16, torch.float32),
    (torch.bfloat16, torch.bfloat16),
    (torch.float16, torch.float32),
    (torch.float16, torch.float16),
]


def _id(case):
    b, q, m, c, lv, p = case
    return f"b{b}q{q}m{m}c{c}L{len(lv)}P{p}"


@pytest.mark.parametrize("dtypes", DTYPES, ids=lambda d: f"{d[0]}-{d[1]}".replace("torch.", ""))
@pytest.mark.parametrize("case", SMALL, ids=_id)
def test_small_shapes_match_oracle(native_lib, case, dtypes):
    value_dtype, geometry_dtype = dtypes
    t, grad = small_case(sum(case[:4]), *case)
    out = run_forward(native_lib, t, value_dtype, geometry_dtype)
    gv, gl, ga = run_backward(native_lib, t, grad, value_dtype, geometry_dtype)
    torch.cuda.synchronize()
    o_out, o_gv, o_gl, o_ga = msda_torch.msda_forward_backward(
        *oracle_inputs(t, value_dtype, geometry_dtype), grad.to(value_dtype).float()
    )
    ftol, btol = TOL[value_dtype]
    _assert_close(out, o_out, ftol, "output")
    _assert_close(gv, o_gv, btol, "grad_value")
    _assert_close(gl, o_gl, btol, "grad_sampling_locations")
    _assert_close(ga, o_ga, btol, "grad_attention_weights")


# Binning-boundary shapes, small enough for the full oracle: several binning
# chunks per (b, m) slab (chunk = max(256, 4096 / pow2(L*P)) queries) with a
# ragged last chunk that also ends inside a sub-chunk (2048 / pow2(L*P)
# queries), and L*P = 3, 5, 6 so that padded sample slots sit inside every
# sub-chunk. Shapes: L*P = 3 -> 1024-query chunks, 512-query sub-chunks,
# 2600 = 2 x 1024 + 552; L*P = 5 -> 512 and 256, 1300 = 2 x 512 + 276;
# L*P = 6 on C = 16 and 64 tiles.
MEDIUM = [
    (1, 2600, 2, 32, ((20, 30), (10, 15), (5, 8)), 1),
    (2, 1300, 2, 32, ((16, 24),), 5),
    (1, 1100, 2, 16, ((12, 18), (6, 9), (3, 5)), 2),
    (1, 1100, 2, 64, ((12, 18), (6, 9), (3, 5)), 2),
]


@pytest.mark.parametrize("dtypes", DTYPES[:2], ids=lambda d: f"{d[0]}-{d[1]}".replace("torch.", ""))
@pytest.mark.parametrize("case", MEDIUM, ids=_id)
def test_binning_chunk_boundaries_match_oracle(native_lib, case, dtypes):
    value_dtype, geometry_dtype = dtypes
    print(f"[parity] medium {_id(case)} {value_dtype}", flush=True)
    t, grad = small_case(sum(case[:4]), *case)
    out = run_forward(native_lib, t, value_dtype, geometry_dtype)
    gv, gl, ga = run_backward(native_lib, t, grad, value_dtype, geometry_dtype)
    torch.cuda.synchronize()
    o_out, o_gv, o_gl, o_ga = msda_torch.msda_forward_backward(
        *oracle_inputs(t, value_dtype, geometry_dtype), grad.to(value_dtype).float()
    )
    ftol, btol = TOL[value_dtype]
    _assert_close(out, o_out, ftol, "output")
    _assert_close(gv, o_gv, btol, "grad_value")
    _assert_close(gl, o_gl, btol, "grad_sampling_locations")
    _assert_close(ga, o_ga, btol, "grad_attention_weights")


# The fused forward + binning (ms_deform_attn_forward_bin, then _rest) on
# small and medium shapes against the full oracle: every row-kernel channel
# count, ragged last forward chunks (L*P = 3: 64-query chunks, 1000 = 15 x 64
# + 40), one chunk shorter than a block, samples outside their level (zero
# gradients written by the forward), a single dense tile split into several
# work items (3 x 4 level, 24000 records per slab), and 16-bit values with
# float32 or 16-bit geometry.
FUSED = [
    (2, 23, 8, 32, ((17, 11),), 4),
    (3, 17, 8, 32, ((8, 9), (4, 5)), 4),
    (2, 9, 8, 32, ((10, 12), (5, 6), (3, 3), (2, 2)), 8),
    (1, 5, 2, 32, ((10, 12), (5, 6), (3, 3), (2, 2)), 16),
    (2, 21, 8, 16, ((9, 10), (4, 5)), 4),
    (2, 21, 4, 64, ((9, 10), (4, 5)), 4),
    (1, 1000, 2, 32, ((20, 30), (10, 15), (5, 8)), 1),
    (1, 300, 8, 32, ((20, 30), (10, 15), (5, 8), (3, 4)), 8),
    (2, 3000, 1, 32, ((3, 4),), 8),
    (1, 1100, 2, 16, ((12, 18), (6, 9), (3, 5)), 2),
    (1, 1100, 2, 64, ((12, 18), (6, 9), (3, 5)), 2),
]


@pytest.mark.parametrize("dtypes", DTYPES, ids=lambda d: f"{d[0]}-{d[1]}".replace("torch.", ""))
@pytest.mark.parametrize("case", FUSED, ids=_id)
def test_fused_forward_binning_matches_oracle(native_lib, case, dtypes):
    value_dtype, geometry_dtype = dtypes
    print(f"[parity] fused {_id(case)} {value_dtype}/{geometry_dtype}", flush=True)
    t, grad = small_case(sum(case[:4]), *case)
    out, gv, gl, ga = run_fused(native_lib, t, grad, value_dtype, geometry_dtype)
    plain = run_forward(native_lib, t, value_dtype, geometry_dtype)
    torch.cuda.synchronize()
    o_out, o_gv, o_gl, o_ga = msda_torch.msda_forward_backward(
        *oracle_inputs(t, value_dtype, geometry_dtype), grad.to(value_dtype).float()
    )
    ftol, btol = TOL[value_dtype]
    _assert_close(out, plain, 1e-6, "output against the plain forward")
    _assert_close(out, o_out, ftol, "output")
    _assert_close(gv, o_gv, btol, "grad_value")
    _assert_close(gl, o_gl, btol, "grad_sampling_locations")
    _assert_close(ga, o_ga, btol, "grad_attention_weights")


def test_fused_forward_binning_records_path_matches_oracle(native_lib):
    """A slab span of queries x L*P x 12 bytes above 8 MB: the tile kernel
    stores the location and weight gradients over the records and
    msda_grad_gather copies them into sample order through the sample ->
    record index, so ms_deform_attn_forward_bin runs the plain forward and
    the binning kernels instead of the fused forward."""
    case = (1, 22000, 2, 32, ((20, 30),), 32)
    print(f"[parity] fused records path {_id(case)}", flush=True)
    t, grad = small_case(91, *case)
    assert not native_lib.forward_bin_fuses(t["value"], t["sampling_locations"])
    out, gv, gl, ga = run_fused(native_lib, t, grad, torch.float32, torch.float32)
    torch.cuda.synchronize()
    o_out, o_gv, o_gl, o_ga = msda_torch.msda_forward_backward(
        *oracle_inputs(t, torch.float32, torch.float32), grad
    )
    _assert_close(out, o_out, 1e-5, "output")
    _assert_close(gv, o_gv, 1e-4, "grad_value")
    _assert_close(gl, o_gl, 1e-4, "grad_sampling_locations")
    _assert_close(ga, o_ga, 1e-4, "grad_attention_weights")


def test_im2col_step_chunking_has_no_numeric_effect(native_lib):
    t, grad = small_case(5, 4, 9, 8, 32, ((6, 7), (3, 4)), 4)
    out_a = run_forward(native_lib, t, torch.float32, torch.float32, im2col_step=64)
    out_b = run_forward(native_lib, t, torch.float32, torch.float32, im2col_step=2)
    assert torch.equal(out_a, out_b)
    with pytest.raises(RuntimeError, match="not divisible by im2col_step"):
        run_forward(native_lib, t, torch.float32, torch.float32, im2col_step=3)


def test_unaligned_views_take_the_generic_path(native_lib):
    """A value view at an odd element offset is still computed correctly."""
    t, grad = small_case(8, 1, 11, 8, 32, ((6, 7),), 4)
    value = t["value"].to(DEV)
    big = torch.empty(value.numel() + 1, device=DEV)
    view = big[1:].view_as(value)
    view.copy_(value)
    loc = t["sampling_locations"].to(DEV)
    attn = t["attention_weights"].to(DEV)
    out = torch.empty((1, 11, 256), device=DEV)
    native_lib.ms_deform_attn_forward(view, t["spatial_shapes"].to(DEV),
                                      t["level_start_index"].to(DEV), loc, attn, out, 64)
    expect = msda_torch.msda_forward(t["value"], t["spatial_shapes"], t["sampling_locations"],
                                     t["attention_weights"])
    _assert_close(out, expect, 1e-5, "output")


def test_out_of_range_locations_give_zero(native_lib):
    t, grad = small_case(3, 2, 6, 8, 32, ((5, 6), (2, 3)), 4)
    t["sampling_locations"].fill_(-1.0)
    out = run_forward(native_lib, t, torch.float32, torch.float32)
    gv, gl, ga = run_backward(native_lib, t, grad, torch.float32, torch.float32)
    for x in (out, gv, gl, ga):
        assert torch.count_nonzero(x) == 0


@pytest.mark.parametrize("path", ["one_call", "fused"])
@pytest.mark.parametrize("value_dtype", [torch.float32, torch.bfloat16])
def test_nan_locations_drop_the_sample(native_lib, path, value_dtype):
    """A sample whose location has a NaN (or infinite) coordinate is dropped, as the
    reference kernel's bounds test (h_im > -1 && ... false for NaN) drops it
    (ms_deform_attn_musa_kernel.muh:289 forward, skipped samples' location
    and weight gradients stored as 0 in the backward): it adds nothing to the
    output or grad_value and gets zero location and weight gradients, while
    every other sample matches the oracle. The oracle (grid_sample) would
    give NaN gradients there, so it runs on the same inputs with those
    samples' weights zeroed (and a finite stand-in location)."""
    t, grad = small_case(11, 2, 37, 8, 32, ((10, 12), (5, 6), (3, 3), (2, 2)), 4)
    g = torch.Generator().manual_seed(5)
    loc = t["sampling_locations"]
    drop = torch.rand(loc.shape[:-1], generator=g) < 0.1
    which = torch.randint(0, 3, loc.shape[:-1], generator=g)  # x, y or both
    # NaN for most dropped samples, +inf or -inf for some
    bad = torch.full(loc.shape[:-1], torch.nan)
    kind = torch.randint(0, 4, loc.shape[:-1], generator=g)
    bad = torch.where(kind == 2, torch.inf, torch.where(kind == 3, -torch.inf, bad))
    loc[..., 0] = torch.where(drop & (which != 1), bad, loc[..., 0])
    loc[..., 1] = torch.where(drop & (which != 0), bad, loc[..., 1])
    geometry = torch.float32
    if path == "one_call":
        out = run_forward(native_lib, t, value_dtype, geometry)
        gv, gl, ga = run_backward(native_lib, t, grad, value_dtype, geometry)
    else:
        out, gv, gl, ga = run_fused(native_lib, t, grad, value_dtype, geometry)
    torch.cuda.synchronize()
    masked = dict(t)
    masked["sampling_locations"] = torch.where(drop[..., None], 0.5, loc)
    masked["attention_weights"] = torch.where(drop, 0.0, t["attention_weights"])
    o_out, o_gv, o_gl, o_ga = msda_torch.msda_forward_backward(
        *oracle_inputs(masked, value_dtype, geometry), grad.to(value_dtype).float()
    )
    o_ga = torch.where(drop, 0.0, o_ga)  # dropped samples: zero weight gradient
    ftol, btol = TOL[value_dtype]
    _assert_close(out, o_out, ftol, "output")
    _assert_close(gv, o_gv, btol, "grad_value")
    _assert_close(gl, o_gl, btol, "grad_sampling_locations")
    _assert_close(ga, o_ga, btol, "grad_attention_weights")
    assert torch.count_nonzero(gl.cpu()[drop]) == 0
    assert torch.count_nonzero(ga.cpu()[drop]) == 0


def _random_case(seed):
    """A seeded random shape: 1-3 batch entries, 1-300 queries, 1-8 heads,
    channels for the row kernels (16, 32, 64) and the generic ones, 1-5
    levels of 1-40 cells a side, 1-8 points, locations in [-0.2, 1.2]."""
    r = torch.Generator().manual_seed(1000 + seed)
    pick = lambda lo, hi: int(torch.randint(lo, hi + 1, (1,), generator=r))
    channels = (4, 8, 12, 16, 32, 64, 48, 32, 16)[pick(0, 8)]
    levels = tuple((pick(1, 40), pick(1, 40)) for _ in range(pick(1, 5)))
    case = (pick(1, 3), pick(1, 300), pick(1, 8), channels, levels, pick(1, 8))
    return case, DTYPES[seed % len(DTYPES)]


@pytest.mark.parametrize("path", ["one_call", "fused"])
@pytest.mark.parametrize("seed", range(16))
def test_random_shapes_match_oracle(native_lib, seed, path):
    case, (value_dtype, geometry_dtype) = _random_case(seed)
    t, grad = small_case(seed, *case, lo=-0.2, hi=1.2)
    if path == "one_call":
        out = run_forward(native_lib, t, value_dtype, geometry_dtype)
        gv, gl, ga = run_backward(native_lib, t, grad, value_dtype, geometry_dtype)
    else:
        out, gv, gl, ga = run_fused(native_lib, t, grad, value_dtype, geometry_dtype)
    torch.cuda.synchronize()
    o_out, o_gv, o_gl, o_ga = msda_torch.msda_forward_backward(
        *oracle_inputs(t, value_dtype, geometry_dtype), grad.to(value_dtype).float()
    )
    ftol, btol = TOL[value_dtype]
    what = f"{_id(case)} {value_dtype}/{geometry_dtype}"
    _assert_close(out, o_out, ftol, f"output {what}")
    _assert_close(gv, o_gv, btol, f"grad_value {what}")
    _assert_close(gl, o_gl, btol, f"grad_sampling_locations {what}")
    _assert_close(ga, o_ga, btol, f"grad_attention_weights {what}")


@pytest.mark.parametrize("path", ["one_call", "fused"])
def test_value_past_2gib_takes_the_wide_paths(native_lib, path):
    """A value tensor over 2 GiB: the row kernels and the tile backward address
    value with 32-bit buffer offsets, so the host takes the generic forward
    and the atomic backward (64-bit slab offsets), and the fused entry its
    two-call fallback. Each batch entry's output and gradients depend on its
    own value slab alone, so the oracle runs on a few entries, the last of
    them past the 2 GiB mark."""
    levels = ((32, 32), (16, 16), (8, 8), (4, 4))
    batch, queries, heads, channels, points = 1600, 2, 8, 32, 4
    nv = sum(h * w for h, w in levels)
    assert batch * nv * heads * channels * 4 > 2**31
    gen = torch.Generator(device=DEV).manual_seed(17)
    L = len(levels)
    t = {
        "value": torch.randn(batch, nv, heads, channels, device=DEV, generator=gen),
        "spatial_shapes": torch.tensor(levels, dtype=torch.int64),
        "level_start_index": level_starts(levels),
        "sampling_locations": torch.rand(batch, queries, heads, L, points, 2, device=DEV,
                                         generator=gen) * 1.2 - 0.1,
        "attention_weights": torch.softmax(
            torch.randn(batch, queries, heads, L * points, device=DEV, generator=gen), -1
        ).view(batch, queries, heads, L, points),
    }
    grad = torch.randn(batch, queries, heads * channels, device=DEV, generator=gen)
    if path == "one_call":
        out = run_forward(native_lib, t, torch.float32, torch.float32)
        gv, gl, ga = run_backward(native_lib, t, grad, torch.float32, torch.float32)
    else:
        out, gv, gl, ga = run_fused(native_lib, t, grad, torch.float32, torch.float32)
    torch.cuda.synchronize()
    for b in (0, 777, batch - 1):
        sl = slice(b, b + 1)
        o_out, o_gv, o_gl, o_ga = msda_torch.msda_forward_backward(
            t["value"][sl].cpu(), t["spatial_shapes"], t["sampling_locations"][sl].cpu(),
            t["attention_weights"][sl].cpu(), grad[sl].cpu()
        )
        _assert_close(out[sl], o_out, 1e-5, f"output[{b}]")
        _assert_close(gv[sl], o_gv, 1e-4, f"grad_value[{b}]")
        _assert_close(gl[sl], o_gl, 1e-4, f"grad_sampling_locations[{b}]")
        _assert_close(ga[sl], o_ga, 1e-4, f"grad_attention_weights[{b}]")


@pytest.mark.parametrize("value_dtype", [torch.float32, torch.bfloat16])
def test_half_pixel_known_answer_2048(native_lib, value_dtype):
    """Reference KAT (tests/ops/test_multi_scale_deformable_attn.py:430-468)."""
    width = 1000
    value = torch.zeros(1, width, 1, 32)
    value[:, width // 2:] = 4096.0
    t = {
        "value": value,
        "spatial_shapes": torch.tensor([[1, width]]),
        "level_start_index": torch.zeros(1, dtype=torch.int64),
        "sampling_locations": torch.full((1, 1, 1, 1, 1, 2), 0.5),
        "attention_weights": torch.ones(1, 1, 1, 1, 1),
    }
    geometry = torch.float32 if value_dtype == torch.float32 else value_dtype
    out = run_forward(native_lib, t, value_dtype, geometry)
    assert torch.all(out.float().cpu() == 2048.0)


def test_inconsistent_level_metadata_reads_nothing_out_of_bounds(native_lib):
    """A level that claims more cells than value holds contributes zero."""
    t, grad = small_case(4, 1, 8, 8, 32, ((4, 5), (2, 3)), 4, lo=0.1, hi=0.9)
    bogus = dict(t)
    bogus["spatial_shapes"] = torch.tensor([[4, 5], [200, 300]])
    out = run_forward(native_lib, bogus, torch.float32, torch.float32)
    only_first = dict(t)
    only_first["attention_weights"] = t["attention_weights"].clone()
    only_first["attention_weights"][:, :, :, 1] = 0
    expect = msda_torch.msda_forward(t["value"], t["spatial_shapes"], t["sampling_locations"],
                                     only_first["attention_weights"])
    _assert_close(out, expect, 1e-5, "output")


def test_add_one_smoke(native_lib):
    """Mirrors /root/reference/tests/test_extension.py:5-16."""
    value = torch.arange(4, dtype=torch.float32, device=DEV)
    actual = torch.empty_like(value)
    native_lib.add_one(value, actual)
    torch.testing.assert_close(actual.cpu(), torch.arange(1, 5, dtype=torch.float32))


# ------------------------------------------------------ BASELINE configs ---


def test_c0_full_oracle(native_lib):
    """BASELINE c0 (bs 1, 1000 queries, levels 32x32..4x4, 4 points, float32;
    locations U(-0.05, 1.05), so samples leave the levels): the HIP forward
    against the oracle on every query at 1e-5, and the backward (c0 names the
    forward only; the gradients are checked as well, at 1e-4)."""
    cfg = CONFIGS["c0"]
    print(f"[parity] c0 bs={cfg.batch} nq={cfg.queries}", flush=True)
    t = make_inputs(cfg, value_dtype=torch.float32)
    grad = t.pop("grad_output")
    out = run_forward(native_lib, t, torch.float32, torch.float32)
    gv, gl, ga = run_backward(native_lib, t, grad, torch.float32, torch.float32)
    torch.cuda.synchronize()
    o_out, o_gv, o_gl, o_ga = msda_torch.msda_forward_backward(
        t["value"], t["spatial_shapes"], t["sampling_locations"], t["attention_weights"], grad)
    _assert_close(out, o_out, 1e-5, "c0 output")
    _assert_close(gv, o_gv, 1e-4, "c0 grad_value")
    _assert_close(gl, o_gl, 1e-4, "c0 grad_sampling_locations")
    _assert_close(ga, o_ga, 1e-4, "c0 grad_attention_weights")
    outside = ((t["sampling_locations"] < 0) | (t["sampling_locations"] > 1)).any(-1)
    assert outside.float().mean() > 0.05  # the zero-padding path is exercised


FULL = [
    ("c1", torch.float32, torch.float32),
    ("c2", torch.float32, torch.float32),
    ("c3", torch.float32, torch.float32),
    ("c4", torch.bfloat16, torch.float32),
    ("c4", torch.float16, torch.float32),
    ("bevformer-1l", torch.float32, torch.float32),
    ("bevformer-1l", torch.bfloat16, torch.float32),
]
SUBSET = 48  # queries per config checked against the oracle


@pytest.mark.parametrize("name,value_dtype,geometry_dtype", FULL,
                         ids=[f"{n}-{str(v).replace('torch.', '')}" for n, v, _ in FULL])
def test_full_config_parity(native_lib, name, value_dtype, geometry_dtype):
    _check_full_config(native_lib, name, value_dtype, geometry_dtype, fused=False)


# The fused forward + binning at full size, at every config the bench times
# through it: float32 (c1, c2, c3) and both 16-bit value types (c4).
FULL_FUSED = [
    ("c1", torch.float32, torch.float32),
    ("c2", torch.float32, torch.float32),
    ("c3", torch.float32, torch.float32),
    ("c4", torch.bfloat16, torch.float32),
    ("c4", torch.float16, torch.float32),
]


@pytest.mark.parametrize("name,value_dtype,geometry_dtype", FULL_FUSED,
                         ids=[f"{n}-{str(v).replace('torch.', '')}" for n, v, _ in FULL_FUSED])
def test_full_config_parity_fused_binning(native_lib, name, value_dtype, geometry_dtype):
    _check_full_config(native_lib, name, value_dtype, geometry_dtype, fused=True)


def _check_full_config(native_lib, name, value_dtype, geometry_dtype, fused):
    cfg = CONFIGS[name]
    print(f"[parity] {name} {value_dtype} bs={cfg.batch} nq={cfg.queries} fused={fused}",
          flush=True)
    t = make_inputs(cfg, value_dtype=torch.float32)
    grad = t.pop("grad_output")
    if fused:
        # the forward kernel itself stores the records here (no fallback to
        # the binning kernels)
        assert native_lib.forward_bin_fuses(t["value"].to(value_dtype), t["sampling_locations"])
        out, gv, gl, ga = run_fused(native_lib, t, grad, value_dtype, geometry_dtype)
        plain = run_forward(native_lib, t, value_dtype, geometry_dtype)
        torch.cuda.synchronize()
        _assert_close(out, plain, 1e-6, "output against the plain forward")
    else:
        out = run_forward(native_lib, t, value_dtype, geometry_dtype)
        gv, gl, ga = run_backward(native_lib, t, grad, value_dtype, geometry_dtype)
    g = torch.Generator().manual_seed(7)
    idx = torch.randperm(cfg.queries, generator=g)[:SUBSET].sort().values
    mask = torch.zeros(cfg.queries, dtype=torch.bool)
    mask[idx] = True
    grad_masked = grad * mask.view(1, -1, 1)
    if fused:
        _, gv_sub, _, _ = run_fused(native_lib, t, grad_masked, value_dtype, geometry_dtype)
    else:
        gv_sub, _, _ = run_backward(native_lib, t, grad_masked, value_dtype, geometry_dtype)
    torch.cuda.synchronize()

    value, shapes, loc, attn = oracle_inputs(t, value_dtype, geometry_dtype)
    gq = grad.to(value_dtype).float()
    o_out, o_gv, o_gl, o_ga = msda_torch.msda_forward_backward(
        value, shapes, loc[:, idx], attn[:, idx], gq[:, idx]
    )
    ftol, btol = TOL[value_dtype]
    _assert_close(out.cpu()[:, idx], o_out, ftol, "output (query subset)")
    _assert_close(gl.cpu()[:, idx], o_gl, btol, "grad_sampling_locations (query subset)")
    _assert_close(ga.cpu()[:, idx], o_ga, btol, "grad_attention_weights (query subset)")
    _assert_close(gv_sub, o_gv, btol, "grad_value (grad_output on the subset)")

    # full size: every element written, and the adjoint identities
    assert torch.isfinite(gl).all() and torch.isfinite(ga).all()
    lhs = float((out.double() * grad.to(value_dtype).to(DEV).double()).sum())
    rhs_v = float((t["value"].to(value_dtype).to(DEV).double() * gv.double()).sum())
    rhs_a = float((attn.to(DEV).double() * ga.double()).sum())
    scale = float((out.double().abs() * grad.to(DEV).double().abs()).sum())
    rel = 1e-5 if value_dtype == torch.float32 else 3e-3
    assert abs(lhs - rhs_v) <= rel * scale, (lhs, rhs_v, scale)
    assert abs(lhs - rhs_a) <= rel * scale, (lhs, rhs_a, scale)
