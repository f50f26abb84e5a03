"""Pins the parity oracle (oracle/) before it is trusted to judge the HIP kernels.

Each check below is a function of a forward (or backward) implementation, so
the same checks run against the two oracles (which must pass) and against
deliberately broken restatements (which must fail): a check that cannot tell
a swapped x/y, a missing half-pixel offset, a dropped corner or border
padding from the real thing pins nothing.

Known answers come from the reference's own tests
(/root/reference/tests/ops/test_multi_scale_deformable_attn.py:245-253,269-280,430-468);
the rest are closed forms of bilinear sampling. The reference stores no golden
tensors: its only fixture file for this path
(/root/reference/tests/fixtures/bevformer_msda_shapes.yaml) holds shape metadata.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from msda_testlib import level_starts, random_case
from oracle import msda_direct, msda_torch

# ------------------------------------------------------------------ oracles ---


def torch_forward(value, shapes, loc, attn):
    with torch.no_grad():
        return msda_torch.msda_forward(
            torch.as_tensor(value), torch.as_tensor(shapes), torch.as_tensor(loc),
            torch.as_tensor(attn),
        ).numpy()


def torch_backward(value, shapes, loc, attn, grad):
    _, gv, gl, ga = msda_torch.msda_forward_backward(
        torch.as_tensor(value), torch.as_tensor(shapes), torch.as_tensor(loc),
        torch.as_tensor(attn), torch.as_tensor(grad),
    )
    return gv.numpy(), gl.numpy(), ga.numpy()


def direct_forward(value, shapes, loc, attn):
    return msda_direct.forward(np.asarray(value), np.asarray(shapes), np.asarray(loc), np.asarray(attn))


def direct_backward(value, shapes, loc, attn, grad):
    return msda_direct.backward(
        np.asarray(value), np.asarray(shapes), np.asarray(loc), np.asarray(attn), np.asarray(grad)
    )


FORWARDS = {"torch": torch_forward, "direct": direct_forward}
BACKWARDS = {"torch": torch_backward, "direct": direct_backward}

# ---------------------------------------------------- planted mistakes ---


def mutant_forward(mutation: str):
    """Pure-Python closed form with one plausible mistake planted (tiny inputs only)."""

    def fwd(value, shapes, loc, attn):
        value, loc, attn = (np.asarray(t, dtype=np.float64) for t in (value, loc, attn))
        shapes = np.asarray(shapes)
        bs, nv, M, C = value.shape
        _, nq, _, L, P, _ = loc.shape
        starts = level_starts([tuple(s) for s in shapes.tolist()]).numpy()
        out = np.zeros((bs, nq, M, C))
        for b in range(bs):
            for q in range(nq):
                for m in range(M):
                    for l in range(L):
                        h, w = (int(v) for v in shapes[l])
                        for p in range(P):
                            lx, ly = loc[b, q, m, l, p]
                            if mutation == "swap_xy":
                                lx, ly = ly, lx
                            off = 0.0 if mutation == "no_half_pixel" else 0.5
                            x, y = lx * w - off, ly * h - off
                            x0, y0 = math.floor(x), math.floor(y)
                            fx, fy = x - x0, y - y0
                            for dy, dx, wt in (
                                (0, 0, (1 - fy) * (1 - fx)),
                                (0, 1, (1 - fy) * fx),
                                (1, 0, fy * (1 - fx)),
                                (1, 1, fy * fx),
                            ):
                                if mutation == "drop_corner" and (dy, dx) == (1, 1):
                                    continue
                                yy, xx = y0 + dy, x0 + dx
                                if mutation == "border_padding":
                                    yy, xx = min(max(yy, 0), h - 1), min(max(xx, 0), w - 1)
                                elif not (0 <= yy < h and 0 <= xx < w):
                                    continue
                                row_stride = h if mutation == "row_stride_h" else w
                                cell = starts[l] + yy * row_stride + xx
                                if mutation == "row_stride_h" and cell >= starts[l] + h * w:
                                    continue
                                out[b, q, m] += attn[b, q, m, l, p] * wt * value[b, cell, m]
        return out.reshape(bs, nq, M * C)

    return fwd


MUTATIONS = ("swap_xy", "no_half_pixel", "drop_corner", "border_padding", "row_stride_h")

# ---------------------------------------------------------------- checks ---

NON_SQUARE = ((3, 5), (2, 7))


def _linear_value(levels, heads, channels, coef):
    """value[cell(y,x), m, c] = a*x + b*y + c0 per level, channel and head."""
    rows = []
    for h, w in levels:
        ys, xs = np.meshgrid(np.arange(h), np.arange(w), indexing="ij")
        xs, ys = xs.reshape(-1, 1, 1), ys.reshape(-1, 1, 1)
        rows.append(coef[0] * xs + coef[1] * ys + coef[2])
    return np.concatenate(rows, 0)[None].repeat(1, 0)


def check_pixel_centres(fwd) -> bool:
    """A sample at a pixel centre returns that pixel's value exactly."""
    rng = np.random.default_rng(1)
    levels, M, C, P, nq = NON_SQUARE, 2, 3, 4, 3
    nv = sum(h * w for h, w in levels)
    value = rng.standard_normal((1, nv, M, C))
    loc = np.zeros((1, nq, M, len(levels), P, 2))
    expect = np.zeros((1, nq, M, C))
    attn = rng.uniform(0.1, 1.0, (1, nq, M, len(levels), P))
    start = 0
    for l, (h, w) in enumerate(levels):
        xs = rng.integers(0, w, (nq, M, P))
        ys = rng.integers(0, h, (nq, M, P))
        loc[0, :, :, l, :, 0] = (xs + 0.5) / w
        loc[0, :, :, l, :, 1] = (ys + 0.5) / h
        for q in range(nq):
            for m in range(M):
                for p in range(P):
                    cell = start + ys[q, m, p] * w + xs[q, m, p]
                    expect[0, q, m] += attn[0, q, m, l, p] * value[0, cell, m]
        start += h * w
    out = fwd(value, np.array(levels), loc, attn)
    return np.allclose(out, expect.reshape(1, nq, M * C), rtol=1e-9, atol=1e-9)


def _interior_linear_case(seed=2):
    rng = np.random.default_rng(seed)
    levels, M, C, P, nq = NON_SQUARE, 2, 3, 3, 4
    coef = rng.standard_normal((3, 1, M, C))
    value = _linear_value(levels, M, C, coef)
    L = len(levels)
    loc = np.zeros((1, nq, M, L, P, 2))
    for l, (h, w) in enumerate(levels):
        # pixel coordinate strictly inside [0, W-1] x [0, H-1]
        ix = rng.uniform(0.05, w - 1.05, (nq, M, P))
        iy = rng.uniform(0.05, h - 1.05, (nq, M, P))
        loc[0, :, :, l, :, 0] = (ix + 0.5) / w
        loc[0, :, :, l, :, 1] = (iy + 0.5) / h
    attn = rng.uniform(0.1, 1.0, (1, nq, M, L, P))
    grad = rng.standard_normal((1, nq, M * C))
    return levels, coef, value, loc, attn, grad


def check_linear_field(fwd) -> bool:
    """Bilinear interpolation reproduces a linear field exactly inside the image."""
    levels, coef, value, loc, attn, _ = _interior_linear_case()
    M, C = value.shape[2], value.shape[3]
    ix = loc[..., 0] * np.array([w for _, w in levels])[None, None, None, :, None] - 0.5
    iy = loc[..., 1] * np.array([h for h, _ in levels])[None, None, None, :, None] - 0.5
    field = (
        coef[0][None, :, :, None, None, :] * ix[..., None]
        + coef[1][None, :, :, None, None, :] * iy[..., None]
        + coef[2][None, :, :, None, None, :]
    )  # [1, nq, M, L, P, C]
    expect = (attn[..., None] * field).sum((3, 4)).reshape(1, -1, M * C)
    out = fwd(value, np.array(levels), loc, attn)
    return np.allclose(out, expect, rtol=1e-9, atol=1e-9)


def check_linear_field_gradients(bwd) -> bool:
    """For a linear field: d out / d loc_x = attn * a * W, d out / d loc_y = attn * b * H."""
    levels, coef, value, loc, attn, grad = _interior_linear_case(3)
    M, C = value.shape[2], value.shape[3]
    _, gl, ga = bwd(value, np.array(levels), loc, attn, grad)
    g = grad.reshape(1, -1, M, C)
    W = np.array([w for _, w in levels])[None, None, None, :, None]
    H = np.array([h for h, _ in levels])[None, None, None, :, None]
    ga_dot = (g * coef[0]).sum(-1)[..., None, None]  # sum_c g*a
    gb_dot = (g * coef[1]).sum(-1)[..., None, None]
    ix, iy = loc[..., 0] * W - 0.5, loc[..., 1] * H - 0.5
    field_dot = (ga_dot * ix + gb_dot * iy + (g * coef[2]).sum(-1)[..., None, None])
    ok_x = np.allclose(gl[..., 0], attn * ga_dot * W, rtol=1e-9, atol=1e-9)
    ok_y = np.allclose(gl[..., 1], attn * gb_dot * H, rtol=1e-9, atol=1e-9)
    ok_a = np.allclose(ga, field_dot, rtol=1e-9, atol=1e-9)
    return ok_x and ok_y and ok_a


def check_out_of_range_is_zero(fwd) -> bool:
    """Reference KAT: every location at -1 samples nothing (test_…:245-253)."""
    value, shapes, _, loc, attn, _ = random_case(5, levels=((2, 2),), points=2)
    loc = torch.full_like(loc, -1.0)
    return np.all(fwd(value.numpy(), shapes.numpy(), loc.numpy(), attn.numpy()) == 0)


def check_half_pixel_2048(fwd) -> bool:
    """Reference KAT (test_…:430-468): width 1000, value 0 | 4096 at pixel 500, loc 0.5 -> 2048."""
    width = 1000
    value = np.zeros((1, width, 1, 1))
    value[:, width // 2:] = 4096.0
    loc = np.full((1, 1, 1, 1, 1, 2), 0.5)
    attn = np.ones((1, 1, 1, 1, 1))
    out = fwd(value, np.array([[1, width]]), loc, attn)
    return out.shape == (1, 1, 1) and out[0, 0, 0] == 2048.0


FORWARD_CHECKS = {
    "pixel_centres": check_pixel_centres,
    "linear_field": check_linear_field,
    "out_of_range": check_out_of_range_is_zero,
    "half_pixel_2048": check_half_pixel_2048,
}

# ------------------------------------------------------------------ tests ---


@pytest.mark.parametrize("oracle", sorted(FORWARDS))
@pytest.mark.parametrize("check", sorted(FORWARD_CHECKS))
def test_forward_oracles_pass_closed_forms_and_kats(oracle, check):
    assert FORWARD_CHECKS[check](FORWARDS[oracle])


@pytest.mark.parametrize("oracle", sorted(BACKWARDS))
def test_backward_oracles_match_linear_field_gradients(oracle):
    assert check_linear_field_gradients(BACKWARDS[oracle])


def test_reference_mutant_restatement_passes_every_check():
    """The pure-Python restatement itself (no mutation) passes: the checks are fair."""
    fwd = mutant_forward("none")
    assert all(check(fwd) for check in FORWARD_CHECKS.values())


@pytest.mark.parametrize("mutation", MUTATIONS)
def test_planted_mistakes_are_caught(mutation):
    fwd = mutant_forward(mutation)
    failed = [name for name, check in FORWARD_CHECKS.items() if not check(fwd)]
    assert failed, f"no check catches the planted mistake {mutation!r}"


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_torch_restatement_equals_direct_closed_form(seed):
    """Two independent formulations (grid_sample sequence vs loops) agree in float64."""
    value, shapes, starts, loc, attn, grad = random_case(seed)
    out_t, gv_t, gl_t, ga_t = msda_torch.msda_forward_backward(value, shapes, loc, attn, grad)
    out_d = msda_direct.forward(value.numpy(), shapes.numpy(), loc.numpy(), attn.numpy(), starts.numpy())
    gv_d, gl_d, ga_d = msda_direct.backward(
        value.numpy(), shapes.numpy(), loc.numpy(), attn.numpy(), grad.numpy(), starts.numpy()
    )
    np.testing.assert_allclose(out_t.numpy(), out_d, rtol=1e-11, atol=1e-11)
    np.testing.assert_allclose(gv_t.numpy(), gv_d, rtol=1e-11, atol=1e-11)
    np.testing.assert_allclose(gl_t.numpy(), gl_d, rtol=1e-10, atol=1e-10)
    np.testing.assert_allclose(ga_t.numpy(), ga_d, rtol=1e-11, atol=1e-11)


def test_adjoint_identities():
    """out is linear in value and in attention: <g, out> = <value, dvalue> = <attn, dattn>."""
    value, shapes, _, loc, attn, grad = random_case(7)
    out, gv, _, ga = msda_torch.msda_forward_backward(value, shapes, loc, attn, grad)
    lhs = float((out * grad).sum())
    assert lhs == pytest.approx(float((value * gv).sum()), rel=1e-12, abs=1e-12)
    assert lhs == pytest.approx(float((attn * ga).sum()), rel=1e-12, abs=1e-12)


def test_gradcheck_of_torch_restatement():
    """Autograd of the grid_sample sequence equals numerical derivatives."""
    value, shapes, _, loc, attn, _ = random_case(11, batch=1, queries=2, heads=2, channels=2,
                                                 levels=((2, 3), (1, 2)), points=2,
                                                 loc_low=0.05, loc_high=0.95)
    # keep pixel coordinates away from integers, where bilinear sampling has kinks
    for l, (h, w) in enumerate(((2, 3), (1, 2))):
        for axis, size in ((0, w), (1, h)):
            px = loc[..., l, :, axis] * size - 0.5
            frac = px - torch.floor(px)
            loc[..., l, :, axis] += torch.where((frac < 0.1) | (frac > 0.9), 0.25 / size, 0.0)
    inputs = (value.requires_grad_(), loc.requires_grad_(), attn.requires_grad_())
    assert torch.autograd.gradcheck(
        lambda v, lc, a: msda_torch.msda_forward(v, shapes, lc, a), inputs, eps=1e-6, atol=1e-6
    )


def test_direct_backward_matches_finite_differences():
    value, shapes, _, loc, attn, grad = random_case(13, batch=1, queries=2, heads=2, channels=2,
                                                    levels=((2, 3),), points=2,
                                                    loc_low=0.2, loc_high=0.8)
    v, lc, a, g = value.numpy(), loc.numpy(), attn.numpy(), grad.numpy()
    sh = shapes.numpy()
    gv, gl, ga = msda_direct.backward(v, sh, lc, a, g)
    eps = 1e-6

    def objective(v_, lc_, a_):
        return float((msda_direct.forward(v_, sh, lc_, a_) * g).sum())

    for arr, analytic, idx in ((v, gv, (0, 3, 1, 0)), (lc, gl, (0, 1, 0, 0, 1, 0)),
                               (lc, gl, (0, 0, 1, 0, 0, 1)), (a, ga, (0, 1, 1, 0, 1))):
        plus, minus = arr.copy(), arr.copy()
        plus[idx] += eps
        minus[idx] -= eps
        args_p = [plus if arr is x else x for x in (v, lc, a)]
        args_m = [minus if arr is x else x for x in (v, lc, a)]
        numeric = (objective(*args_p) - objective(*args_m)) / (2 * eps)
        assert analytic[idx] == pytest.approx(numeric, rel=1e-5, abs=1e-7)


def test_zero_queries_give_empty_output():
    value, shapes, _, loc, attn, _ = random_case(3, queries=0)
    out = msda_torch.msda_forward(value, shapes, loc, attn)
    assert out.shape == (2, 0, 3 * 5)


def test_float32_oracle_uses_grid_sample_fma_coordinate():
    """The float32 oracle's pixel coordinate is fma(2*loc - 1 + 1, W/2, -0.5).

    The HIP kernels evaluate exactly this sequence so that floor() -- and with
    it the corner choice and the location gradient's kink -- matches the
    reference path bit for bit (probed on a value ramp, whose bilinear
    interpolation returns the coordinate itself).
    """
    width, n = 200, 4096
    g = torch.Generator().manual_seed(0)
    loc_x = torch.rand(n, generator=g) * 0.98 + 0.01
    value = torch.arange(width, dtype=torch.float32).view(1, width, 1, 1)
    loc = torch.stack([loc_x, torch.full_like(loc_x, 0.5)], -1).view(1, n, 1, 1, 1, 2)
    out = msda_torch.msda_forward(value, torch.tensor([[1, width]]), loc,
                                  torch.ones(1, n, 1, 1, 1)).view(n)
    x = (2 * loc_x - 1).numpy().astype(np.float32)
    expect = np.array(
        [np.float32(np.float64(np.float32(xi + np.float32(1))) * (width / 2) - 0.5) for xi in x],
        dtype=np.float32,
    )
    assert np.array_equal(out.numpy(), expect)


# ------------------------------------- spatial cross-attention scatter-average ---

def _scatter_div_inputs(seed, **kw):
    from msda_testlib import scatter_div_case

    return scatter_div_case(seed, **kw)


def _direct_scatter_div(value, shapes, loc, attn, indexes, count, slots):
    from oracle import msda_scatter_div

    return msda_scatter_div.scatter_div_direct(
        value.numpy(), shapes.numpy(), loc.numpy(), attn.numpy(),
        [i.numpy() for i in indexes], count.numpy(), slots.numpy())


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_scatter_div_matches_direct_loops(seed):
    """Two formulations: per-camera scaled adds on grid_sample vs float64 loops
    that sum a slot's cameras first and divide once."""
    from oracle import msda_scatter_div

    value, shapes, _, loc, attn, indexes, count, slots = _scatter_div_inputs(
        seed, out_of_range=seed == 2)
    actual = msda_scatter_div.scatter_div(value, shapes, loc, attn, indexes, count, slots)
    expected = _direct_scatter_div(value, shapes, loc, attn, indexes, count, slots)
    np.testing.assert_allclose(actual.numpy(), expected, rtol=1e-12, atol=1e-12)


def test_scatter_div_constant_value_gives_unit_average():
    """value = 1 and every corner inside its level: each camera's MSDA row is
    sum(attn) = 1, so a slot seen by k cameras gets k * (1 / k) = 1 (count here
    is the plain camera count) and an unseen slot keeps its value (0)."""
    from oracle import msda_scatter_div

    levels = ((4, 6), (3, 3))
    value, shapes, _, loc, attn, indexes, _, slots = _scatter_div_inputs(4, levels=levels)
    value = torch.ones_like(value)
    for level, (h, w) in enumerate(levels):  # x = loc*W - 0.5 strictly inside [0, W-1]
        loc[..., level, :, 0] = 0.6 / w + loc[..., level, :, 0].clamp(0, 1) * (1 - 1.2 / w)
        loc[..., level, :, 1] = 0.6 / h + loc[..., level, :, 1].clamp(0, 1) * (1 - 1.2 / h)
    seen = torch.zeros(slots.shape[1], dtype=torch.float64)
    for index in indexes:
        seen[index] += 1
    count = seen.clamp(min=1).expand(slots.shape[0], -1).contiguous()
    result = msda_scatter_div.scatter_div(value, shapes, loc, attn, indexes, count,
                                          torch.zeros_like(slots))
    expected = (seen > 0).to(torch.float64).view(1, -1, 1).expand_as(result)
    np.testing.assert_allclose(result.numpy(), expected.numpy(), rtol=0, atol=1e-12)


def test_scatter_div_direct_check_catches_a_camera_major_row_order():
    """Planted mistake: rows read as cam*batch + b instead of b*cams + cam."""
    from oracle import msda_scatter_div

    batch, cams = 2, 3
    value, shapes, _, loc, attn, indexes, count, slots = _scatter_div_inputs(
        5, batch=batch, cams=cams, lengths=[9, 6, 4])
    perm = torch.tensor([cam * batch + b for b in range(batch) for cam in range(cams)])
    mutant = msda_scatter_div.scatter_div(value[perm], shapes, loc[perm], attn[perm], indexes,
                                          count, slots)
    expected = _direct_scatter_div(value, shapes, loc, attn, indexes, count, slots)
    assert not np.allclose(mutant.numpy(), expected, rtol=1e-6, atol=1e-6)


def test_scatter_div_gradcheck():
    from oracle import msda_scatter_div

    value, shapes, _, loc, attn, indexes, count, slots = _scatter_div_inputs(
        6, batch=1, cams=2, max_len=4, num_query=6, heads=1, channels=2,
        levels=((2, 3),), points=2, lengths=[4, 3])
    args = [t.clone().requires_grad_(True) for t in (value, loc, attn, slots)]
    assert torch.autograd.gradcheck(
        lambda v, l, a, s: msda_scatter_div.scatter_div(v, shapes, l, a, indexes, count, s),
        args, eps=1e-6, atol=1e-6)
