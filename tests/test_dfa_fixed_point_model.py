"""CPU model of the fixed-point sums of the deformable-aggregation backward's
coarse-map kernel (dfa_backward_coarse in muspace_amd/csrc/dfa_kernels.hpp).

The kernel turns each contribution x = w_corner * (grad_out * weight) (float32
operands) into the integer nearest x * 2^S by one float64 fused multiply-add
against 1.5 * 2^52 and reads the integer from the result's bits, adds the
integers in 64-bit LDS accumulators, and converts each sum back with
float(sum * 2^-S). S = 50 - pair_log2 - e where the workgroup's bound
(max |grad_out| * max |weight|) is below 2^e. These tests check, in numpy
float64 arithmetic (the product of two float32 numbers is exact in float64,
so adding the constant rounds once, as the fused multiply-add does):

* the bit trick equals round-half-even of x * 2^S;
* with every contribution at the bound and 2^pair_log2 of them, a sum stays
  below 2^50 (no overflow, the trick's range holds);
* the converted sums are within float32 rounding of the exact float64 sums,
  also for gradients scaled by 1e-30 and 1e30, and the integer sums carry
  less than 2^-30 of the bound in rounding error.
"""

import numpy as np
import pytest

MAGIC = np.float64(1.5 * 2.0**52)
MAGIC_BITS = MAGIC.view(np.int64)


def _shift(bound: np.float32, pair_log2: int) -> int:
    _, e = np.frexp(np.float64(bound))  # bound < 2^e
    return 50 - pair_log2 - int(e)


def _to_fixed(w_corner, top, shift):
    """The kernel's conversion: float64 product, +magic, bits - magic bits."""
    tc = top.astype(np.float64) * np.ldexp(1.0, shift)  # exact power-of-two scaling
    r = w_corner.astype(np.float64) * tc + MAGIC  # one rounding (w * tc is exact)
    return r.view(np.int64) - MAGIC_BITS


def _case(rng, n, scale):
    g = (rng.standard_normal(n) * scale).astype(np.float32)
    wg = rng.random(n, dtype=np.float32)
    w = rng.random(n, dtype=np.float32)  # bilinear corner weights in [0, 1)
    top = (g * wg).astype(np.float32)  # grad_out * weight in float32, as the kernel
    bound = np.float32(np.abs(g).max()) * np.float32(wg.max())
    return w, top, bound


@pytest.mark.parametrize("scale", [1.0, 1e-30, 1e30])
def test_bit_trick_is_round_half_even(scale):
    rng = np.random.default_rng(5)
    w, top, bound = _case(rng, 20000, scale)
    shift = _shift(bound, pair_log2=14)
    q = _to_fixed(w, top, shift)
    exact = w.astype(np.float64) * top.astype(np.float64) * np.ldexp(1.0, shift)
    np.testing.assert_array_equal(q, np.rint(exact).astype(np.int64))


def test_sums_at_the_bound_stay_below_two_to_the_fifty():
    pair_log2 = 14
    bound = np.float32(3.75)  # 2^1 < bound < 2^2: e = 2
    shift = _shift(bound, pair_log2)
    q = _to_fixed(np.ones(1, np.float32), np.array([bound], np.float32), shift)[0]
    assert 0 < q <= 2 ** (50 - pair_log2)
    assert q * 2**pair_log2 <= 2**50


@pytest.mark.parametrize("scale", [1.0, 1e-30, 1e30])
def test_converted_sums_are_within_float32_rounding(scale):
    """Cells that each take up to 2^pair_log2 contributions of mixed sign: the
    fixed-point sum converted to float32 is the exact sum rounded to float32
    (up to the rounding of the contributions, 2^-(S+1) each)."""
    rng = np.random.default_rng(7)
    pair_log2 = 12
    cells, per_cell = 64, 2**pair_log2
    w, top, bound = _case(rng, cells * per_cell, scale)
    shift = _shift(bound, pair_log2)
    q = _to_fixed(w, top, shift).reshape(cells, per_cell)
    sums = q.sum(axis=1)  # exact integer sums
    assert np.abs(sums).max() <= 2**50
    got = (sums.astype(np.float64) * np.ldexp(1.0, -shift)).astype(np.float32)
    exact = (w.astype(np.float64) * top.astype(np.float64)).reshape(cells, per_cell).sum(axis=1)
    # the contributions' rounding: at most per_cell * 2^-(shift+1) in absolute terms
    tol = per_cell * np.ldexp(1.0, -(shift + 1)) + np.abs(exact) * 2.0**-24
    assert np.all(np.abs(got.astype(np.float64) - exact) <= tol)
    # the allowance, 2^pair_log2 roundings of at most 2^-(S+1), is 2^-(51 - 2 pair_log2) of
    # the bound or less; the roundings' signs vary, so what is seen is far smaller
    _, e = np.frexp(np.float64(bound))
    assert per_cell * np.ldexp(1.0, -(shift + 1)) <= np.ldexp(1.0, int(e) - (51 - 2 * pair_log2))
    seen = np.abs(sums.astype(np.float64) * np.ldexp(1.0, -shift) - exact).max()
    assert seen <= np.float64(bound) * 2.0**-30
