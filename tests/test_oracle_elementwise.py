"""Pins of the elementwise oracle (oracle/elementwise_oracle.py): jnp's float32
floor_divide and remainder (QArrayImpl's // and %, pratchya/_qualia/_qarr.py:
199-261 through make_elementwise_impl, :715-720) against exact rational
arithmetic, CPython's float operators and torch's CPU remainder; the fused
composition against its definition."""
import math
from fractions import Fraction

import numpy as np
import pytest
import torch

from oracle import elementwise_oracle as E
from oracle import qarr_oracle as Q


def _pairs(seed, n, spread=8):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal(n) * np.exp2(rng.integers(-spread, spread, n))).astype(np.float32)
    y = (rng.standard_normal(n) * np.exp2(rng.integers(-spread, spread, n))).astype(np.float32)
    y[y == 0] = np.float32(1.0)
    return x, y


def test_floor_divide_is_the_exact_floor():
    """For finite nonzero divisors with |x / y| < 2^20 the quotient is
    floor(x / y) of the exact rationals (the f32 steps cannot move it across
    an integer there)."""
    x, y = _pairs(1, 20000)
    keep = np.abs(x.astype(np.float64) / y) < 2.0 ** 20
    x, y = x[keep], y[keep]
    got = E.jnp_floor_divide(x, y)
    want = np.array([math.floor(Fraction(float(a)) / Fraction(float(b))) for a, b in zip(x, y)], np.float64)
    np.testing.assert_array_equal(got.astype(np.float64), want)


def test_floor_divide_matches_cpython_float_floordiv():
    """CPython's float // is the same divmod algorithm in double precision;
    for finite nonzero f32 operands with moderate quotients both give the same
    integer, including the sign of a zero quotient for positive divisors."""
    x, y = _pairs(2, 5000)
    keep = np.abs(x.astype(np.float64) / y) < 2.0 ** 20
    got = E.jnp_floor_divide(x[keep], y[keep])
    want = np.array([float(a) // float(b) for a, b in zip(x[keep], y[keep])], np.float32)
    np.testing.assert_array_equal(got, want)
    pos = y[keep] > 0
    assert np.array_equal(np.signbit(got[pos]), np.signbit(want[pos]))


def test_floor_divide_known_answers():
    x = np.array([7.0, -7.0, 7.0, -7.0, 0.5, -0.5, 6.0, -3.0, 1.0, 1.0, 0.0, np.inf, np.nan], np.float32)
    y = np.array([2.0, 2.0, -2.0, -2.0, 2.0, 2.0, 3.0, np.inf, 0.0, np.nan, 5.0, 2.0, 1.0], np.float32)
    got = E.jnp_floor_divide(x, y)
    want = np.array([3, -4, -4, 3, 0, -1, 2, -1, np.nan, np.nan, 0, np.nan, np.nan], np.float32)
    np.testing.assert_array_equal(np.isnan(got), np.isnan(want))
    np.testing.assert_array_equal(got[~np.isnan(want)], want[~np.isnan(want)])


@pytest.mark.parametrize("seed", [3, 4])
def test_remainder_matches_torch(seed):
    """torch.remainder is the same definition (fmod, plus the divisor where the
    signs differ and fmod is nonzero), implemented independently."""
    x, y = _pairs(seed, 20000, spread=20)
    x[:6] = [0.0, -0.0, 4.0, -4.0, 3.0, -3.0]
    y[:6] = [3.0, 3.0, 2.0, 2.0, -1.5, 1.5]
    got = E.jnp_remainder(x, y)
    want = torch.remainder(torch.from_numpy(x), torch.from_numpy(y)).numpy()
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


def test_remainder_is_exact_on_finite_values():
    """Where the result is x - floor(x / y) * y exactly representable (Sterbenz
    range), it equals the exact rational remainder."""
    x, y = _pairs(5, 5000)
    got = E.jnp_remainder(x, y)
    for a, b, r in zip(x[:2000], y[:2000], got[:2000]):
        fa, fb = Fraction(float(a)), Fraction(float(b))
        exact = fa - math.floor(fa / fb) * fb
        if float(np.float32(float(exact))) == float(exact):
            assert Fraction(float(r)) == exact


def test_elementwise_is_quantize_of_the_dequantized_op():
    rng = np.random.default_rng(6)
    a = rng.standard_normal((128, 256)).astype(np.float32)
    b = rng.standard_normal((128, 256)).astype(np.float32)
    xa, xb = Q.quantize_impl(a, (1, 128)), Q.quantize_impl(b, (128, 128))
    got = E.elementwise("sub", xa, (1, 128), xb, (128, 128), (1, 32))
    da = Q.dequantize_impl(*xa, "float32", (1, 128))
    db = Q.dequantize_impl(*xb, "float32", (128, 128))
    want = Q.quantize_impl((da - db).astype(np.float32), (1, 32))
    for g, w in zip(got, want):
        np.testing.assert_array_equal(np.asarray(g).view(np.uint8), np.asarray(w).view(np.uint8))
    # (1, 1) grid: quantization is exact for e4m3-representable ratios, so
    # 2 * 3 comes back as 6
    one = Q.quantize_impl(np.full((1, 16), 2.0, np.float32), (1, 1))
    three = Q.quantize_impl(np.full((1, 16), 3.0, np.float32), (1, 1))
    six = E.elementwise("mul", one, (1, 1), three, (1, 1), (1, 1))
    np.testing.assert_array_equal(Q.dequantize_impl(*six, "float32", (1, 1)), np.full((1, 16), 6.0, np.float32))
