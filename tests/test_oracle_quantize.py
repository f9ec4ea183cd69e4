"""Known answers, closed forms and brute force that pin the NumPy oracle's
quantize/dequantize (pratchya/_qualia/_qarr.py:458-506, 541-569).

Each check is chosen so that a plausible slip in the restatement (a dropped
clamp, the dead kernels' x256 instead of x128, a single rounding instead of
two, a transposed block order, grouping across slices) fails at least one.
"""
import math

import numpy as np
import pytest

from oracle import qarr_oracle as O
from tests.exact_ref import quantize_exact

F32 = np.float32


def q(x, tgrid):
    return O.quantize_impl(np.asarray(x, dtype=F32), tgrid)


@pytest.mark.parametrize("shape,tgrid,sc8_shape,sc32_shape", [
    ((1024, 1024), (128, 128), (1, 64), (1, 1, 1)),           # config 1: one group
    ((16384, 2048), (1, 128), (32768, 8), (32768, 1, 1)),     # config 2
    ((2048, 8192), (128, 128), (1, 1024), (1, 1, 1)),         # config 3 weight
    ((16384, 2048), (128, 1), (32768, 8), (32768, 1, 1)),     # config 4 token-axis grid
    ((4096, 16384), (128, 128), (4, 1024), (4, 1, 1)),        # config 5 FFN weight
    ((4, 4096, 2048), (1, 128), (4, 8192, 8), (4, 8192, 1, 1)),
    ((8, 8), (1, 1), (64, 1), (64, 1, 1)),
    ((6, 10), (2, 5), (1, 6), (1, 1, 1)),                      # gcd(max(1,10//16), 6) = 1? -> K=1
])
def test_layout_closed_form(shape, tgrid, sc8_shape, sc32_shape):
    S, H, W = O.as_2d_shape(shape)
    n_blk, K, M = O.group_layout(H, W, tgrid)
    assert K == math.gcd(max(1, tgrid[0] * tgrid[1] // 16), n_blk)
    lead = shape[:-2]
    if shape == (6, 10):
        sc8_shape, sc32_shape = (6, 1), (6, 1, 1)
    assert tuple(lead) + (M, K) == sc8_shape
    assert tuple(lead) + (M, 1, 1) == sc32_shape


def test_non_dividing_tgrid_raises():
    with pytest.raises(ValueError):
        q(np.zeros((10, 10)), (3, 5))


def test_all_zero():
    x8, s8, s32 = q(np.zeros((4, 256)), (1, 128))
    assert np.all(x8 == 0) and np.all(s8 == 0) and np.all(s32 == 0)


def test_negative_zero_keeps_sign():
    x = np.zeros((1, 16), F32)
    x[0, 3] = -0.0
    x8, _, _ = q(x, (1, 16))
    assert x8[0, 3] == 0x80 and x8[0, 2] == 0x00


def test_single_spike_and_powers_of_two():
    # one group of 8 blocks (1,128): block 0 holds 2.0 at its max, block 3 holds 0.25
    x = np.zeros((1, 1024), F32)
    x[0, 5] = 2.0
    x[0, 3 * 128 + 7] = -0.25
    x[0, 3 * 128 + 8] = 0.125
    x8, s8, s32 = q(x, (1, 128))
    assert s32.ravel()[0] == 2.0
    # r = m/G: block0 -> 1 (e=127), block3 -> 0.125 (e=124), empty blocks -> e=0
    assert list(s8.ravel()) == [127, 0, 0, 124, 0, 0, 0, 0]
    # payload = x / (2^(e-127) G) * 128: 2/2*128 = 128 -> 0x70; -0.25/0.25*128 = -128 -> 0xF0
    assert x8[0, 5] == 0x70
    assert x8[0, 3 * 128 + 7] == 0xF0
    assert x8[0, 3 * 128 + 8] == 0x68  # 64
    # dequantize is exact for these
    y = O.dequantize_impl(x8, s8, s32, "float32", (1, 128))
    assert np.array_equal(y, x)


def test_unit_grid_round_trips_exactly():
    # tgrid (1,1): S = max(|x|, 1e-7), payload = +-128, dequant = x for |x| >= 1e-7
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((16, 16)) * 10).astype(F32)
    x8, s8, s32 = q(x, (1, 1))
    assert np.all((x8 == 0x70) | (x8 == 0xF0))
    assert np.all(s8 == 127)
    assert np.array_equal(s32.reshape(16, 16), np.abs(x))
    assert np.array_equal(O.dequantize_impl(x8, s8, s32, "float32", (1, 1)), x)


def test_scale_uses_x128_not_x256():
    # the dead Pallas-style kernel uses x256; the live path x128
    x = np.full((1, 16), 1.0, F32)
    x8, s8, s32 = q(x, (1, 16))
    assert np.all(x8 == 0x70)  # 128 (0x70), not 256 (0x78)


def test_double_rounding_tie_in_quantizer():
    # G = 1 (block max 1.0) -> S = 1; x*128 = 1.0625 + 2^-20 -> bf16 1.0625 -> e4m3 tie -> 1.0
    x = np.zeros((1, 16), F32)
    x[0, 0] = 1.0
    x[0, 1] = F32((1.0625 + 2.0 ** -20) / 128)
    x8, s8, s32 = q(x, (1, 16))
    assert s8.ravel()[0] == 127 and s32.ravel()[0] == 1.0
    assert x8[0, 1] == 0x38  # 1.0 (single rounding would give 0x39 = 1.125)


def test_clamp_fires_for_subnormal_ratio_and_overflows_to_nan():
    # tgrid (1,32) on [1,64]: K = gcd(32//16, 2) = 2, one group of two blocks.
    # group max 2^127, block-1 max 0.5 -> r = 2^-128 (subnormal) -> e = 0 -> S = 1e-7
    x = np.zeros((1, 64), F32)
    x[0, 0] = F32(2.0 ** 127)
    x[0, 32] = 0.5
    x[0, 33] = F32(1e-12)
    x8, s8, s32 = q(x, (1, 32))
    assert list(s8.ravel()) == [127, 0]
    assert x8[0, 32] == 0x7F          # 0.5 / 1e-7 * 128 overflows e4m3 -> NaN
    expected = O.bf16_bits_to_e4m3fn(O.f32_to_bf16_bits(
        np.array([(F32(1e-12) / F32(1e-7)) * F32(128)], F32)))[0]
    assert x8[0, 33] == expected
    # dequant of an e=0 block decodes to 0 (no clamp on the dequant side)
    y = O.dequantize_impl(x8, s8, s32, "float32", (1, 32))
    assert y[0, 33] == 0.0


def test_clamp_small_group():
    # whole group tiny: G = 1e-9 -> r = 1, S = max(1e-9, 1e-7) = 1e-7
    x = np.full((1, 16), F32(1e-9))
    x8, s8, s32 = q(x, (1, 16))
    t = (F32(1e-9) / F32(1e-7)) * F32(128)
    assert np.all(x8 == O.bf16_bits_to_e4m3fn(O.f32_to_bf16_bits(np.array([t], F32)))[0])


def test_nan_and_inf_propagate():
    x = np.ones((1, 32), F32)
    x[0, 3] = np.nan
    x8, s8, s32 = q(x, (1, 16))
    assert np.all((x8[0, :16] & 0x7F) == 0x7F)      # group 0 NaN throughout
    assert np.isnan(s32.ravel()[0]) and s8.ravel()[0] == 0xFF
    x = np.ones((1, 32), F32)
    x[0, 3] = np.inf
    x8, s8, s32 = q(x, (1, 16))
    assert np.isinf(s32.ravel()[0]) and (x8[0, 3] & 0x7F) == 0x7F


def test_slices_are_independent():
    rng = np.random.default_rng(5)
    x = rng.standard_normal((3, 8, 64)).astype(F32)
    x[1] *= 1000
    x8, s8, s32 = q(x, (2, 16))
    for i in range(3):
        a8, b8, c32 = q(x[i], (2, 16))
        assert np.array_equal(x8[i], a8) and np.array_equal(s8[i], b8) and np.array_equal(s32[i], c32)


def test_block_order_is_row_major_over_block_grid():
    # (2,4) blocks on [4,8]: blocks (0,0),(0,1),(1,0),(1,1); K = gcd(max(1,8//16)=1, 4) = 1
    x = np.zeros((4, 8), F32)
    x[0, 4] = 4.0   # block (0,1) -> index 1
    x[2, 0] = 2.0   # block (1,0) -> index 2
    _, s8, s32 = q(x, (2, 4))
    assert s32.ravel().tolist() == [0.0, 4.0, 2.0, 0.0]


def test_dequant_relative_block_error_bound():
    rng = np.random.default_rng(7)
    x = rng.standard_normal((64, 256)).astype(F32)
    x8, s8, s32 = q(x, (16, 16))
    y = O.dequantize_impl(x8, s8, s32, "float32", (16, 16))
    xb = x.reshape(4, 16, 16, 16).transpose(0, 2, 1, 3).reshape(64, 256)
    yb = y.reshape(4, 16, 16, 16).transpose(0, 2, 1, 3).reshape(64, 256)
    err = np.max(np.abs(xb - yb), axis=1) / np.max(np.abs(xb), axis=1)
    assert np.all(err <= 2.0 ** -4)


def test_dequant_bf16_output_is_rounded_f32():
    rng = np.random.default_rng(8)
    x = rng.standard_normal((8, 128)).astype(F32)
    x8, s8, s32 = q(x, (1, 128))
    f = O.dequantize_impl(x8, s8, s32, "float32", (1, 128))
    b = O.dequantize_impl(x8, s8, s32, "bfloat16", (1, 128))
    assert np.array_equal(b, O.f32_to_bf16_bits(f))


def test_dequant_bwd_closed_form():
    # scale = 2^(e-127) * G / 128; with G a power of two the product is exact
    x = np.zeros((1, 32), F32)
    x[0, 0] = 8.0
    x[0, 16] = 1.0
    _, s8, s32 = q(x, (1, 16))
    g = np.full((1, 32), 3.0, F32)
    gx = O.dequantize_bwd(g, s8, s32, (1, 16))
    assert np.all(gx[0, :16] == 3.0 * 8.0 / 128)
    assert np.all(gx[0, 16:] == 3.0 * 1.0 / 128)


@pytest.mark.parametrize("seed,shape,tgrid", [
    (0, (4, 32), (1, 16)), (1, (8, 8), (2, 4)), (2, (4, 16), (4, 4)),
    (3, (2, 48), (1, 16)), (4, (16, 16), (16, 1)), (5, (8, 16), (1, 1)),
])
def test_brute_force_exact_rationals(seed, shape, tgrid):
    rng = np.random.default_rng(seed)
    x = (rng.standard_t(3, size=shape) * np.exp2(rng.integers(-20, 20, size=shape))).astype(F32)
    x[rng.random(shape) < 0.1] = 0.0
    x.flat[0] = F32(1e-9)  # exercise clamps in some blocks
    ref8, ref_e, ref_g = quantize_exact(x.tolist(), tgrid)
    x8, s8, s32 = q(x, tgrid)
    assert np.array_equal(x8, np.array(ref8, np.uint8))
    assert s8.ravel().tolist() == ref_e
    assert s32.ravel().astype(np.float64).tolist() == ref_g
