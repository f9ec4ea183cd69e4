"""The C restatement (oracle/qarr_oracle.c) and the NumPy oracle agree byte
for byte; two independent formulations of the same reference arithmetic."""
import numpy as np
import pytest

from oracle import c_oracle as C
from oracle import qarr_oracle as O


def test_c_bf16_to_e4m3_exhaustive_matches_numpy():
    lib = C.load()
    b = np.arange(65536, dtype=np.uint32)
    got = np.array([lib.oracle_bf16_to_e4m3(int(v)) for v in b], dtype=np.uint8)
    assert np.array_equal(got, O.bf16_bits_to_e4m3fn(b.astype(np.uint16)))


@pytest.mark.parametrize("shape,tgrid", [
    ((256, 2048), (1, 128)), ((512, 512), (128, 128)), ((256, 128), (128, 1)),
    ((3, 64, 96), (16, 32)), ((40, 40), (1, 1)), ((64, 64), (4, 4)), ((8, 64), (1, 16)),
])
def test_c_quantize_matches_numpy(shape, tgrid):
    rng = np.random.default_rng(31)
    x = (rng.standard_t(3, size=shape) * np.exp2(rng.integers(-30, 30, size=shape))).astype(np.float32)
    x[rng.random(shape) < 0.05] = 0.0
    x.flat[5] = np.float32(1e-9)
    a = C.quantize(x, tgrid)
    b = O.quantize_impl(x, tgrid)
    for u, v in zip(a, b):
        assert u.shape == v.shape
        assert np.array_equal(u.view(np.uint8), v.view(np.uint8))
    y1 = C.dequantize(*a, tgrid)
    y2 = O.dequantize_impl(*b, "float32", tgrid)
    assert np.array_equal(np.isnan(y1), np.isnan(y2))
    ok = ~np.isnan(y1)
    assert np.array_equal(y1[ok].view(np.uint32), y2[ok].view(np.uint32))


def test_c_quantize_config2_rows():
    bits = O.activation_input(512, 2048, seed=2)
    x = O.bf16_bits_to_f32(bits)
    a = C.quantize(x, (1, 128))
    b = O.quantize_impl(x, (1, 128))
    for u, v in zip(a, b):
        assert np.array_equal(u.view(np.uint8), v.view(np.uint8))
