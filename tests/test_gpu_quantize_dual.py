"""GPU parity of pratchya_quantize_dual: quantize_impl(x, (1, 128)) and
quantize_impl(dequantize_impl(that), (128, 1)) from one pass
(pratchya/_qualia/_qarr.py:458-506, :541-569; the second is the FP8 weight
gradient's token-axis requantization of the stored activation, Q:784-789).

* Bit for bit against the two-kernel chain (pratchya_quantize, then
  pratchya_quantize_128x1 of its payload): config 2's activation in full,
  config 5's widths (4096 and 16384 channels), f32
  inputs, slices, and rows built to exercise the edge paths: all-zero tokens
  and channels, NaN / inf, values that clamp at 1e-7, near-midpoint products.
* Against the oracle chain (O.quantize_impl twice with O.dequantize_impl
  between) at small sizes: payload, e8m0 and f32 group maxima bit for bit
  (NaN payload bytes compared as NaN).
"""
import numpy as np
import pytest
import torch

from oracle import qarr_oracle as O
from tests.helpers import assert_bytes_equal, assert_f32_bits_equal, assert_payload_equal, f32, u8

pytestmark = pytest.mark.gpu


def _K():
    from pratchya_amd import _kernels
    return _kernels


def _chain(x):
    K = _K()
    a = K.quantize(x, (1, 128))
    b = K.quantize_128x1(a[0], a[1], a[2])
    return a, b


def _same(got, want, what):
    for g, w, name in zip(got, want, ("payload", "e8m0", "G")):
        assert tuple(g.shape) == tuple(w.shape), f"{what} {name}: shape {tuple(g.shape)} != {tuple(w.shape)}"
        if name == "G":
            assert_f32_bits_equal(f32(g), f32(w), f"{what} {name}")
        elif name == "payload":
            assert_payload_equal(u8(g), u8(w), f"{what} {name}")
        else:
            assert_bytes_equal(u8(g), u8(w), f"{what} {name}")


def _check_chain(x, what):
    K = _K()
    got1, got2 = K.quantize_dual(x)
    want1, want2 = _chain(x)
    torch.cuda.synchronize()
    _same(got1, want1, f"{what} (1,128)")
    _same(got2, want2, f"{what} (128,1)")


def test_config2_activation_full():
    bits = O.activation_input(16384, 2048, seed=2)
    x = torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16).cuda()
    _check_chain(x, "config 2")


@pytest.mark.parametrize("shape,dtype,std", [((32768, 4096), torch.bfloat16, 1.0),
                                             ((4096, 16384), torch.bfloat16, 0.5),
                                             ((2048, 3072), torch.float32, 3.0),
                                             ((3, 256, 1024), torch.bfloat16, 1.0),
                                             ((2, 384, 2048), torch.float32, 1e-3)],
                         ids=lambda v: str(v).replace(" ", ""))
def test_against_chain(shape, dtype, std):
    g = torch.Generator(device="cuda").manual_seed(sum(shape))
    x = (torch.randn(shape, generator=g, device="cuda") * std).to(dtype)
    _check_chain(x, f"{shape} {dtype}")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_special_values(dtype):
    """Zero tokens and channels (e8m0 0 blocks, zero groups), a group with a
    NaN and one with an infinity (non-finite group maxima on both grids),
    tiny rows whose scales clamp at 1e-7, one huge outlier per group
    (blocks far below their group max), and values on bf16 rounding
    midpoints after scaling."""
    g = torch.Generator(device="cuda").manual_seed(5)
    x = torch.randn((1024, 2048), generator=g, device="cuda")
    x[0] = 0.0
    x[:, 5] = 0.0
    x[130:140, 1030:1100] = 0.0
    x[3, 17] = float("nan")
    x[300, 1500] = float("inf")
    x[301, 1501] = -float("inf")
    x[400:410] *= 1e-9
    x[500:520, ::1024] = 3.0e4
    x[600:700] = torch.round(x[600:700] * 64) / 64 + 1.0 / 512
    x = x.to(dtype)
    _check_chain(x, f"special {dtype}")


@pytest.mark.parametrize("shape", [(256, 1024), (2, 128, 2048)], ids=lambda s: "x".join(map(str, s)))
def test_against_oracle(shape):
    rng = np.random.default_rng(19)
    xf = (rng.standard_t(3, size=shape) * rng.choice([1.0, 50.0], size=shape[-1], p=[0.98, 0.02])).astype(np.float32)
    xf[..., 7, :] = 0.0
    bits = O.f32_to_bf16_bits(xf)
    x = torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16).reshape(shape).cuda()
    got1, got2 = _K().quantize_dual(x)
    torch.cuda.synchronize()
    xb = O.bf16_bits_to_f32(bits)
    slices = xb.reshape((-1,) + shape[-2:])
    for s in range(slices.shape[0]):
        w1 = O.quantize_impl(slices[s], (1, 128))
        d = O.dequantize_impl(*w1, "float32", (1, 128))
        w2 = O.quantize_impl(d, (128, 1))
        sel = (lambda t: t[s]) if len(shape) == 3 else (lambda t: t)
        assert_payload_equal(u8(sel(got1[0])), w1[0], f"slice {s} (1,128) payload")
        assert_bytes_equal(u8(sel(got1[1])), w1[1], f"slice {s} (1,128) e8m0")
        assert_f32_bits_equal(f32(sel(got1[2])), w1[2], f"slice {s} (1,128) G")
        assert_payload_equal(u8(sel(got2[0])), w2[0], f"slice {s} (128,1) payload")
        assert_bytes_equal(u8(sel(got2[1])), w2[1], f"slice {s} (128,1) e8m0")
        assert_f32_bits_equal(f32(sel(got2[2])), w2[2], f"slice {s} (128,1) G")


def test_rejects_other_widths():
    K = _K()
    with pytest.raises(K.PratchyaUnsupported):
        K.quantize_dual(torch.zeros((128, 2560), dtype=torch.bfloat16, device="cuda"))
    with pytest.raises(ValueError):               # tgrid (128, 1) does not divide 100 tokens
        K.quantize_dual(torch.zeros((100, 1024), dtype=torch.bfloat16, device="cuda"))
