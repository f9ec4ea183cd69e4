"""GPU parity of the transposed requantize grouped along the tokens:
quantize_impl(x^T, (1, 128)) of a [T, C] tensor (pratchya/_qualia/_qarr.py:
458-506; fp8_matmul's backward quantizes its transposed raw inputs this way,
Q:786-788), payload [C, T], groups of 8 token blocks of one channel.

Expected values: the oracle's quantize_impl of the transposed array; for an
fp8 input, of its dequantize_impl; for a bf16 cotangent with scales, of its
dequantize_impl_bwd.  Bit-exact payload, e8m0 and f32 bytes (a NaN payload
byte's sign is compared as NaN-ness only).  Token counts that are not a
multiple of 1024 take the general quantizer on the transposed tensor.
"""
import numpy as np
import pytest
import torch

from oracle import qarr_oracle as O
from tests.helpers import (assert_bytes_equal, assert_f32_bits_equal, assert_payload_equal, f32,
                           to_dev_bf16, to_dev_f32, u8)

pytestmark = pytest.mark.gpu


def _K():
    from pratchya_amd import _kernels
    return _kernels


def check(dev, x_f32, what, x_sc8=None, x_sc32=None):
    xt, s8, s32 = _K().quantize_t1x128(dev, x_sc8, x_sc32)
    torch.cuda.synchronize()
    r8, rs8, rs32 = O.quantize_impl(np.ascontiguousarray(x_f32.T), (1, 128))
    assert tuple(xt.shape) == r8.shape, (tuple(xt.shape), r8.shape)
    assert tuple(s8.shape) == rs8.shape and tuple(s32.shape) == rs32.shape, (tuple(s8.shape), rs8.shape)
    assert_payload_equal(u8(xt), r8, f"{what} payload")
    assert_bytes_equal(u8(s8), rs8, f"{what} e8m0")
    assert_f32_bits_equal(f32(s32), rs32, f"{what} group max")


# C not a multiple of the 64 (bf16) / 32 (f32, fp8) channels of a workgroup,
# and token counts of one and several groups; 512 tokens take the general path
@pytest.mark.parametrize("T,C", [(1024, 64), (2048, 128), (1024, 72), (1024, 8), (3072, 320), (512, 256)])
def test_bf16_activation(T, C):
    bits = O.activation_input(T, C, seed=31)
    check(to_dev_bf16(bits), O.bf16_bits_to_f32(bits), f"bf16 [{T},{C}]")


@pytest.mark.parametrize("T,C", [(1024, 256), (2048, 40)])
def test_f32_normal(T, C):
    """Random f32 inputs hit the bf16-midpoint check and its exact redo."""
    x = np.random.default_rng(T + C).standard_normal((T, C)).astype(np.float32)
    check(to_dev_f32(x), x, f"f32 [{T},{C}]")


def test_edge_values():
    """A channel group of zeros (G = 0), zero blocks inside a live group (e8m0
    0), a clamped group, subnormals, NaN / inf, and a huge block next to
    normal ones in one channel's group."""
    T, C = 2048, 64
    x = np.random.default_rng(33).standard_normal((T, C)).astype(np.float32)
    x[:1024, 0] = 0.0                                 # channel 0, group 0: G = 0
    x[128:256, 1] = 0.0                               # e8m0 0 block in a live group
    x[1024:, 2] *= np.float32(1e-12)                  # clamped group
    x[:1024, 3] = np.float32(2.0 ** -140) * np.arange(1, 1025, dtype=np.float32)
    x[5, 32] = np.inf
    x[700, 40] = -np.inf
    x[1500, 48] = np.nan
    x[1030, 56] = 3.0e38
    check(to_dev_f32(x), x, "f32 edges")
    xb = O.f32_to_bf16_bits(x)
    check(to_dev_bf16(xb), O.bf16_bits_to_f32(xb), "bf16 edges")


@pytest.mark.parametrize("T,C", [(1024, 128), (2048, 1024), (512, 256)])
def test_fp8_input(T, C):
    """A stored (1, 128) activation, dequantized in registers exactly as
    dequantize_impl does, transposed and requantized."""
    bits = O.activation_input(T, C, seed=34)
    x8, s8, s32 = O.quantize_impl(O.bf16_bits_to_f32(bits), (1, 128))
    deq = O.dequantize_impl(x8, s8, s32, "float32", (1, 128))
    check(torch.from_numpy(x8).cuda(), deq, f"fp8 [{T},{C}]", torch.from_numpy(s8).cuda(),
          torch.from_numpy(s32).cuda())


def test_fp8_input_every_payload_byte():
    """Every finite e4m3fn byte under several block scales, then NaN bytes."""
    T, C = 1024, 256
    rng = np.random.default_rng(35)
    finite = np.array([b for b in range(256) if (b & 0x7F) != 0x7F], dtype=np.uint8)
    x8 = rng.choice(finite, size=(T, C)).astype(np.uint8)
    x8[:2, :] = np.resize(finite, (2, C))
    n_blk = T * C // 128
    s8 = rng.integers(100, 140, size=(n_blk // 8, 8)).astype(np.uint8)
    s32 = rng.uniform(0.5, 4.0, size=(n_blk // 8, 1, 1)).astype(np.float32)
    deq = O.dequantize_impl(x8, s8, s32, "float32", (1, 128))
    dev = [torch.from_numpy(a).cuda() for a in (x8, s8, s32)]
    check(dev[0], deq, "fp8 every byte", dev[1], dev[2])
    x8n = x8.copy()
    x8n[5, 7], x8n[930, 200] = 0x7F, 0xFF
    check(torch.from_numpy(x8n).cuda(), O.dequantize_impl(x8n, s8, s32, "float32", (1, 128)), "fp8 NaN bytes",
          dev[1], dev[2])


@pytest.mark.parametrize("T", [1024, 512])
def test_bf16_cotangent_with_scales(T):
    """A bf16 cotangent of a (1, 128)-quantized tensor: dequantize_impl_bwd
    with that tensor's scales (in bf16), then transposed and requantized."""
    C = 256
    bits = O.activation_input(T, C, seed=36)
    _, s8, s32 = O.quantize_impl(O.bf16_bits_to_f32(bits), (1, 128))
    g = O.normal_input((T, C), 1e-3, seed=37)
    g1 = O.bf16_bits_to_f32(O.dequantize_bwd(O.bf16_bits_to_f32(g), s8, s32, (1, 128), "bfloat16"))
    check(to_dev_bf16(g), g1, f"bf16 cotangent [{T},{C}]", torch.from_numpy(s8).cuda(), torch.from_numpy(s32).cuda())
