"""GPU parity of the one-pass fake quantization, pratchya_quantize_dequantize.

Expected values: the oracle's dequantize_impl(*quantize_impl(x, tgrid), dtype,
tgrid) -- QArrayImpl(x, tgrid).astype(dtype) -- and, with fix_nan, the same
with NaN e8m0 bytes replaced by 0x7F first (quantize_impl's backward,
pratchya/_qualia/_qarr.py:512-526).  Bit-exact outputs (NaN compared as
NaN-ness) and bit-exact scales.  Also the one-pass requantization of a
Linear output's cotangent, pratchya_requantize_cotangent, against
quantize_impl(dequantize_bwd(g)).
"""
import ctypes

import numpy as np
import pytest
import torch

from oracle import qarr_oracle as O
from tests.helpers import (assert_bytes_equal, assert_f32_bits_equal, assert_payload_equal, f32,
                           to_dev_bf16, to_dev_f32, u8)
from tests.test_gpu_quantize import edge_tensor, tensor_1x1

pytestmark = pytest.mark.gpu

DT = {"float32": torch.float32, "bfloat16": torch.bfloat16}


def _K():
    from pratchya_amd import _kernels
    return _kernels


def oracle_qdq(x_f32, tgrid, out, fix_nan):
    r8, rs8, rs32 = O.quantize_impl(x_f32, tgrid)
    s8 = np.where(rs8 == 0xFF, np.uint8(0x7F), rs8) if fix_nan else rs8
    return O.dequantize_impl(r8, s8, rs32, out, tgrid), rs8, rs32


def as_f32(y, out):
    """Device output -> f32 ndarray (bf16 widened exactly), for NaN-aware compares."""
    if out == "float32":
        return f32(y)
    return O.bf16_bits_to_f32(y.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16))


def check(dev, x_f32, tgrid, out, fix_nan, what):
    y, s8, s32 = _K().quantize_dequantize(dev, tgrid, DT[out], fix_nan)
    torch.cuda.synchronize()
    want, rs8, rs32 = oracle_qdq(x_f32, tgrid, out, fix_nan)
    want_f = want if out == "float32" else O.bf16_bits_to_f32(want)
    assert y.dtype == DT[out] and tuple(y.shape) == x_f32.shape
    assert_f32_bits_equal(as_f32(y, out), want_f, f"{what} values")
    assert_bytes_equal(u8(s8), rs8, f"{what} e8m0")
    assert_f32_bits_equal(f32(s32), rs32, f"{what} group max")


@pytest.mark.parametrize("shape", [(256, 1024), (64, 384), (3, 128, 2048)])
@pytest.mark.parametrize("xdt", ["bf16", "f32"])
@pytest.mark.parametrize("out", ["bfloat16", "float32"])
def test_row_groups(shape, xdt, out):
    """tgrid (1, 128), 8 blocks per group: the single-pass kernel."""
    rng = np.random.default_rng(abs(hash((shape, xdt, out))) % 2 ** 32)
    x = (rng.standard_normal(shape) * np.exp2(rng.integers(-6, 6, size=shape[:-1] + (1,)))).astype(np.float32)
    if xdt == "bf16":
        bits = O.f32_to_bf16_bits(x)
        check(to_dev_bf16(bits), O.bf16_bits_to_f32(bits), (1, 128), out, False, f"{shape} {xdt}->{out}")
    else:
        check(to_dev_f32(x), x, (1, 128), out, False, f"{shape} {xdt}->{out}")


@pytest.mark.parametrize("shape,tgrid", [
    ((512, 768), (128, 128)), ((1024, 256), (128, 1)), ((64, 256), (1, 32)), ((2, 96, 64), (32, 32)),
])
@pytest.mark.parametrize("out", ["bfloat16", "float32"])
@pytest.mark.parametrize("fix_nan", [False, True])
def test_general_grids(shape, tgrid, out, fix_nan):
    rng = np.random.default_rng(abs(hash((shape, tgrid))) % 2 ** 32)
    x = (rng.standard_normal(shape) * 3).astype(np.float32)
    check(to_dev_f32(x), x, tgrid, out, fix_nan, f"{shape}{tgrid}->{out} fix {fix_nan}")


@pytest.mark.parametrize("xdt", ["bf16", "f32"])
@pytest.mark.parametrize("tgrid", [(1, 128), (16, 128)])
@pytest.mark.parametrize("out", ["bfloat16", "float32"])
@pytest.mark.parametrize("fix_nan", [False, True])
def test_edge_values(xdt, tgrid, out, fix_nan):
    """Zeros, -0, clamped groups, payload overflow to NaN, NaN / inf inputs
    (NaN e8m0 bytes), subnormals and f32 quotients next to bf16 midpoints."""
    x = edge_tensor(xdt)
    dev = to_dev_bf16(O.f32_to_bf16_bits(x)) if xdt == "bf16" else to_dev_f32(x)
    check(dev, x, tgrid, out, fix_nan, f"edge {xdt} {tgrid}->{out} fix {fix_nan}")


@pytest.mark.parametrize("xdt", ["bf16", "f32"])
@pytest.mark.parametrize("out", ["bfloat16", "float32"])
@pytest.mark.parametrize("fix_nan", [False, True])
def test_grid_1x1(xdt, out, fix_nan):
    """tgrid (1, 1) (the output grid of lm_head and LoRA products) on its
    elementwise kernel, and at an element count that is not a multiple of 4
    (the general kernel), against the oracle."""
    x = tensor_1x1()
    if xdt == "bf16":
        bits = O.f32_to_bf16_bits(x)
        x = O.bf16_bits_to_f32(bits)
        check(to_dev_bf16(bits), x, (1, 1), out, fix_nan, f"(1,1) {xdt}->{out} fix {fix_nan}")
        odd = np.ascontiguousarray(bits[:7, :13])
        check(to_dev_bf16(odd), O.bf16_bits_to_f32(odd), (1, 1), out, fix_nan, "(1,1) odd count")
    else:
        check(to_dev_f32(x), x, (1, 1), out, fix_nan, f"(1,1) {xdt}->{out} fix {fix_nan}")
        odd = np.ascontiguousarray(x[:7, :13])
        check(to_dev_f32(odd), odd, (1, 1), out, fix_nan, "(1,1) odd count")


def test_matches_quantize_then_dequantize_on_device():
    """At a Linear-output size the fused pass equals the two-kernel
    composition bit for bit (f32 GEMM-like input, bf16 output)."""
    K = _K()
    g = torch.Generator(device="cuda").manual_seed(9)
    x = torch.randn((4096, 4096), generator=g, device="cuda") * 7.0
    y, s8, s32 = K.quantize_dequantize(x, (1, 128), torch.bfloat16)
    q8, r8, r32 = K.quantize(x, (1, 128))
    ref = K.dequantize(q8, r8, r32, torch.bfloat16, (1, 128))
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int16), ref.view(torch.int16))
    assert torch.equal(s8.view(torch.uint8), r8.view(torch.uint8))
    assert torch.equal(s32, r32)


def test_out_buffers_and_misaligned_output():
    """Preallocated outputs; an output that is not 16-byte aligned runs the
    general path with a workspace and gives the same bytes."""
    from pratchya_amd import _lib
    K = _K()
    rng = np.random.default_rng(5)
    H, W = 64, 1024
    x = rng.standard_normal((H, W)).astype(np.float32)
    want, rs8, rs32 = oracle_qdq(x, (1, 128), "bfloat16", False)
    y = torch.empty((H, W), dtype=torch.bfloat16, device="cuda")
    s8 = torch.empty((H * W // 1024, 8), dtype=torch.uint8, device="cuda")
    s32 = torch.empty((H * W // 1024, 1, 1), dtype=torch.float32, device="cuda")
    K.quantize_dequantize(to_dev_f32(x), (1, 128), torch.bfloat16, out=(y, s8, s32))
    torch.cuda.synchronize()
    assert_bytes_equal(y.view(torch.int16).cpu().numpy().view(np.uint16), want, "out= values")
    assert_bytes_equal(u8(s8), rs8, "out= e8m0")

    lib = _lib.load()
    xd = to_dev_f32(x)
    big = torch.zeros(H * W + 8, dtype=torch.bfloat16, device="cuda")
    ws = torch.empty(H * W // 128 * 4, dtype=torch.uint8, device="cuda")
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    assert lib.pratchya_quantize_dequantize_workspace_bytes(_lib.DT_F32, 1, H, W, 1, 128) == 0
    rc = lib.pratchya_quantize_dequantize(ctypes.c_void_p(xd.data_ptr()), _lib.DT_F32, 1, H, W, 1, 128,
                                          ctypes.c_void_p(big.data_ptr() + 2), _lib.DT_BF16, 0,
                                          ctypes.c_void_p(s8.data_ptr()), ctypes.c_void_p(s32.data_ptr()),
                                          None, 0, st)
    assert rc == _lib.EINVAL and b"workspace" in lib.pratchya_last_error()
    rc = lib.pratchya_quantize_dequantize(ctypes.c_void_p(xd.data_ptr()), _lib.DT_F32, 1, H, W, 1, 128,
                                          ctypes.c_void_p(big.data_ptr() + 2), _lib.DT_BF16, 0,
                                          ctypes.c_void_p(s8.data_ptr()), ctypes.c_void_p(s32.data_ptr()),
                                          ctypes.c_void_p(ws.data_ptr()), ws.numel(), st)
    assert rc == 0, lib.pratchya_last_error()
    torch.cuda.synchronize()
    got = big[1:1 + H * W].view(torch.int16).cpu().numpy().view(np.uint16).reshape(H, W)
    assert_bytes_equal(got, want, "misaligned values")
    assert_bytes_equal(u8(s8), rs8, "misaligned e8m0")
    assert_f32_bits_equal(f32(s32), rs32, "misaligned G")


def test_argument_errors():
    K = _K()
    x = torch.zeros((16, 128), device="cuda")
    with pytest.raises(ValueError, match="output dtype"):
        K.quantize_dequantize(x, (1, 128), torch.float16)
    with pytest.raises(ValueError, match="does not divide"):
        K.quantize_dequantize(x, (1, 96), torch.float32)


@pytest.mark.parametrize("gdt", ["bfloat16", "float32"])
@pytest.mark.parametrize("shape", [(256, 1024), (2, 128, 512)])
def test_requantize_cotangent(gdt, shape):
    """quantize_impl(dequantize_impl_bwd(g, s8, s32, (1, 128)), (1, 128)) in one
    pass, bit-exact, including zero and NaN e8m0 scales and NaN / inf
    cotangent elements."""
    rng = np.random.default_rng(41)
    y = (rng.standard_normal(shape) * 5).astype(np.float32)
    _, s8, s32 = O.quantize_impl(y, (1, 128))
    s8 = s8.copy()
    s8.reshape(-1)[3] = 0
    s8.reshape(-1)[11] = 0xFF
    g = (rng.standard_normal(shape) * 1e-3).astype(np.float32)
    g.reshape(-1)[100] = np.nan
    g.reshape(-1)[2000] = np.inf
    if gdt == "bfloat16":
        gb = O.f32_to_bf16_bits(g)
        g = O.bf16_bits_to_f32(gb)
        dev = to_dev_bf16(gb)
        g1 = O.bf16_bits_to_f32(O.dequantize_bwd(g, s8, s32, (1, 128), "bfloat16"))
    else:
        dev = to_dev_f32(g)
        g1 = O.dequantize_bwd(g, s8, s32, (1, 128), "float32")
    q8, q_s8, q_s32 = _K().requantize_cotangent(dev, torch.from_numpy(s8).cuda(), torch.from_numpy(s32).cuda())
    torch.cuda.synchronize()
    r8, rs8, rs32 = O.quantize_impl(g1, (1, 128))
    assert_payload_equal(u8(q8), r8, f"{gdt}{shape} payload")
    assert_bytes_equal(u8(q_s8), rs8, f"{gdt}{shape} e8m0")
    assert_f32_bits_equal(f32(q_s32), rs32, f"{gdt}{shape} G")


def test_requantize_cotangent_unsupported_layout():
    from pratchya_amd._lib import PratchyaUnsupported
    g = torch.zeros((4, 128), dtype=torch.bfloat16, device="cuda")   # 4 blocks: K = 4
    with pytest.raises(PratchyaUnsupported):
        _K().requantize_cotangent(g, torch.zeros((1, 4), dtype=torch.uint8, device="cuda"),
                                  torch.ones((1, 1, 1), device="cuda"))
