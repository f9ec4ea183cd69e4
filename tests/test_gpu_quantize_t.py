"""GPU parity of the tgrid (128, 1) requantize, with the payload transposed
([C, T], quantize_t128) and in the input's own layout ([T, C],
quantize_128x1, which the K-major FP8 GEMM reads).

Expected values: the oracle's quantize_impl(x, (128, 1)) (its payload's last
two axes swapped for quantize_t128); for an fp8 input,
quantize_impl(dequantize_impl(x8, sc8, sc32, f32, (1, 128)), (128, 1)).
Bit-exact payload, e8m0 and f32 bytes (a NaN payload byte's sign is compared
as NaN-ness only).  Every case runs both entry points.
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


def u8_dev(t):
    return t.view(torch.uint8)


def oracle_t128(x_f32):
    r8, rs8, rs32 = O.quantize_impl(x_f32, (128, 1))
    return np.ascontiguousarray(np.swapaxes(r8, -1, -2)), rs8, rs32


def check(dev, x_f32, what, x_sc8=None, x_sc32=None):
    xt, s8, s32 = _K().quantize_t128(dev, x_sc8, x_sc32)
    xr, q8, q32 = _K().quantize_128x1(dev, x_sc8, x_sc32)
    torch.cuda.synchronize()
    r8, rs8, rs32 = O.quantize_impl(x_f32, (128, 1))
    rt8 = np.ascontiguousarray(np.swapaxes(r8, -1, -2))
    assert tuple(xt.shape) == rt8.shape and tuple(xr.shape) == r8.shape, (tuple(xt.shape), r8.shape)
    for tag, (a8, a32) in (("transposed", (s8, s32)), ("rows", (q8, q32))):
        assert tuple(a8.shape) == rs8.shape and tuple(a32.shape) == rs32.shape
        assert_bytes_equal(u8(a8), rs8, f"{what} {tag} e8m0")
        assert_f32_bits_equal(f32(a32), rs32, f"{what} {tag} group max")
    assert_payload_equal(u8(xt), rt8, f"{what} transposed payload")
    assert_payload_equal(u8(xr), r8, f"{what} rows payload")
    return xt, s8, s32


@pytest.mark.parametrize("T,C", [(128, 64), (256, 128), (384, 72), (128, 8), (512, 320)])
def test_bf16_activation(T, C):
    bits = O.activation_input(T, C, seed=11)
    check(to_dev_bf16(bits), O.bf16_bits_to_f32(bits), f"bf16 [{T},{C}]")


def test_bf16_slices():
    bits = O.activation_input(2 * 256, 128, seed=12).reshape(2, 256, 128)
    check(to_dev_bf16(bits), O.bf16_bits_to_f32(bits), "bf16 [2,256,128]")


@pytest.mark.parametrize("seed", [0, 1])
def test_f32_normal(seed):
    """Random f32 inputs hit the bf16-midpoint check and its exact redo."""
    x = np.random.default_rng(seed).standard_normal((512, 256)).astype(np.float32)
    check(to_dev_f32(x), x, f"f32 normal seed {seed}")


def test_f32_exact_midpoints():
    """Elements whose x/S*128 is exactly a bf16 rounding midpoint (ties to even)
    and one f32 ulp either side of it."""
    T, C = 128, 64
    x = np.zeros((T, C), np.float32)
    x[0, :] = 1.0                        # G = 1, S = 1 for channel maxima 1
    mids = np.float32(1.0) + np.float32(2.0 ** -8) * np.arange(1, 64, 2, dtype=np.float32)
    v = (mids / 128).astype(np.float32)          # x/S*128 = mid exactly (power-of-two scaling)
    x[1:1 + v.size, 0] = v
    x[1:1 + v.size, 1] = np.nextafter(v, np.float32(2))
    x[1:1 + v.size, 2] = np.nextafter(v, np.float32(0))
    check(to_dev_f32(x), x, "f32 midpoints")


def test_edge_values():
    """Zero groups (G = 0), zero blocks inside a group (e8m0 0), tiny groups
    that hit the 1e-7 clamp, subnormals, NaN / inf."""
    T, C = 256, 64
    x = np.random.default_rng(3).standard_normal((T, C)).astype(np.float32)
    x[:128, 0:8] = 0.0                              # group with G = 0
    x[:128, 8] = 0.0                                # e8m0 0 block in a live group
    x[:128, 16:24] *= np.float32(1e-12)             # clamped group
    x[:128, 24:32] = np.float32(2.0 ** -140) * np.arange(1, 129, dtype=np.float32)[:, None]
    x[5, 32] = np.inf
    x[7, 40] = -np.inf
    x[9, 48] = np.nan
    x[130, 56] = 3.0e38                             # huge group next to normal ones
    check(to_dev_f32(x), x, "f32 edges")
    xb = O.f32_to_bf16_bits(x)
    check(to_dev_bf16(xb), O.bf16_bits_to_f32(xb), "bf16 edges")


@pytest.mark.parametrize("T,C", [(256, 256), (384, 1024)])
def test_fp8_input_requantized_along_tokens(T, C):
    """A stored (1, 128) activation requantized to (128, 1): the fp8 payload is
    dequantized in registers exactly as dequantize_impl does."""
    bits = O.activation_input(T, C, seed=21)
    x8, s8, s32 = O.quantize_impl(O.bf16_bits_to_f32(bits), (1, 128))
    deq = O.dequantize_impl(x8, s8, s32, "float32", (1, 128))
    dev8 = torch.from_numpy(x8).cuda()
    check(dev8, deq, f"fp8 [{T},{C}]", torch.from_numpy(s8).cuda(), torch.from_numpy(s32).cuda())


def test_fp8_input_many_tiles_sampled_token_blocks():
    """An fp8 input with more 128 x 128 tiles than the streaming kernel's grid
    (2 slices x 64 token blocks x 16 channel blocks = 2048 tiles), so that each
    workgroup walks several tiles through both LDS buffers: sampled 128-token
    slabs of each slice against the oracle's dequantize -> (128, 1) quantize of
    the same slab (its groups lie inside the slab)."""
    S, T, C = 2, 8192, 2048
    g = torch.Generator(device="cuda").manual_seed(23)
    x = torch.randn((S, T, C), generator=g, device="cuda")
    x[:, :, 5] *= 50.0
    x8, s8, s32 = _K().quantize(x.to(torch.bfloat16), (1, 128))
    xt, t8, t32 = _K().quantize_t128(x8, s8, s32)
    xr, q8, q32 = _K().quantize_128x1(x8, s8, s32)
    torch.cuda.synchronize()
    x8_h, s8_h, s32_h = u8(x8), u8(s8).reshape(S, -1), f32(s32).reshape(S, -1)
    xt_h, t8_h, t32_h = u8(xt), u8(t8).reshape(S, -1), f32(t32).reshape(S, -1)
    assert torch.equal(u8_dev(q8), u8_dev(t8)) and torch.equal(q32.view(torch.int32), t32.view(torch.int32))
    assert torch.equal(u8_dev(xr).transpose(-1, -2), u8_dev(xt))
    gpr = C // 1024                             # input groups per token row
    for s in range(S):
        for tb in (0, 1, 31, 63):
            rows = slice(tb * 128, (tb + 1) * 128)
            g0 = tb * 128 * gpr
            deq = O.dequantize_impl(x8_h[s, rows], s8_h[s, g0 * 8:(g0 + 128 * gpr) * 8].reshape(-1, 8),
                                    s32_h[s, g0:g0 + 128 * gpr].reshape(-1, 1, 1), "float32", (1, 128))
            r8, rs8, rs32 = oracle_t128(deq)
            what = f"slice {s} slab {tb}"
            assert_payload_equal(xt_h[s, :, rows], r8, f"{what} payload")
            assert_bytes_equal(t8_h[s, tb * C:(tb + 1) * C], rs8.reshape(-1), f"{what} e8m0")
            assert_f32_bits_equal(t32_h[s, tb * C // 8:(tb + 1) * C // 8], rs32.reshape(-1), f"{what} G")


def test_fp8_input_every_payload_byte():
    """Every finite e4m3fn byte (normals, subnormals, zeros of both signs) as
    the stored payload, under several block scales; then the NaN bytes."""
    T, C = 256, 256
    rng = np.random.default_rng(22)
    finite = np.array([b for b in range(256) if (b & 0x7F) != 0x7F], dtype=np.uint8)
    x8 = rng.choice(finite, size=(T, C)).astype(np.uint8)
    x8[:2, :] = np.resize(finite, (2, C))            # each byte at least once
    n_blk = T * C // 128
    s8 = rng.integers(100, 140, size=(n_blk // 8, 8)).astype(np.uint8)
    s32 = rng.uniform(0.5, 4.0, size=(n_blk // 8, 1, 1)).astype(np.float32)
    deq = O.dequantize_impl(x8, s8, s32, "float32", (1, 128))
    dev = [torch.from_numpy(a).cuda() for a in (x8, s8, s32)]
    check(dev[0], deq, "fp8 every byte", dev[1], dev[2])
    x8n = x8.copy()
    x8n[5, 7], x8n[130, 200] = 0x7F, 0xFF
    deqn = O.dequantize_impl(x8n, s8, s32, "float32", (1, 128))
    check(torch.from_numpy(x8n).cuda(), deqn, "fp8 NaN bytes", dev[1], dev[2])


def test_config4_dy_full_size_sampled_token_blocks():
    """Config 4: dY bf16 [16384, 8192] ~ N(0, 1e-3), requantized (128, 1).  The
    full tensor goes through the kernel; token blocks are independent under
    (128, 1) groups, so sampled 128-token slabs are checked against the oracle."""
    T, C = 16384, 8192
    g = torch.Generator(device="cuda").manual_seed(4)
    dy = (torch.randn((T, C), generator=g, device="cuda") * 1e-3).to(torch.bfloat16)
    xt, s8, s32 = _K().quantize_t128(dy)
    xr, q8, q32 = _K().quantize_128x1(dy)
    torch.cuda.synchronize()
    assert torch.equal(u8_dev(q8), u8_dev(s8)) and torch.equal(q32.view(torch.int32), s32.view(torch.int32))
    assert torch.equal(u8_dev(xr).T, u8_dev(xt))
    xt_h = u8(xt)
    s8_h = u8(s8).reshape(-1)
    s32_h = f32(s32).reshape(-1)
    for tb in (0, 1, 77, 127):
        slab = dy[tb * 128:(tb + 1) * 128].contiguous().view(torch.int16).cpu().numpy().view(np.uint16)
        r8, rs8, rs32 = oracle_t128(O.bf16_bits_to_f32(slab))
        assert_payload_equal(xt_h[:, tb * 128:(tb + 1) * 128], r8, f"slab {tb} payload")
        assert_bytes_equal(s8_h[tb * C:(tb + 1) * C], rs8.reshape(-1), f"slab {tb} e8m0")
        assert_f32_bits_equal(s32_h[tb * C // 8:(tb + 1) * C // 8], rs32.reshape(-1), f"slab {tb} G")


@pytest.mark.parametrize("fn", ["quantize_t128", "quantize_128x1"])
def test_argument_errors(fn):
    f = getattr(_K(), fn)
    with pytest.raises(ValueError, match="does not divide"):
        f(torch.zeros((100, 64), dtype=torch.bfloat16, device="cuda"))
    from pratchya_amd._lib import PratchyaError
    with pytest.raises(PratchyaError, match="multiple of 8"):
        f(torch.zeros((128, 12), dtype=torch.bfloat16, device="cuda"))


@pytest.mark.parametrize("T,C", [(256, 256), (384, 1024)])
def test_bf16_cotangent_with_output_scales(T, C):
    """A bf16 cotangent g of a (1, 128)-quantized tensor, given with that
    tensor's scales: dequantize_impl_bwd (bf16((g * 2^(e-127) * G) / 128))
    is applied before the token-axis requantization."""
    rng = np.random.default_rng(31)
    y = (rng.standard_normal((T, C)) * 3).astype(np.float32)
    _, s8, s32 = O.quantize_impl(y, (1, 128))
    s8 = s8.copy()
    s8.reshape(-1)[5] = 0                      # a zero e8m0 (dq = 0) and a NaN one
    s8.reshape(-1)[9] = 0xFF
    gb = O.f32_to_bf16_bits((rng.standard_normal((T, C)) * 1e-3).astype(np.float32))
    gb[3, 17] = 0x7FC0                          # NaN cotangent element
    g1 = O.bf16_bits_to_f32(O.dequantize_bwd(O.bf16_bits_to_f32(gb), s8, s32, (1, 128), "bfloat16"))
    check(to_dev_bf16(gb), g1, f"bf16 cotangent [{T},{C}]", torch.from_numpy(s8).cuda(),
          torch.from_numpy(s32).cuda())


def test_scales_rejected_for_f32_input():
    x = torch.zeros((128, 128), device="cuda")
    with pytest.raises(ValueError, match="input scales"):
        _K().quantize_t128(x, torch.zeros(16, dtype=torch.uint8, device="cuda"), torch.ones(2, device="cuda"))


@pytest.mark.parametrize("kind,T,C", [("bf16", 32768, 2048), ("f32", 32768, 2048), ("fp8", 32768, 2048),
                                      ("bf16_scaled", 16384, 4096), ("bf16", 65536, 1032)])
def test_rows_layout_equals_transposed_at_size(kind, T, C):
    """Sizes where a workgroup of the row-layout kernel walks 2 or more token
    blocks (and, with 1032 channels, a partial last column): every byte of
    quantize_128x1 against quantize_t128's (oracle-checked above) transposed
    back, and the same scales."""
    print(f"rows vs transposed {kind} [{T},{C}]", flush=True)
    K = _K()
    g = torch.Generator(device="cuda").manual_seed(T + C)
    x = torch.randn((T, C), generator=g, device="cuda")
    x[:, 3] *= 40.0
    if kind == "f32":
        args = (x,)
    elif kind == "bf16":
        args = (x.to(torch.bfloat16),)
    elif kind == "fp8":
        args = K.quantize(x.to(torch.bfloat16), (1, 128))
    else:
        y8 = K.quantize((x * 3).to(torch.bfloat16), (1, 128))
        args = ((x * 1e-3).to(torch.bfloat16), y8[1], y8[2])
    xt, s8, s32 = K.quantize_t128(*args)
    xr, q8, q32 = K.quantize_128x1(*args)
    torch.cuda.synchronize()
    assert torch.equal(u8_dev(q8), u8_dev(s8)), "e8m0 bytes differ"
    assert torch.equal(q32.view(torch.int32), s32.view(torch.int32)), "group maxima differ"
    assert torch.equal(u8_dev(xr), u8_dev(xt).T), "payloads differ"
