"""GPU parity of quantize / dequantize / dequantize_bwd against the oracle.

Bit-exact: payload bytes, e8m0 bytes and f32 group maxima (and dequantized
values) must equal the oracle's on the same seeded inputs.  Only a NaN
payload's sign is compared as NaN-ness (unpinned by the reference).
"""
import ctypes

import numpy as np
import pytest
import torch

from oracle import qarr_oracle as O
from tests.helpers import (assert_bytes_equal, assert_f32_bits_equal, assert_payload_equal,
                           bf16_bits, f32, to_dev_bf16, to_dev_f32, u8)

pytestmark = pytest.mark.gpu


def _kernels():
    from pratchya_amd import _kernels
    return _kernels


def run_and_compare(x_host_f32, dev, tgrid, what):
    K = _kernels()
    x8, s8, s32 = K.quantize(dev, tgrid)
    torch.cuda.synchronize()
    r8, rs8, rs32 = O.quantize_impl(x_host_f32, tgrid)
    assert tuple(x8.shape) == r8.shape and tuple(s8.shape) == rs8.shape and tuple(s32.shape) == rs32.shape
    assert_payload_equal(u8(x8), r8, f"{what} payload")
    assert_bytes_equal(u8(s8), rs8, f"{what} e8m0")
    assert_f32_bits_equal(f32(s32), rs32, f"{what} group max")
    return x8, s8, s32


# ---------------------------------------------------------------- conversions
def test_debug_bf16_to_e4m3_software_exhaustive():
    K = _kernels()
    b = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = u8(K.debug_bf16_to_e4m3(torch.from_numpy(b.view(np.int16)).cuda(), 0))
    # the fast-path helper is only fed finite values; compare finite patterns
    finite = (b & 0x7F80) != 0x7F80
    assert_bytes_equal(got[finite], O.bf16_bits_to_e4m3fn(b)[finite], "sw bf16->e4m3")


def test_debug_bf16_to_e4m3_gfx950_instruction_exhaustive():
    """v_cvt_scalef32_pk_fp8_bf16 (scale 1.0) as used by the single-pass
    kernel: RNE and non-saturating on every finite bf16 (overflow -> NaN)."""
    K = _kernels()
    b = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = u8(K.debug_bf16_to_e4m3(torch.from_numpy(b.view(np.int16)).cuda(), 1))
    finite = (b & 0x7F80) != 0x7F80
    assert_bytes_equal(got[finite], O.bf16_bits_to_e4m3fn(b)[finite], "hw bf16->e4m3")


@pytest.mark.parametrize("mode", [0, 1])
def test_debug_f32_to_bf16_ties_and_subnormals(mode):
    """f32 -> bf16 rounding (software and v_cvt_pk_bf16_f32) on exact ties,
    one ulp either side of them, and every subnormal high-half pattern."""
    K = _kernels()
    hi = np.arange(65536, dtype=np.uint32) << 16
    u = np.concatenate([hi | 0x8000, hi | 0x7FFF, hi | 0x8001, np.arange(65536, dtype=np.uint32)])
    x = u.view(np.float32)
    got = K.debug_f32_to_bf16(torch.from_numpy(x).cuda(), mode).cpu().numpy().view(np.uint16)
    nan = np.isnan(x)
    assert_bytes_equal(got[~nan], O.f32_to_bf16_bits(x)[~nan], f"f32->bf16 mode {mode}")
    assert np.all((got[nan] & 0x7FFF) > 0x7F80), f"f32->bf16 mode {mode}: NaN not kept"


def test_debug_f32_to_bf16_software():
    K = _kernels()
    rng = np.random.default_rng(11)
    u = rng.integers(0, 2 ** 32, size=1 << 20, dtype=np.uint64).astype(np.uint32)
    x = u.view(np.float32)
    got = K.debug_f32_to_bf16(torch.from_numpy(x).cuda(), 0).cpu().numpy().view(np.uint16)
    nan = np.isnan(x)
    assert_bytes_equal(got[~nan], O.f32_to_bf16_bits(x)[~nan], "sw f32->bf16")


# ---------------------------------------------------------------- quantize
def test_config2_activation_bf16_1x128_bit_exact():
    bits = O.activation_input(16384, 2048, seed=2)
    run_and_compare(O.bf16_bits_to_f32(bits), to_dev_bf16(bits), (1, 128), "cfg2")


def test_config2_as_3d_batch():
    bits = O.activation_input(4 * 512, 2048, seed=21).reshape(4, 512, 2048)
    run_and_compare(O.bf16_bits_to_f32(bits), to_dev_bf16(bits), (1, 128), "cfg2-3d")


@pytest.mark.parametrize("shape,tgrid", [
    ((1024, 1024), (128, 128)),    # config 1
    ((2048, 8192), (128, 128)),    # config 3 weight (one group over the matrix)
    ((1024, 2048), (128, 1)),      # token-axis grid of config 4
    ((256, 512), (1, 128)),
    ((64, 256), (16, 16)),
    ((96, 64), (32, 32)),
    ((64, 64), (4, 4)),
    ((32, 48), (1, 16)),
    ((16, 40), (1, 1)),
    ((8, 1024), (1, 1024)),
    ((12, 256), (4, 64)),
    ((3, 64, 256), (16, 128)),
])
@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_quantize_grids(shape, tgrid, dtype):
    rng = np.random.default_rng(abs(hash((shape, tgrid))) % 2 ** 32)
    x = (rng.standard_normal(shape) * np.exp2(rng.integers(-8, 8, size=shape[:-1] + (1,)))).astype(np.float32)
    if dtype == "bf16":
        bits = O.f32_to_bf16_bits(x)
        run_and_compare(O.bf16_bits_to_f32(bits), to_dev_bf16(bits), tgrid, f"{shape}{tgrid}bf16")
    else:
        run_and_compare(x, to_dev_f32(x), tgrid, f"{shape}{tgrid}f32")


@pytest.mark.parametrize("shape", [(), (7,), (1, 16), (0, 128), (2, 0, 128)])
def test_quantize_degenerate_shapes(shape):
    rng = np.random.default_rng(1)
    x = rng.standard_normal(shape).astype(np.float32)
    tgrid = (1, 1) if len(shape) < 2 or shape[-1] != 128 else (1, 128)
    if shape == (1, 16):
        tgrid = (1, 16)
    run_and_compare(x, to_dev_f32(x), tgrid, f"degenerate{shape}")


def tensor_1x1():
    """Every case of tgrid (1, 1)'s closed forms (each element its own block
    and group): zeros and -0, values around the 1e-7 clamp and below it,
    subnormals, ordinary values over a wide exponent range, values around
    2^121 (where 128 |x| overflows and the dequantized value is +-inf), the
    largest finite values, +-inf and NaN."""
    rng = np.random.default_rng(111)
    x = (rng.standard_normal((64, 96)) * np.exp2(rng.integers(-40, 40, size=(64, 1)))).astype(np.float32)
    sign = np.where(rng.random(96) < 0.5, -1.0, 1.0)
    x[0] = 0.0
    x[1] = -0.0
    x[2] = rng.uniform(-2e-7, 2e-7, 96)
    x[3] = rng.standard_normal(96) * 1e-38
    x[4] = sign * 2.0 ** 121 * rng.uniform(0.5, 2.0, 96)
    x[5, :5] = [3.4028235e38, -3.4028235e38, np.inf, -np.inf, np.nan]
    c = np.float32(1e-7)
    x[6, :4] = [c, -c, np.nextafter(c, np.float32(0)), np.nextafter(c, np.float32(1))]
    return x.astype(np.float32)


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_quantize_grid_1x1_edges(dtype):
    """tgrid (1, 1) payloads and scales on the elementwise kernel (zeros, the
    clamp, subnormals, values near 2^121 and the largest finite, inf, NaN),
    and at an element count that is not a multiple of 4 (the general
    kernel)."""
    x = tensor_1x1()
    for arr, what in ((x, "(1,1) edges"), (np.ascontiguousarray(x[:7, :13]), "(1,1) odd count")):
        if dtype == "bf16":
            bits = O.f32_to_bf16_bits(arr)
            run_and_compare(O.bf16_bits_to_f32(bits), to_dev_bf16(bits), (1, 1), f"{what} bf16")
        else:
            run_and_compare(arr, to_dev_f32(arr), (1, 1), f"{what} f32")


def edge_tensor(dtype):
    """Rows exercising zeros, -0, clamps, overflow via clamp, NaN, inf and
    near-midpoint f32 quotients; (1,128) groups of 8 blocks."""
    rng = np.random.default_rng(99)
    x = rng.standard_normal((16, 1024)).astype(np.float32)
    x[0] = 0.0
    x[1, :] = -0.0
    x[2, :] = 1e-9                       # whole group clamped
    x[3, :128] = 2.0 ** 127              # r subnormal in other blocks -> e=0, S=1e-7
    x[3, 128:] = 0.5                     #   -> overflow to NaN payloads
    x[4, 5] = np.nan
    x[5, 700] = np.inf
    x[6, 3] = -np.inf
    x[7, :] = rng.standard_normal(1024) * 1e-38   # subnormal-range values
    x[8, 130:140] = 0.0                  # empty values inside a block
    x[9, 128:256] = 0.0                  # empty block in a live group (e=0)
    # rows 10-15: every block holds G at its first element, so S = G and the
    # quotient x / S * 128 is t = RN(x/G*128) with x = RN(t*G/128); t is drawn
    # with its low 16 bits within 4 of the bf16 rounding midpoint.
    for r in range(10, 16):
        G = np.float32(rng.uniform(1, 2))
        hi = (rng.integers(0x3F80, 0x42FF, size=1024).astype(np.uint32) << 16)
        lo = (0x8000 + rng.integers(-4, 5, size=1024)).astype(np.uint32)
        t = (hi | lo).view(np.float32)
        x[r] = (t * G / np.float32(128)).astype(np.float32)
        x[r, 0::128] = G
    if dtype == "bf16":
        x = O.bf16_bits_to_f32(O.f32_to_bf16_bits(x))
    return x


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
@pytest.mark.parametrize("tgrid", [(1, 128), (16, 128), (1, 32)])
def test_quantize_edge_values(dtype, tgrid):
    x = edge_tensor(dtype)
    dev = to_dev_bf16(O.f32_to_bf16_bits(x)) if dtype == "bf16" else to_dev_f32(x)
    run_and_compare(x, dev, tgrid, f"edge-{dtype}-{tgrid}")


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_misaligned_input_takes_general_path(dtype):
    """The C entry point falls back to the multi-pass kernels for buffers that
    are not 16-byte aligned; results are identical."""
    from pratchya_amd import _lib
    lib = _lib.load()
    rng = np.random.default_rng(4)
    H, W = 64, 1024
    x = rng.standard_normal((H, W)).astype(np.float32) * 3
    if dtype == "bf16":
        bits = O.f32_to_bf16_bits(x)
        x = O.bf16_bits_to_f32(bits)
        big = torch.zeros(H * W + 8, dtype=torch.bfloat16, device="cuda")
        big[1:1 + H * W] = to_dev_bf16(bits).reshape(-1)
        code, esz = _lib.DT_BF16, 2
    else:
        big = torch.zeros(H * W + 8, dtype=torch.float32, device="cuda")
        big[1:1 + H * W] = to_dev_f32(x).reshape(-1)
        code, esz = _lib.DT_F32, 4
    x8 = torch.empty(H * W + 8, dtype=torch.uint8, device="cuda")
    s8 = torch.empty(H * W // 128, dtype=torch.uint8, device="cuda")
    s32 = torch.empty(H * W // 1024, dtype=torch.float32, device="cuda")
    ws = torch.empty(H * W // 128 * 4, dtype=torch.uint8, device="cuda")
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    rc = lib.pratchya_quantize(ctypes.c_void_p(big.data_ptr() + esz), code, 1, H, W, 1, 128,
                               ctypes.c_void_p(x8.data_ptr() + 1), ctypes.c_void_p(s8.data_ptr()),
                               ctypes.c_void_p(s32.data_ptr()), ctypes.c_void_p(ws.data_ptr()),
                               ws.numel(), st)
    assert rc == 0, lib.pratchya_last_error()
    torch.cuda.synchronize()
    r8, rs8, rs32 = O.quantize_impl(x, (1, 128))
    assert_payload_equal(u8(x8)[1:1 + H * W].reshape(H, W), r8, "misaligned payload")
    assert_bytes_equal(u8(s8), rs8.reshape(-1), "misaligned e8m0")
    assert_f32_bits_equal(f32(s32), rs32.reshape(-1), "misaligned G")


# ---------------------------------------------------------------- dequantize
@pytest.mark.parametrize("shape,tgrid", [
    ((1024, 1024), (128, 128)), ((512, 2048), (1, 128)), ((1024, 256), (128, 1)),
    ((64, 64), (4, 4)), ((16, 40), (1, 1)), ((2, 32, 256), (16, 128)),
])
@pytest.mark.parametrize("out", ["float32", "bfloat16"])
def test_dequantize_bit_exact(shape, tgrid, out):
    K = _kernels()
    rng = np.random.default_rng(17)
    x = (rng.standard_normal(shape) * 5).astype(np.float32)
    x8, s8, s32 = K.quantize(to_dev_f32(x), tgrid)
    dt = torch.float32 if out == "float32" else torch.bfloat16
    y = K.dequantize(x8, s8, s32, dt, tgrid)
    torch.cuda.synchronize()
    want = O.dequantize_impl(u8(x8), u8(s8), f32(s32), out, tgrid)
    if out == "float32":
        assert_f32_bits_equal(f32(y), want, "dequant f32")
    else:
        assert_bytes_equal(bf16_bits(y), want, "dequant bf16")


def test_dequantize_all_payload_bytes_and_scales():
    """Every e4m3fn byte against a spread of e8m0 exponents (incl. 0 and 255)."""
    K = _kernels()
    q = np.tile(np.arange(256, dtype=np.uint8), (64, 1))           # [64, 256]
    e = np.array([0, 1, 60, 100, 120, 126, 127, 128, 130, 140, 200, 254, 255, 127, 64, 3],
                 dtype=np.uint8)
    n_blk, Kg, M = K.group_layout(64, 256, (1, 128))
    sc8 = np.resize(e, n_blk).reshape(M, Kg)
    G = np.array([1.0, 3.0, 1e-30, 2.0 ** 100, 0.0, 7.5, 1e10, 0.125] * (M // 8 + 1),
                 dtype=np.float32)[:M].reshape(M, 1, 1)
    for out in ("float32", "bfloat16"):
        dt = torch.float32 if out == "float32" else torch.bfloat16
        y = K.dequantize(torch.from_numpy(q).cuda().view(torch.float8_e4m3fn),
                         torch.from_numpy(sc8).cuda().view(torch.float8_e8m0fnu),
                         torch.from_numpy(G).cuda(), dt, (1, 128))
        want = O.dequantize_impl(q, sc8, G, out, (1, 128))
        if out == "float32":
            assert_f32_bits_equal(f32(y), want, "dequant all bytes f32")
        else:
            got = bf16_bits(y)
            nan = (want & 0x7FFF) > 0x7F80
            assert np.array_equal((got & 0x7FFF) > 0x7F80, nan)
            assert_bytes_equal(got[~nan], want[~nan], "dequant all bytes bf16")


@pytest.mark.parametrize("gdtype", ["float32", "bfloat16"])
def test_dequantize_bwd_bit_exact(gdtype):
    K = _kernels()
    rng = np.random.default_rng(23)
    x = (rng.standard_normal((256, 512)) * 2).astype(np.float32)
    x8, s8, s32 = K.quantize(to_dev_f32(x), (1, 128))
    g = rng.standard_normal((256, 512)).astype(np.float32)
    if gdtype == "bfloat16":
        gb = O.f32_to_bf16_bits(g)
        g = O.bf16_bits_to_f32(gb)
        gd = to_dev_bf16(gb)
    else:
        gd = to_dev_f32(g)
    out = K.dequantize_bwd(gd, s8, s32, (1, 128))
    torch.cuda.synchronize()
    want = O.dequantize_bwd(g, u8(s8), f32(s32), (1, 128), gdtype)
    if gdtype == "float32":
        assert_f32_bits_equal(f32(out), want, "dequant_bwd f32")
    else:
        assert_bytes_equal(bf16_bits(out), want, "dequant_bwd bf16")
