"""GPU parity of the GEMM with the (1, 1) output requantization in its
epilogue (pratchya_gemm_bs_nt_q11): ``QArrayImpl(matmul_impl(x, y),
(1, 1)).astype(dtype)`` (pratchya/_qualia/_qarr.py:104-105, 605-608, 458-506,
541-569), the output of a weight quantized (a, 1): lm_head
(pratchya/_nnx_impl/_model.py:77) and the LoRA projections
(pratchya/_nnx_impl/_module.py:82-84).

The f32 product is the plain GEMM's (same kernel, same arithmetic), so the
fused results must equal the plain GEMM to f32 followed by the one-pass fake
quantization at tgrid (1, 1) bit for bit (values, e8m0 bytes, group maxima),
and equal the oracle's quantize_impl / dequantize_impl of that f32 product.
Operands cover the three B scale layouts the kernel distinguishes ((128, 1)
and (128, 128) weights read transposed, (1, 128) rows), ragged and short M,
N below one tile and not a multiple of 256, leading dimensions, and products
with zero, clamped, overflowing, infinite and NaN rows.
"""
import numpy as np
import pytest
import torch

from oracle import qarr_oracle as O
from tests.helpers import assert_bytes_equal, assert_f32_bits_equal, f32, to_dev_bf16, u8

pytestmark = pytest.mark.gpu


def _K():
    from pratchya_amd import _kernels
    return _kernels


def _b_operand(w, kind):
    """The GEMM's B operand from a weight w [K, N] (bf16 on the device):
    quantized (128, 1) or (128, 128) and read transposed, or its transpose
    quantized (1, 128) as rows.  An operand of fewer than 256 rows is made
    readable for 256 (the kernel reads whole tiles)."""
    K = _K()
    Kd, N = w.shape
    if kind == "rows":
        q = K.quantize(w.t().contiguous(), (1, 128))
        if N < 256:
            full = torch.zeros((256, Kd), dtype=torch.uint8, device=w.device)
            full[:N] = q[0].view(torch.uint8)
            q = (full[:N].view(q[0].dtype),) + tuple(q[1:])
        return K.operand_rows(*q, (1, 128))
    grid = (128, 1) if kind == "w128x1" else (128, 128)
    q = K.quantize(w, grid)
    pt = None
    if N < 256:
        pt = torch.zeros((256, Kd), dtype=torch.uint8, device=w.device)
        pt[:N] = K.transpose_u8(q[0])
        pt = pt[:N]
    return K.operand_transposed(*q, grid, payload_t=pt)


def _operands(M, Kd, N, seed, kind, wscale=0.02):
    K = _K()
    x = O.activation_input(M, Kd, seed=seed)
    w = O.normal_input((Kd, N), wscale, seed=seed + 1)
    xq = K.quantize(to_dev_bf16(x), (1, 128))
    return K.operand_rows(*xq, (1, 128)), _b_operand(to_dev_bf16(w), kind)


def _compare(a, b, dt, what, lead=None):
    K = _K()
    c32 = K.gemm_nt(a, b, torch.float32)
    shaped = c32 if lead is None else c32.reshape(tuple(lead) + (c32.shape[-1],))
    y0, s80, s320 = K.quantize_dequantize(shaped, (1, 1), dt)
    y1, s81, s321 = K.gemm_nt_q11(a, b, dt, lead=lead)
    torch.cuda.synchronize()
    assert y1.shape == c32.shape and y1.dtype == dt
    assert tuple(s81.shape) == tuple(s80.shape) and tuple(s321.shape) == tuple(s320.shape), what
    assert_f32_bits_equal(f32(y1), f32(y0).reshape(y1.shape), f"{what}: values")
    assert_bytes_equal(u8(s81).reshape(-1), u8(s80).reshape(-1), f"{what}: e8m0")
    assert_f32_bits_equal(f32(s321).reshape(-1), f32(s320).reshape(-1), f"{what}: group maxima")
    return c32, y1, s81, s321


# (M, K, N); B scale layouts: "w128x1" groups of 8 rows (kernel BG 1),
# "w128x128" 128-row groups (BG 0), "rows" per-row units (BG 2)
SHAPES = [
    (512, 256, 1024),
    (2048, 512, 4096),     # 128 tiles
    (300, 256, 2048),      # ragged M: the last tile row overlaps the one before
    (100, 128, 512),       # M below one tile
    (1024, 256, 1040),     # N not a multiple of 256: the last tile column overlaps
    (512, 384, 48),        # N below one tile (a LoRA rank)
]


# (a (128, 128) weight grid needs N a multiple of 128)
CASES = [(shape, kind) for shape in SHAPES for kind in ("w128x1", "w128x128", "rows")
         if not (kind == "w128x128" and shape[2] % 128)]


@pytest.mark.parametrize("out", ["bf16", "f32"])
@pytest.mark.parametrize("shape,kind", CASES, ids=lambda c: "x".join(map(str, c)) if isinstance(c, tuple) else c)
def test_fused_equals_gemm_then_fake_quant(shape, out, kind):
    M, Kd, N = shape
    a, b = _operands(M, Kd, N, seed=101, kind=kind)
    dt = torch.bfloat16 if out == "bf16" else torch.float32
    _compare(a, b, dt, f"{shape} {out} {kind}")


@pytest.mark.parametrize("out", ["bf16", "f32"])
def test_fused_matches_oracle(out):
    """The fused outputs against the oracle's quantize_impl and
    dequantize_impl at tgrid (1, 1) of the plain GEMM's f32 product."""
    K = _K()
    a, b = _operands(512, 256, 1024, seed=103, kind="w128x1")
    dt = torch.bfloat16 if out == "bf16" else torch.float32
    c32 = K.gemm_nt(a, b, torch.float32)
    y, s8, s32 = K.gemm_nt_q11(a, b, dt)
    torch.cuda.synchronize()
    q8, e8, g32 = O.quantize_impl(f32(c32), (1, 1))
    assert_bytes_equal(u8(s8).reshape(-1), e8.view(np.uint8).reshape(-1), "e8m0 vs oracle")
    assert_f32_bits_equal(f32(s32).reshape(-1), g32.reshape(-1), "group maxima vs oracle")
    if out == "bf16":
        want = O.bf16_bits_to_f32(O.dequantize_impl(q8, e8, g32, "bfloat16", (1, 1)))
    else:
        want = O.dequantize_impl(q8, e8, g32, "float32", (1, 1))
    assert_f32_bits_equal(f32(y), want, "values vs oracle")


def test_special_rows():
    """Rows whose product is zero (e8m0 0, the value itself), tiny (the 1e-7
    clamp: S = 1e-7, the value requantized), at or above 2^121 (the payload
    +-128 and 128 |c| overflows: +-inf), infinite or NaN (e8m0 255, NaN):
    each of fake_quant11's closed forms against the unfused pass and the
    oracle."""
    K = _K()
    M, Kd, N = 1024, 1024, 1024
    x = O.activation_input(M, Kd, seed=105)
    w = O.normal_input((Kd, N), 1.0, seed=106)    # products ~0.7 of a row's group max
    x8, xs8, xs32 = K.quantize(to_dev_bf16(x), (1, 128))
    x8, xs32 = x8.clone(), xs32.clone()
    x8.view(torch.uint8)[3].zero_()        # row 3: a zero product row
    g = xs32.view(-1)                      # (1,128) with K = 1024: one group per row
    g[5] = 1e-12                           # row 5: products ~1e-13, below the clamp
    g[6] = 1.5e-7                          # row 6: products around the clamp
    g[7] = float("inf")                    # row 7: infinite / NaN products
    g[9] = float("nan")                    # row 9: NaN products
    g[11] = 3e37                           # row 11: products around 2^121 and beyond
    a = K.operand_rows(x8, xs8, xs32, (1, 128))
    b = _b_operand(to_dev_bf16(w), "w128x1")
    for dt in (torch.bfloat16, torch.float32):
        c32, y, s8, s32 = _compare(a, b, dt, f"special rows {dt}")
        c = f32(c32)
        big = np.abs(c[11][np.isfinite(c[11])])
        assert (big >= 2.0 ** 121).any() and (big < 2.0 ** 121).any(), "row 11 spans 2^121"
        assert (np.abs(c[5]) < 1e-7).all() and (c[5] != 0).any(), "row 5 is clamped"
        assert (np.abs(c[6]) < 1e-7).any() and (np.abs(c[6]) >= 1e-7).any(), "row 6 spans the clamp"
        q8, e8, g32 = O.quantize_impl(c, (1, 1))
        assert_bytes_equal(u8(s8).reshape(-1), e8.view(np.uint8).reshape(-1), "e8m0 vs oracle")
        if dt == torch.float32:
            assert_f32_bits_equal(f32(y), O.dequantize_impl(q8, e8, g32, "float32", (1, 1)), "values vs oracle")
        yv = f32(y)
        assert np.isinf(yv[11][np.abs(c[11]) >= 2.0 ** 121]).all()


def test_leading_dimensions():
    """A 3-D product (two slices of 256 rows): the scales shaped per slice as
    quantize_impl returns them ([S, H * N, 1] and [S, H * N, 1, 1])."""
    a, b = _operands(512, 256, 1024, seed=107, kind="w128x1")
    _, y, s8, s32 = _compare(a, b, torch.bfloat16, "3-D", lead=(2, 256))
    assert tuple(s8.shape) == (2, 256 * 1024, 1) and tuple(s32.shape) == (2, 256 * 1024, 1, 1)


def test_rejects_what_it_does_not_fuse():
    K = _K()
    x = O.activation_input(256, 256, seed=109)
    xq = K.quantize(to_dev_bf16(x), (1, 128))
    a = K.operand_rows(*xq, (1, 128))
    w = to_dev_bf16(O.normal_input((256, 1000), 0.02, seed=110))
    b = K.operand_rows(*K.quantize(w.t().contiguous(), (1, 128)), (1, 128))
    with pytest.raises(K.PratchyaUnsupported):
        K.gemm_nt_q11(a, b, torch.bfloat16)                    # N = 1000, not a multiple of 16


# --------------------------------------------------------------------------
# Through the quantized-array API: a Linear whose weight grid is (128, 1)
# --------------------------------------------------------------------------
def _lm_head(x0, w0, g, fused, mode, monkeypatch):
    """``(QArrayImpl(x, (1, 128)) @ QArrayImpl(w, (128, 1))).astype(bf16)``
    (output grid (1, 1), pratchya/_nnx_impl/_model.py:77) and its backward;
    with ``fused`` off the epilogue entry point reports the shape unsupported,
    so the API takes the f32 product and the separate requantization."""
    from pratchya_amd import _kernels as K
    from pratchya_amd import qarr as Q
    prev = Q.get_matmul_backward()
    Q.set_matmul_backward(mode)
    with monkeypatch.context() as mp:
        calls = []
        real = K.gemm_nt_q11

        def spy(*args, **kw):
            calls.append(1)
            if not fused:
                raise K.PratchyaUnsupported("fused (1, 1) requantization switched off")
            return real(*args, **kw)

        mp.setattr(K, "gemm_nt_q11", spy)
        try:
            x = x0.detach().clone().requires_grad_(True)
            w = w0.detach().clone().requires_grad_(True)
            y = (Q.QArrayImpl(x, (1, 128)) @ Q.QArrayImpl(w, (128, 1))).astype(torch.bfloat16)
            y.backward(g)
            torch.cuda.synchronize()
        finally:
            Q.set_matmul_backward(prev)
        assert calls, "the Linear did not reach the (1, 1) epilogue"
        return y.detach(), x.grad, w.grad


@pytest.mark.parametrize("mode", ["fp8", "f32"])
@pytest.mark.parametrize("shape", [(1024, 1024, 2048), (2, 256, 512, 1040)], ids=lambda s: "x".join(map(str, s)))
def test_lm_head_linear_matches_separate_pass(shape, mode, monkeypatch):
    """Output and both gradients with the (1, 1) requantization in the
    epilogue bit-identical to the f32 product followed by the separate
    requantization (the backward reads the same output scales)."""
    *xs, N = shape
    gen = torch.Generator(device="cuda").manual_seed(111)
    x0 = torch.randn(tuple(xs), generator=gen, device="cuda").to(torch.bfloat16)
    w0 = (torch.randn((xs[-1], N), generator=gen, device="cuda") * 0.02).to(torch.bfloat16)
    g = (torch.randn(tuple(xs[:-1]) + (N,), generator=gen, device="cuda") * 1e-3).to(torch.bfloat16)
    got = _lm_head(x0, w0, g, True, mode, monkeypatch)
    want = _lm_head(x0, w0, g, False, mode, monkeypatch)
    for a, b, what in zip(got, want, ("output", "x.grad", "w.grad")):
        assert a.dtype == b.dtype and a.shape == b.shape, what
        assert torch.equal(a.view(torch.int16), b.view(torch.int16)), f"{what} differs with the fused epilogue ({mode})"
