"""GPU parity of the GEMM with the output requantization in its epilogue
(pratchya_gemm_bs_nt_fq): ``QArrayImpl(matmul_impl(x, y), (1, 128)).astype(dtype)``
(pratchya/_qualia/_qarr.py:605-608, 458-506, 541-569; the quantized Linear
output, pratchya/_nnx_impl/_module.py:46-50) and, with fix_nan, the dgrad
cotangent through quantize_impl_bwd (Q:521-526).

The f32 product is the plain GEMM's (same kernel, same arithmetic), so the
fused results must equal the plain GEMM to f32 followed by the one-pass fake
quantization bit for bit (values, e8m0 bytes, group maxima), and equal the
oracle's quantize_impl / dequantize_impl of that f32 product.  Shapes cover
both strip schedules (workgroup partners on one XCD when the tile count is a
multiple of 32, consecutive workgroups otherwise), several rounds of the
persistent schedule, ragged and short M, and products with zero, clamped,
infinite and NaN rows.
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


def _operands(M, Kd, N, seed, wscale=0.02):
    K = _K()
    x = O.activation_input(M, Kd, seed=seed)
    w = O.normal_input((Kd, N), wscale, seed=seed + 1)
    xq = K.quantize(to_dev_bf16(x), (1, 128))
    wq = K.quantize(to_dev_bf16(w), (128, 128))
    return xq, wq


def _unfused(a, b, dt, fix_nan):
    K = _K()
    c32 = K.gemm_nt(a, b, torch.float32)
    y, s8, s32 = K.quantize_dequantize(c32, (1, 128), dt, fix_nan=fix_nan)
    return c32, y, s8, s32


def _compare(a, b, dt, fix_nan, what):
    K = _K()
    c32, y0, s80, s320 = _unfused(a, b, dt, fix_nan)
    y1, s81, s321 = K.gemm_nt_fq(a, b, dt, fix_nan=fix_nan)
    torch.cuda.synchronize()
    assert y1.shape == y0.shape and y1.dtype == dt
    assert_f32_bits_equal(f32(y1), f32(y0), f"{what}: values")
    assert_bytes_equal(u8(s81).reshape(-1), u8(s80).reshape(-1), f"{what}: e8m0")
    assert_f32_bits_equal(f32(s321).reshape(-1), f32(s320).reshape(-1), f"{what}: group maxima")
    return c32, y1, s81, s321


# (M, K, N): tiles (M/256 rounded up) x N/256
SHAPES = [
    (512, 256, 1024),      # 8 tiles: consecutive-workgroup partners
    (2048, 384, 1024),     # 32 tiles: partners on one XCD
    (4096, 512, 2048),     # 128 tiles
    (8192, 256, 4096),     # 512 tiles: two rounds of the persistent schedule
    (1280, 256, 3072),     # 60 tiles, consecutive partners
    (300, 256, 1024),      # ragged M: the last tile row overlaps the first
    (100, 128, 2048),      # M below one tile
]


@pytest.mark.parametrize("fix_nan", [False, True], ids=["fwd", "fixnan"])
@pytest.mark.parametrize("out", ["bf16", "f32"])
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_fused_equals_gemm_then_fake_quant(shape, out, fix_nan):
    K = _K()
    M, Kd, N = shape
    xq, wq = _operands(M, Kd, N, seed=61)
    a = K.operand_rows(*xq, (1, 128))
    b = K.operand_transposed(*wq, (128, 128))
    dt = torch.bfloat16 if out == "bf16" else torch.float32
    _compare(a, b, dt, fix_nan, f"{shape} {out} fix_nan={fix_nan}")


@pytest.mark.parametrize("out", ["bf16", "f32"])
def test_fused_matches_oracle(out):
    """The fused output against the oracle's quantize_impl and
    dequantize_impl of the plain GEMM's f32 product (host arithmetic)."""
    K = _K()
    xq, wq = _operands(512, 256, 2048, seed=63)
    a = K.operand_rows(*xq, (1, 128))
    b = K.operand_transposed(*wq, (128, 128))
    dt = torch.bfloat16 if out == "bf16" else torch.float32
    c32 = K.gemm_nt(a, b, torch.float32)
    y, s8, s32 = K.gemm_nt_fq(a, b, dt)
    torch.cuda.synchronize()
    q8, e8, g32 = O.quantize_impl(f32(c32), (1, 128))
    assert_bytes_equal(u8(s8).reshape(-1), e8.view(np.uint8).reshape(-1), "e8m0 vs oracle")
    assert_f32_bits_equal(f32(s32).reshape(-1), g32.reshape(-1), "group maxima vs oracle")
    if out == "bf16":
        want = O.bf16_bits_to_f32(O.dequantize_impl(q8, e8, g32, "bfloat16", (1, 128)))
    else:
        want = O.dequantize_impl(q8, e8, g32, "float32", (1, 128))
    assert_f32_bits_equal(f32(y), want, "values vs oracle")


@pytest.mark.parametrize("fix_nan", [False, True], ids=["fwd", "fixnan"])
def test_special_rows(fix_nan):
    """Rows whose product is zero (G = 0, e8m0 0), tiny (the 1e-7 clamp),
    infinite or NaN (an activation group max set to inf / NaN: the exact
    path, e8m0 byte 255, and quantize_impl_bwd's repair of it)."""
    K = _K()
    M, Kd, N = 1024, 1024, 1024
    xq, wq = _operands(M, Kd, N, seed=65)
    x8, xs8, xs32 = xq
    x8, xs32 = x8.clone(), xs32.clone()
    x8.view(torch.uint8)[3].zero_()        # row 3: all-zero payload, a zero product row
    g = xs32.view(-1)                      # (1,128) with K = 1024: one group per row
    g[5] = 1e-12                           # row 5: products ~1e-13, clamped output blocks
    g[7] = float("inf")                    # row 7: infinite / NaN products
    g[9] = float("nan")                    # row 9: NaN products
    a = K.operand_rows(x8, xs8, xs32, (1, 128))
    b = K.operand_transposed(*wq, (128, 128))
    _compare(a, b, torch.bfloat16, fix_nan, f"special rows fix_nan={fix_nan}")
    _compare(a, b, torch.float32, fix_nan, f"special rows f32 fix_nan={fix_nan}")


def test_workspace_status_and_reuse():
    """The bounded wait never runs out (status word 0), and two calls in a row
    on one workspace give identical results (the workspace is cleared by the
    call's own kernel)."""
    K = _K()
    lib = K._lib.load()
    M, Kd, N = 2048, 256, 2048
    xq, wq = _operands(M, Kd, N, seed=67)
    a = K.operand_rows(*xq, (1, 128))
    b = K.operand_transposed(*wq, (128, 128))
    ws_bytes = lib.pratchya_gemm_bs_nt_fq_workspace_bytes(M, N)
    assert ws_bytes > 0 and ws_bytes % 256 == 0
    ws = torch.full((ws_bytes,), 0xAB, dtype=torch.uint8, device="cuda")   # not zero: the call clears it
    outs = []
    for _ in range(2):
        y = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
        s8 = torch.empty(M * N // 128, dtype=torch.uint8, device="cuda")
        s32 = torch.empty(M * N // 1024, dtype=torch.float32, device="cuda")
        K._lib.check(lib.pratchya_gemm_bs_nt_fq(
            K._ptr(a.payload), Kd, K._ptr(a.sc8), K._ptr(a.sc32), *a.desc,
            K._ptr(b.payload), Kd, K._ptr(b.sc8), K._ptr(b.sc32), *b.desc,
            M, N, Kd, K._ptr(y), N, K._lib.DT_BF16, 0, K._ptr(s8), K._ptr(s32), K._ptr(ws), ws_bytes,
            K._stream(y)), "gemm_fq")
        torch.cuda.synchronize()
        outs.append((f32(y), u8(s8), f32(s32)))
        n_words = (M // 256) * (N // 1024) * 257 + 1   # maxima, arrival counts, status
        assert lib.pratchya_gemm_bs_nt_fq_status_offset(M, N) == (n_words - 1) * 4
        assert int(ws.view(torch.int32)[n_words - 1].item()) == 0, "strip wait ran out"
    assert_f32_bits_equal(outs[0][0], outs[1][0], "repeat values")
    assert_bytes_equal(outs[0][1], outs[1][1], "repeat e8m0")
    c32, y0, s80, s320 = _unfused(a, b, torch.bfloat16, False)
    assert_f32_bits_equal(outs[1][0], f32(y0), "values vs unfused")


def test_fused_linear_forward_and_dgrad(monkeypatch):
    """The quantized Linear takes the fused path for N a multiple of 1024
    (forward) and for the FP8 dgrad of an input 1024 wide: results equal the
    unfused composition bit for bit."""
    from pratchya_amd import qarr as Q
    K = _K()
    M, Kd, N = 512, 1024, 2048
    x = to_dev_bf16(O.activation_input(M, Kd, seed=69)).reshape(2, M // 2, Kd)
    w = to_dev_bf16(O.normal_input((Kd, N), 0.02, seed=70))
    g = to_dev_bf16(O.normal_input((M, N), 1e-3, seed=71)).reshape(2, M // 2, N)
    results = []
    prev = Q.get_matmul_backward()
    Q.set_matmul_backward("fp8")
    try:
        for fused in (True, False):
            calls = []
            if not fused:
                monkeypatch.setattr(Q, "_linear_forward_fused", lambda *a, **k: None)
                real_bwd = Q._fp8_backward
                monkeypatch.setattr(Q, "_fp8_backward",
                                    lambda *a, **k: real_bwd(*a, **{**k, "x_dtype": None}))
            else:
                real_fq = K.gemm_nt_fq
                monkeypatch.setattr(K, "gemm_nt_fq", lambda *a, **k: calls.append(1) or real_fq(*a, **k))
            xx = x.detach().requires_grad_(True)
            ww = w.detach().requires_grad_(True)
            y = (Q.QArrayImpl(xx, (1, 128)) @ Q.QArrayImpl(ww, (128, 128))).astype(torch.bfloat16)
            y.backward(g)
            torch.cuda.synchronize()
            if fused:
                assert len(calls) == 2             # forward output and x's cotangent
            results.append([f32(t) for t in (y, xx.grad, ww.grad)])
            monkeypatch.undo()
    finally:
        Q.set_matmul_backward(prev)
    for a, b, what in zip(results[0], results[1], ("y", "x.grad", "w.grad")):
        assert_f32_bits_equal(a, b, f"fused vs unfused Linear {what}")


def test_status_word_at_ffn_size():
    """Config 5's FFN up-projection with the requantization in the epilogue
    ([32768, 4096] x [4096, 16384], 512 strips of four tiles exchanged over
    32 persistent rounds): the status tensor receives 0 (no bounded wait ran
    out) and no output is NaN."""
    K = _K()
    M, Kd, N = 32768, 4096, 16384
    g = torch.Generator(device="cuda").manual_seed(5)
    x = torch.randn((M, Kd), generator=g, device="cuda").to(torch.bfloat16)
    w = (torch.randn((Kd, N), generator=g, device="cuda") * 0.02).to(torch.bfloat16)
    a = K.operand_rows(*K.quantize(x, (1, 128)), (1, 128))
    b = K.operand_transposed(*K.quantize(w, (128, 128)), (128, 128))
    del x, w
    st = torch.full((1,), -1, dtype=torch.int32, device="cuda")
    y, s8, s32 = K.gemm_nt_fq(a, b, torch.bfloat16, status=st)
    torch.cuda.synchronize()
    assert int(st.item()) == 0, "strip wait ran out"
    assert not torch.isnan(y).any()
