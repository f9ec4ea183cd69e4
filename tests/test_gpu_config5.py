"""Config 5 at its real sizes: the RWKV-7 block linears at d_model 4096 over
32768 tokens (batch 8 x seq 4096).

The GEMM kernel is checked at the FFN up-projection [32768,4096] x
[4096,16384] (a (128,128) weight with four group maxima) and the down
projection [32768,16384] x [16384,4096] (four group maxima along K), forward
and the FP8 weight gradient; the quantized Linear composition
(pratchya/_nnx_impl/_module.py:46-50 over pratchya/_qualia/_qarr.py:605-640,
FP8 backward) at [4096,4096] and at the FFN up shape.

Operands are quantized on the GPU (the quantizers' bytes are pinned bit for
bit by the quantize tests) and dequantized on the host by the oracle; the
oracle's float64 product is evaluated on sampled output rows (or channels).
Tolerances are the GEMM contract's: relative Frobenius error <= 1e-2 for bf16
outputs, <= 1e-3 for f32 outputs.
"""
import numpy as np
import pytest
import torch

from oracle import qarr_oracle as O
from tests.helpers import f32, u8

pytestmark = pytest.mark.gpu

BF16_TOL = 1e-2
F32_TOL = 1e-3
T_, D_, F_ = 32768, 4096, 16384


def _K():
    from pratchya_amd import _kernels
    return _kernels


def _randn(shape, std, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    return (torch.randn(shape, generator=g, device="cuda") * std).to(torch.bfloat16)


def _deq_rows(q, rows):
    """Host dequantization of rows ``rows`` of a 2-D (1,128)-quantized triple."""
    x8, s8, s32 = q
    R, C = x8.shape
    nb = C // 128
    ridx = torch.from_numpy(np.asarray(rows)).cuda()
    p = u8(x8[ridx])
    e = u8(s8.view(torch.uint8).reshape(R, nb)[ridx]).reshape(-1, 8)
    g = f32(s32.reshape(R, nb // 8)[ridx]).reshape(-1, 1, 1)
    return O.dequantize_impl(p, e, g, "float32", (1, 128)).astype(np.float64), (e, g)


def _deq_full(q, tgrid):
    x8, s8, s32 = q
    return O.dequantize_impl(u8(x8), u8(s8), f32(s32), "float32", tgrid).astype(np.float64)


def _deq_t128_rows(xt8, s8, s32, T, C, rows):
    """Host dequantization of rows ``rows`` of a transposed (128,1) payload
    [C, T] (quantize_impl(x, (128,1)) of x [T, C] with the payload transposed)."""
    lut = O.e4m3fn_to_f32(np.arange(256, dtype=np.uint8))
    ridx = torch.from_numpy(np.asarray(rows)).cuda()
    q = lut[u8(xt8[ridx])]                                            # [n, T]
    e = u8(s8).reshape(T // 128, C)[:, rows]                          # [T/128, n]
    G = f32(s32).reshape(-1)[(np.arange(T // 128)[:, None] * C + np.asarray(rows)[None, :]) // 8]
    sc = (O.e8m0_to_f32(e) * G).astype(np.float32)                   # [T/128, n]
    return ((q * np.repeat(sc.T, 128, axis=1)).astype(np.float32) / np.float32(128.0)).astype(np.float64)


def _check(got, ref, tol, what):
    err = O.rel_fro(got, ref)
    assert err <= tol, f"{what}: relative Frobenius error {err:.3e} > {tol}"


@pytest.mark.parametrize("proj", ["ffn_up", "ffn_down"])
def test_ffn_forward_gemm_sampled_rows(proj):
    """x (1,128) @ W (128,128) at the d=4096 FFN shapes, bf16 and f32 outputs;
    the weight has four group maxima (along N for the up projection's
    transposed operand rows, along K for the down projection)."""
    K = _K()
    Din, Dout = (D_, F_) if proj == "ffn_up" else (F_, D_)
    xq = K.quantize(_randn((T_, Din), 1.0, 51), (1, 128))
    w = _randn((Din, Dout), 0.02, 52).float()
    w[: Din // 4] *= 16.0                      # group maxima that differ by orders of magnitude
    w[Din // 2: 3 * Din // 4] *= 1.0 / 64.0
    wq = K.quantize(w, (128, 128))
    assert wq[2].numel() == 4
    a = K.operand_rows(*xq, (1, 128))
    b = K.operand_transposed(*wq, (128, 128))
    cb = K.gemm_nt(a, b, torch.bfloat16)
    cf = K.gemm_nt(a, b, torch.float32)
    torch.cuda.synchronize()
    rows = np.sort(np.random.default_rng(5).choice(T_, 64, replace=False))
    xr, _ = _deq_rows(xq, rows)
    ref = xr @ _deq_full(wq, (128, 128))
    ridx = torch.from_numpy(rows).cuda()
    _check(f32(cb[ridx]), ref, BF16_TOL, f"{proj} bf16")
    _check(f32(cf[ridx]), ref, F32_TOL, f"{proj} f32")


@pytest.mark.parametrize("proj", ["ffn_up", "ffn_down"])
def test_ffn_weight_gradient_gemm_sampled(proj):
    """wgrad A^T dY at the FFN shapes, K = 32768 tokens: the stored (1,128)
    activation requantized (128,1) from its fp8 payload, dY requantized (128,1)
    from bf16, f32 output; the oracle product on 16 sampled channels of A
    against 512 sampled channels of dY."""
    K = _K()
    Din, Dout = (D_, F_) if proj == "ffn_up" else (F_, D_)
    a8 = K.quantize(_randn((T_, Din), 1.0, 53), (1, 128))
    dy = _randn((T_, Dout), 1e-3, 54)
    at = K.quantize_t128(*a8)
    dt = K.quantize_t128(dy)
    del dy
    dw = K.gemm_nt(K.operand_t128(*at), K.operand_t128(*dt), torch.float32)
    torch.cuda.synchronize()
    rng = np.random.default_rng(6)
    ch = np.sort(rng.choice(Din, 16, replace=False))
    cols = np.sort(rng.choice(Dout, 512, replace=False))
    ref = _deq_t128_rows(*at, T_, Din, ch) @ _deq_t128_rows(*dt, T_, Dout, cols).T
    got = f32(dw[torch.from_numpy(ch).cuda()][:, torch.from_numpy(cols).cuda()])
    _check(got, ref, F32_TOL, f"{proj} wgrad")


def _linear(x, w):
    """The reference Linear (M:46-50) with the FP8 backward: returns y, x.grad,
    w.grad for the output cotangent built by the caller."""
    from pratchya_amd import qarr as Q
    xx = x.detach().requires_grad_(True)
    ww = w.detach().requires_grad_(True)
    y = (Q.QArrayImpl(xx, (1, 128)) @ Q.QArrayImpl(ww, (128, 128))).astype(torch.bfloat16)
    return xx, ww, y


def _bf16_of(bits):
    return O.bf16_bits_to_f32(bits).astype(np.float64)


@pytest.mark.parametrize("shape", [(D_, D_), (D_, F_)], ids=["rkvo_4096x4096", "ffn_up_4096x16384"])
def test_linear_composition_d4096(shape):
    """QArrayImpl(x,(1,128)) @ W -> astype(bf16) and its FP8 backward at
    config 5's sizes.  Forward and x.grad on 32 sampled token rows against
    the oracle's chain (output requantized (1,128); the cotangent through
    dequantize_impl_bwd with the output's scales, requantized (1,128),
    multiplied by W^T, requantized with x's grid and dequantized to bf16).
    For the [4096,4096] projection, the whole w.grad against the oracle
    product of the token-axis requantized operands, requantized (128,128)."""
    from pratchya_amd import qarr as Q
    K = _K()
    Din, Dout = shape
    x = _randn((T_, Din), 1.0, 55)
    w = _randn((Din, Dout), 0.02, 56)
    g = _randn((T_, Dout), 1e-3, 57)
    prev = Q.get_matmul_backward()
    Q.set_matmul_backward("fp8")
    try:
        xx, ww, y = _linear(x, w)
        y.backward(g)
    finally:
        Q.set_matmul_backward(prev)
    torch.cuda.synchronize()
    xq = K.quantize(x, (1, 128))
    wq = K.quantize(w, (128, 128))
    wd = _deq_full(wq, (128, 128))
    rows = np.sort(np.random.default_rng(7).choice(T_, 32, replace=False))
    ridx = torch.from_numpy(rows).cuda()
    xr, _ = _deq_rows(xq, rows)
    prod = (xr @ wd).astype(np.float32)
    o8, os8, os32 = O.quantize_impl(prod, (1, 128))
    y_ref = _bf16_of(O.dequantize_impl(o8, os8, os32, "bfloat16", (1, 128)))
    _check(f32(y[ridx]), y_ref, BF16_TOL, "forward")
    # dgrad chain on the sampled rows
    g1 = O.bf16_bits_to_f32(O.dequantize_bwd(f32(g[ridx]), os8, os32, (1, 128), "bfloat16"))
    gq = O.quantize_impl(g1, (1, 128))
    gx = (O.dequantize_impl(*gq, "float32", (1, 128)).astype(np.float64) @ wd.T).astype(np.float32)
    gxq = O.quantize_impl(gx, (1, 128))
    sc8 = gxq[1].view(np.uint8).copy()
    sc8[sc8 == 0xFF] = 127                   # quantize_impl_bwd reads NaN e8m0 as 1.0 (Q:521-526)
    gx_ref = _bf16_of(O.dequantize_impl(gxq[0], sc8, gxq[2], "bfloat16", (1, 128)))
    _check(f32(xx.grad[ridx]), gx_ref, BF16_TOL, "x.grad")
    if shape == (D_, D_):
        # wgrad chain: token-axis requantized operands (their bytes are the
        # kernels' own quantize_t128, pinned separately), float64 product,
        # requantized (128,128) and dequantized to bf16 by the oracle
        at = K.quantize_t128(*xq)
        _, gos8, gos32 = K.quantize(_linear_output_f32(xq, wq), (1, 128))
        dt = K.quantize_t128(g, gos8, gos32)
        a_all = _deq_t128_rows(*at, T_, Din, np.arange(Din))
        g_all = _deq_t128_rows(*dt, T_, Dout, np.arange(Dout))
        gw = (a_all @ g_all.T).astype(np.float32)
        gwq = O.quantize_impl(gw, (128, 128))
        sc8 = gwq[1].view(np.uint8).copy()
        sc8[sc8 == 0xFF] = 127
        gw_ref = _bf16_of(O.dequantize_impl(gwq[0], sc8, gwq[2], "bfloat16", (128, 128)))
        _check(f32(ww.grad), gw_ref, BF16_TOL, "w.grad")


def _linear_output_f32(xq, wq):
    """The Linear's f32 product on the GPU kernel (its output quantization's
    scales take the cotangent through dequantize_impl_bwd in the wgrad chain)."""
    K = _K()
    return K.gemm_nt(K.operand_rows(*xq, (1, 128)), K.operand_transposed(*wq, (128, 128)), torch.float32)
