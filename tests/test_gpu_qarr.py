"""GPU parity of the quantized-array API (pratchya_amd.qarr) against the
oracle's composition of the reference's steps (pratchya/_qualia/_qarr.py).

Quantize / dequantize / requantize results are bit-exact.  Anything that goes
through a GEMM is compared by relative Frobenius error (1e-2, the contract's
bf16 bar): the reference's f32 dot and the MFMA kernel sum in different
orders, which can move an element of a requantized result across a rounding
boundary.
"""
import numpy as np
import pytest
import torch

from oracle import qarr_oracle as O
from tests.helpers import (assert_bytes_equal, assert_f32_bits_equal, assert_payload_equal, bf16_bits,
                           f32, to_dev_bf16, to_dev_f32, u8)

pytestmark = pytest.mark.gpu

TOL = 1e-2


@pytest.fixture
def Q():
    from pratchya_amd import qarr
    prev = qarr.get_matmul_backward()
    yield qarr
    qarr.set_matmul_backward(prev)


def oq(x, grid):
    return O.quantize_impl(np.asarray(x, np.float32), grid)


def odq(trip, grid, dtype="float32"):
    return O.dequantize_impl(*trip, dtype, grid)


def triple(q):
    v, s8, s32 = q._tree_flatten()[0]
    return u8(v), u8(s8), f32(s32)


def assert_triple(q, want, what):
    got = triple(q)
    assert_payload_equal(got[0], want[0], f"{what} payload")
    assert_bytes_equal(got[1], want[1], f"{what} e8m0")
    assert_f32_bits_equal(got[2], want[2], f"{what} G")


def rel(a, b):
    return O.rel_fro(np.asarray(a, np.float64), np.asarray(b, np.float64))


# --------------------------------------------------------------- construction
def test_construct_and_dequantize_bit_exact(Q):
    bits = O.activation_input(256, 512, seed=31)
    x = to_dev_bf16(bits)
    q = Q.QArrayImpl(x, (1, 128))
    ref = oq(O.bf16_bits_to_f32(bits), (1, 128))
    assert_triple(q, ref, "QArrayImpl(x, (1,128))")
    assert q.shape == (256, 512) and q.size == 256 * 512 and q.tgrid == (1, 128)
    assert q.dtype == torch.float8_e4m3fn
    assert_bytes_equal(bf16_bits(q.astype(torch.bfloat16)), odq(ref, (1, 128), "bfloat16"), "astype bf16")
    assert_f32_bits_equal(f32(q.dequantize(torch.float32)), odq(ref, (1, 128)), "dequantize f32")
    # copy construction shares the buffers (Q:20-24)
    q2 = Q.QArrayImpl(q)
    assert q2.get_value() is q.get_value() and q2.tgrid == q.tgrid


def test_three_d_slices(Q):
    x = np.random.default_rng(1).standard_normal((3, 256, 256)).astype(np.float32)
    q = Q.QArrayImpl(to_dev_f32(x), (128, 128))
    assert_triple(q, oq(x, (128, 128)), "3-D")


def test_module_functions(Q):
    x = np.random.default_rng(2).standard_normal((128, 384)).astype(np.float32)
    t = Q.quantize_impl(to_dev_f32(x), (1, 128))
    ref = oq(x, (1, 128))
    assert_payload_equal(u8(t[0]), ref[0], "quantize_impl")
    y = Q.dequantize_impl(*t, torch.bfloat16, (1, 128))
    assert_bytes_equal(bf16_bits(y), odq(ref, (1, 128), "bfloat16"), "dequantize_impl")


# ------------------------------------------------------------------ Linear
def _linear_case(seed=7, M=512, Kd=1024, N=768):
    x = O.activation_input(M, Kd, seed=seed)
    w = O.normal_input((Kd, N), 0.02, seed=seed + 1)
    g = O.normal_input((M, N), 1.0, seed=seed + 2)
    return x, w, g


def _linear_reference(xb, wb, gb, out_scales, fp8_bwd=False):
    """The reference's Linear (M:46-50) on the oracle: forward, and the
    cotangents of x and W for the output cotangent g.

    The output cotangent reaching the matmul is g * 2^(e-127) * G / 128 with
    the *output's* block scales (Q:596-599 through Q:518-519), which jump by 2x
    when an output block's m/G sits at a power of two -- where the f32 dot and
    the MFMA can round to different sides.  The backward is therefore checked
    from the output scales the forward under test produced (``out_scales``);
    the forward is checked on its own."""
    xq = oq(O.bf16_bits_to_f32(xb), (1, 128))
    wq = oq(O.bf16_bits_to_f32(wb), (128, 128))
    xd, wd = odq(xq, (1, 128)).astype(np.float64), odq(wq, (128, 128)).astype(np.float64)
    out32 = (xd @ wd).astype(np.float32)
    outq = oq(out32, (1, 128))
    y = odq(outq, (1, 128), "bfloat16")
    # dequantize_impl_bwd in g.dtype (bf16), passed through the output quantize
    o8, o32 = out_scales
    g1 = O.bf16_bits_to_f32(O.dequantize_bwd(O.bf16_bits_to_f32(gb), o8, o32, (1, 128), "bfloat16"))
    if fp8_bwd:
        gd = odq(oq(g1, (1, 128)), (1, 128)).astype(np.float64)
        gx = gd @ wd.T
        xt = odq(oq(xd.astype(np.float32), (128, 1)), (128, 1)).astype(np.float64)
        gt = odq(oq(g1, (128, 1)), (128, 1)).astype(np.float64)
        gw = xt.T @ gt
    else:
        gx = g1.astype(np.float64) @ wd.T
        gw = xd.T @ g1.astype(np.float64)
    gx = odq(oq(gx.astype(np.float32), (1, 128)), (1, 128))
    gw = odq(oq(gw.astype(np.float32), (128, 128)), (128, 128))
    return y, O.bf16_round(gx), O.bf16_round(gw)


@pytest.mark.parametrize("mode", ["f32", "fp8"])
def test_linear_forward_backward(Q, mode):
    Q.set_matmul_backward(mode)
    xb, wb, gb = _linear_case()
    x = to_dev_bf16(xb).requires_grad_(True)
    w = to_dev_bf16(wb).requires_grad_(True)
    W = Q.QArrayImpl(w, (128, 128))
    out = Q.QArrayImpl(x, (1, 128)) @ W
    y = out.astype(torch.bfloat16)
    y.backward(to_dev_bf16(gb))
    _, o8, o32 = triple(out)
    y_ref, gx_ref, gw_ref = _linear_reference(xb, wb, gb, (o8, o32), fp8_bwd=(mode == "fp8"))
    assert y.dtype == torch.bfloat16 and x.grad.dtype == torch.bfloat16
    assert rel(f32(y), O.bf16_bits_to_f32(y_ref)) <= TOL
    assert rel(f32(x.grad), gx_ref) <= TOL, rel(f32(x.grad), gx_ref)
    assert rel(f32(w.grad), gw_ref) <= TOL, rel(f32(w.grad), gw_ref)


def _linear_reference_grid(xb, wb, gb, blk, out_scales):
    """The reference Linear (M:46-50) with the preset grids of block size
    ``blk``: x quantized (1, blk), W (blk, blk), the product requantized
    (1, blk) (Q:104-105); the backward's f32 dots (Q:618-622), x's cotangent
    requantized (1, blk) and W's (blk, blk) (Q:637-638), each dequantized to
    bf16 (Q:525).  The output cotangent is taken through dequantize_impl_bwd
    with the output scales of the forward under test (see _linear_reference)."""
    gx_, gw_ = (1, blk), (blk, blk)
    xq = oq(O.bf16_bits_to_f32(xb), gx_)
    wq = oq(O.bf16_bits_to_f32(wb), gw_)
    xd, wd = odq(xq, gx_).astype(np.float64), odq(wq, gw_).astype(np.float64)
    y = odq(oq((xd @ wd).astype(np.float32), (1, blk)), (1, blk), "bfloat16")
    o8, o32 = out_scales
    g1 = O.bf16_bits_to_f32(O.dequantize_bwd(O.bf16_bits_to_f32(gb), o8, o32, (1, blk), "bfloat16"))
    gx = odq(oq((g1.astype(np.float64) @ wd.T).astype(np.float32), gx_), gx_)
    gw = odq(oq((xd.T @ g1.astype(np.float64)).astype(np.float32), gw_), gw_)
    return y, O.bf16_round(gx), O.bf16_round(gw)


@pytest.mark.parametrize("mode", ["f32", "fp8"])
@pytest.mark.parametrize("blk", [16, 32])
def test_linear_preset_block_sizes(Q, mode, blk, monkeypatch):
    """The reference's presets (pratchya/preset.py:21, :30, :39, :48: blksize 16
    and 32): Linear's x (1, blk) @ W (blk, blk), forward and both backward
    modes against the oracle.  These grids' f32 group maxima change along K
    every 16 (x (1, 16): one block per group), 64 (x (1, 32): two blocks) or
    32 K values (W (32, 32) read transposed), below the 128-wide K block
    whose scale the FP8 kernel applies, so their products run on the exact
    f32 product over bf16 pieces in either mode (asserted: no FP8 GEMM)."""
    Q.set_matmul_backward(mode)
    calls = []
    for name in ("gemm_nt", "gemm_nt_fq", "gemm_nt_q11"):
        real = getattr(Q.K, name)
        monkeypatch.setattr(Q.K, name, (lambda r: (lambda *a, **k: calls.append(1) or r(*a, **k)))(real))
    xb, wb, gb = _linear_case(seed=11, M=256, Kd=512, N=384)
    x = to_dev_bf16(xb).requires_grad_(True)
    w = to_dev_bf16(wb).requires_grad_(True)
    out = Q.QArrayImpl(x, (1, blk)) @ Q.QArrayImpl(w, (blk, blk))
    y = out.astype(torch.bfloat16)
    y.backward(to_dev_bf16(gb))
    assert not calls, "a non-128 grid reached the FP8 GEMM"
    _, o8, o32 = triple(out)
    assert out.tgrid == (1, blk)
    y_ref, gx_ref, gw_ref = _linear_reference_grid(xb, wb, gb, blk, (o8, o32))
    assert rel(f32(y), O.bf16_bits_to_f32(y_ref)) <= TOL
    assert rel(f32(x.grad), gx_ref) <= TOL, rel(f32(x.grad), gx_ref)
    assert rel(f32(w.grad), gw_ref) <= TOL, rel(f32(w.grad), gw_ref)


def test_fp8_dgrad_with_narrow_weight_row_groups(Q, monkeypatch):
    """x (1, 128) @ W (16, 128) in the "fp8" backward: W's scale groups span
    16 rows, which the requantizing epilogue does not take; the dgrad still
    runs on the FP8 kernel (gemm_nt) with the requantization as its own
    pass, and the results match the oracle's FP8 backward chain."""
    Q.set_matmul_backward("fp8")
    calls = []
    real = Q.K.gemm_nt
    monkeypatch.setattr(Q.K, "gemm_nt", lambda *a, **k: calls.append(1) or real(*a, **k))
    xb, wb, gb = _linear_case(seed=13, M=256, Kd=1024, N=512)
    x = to_dev_bf16(xb).requires_grad_(True)
    w = to_dev_bf16(wb).requires_grad_(True)
    out = Q.QArrayImpl(x, (1, 128)) @ Q.QArrayImpl(w, (16, 128))
    y = out.astype(torch.bfloat16)
    n_fwd = len(calls)
    y.backward(to_dev_bf16(gb))
    assert len(calls) - n_fwd == 2, "dgrad and wgrad on the FP8 kernel"
    _, o8, o32 = triple(out)
    wq = oq(O.bf16_bits_to_f32(wb), (16, 128))
    wd = odq(wq, (16, 128)).astype(np.float64)
    xd = odq(oq(O.bf16_bits_to_f32(xb), (1, 128)), (1, 128)).astype(np.float64)
    g1 = O.bf16_bits_to_f32(O.dequantize_bwd(O.bf16_bits_to_f32(gb), o8, o32, (1, 128), "bfloat16"))
    gd = odq(oq(g1, (1, 128)), (1, 128)).astype(np.float64)
    gx = O.bf16_round(odq(oq((gd @ wd.T).astype(np.float32), (1, 128)), (1, 128)))
    xt = odq(oq(xd.astype(np.float32), (128, 1)), (128, 1)).astype(np.float64)
    gt = odq(oq(g1, (128, 1)), (128, 1)).astype(np.float64)
    gw = O.bf16_round(odq(oq((xt.T @ gt).astype(np.float32), (16, 128)), (16, 128)))
    assert rel(f32(x.grad), gx) <= TOL
    assert rel(f32(w.grad), gw) <= TOL


# lm_head: Linear(hidden, vocab, (blksize, 1)) (_model.py:77); LoRA:
# Linear(hidden, rank, (a, 1)) then Linear(rank, hidden, (b, 1)) (M:75-88).
# The product's grid is (1, 1): every element is its own group.
# (K, N, tokens): widths below one 256-wide tile (LoRA ranks 32 and 128) and
# not a multiple of it (a 1008-entry vocabulary, 300 tokens) run on the FP8
# kernel's edge tiles.
ODD_LINEARS = {"lm_head": (256, 512, 256), "lm_head_ragged": (256, 1008, 300), "lora_down": (1024, 128, 256),
               "lora_down_r32": (1024, 32, 300), "lora_up": (128, 1024, 256)}


@pytest.mark.parametrize("mode", ["f32", "fp8"])
@pytest.mark.parametrize("case", sorted(ODD_LINEARS))
def test_odd_grid_linears(Q, mode, case, monkeypatch):
    Q.set_matmul_backward(mode)
    Kd, N, M = ODD_LINEARS[case]
    calls = []
    real, real11 = Q.K.gemm_nt, Q.K.gemm_nt_q11
    monkeypatch.setattr(Q.K, "gemm_nt", lambda *a, **k: calls.append("nt") or real(*a, **k))
    monkeypatch.setattr(Q.K, "gemm_nt_q11", lambda *a, **k: calls.append("q11") or real11(*a, **k))
    xb, wb, gb = _linear_case(seed=31, M=M, Kd=Kd, N=N)
    x = to_dev_bf16(xb).requires_grad_(True)
    w = to_dev_bf16(wb).requires_grad_(True)
    out = Q.QArrayImpl(x, (1, 128)) @ Q.QArrayImpl(w, (128, 1))
    assert out.tgrid == (1, 1)
    y = out.astype(torch.bfloat16)
    # the forward ran on the FP8 kernel, with the (1, 1) requantization in its
    # epilogue (every width here is a multiple of 16)
    assert calls == ["q11"], calls
    y.backward(to_dev_bf16(gb))
    _, o8, o32 = triple(out)
    xq, wq = oq(O.bf16_bits_to_f32(xb), (1, 128)), oq(O.bf16_bits_to_f32(wb), (128, 1))
    xd, wd = odq(xq, (1, 128)).astype(np.float64), odq(wq, (128, 1)).astype(np.float64)
    out32 = (xd @ wd).astype(np.float32)
    y_ref = O.bf16_bits_to_f32(odq(oq(out32, (1, 1)), (1, 1), "bfloat16"))
    assert rel(f32(y), y_ref) <= TOL
    # the product's (1,1) scales: e8m0 127 and G = |element| (r = 1) wherever |out| >= 1e-7
    big = np.abs(out32) > 1e-3
    assert np.all(o8.reshape(out32.shape)[big] == 127)
    g1 = O.bf16_bits_to_f32(O.dequantize_bwd(O.bf16_bits_to_f32(gb), o8, o32, (1, 1), "bfloat16")).astype(np.float64)
    gx = O.bf16_round(odq(oq((g1 @ wd.T).astype(np.float32), (1, 128)), (1, 128)))
    gw = O.bf16_round(odq(oq((xd.T @ g1).astype(np.float32), (128, 1)), (128, 1)))
    assert rel(f32(x.grad), gx) <= TOL, rel(f32(x.grad), gx)
    assert rel(f32(w.grad), gw) <= TOL, rel(f32(w.grad), gw)


def test_linear_forward_uses_the_fp8_kernel(Q, monkeypatch):
    """A (1,128) x (128,128) forward of tile-multiple shape must run the MFMA
    GEMM, not the dequantize-and-matmul path."""
    calls = []
    real = Q.K.gemm_nt
    monkeypatch.setattr(Q.K, "gemm_nt", lambda *a, **k: calls.append(1) or real(*a, **k))
    xb, wb, _ = _linear_case(M=256, Kd=256, N=256)
    prod = Q.QArrayImpl(to_dev_bf16(xb), (1, 128)) @ Q.QArrayImpl(to_dev_bf16(wb), (128, 128))
    prod.astype(torch.bfloat16)              # the fused Linear output
    assert len(calls) == 1
    prod.get_value()                         # the materialised quantized product
    assert len(calls) == 2


@pytest.mark.parametrize("M,Kd,N", [(512, 1024, 768), (1024, 256, 384)])
def test_fp8_wgrad_layouts_same_bits(Q, M, Kd, N):
    """The fp8 weight gradient from (128, 1) payloads in the [tokens, channels]
    layout read K-major, and from transposed payloads read K-contiguous: the
    same MFMA K order per lane, so W's cotangent has the same bits (x's does
    not depend on the layout)."""
    assert Kd <= Q._WGRAD_K_MAJOR_ROWS          # the K-major path is taken
    Q.set_matmul_backward("fp8")
    xb, wb, gb = _linear_case(seed=21, M=M, Kd=Kd, N=N)
    grads = []
    try:
        for k_major in (True, False):
            Q._wgrad_k_major = k_major
            x = to_dev_bf16(xb).requires_grad_(True)
            w = to_dev_bf16(wb).requires_grad_(True)
            y = (Q.QArrayImpl(x, (1, 128)) @ Q.QArrayImpl(w, (128, 128))).astype(torch.bfloat16)
            y.backward(to_dev_bf16(gb))
            grads.append((w.grad.clone(), x.grad.clone()))
    finally:
        Q._wgrad_k_major = True
    torch.cuda.synchronize()
    assert torch.equal(grads[0][0].view(torch.int16), grads[1][0].view(torch.int16)), "W cotangents differ"
    assert torch.equal(grads[0][1].view(torch.int16), grads[1][1].view(torch.int16))


@pytest.mark.parametrize("mode", ["f32", "fp8"])
@pytest.mark.parametrize("xdtype", ["bf16", "f32"])
def test_fused_linear_matches_materialised_composition(Q, mode, xdtype):
    """``(QArrayImpl(x) @ W).astype(x.dtype)`` runs as one node; forcing the
    quantized product first (payload access) runs the step-by-step graph.
    Output and both input cotangents agree bit for bit."""
    Q.set_matmul_backward(mode)
    xb, wb, gb = _linear_case(seed=13)
    dt = torch.bfloat16 if xdtype == "bf16" else torch.float32
    results = []
    for materialise in (False, True):
        x = to_dev_bf16(xb).to(dt).requires_grad_(True)
        w = to_dev_bf16(wb).requires_grad_(True)
        prod = Q.QArrayImpl(x, (1, 128)) @ Q.QArrayImpl(w, (128, 128))
        assert prod.shape == (512, 768) and prod.dtype == torch.float8_e4m3fn
        assert ("_operands" in prod.__dict__) is True      # shape / dtype do not materialise
        if materialise:
            prod.get_value()
        y = prod.astype(dt)
        if not materialise:
            y2 = prod.astype(dt)                 # one product per dtype, returned as a copy
            assert y2 is not y and torch.equal(y2, y)
        y.backward(to_dev_bf16(gb).to(dt))
        assert x.grad.dtype == dt and w.grad.dtype == torch.bfloat16
        results.append([t.detach().float().cpu().numpy() for t in (y, x.grad, w.grad)])
    for a, b, what in zip(results[0], results[1], ("y", "x.grad", "w.grad")):
        assert_f32_bits_equal(a, b, f"fused vs materialised {what} ({mode}, {xdtype})")


def test_lazy_product_results_are_independent(Q):
    """A second dequantization of a lazy product is not changed by an in-place
    change of the first (jnp arrays are immutable; torch tensors are not)."""
    xb, wb, _ = _linear_case(seed=15, M=256, Kd=256, N=256)
    with torch.no_grad():
        prod = Q.QArrayImpl(to_dev_bf16(xb), (1, 128)) @ Q.QArrayImpl(to_dev_bf16(wb), (128, 128))
        y1 = prod.astype(torch.bfloat16)
        want = y1.clone()
        y1.add_(1.0)
        y2 = prod.astype(torch.bfloat16)
        assert torch.equal(y2, want)
        y2.mul_(2.0)
        assert torch.equal(prod.astype(torch.bfloat16), want)


def test_fused_linear_without_grad(Q):
    xb, wb, _ = _linear_case(seed=14, M=256, Kd=256, N=512)
    with torch.no_grad():
        prod = Q.QArrayImpl(to_dev_bf16(xb), (1, 128)) @ Q.QArrayImpl(to_dev_bf16(wb), (128, 128))
        y = prod.astype(torch.bfloat16)
        trip = triple(prod)
    assert_bytes_equal(bf16_bits(y), odq(trip, (1, 128), "bfloat16"), "no-grad fused output")


def test_batched_activation(Q):
    """[B, T, K] @ W: slices flatten into GEMM rows; W's cotangent sums the batch."""
    Q.set_matmul_backward("f32")
    xb = O.activation_input(2 * 256, 256, seed=9).reshape(2, 256, 256)
    wb = O.normal_input((256, 256), 0.02, seed=10)
    x = to_dev_bf16(xb).requires_grad_(True)
    w = to_dev_bf16(wb).requires_grad_(True)
    out = Q.QArrayImpl(x, (1, 128)) @ Q.QArrayImpl(w, (128, 128))
    assert out.shape == (2, 256, 256)
    out.astype(torch.float32).sum().backward()
    xq = oq(O.bf16_bits_to_f32(xb), (1, 128))
    wq = oq(O.bf16_bits_to_f32(wb), (128, 128))
    ref = odq(xq, (1, 128)).astype(np.float64) @ odq(wq, (128, 128)).astype(np.float64)
    ref = odq(oq(ref.astype(np.float32), (1, 128)), (1, 128))   # the output is requantized (Q:104-105)
    assert rel(f32(out.astype(torch.float32)), ref) <= TOL
    assert w.grad is not None and x.grad is not None


# -------------------------------------------------------------- mixed / fp8
def test_mixed_matmuls(Q):
    x = np.random.default_rng(3).standard_normal((128, 256)).astype(np.float32)
    y = np.random.default_rng(4).standard_normal((256, 64)).astype(np.float32)
    q = Q.QArrayImpl(to_dev_f32(x), (1, 128))
    yd = to_dev_f32(y).requires_grad_(True)
    out = q @ yd
    ref = odq(oq(x, (1, 128)), (1, 128)).astype(np.float64) @ y
    assert rel(f32(out), ref) <= 1e-5
    out.sum().backward()
    assert rel(f32(yd.grad), odq(oq(x, (1, 128)), (1, 128)).T @ np.ones((128, 64))) <= 1e-5
    z = torch.ones((32, 128), device="cuda") @ q          # rmatmul_mixed via __rmatmul__
    assert tuple(z.shape) == (32, 256)


def test_fp8_matmul(Q):
    rng = np.random.default_rng(5)
    x = rng.standard_normal((256, 256)).astype(np.float32)
    y = rng.standard_normal((256, 256)).astype(np.float32)
    g = rng.standard_normal((256, 256)).astype(np.float32)
    xd = to_dev_f32(x).requires_grad_(True)
    yd = to_dev_f32(y).requires_grad_(True)
    out = Q.fp8_matmul(xd, yd, (1, 128))

    def fwd(a, b):
        p = odq(oq(a, (1, 128)), (1, 128)).astype(np.float64) @ odq(oq(b, (1, 128)), (1, 128)).astype(np.float64)
        return odq(oq(p.astype(np.float32), (1, 128)), (1, 128))

    assert rel(f32(out), fwd(x, y)) <= TOL
    out.backward(to_dev_f32(g))
    assert rel(f32(xd.grad), fwd(g, y.T.copy())) <= TOL
    assert rel(f32(yd.grad), fwd(x.T.copy(), g)) <= TOL


@pytest.mark.parametrize("tgrid", [(1, 16), (1, 32)])
def test_fp8_matmul_default_and_preset_grids(Q, tgrid):
    """fp8_matmul at its default tgrid (1, 16) (Q:766) and at (1, 32): forward
    and the backward's products of the transposed raw inputs, each quantized
    with the same grid (Q:784-789), against the oracle's chain."""
    rng = np.random.default_rng(9)
    x = rng.standard_normal((256, 384)).astype(np.float32)
    y = rng.standard_normal((384, 128)).astype(np.float32)
    g = rng.standard_normal((256, 128)).astype(np.float32)
    xd = to_dev_f32(x).requires_grad_(True)
    yd = to_dev_f32(y).requires_grad_(True)
    out = Q.fp8_matmul(xd, yd) if tgrid == (1, 16) else Q.fp8_matmul(xd, yd, tgrid)

    def fwd(a, b):
        p = odq(oq(a, tgrid), tgrid).astype(np.float64) @ odq(oq(b, tgrid), tgrid).astype(np.float64)
        return odq(oq(p.astype(np.float32), tgrid), tgrid)

    assert rel(f32(out), fwd(x, y)) <= TOL
    out.backward(to_dev_f32(g))
    assert rel(f32(xd.grad), fwd(g, y.T.copy())) <= TOL
    assert rel(f32(yd.grad), fwd(x.T.copy(), g)) <= TOL


def test_fp8_matmul_transposed_quantizer(Q):
    """Token counts that are multiples of 1024: the backward's transposed
    operands are quantized by quantize_t1x128 (x^T and y^T), with the same
    expected values as the general path."""
    rng = np.random.default_rng(8)
    x = rng.standard_normal((1024, 1024)).astype(np.float32)
    y = rng.standard_normal((1024, 512)).astype(np.float32)
    g = rng.standard_normal((1024, 512)).astype(np.float32)
    xd = to_dev_f32(x).requires_grad_(True)
    yd = to_dev_f32(y).requires_grad_(True)
    out = Q.fp8_matmul(xd, yd, (1, 128))

    def fwd(a, b):
        p = odq(oq(a, (1, 128)), (1, 128)).astype(np.float64) @ odq(oq(b, (1, 128)), (1, 128)).astype(np.float64)
        return odq(oq(p.astype(np.float32), (1, 128)), (1, 128))

    out.backward(to_dev_f32(g))
    assert rel(f32(xd.grad), fwd(g, y.T.copy())) <= TOL
    assert rel(f32(yd.grad), fwd(x.T.copy(), g)) <= TOL
    # the quantized transpose is the general quantizer's, byte for byte
    qt = Q._quantized_transpose(xd.detach(), (1, 128))
    assert_triple(qt, oq(np.ascontiguousarray(x.T), (1, 128)), "x^T")


# ------------------------------------------------------------ elementwise
@pytest.mark.parametrize("opname", ["add", "sub", "mul", "truediv"])
def test_elementwise_bit_exact(Q, opname):
    rng = np.random.default_rng(6)
    a = rng.standard_normal((128, 256)).astype(np.float32)
    b = rng.standard_normal((128, 256)).astype(np.float32) + np.float32(3.0)
    qa, qb = Q.QArrayImpl(to_dev_f32(a), (1, 128)), Q.QArrayImpl(to_dev_f32(b), (1, 128))
    out = {"add": qa + qb, "sub": qa - qb, "mul": qa * qb, "truediv": qa / qb}[opname]
    da, db = odq(oq(a, (1, 128)), (1, 128)), odq(oq(b, (1, 128)), (1, 128))
    r = {"add": da + db, "sub": da - db, "mul": da * db, "truediv": da / db}[opname].astype(np.float32)
    assert_triple(out, oq(r, (1, 128)), opname)


def test_elementwise_gradient(Q):
    rng = np.random.default_rng(7)
    a = rng.standard_normal((128, 256)).astype(np.float32)
    b = rng.standard_normal((128, 256)).astype(np.float32)
    ad, bd = to_dev_f32(a).requires_grad_(True), to_dev_f32(b).requires_grad_(True)
    (Q.QArrayImpl(ad, (1, 128)) * Q.QArrayImpl(bd, (1, 128))).astype(torch.float32).sum().backward()
    # d/da = db (dequantized), requantized with the grid and dequantized (Q:750-763, Q:521-526);
    # the cotangent reaching the product is dequantize_bwd(1) of the product's scales
    da, db = odq(oq(a, (1, 128)), (1, 128)), odq(oq(b, (1, 128)), (1, 128))
    prodq = oq((da * db).astype(np.float32), (1, 128))
    g1 = O.dequantize_bwd(np.ones((128, 256), np.float32), prodq[1], prodq[2], (1, 128))
    want = odq(oq((g1 * db).astype(np.float32), (1, 128)), (1, 128))
    assert_f32_bits_equal(f32(ad.grad), want, "grad a")


def test_scalar_and_mismatched_grid_ops(Q):
    a = np.random.default_rng(8).standard_normal((128, 256)).astype(np.float32)
    qa = Q.QArrayImpl(to_dev_f32(a), (1, 128))
    da = odq(oq(a, (1, 128)), (1, 128))
    assert_f32_bits_equal(f32(qa * 2.0), (da * np.float32(2.0)).astype(np.float32), "q * 2")
    assert_f32_bits_equal(f32(1.0 - qa), (np.float32(1.0) - da).astype(np.float32), "1 - q")
    qb = Q.QArrayImpl(to_dev_f32(a), (128, 128))
    out = qa + qb           # different grids: f32 sum requantized with self's grid
    db = odq(oq(a, (128, 128)), (128, 128))
    assert_triple(out, oq((da + db).astype(np.float32), (1, 128)), "mismatched grids")


# -------------------------------------------------------- views and layout
def test_neg_abs(Q):
    a = np.random.default_rng(9).standard_normal((128, 256)).astype(np.float32)
    qa = Q.QArrayImpl(to_dev_f32(a), (1, 128))
    da = odq(oq(a, (1, 128)), (1, 128))
    assert_f32_bits_equal(f32((-qa).astype(torch.float32)), -da, "neg")
    assert_f32_bits_equal(f32(abs(qa).astype(torch.float32)), np.abs(da), "abs")


def test_transpose_reshape_sum_getitem_concat_apply(Q):
    a = np.random.default_rng(10).standard_normal((256, 128)).astype(np.float32)
    qa = Q.QArrayImpl(to_dev_f32(a), (1, 128))
    da = odq(oq(a, (1, 128)), (1, 128))
    assert qa.T.tgrid == (128, 1)
    assert_triple(qa.T, oq(da.T.copy(), (128, 1)), ".T")
    assert_triple(qa.mT, oq(da.T.copy(), (128, 1)), ".mT")
    assert_triple(qa.reshape(128, 256), oq(da.reshape(128, 256), (1, 128)), "reshape")
    assert_triple(qa.transpose(1, 0), oq(da.T.copy(), (1, 128)), "transpose")
    s = qa.sum(axis=0)
    assert s.tgrid == (1, 128)
    # the f32 sum's order differs from NumPy's, so compare values, not bytes
    want = odq(oq(da.sum(axis=0, dtype=np.float64).astype(np.float32), (1, 128)), (1, 128))
    assert rel(f32(s.astype(torch.float32)), want) <= TOL
    sl = qa[:64, :64]
    assert sl.tgrid == (1, 64)
    assert_triple(sl, oq(da[:64, :64].copy(), (1, 64)), "getitem")
    cat = Q.QArrayImpl.concat([qa, qa], axis=0)
    assert_triple(cat, oq(np.concatenate([da, da], 0), (1, 128)), "concat")
    ap = qa.apply(lambda t: t * 3.0)
    assert_triple(ap, oq(da * np.float32(3.0), (1, 128)), "apply")
    upd = qa.at[0, 0].set(5.0)
    d2 = da.copy()
    d2[0, 0] = 5.0
    assert_triple(upd, oq(d2, (1, 128)), "at.set")


def test_pytree_round_trip(Q):
    import torch.utils._pytree as pytree
    a = np.random.default_rng(11).standard_normal((128, 128)).astype(np.float32)
    qa = Q.QArrayImpl(to_dev_f32(a), (1, 128))
    leaves, spec = pytree.tree_flatten({"w": qa})
    assert len(leaves) == 3
    back = pytree.tree_unflatten(leaves, spec)["w"]
    assert back.tgrid == (1, 128) and back.get_value() is qa.get_value()
    plain = Q.QArrayImpl(torch.ones(4, device="cuda"), quant=False)
    assert plain._tree_flatten()[1] == (False, None)
    assert plain[1:3].get_value().shape == (2,)


def test_torch_functions_see_dequantized_values(Q):
    a = np.random.default_rng(12).standard_normal((128, 128)).astype(np.float32)
    qa = Q.QArrayImpl(to_dev_f32(a), (1, 128))
    da = odq(oq(a, (1, 128)), (1, 128))
    assert_f32_bits_equal(f32(torch.relu(qa)), np.maximum(da, 0), "relu(q)")


# ------------------------------------------------------------- embedding lookup
def test_embedding_lookup_matches_full_dequantize(Q):
    """table[ids] reads only the indexed rows; the value and the requantized
    result equal the reference's dequantize-then-index path bit for bit,
    including negative and out-of-range ids (jnp clamps)."""
    from pratchya_amd import _kernels as K
    V, D = 1024, 512
    tb = O.normal_input((V, D), 1.0, seed=51)
    table = Q.QArrayImpl(to_dev_bf16(tb), (16, 128))
    ids = torch.tensor([[0, 5, 1023, -1], [17, 17, 1200, -2000]], device="cuda")
    got = table[ids]
    full = K.dequantize(*table._tree_flatten()[0], torch.float32, (16, 128))
    idx = torch.where(ids < 0, ids + V, ids).clamp(0, V - 1)
    want = full[idx]
    assert got.shape == (2, 4, D) and got.tgrid == (4, 128)
    # the gathered values, then the reference's requantization of them
    g8 = K.gather_dequantize(*table._tree_flatten()[0], (16, 128), ids, torch.float32)
    assert torch.equal(g8.view(torch.int32), want.view(torch.int32))
    ref = oq(want.cpu().numpy(), (4, 128))
    assert_triple(got, ref, "table[ids]")
    bf = K.gather_dequantize(*table._tree_flatten()[0], (16, 128), ids, torch.bfloat16)
    assert torch.equal(bf.view(torch.int16), want.to(torch.bfloat16).view(torch.int16))


@pytest.mark.parametrize("V,D,grid", [(384, 4096, (128, 128)), (64, 24, (4, 4))], ids=["wide", "narrow"])
def test_gather_dequantize_paths(V, D, grid):
    """gather_dequantize against the whole-table dequantization indexed, f32
    and bf16 output, for a wide table (the split kernel: whole-line loads and
    non-temporal stores) and a table whose 4-wide blocks send the bf16 output
    down the per-thread-chunk kernel; 1000 ids with repeats, negatives and
    out-of-range values (clamped as jnp does)."""
    from pratchya_amd import _kernels as K
    tb = O.normal_input((V, D), 1.0, seed=53)
    x8, s8, s32 = K.quantize(to_dev_bf16(tb), grid)
    gen = torch.Generator(device="cuda").manual_seed(54)
    ids = torch.randint(-V - 50, V + 50, (1000,), generator=gen, device="cuda")
    full = K.dequantize(x8, s8, s32, torch.float32, grid)
    idx = torch.where(ids < 0, ids + V, ids).clamp(0, V - 1)
    want = full[idx]
    got = K.gather_dequantize(x8, s8, s32, grid, ids, torch.float32)
    assert torch.equal(got.view(torch.int32), want.view(torch.int32))
    gotb = K.gather_dequantize(x8, s8, s32, grid, ids, torch.bfloat16)
    assert torch.equal(gotb.view(torch.int16), want.to(torch.bfloat16).view(torch.int16))


def test_embedding_lookup_gradient(Q):
    """The table's gradient through the fast path equals the dequantize-then-
    index path (distinct ids: no summation-order freedom)."""
    V, D = 512, 256
    tb = O.normal_input((V, D), 1.0, seed=52)
    ids = torch.tensor([3, 100, 511, 0, 64], device="cuda")
    gy = torch.randn((5, D), device="cuda")
    grads = []
    for fast in (True, False):
        w = to_dev_bf16(tb).float().requires_grad_(True)
        table = Q.QArrayImpl(w, (1, 128))
        out = table[ids] if fast else Q.QArrayImpl(table.dequantize(torch.float32)[ids], (1, 128))
        out.astype(torch.float32).backward(gy)
        grads.append(w.grad.detach().clone())
    assert torch.equal(grads[0].view(torch.int32), grads[1].view(torch.int32))
