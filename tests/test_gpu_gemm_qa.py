"""GPU parity of the quantize prologue, pratchya_gemm_bs_nt_qa: the quantized
Linear's ``QArrayImpl(x, (1, 128)) @ kernel`` (pratchya/_nnx_impl/_module.py:
46-50; quantize_impl Q:458-506, then matmul_impl Q:605-608) in one launch.

* Bit for bit against the two-kernel chain it replaces -- pratchya_quantize
  of x, then pratchya_gemm_bs_nt (or pratchya_gemm_bs_nt_fq with the output
  requantization) on that payload: the activation's payload, e8m0 bytes and
  group maxima, and the GEMM's output (same A bytes, same accumulation
  order), at config 3's, the d=4096 FFN's and config 5's shapes, row counts
  that are not multiples of 256, a 3-D activation, f32 output and rows of
  special values.
* Calls in a row with fresh inputs whose outputs reuse the same device memory
  (the allocator hands the freed blocks back): a unit must never be read
  from a cache line left by an earlier launch.
* The status word stays 0 (every wait between workgroups completed).
* The activation's quantization against the oracle (C restatement) at a small
  size, so the chain itself is not the only reference.
"""
import numpy as np
import pytest
import torch

from oracle import c_oracle as C
from tests.helpers import assert_bytes_equal, assert_f32_bits_equal, assert_payload_equal, f32, u8

pytestmark = pytest.mark.gpu


def _K():
    from pratchya_amd import _kernels
    return _kernels


def _weight(k, n, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    w = (torch.randn((k, n), generator=g, device="cuda") * 0.02).to(torch.bfloat16)
    K = _K()
    return K.operand_transposed(*K.quantize(w, (128, 128)), (128, 128))


def _act(shape, seed, std=1.0):
    g = torch.Generator(device="cuda").manual_seed(seed)
    return (torch.randn(shape, generator=g, device="cuda") * std).to(torch.bfloat16)


def _same_q(got, want, what):
    for g, w, name in zip(got, want, ("payload", "e8m0", "G")):
        assert tuple(g.shape) == tuple(w.shape), f"{what} {name}: shape {tuple(g.shape)} != {tuple(w.shape)}"
        if name == "G":
            assert_f32_bits_equal(f32(g), f32(w), f"{what} {name}")
        elif name == "payload":
            assert_payload_equal(u8(g), u8(w), f"{what} {name}")
        else:
            assert_bytes_equal(u8(g), u8(w), f"{what} {name}")


def _check(x, wop, out_dtype=torch.bfloat16, fq=False, what=""):
    K = _K()
    status = torch.full((1,), -1, dtype=torch.int32, device="cuda")
    y, xq, osc = K.gemm_nt_qa(x, wop, out_dtype, fq=fq, lead=tuple(x.shape[:-1]), status=status)
    wq = K.quantize(x, (1, 128))
    a = K.operand_rows(wq[0].reshape(-1, x.shape[-1]), wq[1], wq[2], (1, 128))
    if fq:
        wy, ws8, ws32 = K.gemm_nt_fq(a, wop, out_dtype, lead=tuple(x.shape[:-1]))
    else:
        wy = K.gemm_nt(a, wop, out_dtype)
    torch.cuda.synchronize()
    assert int(status.item()) == 0, f"{what}: status word {int(status.item())}"
    _same_q(xq, wq, f"{what} activation")
    yb, wyb = y.view(torch.int16 if out_dtype == torch.bfloat16 else torch.int32), \
        wy.view(torch.int16 if out_dtype == torch.bfloat16 else torch.int32)
    bad = (yb != wyb) & ~(torch.isnan(y) & torch.isnan(wy))
    assert not bool(bad.any()), f"{what}: {int(bad.sum())} output values differ from the chain"
    if fq:
        assert_bytes_equal(u8(osc[0]), u8(ws8), f"{what} output e8m0")
        assert_f32_bits_equal(f32(osc[1]), f32(ws32), f"{what} output G")


@pytest.mark.parametrize("M,Kd,N", [(16384, 2048, 8192), (32768, 4096, 16384), (1000, 2048, 1024),
                                    (300, 1024, 512), (4096, 3072, 2048)],
                         ids=lambda v: str(v))
def test_against_chain(M, Kd, N):
    x = _act((M, Kd), seed=M + Kd)
    _check(x, _weight(Kd, N, seed=N), what=f"[{M},{Kd}]x[{Kd},{N}]")


def test_config5_projection_shape():
    x = _act((32768, 4096), seed=11)
    _check(x, _weight(4096, 4096, seed=12), fq=True, what="config 5 [4096,4096] projection")


@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float32])
def test_with_output_requantization(out_dtype):
    x = _act((4096, 4096), seed=21)
    _check(x, _weight(4096, 4096, seed=22), out_dtype=out_dtype, fq=True, what=f"fq {out_dtype}")


def test_ffn_shape_with_output_requantization():
    x = _act((32768, 4096), seed=23)
    _check(x, _weight(4096, 16384, seed=24), fq=True, what="FFN fq")


def test_f32_output_and_3d_activation():
    x = _act((2, 768, 2048), seed=31)
    _check(x, _weight(2048, 2048, seed=32), out_dtype=torch.float32, what="3-D f32")


def test_special_rows():
    """All-zero rows and groups, NaN and infinities (non-finite group maxima),
    rows small enough to clamp at 1e-7, and one outlier per group (blocks far
    below their group max)."""
    g = torch.Generator(device="cuda").manual_seed(41)
    x = torch.randn((1024, 2048), generator=g, device="cuda")
    x[0] = 0.0
    x[5, 1024:] = 0.0
    x[7, 3] = float("nan")
    x[300, 1500] = float("inf")
    x[301, 17] = -float("inf")
    x[400:420] *= 1e-9
    x[500:520, ::1024] = 3.0e4
    _check(x.to(torch.bfloat16), _weight(2048, 2048, seed=42), what="special rows")


def test_calls_reusing_memory():
    """Three calls in a row on fresh activations; the outputs of one call are
    freed before the next, so the allocator gives the next call the same
    blocks."""
    wop = _weight(4096, 4096, seed=51)
    for i in range(3):
        x = _act((16384, 4096), seed=52 + i, std=1.0 + i)
        _check(x, wop, what=f"call {i}")
        del x
        torch.cuda.synchronize()


def test_activation_against_oracle():
    rng = np.random.default_rng(61)
    xf = (rng.standard_t(3, size=(512, 2048)) * rng.choice([1.0, 50.0], size=2048, p=[0.98, 0.02])).astype(np.float32)
    x = torch.from_numpy(xf).to(torch.bfloat16).cuda()
    _, xq, _ = _K().gemm_nt_qa(x, _weight(2048, 1024, seed=62), torch.bfloat16)
    torch.cuda.synchronize()
    want = C.quantize(x.float().cpu().numpy(), (1, 128))
    assert_payload_equal(u8(xq[0]), want[0], "oracle payload")
    assert_bytes_equal(u8(xq[1]), want[1], "oracle e8m0")
    assert_f32_bits_equal(f32(xq[2]), want[2], "oracle G")


def test_rejects_what_it_does_not_fuse():
    K = _K()
    wop = _weight(1024, 1024, seed=71)
    with pytest.raises(K.PratchyaUnsupported):
        K.gemm_nt_qa(_act((128, 1024), seed=72), wop, torch.bfloat16)          # fewer than 256 rows
    with pytest.raises(K.PratchyaUnsupported):
        K.gemm_nt_qa(_act((512, 1024), seed=73).float(), wop, torch.bfloat16)  # not bf16


# --------------------------------------------------------------------------
# The quantized-array API with the prologue on (qarr.set_quantize_prologue)
# --------------------------------------------------------------------------
def _linear(x0, w0, g, prologue, mode):
    """``(QArrayImpl(x, (1, 128)) @ QArrayImpl(w, (128, 128))).astype(bf16)``
    and its backward (pratchya/_nnx_impl/_module.py:46-50): output, x.grad,
    w.grad, and x's quantized fields read after the step."""
    from pratchya_amd import qarr as Q
    prev = (Q.get_quantize_prologue(), Q.get_matmul_backward())
    Q.set_quantize_prologue(prologue)
    Q.set_matmul_backward(mode)
    try:
        x = x0.detach().clone().requires_grad_(True)
        w = w0.detach().clone().requires_grad_(True)
        xq = Q.QArrayImpl(x, (1, 128))
        assert isinstance(xq, Q._PendingQuant) == prologue
        y = (xq @ Q.QArrayImpl(w, (128, 128))).astype(torch.bfloat16)
        y.backward(g)
        fields = (xq._QArrayImpl__value, xq._QArrayImpl__sc_fp8, xq._QArrayImpl__sc_fp32)
        torch.cuda.synchronize()
        return y.detach(), x.grad, w.grad, fields
    finally:
        Q.set_quantize_prologue(prev[0])
        Q.set_matmul_backward(prev[1])


@pytest.mark.parametrize("mode", ["fp8", "f32"])
@pytest.mark.parametrize("shape", [(4096, 4096, 4096), (2, 1024, 2048, 1024)], ids=lambda s: "x".join(map(str, s)))
def test_linear_with_prologue_matches_separate_pass(shape, mode):
    """The Linear through the API with the quantize prologue on: output, both
    gradients and x's quantized fields bit-identical to the default path
    (the activation quantized by its own kernel)."""
    *xs, N = shape
    x0 = _act(tuple(xs), seed=81)
    g_ = torch.Generator(device="cuda").manual_seed(82)
    w0 = (torch.randn((xs[-1], N), generator=g_, device="cuda") * 0.02).to(torch.bfloat16)
    g = (torch.randn(tuple(xs[:-1]) + (N,), generator=g_, device="cuda") * 1e-3).to(torch.bfloat16)
    got = _linear(x0, w0, g, True, mode)
    want = _linear(x0, w0, g, False, mode)
    for a, b, what in zip(got[:3], want[:3], ("output", "x.grad", "w.grad")):
        assert a.dtype == b.dtype and a.shape == b.shape, what
        assert torch.equal(a.view(torch.int16), b.view(torch.int16)), f"{what} differs with the prologue ({mode})"
    _same_q(got[3], want[3], f"x fields ({mode})")


def test_pending_activation_other_uses():
    """A pending activation used other than through the Linear quantizes as
    before: fields, dequantize, arithmetic, a product materialized by its
    payload, and shapes the fused kernel does not take (stay eager)."""
    from pratchya_amd import qarr as Q
    prev = Q.get_quantize_prologue()
    Q.set_quantize_prologue(True)
    try:
        x = _act((512, 2048), seed=91)
        want = _K().quantize(x, (1, 128))
        q = Q.QArrayImpl(x, (1, 128))
        assert isinstance(q, Q._PendingQuant) and q.shape == (512, 2048)
        _same_q((q._QArrayImpl__value, q._QArrayImpl__sc_fp8, q._QArrayImpl__sc_fp32), want, "fields")
        d = Q.QArrayImpl(x, (1, 128)).astype(torch.float32)
        assert torch.equal(d, _K().dequantize(*want, torch.float32, (1, 128)))
        wq = Q.QArrayImpl((torch.randn((2048, 1024), device="cuda") * 0.02).to(torch.bfloat16), (128, 128))
        p = Q.QArrayImpl(x, (1, 128)) @ wq
        assert p.shape == (512, 1024)
        v = p._QArrayImpl__value                          # materialized as the reference builds it
        Q.set_quantize_prologue(False)
        p2 = Q.QArrayImpl(x, (1, 128)) @ wq
        assert torch.equal(v.view(torch.uint8), p2._QArrayImpl__value.view(torch.uint8))
        Q.set_quantize_prologue(True)
        assert not isinstance(Q.QArrayImpl(_act((512, 1536), seed=92), (1, 128)), Q._PendingQuant)
        assert not isinstance(Q.QArrayImpl(_act((128, 2048), seed=93), (1, 128)), Q._PendingQuant)
        assert not isinstance(Q.QArrayImpl(x.float(), (1, 128)), Q._PendingQuant)
        assert not isinstance(Q.QArrayImpl(x, (128, 128)), Q._PendingQuant)
        torch.cuda.synchronize()
    finally:
        Q.set_quantize_prologue(prev)
