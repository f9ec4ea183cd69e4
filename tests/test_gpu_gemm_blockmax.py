"""GPU parity of the weight gradient's requantization with its block maxima
taken from the GEMM (pratchya_gemm_bs_blockmax, then
pratchya_quantize_dequantize_premax): matmul_impl's weight cotangent
(pratchya/_qualia/_qarr.py:621-622) requantized with the weight's (128, 128)
grid and dequantized by quantize_impl's backward (Q:637-638, :521-526).

* The GEMM's f32 output bit for bit against pratchya_gemm_bs_nt, and its
  block maxima against max |c| of that output computed by torch (f32 bits),
  for K-contiguous (transposed (128,1) payloads) and K-major operands, at
  config 4's and config 5's weight-gradient shapes.
* The premax requantization against pratchya_quantize_dequantize with the
  same grid, bit for bit, bf16 and f32 outputs, on those GEMM outputs and on
  synthetic inputs with zero blocks, NaN, infinities and values that clamp.
* The FP8 Linear backward with the (128, 128) weight: the weight's gradient
  unchanged bit for bit against the unfused requantization (qarr routes it
  through the pair).
"""
import pytest
import torch

pytestmark = pytest.mark.gpu


def _K():
    from pratchya_amd import _kernels
    return _kernels


def _torch_block_max(c, a=128, b=128):
    H, W = c.shape
    bits = c.contiguous().view(torch.int32) & 0x7FFFFFFF
    return bits.reshape(H // a, a, W // b, b).amax(dim=(1, 3))


def _operands(T, Cin, Cout, kmajor, seed):
    K = _K()
    g_ = torch.Generator(device="cuda").manual_seed(seed)
    x = torch.randn((T, Cin), generator=g_, device="cuda").to(torch.bfloat16)
    dy = (torch.randn((T, Cout), generator=g_, device="cuda") * 1e-3).to(torch.bfloat16)
    if kmajor:
        return K.operand_k128(*K.quantize_128x1(x)), K.operand_k128(*K.quantize_128x1(dy))
    return K.operand_t128(*K.quantize_t128(x)), K.operand_t128(*K.quantize_t128(dy))


@pytest.mark.parametrize("T,Cin,Cout,kmajor", [(16384, 2048, 8192, True), (16384, 2048, 8192, False),
                                               (32768, 4096, 4096, False), (32768, 4096, 16384, False),
                                               (32768, 16384, 4096, False), (4096, 384, 640, True)],
                         ids=lambda v: str(v))
def test_gemm_block_max(T, Cin, Cout, kmajor):
    K = _K()
    a, b = _operands(T, Cin, Cout, kmajor, seed=T + Cin)
    c, bmax = K.gemm_nt_blockmax(a, b)
    want = K.gemm_nt(a, b, torch.float32)
    torch.cuda.synchronize()
    assert torch.equal(c.view(torch.int32), want.view(torch.int32)), "f32 output differs from pratchya_gemm_bs_nt"
    assert torch.equal(bmax, _torch_block_max(want)), "block maxima differ from max |c|"
    for dt in (torch.bfloat16, torch.float32):
        got = K.quantize_dequantize_premax(c, bmax, (128, 128), dt, fix_nan=True)
        ref = K.quantize_dequantize(want, (128, 128), dt, fix_nan=True)
        torch.cuda.synchronize()
        for g, r, what in zip(got, ref, ("values", "e8m0", "G")):
            assert torch.equal(g.view(torch.uint8), r.view(torch.uint8)), f"{what} ({dt})"


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float32])
def test_premax_special_values(dt):
    K = _K()
    g_ = torch.Generator(device="cuda").manual_seed(7)
    x = torch.randn((1024, 2048), generator=g_, device="cuda")
    x[:128, :128] = 0.0                       # a zero block
    x[300, 5] = float("nan")
    x[600, 1500] = float("inf")
    x[700, 100] = -float("inf")
    x[800:900] *= 1e-9                        # clamped scales
    x[900:1024, 1024:1152] *= 3.0e4
    bmax = _torch_block_max(x)
    got = K.quantize_dequantize_premax(x, bmax, (128, 128), dt, fix_nan=True)
    ref = K.quantize_dequantize(x, (128, 128), dt, fix_nan=True)
    torch.cuda.synchronize()
    for g, r, what in zip(got, ref, ("values", "e8m0", "G")):
        gb, rb = g.view(torch.uint8), r.view(torch.uint8)
        if what == "values":
            gv, rv = g.float(), r.float()
            same = (gb.reshape(gv.shape + (-1,)) == rb.reshape(rv.shape + (-1,))).all(-1) | (gv.isnan() & rv.isnan())
            assert bool(same.all()), what
        elif what == "G":
            assert bool(((g == r) | (g.isnan() & r.isnan())).all()), what
        else:
            assert torch.equal(gb, rb), what


@pytest.mark.parametrize("din,dout", [(2048, 8192), (4096, 4096)])
def test_linear_weight_gradient_unchanged(din, dout, monkeypatch):
    """The FP8 Linear backward's weight gradient with the GEMM's block
    maxima (the default) equals the unfused requantization bit for bit."""
    from pratchya_amd import qarr as Q
    g_ = torch.Generator(device="cuda").manual_seed(din)
    x0 = torch.randn((8192, din), generator=g_, device="cuda").to(torch.bfloat16)
    w0 = (torch.randn((din, dout), generator=g_, device="cuda") * 0.02).to(torch.bfloat16)
    gy = (torch.randn((8192, dout), generator=g_, device="cuda") * 1e-3).to(torch.bfloat16)

    def step():
        prev = Q.get_matmul_backward()
        Q.set_matmul_backward("fp8")
        try:
            x = x0.clone().requires_grad_(True)
            w = w0.clone().requires_grad_(True)
            (Q.QArrayImpl(x, (1, 128)) @ Q.QArrayImpl(w, (128, 128))).astype(torch.bfloat16).backward(gy)
            torch.cuda.synchronize()
            return x.grad, w.grad
        finally:
            Q.set_matmul_backward(prev)

    gx1, gw1 = step()
    K = _K()
    # unfused: the block maxima pass refused, so qarr falls back to the f32 GEMM + requantization
    monkeypatch.setattr(K, "gemm_nt_blockmax", lambda a, b: (_ for _ in ()).throw(K.PratchyaUnsupported("off")))
    gx2, gw2 = step()
    assert torch.equal(gw1.view(torch.int16), gw2.view(torch.int16)), "weight gradient differs"
    assert torch.equal(gx1.view(torch.int16), gx2.view(torch.int16)), "activation gradient differs"
