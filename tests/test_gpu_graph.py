"""The C ABI's entry points captured in a HIP graph (torch.cuda.CUDAGraph):
each replay, with new inputs copied in eagerly between replays, gives the
bytes of the same calls made eagerly.  This covers the contract that the
entry points only enqueue work (no allocation, no host synchronisation, no
memset nodes): the general quantizer clears its block-max workspace with a
kernel on every replay, and the fused elementwise general path and the Gram
product's partial-tile flags likewise; the (1, 1) requantization epilogue,
the elementwise (1, 1) quantizer, and the weight gradient's block maxima with
the requantization that starts from them are captured too."""
import numpy as np
import pytest
import torch

from oracle import qarr_oracle as O

pytestmark = pytest.mark.gpu


def _K():
    from pratchya_amd import _kernels
    return _kernels


def _same(a, b, what):
    """Bitwise equality of two tensors of one dtype and shape."""
    assert a.dtype == b.dtype and a.shape == b.shape, what
    assert torch.equal(a.contiguous().view(torch.uint8), b.contiguous().view(torch.uint8)), what


def test_graph_replays_match_eager():
    K = _K()
    gen = torch.Generator(device="cuda").manual_seed(41)
    M, Kd, N = 512, 1024, 768
    x = torch.empty((M, Kd), dtype=torch.bfloat16, device="cuda")
    w = torch.empty((Kd, N), dtype=torch.bfloat16, device="cuda")
    y = torch.empty((M, Kd), dtype=torch.bfloat16, device="cuda")

    def fill():
        x.copy_(torch.randn((M, Kd), generator=gen, device="cuda").to(torch.bfloat16))
        w.copy_((torch.randn((Kd, N), generator=gen, device="cuda") * 0.02).to(torch.bfloat16))
        y.copy_(torch.randn((M, Kd), generator=gen, device="cuda").to(torch.bfloat16))

    def work():
        xq = K.quantize(x, (1, 128))                                    # one-pass kernel
        wq = K.quantize(w, (128, 128))                                  # general path, workspace
        yq = K.quantize(y, (1, 128))
        a = K.operand_rows(*xq, (1, 128))
        b = K.operand_transposed(*wq, (128, 128))
        c = K.gemm_nt(a, b, torch.bfloat16)                            # block-scaled FP8 GEMM
        s = K.elementwise("add", xq, (1, 128), yq, (1, 128), (1, 128))  # fused, one pass
        d = K.elementwise("mul", xq, (1, 128), yq, (1, 128), (4, 64))   # fused, general path
        t = K.quantize_t128(x)                                          # transposed requantize
        q = K.dequantize(*xq, torch.float32, (1, 128))
        gr = K.gemm_bf16_gram(x)                                        # stream-K, flags cleared by a kernel
        ns = K.gemm_bf16_nt_ns(x, x, gr)                                # Newton-Schulz epilogue
        b11 = K.operand_transposed(*K.quantize(w, (128, 1)), (128, 1))
        o11 = K.gemm_nt_q11(a, b11, torch.bfloat16)                     # (1, 1) requantization epilogue
        x11 = K.quantize(x, (1, 1))                                     # elementwise (1, 1) kernel
        c32, bm = K.gemm_nt_blockmax(a, b)                              # block maxima from the epilogue
        wg = K.quantize_dequantize_premax(c32, bm, (128, 128), torch.bfloat16)
        return [*xq, *wq, c, *s, *d, *t, q, gr, ns, *o11, *x11, c32, bm, *wg]

    fill()
    torch.cuda.synchronize()
    work()                                   # warm up outside the capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        outs = work()
    for rep in range(3):
        fill()                               # eager work between replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        want = work()
        torch.cuda.synchronize()
        assert len(want) == len(outs)
        for i, (got, ref) in enumerate(zip(outs, want)):
            _same(got, ref, f"replay {rep}, output {i}")
    # and the replayed quantize is the oracle's
    xo = O.quantize_impl(x.float().cpu().numpy(), (1, 128))
    assert np.array_equal(outs[0].view(torch.uint8).cpu().numpy(), xo[0])
