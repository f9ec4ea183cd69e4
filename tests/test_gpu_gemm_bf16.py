"""GPU parity of the bf16 MFMA GEMM and the 16-bit transpose behind
newton_schulz (pratchya/_nnx_impl/_optimizer.py:11-29: ``A = X @ X.T``,
``B = A @ X`` in the leaf's dtype, f32 accumulation).

* pratchya_gemm_bf16_nt against a float64 product of the same bf16 inputs:
  relative Frobenius error <= 1e-5 for f32 outputs (summation order) and the
  bf16 output within one bf16 rounding of the f64 product (|err| <= 2^-8
  relative per element, plus the f32 error); exact sums bit for bit (small
  integers); edge tiles (M, N not multiples of 256, operands below 256 rows).
* pratchya_transpose_b16: bit for bit against torch's transpose copy.
* newton_schulz on the kernel: against the oracle at (1024, 2048) and
  (2048, 1024) within the bf16 tolerance of the optimizer tests (3e-2), and at
  the [16384, 4096] leaf against the BLAS-library iteration (same tolerance).
"""
import numpy as np
import pytest
import torch

from oracle import optim_oracle as OO
from oracle import qarr_oracle as O
from tests.helpers import f32

pytestmark = pytest.mark.gpu


def _K():
    from pratchya_amd import _kernels
    return _kernels


def _bf16(shape, seed, scale=1.0):
    g = torch.Generator(device="cuda").manual_seed(seed)
    return (torch.randn(shape, generator=g, device="cuda") * scale).to(torch.bfloat16)


SHAPES = [(256, 256, 64), (512, 768, 1024), (300, 1000, 128), (1024, 2048, 4096), (100, 64, 192),
          (2048, 40, 256)]


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_gemm_bf16_against_f64(shape):
    K = _K()
    M, N, Kd = shape
    a, b = _bf16((M, Kd), 1), _bf16((N, Kd), 2)
    c32 = K.gemm_bf16_nt(a, b, torch.float32)
    cbf = K.gemm_bf16_nt(a, b, torch.bfloat16)
    torch.cuda.synchronize()
    ref = f32(a).astype(np.float64) @ f32(b).astype(np.float64).T
    got = f32(c32)
    assert O.rel_fro(got, ref) <= 1e-5
    # the bf16 output is the f32 result rounded once (RNE)
    assert np.array_equal(f32(cbf), O.bf16_round(got.astype(np.float32)))


def test_gemm_bf16_exact_integers():
    """Small integers: every product and partial sum is exact in f32, so the
    result is bit for bit the integer dot product (indexing and tiling)."""
    K = _K()
    M, N, Kd = 512, 384, 2048
    rng = np.random.default_rng(4)
    A = rng.integers(-8, 9, (M, Kd)).astype(np.float32)
    B = rng.integers(-8, 9, (N, Kd)).astype(np.float32)
    a = torch.from_numpy(A).cuda().to(torch.bfloat16)
    b = torch.from_numpy(B).cuda().to(torch.bfloat16)
    c = K.gemm_bf16_nt(a, b, torch.float32)
    torch.cuda.synchronize()
    want = (A.astype(np.int64) @ B.astype(np.int64).T).astype(np.float32)
    assert np.array_equal(f32(c), want)


def test_gemm_bf16_unsupported_k():
    K = _K()
    with pytest.raises(K.PratchyaUnsupported):
        K.gemm_bf16_nt(_bf16((256, 96), 5), _bf16((256, 96), 6))


@pytest.mark.parametrize("shape", [(64, 64), (72, 136), (4096, 1024), (1000, 8), (8, 520)])
def test_transpose_b16(shape):
    K = _K()
    x = _bf16(shape, 7)
    got = K.transpose_b16(x)
    torch.cuda.synchronize()
    assert tuple(got.shape) == shape[::-1]
    assert torch.equal(got.view(torch.int16), x.t().contiguous().view(torch.int16))


@pytest.mark.parametrize("shape", [(1024, 2048), (2048, 1024)])
def test_newton_schulz_kernel_against_oracle(shape):
    from pratchya_amd.optim import newton_schulz
    rng = np.random.default_rng(23)
    G = O.bf16_round((rng.standard_normal(shape) * 1e-3).astype(np.float32))
    got = newton_schulz(torch.from_numpy(G).cuda().to(torch.bfloat16), 5)
    torch.cuda.synchronize()
    want = OO.newton_schulz(G, 5, "bfloat16")
    assert O.rel_fro(f32(got), want) <= 3e-2


def test_newton_schulz_leaf_against_library():
    """The [16384, 4096] leaf (config 5's FFN weights): the kernel iteration
    against the same iteration on the BLAS library (both round every product
    and operation to bf16; they differ in summation order only)."""
    from pratchya_amd import optim
    G = _bf16((16384, 4096), 9, 1e-3)
    got = optim.newton_schulz(G, 5)
    X = G.contiguous()
    X = X / (torch.sqrt(torch.sum(X * X)) + 1e-7)
    K = _K()
    for _ in range(5):
        A = X.T @ X
        B = X @ A
        X = K.ns_combine(X, B, out=X)
    torch.cuda.synchronize()
    err = (got.float() - X.float()).norm() / X.float().norm()
    assert err.item() <= 3e-2
