"""GPU parity of the bf16 MFMA GEMM and the 16-bit transpose behind
newton_schulz (pratchya/_nnx_impl/_optimizer.py:11-29: ``A = X @ X.T``,
``B = A @ X`` in the leaf's dtype, f32 accumulation).

* pratchya_gemm_bf16_nt against a float64 product of the same bf16 inputs:
  relative Frobenius error <= 1e-5 for f32 outputs (summation order) and the
  bf16 output within one bf16 rounding of the f64 product (|err| <= 2^-8
  relative per element, plus the f32 error); exact sums bit for bit (small
  integers); edge tiles (M, N not multiples of 256, operands below 256 rows).
* pratchya_transpose_b16: bit for bit against torch's transpose copy.
* pratchya_ns_normalize_f32: quotients bit for bit against the host's f32
  expression for a denominator within 64 ulps of the host's.
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


@pytest.mark.parametrize("shape", SHAPES + [(16384, 4096, 4096)], ids=lambda s: "x".join(map(str, s)))
def test_gemm_bf16_ns_equals_product_then_combine(shape):
    """pratchya_gemm_bf16_nt_ns: the product's epilogue forms 1.5 X - 0.5 B
    with the same bits as pratchya_ns_combine applied to the bf16 product,
    including edge tiles and short operands; run twice into the same output;
    and with B given K-major."""
    M, N, Kd = shape
    K = _K()
    a, b, x = _bf16((M, Kd), 31, 0.05), _bf16((N, Kd), 32, 0.05), _bf16((M, N), 33)
    want = K.ns_combine(x, K.gemm_bf16_nt(a, b))
    out = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device="cuda")
    for _ in range(2):
        got = K.gemm_bf16_nt_ns(a, b, x, out=out)
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), want.view(torch.int16))
    # B given K-major ([K, N]) and read through the LDS transposing loads: the
    # same K values per MFMA lane, so the same bits
    got_k = K.gemm_bf16_nt_ns(a, b.T.contiguous(), x, b_k_major=True)
    torch.cuda.synchronize()
    assert torch.equal(got_k.view(torch.int16), want.view(torch.int16))


def test_gemm_bf16_ns_rejects_output_over_x():
    K = _K()
    a, b, x = _bf16((256, 128), 1), _bf16((256, 128), 2), _bf16((256, 256), 3)
    with pytest.raises(ValueError, match="overlaps"):
        K.gemm_bf16_nt_ns(a, b, x, out=x)


@pytest.mark.parametrize("shape", [(16384, 4096), (4096, 4096), (999, 7), (8, 8)], ids=lambda s: "x".join(map(str, s)))
def test_ns_normalize_roundings(shape):
    """pratchya_ns_normalize against the bf16 expression's roundings computed
    on the host: each square rounded to bf16, the sum rounded to bf16, the
    square root and the sum with 1e-7 rounded to bf16, each quotient rounded
    to bf16.  The kernel sums in f32 (a fixed order) and the host in f64: both
    candidates for the rounded sum next to the f64 sum are accepted, and the
    quotients must then match bit for bit (with a tail of n % 8 elements for
    [999, 7])."""
    K = _K()
    g = _bf16(shape, 17, 1e-3)
    got = K.ns_normalize(g)
    torch.cuda.synchronize()
    G = f32(g)
    sq = O.bf16_round((G * G).astype(np.float32))
    s = float(sq.astype(np.float64).sum())
    wants = []
    for t in {float(O.bf16_round(np.array([np.float32(s * f)], np.float32))[0]) for f in (1 - 1e-6, 1.0, 1 + 1e-6)}:
        norm = O.bf16_round(np.sqrt(np.array([t], np.float32)))
        den = O.bf16_round((norm + np.float32(1e-7)).astype(np.float32))
        wants.append(O.bf16_round((G / den[0]).astype(np.float32)))
    gb = f32(got)
    assert any(np.array_equal(gb, w) for w in wants)
    # and the same bits on a second call (fixed reduction order)
    again = K.ns_normalize(g)
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16), again.view(torch.int16))


@pytest.mark.parametrize("shape", [(1024, 1024), (999, 7), (3, 5)], ids=lambda s: "x".join(map(str, s)))
def test_ns_normalize_f32(shape):
    """pratchya_ns_normalize_f32 against the f32 expression on the host: the
    denominator is sqrt(sum of f32 squares) + 1e-7 in f32, where the kernel's
    f32 sum (a fixed order) may differ from the host's f64 sum in its last
    bits, so every f32 denominator within 64 ulps of the host's is tried; the
    quotients must then match bit for bit for one of them.  Deterministic."""
    K = _K()
    rng = np.random.default_rng(31)
    G = (rng.standard_normal(shape) * 1e-3).astype(np.float32)
    g = torch.from_numpy(G).cuda()
    got = K.ns_normalize(g)
    torch.cuda.synchronize()
    out = got.cpu().numpy()
    sq = (G * G).astype(np.float32)
    den64 = np.float32(np.sqrt(np.float32(sq.astype(np.float64).sum())) + np.float32(1e-7))
    bits = np.array([den64], np.float32).view(np.int32)[0]
    cands = np.arange(bits - 64, bits + 65, dtype=np.int32).view(np.float32)
    assert any(np.array_equal((G / d).astype(np.float32).view(np.uint32), out.view(np.uint32)) for d in cands)
    again = K.ns_normalize(g)
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int32), again.view(torch.int32))


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


# ---- f32 products over exact bf16 pieces (pratchya_split_pack_bf16) ----

F32_SHAPES = [(256, 256, 256), (300, 1000, 100), (64, 40, 7), (1, 1, 1), (1024, 768, 4096), (513, 3, 65)]


@pytest.mark.parametrize("a_t", [False, True], ids=["a", "aT"])
@pytest.mark.parametrize("b_t", [False, True], ids=["b", "bT"])
@pytest.mark.parametrize("shape", F32_SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_matmul_f32_against_f64(shape, a_t, b_t):
    """op(a) @ op(b) for f32 operands with heavy-tailed magnitudes: the f32
    product's error against float64 stays at the f32 accumulation level
    (relative Frobenius <= 2e-6, far below bf16's 4e-3)."""
    K = _K()
    M, N, Kd = shape
    rng = np.random.default_rng(11)
    A = (rng.standard_normal((M, Kd)) * np.exp2(rng.integers(-8, 8, (M, Kd)))).astype(np.float32)
    B = (rng.standard_normal((Kd, N)) * np.exp2(rng.integers(-8, 8, (Kd, N)))).astype(np.float32)
    a = torch.from_numpy(A.T.copy() if a_t else A).cuda()
    b = torch.from_numpy(B.T.copy() if b_t else B).cuda()
    c = K.matmul_f32(a, b, a_t, b_t)
    torch.cuda.synchronize()
    assert tuple(c.shape) == (M, N) and c.dtype == torch.float32
    ref = A.astype(np.float64) @ B.astype(np.float64)
    assert O.rel_fro(f32(c), ref) <= 2e-6


@pytest.mark.parametrize("dt", ["bf16_a", "bf16_b", "bf16_both"])
def test_matmul_f32_bf16_operands(dt):
    """A bf16 operand is its own single piece (fewer pairs); the result is the
    same f32 product."""
    K = _K()
    rng = np.random.default_rng(12)
    A = O.bf16_round(rng.standard_normal((384, 512)).astype(np.float32))
    B = rng.standard_normal((512, 320)).astype(np.float32)
    if dt != "bf16_a":
        B = O.bf16_round(B)
    a = torch.from_numpy(A).cuda()
    b = torch.from_numpy(B).cuda()
    if dt in ("bf16_a", "bf16_both"):
        a = a.to(torch.bfloat16)
    if dt in ("bf16_b", "bf16_both"):
        b = b.to(torch.bfloat16)
    c = K.matmul_f32(a, b)
    torch.cuda.synchronize()
    assert O.rel_fro(f32(c), A.astype(np.float64) @ B.astype(np.float64)) <= 2e-6


def test_matmul_f32_exact_and_special_values():
    """24-bit integers (every piece product and sum exact) give the exact
    product; inf and NaN propagate as in an f32 dot product."""
    K = _K()
    rng = np.random.default_rng(13)
    A = rng.integers(-512, 512, (256, 32)).astype(np.float32)         # 10 bits: two pieces
    B = rng.integers(-3, 4, (32, 256)).astype(np.float32) * 257.0     # 9-bit values: two pieces
    c = K.matmul_f32(torch.from_numpy(A).cuda(), torch.from_numpy(B).cuda())
    torch.cuda.synchronize()
    want = (A.astype(np.int64) @ B.astype(np.int64)).astype(np.float64)
    assert np.all(np.abs(want) < 2 ** 24)
    assert np.array_equal(f32(c).astype(np.float64), want)
    A2 = np.ones((256, 64), np.float32)
    A2[3, 5] = np.inf
    A2[7, 9] = np.nan
    B2 = np.full((64, 256), 1.5, np.float32)               # exact in bf16: lower pieces are 0
    B2[11, 17] = -np.inf
    c2 = f32(K.matmul_f32(torch.from_numpy(A2).cuda(), torch.from_numpy(B2).cuda()))
    torch.cuda.synchronize()
    with np.errstate(invalid="ignore"):
        want2 = A2.astype(np.float64) @ B2.astype(np.float64)
    assert np.array_equal(np.isnan(c2), np.isnan(want2))   # row 7; (3, 17): inf - inf
    fin = ~np.isnan(want2)
    assert np.array_equal(c2[fin], want2[fin].astype(np.float32))   # +inf in row 3, -inf in column 17
