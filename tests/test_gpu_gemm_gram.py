"""GPU parity of the symmetric bf16 product behind newton_schulz's Gram
product (pratchya/_nnx_impl/_optimizer.py:20-22: ``A = X @ X.T`` in bf16
with f32 accumulation), pratchya_gemm_bf16_gram.

* Small integers: every product and partial sum is exact in f32 whatever the
  split of K between workgroups, so the result is bit for bit the integer
  Gram matrix rounded once to bf16 (tile numbering, the K ranges of the
  stream-K split, the partial sums and the mirrored lower triangle).
* Normal inputs: within one bf16 rounding of the float64 product (relative
  Frobenius error <= 4e-3, the bf16 output's rounding) and within one bf16
  ulp (plus 2^-20 for values that cancel to near zero) of
  pratchya_gemm_bf16_nt's result on every element (the two differ only in how
  K is split before the f32 sums are added); exactly symmetric;
  identical bits on a repeated call (the partials are added in a fixed order).
* Shapes cover one tile (a single range), tiles split between two or three
  ranges, K of a single step (no split), and newton_schulz's [4096, 16384];
  A given K-major (the tall iterate's own layout) gives the same bits.
"""
import numpy as np
import pytest
import torch

from oracle import qarr_oracle as O
from tests.helpers import f32

pytestmark = pytest.mark.gpu


def _K():
    from pratchya_amd import _kernels
    return _kernels


def _bf16(shape, seed, scale=1.0):
    g = torch.Generator(device="cuda").manual_seed(seed)
    return (torch.randn(shape, generator=g, device="cuda") * scale).to(torch.bfloat16)


# (M, K): one tile; K of one 64-wide step (every range one whole tile);
# three tiles per side with 3 steps each (ranges of 1-2 steps); 10 tiles with
# 32 steps on 20 ranges; the Newton-Schulz shapes (the 16 x 16 tile grid in
# its L2-aware order); 528 tiles of 4 steps on 256 ranges (a range holds the
# end of one tile, whole tiles and the start of another)
SHAPES = [(256, 512), (768, 64), (768, 192), (1024, 2048), (2048, 1024), (4096, 4096), (4096, 16384),
          (8192, 256)]


@pytest.mark.parametrize("k_major", [False, True], ids=["rows", "kmajor"])
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_gram_exact_integers(shape, k_major):
    """Also with A given K-major ([K, M], the tall iterate itself), read
    through the LDS transposing loads."""
    M, Kd = shape
    print(f"gram exact integers M={M} K={Kd} k_major={k_major}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(M + Kd)
    a = torch.randint(-4, 5, (M, Kd), generator=g, device="cuda").to(torch.bfloat16)
    c = _K().gemm_bf16_gram(a.T.contiguous(), k_major=True) if k_major else _K().gemm_bf16_gram(a)
    ad = a.double()
    ref = (ad @ ad.T).to(torch.bfloat16)        # exact integers, rounded once (RNE)
    torch.cuda.synchronize()
    assert torch.equal(c.view(torch.int16), ref.view(torch.int16)), \
        f"{(c != ref).sum().item()} elements differ"


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_gram_normal_against_f64_and_nt(shape):
    M, Kd = shape
    print(f"gram normal M={M} K={Kd}", flush=True)
    K = _K()
    a = _bf16((M, Kd), 7, 1.0 / np.sqrt(Kd))
    c = K.gemm_bf16_gram(a)
    c2 = K.gemm_bf16_gram(a)
    # the K-major read of the same matrix: each MFMA lane holds the same K
    # values as in the K-contiguous read, so the bits are the same
    ck = K.gemm_bf16_gram(a.T.contiguous(), k_major=True)
    nt = K.gemm_bf16_nt(a, a, torch.bfloat16)
    torch.cuda.synchronize()
    assert torch.equal(ck.view(torch.int16), c.view(torch.int16)), "K-major result differs"
    ad = a.double()
    ref = (ad @ ad.T).cpu().numpy()
    torch.cuda.synchronize()
    assert torch.equal(c.view(torch.int16), c2.view(torch.int16)), "repeated calls differ"
    assert torch.equal(c.view(torch.int16), c.T.contiguous().view(torch.int16)), "not exactly symmetric"
    got = f32(c).astype(np.float64)
    assert O.rel_fro(got, ref) <= 4e-3
    # against the NT kernel's upper triangle: one bf16 ulp of the larger
    # magnitude, plus the f32 sums' own rounding where a value cancels to
    # near zero (|sum| of the products of a row pair is about 1 here, so
    # differently split f32 sums differ by a few 2^-24)
    other = f32(nt).astype(np.float64)
    iu = np.triu_indices(M)
    d = np.abs(got[iu] - other[iu])
    tol = np.maximum(np.abs(got[iu]), np.abs(other[iu])) * 2.0 ** -7 + 2.0 ** -20
    assert np.all(d <= tol), f"max excess {np.max(d - tol)}"


def test_gram_rejects_bad_shapes():
    from pratchya_amd._lib import PratchyaUnsupported
    K = _K()
    with pytest.raises(PratchyaUnsupported):
        K.gemm_bf16_gram(torch.zeros((300, 128), dtype=torch.bfloat16, device="cuda"))
    with pytest.raises(PratchyaUnsupported):
        K.gemm_bf16_gram(torch.zeros((256, 96), dtype=torch.bfloat16, device="cuda"))


def test_gram_two_streams_keep_their_workspaces():
    """Calls on two streams at once use separate partial-tile workspaces."""
    K = _K()
    a = _bf16((2048, 4096), 11, 1.0 / 64)
    b = _bf16((2048, 4096), 12, 1.0 / 64)
    ref_a, ref_b = K.gemm_bf16_gram(a), K.gemm_bf16_gram(b)
    torch.cuda.synchronize()
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    with torch.cuda.stream(s1):
        ca = K.gemm_bf16_gram(a)
    with torch.cuda.stream(s2):
        cb = K.gemm_bf16_gram(b)
    torch.cuda.synchronize()
    assert torch.equal(ca.view(torch.int16), ref_a.view(torch.int16))
    assert torch.equal(cb.view(torch.int16), ref_b.view(torch.int16))


def test_gram_status_word_at_config5_leaf():
    """The tall [16384, 4096] iterate's Gram product (newton_schulz on config
    5's FFN weight, K-major): the status word of the bounded partial-tile
    waits is 0 after the call, on a stream the call shares with no other,
    and the result equals the NT kernel's within the bf16 tolerance."""
    K = _K()
    y = _bf16((16384, 4096), 41, 1.0 / 64)
    st = torch.full((1,), -1, dtype=torch.int32, device="cuda")
    c = K.gemm_bf16_gram(y, k_major=True, status=st)
    torch.cuda.synchronize()
    assert int(st.item()) == 0, "a partial tile of the Gram product did not arrive in time"
    assert not torch.isnan(c.float()).any()
    ref = K.gemm_bf16_nt(K.transpose_b16(y), K.transpose_b16(y))
    torch.cuda.synchronize()
    err = (c.float() - ref.float()).norm() / ref.float().norm()
    assert err.item() <= 4e-3


def test_gram_workspace_is_fixed_per_stream():
    """A smaller call after a larger one keeps the same workspace (a graph
    that captured the larger call would keep writing into it)."""
    K = _K()
    K.gemm_bf16_gram(_bf16((4096, 4096), 42))
    key = (torch.cuda.current_device(), torch.cuda.current_stream().cuda_stream)
    ws = K._GRAM_WS[key]
    K.gemm_bf16_gram(_bf16((512, 256), 43))
    K.gemm_bf16_gram(_bf16((8192, 256), 44))
    torch.cuda.synchronize()
    assert K._GRAM_WS[key] is ws
