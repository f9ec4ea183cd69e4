"""Arrays of 2^31 elements: the kernels' 64-bit index paths (quantize_impl,
pratchya/_qualia/_qarr.py:458-506; dequantize_impl, :541-569;
QArrayImpl(x).astype, :339-342; indexing, :263-284; the binary operators,
:121-261).

No configuration of the reference reaches 2^31 elements and the CPU oracle
cannot run at that size, so these tests use a property that does not depend
on the size: a [524288, 4096] array made of 64 copies of an [8192, 4096]
slice, with grids whose blocks and groups tile each copy exactly (tgrid
(128, 128): groups of 1024 blocks = 4096 rows, two per slice; (1, 128):
groups of 8 blocks inside a row), must quantize to 64 copies of the slice's
own result, and dequantize to 64 copies of the slice's dequantization.  The slice runs on
the 32-bit index paths, which the oracle tests pin; the copy runs on the
64-bit ones (more than 0x7FFFFFFF elements).  Bitwise comparisons (NaN and
inf included).
"""
import pytest
import torch

from pratchya_amd import _kernels as K

pytestmark = pytest.mark.gpu

REPS = 64
ROWS, COLS = 8192, 4096


def _slice():
    g = torch.Generator(device="cuda").manual_seed(31)
    x = torch.randn((ROWS, COLS), generator=g, device="cuda")
    # per 128-row band magnitudes from 2^-20 to 2^20 (different e8m0 bytes and
    # group maxima), an all-zero block; a NaN and an inf in the second 4096
    # rows only (a (128, 128) group of their own)
    band = torch.arange(ROWS, device="cuda") // 128
    x = x * torch.exp2((band % 41).float() - 20.0)[:, None]
    x[:128, :128] = 0.0
    x[4096 + 1024 + 5, 300] = float("nan")
    x[4096 + 2048 + 7, 4000] = float("inf")
    return x.to(torch.bfloat16)


def _bits(t: torch.Tensor) -> torch.Tensor:
    return t.view(torch.uint8) if t.element_size() == 1 else t.view(torch.int16 if t.element_size() == 2 else torch.int32)


def _assert_copies(big: torch.Tensor, small: torch.Tensor, what: str, reps: int = REPS) -> None:
    b = _bits(big.contiguous()).reshape(reps, -1)
    s = _bits(small.contiguous()).reshape(1, -1)
    assert b.shape[1] == s.shape[1], what
    step = min(16, reps)
    for r in range(0, reps, step):
        assert torch.equal(b[r:r + step], s.expand(step, -1)), f"{what}: copies {r}..{r + step - 1} differ"


@pytest.fixture(scope="module")
def arrays():
    xs = _slice()
    xb = xs.repeat(REPS, 1)
    assert xb.numel() > 0x7FFFFFFF
    yield xs, xb
    del xb
    torch.cuda.empty_cache()


@pytest.mark.parametrize("tgrid", [(128, 128), (1, 128)])
def test_quantize_dequantize_past_2_31(arrays, tgrid):
    xs, xb = arrays
    qs = K.quantize(xs, tgrid)
    # the slice's result is not degenerate: block scales 2^(e - 127) G over
    # many exponents, finite and NaN groups
    assert bool(qs[0].view(torch.uint8).any())
    e = qs[1].view(torch.uint8).float()
    scale = torch.exp2(e - 127.0) * qs[2].reshape(e.shape[0], 1)
    live = torch.isfinite(scale) & (scale > 0)
    assert torch.unique(torch.floor(torch.log2(scale[live]))).numel() > 20
    assert bool(torch.isnan(qs[2]).any()) and bool(torch.isfinite(qs[2]).any())
    qb = K.quantize(xb, tgrid)
    for name, big, small in zip(("payload", "e8m0", "group max"), qb, qs):
        _assert_copies(big, small, f"quantize {tgrid} {name}")
    ds = K.dequantize(*qs, torch.bfloat16, tgrid)
    db = K.dequantize(*qb, torch.bfloat16, tgrid)
    del qb
    _assert_copies(db, ds, f"dequantize {tgrid}")
    del db
    torch.cuda.empty_cache()


def test_fake_quantize_past_2_31(arrays):
    """One-pass QArrayImpl(x, (128, 128)).astype(bf16) on the general cast's
    64-bit path."""
    xs, xb = arrays
    ys = K.quantize_dequantize(xs, (128, 128), torch.bfloat16)
    yb = K.quantize_dequantize(xb, (128, 128), torch.bfloat16)
    for name, big, small in zip(("values", "e8m0", "group max"), yb, ys):
        _assert_copies(big, small, f"quantize_dequantize {name}")
    del yb
    torch.cuda.empty_cache()


def _repeat_q(q):
    """A quantized triple of one slice, as the triple of REPS stacked copies
    (blocks and groups tile each copy, so the scale arrays stack too)."""
    return (q[0].view(torch.uint8).repeat(REPS, 1), q[1].view(torch.uint8).repeat(REPS, 1), q[2].repeat(REPS, 1, 1))


@pytest.mark.parametrize("op,tgrid", [("add", (1, 128)), ("mul", (128, 128))])
def test_elementwise_past_2_31(arrays, op, tgrid):
    """The fused binary operators on operands of 2^31 elements: the one-pass
    kernel (result grid (1, 128)) and the general path (block maxima, group
    scales, cast; result grid (128, 128)) on 64-bit indices."""
    xs, _ = arrays
    ys = (xs.float() * -0.75 + 0.5).to(torch.bfloat16)
    gx = (1, 128)
    qx, qy = K.quantize(xs, gx), K.quantize(ys, gx)
    rs = K.elementwise(op, qx, gx, qy, gx, tgrid)
    bx, by = _repeat_q(qx), _repeat_q(qy)
    assert bx[0].numel() > 0x7FFFFFFF
    rb = K.elementwise(op, bx, gx, by, gx, tgrid)
    del bx, by
    for name, big, small in zip(("payload", "e8m0", "group max"), rb, rs):
        _assert_copies(big, small, f"{op} {tgrid} {name}")
    del rb
    torch.cuda.empty_cache()


@pytest.mark.parametrize("tgrid,dtype", [((128, 128), torch.bfloat16), ((128, 128), torch.float32),
                                         ((1, 4), torch.bfloat16)])
def test_gather_dequantize_past_2_31(tgrid, dtype):
    """Embedding lookups whose output passes 2^31 elements: 524288 indices
    into a [65536, 4096] table, every row eight times (odd passes as negative
    indices), equal eight copies of the dequantized table (the split kernel for
    (128, 128), the per-chunk kernel for (1, 4))."""
    g = torch.Generator(device="cuda").manual_seed(7)
    table = (torch.randn((65536, 4096), generator=g, device="cuda") * 0.02).to(torch.bfloat16)
    q = K.quantize(table, tgrid)
    ref = K.dequantize(*q, dtype, tgrid)
    rows = torch.arange(65536, device="cuda")
    idx = torch.cat([rows - 65536 if k % 2 else rows for k in range(8)])
    out = K.gather_dequantize(*q, tgrid, idx, dtype)
    assert out.numel() > 0x7FFFFFFF
    _assert_copies(out, ref, f"gather {tgrid} {dtype}", reps=8)
    del out
    torch.cuda.empty_cache()
