"""GPU parity of the fused quantized arithmetic (pratchya_elementwise, through
the C ABI wrapper and through QArrayImpl's operators) against the oracle's
composition QArrayImpl(op(dequantize_impl(x), dequantize_impl(y)), tgrid)
(pratchya/_qualia/_qarr.py:121-261, 715-720): payload, e8m0 and group maxima
bit-exact."""
import numpy as np
import pytest
import torch

from oracle import elementwise_oracle as E
from oracle import qarr_oracle as O
from tests.helpers import assert_bytes_equal, assert_f32_bits_equal, assert_payload_equal, f32, to_dev_f32, u8

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def K():
    from pratchya_amd import _kernels
    return _kernels


def _values(rng, shape, spread=6, edge=False):
    x = (rng.standard_normal(shape) * np.exp2(rng.integers(-spread, spread, shape))).astype(np.float32)
    if edge:
        flat = x.reshape(-1)
        flat[:16] = [0.0, -0.0, 1.0, -1.0, 448.0, -448.0, 1e-30, -1e-30, 3.0, -3.0, 0.5, -0.5, 2.0, -2.0,
                     1e20, -1e20]
        flat[rng.integers(0, flat.size, 64)] = 0.0           # zero divisors for / // %
    return x


def _dev(trip):
    v, s8, s32 = trip
    return (torch.from_numpy(np.ascontiguousarray(v)).cuda().view(torch.float8_e4m3fn),
            torch.from_numpy(np.ascontiguousarray(s8)).cuda().view(torch.float8_e8m0fnu),
            torch.from_numpy(np.ascontiguousarray(s32)).cuda())


def _check(got, want, what):
    assert_payload_equal(u8(got[0]), want[0], f"{what} payload")
    assert_bytes_equal(u8(got[1]), want[1], f"{what} e8m0")
    assert_f32_bits_equal(f32(got[2]), want[2], f"{what} G")


CASES = [
    # shape, grid_x, grid_y, result grid        (path)
    ((256, 2048), (1, 128), (1, 128), (1, 128)),     # one pass, K = 8 (activation layout)
    ((3, 128, 512), (1, 128), (1, 128), (1, 128)),   # one pass, slices
    ((64, 256), (1, 16), (1, 16), (1, 16)),          # one pass, K = 1
    ((64, 192), (1, 32), (1, 64), (1, 64)),          # one pass, K = 4, mixed operand grids
    ((256, 512), (128, 128), (128, 128), (128, 128)),  # general, K = 1024 > n_blk -> gcd
    ((2, 256, 256), (128, 1), (128, 1), (128, 1)),   # general, column blocks
    ((64, 96), (4, 8), (4, 8), (4, 8)),              # general, CH = 8
    ((30, 50), (3, 5), (3, 5), (3, 5)),              # general, CH = 1
    ((128, 256), (1, 128), (128, 128), (1, 128)),    # one pass, operand grids differ
    ((128, 256), (128, 128), (1, 128), (16, 16)),    # general, three grids
]


@pytest.mark.parametrize("op", E.OPS)
@pytest.mark.parametrize("case", range(len(CASES)), ids=[f"{c[0]}-{c[3]}" for c in CASES])
def test_elementwise_matches_oracle(K, op, case):
    shape, gx, gy, go = CASES[case]
    rng = np.random.default_rng(100 + case)
    a = _values(rng, shape, edge=True)
    b = _values(rng, shape, edge=True)      # with zeros: x / 0, fmod(x, 0)
    xa, xb = O.quantize_impl(a, gx), O.quantize_impl(b, gy)
    want = E.elementwise(op, xa, gx, xb, gy, go)
    got = K.elementwise(op, _dev(xa), gx, _dev(xb), gy, go)
    _check(got, want, f"{op} {shape} {gx}/{gy}->{go}")


@pytest.mark.parametrize("op", ["add", "mul", "div"])
def test_elementwise_special_values(K, op):
    """inf and NaN results (1/0, 0/0, overflow) reach the quantizer as the
    reference's would; the clamp fires on tiny blocks."""
    a = np.zeros((16, 128), np.float32)
    b = np.ones((16, 128), np.float32)
    a[0, :5] = [1.0, -1.0, 0.0, 448.0, 3e38]
    b[0, :5] = [0.0, 0.0, 0.0, 1e-3, 3e38]
    a[1] = 1e-30
    b[1] = 1e-30
    a[2, :64] = 3e-36            # block scales below 2^-110: the unfolded dequantization
    b[2, 64:] = -2e-37
    a[3] = 1e36                  # block scales at or above 2^119
    xa, xb = O.quantize_impl(a, (1, 128)), O.quantize_impl(b, (1, 128))
    for go in ((1, 128), (4, 32)):
        want = E.elementwise(op, xa, (1, 128), xb, (1, 128), go)
        got = K.elementwise(op, _dev(xa), (1, 128), _dev(xb), (1, 128), go)
        _check(got, want, f"{op} special {go}")


def test_elementwise_unaligned_payloads_take_the_general_path(K):
    rng = np.random.default_rng(7)
    a, b = _values(rng, (64, 256)), _values(rng, (64, 256))
    xa, xb = O.quantize_impl(a, (1, 128)), O.quantize_impl(b, (1, 128))
    want = E.elementwise("sub", xa, (1, 128), xb, (1, 128), (1, 128))
    da, db = _dev(xa), _dev(xb)
    # payloads at an odd byte offset inside larger buffers
    pa = torch.empty(a.size + 1, dtype=torch.uint8, device="cuda")[1:].view(64, 256)
    pa.copy_(da[0].view(torch.uint8))
    got = K.elementwise("sub", (pa.view(torch.float8_e4m3fn), da[1], da[2]), (1, 128), db, (1, 128), (1, 128))
    _check(got, want, "unaligned")


def test_elementwise_argument_errors(K):
    """Invalid grids are the reference's trace-time errors (PRATCHYA_EINVAL,
    raised as ValueError); pow is not a fused operator."""
    rng = np.random.default_rng(8)
    xa = _dev(O.quantize_impl(_values(rng, (64, 256)), (1, 128)))
    with pytest.raises(ValueError, match="operator"):
        K.elementwise("pow", xa, (1, 128), xa, (1, 128), (1, 128))
    with pytest.raises(ValueError, match="does not divide"):
        K.elementwise("add", xa, (1, 128), xa, (1, 128), (3, 128))     # 3 does not divide 64
    with pytest.raises(ValueError, match="y grid"):
        K.elementwise("add", xa, (1, 128), xa, (1, 96), (1, 128))      # 96 does not divide 256


# ---------------------------------------------------------- QArrayImpl operators
@pytest.fixture
def Q():
    from pratchya_amd import qarr
    return qarr


def _triple(q):
    v, s8, s32 = q._tree_flatten()[0]
    return v, s8, s32


@pytest.mark.parametrize("opname", ["add", "sub", "mul", "truediv", "floordiv", "mod", "rsub", "rtruediv"])
def test_operators_use_the_fused_kernel(Q, K, monkeypatch, opname):
    rng = np.random.default_rng(9)
    a = _values(rng, (128, 256))
    b = _values(rng, (128, 256)) + np.float32(0.25)
    qa, qb = Q.QArrayImpl(to_dev_f32(a), (1, 128)), Q.QArrayImpl(to_dev_f32(b), (1, 128))
    calls = []
    real = K.elementwise
    monkeypatch.setattr(K, "elementwise", lambda *args, **kw: calls.append(args[0]) or real(*args, **kw))
    out = {"add": lambda: qa + qb, "sub": lambda: qa - qb, "mul": lambda: qa * qb, "truediv": lambda: qa / qb,
           "floordiv": lambda: qa // qb, "mod": lambda: qa % qb, "rsub": lambda: qb.__rsub__(qa),
           "rtruediv": lambda: qb.__rtruediv__(qa)}[opname]()
    assert len(calls) == 1
    op = {"add": "add", "sub": "sub", "mul": "mul", "truediv": "div", "floordiv": "floordiv", "mod": "mod",
          "rsub": "sub", "rtruediv": "div"}[opname]
    xa, xb = O.quantize_impl(a, (1, 128)), O.quantize_impl(b, (1, 128))
    _check(_triple(out), E.elementwise(op, xa, (1, 128), xb, (1, 128), (1, 128)), opname)


def test_fused_gradient_matches_unfused(Q, K, monkeypatch):
    """The fused result's autograd node gives the cotangents of the step by
    step composition (make_elementwise_impl's vjp, Q:722-750)."""
    rng = np.random.default_rng(10)
    a, b = _values(rng, (128, 256), spread=2), _values(rng, (128, 256), spread=2)

    def run():
        ad, bd = to_dev_f32(a).requires_grad_(True), to_dev_f32(b).requires_grad_(True)
        qa, qb = Q.QArrayImpl(ad, (1, 128)), Q.QArrayImpl(bd, (1, 128))
        (qa * qb - qa).astype(torch.float32).sum().backward()
        return f32(ad.grad), f32(bd.grad)

    fused = run()
    monkeypatch.setattr(Q, "_FUSED", {})
    unfused = run()
    assert_f32_bits_equal(fused[0], unfused[0], "grad a")
    assert_f32_bits_equal(fused[1], unfused[1], "grad b")


def test_floor_divide_follows_jnp_in_the_unfused_path(Q):
    """Broadcast operands take the torch composition; its floor division is
    jnp's (a zero divisor gives NaN, not inf)."""
    a = np.array([[7.0, -7.0, 1.0, 0.5]], np.float32).repeat(16, 0).repeat(32, 1)
    b = np.array([[2.0, 2.0, 0.0, -2.0]], np.float32).repeat(32, 1)
    got = Q._floor_divide(to_dev_f32(a), to_dev_f32(b))
    assert_f32_bits_equal(f32(got), E.jnp_floor_divide(a, np.broadcast_to(b, a.shape)), "floor_divide")


# ------------------------------------------------------------ embedding lookup
@pytest.mark.parametrize("ids_shape,out_grid", [((2, 256), (128, 128)), ((384,), (128, 128)), ((3, 40), (8, 128)),
                                                ((2, 256), (1, 128))])
def test_gather_quantize_matches_oracle(K, ids_shape, out_grid):
    """quantize_impl(dequantize_impl(table)[ids], grid) in one pass, ids with
    negative and out-of-range entries (clamped as jnp's gather)."""
    rng = np.random.default_rng(60)
    table = (rng.standard_normal((512, 256)) * np.exp2(rng.integers(-3, 3, (512, 1)))).astype(np.float32)
    tq = O.quantize_impl(table, (128, 128))
    ids = rng.integers(-600, 700, ids_shape).astype(np.int64)
    got = K.gather_quantize(*_dev(tq), (128, 128), torch.from_numpy(ids).cuda(), out_grid)
    rows = np.clip(np.where(ids < 0, ids + 512, ids), 0, 511)
    deq = O.dequantize_impl(*tq, "float32", (128, 128))[rows]
    _check(got, O.quantize_impl(deq, out_grid), f"gather {ids_shape} -> {out_grid}")


def test_getitem_fuses_the_requantization(Q, K, monkeypatch):
    """QArrayImpl.__getitem__ with an index array (no gradient) gives the bytes
    of the gather-then-quantize composition through the fused kernel."""
    rng = np.random.default_rng(61)
    table = torch.from_numpy(rng.standard_normal((512, 256)).astype(np.float32)).cuda()
    qt = Q.QArrayImpl(table, (128, 128))
    ids = torch.from_numpy(rng.integers(0, 512, (2, 128))).cuda()
    calls = []
    real = K.gather_quantize
    monkeypatch.setattr(K, "gather_quantize", lambda *a, **k: calls.append(1) or real(*a, **k))
    got = qt[ids]
    assert len(calls) == 1 and got.tgrid == (128, 128)
    v, s8, s32 = qt._tree_flatten()[0]
    want = K.quantize(K.gather_dequantize(v, s8, s32, (128, 128), ids, torch.float32), (128, 128))
    _check(_triple(got), (u8(want[0]), u8(want[1]), f32(want[2])), "getitem")
