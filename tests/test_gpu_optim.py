"""GPU parity of the quantized Miulion optimizer step
(pratchya/_nnx_impl/_optimizer.py:11-217) against the NumPy oracle.

* pratchya_momentum: c and the new momentum bit-exact (f32 and bf16
  arithmetic; gradients as fp8 triples, bf16 and f32), and the requantized
  momentum's payload and scales bit-exact.
* pratchya_apply_update: bit-exact (Lion and Muon forms, fp8 / bf16 / f32
  parameters).
* newton_schulz on the hand-written kernels (bf16 MFMA products; f32 products
  over exact bf16 pieces): relative Frobenius error <= 1e-4 (f32) and
  <= 3e-2 (bf16) against the oracle (summation order differs), for aligned,
  unaligned, tall and wide slices and at config 5's [16384, 4096] leaf; with
  torch's products disabled, so that no library GEMM takes part.
* A two-step miulion_optimizer update over a tree with a layer-stacked (3-D,
  bf16) leaf, a 2-D (f32) Muon leaf, an embed_tokens (Lion) leaf and a plain
  1-D leaf: momentum triples bit-exact; Lion updates bit-exact; Muon updates
  within the Newton-Schulz tolerance (relative Frobenius <= 1e-4 in f32,
  <= 3e-2 in bf16).
"""
import numpy as np
import pytest
import torch

from oracle import optim_oracle as OO
from oracle import qarr_oracle as O
from tests.helpers import assert_bytes_equal, assert_f32_bits_equal, f32, u8

pytestmark = pytest.mark.gpu

TDT = {"float32": torch.float32, "bfloat16": torch.bfloat16}


def _K():
    from pratchya_amd import _kernels
    return _kernels


def _quantized(rng, shape, tgrid, scale=1.0):
    x = (rng.standard_normal(shape) * scale).astype(np.float32)
    return O.quantize_impl(x, tgrid)


def _dev_triple(t):
    x8, s8, s32 = t
    return (torch.from_numpy(x8).cuda().view(torch.float8_e4m3fn), torch.from_numpy(s8).cuda(),
            torch.from_numpy(s32).cuda())


def _deq(t, tgrid, dtype):
    if dtype == "bfloat16":
        return O.bf16_bits_to_f32(O.dequantize_impl(*t, "bfloat16", tgrid))
    return O.dequantize_impl(*t, "float32", tgrid)


def _host(t: torch.Tensor) -> np.ndarray:
    return t.float().cpu().numpy()


@pytest.mark.parametrize("shape,tgrid", [((256, 384), (128, 128)), ((64, 256), (1, 128)), ((2, 6, 12), (3, 6)),
                                         ((4, 8, 16), (2, 4))])
@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
@pytest.mark.parametrize("gmode", ["fp8", "bf16", "f32"])
def test_momentum_kernel(shape, tgrid, dtype, gmode):
    rng = np.random.default_rng(abs(hash((shape, dtype, gmode))) % 2 ** 32)
    m = _quantized(rng, shape, tgrid)
    if gmode == "fp8":
        g_t = _quantized(rng, shape, tgrid, 1e-3)
        g_dev, g_val = _dev_triple(g_t), _deq(g_t, tgrid, dtype)
    else:
        gv = (rng.standard_normal(shape) * 1e-3).astype(np.float32)
        if gmode == "bf16":
            gv = O.bf16_round(gv)
            g_dev = torch.from_numpy(gv).cuda().to(torch.bfloat16)
        else:
            g_dev = torch.from_numpy(gv).cuda()
        g_val = gv if dtype == "float32" else O.bf16_round(gv)
    consts = [float(OO.const(v, dtype)) for v in (0.9, 1.0 - 0.9, 0.99, 1.0 - 0.99)]
    c, nm = _K().momentum(_dev_triple(m), g_dev, tgrid, TDT[dtype], *consts)
    torch.cuda.synchronize()
    wc, wnm = OO.momentum(_deq(m, tgrid, dtype), g_val, 0.9, 0.99, dtype)
    assert c.dtype == TDT[dtype] and tuple(c.shape) == shape
    assert_f32_bits_equal(_host(c), wc, f"c {shape}{tgrid} {dtype} {gmode}")
    assert_f32_bits_equal(_host(nm), wnm, f"m_new {shape}{tgrid} {dtype} {gmode}")
    # the new momentum's quantization
    q8, q_s8, q_s32 = _K().quantize(nm, tgrid)
    r8, rs8, rs32 = O.quantize_impl(wnm, tgrid)
    assert_bytes_equal(u8(q8), r8, "momentum payload")
    assert_bytes_equal(u8(q_s8), rs8, "momentum e8m0")
    assert_f32_bits_equal(f32(q_s32), rs32, "momentum G")


@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
@pytest.mark.parametrize("use_sign", [True, False])
@pytest.mark.parametrize("pmode", ["fp8", "bf16", "f32"])
def test_apply_update_kernel(dtype, use_sign, pmode):
    rng = np.random.default_rng(3)
    shape, tgrid = (256, 512), (128, 128)
    u = (rng.standard_normal(shape)).astype(np.float32)
    u[0, :4] = [0.0, -0.0, np.nan, 1e-30]
    if dtype == "bfloat16":
        u = O.bf16_round(u)
    if pmode == "fp8":
        p_t = _quantized(rng, shape, tgrid, 0.02)
        p_dev, p_val = _dev_triple(p_t), _deq(p_t, tgrid, dtype)
    else:
        pv = (rng.standard_normal(shape) * 0.02).astype(np.float32)
        if pmode == "bf16":
            pv = O.bf16_round(pv)
            p_dev = torch.from_numpy(pv).cuda().to(torch.bfloat16)
        else:
            p_dev = torch.from_numpy(pv).cuda()
        p_val = pv
    scale = float(OO.const(np.sqrt(512.0), dtype))
    lr, wd = 0.02, 0.1
    lr_wd = float(np.float32(np.float32(lr) * np.float32(wd)))
    out_dt = TDT[dtype]
    got = _K().apply_update(torch.from_numpy(u).cuda().to(TDT[dtype]), use_sign, scale, p_dev, tgrid, TDT[dtype],
                            float(np.float32(lr)), lr_wd, out_dt)
    torch.cuda.synchronize()
    want = OO.apply_update(u, use_sign, np.sqrt(512.0), p_val, lr, wd, dtype)
    if dtype == "bfloat16":
        want = O.bf16_round(want)
    assert_f32_bits_equal(_host(got), want, f"update {dtype} sign={use_sign} p={pmode}")


@pytest.mark.parametrize("n", [64 * 1024, 1001])        # vector and scalar paths
@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
def test_ns_combine_kernel(n, dtype):
    """1.5 X - 0.5 B of a Newton-Schulz step, each operation rounded to the
    dtype, bit for bit; in place as newton_schulz calls it."""
    K = _K()
    rng = np.random.default_rng(31)
    X = (rng.standard_normal(n) * np.exp2(rng.integers(-30, 30, n))).astype(np.float32)
    B = (rng.standard_normal(n) * np.exp2(rng.integers(-30, 30, n))).astype(np.float32)
    X[:6] = [0.0, -0.0, 3e38, 1e-40, np.inf, 1.0]
    B[:6] = [-0.0, 0.0, -3e38, 1e-40, 1.0, 2.0]
    if dtype == "bfloat16":
        X, B = O.bf16_round(X), O.bf16_round(B)
    xd = torch.from_numpy(X).cuda().to(TDT[dtype])
    bd = torch.from_numpy(B).cuda().to(TDT[dtype])
    got = K.ns_combine(xd, bd, out=xd)
    torch.cuda.synchronize()
    assert got.data_ptr() == xd.data_ptr()
    assert_f32_bits_equal(_host(got), OO.ns_combine(X, B, dtype), f"ns_combine {dtype} n={n}")


@pytest.fixture
def no_library_products(monkeypatch):
    """torch's matrix products raise: a product that is not on the
    hand-written kernels fails the test."""
    def refuse(*a, **k):
        raise AssertionError("a torch matrix product was called")
    for name in ("matmul", "mm", "bmm", "einsum", "addmm", "baddbmm", "tensordot", "inner", "dot"):
        monkeypatch.setattr(torch, name, refuse)
    for name in ("__matmul__", "__rmatmul__", "matmul", "mm", "bmm", "addmm"):
        monkeypatch.setattr(torch.Tensor, name, refuse)
    monkeypatch.setattr(torch.nn.functional, "linear", refuse)


NS_SHAPES = [(256, 384), (384, 256), (100, 37), (37, 100), (70, 65), (1, 130), (512, 512), (300, 1024)]


@pytest.mark.parametrize("shape", NS_SHAPES, ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("dtype,tol", [("float32", 1e-4), ("bfloat16", 3e-2)])
def test_newton_schulz(shape, dtype, tol, no_library_products):
    from pratchya_amd.optim import newton_schulz
    rng = np.random.default_rng(21)
    G = (rng.standard_normal(shape) * 1e-3).astype(np.float32)
    if dtype == "bfloat16":
        G = O.bf16_round(G)
    got = newton_schulz(torch.from_numpy(G).cuda().to(TDT[dtype]), 5)
    torch.cuda.synchronize()
    assert got.dtype == TDT[dtype] and tuple(got.shape) == shape and got.is_contiguous()
    want = OO.newton_schulz(G, 5, dtype)
    assert O.rel_fro(_host(got), want) <= tol


@pytest.mark.parametrize("dtype,tol", [("float32", 1e-4), ("bfloat16", 3e-2)])
def test_newton_schulz_config5_leaf_against_oracle(dtype, tol, no_library_products):
    """Config 5's FFN weight shape [16384, 4096] (the tall iteration, K-major
    Gram product for bf16): against the oracle's f64-accumulated iteration
    with the same roundings (about 5.5 TFLOP of host f64 BLAS)."""
    from pratchya_amd.optim import newton_schulz
    rng = np.random.default_rng(24)
    G = (rng.standard_normal((16384, 4096)) * 1e-3).astype(np.float32)
    if dtype == "bfloat16":
        G = O.bf16_round(G)
    got = newton_schulz(torch.from_numpy(G).cuda().to(TDT[dtype]), 5)
    torch.cuda.synchronize()
    want = OO.newton_schulz(G, 5, dtype)
    assert O.rel_fro(_host(got), want) <= tol


def test_newton_schulz_rejects_other_dtypes():
    from pratchya_amd.optim import newton_schulz
    with pytest.raises(TypeError):
        newton_schulz(torch.zeros((64, 64), dtype=torch.float16, device="cuda"))
    with pytest.raises(ValueError):
        newton_schulz(torch.zeros((2, 64, 64), dtype=torch.float32, device="cuda"))


def _np_triple(q):
    x8, s8, s32 = q._tree_flatten()[0]
    return (u8(x8), u8(s8), f32(s32))


def _oracle_leaf(path, g, m, p, tgrid, dtype, lion_lr, muon_lr, wd):
    """Oracle step of a quantized leaf (3-D: per layer in bf16)."""
    if p[0].ndim == 3:
        ups, n8, ns8, ns32 = [], [], [], []
        for l in range(p[0].shape[0]):
            sl = lambda t: tuple(a[l] for a in t)
            upd, (x8, s8, s32), _ = OO.quantized_leaf_step(path, sl(g), sl(m), sl(p), tgrid, 0.9, 0.99, 5,
                                                           lion_lr, muon_lr, wd, "bfloat16")
            ups.append(O.bf16_round(upd))
            n8.append(x8)
            ns8.append(s8)
            ns32.append(s32)
        return np.stack(ups), (np.stack(n8), np.stack(ns8), np.stack(ns32))
    upd, nm, _ = OO.quantized_leaf_step(path, g, m, p, tgrid, 0.9, 0.99, 5, lion_lr, muon_lr, wd, dtype)
    return upd, nm


def test_miulion_two_steps(no_library_products):
    from pratchya_amd.optim import MiulionHyperParams, MiulionScheduler, miulion_optimizer
    from pratchya_amd.qarr import QArrayImpl
    torch.manual_seed(0)
    tg = (128, 128)
    dev = "cuda"
    params = {
        "blocks": {"w3": QArrayImpl(torch.randn(2, 256, 384, device=dev) * 0.02, tg)},
        "w2": QArrayImpl(torch.randn(256, 512, device=dev) * 0.02, tg),
        "embed_tokens": QArrayImpl(torch.randn(512, 256, device=dev), tg),
        "norm": torch.ones(256, device=dev),
    }
    lion_lr, muon_lr, wd = 4e-3, 5e-2, 0.1
    hp = MiulionHyperParams(lion_lr=lion_lr, muon_lr=muon_lr, weight_decay=wd)
    sched = MiulionScheduler(muon_schedule=lambda s: muon_lr, lion_schedule=lambda s: lion_lr, weight_decay=wd)
    tx = miulion_optimizer(hp, sched)
    state = tx.init(params)
    assert int(state.count) == 0
    m0 = state.momentum["w2"]
    assert not u8(m0._tree_flatten()[0][0]).any() and not u8(m0._tree_flatten()[0][1]).any()

    paths = {"w3": "['blocks']['w3']", "w2": "['w2']", "embed_tokens": "['embed_tokens']"}
    leaf = {"w3": lambda t: t["blocks"]["w3"], "w2": lambda t: t["w2"], "embed_tokens": lambda t: t["embed_tokens"]}
    for step in range(2):
        grads = {
            "blocks": {"w3": QArrayImpl(torch.randn(2, 256, 384, device=dev) * 1e-3, tg)},
            "w2": QArrayImpl(torch.randn(256, 512, device=dev) * 1e-3, tg),
            "embed_tokens": QArrayImpl(torch.randn(512, 256, device=dev) * 1e-3, tg),
            "norm": torch.randn(256, device=dev) * 1e-3,
        }
        old_m = state.momentum
        updates, state = tx.update(grads, state, params)
        torch.cuda.synchronize()
        assert int(state.count) == step + 1
        for name in ("w3", "w2", "embed_tokens"):
            dtype = "bfloat16" if name == "w3" else "float32"
            want_u, want_m = _oracle_leaf(paths[name], _np_triple(leaf[name](grads)), _np_triple(leaf[name](old_m)),
                                          _np_triple(leaf[name](params)), tg, dtype, lion_lr, muon_lr, wd)
            got_m = _np_triple(leaf[name](state.momentum))
            for k, what in enumerate(("payload", "e8m0", "G")):
                if what == "G":
                    assert_f32_bits_equal(got_m[k], want_m[k], f"{name} step {step} momentum {what}")
                else:
                    assert_bytes_equal(got_m[k], want_m[k], f"{name} step {step} momentum {what}")
            got_u = leaf[name](updates)
            assert got_u.dtype == (torch.bfloat16 if name == "w3" else torch.float32)
            if name == "embed_tokens":
                assert_f32_bits_equal(_host(got_u), want_u, f"{name} step {step} update")
            else:
                tol = 3e-2 if name == "w3" else 1e-4
                err = O.rel_fro(_host(got_u), want_u)
                assert err <= tol, f"{name} step {step} update error {err}"
        # plain 1-D leaf: f32 Lion
        g = _host(grads["norm"])
        m = _host(old_m["norm"])
        c = (np.float32(0.9) * m + np.float32(0.1) * g).astype(np.float32)
        lr32 = np.float32(lion_lr)
        want = -(lr32 * OO.jnp_sign(c) + np.float32(lr32 * np.float32(wd)) * np.ones(256, np.float32))
        assert_f32_bits_equal(_host(updates["norm"]), want.astype(np.float32), f"norm step {step} update")
        assert_f32_bits_equal(_host(state.momentum["norm"]),
                              (np.float32(0.99) * m + np.float32(1.0 - 0.99) * g).astype(np.float32),
                              f"norm step {step} momentum")


def test_misaligned_operands():
    """Operands at offsets that rule out vector accesses take the scalar path
    with the same results."""
    rng = np.random.default_rng(8)
    shape, tgrid = (128, 256), (128, 128)
    m = _quantized(rng, shape, tgrid)
    gv = (rng.standard_normal(shape) * 1e-3).astype(np.float32)
    big = torch.zeros(shape[0] * shape[1] + 1, device="cuda")
    big[1:] = torch.from_numpy(gv.reshape(-1)).cuda()
    g_dev = big[1:].view(shape)                      # 4-byte aligned only
    c, nm = _K().momentum(_dev_triple(m), g_dev, tgrid, torch.float32, 0.9, 0.1, 0.99, 0.01)
    torch.cuda.synchronize()
    wc, wnm = OO.momentum(_deq(m, tgrid, "float32"), gv, 0.9, 0.99, "float32")
    assert_f32_bits_equal(_host(c), wc, "misaligned c")
    assert_f32_bits_equal(_host(nm), wnm, "misaligned m_new")
    upd = _K().apply_update(g_dev, True, 0.0, _dev_triple(m), tgrid, torch.float32, 0.02, 0.002, torch.float32)
    torch.cuda.synchronize()
    want = OO.apply_update(gv, True, 0.0, _deq(m, tgrid, "float32"), 0.02, 0.1, "float32")
    assert_f32_bits_equal(_host(upd), want, "misaligned update")


def test_argument_errors():
    K = _K()
    m = _dev_triple(O.quantize_impl(np.zeros((128, 128), np.float32), (128, 128)))
    with pytest.raises(ValueError, match="shape"):
        K.momentum(m, torch.zeros((128, 256), device="cuda"), (128, 128), torch.float32, 0.9, 0.1, 0.99, 0.01)
    with pytest.raises(Exception, match="does not fit|tgrid"):
        K.momentum(m, torch.zeros((128, 128), device="cuda"), (96, 128), torch.float32, 0.9, 0.1, 0.99, 0.01)
    with pytest.raises(Exception, match="f32 direction"):
        K.apply_update(torch.zeros((128, 128), device="cuda"), False, 1.0, m, (128, 128), torch.bfloat16, 0.1,
                       0.01, torch.bfloat16)
