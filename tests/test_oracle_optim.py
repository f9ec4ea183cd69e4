"""Pins of the optimizer oracle (oracle/optim_oracle.py) against mathematics
and against an independent implementation of the arithmetic (torch's CPU
f32 / bf16 operations), for pratchya/_nnx_impl/_optimizer.py:11-199.

* Newton-Schulz: the closed form through the SVD.  With G = U diag(s) V^T,
  X0 = G / (||s||_2 + 1e-7) and each step X <- 1.5 X - 0.5 X X^T X maps every
  singular value through p(x) = 1.5 x - 0.5 x^3 and keeps U, V, so NS(G) =
  U diag(p^5(s / (||s|| + 1e-7))) V^T.  A wrong coefficient, step count,
  normalization or transpose handling fails it.
* bf16 arithmetic: the oracle's per-operation rounding against torch CPU bf16
  operations with the same (bf16-valued) constants.
* Known answers: zero momentum, jnp.sign on +-0 and NaN, zero weight decay.
"""
import math

import numpy as np
import pytest
import torch

from oracle import optim_oracle as OO
from oracle import qarr_oracle as Q


def _orthonormal(rng, n, k):
    q, _ = np.linalg.qr(rng.standard_normal((n, k)))
    return q[:, :k]


@pytest.mark.parametrize("shape", [(24, 40), (40, 24), (32, 32)])
def test_newton_schulz_closed_form(shape):
    rng = np.random.default_rng(7)
    m, n = shape
    k = min(m, n)
    U, V = _orthonormal(rng, m, k), _orthonormal(rng, n, k)
    s = np.linspace(0.2, 3.0, k)
    G = (U * s) @ V.T
    x = s / (np.sqrt((s ** 2).sum()) + 1e-7)
    for _ in range(5):
        x = 1.5 * x - 0.5 * x ** 3
    want = (U * x) @ V.T
    got = OO.newton_schulz(G.astype(np.float32), 5, "float32")
    assert got.shape == shape
    assert np.abs(got - want).max() < 2e-5


def test_newton_schulz_steps_and_fixed_point():
    """Zero steps only normalizes; an orthogonal matrix divided by its norm
    converges back toward orthogonality (singular values -> 1)."""
    rng = np.random.default_rng(3)
    G = rng.standard_normal((16, 16)).astype(np.float32)
    got0 = OO.newton_schulz(G, 0, "float32")
    assert np.allclose(got0, G / (np.linalg.norm(G) + 1e-7), rtol=1e-6, atol=1e-7)
    Qm = _orthonormal(rng, 16, 16).astype(np.float32)
    sv = np.linalg.svd(OO.newton_schulz(Qm, 30, "float32"), compute_uv=False)
    assert np.allclose(sv, 1.0, atol=1e-4)


def _torch_ns_bf16(G):
    X = torch.from_numpy(G).to(torch.bfloat16)
    if X.shape[0] > X.shape[1]:
        X = X.T
    X = X / (torch.sqrt(torch.sum(X * X)) + 1e-7)
    for _ in range(5):
        A = (X.double() @ X.T.double()).to(torch.bfloat16)
        B = (A.double() @ X.double()).to(torch.bfloat16)
        X = 1.5 * X - 0.5 * B
    return X.float().numpy()


def test_newton_schulz_bf16_rounding_matches_torch():
    rng = np.random.default_rng(11)
    G = Q.bf16_round(rng.standard_normal((24, 48)).astype(np.float32))
    got = OO.newton_schulz(G, 5, "bfloat16")
    want = _torch_ns_bf16(G)
    assert np.array_equal(got, Q.bf16_round(got))          # every element a bf16 value
    assert Q.rel_fro(got, want) < 2e-3
    assert np.mean(got == want) > 0.97


def _edge_values(rng, n):
    v = rng.standard_normal(n).astype(np.float32) * np.exp2(rng.integers(-20, 20, n)).astype(np.float32)
    v[:8] = [0.0, -0.0, 1.0, -1.0, 3.0e38, -3.0e38, 1e-40, np.inf]
    return v


@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
def test_momentum_matches_torch_ops(dtype):
    rng = np.random.default_rng(5)
    m = _edge_values(rng, 4096)
    g = _edge_values(rng, 4096)[::-1].copy()
    tdt = torch.float32 if dtype == "float32" else torch.bfloat16
    if dtype == "bfloat16":
        m, g = Q.bf16_round(m), Q.bf16_round(g)
    c, nm = OO.momentum(m, g, 0.9, 0.99, dtype)
    tm, tg = torch.from_numpy(m).to(tdt), torch.from_numpy(g).to(tdt)
    b1, b1c = float(OO.const(0.9, dtype)), float(OO.const(1.0 - 0.9, dtype))
    b2, b2c = float(OO.const(0.99, dtype)), float(OO.const(1.0 - 0.99, dtype))
    tc = (b1 * tm + b1c * tg).float().numpy()
    tnm = (b2 * tm + b2c * tg).float().numpy()
    np.testing.assert_array_equal(c.view(np.uint32), tc.view(np.uint32))
    np.testing.assert_array_equal(nm.view(np.uint32), tnm.view(np.uint32))


def test_momentum_known_answers():
    """Zero momentum: c = round((1 - beta1) g), m_new = round((1 - beta2) g);
    the bf16 constants are bf16(0.9) = 0.8984375, bf16(0.1) = 0.10009765625."""
    g = np.array([1.0, -2.0, 0.5], np.float32)
    c, nm = OO.momentum(np.zeros(3, np.float32), g, 0.9, 0.99, "bfloat16")
    assert float(OO.const(0.9, "bfloat16")) == 0.8984375
    assert float(OO.const(1.0 - 0.9, "bfloat16")) == 0.10009765625
    np.testing.assert_array_equal(c, Q.bf16_round(np.float32(0.10009765625) * g))
    c32, _ = OO.momentum(np.zeros(3, np.float32), g, 0.9, 0.99, "float32")
    np.testing.assert_array_equal(c32, np.float32(0.1) * g)


def test_sign_known_answers():
    s = OO.jnp_sign(np.array([2.0, -3.0, 0.0, -0.0, np.nan], np.float32))
    assert s[0] == 1 and s[1] == -1 and s[2] == 0 and not np.signbit(s[2])
    assert s[3] == 0 and np.signbit(s[3]) and np.isnan(s[4])


@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
@pytest.mark.parametrize("use_sign", [True, False])
def test_apply_update_matches_torch_ops(dtype, use_sign):
    rng = np.random.default_rng(9)
    u = rng.standard_normal(2048).astype(np.float32)
    p = (rng.standard_normal(2048) * 0.02).astype(np.float32)
    if dtype == "bfloat16":
        u, p = Q.bf16_round(u), Q.bf16_round(p)
    lr, wd, scale = 0.02, 0.1, math.sqrt(2048)
    got = OO.apply_update(u, use_sign, scale, p, lr, wd, dtype)
    tdt = torch.float32 if dtype == "float32" else torch.bfloat16
    tu = torch.from_numpy(u).to(tdt)
    ut = torch.sign(tu) if use_sign else tu * float(OO.const(scale, dtype))
    lr32 = torch.tensor(lr, dtype=torch.float32)
    want = -(lr32 * ut.float() + (lr32 * torch.tensor(wd, dtype=torch.float32)) * torch.from_numpy(p).float())
    np.testing.assert_array_equal(got.view(np.uint32), want.numpy().view(np.uint32))
    # zero weight decay leaves -lr * u'
    got0 = OO.apply_update(u, use_sign, scale, p, lr, 0.0, dtype)
    np.testing.assert_array_equal(got0, (-(np.float32(lr) * ut.float().numpy())).astype(np.float32))


def test_should_use_muon():
    assert OO.should_use_muon("['blocks']['att']['w_r']", 2)
    assert not OO.should_use_muon("['model']['embed_tokens']", 2)
    assert not OO.should_use_muon("['LM_HEAD']", 2)
    assert not OO.should_use_muon("['norm']", 1)
