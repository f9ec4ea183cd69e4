"""CPU oracle for the quantized Miulion optimizer step.

TEST INFRASTRUCTURE ONLY.  Nothing in the shipped package imports this module;
only ``tests/`` and ``bench.py`` use it, and only as the checker.

A from-scratch NumPy restatement of ``pratchya/_nnx_impl/_optimizer.py``
(abbreviated ``O`` below): ``newton_schulz`` (O:11-29) and the quantized
``update_leaf`` of ``miulion_optimizer`` (O:111-199), built on the quantizer
restatement in ``qarr_oracle``.

Dtype flow restated (the reference is JAX; Python-float constants are weakly
typed and take the array's dtype, the learning rates are f32 arrays computed
from the int32 step count by optax schedules):

* 3-D (layer-stacked) quantized leaves (O:117-142): momentum, gradient and
  parameter dequantized to bf16; ``c`` and the new momentum in bf16 with every
  product and sum rounded to bf16 and the constants ``beta``, ``1 - beta``
  rounded to bf16; Newton-Schulz in bf16 (matmul outputs rounded to bf16);
  ``u * sqrt(max(N, M))`` in bf16; ``-(lr * u + (lr * wd) * p)`` in f32, cast
  to bf16.
* 2-D quantized leaves (O:155-199): all f32, update returned in f32.

Pinning (``tests/test_oracle_optim.py``):

==========================  ==================================================
``newton_schulz``           pinned: closed form through the SVD (each singular
                            value maps through p(s) = 1.5 s - 0.5 s^3 five
                            times after Frobenius normalization; tall inputs
                            transposed); bf16 variant: per-op rounding checked
                            against torch's CPU bf16 operations.
``momentum``                pinned: torch CPU f32 / bf16 elementwise operations
                            (one rounding per operation) on random and edge
                            values; known answers for zero momentum.
``apply_update``            pinned: torch CPU f32 operations; jnp.sign's
                            treatment of +-0 and NaN by known answers.
==========================  ==================================================

Parity unpinned (only an import of the pinned JAX/XLA could settle it):
whether XLA keeps bf16 intermediates in excess precision (this oracle rounds
every bf16 operation, the literal HLO semantics); the summation order of
XLA:CPU's bf16 dots and norm reduction (NS results are compared with a
relative tolerance); and fused multiply-add contraction (none assumed).
"""
from __future__ import annotations

import math

import numpy as np

from oracle import qarr_oracle as Q

F32 = np.float32


def bf(x: np.ndarray) -> np.ndarray:
    """Round to bf16 (RNE), returned as f32 values."""
    return Q.bf16_round(np.asarray(x, dtype=F32))


def _rnd(x: np.ndarray, dtype: str) -> np.ndarray:
    return bf(x) if dtype == "bfloat16" else np.asarray(x, dtype=F32)


def const(x: float, dtype: str) -> F32:
    """A Python float constant meeting an array of ``dtype`` (weak typing)."""
    v = F32(x)
    return F32(bf(np.array([v]))[0]) if dtype == "bfloat16" else v


def newton_schulz(G: np.ndarray, steps: int = 5, dtype: str = "float32") -> np.ndarray:
    """O:11-29 in ``dtype``: X = G / (||G||_F + 1e-7) (transposed when tall),
    then X <- 1.5 X - 0.5 (X X^T) X ``steps`` times.  Products accumulate in
    f64 and round to ``dtype``; every elementwise operation rounds to it."""
    G = np.asarray(G, dtype=F32)
    m, n = G.shape
    transpose = m > n
    if transpose:
        G = G.T
    G = _rnd(G, dtype)
    sq = _rnd(G * G, dtype)
    total = _rnd(np.array([sq.astype(np.float64).sum()]), dtype)[0]    # the sum is a value of dtype
    norm = _rnd(np.array([np.sqrt(np.float64(total))]), dtype)[0]
    den = _rnd(np.array([norm + const(1e-7, dtype)]), dtype)[0]
    X = _rnd(G / den, dtype)
    for _ in range(steps):
        A = _rnd(X.astype(np.float64) @ X.T.astype(np.float64), dtype)
        B = _rnd(A.astype(np.float64) @ X.astype(np.float64), dtype)
        X = ns_combine(X, B, dtype)
    if transpose:
        X = X.T
    return np.ascontiguousarray(X)


def ns_combine(X: np.ndarray, B: np.ndarray, dtype: str) -> np.ndarray:
    """O:26-27's ``1.5 * X - 0.5 * B`` with every operation rounded to ``dtype``."""
    c15, c05 = const(1.5, dtype), const(0.5, dtype)
    with np.errstate(all="ignore"):
        return _rnd(_rnd(c15 * np.asarray(X, F32), dtype) - _rnd(c05 * np.asarray(B, F32), dtype), dtype)


def momentum(m: np.ndarray, g: np.ndarray, beta1: float, beta2: float, dtype: str):
    """``c = beta1*m + (1-beta1)*g`` and ``m_new = beta2*m + (1-beta2)*g``
    (O:134-135, O:175-176) with one rounding per operation in ``dtype``; ``m``
    and ``g`` are values of ``dtype`` (given as f32 arrays)."""
    m = np.asarray(m, dtype=F32)
    g = np.asarray(g, dtype=F32)
    b1, b1c = const(beta1, dtype), const(1.0 - beta1, dtype)
    b2, b2c = const(beta2, dtype), const(1.0 - beta2, dtype)
    with np.errstate(all="ignore"):
        c = _rnd(_rnd(b1 * m, dtype) + _rnd(b1c * g, dtype), dtype)
        nm = _rnd(_rnd(b2 * m, dtype) + _rnd(b2c * g, dtype), dtype)
    return c, nm


def jnp_sign(x: np.ndarray) -> np.ndarray:
    """jnp.sign: +-1 for nonzero values, the value itself for +-0 and NaN."""
    x = np.asarray(x, dtype=F32)
    return np.where(x > 0, F32(1), np.where(x < 0, F32(-1), x)).astype(F32)


def apply_update(u: np.ndarray, use_sign: bool, scale: float, p: np.ndarray, lr: float, wd: float,
                 dtype: str) -> np.ndarray:
    """O:147-153 / O:189-197: ``-(lr * u' + (lr * wd) * p)`` in f32 with
    ``u' = sign(u)`` or ``u * scale`` in ``dtype``; ``p`` in ``dtype``; lr f32."""
    u = np.asarray(u, dtype=F32)
    p = _rnd(np.asarray(p, dtype=F32), dtype)
    lr32 = F32(lr)
    lr_wd = F32(lr32 * F32(wd))
    with np.errstate(all="ignore"):
        ut = jnp_sign(u) if use_sign else _rnd(u * const(scale, dtype), dtype)
        return (-((lr32 * ut).astype(F32) + (lr_wd * p).astype(F32))).astype(F32)


def should_use_muon(path_str: str, ndim: int) -> bool:
    """O:96-109."""
    if ndim != 2:
        return False
    s = path_str.lower()
    return not any(k in s for k in ("embed_tokens", "lm_head"))


def quantized_leaf_step(path_str: str, g, m, p, tgrid, beta1, beta2, ns_steps, lion_lr, muon_lr, wd,
                        dtype: str):
    """One quantized 2-D slice of ``update_leaf`` (O:117-153 per layer with
    dtype "bfloat16", O:155-199 with "float32").  ``g``, ``m``, ``p``:
    (payload, sc8, sc32) triples (``g`` may also be an f32 array of values).
    Returns ``(update f32 values, (nm8, nm_s8, nm_s32), c)``."""
    deq = lambda t: (Q.bf16_bits_to_f32(Q.dequantize_impl(*t, "bfloat16", tgrid)) if dtype == "bfloat16"
                     else Q.dequantize_impl(*t, "float32", tgrid))
    mv = deq(m)
    gv = deq(g) if isinstance(g, tuple) else _rnd(g, dtype)
    pv = deq(p)
    c, nm = momentum(mv, gv, beta1, beta2, dtype)
    new_m = Q.quantize_impl(nm, tgrid)
    if should_use_muon(path_str, c.ndim):
        u = newton_schulz(c, ns_steps, dtype)
        upd = apply_update(u, False, math.sqrt(max(c.shape)), pv, muon_lr, wd, dtype)
    else:
        upd = apply_update(c, True, 0.0, pv, lion_lr, wd, dtype)
    return upd, new_m, c
