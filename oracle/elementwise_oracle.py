"""CPU oracle for the fused arithmetic of two quantized arrays.

TEST INFRASTRUCTURE ONLY.  Nothing in the shipped package imports this module;
only ``tests/`` uses it, and only as the checker.

Restates QArrayImpl's binary operators on two quantized arrays
(``pratchya/_qualia/_qarr.py``, "Q"): ``make_elementwise_impl`` (Q:715-720)
computes ``op(dequantize_impl(x, f32), dequantize_impl(y, f32))``, and the
operator returns ``QArrayImpl(out, tgrid)`` (Q:129-130 and the other
operators through Q:261), i.e. ``quantize_impl`` of the f32 result
(``qarr_oracle``).  Arrays quantized with different grids are dequantized each
with its own grid (Q:127-128), which is the same value.

The operators are jnp's float32 ufuncs, restated from JAX's published source
(``jax/_src/numpy/ufuncs.py``; the pinned jax commit ``48f94e65d`` is not
installed here):

==================  ===========================================================
add/sub/mul/divide  IEEE float32, round to nearest even (NumPy float32).
``floor_divide``    ``_float_divmod``: mod = rem(x, y) (C fmod), div =
                    (x - mod) / y; where mod != 0 and sign(y) != sign(mod),
                    div -= 1; result ``lax.round(div)`` (half away from zero).
``remainder``       r = rem(x, y); r + y where r != 0 and (r < 0) != (y < 0).
==================  ===========================================================

Pinning (``tests/test_oracle_elementwise.py``): add/sub/mul/divide are NumPy's
correctly rounded float32 operations; ``remainder`` against torch's CPU
``torch.remainder`` (same definition, independent implementation) on random and
edge values, signed zeros included; ``floor_divide`` against exact rational
floors (``fractions``) and CPython's float ``//`` for finite nonzero
divisors.  Parity unpinned: ``floor_divide``'s results for a zero, infinite or
NaN divisor and its sign of zero (only the restated formula fixes them; CPython
and torch differ there), and ``remainder``'s NaN payloads.
"""
from __future__ import annotations

import numpy as np

from oracle import qarr_oracle as Q

F32 = np.float32

OPS = ("add", "sub", "mul", "div", "floordiv", "mod")
OP_CODES = {name: i for i, name in enumerate(OPS)}


def jnp_floor_divide(x: np.ndarray, y: np.ndarray) -> np.ndarray:
    """jnp.floor_divide on float32 arrays (``_float_divmod``'s quotient)."""
    x = np.asarray(x, dtype=F32)
    y = np.asarray(y, dtype=F32)
    with np.errstate(all="ignore"):
        mod = np.fmod(x, y).astype(F32)
        div = ((x - mod).astype(F32) / y).astype(F32)
        ind = (mod != 0) & (np.sign(y) != np.sign(mod))
        div = np.where(ind, (div - F32(1)).astype(F32), div).astype(F32)
        # lax.round, ROUND_AWAY_FROM_ZERO: trunc(div) plus sign(div) when |frac| >= 1/2
        t = np.trunc(div).astype(F32)
        frac = (div - t).astype(F32)
        return np.where(np.abs(frac) >= F32(0.5), (t + np.sign(div)).astype(F32), t).astype(F32)


def jnp_remainder(x: np.ndarray, y: np.ndarray) -> np.ndarray:
    """jnp.remainder (jnp.mod) on float32 arrays."""
    x = np.asarray(x, dtype=F32)
    y = np.asarray(y, dtype=F32)
    with np.errstate(all="ignore"):
        r = np.fmod(x, y).astype(F32)
        plus = (r != 0) & ((r < 0) != (y < 0))
        return np.where(plus, (r + y).astype(F32), r).astype(F32)


def apply(op: str, x: np.ndarray, y: np.ndarray) -> np.ndarray:
    """The jnp operator ``op`` on float32 arrays of one shape."""
    x = np.asarray(x, dtype=F32)
    y = np.asarray(y, dtype=F32)
    with np.errstate(all="ignore"):
        if op == "add":
            return (x + y).astype(F32)
        if op == "sub":
            return (x - y).astype(F32)
        if op == "mul":
            return (x * y).astype(F32)
        if op == "div":
            return (x / y).astype(F32)
        if op == "floordiv":
            return jnp_floor_divide(x, y)
        if op == "mod":
            return jnp_remainder(x, y)
    raise ValueError(f"unknown operator {op!r}")


def elementwise(op: str, x, grid_x, y, grid_y, tgrid):
    """``QArrayImpl(op(dequant(x), dequant(y)), tgrid)`` for quantized triples
    ``x`` (grid ``grid_x``) and ``y`` (``grid_y``) of one shape; returns the
    result's ``(payload, sc_fp8, sc_fp32)``."""
    xf = Q.dequantize_impl(*x, "float32", tuple(grid_x))
    yf = Q.dequantize_impl(*y, "float32", tuple(grid_y))
    return Q.quantize_impl(apply(op, xf, yf), tuple(tgrid))
