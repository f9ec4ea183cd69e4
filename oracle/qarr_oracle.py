"""CPU oracle for pratchya's FP8 block-quantization path.

TEST INFRASTRUCTURE ONLY.  Nothing in the shipped package imports this module;
only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg use it, and only as the checker (or as the timed CPU baseline), never as
the thing that is measured or shipped.

This is a from-scratch NumPy restatement of the reference's live jnp path in
``pratchya/_qualia/_qarr.py`` (abbreviated ``Q`` below).  The reference needs
JAX (absent from this image), so the restatement is pinned by:

* exhaustive comparison of the two rounding steps against torch's CPU casts
  (all 65,536 bf16 patterns through ``bf16 -> float8_e4m3fn``; random and edge
  f32 patterns through ``f32 -> bf16``), ``tests/test_oracle_conversions.py``;
* hand-derived known answers and closed forms (zero blocks, spikes, powers of
  two, the ``(1,1)`` grid round trip, the 1e-7 clamp, e8m0 = 0 blocks, double
  rounding ties, overflow through the clamp), ``tests/test_oracle_quantize.py``;
* brute force on tiny inputs with pure-Python float arithmetic
  (``fractions.Fraction`` rounding), ``tests/test_oracle_quantize.py``;
* a second, independent restatement in C (``oracle/qarr_oracle.c``) compared
  byte for byte on seeded inputs.

Pinning status per function (the reference ships no tests, fixtures or golden
vectors for this path, so no reference KAT exists):

==========================  ==================================================
``f32_to_bf16``             pinned: torch ``.to(bfloat16)`` on 2^20 random +
                            edge patterns; NaN sign/payload unpinned (XLA).
``bf16_to_e4m3fn``          pinned: exhaustive vs torch ``.to(float8_e4m3fn)``.
``quantize_impl``           pinned: KATs + brute force + C restatement.
``dequantize_impl``         pinned: closed forms (exact values where the scale
                            is a power of two, (1,1) grids, e8m0 0 blocks),
                            the 2^-4 block error bound, bf16 = RNE(f32).
``dequantize_bwd``          pinned: closed form on power-of-two scales.
``matmul_*`` (f32 GEMM)     pinned: float64 matmul of the dequantized operands;
                            tolerance-based, as the reference GEMM is f32.
==========================  ==================================================

Semantics that only an import of the pinned JAX/XLA could settle are listed
as "unpinned" in the module docstrings below: the NaN byte's sign for NaN/inf
inputs, and XLA:CPU denormal flushing (this oracle keeps denormals).
"""
from __future__ import annotations

import math
from typing import Tuple

import numpy as np

F32 = np.float32
U32 = np.uint32

# f32(1e-7): the clamp constant of Q:497 (a weakly-typed Python float that
# jnp.maximum converts to the operand's float32 type).
CLAMP = F32(1e-7)


# --------------------------------------------------------------------------
# Bit-level conversions
# --------------------------------------------------------------------------

def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """f32 -> bf16 bit pattern, round to nearest even (Q:499 ``astype(bfloat16)``).

    NaN maps to a quiet NaN with the input's sign (0x7FC0 / 0xFFC0).  Which NaN
    XLA produces is unpinned; only its NaN-ness and sign reach the e4m3fn byte.
    """
    x = np.ascontiguousarray(x, dtype=F32)
    u = x.view(U32).astype(np.uint64)
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF
    is_nan = (u & 0x7FFFFFFF) > 0x7F800000
    nan_bits = ((u >> 16) & 0x8000) | 0x7FC0
    return np.where(is_nan, nan_bits, rounded).astype(np.uint16)


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    """bf16 bit pattern -> f32 (exact)."""
    return (np.asarray(b, dtype=np.uint16).astype(U32) << 16).view(F32)


def bf16_bits_to_e4m3fn(b: np.ndarray) -> np.ndarray:
    """bf16 -> OCP float8_e4m3fn byte, round to nearest even, non-saturating
    (Q:499 ``astype(float8_e4m3fn)``).

    Magnitudes that round above 448 (i.e. >= 466 in bf16; 464 is the tie and
    rounds to even = 448), infinities and NaNs give NaN = 0x7F | sign.
    Subnormal targets (|v| < 2^-6) are multiples of 2^-9.
    """
    b = np.asarray(b, dtype=np.uint16).astype(np.int64)
    sign = (b >> 8) & 0x80
    mag = b & 0x7FFF
    # normal e4m3 range: rebias exponent 127 -> 7 (subtract 120 << 7) and
    # round the 7-bit bf16 mantissa to 3 bits, ties to even.
    normal = (mag - (120 << 7) + 7 + ((mag >> 4) & 1)) >> 4
    # subnormal range: value / 2^-9 rounded to an integer, ties to even.
    v = bf16_bits_to_f32(np.minimum(mag, 0x3C80).astype(np.uint16)).astype(np.float64)
    sub = np.rint(v * 512.0).astype(np.int64)
    code = np.where(mag >= 0x3C80, normal, sub)
    code = np.minimum(code, 0x7F)
    return (code | sign).astype(np.uint8)


def e4m3fn_to_f32(q: np.ndarray) -> np.ndarray:
    """float8_e4m3fn byte -> f32 (exact; 0x7F/0xFF -> NaN)."""
    q = np.asarray(q, dtype=np.uint8).astype(np.int64)
    sign = np.where(q & 0x80, -1.0, 1.0)
    e = (q >> 3) & 0xF
    m = q & 0x7
    val = np.where(e == 0, m * 2.0 ** -9, (1.0 + m / 8.0) * np.exp2(e - 7.0))
    val = np.where((q & 0x7F) == 0x7F, np.nan, val)
    return (sign * val).astype(F32)


def e8m0_to_f32(e: np.ndarray) -> np.ndarray:
    """e8m0 byte -> f32 by the reference's bit trick ``u32(e) << 23`` (Q:495,
    Q:562): e=0 decodes to +0.0 and e=255 to +inf (not NaN)."""
    return (np.asarray(e, dtype=np.uint8).astype(U32) << 23).view(F32)


# --------------------------------------------------------------------------
# Layout (Q:466-482)
# --------------------------------------------------------------------------

def as_2d_shape(shape: Tuple[int, ...]) -> Tuple[int, int, int]:
    """(slices, H, W) view used by quantize/dequantize: 0-d -> (1,1),
    1-d -> (1,n) (Q:461-464); leading dims are independent slices (Q:470)."""
    if len(shape) == 0:
        return 1, 1, 1
    if len(shape) == 1:
        return 1, 1, int(shape[0])
    return int(np.prod(shape[:-2], dtype=np.int64)), int(shape[-2]), int(shape[-1])


def group_layout(H: int, W: int, tgrid: Tuple[int, int]) -> Tuple[int, int, int]:
    """Blocks per 2-D slice and their grouping (Q:474-480).

    Returns ``(n_blk, K, M)``: ``n_blk = (H/a)(W/b)`` blocks numbered row-major
    over the block grid; ``K = gcd(max(1, a*b//16), n_blk)`` consecutive blocks
    share one f32 group max; ``M = n_blk / K`` groups.
    """
    a, b = tgrid
    if H % a or W % b:
        raise ValueError(f"tgrid {tgrid} does not divide the slice shape {(H, W)}")
    n_blk = (H // a) * (W // b)
    K = math.gcd(max(1, (a * b) // 16), n_blk)
    return n_blk, K, n_blk // K


def _to_blocks(x: np.ndarray, S: int, H: int, W: int, a: int, b: int) -> np.ndarray:
    """[S,H,W] -> [S, n_blk, a*b] with blocks in row-major block order (Q:470-472)."""
    return (x.reshape(S, H // a, a, W // b, b).transpose(0, 1, 3, 2, 4)
            .reshape(S, (H // a) * (W // b), a * b))


def _from_blocks(xb: np.ndarray, S: int, H: int, W: int, a: int, b: int) -> np.ndarray:
    """Inverse of ``_to_blocks`` (Q:503-504)."""
    return (xb.reshape(S, H // a, W // b, a, b).transpose(0, 1, 3, 2, 4)
            .reshape(S, H, W))


# --------------------------------------------------------------------------
# quantize_impl / dequantize_impl
# --------------------------------------------------------------------------

def quantize_impl(x: np.ndarray, tgrid: Tuple[int, int] = (128, 128)):
    """Restatement of ``quantize_impl`` (Q:458-506).

    ``x`` is float32 (a bf16 input must be widened first with
    ``bf16_bits_to_f32``; widening is exact and the reference promotes bf16 to
    f32 for the division at Q:499).  Returns ``(x_fp8 uint8 [x.shape],
    sc_fp8 uint8 [..., M, K], sc_fp32 float32 [..., M, 1, 1])``.

    Per block n of group j (Q:484-499):
      m_n = max|x| over the block;  G_j = max m_n over the group (NaN-propagating)
      r_n = m_n / (G_j == 0 ? 1 : G_j)            (IEEE f32 division)
      e_n = (bits(r_n) >> 23) & 0xFF               (e8m0 byte)
      S_n = max(f32(e_n << 23) * G_j, f32(1e-7))   (unguarded G_j; NaN-propagating)
      payload = e4m3fn(bf16(x / S_n * 128))
    """
    x = np.asarray(x, dtype=F32)
    orig_shape = x.shape
    S, H, W = as_2d_shape(orig_shape)
    a, b = tgrid
    n_blk, K, M = group_layout(H, W, tgrid)
    lead = orig_shape[:-2] if len(orig_shape) >= 2 else ()

    xb = _to_blocks(x.reshape(S, H, W), S, H, W, a, b).reshape(S, M, K, a * b)
    with np.errstate(all="ignore"):
        m = np.max(np.abs(xb), axis=-1)                      # [S,M,K]
        G = np.max(m, axis=-1, keepdims=True)                # [S,M,1]
        safe_G = np.where(G == 0, F32(1.0), G).astype(F32)
        r = (m / safe_G).astype(F32)
        e = ((r.view(U32) >> 23) & 0xFF).astype(np.uint8)
        s = e8m0_to_f32(e)
        S_eff = (s * G).astype(F32)
        S_eff = np.where(np.isnan(S_eff), S_eff, np.maximum(S_eff, CLAMP)).astype(F32)
        q = ((xb / S_eff[..., None]).astype(F32) * F32(128.0)).astype(F32)
    payload = bf16_bits_to_e4m3fn(f32_to_bf16_bits(q))
    payload = _from_blocks(payload.reshape(S, n_blk, a * b), S, H, W, a, b)
    return (payload.reshape(orig_shape),
            e.reshape(*lead, M, K),
            G.astype(F32).reshape(*lead, M, 1, 1))


def block_scale(sc_fp8: np.ndarray, sc_fp32: np.ndarray) -> np.ndarray:
    """Per-block dequant scale ``f32(e << 23) * G`` as an f32 [.., M, K] array
    (Q:562-563; no clamp on the dequant side)."""
    M, K = sc_fp8.shape[-2:]
    with np.errstate(all="ignore"):
        return (e8m0_to_f32(sc_fp8) * sc_fp32.reshape(*sc_fp8.shape[:-2], M, 1)).astype(F32)


def _dequant_like(v: np.ndarray, sc_fp8, sc_fp32, tgrid, shape) -> np.ndarray:
    """``(v * (f32(e<<23) * G)) / 128`` blockwise in f32 (Q:562-564, Q:594-597)."""
    S, H, W = as_2d_shape(shape)
    a, b = tgrid
    n_blk, K, M = group_layout(H, W, tgrid)
    vb = _to_blocks(v.reshape(S, H, W), S, H, W, a, b).reshape(S, M, K, a * b)
    sc = block_scale(np.asarray(sc_fp8), np.asarray(sc_fp32, dtype=F32)).reshape(S, M, K, 1)
    with np.errstate(all="ignore"):
        y = ((vb * sc).astype(F32) / F32(128.0)).astype(F32)
    return _from_blocks(y.reshape(S, n_blk, a * b), S, H, W, a, b).reshape(shape)


def dequantize_impl(x_fp8: np.ndarray, sc_fp8: np.ndarray, sc_fp32: np.ndarray,
                    dtype: str = "float32", tgrid: Tuple[int, int] = (128, 128)) -> np.ndarray:
    """Restatement of ``dequantize_impl`` (Q:541-569).

    ``y = (f32(bf16(x8)) * (f32(e<<23) * G)) / 128`` then ``astype(dtype)``.
    ``dtype`` is "float32" (returns float32) or "bfloat16" (returns uint16 bf16
    bit patterns).
    """
    x_fp8 = np.asarray(x_fp8, dtype=np.uint8)
    y = _dequant_like(e4m3fn_to_f32(x_fp8), sc_fp8, sc_fp32, tgrid, x_fp8.shape)
    return cast_out(y, dtype)


def dequantize_bwd(g: np.ndarray, sc_fp8, sc_fp32, tgrid, g_dtype: str = "float32") -> np.ndarray:
    """Restatement of ``dequantize_impl_bwd`` (Q:575-601): the cotangent of the
    payload is ``(g * (f32(e<<23) * G) / 128).astype(g.dtype)``; ``g`` is given
    as f32 values (bf16 cotangents widened exactly)."""
    g = np.asarray(g, dtype=F32)
    return cast_out(_dequant_like(g, sc_fp8, sc_fp32, tgrid, g.shape), g_dtype)


def cast_out(y: np.ndarray, dtype: str) -> np.ndarray:
    if dtype in ("float32", "f32"):
        return y.astype(F32)
    if dtype in ("bfloat16", "bf16"):
        return f32_to_bf16_bits(y)
    raise ValueError(dtype)


# --------------------------------------------------------------------------
# Matmuls (Q:605-712, Q:766-793).  The reference multiplies dequantized f32
# operands with an f32 dot; the oracle uses float64 (closer to exact) and the
# tests compare with a relative Frobenius tolerance.
# --------------------------------------------------------------------------

def matmul_impl(x_fp8, x_sc8, x_sc32, y_fp8, y_sc8, y_sc32, grid_x, grid_y) -> np.ndarray:
    """``dequant(x) @ dequant(y)`` (Q:605-608)."""
    xf = dequantize_impl(x_fp8, x_sc8, x_sc32, "float32", grid_x).astype(np.float64)
    yf = dequantize_impl(y_fp8, y_sc8, y_sc32, "float32", grid_y).astype(np.float64)
    return xf @ yf


def matmul_impl_bwd_f32(x_fp8, x_sc8, x_sc32, y_fp8, y_sc8, y_sc32, grid_x, grid_y, g_out):
    """f32 part of ``matmul_impl_bwd`` (Q:616-622) for 2-D operands:
    ``g_x = g @ dequant(y)^T``, ``g_y = dequant(x)^T @ g`` (before the
    requantization of Q:637-638)."""
    xf = dequantize_impl(x_fp8, x_sc8, x_sc32, "float32", grid_x).astype(np.float64)
    yf = dequantize_impl(y_fp8, y_sc8, y_sc32, "float32", grid_y).astype(np.float64)
    g = np.asarray(g_out, dtype=np.float64)
    return g @ yf.T, xf.T @ g


def rel_fro(a: np.ndarray, b: np.ndarray) -> float:
    """Relative Frobenius error ||a-b|| / ||b||."""
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    den = np.linalg.norm(b)
    return float(np.linalg.norm(a - b) / (den if den > 0 else 1.0))


# --------------------------------------------------------------------------
# Seeded inputs of the benchmark configurations.
# --------------------------------------------------------------------------

def bf16_round(x: np.ndarray) -> np.ndarray:
    """Round f32/f64 values to bf16 (RNE) and return them as f32 values."""
    return bf16_bits_to_f32(f32_to_bf16_bits(np.asarray(x, dtype=F32)))


def activation_input(rows: int, cols: int, seed: int = 2, outlier_frac: float = 0.01,
                     outlier_scale: float = 50.0) -> np.ndarray:
    """Student-t(df=3) activations with 1% of channels scaled x50, bf16-rounded
    (returned as bf16 bit patterns)."""
    rng = np.random.Generator(np.random.PCG64(seed))
    x = rng.standard_t(3, size=(rows, cols)).astype(F32)
    n_out = max(1, int(round(cols * outlier_frac)))
    ch = rng.choice(cols, n_out, replace=False)
    x[:, ch] *= F32(outlier_scale)
    return f32_to_bf16_bits(x)


def normal_input(shape, std: float, seed: int) -> np.ndarray:
    """N(0, std^2) values rounded to bf16 (returned as bf16 bit patterns)."""
    rng = np.random.Generator(np.random.PCG64(seed))
    return f32_to_bf16_bits((rng.standard_normal(size=shape) * std).astype(F32))
