"""Exact-rational restatement of the quantizer for tiny finite inputs.

Independent of NumPy's float32 arithmetic: every reference operation
(pratchya/_qualia/_qarr.py:484-499) is evaluated exactly with
``fractions.Fraction`` and then rounded by an explicit round-to-nearest-even
into the target format (binary32, bfloat16, OCP e4m3fn).  Used by the CPU
tests to pin the NumPy oracle on small inputs.
"""
from __future__ import annotations

import math
from fractions import Fraction
from typing import List, Optional, Tuple


def round_rne(v: Fraction, p: int, emin: int, emax: Optional[int]) -> Fraction:
    """Round ``v`` to a binary format with ``p`` significand bits (hidden bit
    included), minimum normal exponent ``emin`` (subnormals below it) and
    overflow above ``emax`` (returns ``inf`` as a float), ties to even."""
    if v == 0:
        return Fraction(0)
    sign = -1 if v < 0 else 1
    a = abs(v)
    e = math.floor(math.log2(a.numerator) - math.log2(a.denominator))
    # fix floating error of log2
    while Fraction(2) ** e > a:
        e -= 1
    while Fraction(2) ** (e + 1) <= a:
        e += 1
    e = max(e, emin)
    quantum = Fraction(2) ** (e - p + 1)
    n = a / quantum
    fl = n.numerator // n.denominator
    rem = n - fl
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and fl % 2 == 1):
        fl += 1
    r = fl * quantum
    if emax is not None and r >= Fraction(2) ** (emax + 1):
        return float("inf") * sign  # type: ignore[return-value]
    return sign * r


def rn32(v: Fraction) -> Fraction:
    return round_rne(v, 24, -126, 127)


def rnbf16(v: Fraction) -> Fraction:
    return round_rne(v, 8, -126, 127)


def e4m3_byte(v: Fraction, negative_zero: bool) -> int:
    """RNE to OCP e4m3fn and encode; > 448 after rounding -> NaN (0x7F|sign)."""
    sign = 0x80 if (v < 0 or (v == 0 and negative_zero)) else 0
    r = round_rne(abs(v), 4, -6, None)
    if r > 448:
        return 0x7F | sign
    if r == 0:
        return sign
    if r < Fraction(1, 64):  # subnormal: m * 2^-9
        return sign | int(r * 512)
    e = 0
    while Fraction(2) ** (e + 1) <= r:
        e += 1
    while Fraction(2) ** e > r:
        e -= 1
    m = int((r / Fraction(2) ** e - 1) * 8)
    return sign | ((e + 7) << 3) | m


def f32_bits_exponent(r: Fraction) -> int:
    """Biased exponent field of the binary32 number r (0 for zero/subnormal)."""
    if r == 0 or r < Fraction(2) ** -126:
        return 0
    e = 0
    while Fraction(2) ** (e + 1) <= r:
        e += 1
    while Fraction(2) ** e > r:
        e -= 1
    return e + 127


CLAMP = Fraction(1e-7).limit_denominator(1 << 200)


def quantize_exact(x: List[List[float]], tgrid: Tuple[int, int]):
    """Quantize a small 2-D list of finite float32 values.  Returns
    (payload bytes [H][W], e8m0 bytes [n_blk], group maxima [M] as floats)."""
    import numpy as np
    clamp = Fraction(float(np.float32(1e-7)))
    H, W = len(x), len(x[0])
    a, b = tgrid
    n_blk = (H // a) * (W // b)
    K = math.gcd(max(1, a * b // 16), n_blk)
    M = n_blk // K
    blocks = []
    for bi in range(H // a):
        for bj in range(W // b):
            blocks.append([(i, j) for i in range(bi * a, bi * a + a) for j in range(bj * b, bj * b + b)])
    m = [max(abs(Fraction(x[i][j])) for i, j in blk) for blk in blocks]
    payload = [[0] * W for _ in range(H)]
    e8 = [0] * n_blk
    gmax = []
    for g in range(M):
        G = max(m[g * K:(g + 1) * K])
        gmax.append(float(G))
        safe = G if G != 0 else Fraction(1)
        for n in range(g * K, (g + 1) * K):
            r = rn32(m[n] / safe)
            e = f32_bits_exponent(r)
            e8[n] = e
            s = Fraction(2) ** (e - 127) if e > 0 else Fraction(0)
            S = rn32(s * G)
            S = S if S > clamp else clamp
            for i, j in blocks[n]:
                xv = Fraction(x[i][j])
                q = rn32(rn32(xv / S) * 128)
                h = rnbf16(q)
                neg0 = (xv == 0 and math.copysign(1.0, x[i][j]) < 0)
                payload[i][j] = e4m3_byte(h, negative_zero=neg0 or (h == 0 and xv < 0))
    return payload, e8, gmax
