"""Exact-rational restatement of the quantizer (pure Python ``fractions``).

Used only to pin the oracle.  Every rounding step is done on exact rationals
with an explicit round-to-nearest-even into the target binary format, so the
result depends on nothing but the IEEE-754 definitions:

    fl32(a / b)         binary32 true division
    fp16(s)             binary16 with subnormals and overflow to inf
    rne_int(t)          round half to even to an integer

Slow (pure Python); meant for inputs of a few thousand elements.
"""

from __future__ import annotations

import math
from fractions import Fraction
from typing import List, Tuple

import numpy as np

F32 = (23, -126, 127)   # (fraction bits, min normal exponent, max exponent)
F16 = (10, -14, 15)
INF = float("inf")


def round_to_format(x: Fraction, fmt) -> object:
    """Nearest value of the binary format (ties to even); +-INF on overflow."""
    mant_bits, emin, emax = fmt
    if x == 0:
        return Fraction(0)
    sign = -1 if x < 0 else 1
    a = -x if x < 0 else x
    e = a.numerator.bit_length() - a.denominator.bit_length()
    while Fraction(2) ** e > a:
        e -= 1
    while Fraction(2) ** (e + 1) <= a:
        e += 1
    e = max(e, emin)                      # subnormals share the min exponent's quantum
    quantum = Fraction(2) ** (e - mant_bits)
    t = a / quantum
    fl = t.numerator // t.denominator
    rem = t - fl
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and fl % 2 == 1):
        fl += 1
    v = fl * quantum
    if v >= Fraction(2) ** (emax + 1):
        return sign * INF
    return sign * v


def rne_int(t: Fraction) -> int:
    fl = t.numerator // t.denominator
    rem = t - fl
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and fl % 2 == 1):
        fl += 1
    return fl


def _div_then_round(w: Fraction, s, lo: int, hi: int) -> int:
    """clamp(rne_int(fl32(w / s)), lo, hi) with IEEE semantics for s == 0 / inf."""
    if isinstance(s, float):                 # s == +inf: finite / inf = +-0
        return 0
    if s == 0:
        if w == 0:
            return 0                         # 0/0 = NaN -> int8 0
        return hi if w > 0 else lo           # +-inf clamps
    t = round_to_format(w / s, F32)
    if isinstance(t, float):                 # overflowed to +-inf
        return hi if t > 0 else lo
    return max(lo, min(hi, rne_int(t)))


def _scale(m: Fraction, div: int) -> Fraction:
    s32 = round_to_format(m / div, F32)
    floor = round_to_format(Fraction(1e-8), F32)
    if s32 < floor:
        s32 = floor
    return round_to_format(s32, F16)        # may be +inf for |w| > ~8.3e6


def exact_quantize_int8(w: np.ndarray) -> Tuple[np.ndarray, np.ndarray]:
    w = np.asarray(w, np.float32)
    n, k = w.shape
    q = np.zeros((n, k), np.int8)
    s = np.zeros((n,), np.float16)
    for r in range(n):
        row = [Fraction(float(v)) for v in w[r]]
        m = max(abs(v) for v in row)
        s16 = _scale(m, 127)
        s[r] = np.float16(float(s16))
        for c in range(k):
            q[r, c] = _div_then_round(row[c], s16, -127, 127)
    return q, s


def exact_quantize_int4(w: np.ndarray, g: int) -> Tuple[np.ndarray, np.ndarray]:
    """Returns (signed q [N, Kp] int8, scales [N, ng] fp16)."""
    w = np.asarray(w, np.float32)
    n, k = w.shape
    ng = (k + g - 1) // g
    kp = ng * g
    q = np.zeros((n, kp), np.int8)
    s = np.zeros((n, ng), np.float16)
    for r in range(n):
        row = [Fraction(float(v)) for v in w[r]] + [Fraction(0)] * (kp - k)
        for gi in range(ng):
            grp = row[gi * g:(gi + 1) * g]
            s16 = _scale(max(abs(v) for v in grp), 7)
            s[r, gi] = np.float16(float(s16))
            for j, v in enumerate(grp):
                q[r, gi * g + j] = _div_then_round(v, s16, -8, 7)
    return q, s


def exact_f16(x: float) -> float:
    v = round_to_format(Fraction(x), F16)
    return v if isinstance(v, float) else float(v)


def exact_dot(x: List[float], w: List[float]) -> Fraction:
    return sum((Fraction(float(a)) * Fraction(float(b)) for a, b in zip(x, w)), Fraction(0))


def is_close_f32(a: float, b: float) -> bool:
    return math.isclose(a, b, rel_tol=0, abs_tol=0)
