"""Exact-rational brute force of the v3 codec for tiny inputs (CPU oracle).

TEST INFRASTRUCTURE ONLY.  An implementation independent of oracle/codec.py:
every IEEE step of `v3_quantize_group_absmax` (reference
src/flashffn.py:1071-1088) is done in `fractions.Fraction` arithmetic with an
explicit rounding function, so numpy's float32 division, float16 cast and
`rint` are checked against the definition of round-to-nearest-even rather than
against another floating-point library.

Rounding model (IEEE 754 binary formats, round-to-nearest, ties-to-even,
gradual underflow, overflow to +-inf):
  binary32: 24-bit significand, emin = -126;  binary16: 11-bit, emin = -14.
"""

from __future__ import annotations

import math
from fractions import Fraction

INF = float("inf")


def _round_half_even(x: Fraction) -> int:
    fl = math.floor(x)
    rem = x - fl
    if rem > Fraction(1, 2):
        return fl + 1
    if rem < Fraction(1, 2):
        return fl
    return fl if fl % 2 == 0 else fl + 1


def round_to_format(x: Fraction, precision: int, emin: int, emax: int):
    """Round an exact rational to the nearest value of a binary format.
    Returns a Fraction, or +-inf on overflow."""
    if x == 0:
        return Fraction(0)
    sign = -1 if x < 0 else 1
    a = -x if x < 0 else x
    # exponent e with 2**e <= a < 2**(e+1)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    elif Fraction(2) ** (e + 1) <= a:
        e += 1
    e = max(e, emin)                       # subnormals share emin's quantum
    quantum = Fraction(2) ** (e - (precision - 1))
    m = _round_half_even(a / quantum)
    r = m * quantum
    max_finite = (2 - Fraction(2) ** (1 - precision)) * Fraction(2) ** emax
    if r > max_finite:
        return -INF if sign < 0 else INF
    return sign * r


def to_f32(x: Fraction):
    return round_to_format(x, 24, -126, 127)


def to_f16(x: Fraction):
    return round_to_format(x, 11, -14, 15)


def quantize_group_exact(values, bits: int):
    """One group of exactly representable floats -> (scale, codes).

    scale = f16(f32(absmax / qmax)); safe = scale if scale > 0 else 1;
    code  = clamp(rint(f32(v / safe)), -qmax, qmax).
    scale is returned as a Fraction or +-inf."""
    qmax = 2 ** (bits - 1) - 1
    vals = [Fraction(v) for v in values]
    absmax = max(abs(v) for v in vals)
    s32 = to_f32(absmax / qmax)
    scale = to_f16(s32) if not isinstance(s32, float) else s32
    if isinstance(scale, float):           # overflow: safe = inf -> v/inf = 0
        return scale, [0 for _ in vals]
    safe = scale if scale > 0 else Fraction(1)
    codes = []
    for v in vals:
        qv = to_f32(v / safe)
        if isinstance(qv, float):          # quotient overflowed f32
            c = qmax if qv > 0 else -qmax
        else:
            c = max(-qmax, min(qmax, _round_half_even(qv)))
        codes.append(c)
    return scale, codes


def quantize_exact(rows, bits: int, group_size: int):
    """rows: list of lists of floats. Returns (codes [N][D], scales [N][G])."""
    codes, scales = [], []
    for row in rows:
        assert len(row) % group_size == 0
        crow, srow = [], []
        for g0 in range(0, len(row), group_size):
            s, c = quantize_group_exact(row[g0:g0 + group_size], bits)
            crow.extend(c)
            srow.append(s)
        codes.append(crow)
        scales.append(srow)
    return codes, scales
