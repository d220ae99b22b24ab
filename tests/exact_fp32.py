"""Exact binary32 arithmetic in pure Python, for pinning the oracle.

Every operation is computed exactly on rationals (fractions.Fraction) and then
rounded once to the nearest binary32 value, ties to even, with subnormals and
overflow to infinity. This is the IEEE-754 definition of a correctly rounded
fp32 operation, independent of any C library or compiler: the tests use it to
check the oracle's quantizer, weight expansion and epilogue on small inputs.
Only finite values are handled; callers treat NaN/Inf cases separately.
"""
from __future__ import annotations

import math
from fractions import Fraction

_EMIN = -126      # smallest normal exponent
_MANT = 23        # fraction bits
_MAX = (2 - Fraction(1, 2**23)) * Fraction(2) ** 127


def round_f32(v: Fraction) -> float:
    """Round a rational to the nearest binary32 (ties to even); returns a Python float."""
    if v == 0:
        return 0.0
    sign = -1.0 if v < 0 else 1.0
    a = abs(v)
    # exponent e with 2^e <= a < 2^(e+1)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    elif Fraction(2) ** (e + 1) <= a:
        e += 1
    ulp_exp = max(e, _EMIN) - _MANT
    ulp = Fraction(2) ** ulp_exp
    n = a / ulp
    fl = n.numerator // n.denominator
    rem = n - fl
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and fl % 2 == 1):
        fl += 1
    r = fl * ulp
    if r > _MAX:
        return sign * math.inf
    return sign * float(r)


def f32(x) -> float:
    """Round a Python float (double) to binary32."""
    return round_f32(_q(x))


def _q(a) -> Fraction:
    return Fraction(float(a))


def mul(a: float, b: float) -> float:
    return round_f32(_q(a) * _q(b))


def div(a: float, b: float) -> float:
    return round_f32(_q(a) / _q(b))


def add(a: float, b: float) -> float:
    return round_f32(_q(a) + _q(b))


def fma(a: float, b: float, c: float) -> float:
    return round_f32(_q(a) * _q(b) + _q(c))


def sqrt(a: float) -> float:
    """Correctly rounded square root of a finite a >= 0. floor(sqrt(q) * 2^p) is an
    integer square root; with p = 160 every binary32 rounding midpoint times 2^p is an
    integer, so a remainder (inexact root) can be represented by adding half a unit."""
    q = _q(a)
    if q < 0:
        raise ValueError("sqrt of a negative value")
    if q == 0:
        return float(a)
    p = 160
    num, den = q.numerator << (2 * p), q.denominator
    S = math.isqrt(num // den)
    exact = S * S * den == num
    return round_f32(Fraction(S, 2 ** p) if exact else Fraction(2 * S + 1, 2 ** (p + 1)))


def rne_int(y: float) -> int:
    """Round to the nearest integer, ties to even (CVTPS2DQ's default mode)."""
    fy = _q(y)
    fl = fy.numerator // fy.denominator
    rem = fy - fl
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and fl % 2 == 1):
        fl += 1
    return int(fl)


def lround(y: float) -> int:
    """Round to the nearest integer, ties away from zero (C lround)."""
    fy = abs(_q(y))
    n = (fy + Fraction(1, 2))
    r = n.numerator // n.denominator
    return int(-r if y < 0 else r)


# --- the path, restated on exact arithmetic ---------------------------------

BLOCK = 256


def quantize_block(xs, act_max: int = 127):
    """One (token, block): returns (u8 values, scale). Finite inputs only."""
    amax = 0.0
    for v in xs:
        amax = max(amax, abs(v))
    sx = div(amax, float(act_max))
    inv = div(float(act_max), amax) if amax > 0 else 0.0
    q = []
    for v in xs:
        c = rne_int(mul(v, inv))
        u = c + act_max + 1
        q.append(min(255, max(0, u)))
    return q, sx


def expand_block(ws):
    """One (weight row, block): returns (s8 values, scale, sum)."""
    amax = 0.0
    for v in ws:
        amax = max(amax, abs(v))
    inv = div(127.0, amax) if amax > 0 else 0.0
    q = [lround(mul(v, inv)) for v in ws]
    return q, div(amax, 127.0), sum(q)


def linear_point(wrow, srow, orow, qrow, sxrow, res=None):
    """y[t, r] for one (token, row): wrow s8 list, srow/orow per-block scale/off,
    qrow u8 list, sxrow per-block activation scales."""
    n_in = len(wrow)
    f = 0.0
    for B in range((n_in + BLOCK - 1) // BLOCK):
        i0, i1 = B * BLOCK, min(n_in, (B + 1) * BLOCK)
        s = sum(int(wrow[i]) * int(qrow[i]) for i in range(i0, i1)) + int(orow[B])
        p = mul(f32(float(s)), sxrow[B])
        f = fma(p, srow[B], f)
    return f if res is None else add(res, f)
