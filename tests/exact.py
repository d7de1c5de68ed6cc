"""Exact rational helpers for pinning the oracle's rounding (test infrastructure)."""
from fractions import Fraction

import numpy as np


def round_f32(x: Fraction) -> np.float32:
    """The f32 nearest to the rational x, ties to even (overflow to infinity)."""
    if x == 0:
        return np.float32(0.0)
    neg = x < 0
    x = -x if neg else x
    e = x.numerator.bit_length() - x.denominator.bit_length()
    if Fraction(2) ** e > x:
        e -= 1
    ulp_e = max(e, -126) - 23
    scaled = x / (Fraction(2) ** ulp_e)
    q, r = divmod(scaled.numerator, scaled.denominator)
    twice = 2 * r
    if twice > scaled.denominator or (twice == scaled.denominator and q % 2 == 1):
        q += 1
    value = Fraction(q) * Fraction(2) ** ulp_e
    if value >= Fraction(2) ** 128:
        f = np.float32(np.inf)
    else:
        f = np.float32(float(value))
    return np.float32(-f) if neg else f


def fma32(a, b, c) -> np.float32:
    """fmaf(a, b, c) from exact arithmetic: one rounding of a*b + c."""
    return round_f32(Fraction(float(a)) * Fraction(float(b)) + Fraction(float(c)))
