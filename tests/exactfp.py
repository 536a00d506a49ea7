"""Exact IEEE-754 binary32 arithmetic on rationals, for pinning operation order.

round_f32(q) rounds a Fraction to the nearest binary32 (ties to even), so that
fma(a, b, c) = round_f32(a*b + c) and add(a, b) = round_f32(a + b) are exact
models of the hardware operations, independent of numpy and of any FMA unit.
"""
from fractions import Fraction

import numpy as np


def round_f32(q: Fraction) -> np.float32:
    if q == 0:
        return np.float32(0.0)
    sign = -1 if q < 0 else 1
    a = -q if q < 0 else q
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    # now 2^e <= a < 2^(e+1)
    e = max(e, -126)  # subnormal range shares the 2^-149 quantum
    quantum = Fraction(2) ** (e - 23)
    m = a / quantum
    n = m.numerator // m.denominator
    rem = m - n
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and n % 2 == 1):
        n += 1
    val = n * quantum
    if val >= Fraction(2) ** 128:
        return np.float32(sign * np.inf)
    return np.float32(sign * float(val))


def F(x) -> Fraction:
    return Fraction(float(x))


def fma(a, b, c) -> np.float32:
    return round_f32(F(a) * F(b) + F(c))


def add(a, b) -> np.float32:
    return round_f32(F(a) + F(b))


def mul(a, b) -> np.float32:
    return round_f32(F(a) * F(b))
