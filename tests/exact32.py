"""Correctly rounded float32 arithmetic from exact rationals (fractions.Fraction): the IEEE-754 binary32 results of a
product, a sum and a fused multiply-add (one rounding, to nearest, ties to even), computed from first principles and
not through the C library or the FPU's float32 path. Tests use it to pin an oracle's operation order bit for bit:
an fma in place of a product and a sum, or sums taken in another order, give other bits here."""
from fractions import Fraction

import numpy as np


def rn32(q):
    """Fraction -> np.float32, round to nearest, ties to even (normal and subnormal range; no overflow expected)"""
    q = Fraction(q)
    if q == 0:
        return np.float32(0.0)
    neg = q < 0
    a = -q if neg else q
    e = a.numerator.bit_length() - a.denominator.bit_length()  # 2^e <= a < 2^(e + 2)
    if Fraction(2) ** e > a:
        e -= 1
    while Fraction(2) ** (e + 1) <= a:
        e += 1
    e = max(e, -126)  # subnormals share the least exponent
    m = a * Fraction(2) ** (23 - e)  # the significand scaled to an integer of 24 bits
    n = m.numerator // m.denominator
    rem = m - n
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and n % 2 == 1):
        n += 1
    r = float(Fraction(n) * Fraction(2) ** (e - 23))  # exact in float64 (24 significant bits)
    return np.float32(-r if neg else r)


def F(x):
    return Fraction(float(np.float32(x)))


def mul(a, b):
    return rn32(F(a) * F(b))


def add(a, b):
    return rn32(F(a) + F(b))


def fma(a, b, c):
    return rn32(F(a) * F(b) + F(c))
