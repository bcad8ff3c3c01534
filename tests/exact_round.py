"""Exact binary rounding of rationals, for tests that pin the oracle's
floating-point steps with arithmetic independent of numpy's.

rne(q, p) rounds the rational q to the nearest number with a p-bit
significand and the fp32/bf16 exponent range (normal exponents down to -126,
subnormals below), ties to even; p = 24 is fp32, p = 8 is bf16.  The
routine is the textbook definition; tests/test_oracle_pins.py checks it
against numpy's float64 -> float32 cast and torch's float32 -> bfloat16 cast.
"""
from fractions import Fraction

EMIN = -126


def floor_log2(a):
    """floor(log2(a)) of a positive Fraction."""
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    while Fraction(2) ** (e + 1) <= a:
        e += 1
    return e


def rne(q, p):
    q = Fraction(q)
    if q == 0:
        return Fraction(0)
    sign = -1 if q < 0 else 1
    a = abs(q)
    e = max(floor_log2(a), EMIN)
    quantum = Fraction(2) ** (e - p + 1)
    n = a / quantum
    f = n.numerator // n.denominator
    rem = n - f
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and f % 2 == 1):
        f += 1
    return sign * f * quantum


def f32(q):
    return rne(q, 24)


def bf16(q):
    return rne(q, 8)


def frac(v):
    """Exact Fraction of a finite float or numpy float."""
    return Fraction(float(v))
