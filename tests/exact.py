"""Exact-arithmetic helpers for pinning the oracle: IEEE rounding of rationals."""
from fractions import Fraction
import math

import numpy as np

HALF = (10, -14, 15)     # fraction bits, minimum normal exponent, maximum exponent
SINGLE = (23, -126, 127)


def round_fraction(value, fmt):
    """Round a Fraction to the nearest value of an IEEE binary format, ties to even.
    Returns a Fraction, or +-inf (as float) on overflow."""
    bits, emin, emax = fmt
    if value == 0:
        return Fraction(0)
    sign = -1 if value < 0 else 1
    a = abs(value)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    if Fraction(2) ** (e + 1) <= a:
        e += 1
    e = max(e, emin)
    quantum = Fraction(2) ** (e - bits)
    q = a / quantum
    n = math.floor(q)
    r = q - n
    if r > Fraction(1, 2) or (r == Fraction(1, 2) and n % 2 == 1):
        n += 1
    result = n * quantum
    largest = (2 - Fraction(2) ** -bits) * Fraction(2) ** emax
    if result > largest:
        return sign * math.inf
    return sign * result


def half_value(bits):
    return Fraction(float(np.array([bits], dtype=np.uint16).view(np.float16)[0]))


def to_half_bits(value):
    if isinstance(value, float) and math.isinf(value):
        return 0x7c00 if value > 0 else 0xfc00
    return int(np.array([float(value)], dtype=np.float16).view(np.uint16)[0])


def to_f32(value):
    return np.float32(float(value))
