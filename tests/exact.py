"""Exact rational arithmetic with explicit IEEE rounding, used to pin the oracle.

Independent of numpy's float32 implementation: every value is a fractions.Fraction and
rounding to a binary format (p significand bits, minimum normal exponent emin) is done
by hand with round-half-to-even, so a mistake in the oracle's float handling (a wrong
rounding mode, a fused multiply, a transposed operand order) shows up as a mismatch.
"""

from __future__ import annotations

import math
from fractions import Fraction

import numpy as np


def round_binary(value: Fraction, p: int, emin: int, emax: int) -> Fraction | float:
    """Round `value` to the nearest p-bit binary float (ties to even); inf on overflow."""
    if value == 0:
        return Fraction(0)
    sign = -1 if value < 0 else 1
    a = abs(value)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    elif Fraction(2) ** (e + 1) <= a:
        e += 1
    e = max(e, emin)
    ulp = Fraction(2) ** (e - (p - 1))
    q = a // ulp
    r = a - q * ulp
    half = ulp / 2
    if r > half or (r == half and q % 2 == 1):
        q += 1
    result = q * ulp
    if result >= Fraction(2) ** (emax + 1):
        return sign * math.inf
    return sign * result


def f32(value: Fraction) -> Fraction | float:
    return round_binary(Fraction(value), 24, -126, 127)


def bf16(value: Fraction) -> Fraction | float:
    return round_binary(Fraction(value), 8, -126, 127)


def frac(x) -> Fraction:
    return Fraction(float(x))


def bf16_bits(value) -> int:
    """BF16 bit pattern of a value that is already exactly representable in BF16."""
    return int(np.array([float(value)], dtype=np.float32).view(np.uint32)[0] >> 16)


def rne_int(value: Fraction) -> int:
    """Round a rational to the nearest integer, ties to even."""
    q = math.floor(value)
    r = value - q
    if r > Fraction(1, 2) or (r == Fraction(1, 2) and q % 2 == 1):
        q += 1
    return q
