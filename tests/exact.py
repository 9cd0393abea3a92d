"""Exact-rational float32 arithmetic for pinning the oracle on tiny inputs.

``fma32`` rounds a*b+c computed exactly in rationals to the nearest float32
(ties to even), i.e. the IEEE-754 fusedMultiplyAdd the reference's
``f32::mul_add`` specifies.  No float arithmetic is involved, so it is
independent of numpy, libm and the C oracle.
"""
from __future__ import annotations

from fractions import Fraction

import numpy as np


def f32_fraction(v) -> Fraction:
    return Fraction(float(np.float32(v)))


def round_f32(q: Fraction) -> np.float32:
    if q == 0:
        return np.float32(0.0)
    sign = -1 if q < 0 else 1
    a = -q if q < 0 else q
    # exponent e with 2^e <= a < 2^(e+1)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    elif Fraction(2) ** (e + 1) <= a:
        e += 1
    e = max(e, -126)                      # subnormal range keeps the 2^-149 grid
    scaled = a / (Fraction(2) ** (e - 23))  # in [2^23, 2^24) for normals
    m = scaled.numerator // scaled.denominator
    rem = scaled - m
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and m % 2 == 1):
        m += 1
    value = Fraction(m) * (Fraction(2) ** (e - 23))
    if value >= Fraction(2) ** 128:
        return np.float32(sign * np.inf)
    return np.float32(sign * float(value))


def fma32(a, b, c) -> np.float32:
    return round_f32(f32_fraction(a) * f32_fraction(b) + f32_fraction(c))


def fold_dot(weights, x) -> np.float32:
    """sum = fma(w[c], x[c], sum) for c = 0.. in order (src/cpu.rs:391-394)."""
    s = np.float32(0.0)
    for w, v in zip(weights, x):
        s = fma32(w, v, s)
    return s
