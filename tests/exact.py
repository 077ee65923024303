"""Exact rational arithmetic used to pin the oracle: IEEE round-to-nearest-even of a Fraction into a binary format
(bf16, fp32, fp16), independent of numpy's and torch's float conversions."""

from __future__ import annotations

import math
import struct
from fractions import Fraction

INF = float("inf")

# (precision bits incl. the implicit one, minimum normal exponent, maximum exponent)
BF16 = (8, -126, 127)
FP32 = (24, -126, 127)
FP16 = (11, -14, 15)


def exact_round(x: Fraction, fmt) -> Fraction | float:
    """x rounded to nearest, ties to even, in the format; +-inf on overflow."""
    p, emin, emax = fmt
    if x == 0:
        return Fraction(0)
    sign = -1 if x < 0 else 1
    a = abs(x)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    if Fraction(2) ** (e + 1) <= a:
        e += 1
    e = max(e, emin)
    ulp = Fraction(2) ** (e - (p - 1))
    r = a / ulp
    n = math.floor(r)
    rem = r - n
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and n % 2 == 1):
        n += 1
    res = n * ulp
    if res >= Fraction(2) ** (emax + 1):
        return sign * INF
    return sign * res


def f32_bits(x: float) -> int:
    return struct.unpack("<I", struct.pack("<f", x))[0]


def f32_from_bits(b: int) -> float:
    return struct.unpack("<f", struct.pack("<I", b))[0]


def bf16_bits_exact(x: float) -> int:
    """bf16 pattern of the float32 value x by exact rounding (NaN -> quiet NaN with x's top bits)."""
    if math.isnan(x):
        return ((f32_bits(x) >> 16) | 0x40) & 0xFFFF
    if math.isinf(x):
        return f32_bits(x) >> 16
    r = exact_round(Fraction(x), BF16)
    if isinstance(r, float):  # overflow
        return 0x7F80 if r > 0 else 0xFF80
    if r == 0:
        return f32_bits(x) >> 16 & 0x8000  # keeps the sign of zero
    return f32_bits(float(r)) >> 16


def fp32(x: Fraction) -> Fraction:
    r = exact_round(x, FP32)
    if isinstance(r, float):
        raise OverflowError
    return r
