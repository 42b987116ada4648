"""Exact-arithmetic helpers used to pin the oracle: IEEE binary16/binary32
rounding of rational numbers, written from the IEEE-754 definition (round to
nearest, ties to even; gradual underflow; overflow to infinity)."""
import math
import struct
from fractions import Fraction


def round_to_format(v: Fraction, mant_bits: int, emin: int, emax: int):
    """Round the rational v to the binary format with `mant_bits` explicit
    fraction bits, minimum normal exponent emin and maximum exponent emax.
    Returns a Fraction, or ±math.inf."""
    if v == 0:
        return Fraction(0)
    sign = -1 if v < 0 else 1
    a = abs(v)
    e = math.floor(math.log2(a.numerator) - math.log2(a.denominator))
    # fix floating error in the log estimate
    while Fraction(2) ** e > a:
        e -= 1
    while Fraction(2) ** (e + 1) <= a:
        e += 1
    e = max(e, emin)
    ulp = Fraction(2) ** (e - mant_bits)
    q = a / ulp
    fl = q.numerator // q.denominator
    rem = q - fl
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and fl % 2 == 1):
        fl += 1
    r = fl * ulp
    max_val = (2 - Fraction(2) ** (-mant_bits)) * Fraction(2) ** emax
    if r > max_val:
        return sign * math.inf
    return sign * r


def to_f16(v: Fraction):
    return round_to_format(v, 10, -14, 15)


def to_f32(v: Fraction):
    return round_to_format(v, 23, -126, 127)


def round_half_even(v: Fraction) -> int:
    fl = v.numerator // v.denominator
    rem = v - fl
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and fl % 2 == 1):
        fl += 1
    return fl


def f32(x: float) -> float:
    """Round a Python float (double) to binary32."""
    return struct.unpack("f", struct.pack("f", x))[0]
