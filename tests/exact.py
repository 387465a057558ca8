"""Exact rational arithmetic with explicit IEEE-754 rounding, used to pin the oracle's f32/f16 steps.

Nothing here calls numpy's float arithmetic: values are fractions.Fraction, and round_ieee() rounds a rational to the
nearest binary32 / binary16 value (ties to even, overflow to infinity, gradual underflow), from the definition of
the formats.  A computation rebuilt from these pieces is an independent restatement of "each f32 operation is
correctly rounded", so a dropped rounding step or an operation done in the wrong precision shows up as a mismatch.
"""

from __future__ import annotations

import math
import struct
from fractions import Fraction

F32 = dict(mant=24, emin=-126, emax=127)
F16 = dict(mant=11, emin=-14, emax=15)


def round_ieee(q: Fraction, fmt=F32):
    """Nearest representable value of `fmt` to the rational q (ties to even); returns a Fraction or +-inf."""
    if q == 0:
        return Fraction(0)
    sign = -1 if q < 0 else 1
    a = abs(q)
    # exponent e with 2^e <= a < 2^(e+1)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    elif Fraction(2) ** (e + 1) <= a:
        e += 1
    e = max(e, fmt["emin"])  # subnormals share the minimum exponent
    ulp = Fraction(2) ** (e - (fmt["mant"] - 1))
    n = a / ulp
    fl = n.numerator // n.denominator
    rem = n - fl
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and fl % 2 == 1):
        fl += 1
    r = fl * ulp
    max_finite = (2 - Fraction(2) ** (1 - fmt["mant"])) * Fraction(2) ** fmt["emax"]
    if r > max_finite:
        return sign * math.inf
    return sign * r


def f32(x) -> Fraction:
    """Exact value of a Python float / numpy float32 known to be binary32-representable."""
    return Fraction(float(x))


def to_float(q):
    return float(q) if not isinstance(q, float) else q


def f16_from_bits(bits: int):
    """binary16 bit pattern -> exact value (Fraction) or +-inf / nan, from the field definitions."""
    s = -1 if bits & 0x8000 else 1
    e = (bits >> 10) & 0x1F
    m = bits & 0x3FF
    if e == 0x1F:
        return s * math.inf if m == 0 else math.nan
    if e == 0:
        return s * Fraction(m, 1024) * Fraction(1, 2**14)
    return s * (1 + Fraction(m, 1024)) * Fraction(2) ** (e - 15)


def round_half_away(q: Fraction) -> int:
    a = abs(q)
    f = a.numerator // a.denominator
    r = f + 1 if a - f >= Fraction(1, 2) else f
    return -r if q < 0 else r


def round_half_even(q: Fraction) -> int:
    a = abs(q)
    f = a.numerator // a.denominator
    d = a - f
    r = f + 1 if d > Fraction(1, 2) or (d == Fraction(1, 2) and f % 2 == 1) else f
    return -r if q < 0 else r


def q8_0_block(xs):
    """ggml quantize_row_q8_0_ref on one block of 32 f32 values, in exact arithmetic with explicit roundings.
    -> (q list, stored d as a float (f32 of the f16-rounded d))."""
    vals = [f32(v) for v in xs]
    amax = max(abs(v) for v in vals)
    d = round_ieee(amax / 127)
    idv = round_ieee(1 / d) if d != 0 else Fraction(0)
    q = [round_half_away(round_ieee(v * idv)) for v in vals]
    d16 = round_ieee(d, F16)
    return q, (float(d16) if not isinstance(d16, float) else d16)


def q8_K_block(xs):
    """ggml quantize_row_q8_K_ref on one block of 256 f32 values, exactly.  -> (q list, d float, bsums list)."""
    vals = [f32(v) for v in xs]
    amax = max(abs(v) for v in vals)
    if amax == 0:
        return [0] * len(vals), 0.0, [0] * (len(vals) // 16)
    first = next(i for i, v in enumerate(vals) if abs(v) == amax)
    iscale = round_ieee(Fraction(-127) / vals[first])
    q = [min(127, round_half_even(round_ieee(iscale * v))) for v in vals]
    d = round_ieee(1 / iscale)
    bs = [sum(q[j * 16 : (j + 1) * 16]) for j in range(len(vals) // 16)]
    return q, float(d), bs


def f32_bits(x: float) -> int:
    return struct.unpack("<I", struct.pack("<f", x))[0]
