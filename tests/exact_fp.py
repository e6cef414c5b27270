"""Exact-rational IEEE binary32 / binary16 arithmetic for pinning the oracle.

Independent of numpy's float32 implementation: every value is a Fraction and
every operation is rounded to the target format with explicit
round-to-nearest-ties-to-even integer code.  Used only by tests.
"""
from __future__ import annotations

import math
import struct
from fractions import Fraction


def _round_to_format(x: Fraction, mant_bits: int, emin: int, emax: int) -> Fraction:
    """Round a rational to the nearest binary float with ``mant_bits`` fraction
    bits (ties to even), minimum normal exponent ``emin``; no overflow handling
    beyond returning inf."""
    if x == 0:
        return Fraction(0)
    sign = -1 if x < 0 else 1
    a = abs(x)
    # exponent e such that 2^e <= a < 2^(e+1)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    while Fraction(2) ** (e + 1) <= a:
        e += 1
    e = max(e, emin)                       # subnormal range shares emin's quantum
    quantum = Fraction(2) ** (e - mant_bits)
    q = a / quantum
    n = q.numerator // q.denominator
    rem = q - n
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and n % 2 == 1):
        n += 1
    r = n * quantum
    if r >= Fraction(2) ** (emax + 1):
        return Fraction(sign) * Fraction(10) ** 400  # stands in for inf
    return sign * r


def f32(x) -> Fraction:
    return _round_to_format(Fraction(x), 23, -126, 127)


def f16(x) -> Fraction:
    return _round_to_format(Fraction(x), 10, -14, 15)


def from_f32_bits(v: float) -> Fraction:
    """Exact value of a Python float that holds an fp32 value."""
    assert struct.unpack("<f", struct.pack("<f", v))[0] == v
    return Fraction(v)


def floor_frac(x: Fraction) -> int:
    return math.floor(x)


def ceil_frac(x: Fraction) -> int:
    return math.ceil(x)


EPS32 = f32(Fraction(1, 10 ** 8))       # fp32(1e-8)


def round_half_away_exact(t: Fraction) -> int:
    """F:198-202 with the +-0.5 added in fp32 (exactly rounded)."""
    if t >= 0:
        return floor_frac(f32(t + Fraction(1, 2)))
    return ceil_frac(f32(t - Fraction(1, 2)))


def quantize_int4_group_exact(vals, asymmetric: bool, clip_ratio: float):
    """Exact-rational restatement of one INT4 group (F:308-357).

    ``vals``: list of Fractions (fp32-representable inputs).  Returns
    ``(codes list[int], scale_f16 Fraction, zero_f16 Fraction or None)``.
    """
    if asymmetric:
        mn, mx = min(vals), max(vals)
        rng = max(f32(mx - mn), EPS32)
        scale = f32(rng / 15)
        codes = []
        for x in vals:
            t = f32(f32(x - mn) / scale)
            codes.append(min(max(round_half_away_exact(t), 0), 15))
        return codes, f16(scale), f16(mn)
    ax = [abs(x) for x in vals]
    amax = max(max(ax), EPS32)
    if clip_ratio > 0:
        below = [a if a < amax else Fraction(0) for a in ax]
        cnt = max(sum(1 for a in ax if a < amax), 1)
        # butterfly order: element i adds element i + stride
        v = list(below)
        n = len(v)
        while n > 1:
            n //= 2
            v = [f32(v[i] + v[i + n]) for i in range(n)]
        tmean = f32(v[0] / cnt)
        clip = f32(tmean * f32(Fraction(clip_ratio)))
        amax = min(amax, max(clip, EPS32))
    scale = f32(amax / 7)
    codes = []
    for x in vals:
        t = f32(x / scale)
        codes.append(min(max(round_half_away_exact(t), -8), 7) + 8)
    return codes, f16(scale), None


def quantize_int8_group_exact(vals):
    amax = max(max(abs(x) for x in vals), EPS32)
    scale = f32(amax / 127)
    codes = [min(max(round_half_away_exact(f32(x / scale)), -128), 127) for x in vals]
    return codes, f16(scale)
