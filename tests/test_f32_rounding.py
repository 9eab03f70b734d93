"""The f32 form of the int8 rounding used by the single-pass quantize kernel
(rne_clamp127_f32 in csrc/tkv_device.h), restated with exact rationals.

The device helper computes r = fma(x, inv, 1.5 * 2^23) (the exact product
plus the constant, rounded once to nearest even in f32), clamps r to
1.5 * 2^23 +- 127, reads its bits minus those of 1.5 * 2^23, and gives 0 for
NaN.  This test emulates those steps with Fractions and a correct f32
rounding, and checks them against the reference's reading of
quantize_int8_symmetric (tv/quantization/engine.tkv:216-226): clamp(int(round(
x * inv)), -127, 127) with the product exact in f64 (two f32 factors), round
half to even, NaN -> 0, saturation.  Cases: random magnitudes from 2^-40 to
2^40, exact ties of both signs, neighbours of ties, products beyond 2^22
(where the constant's grid no longer holds), infinities and NaN.
"""
import math
import struct
from fractions import Fraction

import numpy as np

MAGIC = 12582912.0          # 1.5 * 2^23
MAGIC_BITS = 0x4B400000


def f32_round(v):
    """Correctly rounded (nearest even) f32 of an exact Fraction."""
    if v == 0:
        return 0.0
    sign = -1.0 if v < 0 else 1.0
    a = -v if v < 0 else v
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    e = max(e, -126)
    spacing = Fraction(2) ** (e - 23)
    q = a / spacing
    n = q.numerator // q.denominator
    rem = q - n
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and n % 2 == 1):
        n += 1
    r = n * spacing
    if r >= Fraction(2) ** 128:
        return sign * math.inf
    return sign * float(np.float32(float(r)))


def bits(f):
    return struct.unpack("<i", struct.pack("<f", f))[0]


def helper(x, inv):
    """The device helper's steps on f32 values x, inv (Python floats)."""
    if math.isnan(x) or math.isnan(inv):
        return 0
    if math.isinf(x) or math.isinf(inv):
        p = x * inv  # inf or nan (inf * 0)
        if math.isnan(p):
            return 0
        r = p         # fma of an infinite product: that infinity
    else:
        r = f32_round(Fraction(x) * Fraction(inv) + Fraction(MAGIC))
    c = min(max(r, MAGIC - 127.0), MAGIC + 127.0)
    return bits(c) - MAGIC_BITS


def reference(x, inv):
    with np.errstate(invalid="ignore"):
        p = np.float64(x) * np.float64(inv)   # exact: two f32 factors (inf * 0 is NaN)
    if np.isnan(p):
        return 0
    q = np.rint(p)
    return int(max(-127.0, min(127.0, q)))


def test_f32_rounding_matches_reference():
    rng = np.random.default_rng(20261202)
    cases = []
    for _ in range(6000):
        e = rng.integers(-40, 40)
        x = np.float32(rng.uniform(-1.0, 1.0) * 2.0 ** e)
        inv = np.float32(1.0 / np.float32(rng.uniform(1e-3, 1e3)))
        cases.append((float(x), float(inv)))
    # products near the codes' range, from the scale the kernel derives
    for _ in range(6000):
        am = np.float32(rng.uniform(1e-6, 1e6))
        scale = np.float32(np.float64(am) / 127.0)
        inv = np.float32(np.float32(1.0) / scale)
        x = np.float32(rng.uniform(-1.0, 1.0) * am)
        cases.append((float(x), float(inv)))
    # exact ties k + 1/2 of both signs and their f32 neighbours
    for k in range(-130, 130):
        x = np.float32(2 * k + 1)
        cases.append((float(x), 0.5))
        cases.append((float(np.nextafter(x, np.float32(np.inf))), 0.5))
        cases.append((float(np.nextafter(x, np.float32(-np.inf))), 0.5))
    # ties with a product of many significant bits: x * inv = k + 1/2 with
    # inv = 2^-20
    for k in (-127, -3, -1, 0, 1, 2, 126, 127, 128):
        x = np.float32((k + 0.5) * 2.0 ** 20)
        cases.append((float(x), 2.0 ** -20))
    # beyond the constant's exact range, huge, infinite and NaN
    for x in (2.0 ** 22, -2.0 ** 22, 2.0 ** 22 + 1, -(2.0 ** 22) - 1, 3.0e7, -3.0e7,
              1.5 * 2 ** 23, -1.5 * 2 ** 23, -1.6e7, -2.4e7, 3.0e38, -3.0e38,
              math.inf, -math.inf, math.nan, 0.0, -0.0, 1e-45, -1e-45):
        for inv in (1.0, 1e8, 0.0, 1.0 / 127.0):
            cases.append((float(np.float32(x)), float(np.float32(inv))))
    bad = [(x, inv, helper(x, inv), reference(x, inv)) for x, inv in cases
           if helper(x, inv) != reference(x, inv)]
    assert not bad, bad[:10]
