"""The scaled attention score's division by sqrt(128) on the device
(`div_sqrt128_bf16`, re_device.h) is the product with the rounded
reciprocal.  Checked here for every bf16 dividend with exact integer
arithmetic: after the bf16 rounding that follows it in the kernels, it
equals the bf16 rounding of the correctly rounded fp32 quotient
x / fp32(sqrt(128)), the IEEE division the reference performs.  Planted: a
reciprocal held in bf16 and a truncating bf16 rounding must fail (the
quotients sit far from every bf16 rounding boundary, so the fp32
reciprocal's neighbours a few ulps away would still pass)."""
from __future__ import annotations

import math
import struct
from fractions import Fraction

C_BITS, RC_BITS = 0x413504F3, 0x3DB504F3


def f32_value(bits: int) -> Fraction:
    return Fraction(struct.unpack("<f", struct.pack("<I", bits))[0])


def rne32(v: Fraction) -> Fraction:
    """Round a finite rational to the nearest fp32 value (ties to even),
    subnormals included, without overflow handling (not reached here)."""
    if v == 0:
        return Fraction(0)
    sign = -1 if v < 0 else 1
    num, den = abs(v.numerator), v.denominator
    e = num.bit_length() - den.bit_length()
    if (num << max(0, -e)) < (den << max(0, e)):
        e -= 1  # now 2^e <= |v| < 2^(e+1)
    q = max(e, -126) - 23  # exponent of one unit in the last place
    n_num, n_den = (num << -q, den) if q < 0 else (num, den << q)
    n, rem = divmod(n_num, n_den)
    if 2 * rem > n_den or (2 * rem == n_den and n & 1):
        n += 1
    return sign * Fraction(n) * (Fraction(2) ** q)


def bf16_bits(v: Fraction) -> int:
    b = struct.unpack("<I", struct.pack("<f", float(v)))[0]  # v is an fp32 value: exact
    return ((b + 0x7FFF + ((b >> 16) & 1)) >> 16) & 0xFFFF


def test_constants_are_the_rounded_sqrt_and_reciprocal():
    c = f32_value(C_BITS)
    assert c == Fraction(struct.unpack("<f", struct.pack("<f", math.sqrt(128.0)))[0])
    half_ulp = Fraction(1, 2 ** 21)  # c lies in [8, 16): one ulp is 2^-20
    assert (c - half_ulp) ** 2 < 128 < (c + half_ulp) ** 2  # c is sqrt(128) correctly rounded
    assert f32_value(RC_BITS) == rne32(1 / c)


def product_mismatches(rc_bits: int, rounding=None) -> tuple[int, int]:
    """(fp32 results that differ from the division, bf16 results that differ)
    over every finite nonzero bf16 dividend, for the product x * rc."""
    rounding = rounding or bf16_bits
    c, rc = f32_value(C_BITS), f32_value(rc_bits)
    fp32_differ = bf16_differ = 0
    for hi in range(1 << 16):
        if (hi >> 7) & 0xFF == 0xFF or hi & 0x7FFF == 0:
            continue  # inf / NaN and zeros pass through the product unchanged
        x = f32_value(hi << 16)
        exact = rne32(x / c)
        q = rne32(x * rc)
        fp32_differ += q != exact
        bf16_differ += rounding(q) != bf16_bits(exact)
    return fp32_differ, bf16_differ


def test_every_finite_bf16_dividend():
    fp32_differ, bf16_differ = product_mismatches(RC_BITS)
    assert bf16_differ == 0
    assert fp32_differ == 26650  # the fp32 products differ; the bf16 roundings never do


def test_planted_mistakes_fail():
    # the reciprocal held in bf16, the reciprocal of a bf16 sqrt(128), and a
    # bf16 rounding that truncates
    assert product_mismatches(0x3DB50000)[1] > 0
    c_bf16 = struct.unpack("<f", struct.pack("<I", 0x41350000))[0]
    assert product_mismatches(struct.unpack("<I", struct.pack("<f", 1.0 / c_bf16))[0])[1] > 0
    truncate = lambda v: (struct.unpack("<I", struct.pack("<f", float(v)))[0] >> 16) & 0xFFFF
    assert product_mismatches(RC_BITS, truncate)[1] > 0
