"""The scaled attention score's division by sqrt(128) on the device
(`div_sqrt128_bf16`, re_device.h) is a product with the rounded reciprocal
and two fused corrections.  Checked here for every finite bf16 dividend with
exact integer arithmetic: after the bf16 rounding that follows it in the
kernels, it equals the bf16 rounding of the correctly rounded fp32 quotient
x / fp32(sqrt(128)), the IEEE division the reference performs."""
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


def test_every_finite_bf16_dividend():
    c, rc = f32_value(C_BITS), f32_value(RC_BITS)
    fp32_differ = 0
    for hi in range(1 << 16):
        if (hi >> 7) & 0xFF == 0xFF or hi & 0x7FFF == 0:
            continue  # inf / NaN (the kernel keeps the plain product there), zeros
        x = f32_value(hi << 16)
        exact = rne32(x / c)
        q0 = rne32(x * rc)
        q1 = rne32(q0 + rne32(x - q0 * c) * rc)  # fmaf(fmaf(-q0, c, x), rc, q0)
        if q1 != exact:
            fp32_differ += 1
            assert abs(x) < Fraction(2) ** -120, hex(hi)  # only where the correction underflows
        assert bf16_bits(q1) == bf16_bits(exact), hex(hi)
    assert fp32_differ == 28
