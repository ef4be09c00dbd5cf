"""The fp8 cache writer divides by reciprocal and one FMA correction; pin it to IEEE division.

``mla_kvcache_write_kernel`` (flagattention_amd/csrc/fa_kvcache.hip) computes the e4m3 code
input ``x / scale`` as ``q0 = x * y`` with ``y = 1 / scale``, ``r = fma(-scale, q0, x)``,
``q = copysign(fma(r, y, q0), x)`` (every step one fp32 operation, rounded to nearest even),
and the oracle uses IEEE division.  The writer's divisors are ``scale = amax / 448`` for a
bf16 ``amax``, and its dividends are bf16, so every (x, scale) pair is one of 128 x 128
mantissa pairs times a power of two; powers of two scale every step exactly (the kernel
takes this path only for finite tiles with scales of at least 2^-60, where no step that matters
underflows or overflows).
So checking all 16,384 mantissa pairs with exact rational arithmetic covers the domain.
Planted mistakes (the uncorrected ``q0``; no sign copy) must fail.
"""
from fractions import Fraction

import numpy as np

BF16_MANT = [Fraction(128 + m, 128) for m in range(128)]  # 1.0 .. 1.9921875


def rn32(v: Fraction) -> Fraction:
    """Round a rational to the nearest float32 (ties to even mantissa), exactly."""
    if v == 0:
        return Fraction(0)
    c = np.float32(float(v))  # within one float32 step of the answer
    best = None
    for cand in (np.nextafter(c, np.float32(-np.inf)), c, np.nextafter(c, np.float32(np.inf))):
        d = abs(Fraction(float(cand)) - v)
        even = (np.array([cand], dtype=np.float32).view(np.uint32)[0] & 1) == 0
        if best is None or d < best[0] or (d == best[0] and even):
            best = (d, cand)
    return Fraction(float(best[1]))


def kernel_quotient(x: Fraction, s: Fraction, y: Fraction, correct: bool = True) -> Fraction:
    q0 = rn32(x * y)
    if not correct:
        return q0
    r = rn32(x - s * q0)       # fma(-scale, q0, x)
    return rn32(q0 + r * y)     # fma(r, y, q0)


def _scales():
    return sorted({rn32(a / 448) for a in BF16_MANT})


def test_scale_mantissas_cover_the_writer():
    """128 amax mantissas give 128 distinct scale mantissas, 1 / 448 * [1, 2)."""
    s = _scales()
    assert len(s) == 128 and s[0] == rn32(Fraction(1, 448))


def test_corrected_quotient_equals_ieee_division_exhaustively():
    bad = []
    for s in _scales():
        y = rn32(1 / s)
        for xm in BF16_MANT:
            for x in (xm, xm * 2, -xm):  # quotients on both sides of a binade edge, and the sign
                if kernel_quotient(x, s, y) != rn32(x / s):
                    bad.append((float(x), float(s)))
    assert bad == []


def test_planted_uncorrected_quotient_fails():
    bad = 0
    for s in _scales():
        y = rn32(1 / s)
        for xm in BF16_MANT:
            bad += kernel_quotient(xm, s, y, correct=False) != rn32(xm / s)
    assert bad > 0  # the correction is needed: x * (1 / scale) alone is not the IEEE quotient


def test_negative_zero_keeps_its_sign_only_with_copysign():
    """fma(r, y, q0) turns x = -0 into +0 (the e4m3 code 0x00 instead of 0x80)."""
    s = np.float32(1.0 / 448.0)
    y = np.float32(1.0) / s
    x = np.float32(-0.0)
    q0 = x * y
    r = np.float32(np.float64(-s) * np.float64(q0) + np.float64(x))  # exact: all terms are zero
    q = np.float32(np.float64(r) * np.float64(y) + np.float64(q0))
    assert np.signbit(q0) and not np.signbit(q)  # the correction loses the sign...
    assert np.signbit(np.copysign(q, x))         # ...and copysign restores it
