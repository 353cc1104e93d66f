"""The pack kernels' scale and quotient arithmetic against exact arithmetic (CPU).

The HIP pack (csrc/kv_pages.hip) computes the reference's per-row scale and codes
(wave_rt/denoiser/exchange/common.py:145-150, per (token, head)) with cheaper
operations than the IEEE divisions the reference's torch ops perform:

* s = bf16(amax * RN(1/448)) in place of bf16(amax / 448);
* the quotient |x| / s as q = RN(|x| * r), q' = RN(q + RN(|x| - q s) * r) with r
  from the hardware reciprocal, which is within one ulp of 1/s.

These tests check both claims against exact arithmetic: the first over every
non-negative finite bf16 amax, the second over every pair of 8-bit significands
of x and s, both neighbours of 1/s in fp32 as r, and every power-of-two scaling
that reaches an e4m3 code, compared through the independent e4m3 encoder.
"""

from __future__ import annotations

from fractions import Fraction

import numpy as np

from oracle import fp8 as of8

F32 = np.float32


def _bf16_rne(x: np.ndarray) -> np.ndarray:
    u = x.astype(F32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return (u.astype(np.uint32) << 16).view(F32)


def test_scale_by_reciprocal_equals_bf16_of_the_division_for_every_bf16_amax():
    amax = (np.arange(0, 0x7F80, dtype=np.uint32) << 16).view(F32)   # +0 .. largest finite bf16
    inv = F32(1) / F32(448)
    by_mul = _bf16_rne((amax * inv).astype(F32))
    by_div = _bf16_rne((amax / F32(448)).astype(F32))
    assert np.array_equal(by_mul.view(np.uint32), by_div.view(np.uint32))
    # a wrong constant (bf16-rounded 1/448) is caught
    inv_bf16 = _bf16_rne(np.array([inv]))[0]
    assert not np.array_equal(_bf16_rne((amax * inv_bf16).astype(F32)), by_div)


def _rn32(v: Fraction) -> Fraction:
    """Round a rational to the nearest fp32 value, ties to even (normal range)."""
    if v == 0:
        return Fraction(0)
    sign = -1 if v < 0 else 1
    a = abs(v)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    scale = Fraction(2) ** (23 - e)            # a * scale in [2^23, 2^24)
    m = a * scale
    n, rem = divmod(m.numerator, m.denominator)
    twice = 2 * rem
    if twice > m.denominator or (twice == m.denominator and n % 2 == 1):
        n += 1
    return sign * Fraction(n) / scale


def _quotient(x: Fraction, s: Fraction, r: Fraction) -> Fraction:
    q = _rn32(x * r)
    e = _rn32(x - q * s)
    return _rn32(e * r + q)


def test_quotient_with_either_reciprocal_neighbour_gives_the_exact_quotients_code():
    ks = np.arange(-17, 10)
    scale = np.exp2(ks.astype(np.float64))
    mismatches = 0
    checked = 0
    for ms in range(128, 256):
        s = Fraction(ms, 128)
        inv = F32(128.0 / ms)
        cands = {Fraction(float(np.nextafter(inv, F32(0)))), Fraction(float(inv)),
                 Fraction(float(np.nextafter(inv, F32(4))))}
        cands = {c for c in cands if abs(c - 1 / s) < Fraction(1, 1 << 23)}    # within one ulp of 1/s
        assert len(cands) >= 2
        xs = [Fraction(mx, 128) for mx in range(1, 256)]
        exact = np.array([float(x / s) for x in xs])      # exact when dyadic, else ~2^-53 off (far from boundaries)
        want = of8.encode_bits(np.minimum(exact[:, None] * scale[None, :], 448.0).astype(F32))
        for r in cands:
            got_q = np.array([float(_quotient(x, s, r)) for x in xs])
            got = of8.encode_bits(np.minimum(got_q[:, None] * scale[None, :], 448.0).astype(F32))
            mismatches += int((got != want).sum())
            checked += got.size
    assert checked > 200_000 and mismatches == 0


def test_quotient_without_the_residual_step_misses_exact_ties():
    """The residual step is needed: x * r alone lands on the wrong side of an exact e4m3 tie."""
    misses = 0
    for ms in range(129, 256):
        s = Fraction(ms, 128)
        inv = F32(128.0 / ms)
        for r in (Fraction(float(np.nextafter(inv, F32(0)))), Fraction(float(np.nextafter(inv, F32(4))))):
            for mx in range(1, 256):
                x = Fraction(mx, 128)
                exact = x / s
                if exact.denominator & (exact.denominator - 1):
                    continue                                  # only exact (dyadic) quotients
                one_step = float(_rn32(x * r))
                for k in range(-17, 10):
                    w = of8.encode_bits(np.array([min(float(exact) * 2.0 ** k, 448.0)], dtype=F32))[0]
                    g = of8.encode_bits(np.array([min(one_step * 2.0 ** k, 448.0)], dtype=F32))[0]
                    misses += int(w != g)
    assert misses > 0
