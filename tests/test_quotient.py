"""The attention kernels' division: q = acc * (1/l), then one residual step
q + fma(-q, l, acc) * (1/l) with the correctly rounded fp32 reciprocal
(Markstein's correction), stands in for the correctly rounded acc / l that
the HTile program's arith.divf asks for (HTile:137-140). This checks the
identity on random fp32 pairs over the ranges the kernels meet: row sums l
in [2^-10, 2^40], accumulators in [2^-60, 2^60], both signs.

The two fused multiply-adds are emulated exactly: their exact values are
rationals, rounded once to fp32 (round to nearest, ties to even); the
reciprocal, the plain product and the reference quotient are numpy's
correctly rounded fp32 operations.
"""

from fractions import Fraction

import numpy as np


def _rn32(x: Fraction) -> np.float32:
    """x rounded to the nearest fp32, ties to even (normal range)."""
    if x == 0:
        return np.float32(0.0)
    sign = -1 if x < 0 else 1
    a = abs(x)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    # a in [2^e, 2^(e+1)): 24 significant bits
    scaled = a / Fraction(2) ** (e - 23)
    m = scaled.numerator // scaled.denominator
    rem = scaled - m
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and m % 2 == 1):
        m += 1
    return np.float32(sign * m * 2.0 ** (e - 23))


def _quotient(acc: np.float32, lsum: np.float32) -> np.float32:
    inv = np.float32(np.float32(1.0) / lsum)
    q0 = np.float32(acc * inv)
    r = _rn32(Fraction(float(acc)) - Fraction(float(q0)) * Fraction(float(lsum)))
    return _rn32(Fraction(float(r)) * Fraction(float(inv)) + Fraction(float(q0)))


def _rand_f32(rng, n, lo, hi):
    m = rng.integers(0, 1 << 23, n, dtype=np.uint32)
    e = rng.integers(lo, hi + 1, n).astype(np.uint32) + 127
    s = rng.integers(0, 2, n, dtype=np.uint32) << 31
    return ((e << 23) | m | s).view(np.float32)


def test_reciprocal_plus_residual_is_the_correctly_rounded_quotient():
    rng = np.random.default_rng(20261202)
    n = 20000
    lsum = np.abs(_rand_f32(rng, n, -10, 40))
    acc = _rand_f32(rng, n, -60, 60)
    # powers of two and one ulp either side, where 1/l is exact or nearly so
    pw = np.float32(2.0) ** np.arange(-10, 40, dtype=np.float32)
    ulp = np.nextafter(pw, np.float32(np.inf))
    lsum = np.concatenate([lsum, pw, ulp, np.nextafter(pw, np.float32(0))]).astype(np.float32)
    acc = np.concatenate([acc, _rand_f32(rng, 3 * len(pw), -60, 60)]).astype(np.float32)
    for a, l in zip(acc, lsum):
        want = np.float32(a / l)
        got = _quotient(a, l)
        assert got.view(np.uint32) == want.view(np.uint32), (a, l, got, want)


def test_the_plain_product_is_not_always_correctly_rounded():
    """Without the residual step, acc * (1/l) misses the correctly rounded
    quotient for a visible share of pairs: the step is needed."""
    rng = np.random.default_rng(7)
    n = 1 << 20
    lsum = np.abs(_rand_f32(rng, n, -10, 40))
    acc = _rand_f32(rng, n, -60, 60)
    inv = (np.float32(1.0) / lsum).astype(np.float32)
    q0 = (acc * inv).astype(np.float32)
    want = (acc / lsum).astype(np.float32)
    assert (q0.view(np.uint32) != want.view(np.uint32)).mean() > 0.05


def test_exact_rounding_matches_fp32_arithmetic():
    """The emulation's rounding against numpy's correctly rounded fp32
    products and sums (whose exact values the rationals hold)."""
    rng = np.random.default_rng(11)
    a = _rand_f32(rng, 5000, -40, 40)
    b = _rand_f32(rng, 5000, -40, 40)
    for x, y in zip(a, b):
        assert _rn32(Fraction(float(x)) * Fraction(float(y))).view(np.uint32) == \
            np.float32(x * y).view(np.uint32)
        assert _rn32(Fraction(float(x)) + Fraction(float(y))).view(np.uint32) == \
            np.float32(x + y).view(np.uint32)
