"""The one-reciprocal division the norm kernels use (`div_by` in
crane_amd/csrc/common.h): with r = RN(1/d), q0 = RN(x r), e = RN(x - q0 d)
and q = RN(q0 + e r) (two FMAs), q is the correctly rounded f32 quotient
RN(x / d) for finite nonzero d and no over- or underflow (Markstein's
theorem).  Checked here with exact rational arithmetic
against IEEE float32 division on random bf16 inputs over the kernels' range
(|d| in [2^-20, 2^20], norms of bf16 rows) and on random f32 pairs; a planted
variant without the correction step is caught."""
from fractions import Fraction

import numpy as np

import cases


def _rn32(fr: Fraction) -> np.float32:
    """Round an exact rational to the nearest float32, ties to even."""
    a = np.float32(float(fr))
    best = None
    for c in (np.nextafter(a, np.float32(-np.inf)), a, np.nextafter(a, np.float32(np.inf))):
        d = abs(Fraction(float(c)) - fr)
        if best is None or d < best[0] or (d == best[0] and (int(np.float32(c).view(np.uint32)) & 1) == 0):
            best = (d, c)
    return np.float32(best[1])


def _div_by(x: np.float32, d: np.float32, correct: bool = True) -> np.float32:
    r = np.float32(1) / d
    q0 = np.float32(x * r)
    if not correct:
        return q0
    e_exact = Fraction(float(x)) - Fraction(float(q0)) * Fraction(float(d))
    e = _rn32(e_exact)
    # (the FMA rounds the remainder once; it is exact when q0 is within an ulp of x / d)
    return _rn32(Fraction(float(q0)) + Fraction(float(e)) * Fraction(float(r)))


def _pairs(seed, n, bf16):
    r = np.random.Generator(np.random.PCG64(seed))
    x = r.standard_normal(n).astype(np.float32) * np.exp2(r.integers(-20, 21, n)).astype(np.float32)
    d = np.exp2(r.uniform(-20, 20, n)).astype(np.float32)
    if bf16:
        x, d = cases.bf16(x), cases.bf16(d)
    return x, d


def test_div_by_is_ieee_division():
    for seed, bf16 in ((1, True), (2, False)):
        x, d = _pairs(seed, 10000, bf16)
        for xi, di in zip(x, d):
            assert _div_by(xi, di) == xi / di, (xi, di)


def test_uncorrected_product_differs():
    x, d = _pairs(3, 3000, False)
    assert sum(_div_by(xi, di, correct=False) != xi / di for xi, di in zip(x, d)) > 100
