"""The sampler kernel's fp64 exp for d <= 0 (common.cuh: exp_nonpos), restated step by step in
exact rational arithmetic with one rounding per fp64 operation, against exp to 60 digits: the
method must stay within one ulp, and be exact at 0."""

from __future__ import annotations

import math
from decimal import Decimal, getcontext
from fractions import Fraction

import numpy as np
import pytest

getcontext().prec = 60

TAB = [float.fromhex(h) for h in (
    "0x1.0000000000000p+0", "0x1.0b5586cf9890fp+0", "0x1.172b83c7d517bp+0", "0x1.2387a6e756238p+0",
    "0x1.306fe0a31b715p+0", "0x1.3dea64c123422p+0", "0x1.4bfdad5362a27p+0", "0x1.5ab07dd485429p+0",
    "0x1.6a09e667f3bcdp+0", "0x1.7a11473eb0187p+0", "0x1.8ace5422aa0dbp+0", "0x1.9c49182a3f090p+0",
    "0x1.ae89f995ad3adp+0", "0x1.c199bdd85529cp+0", "0x1.d5818dcfba487p+0", "0x1.ea4afa2a490dap+0",
)]
SIXTEEN_OVER_LN2 = float.fromhex("0x1.71547652b82fep+4")
HI = float.fromhex("0x1.62e42fefa0000p-5")
LO = float.fromhex("0x1.cf79abc9e3b3ap-44")


def fma(a: float, b: float, c: float) -> float:
    return float(Fraction(a) * Fraction(b) + Fraction(c))  # one rounding (to nearest even)


def exp_nonpos(d: float) -> float:
    if not d >= -745.5:
        return 0.0
    kd = float(np.rint(d * SIXTEEN_OVER_LN2))
    r = fma(-kd, HI, d)
    r = fma(-kd, LO, r)
    q = fma(r, 1.0 / 5040.0, 1.0 / 720.0)
    q = fma(r, q, 1.0 / 120.0)
    q = fma(r, q, 1.0 / 24.0)
    q = fma(r, q, 1.0 / 6.0)
    q = fma(r, q, 0.5)
    em1 = fma(r * r, q, r)
    k = int(kd)
    t = TAB[k & 15]
    return math.ldexp(fma(t, em1, t), k >> 4)


def test_table_is_correctly_rounded():
    ln2 = Decimal(2).ln()
    for j, t in enumerate(TAB):
        assert t == float((Decimal(j) / 16 * ln2).exp()), j
    assert HI + LO == float(ln2 / 16) and HI.hex().endswith("0000p-5")


def test_exact_at_zero_and_zero_below_the_range():
    assert exp_nonpos(0.0) == 1.0 and exp_nonpos(-0.0) == 1.0
    assert exp_nonpos(-800.0) == 0.0 and exp_nonpos(-math.inf) == 0.0 and exp_nonpos(math.nan) == 0.0


@pytest.mark.parametrize("lo,hi", [(-1e-3, 0.0), (-3.0, 0.0), (-40.0, -3.0), (-700.0, -40.0)])
def test_within_one_ulp(lo, hi):
    rng = np.random.default_rng(int(-lo * 1000))
    for d in np.concatenate([rng.uniform(lo, hi, 400), [lo, hi]]):
        d = float(d)
        got = exp_nonpos(d)
        ref = Decimal(d).exp()
        ulp = math.ulp(float(ref))
        assert abs(Decimal(got) - ref) <= Decimal(ulp), (d, got, float(ref))


def test_fixed_point_mass_is_rint():
    import struct

    rng = np.random.default_rng(5)
    for p in np.concatenate([rng.random(2000), [0.0, 1.0, 0.5 / 2**42, 1.5 / 2**42, 2.5 / 2**42]]):
        b = fma(float(p), 2.0**42, 2.0**52)
        q = struct.unpack("<Q", struct.pack("<d", b))[0] - 0x4330000000000000
        assert q == int(np.rint(float(p) * 2.0**42)), p
