"""Pins the oracle's fp16 conversion (tensor.cpp:276-344) and checks the product's host-side
restatement against it.

Pins: exhaustive IEEE widening (numpy); agreement with round-to-nearest-even away from ties;
the half-away-from-zero tie rule from an exact rational rounding written independently of the
bit manipulation; the reference test's rounding-boundary literals (tests/golden)."""

import json
import os
from fractions import Fraction

import numpy as np

from mtorch_amd import _random

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def _all_halves():
    return np.arange(65536, dtype=np.uint32).astype(np.uint16)


def test_h2f_exhaustive_matches_ieee(orc):
    h = _all_halves()
    got = orc.h2f(h)
    ref = h.view(np.float16).astype(np.float32)
    finite = ~np.isnan(ref)
    assert np.array_equal(got[finite].view(np.uint32), ref[finite].view(np.uint32))
    # NaNs keep sign and payload: sign | 0x7f800000 | mantissa << 13
    nan_bits = ((h[~finite].astype(np.uint32) & 0x8000) << 16) | 0x7F800000 | ((h[~finite].astype(np.uint32) & 0x3FF) << 13)
    assert np.array_equal(got[~finite].view(np.uint32), nan_bits)


def test_f2h_round_trips_every_half(orc):
    h = _all_halves()
    f = orc.h2f(h)
    finite = ~np.isnan(f)
    assert np.array_equal(orc.f2h(f)[finite], h[finite])


def _round_half_away_exact(x: float) -> float:
    """binary16 rounding of x with ties away from zero, by exact rational arithmetic."""
    if x != x or x in (float("inf"), float("-inf")):
        return x
    sign = -1.0 if x < 0 or (x == 0 and str(x).startswith("-")) else 1.0
    a = Fraction(abs(x))
    if a == 0:
        return sign * 0.0
    e = a.numerator.bit_length() - a.denominator.bit_length()
    while Fraction(2) ** e > a:
        e -= 1
    while Fraction(2) ** (e + 1) <= a:
        e += 1
    e = max(e, -14)  # subnormal binade shares the 2^-24 spacing
    ulp = Fraction(2) ** (e - 10)
    q, r = divmod(a, ulp)
    if r * 2 >= ulp:
        q += 1
    v = q * ulp
    if v >= 65520:  # beyond the largest finite half after rounding -> inf
        return sign * float("inf")
    return sign * float(v)


def test_f2h_ties_round_away_from_zero(orc):
    h = _all_halves()
    f = orc.h2f(h)
    pos = f[(f >= 0) & np.isfinite(f)]
    pos = np.sort(pos)
    mids = ((pos[:-1].astype(np.float64) + pos[1:].astype(np.float64)) / 2).astype(np.float32)
    mids = np.concatenate([mids, -mids])
    got = orc.h2f(orc.f2h(mids))
    expect = np.array([_round_half_away_exact(float(m)) for m in mids], dtype=np.float32)
    assert np.array_equal(got, expect)
    # and they differ from round-to-nearest-even on half of the ties
    rne = mids.astype(np.float16).astype(np.float32)
    assert np.count_nonzero(rne != got) > 1000


def test_f2h_matches_exact_rounding_on_random_values(orc):
    rng = np.random.default_rng(7)
    bits = rng.integers(0, 2**32, size=20000, dtype=np.uint64).astype(np.uint32)
    vals = bits.view(np.float32)
    vals = vals[np.isfinite(vals)]
    # concentrate on the half range, including subnormals and the flush boundary
    scaled = (rng.standard_normal(20000) * np.exp2(rng.uniform(-27, 17, 20000))).astype(np.float32)
    sample = np.concatenate([vals[:5000], scaled, np.float32([2.0**-25, -(2.0**-25), 2.0**-26, 65504, 65519.99, 65520])])
    got = orc.h2f(orc.f2h(sample))
    expect = np.array([_round_half_away_exact(float(v)) for v in sample], dtype=np.float32)
    assert np.array_equal(got.view(np.uint32), expect.view(np.uint32))


def test_f2h_specials(orc):
    assert orc.f2h(np.float32([np.inf]))[0] == 0x7C00
    assert orc.f2h(np.float32([-np.inf]))[0] == 0xFC00
    assert orc.f2h(np.float32([1e6]))[0] == 0x7C00
    assert orc.f2h(np.float32([-0.0]))[0] == 0x8000
    nan = np.array([0x7FC00000, 0x7F800001, 0xFFC12345], dtype=np.uint32).view(np.float32)
    out = orc.f2h(nan)
    assert all((o & 0x7C00) == 0x7C00 and (o & 0x3FF) != 0 for o in out)
    assert out[1] == 0x7E00  # payload lost in the shift -> canonical 0x200 quiet bit


def test_reference_rounding_boundary_literals(orc):
    """tests/compat/test_tensor_ops.py:1308-1320 of the reference."""
    with open(os.path.join(GOLDEN, "fp16_rounding_boundaries.json")) as fh:
        case = json.load(fh)
    got = orc.h2f(orc.f2h(np.float32(case["input"]))).tolist()
    assert got == case["expected"]


def test_product_host_conversion_matches_oracle(orc):
    rng = np.random.default_rng(11)
    bits = rng.integers(0, 2**32, size=200000, dtype=np.uint64).astype(np.uint32)
    vals = np.concatenate([bits.view(np.float32), (rng.standard_normal(100000) * 1e-5).astype(np.float32)])
    assert np.array_equal(_random.float_to_half_bits(vals), orc.f2h(vals))
    h = _all_halves()
    assert np.array_equal(_random.half_bits_to_float(h).view(np.uint32), orc.h2f(h).view(np.uint32))
