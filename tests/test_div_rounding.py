"""The prefill epilogue's division: f16(f32(o / l)) from an f64 reciprocal.

The kernel writes out = f16(acc / max(l, 1e-8)) with the quotient rounded to
f32 first (the reference's true_div, src/kernels.rs:1289-1291).  It evaluates
the quotient as f32(o * r) in f64 with r = 1/l rounded to f64, which is the
same f32 for every f32 o and l > 0 (the product is within 2^-52 of o/l; an f32
quotient in the normal range lies more than 2^-49 from every f32 rounding
midpoint).  These CPU checks pin that claim on random and adversarial pairs
(quotients placed next to f32 and f16 rounding midpoints), and show that the
same pairs tell apart the two near-misses: one f64 -> f16 rounding (what the
code generator folds the two conversions into unless stopped) and an f32
reciprocal times o.
"""
import numpy as np


def _exact(a, b):
    return (a / b).astype(np.float16)  # f32 division (IEEE, correctly rounded), then f16


def _f64_recip(a, b):
    r = 1.0 / b.astype(np.float64)
    return (a.astype(np.float64) * r).astype(np.float32).astype(np.float16)


def _bits(x):
    return x.view(np.uint16)


def _pairs(rng, n):
    """(o, l) f32 pairs: plain random, near f32 midpoints, near f16 midpoints."""
    out = []
    # Plain: attention-like magnitudes and wide exponents.
    l = np.exp(rng.uniform(np.log(1e-8), np.log(1e7), n)).astype(np.float32)
    o = (rng.standard_normal(n) * l * np.exp(rng.uniform(-20, 3, n))).astype(np.float32)
    out.append((o, l))
    # Quotients next to an f32 rounding midpoint: o = f32(M * l).
    l = rng.uniform(1.0, 2.0, n).astype(np.float32) * np.float32(2.0) ** rng.integers(-20, 20, n)
    l = l.astype(np.float32)
    j = rng.integers(1 << 23, 1 << 24, n)
    e = rng.integers(-30, 10, n)
    mid = (2.0 * j + 1.0) * np.exp2(e - 24.0)
    o = (mid * l.astype(np.float64)).astype(np.float32)
    out.append((o * np.where(rng.random(n) < 0.5, -1, 1).astype(np.float32), l))
    # Quotients next to an f16 rounding midpoint, so that the f32 rounding can
    # land exactly on it (the case where one f64 -> f16 rounding differs).
    l = (rng.uniform(1.0, 2.0, n) * np.exp2(rng.integers(-10, 10, n))).astype(np.float32)
    k = rng.integers(1 << 10, 1 << 11, n)
    e = rng.integers(-14, 15, n)
    mid16 = (2.0 * k + 1.0) * np.exp2(e - 11.0)
    eps = rng.integers(-4, 5, n) * np.exp2(e - 35.0)  # a few f32 ulps around it
    o = ((mid16 + eps) * l.astype(np.float64)).astype(np.float32)
    out.append((o, l))
    return out


def test_f64_reciprocal_matches_true_division():
    rng = np.random.default_rng(20261202)
    for o, l in _pairs(rng, 400_000):
        np.testing.assert_array_equal(_bits(_f64_recip(o, l)), _bits(_exact(o, l)))
        # Stronger: the f32 quotients themselves agree wherever they are normal.
        q32 = o / l
        q64 = (o.astype(np.float64) * (1.0 / l.astype(np.float64))).astype(np.float32)
        normal = np.abs(q32) >= np.float32(2.0 ** -126)
        np.testing.assert_array_equal(q64[normal].view(np.uint32), q32[normal].view(np.uint32))


def test_special_values():
    o = np.array([0.0, -0.0, 1e-45, -1e-45, 65504.0, 70000.0, -70000.0, 1.0, 3.0],
                 dtype=np.float32)
    l = np.array([1e-8, 1e-8, 1e-8, 1e-8, 1.0, 1.0, 1.0, np.inf, 3.0], dtype=np.float32)
    with np.errstate(over="ignore"):  # 70000 is past f16 range: inf either way
        np.testing.assert_array_equal(_bits(_f64_recip(o, l)), _bits(_exact(o, l)))


def test_near_misses_are_caught():
    rng = np.random.default_rng(7)
    pairs = _pairs(rng, 400_000)
    # One f64 -> f16 rounding: differs on the f16-midpoint pairs.
    o, l = pairs[2]
    single = (o.astype(np.float64) * (1.0 / l.astype(np.float64))).astype(np.float16)
    assert np.any(_bits(single) != _bits(_exact(o, l)))
    # An f32 reciprocal times o: differs too.
    o, l = pairs[0]
    with np.errstate(over="ignore"):
        rcp32 = (o * (np.float32(1.0) / l)).astype(np.float16)
    assert np.any(_bits(rcp32) != _bits(_exact(o, l)))
