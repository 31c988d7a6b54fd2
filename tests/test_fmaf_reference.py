"""The tests' float32 fma reference (conftest.fmaf_exact) against exact
rational arithmetic: random triples over wide exponent ranges, and the triples
where (double)a*b + c rounded to float misses the correctly rounded result
(the exact sum just past a float tie), which fmaf_exact must get right."""

from fractions import Fraction

import numpy as np

from conftest import fmaf_exact


def _round_f32(x):
    """The float32 nearest the rational x, ties to even (finite range)."""
    f0 = np.float32(float(x))
    cands = {f0, np.nextafter(f0, np.float32(np.inf)), np.nextafter(f0, np.float32(-np.inf))}
    best = None
    for f in cands:
        if not np.isfinite(f):
            continue
        d = abs(Fraction(float(f)) - x)
        key = (d, int(np.array(f).view(np.uint32)) & 1)
        if best is None or key < best[0]:
            best = (key, f)
    return best[1]


def _exact(a, b, c):
    return _round_f32(Fraction(float(a)) * Fraction(float(b)) + Fraction(float(c)))


def test_random_triples_match_exact_rounding():
    rng = np.random.default_rng(77)
    n = 20000
    e = rng.integers(-60, 60, (3, n))
    a, b, c = (rng.uniform(-2, 2, n) * 2.0 ** e[i] for i in range(3))
    a, b, c = (v.astype(np.float32) for v in (a, b, c))
    got = fmaf_exact(a, b, c)
    for i in range(n):
        assert got[i] == _exact(a[i], b[i], c[i]), (i, a[i], b[i], c[i])


def test_double_rounding_cases():
    # a*b = 1 + 2^-11 + 2^-24 exactly: halfway between two floats; a c far
    # below double's ulp of 1 decides the direction, which the double sum loses
    u = np.float32(1 + 2.0 ** -12)
    cases = [(u, u, np.float32(2.0 ** -80)), (u, u, np.float32(-(2.0 ** -80))),
             (-u, u, np.float32(2.0 ** -80)), (-u, u, np.float32(-(2.0 ** -80))),
             (u, u, np.float32(0.0))]
    a, b, c = (np.array(v, dtype=np.float32) for v in zip(*cases))
    naive = (a.astype(np.float64) * b.astype(np.float64) + c.astype(np.float64)).astype(np.float32)
    got = fmaf_exact(a, b, c)
    want = np.array([_exact(*t) for t in cases], dtype=np.float32)
    assert np.array_equal(got, want)
    assert not np.array_equal(naive, want)  # the cases do separate the two
    assert got[0] > got[4] and got[1] == got[4]  # up past the tie; a tie alone goes to even


def test_specials():
    a = np.array([np.inf, 0.0, np.nan, 3e38, -0.0], dtype=np.float32)
    b = np.array([0.0, 5.0, 1.0, 10.0, 1.0], dtype=np.float32)
    c = np.array([1.0, -0.0, 1.0, 0.0, 0.0], dtype=np.float32)
    got = fmaf_exact(a, b, c)
    assert np.isnan(got[0]) and np.isnan(got[2])
    assert got[1] == 0.0 and not np.signbit(got[1])
    assert got[3] == np.inf
    assert got[4] == 0.0 and not np.signbit(got[4])  # -0 * 1 + +0 = +0
