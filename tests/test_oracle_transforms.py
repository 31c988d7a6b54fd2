"""CPU checks of the per-feature transform oracle (transforms.c:27-143).

ora_transform_stats / ora_transform_apply restate the reference's
transforms.c; the reference's own file is compiled unchanged into
oracle/_ref, and the two must agree bit for bit, including NaN, +-Inf, +-0
(the first of equal values stays the min / max), values beyond +-1e308 (the
start values win), constant features (variance clamped at 0), and the -1
argument checks.  Closed forms pin what the reference build cannot: numpy's
fp64 mean / population std within rounding, and normalize -> unnormalize
round trips.
"""

import math

import numpy as np
import pytest

import ora


def _ref_or_skip():
    if ora.ref() is None:
        pytest.skip("reference C build (oracle/_ref) absent")


def _cases():
    rng = np.random.default_rng(3)
    out = [rng.normal(0, 3, (1000, 7)), rng.normal(5, 0.1, (33, 64)), np.ones((5, 3)) * 2.5,
           rng.normal(0, 1, (1, 9))]
    x = rng.normal(0, 1, (64, 12))
    x[3, 0] = np.nan
    x[:, 1] = np.nan
    x[5, 2], x[9, 2] = np.inf, -np.inf
    x[:, 3] = 0.0
    x[4, 3] = -0.0
    x[:, 4] = -0.0
    x[7, 4] = 0.0
    x[:, 5] = np.inf
    x[:, 6] = 1e308
    x[2, 7] = 1.5e308
    x[:, 8] = -np.inf
    out.append(x)
    return out


def test_stats_bit_exact_vs_reference():
    _ref_or_skip()
    for x in _cases():
        got = ora.transform_stats(x)
        want = ora.transform_stats(x, use_ref=True)
        assert got[0] == want[0] == 0
        for g, w in zip(got[1:], want[1:]):
            assert np.array_equal(g.view(np.uint64)[~np.isnan(g)], w.view(np.uint64)[~np.isnan(w)])
            assert np.array_equal(np.isnan(g), np.isnan(w))


@pytest.mark.parametrize("mode", [0, 1, 2])
def test_apply_bit_exact_vs_reference(mode):
    _ref_or_skip()
    rng = np.random.default_rng(mode)
    for x in _cases():
        nf = x.shape[1]
        p0 = rng.normal(0, 1, nf)
        p1 = np.abs(rng.normal(1, 0.5, nf))
        p1[0] = 0.0
        for eps in [1e-8, 0.0]:
            got = ora.transform_apply(mode, x, p0, p1, eps)
            want = ora.transform_apply(mode, x, p0, p1, eps, use_ref=True)
            assert got[0] == want[0] == 0
            g, w = got[1], want[1]
            assert np.array_equal(np.isnan(g), np.isnan(w))
            m = ~np.isnan(g)
            assert np.array_equal(g.view(np.uint64)[m], w.view(np.uint64)[m])


def test_argument_checks():
    assert ora.transform_stats(np.ones((0, 3)))[0] == -1
    assert ora.transform_apply(0, np.ones((0, 3)), np.ones(3), np.ones(3), 1e-8)[0] == -1


def test_closed_forms():
    rng = np.random.default_rng(8)
    x = rng.normal(2, 3, (5000, 6))
    rc, mean, std, mn, mx = ora.transform_stats(x)
    assert rc == 0
    assert np.allclose(mean, x.mean(axis=0), rtol=1e-13, atol=1e-13)
    assert np.allclose(std, x.std(axis=0), rtol=1e-10)
    assert np.array_equal(mn, x.min(axis=0)) and np.array_equal(mx, x.max(axis=0))
    # first of equal zeros stays
    z = np.array([[0.0], [-0.0]])
    _, _, _, zmn, zmx = ora.transform_stats(z)
    assert math.copysign(1, zmn[0]) > 0 and math.copysign(1, zmx[0]) > 0
    _, _, _, zmn, _ = ora.transform_stats(z[::-1].copy())
    assert math.copysign(1, zmn[0]) < 0
    # start values: +inf column reports min 1e308, -inf column max -1e308
    _, _, _, imn, imx = ora.transform_stats(np.full((3, 1), np.inf))
    assert imn[0] == 1e308 and imx[0] == np.inf
    # constant column: var clamps at 0 (sum2/b - m*m may round negative)
    _, _, s, _, _ = ora.transform_stats(np.full((7, 1), 0.1))
    assert s[0] == 0.0 or s[0] < 1e-8
    # round trip
    _, y = ora.transform_apply(0, x, mean, std, 1e-8)
    _, back = ora.transform_apply(1, y, mean, std, 1e-8)
    assert np.allclose(back, x, rtol=1e-14, atol=1e-13)
    _, mm = ora.transform_apply(2, x, mn, mx, 1e-8)
    assert mm.min() >= 0.0 and mm.max() <= 1.0
