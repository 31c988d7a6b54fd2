"""CPU checks of the oracle's gradient-clipping restatements.

ora_clip_grad_norm / ora_clip_grad_value restate clip_grad_norm_ and
clip_grad_value_ (optimizers.asm:1370-1620).  The reference has no test or
vector for them, so they are pinned by what the mathematics fixes:
  - the pre-clip norm against sqrt(math.fsum(g*g)) (fp64-exact sum);
  - after a clip, the gradients' norm equals max_norm (float rounding aside);
  - the threshold is strict (norm == max_norm leaves the data untouched) and
    a NaN norm or a NaN max_norm clips nothing, bit for bit;
  - hand-derived cases: 3-4-5 triangles, a negative max_norm (scale -1), an
    infinite gradient (scale 0: finite values -> 0, infinities -> NaN), and
    the maxsd/minsd value clip (NaN -> lo, reversed bounds -> hi, -0 vs +0).
"""

import math

import numpy as np
import pytest

import ora


def _bits(a):
    a = np.asarray(a)
    return a.view(np.uint32 if a.dtype == np.float32 else np.uint64)


def test_norm_matches_exact_sum():
    rng = np.random.default_rng(21)
    g = [rng.normal(0, 1e-3, 100_003).astype(np.float32), None, rng.normal(0, 2.0, 4097),
         np.zeros(0, np.float32), rng.normal(0, 1, 7).astype(np.float32)]
    norm, out = ora.clip_grad_norm(g, 1e30)
    terms = []
    for a in g:
        if a is not None:
            d = a.astype(np.float64)
            terms.extend((d * d).tolist())
    exact = math.sqrt(math.fsum(terms))
    # sequential double sum of >= 0 terms: relative error <= n * 2^-53
    assert abs(norm - exact) <= len(terms) * 2.0 ** -53 * exact
    for a, b in zip(g, out):
        if a is not None:
            assert np.array_equal(_bits(a), _bits(b))  # below threshold: untouched


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_clipped_norm_equals_max_norm(dtype):
    rng = np.random.default_rng(22)
    g = [rng.normal(0, 1, 10_000).astype(dtype), rng.normal(0, 3, 333).astype(dtype)]
    norm0 = math.sqrt(math.fsum((a.astype(np.float64) ** 2).sum() for a in g))
    max_norm = 0.25 * norm0
    norm, out = ora.clip_grad_norm(g, max_norm)
    assert abs(norm - norm0) <= 1e-12 * norm0
    after = math.sqrt(math.fsum(math.fsum((a.astype(np.float64) ** 2).tolist()) for a in out))
    tol = 2e-7 if dtype == np.float32 else 1e-14
    assert abs(after - max_norm) <= tol * max_norm
    # every gradient scaled by one common factor
    ratios = np.concatenate([(b.astype(np.float64) / a.astype(np.float64))[a != 0] for a, b in zip(g, out)])
    assert np.max(np.abs(ratios / (max_norm / norm) - 1)) <= (1.2e-7 if dtype == np.float32 else 1e-15)


def test_threshold_is_strict_and_exact():
    g = [np.array([3.0, 4.0]), np.array([0.0], np.float32)]
    norm, out = ora.clip_grad_norm(g, 5.0)
    assert norm == 5.0
    assert out[0].tolist() == [3.0, 4.0]
    norm, out = ora.clip_grad_norm(g, 2.5)
    assert out[0].tolist() == [1.5, 2.0]
    norm, out = ora.clip_grad_norm([np.array([3.0, 4.0], np.float32)], 1.0)
    assert out[0].dtype == np.float32 and out[0].tolist() == [np.float32(3.0) * np.float32(0.2),
                                                             np.float32(4.0) * np.float32(0.2)]


def test_negative_max_norm_flips_sign():
    norm, out = ora.clip_grad_norm([np.array([3.0, -4.0])], -5.0)
    assert norm == 5.0 and out[0].tolist() == [-3.0, 4.0]


def test_nan_norm_and_nan_max_clip_nothing():
    g = np.array([1.0, np.nan, 100.0], np.float32)
    norm, out = ora.clip_grad_norm([g], 1.0)
    assert math.isnan(norm)
    assert np.array_equal(_bits(out[0]), _bits(g))
    h = np.array([30.0, 40.0])
    norm, out = ora.clip_grad_norm([h], float("nan"))
    assert norm == 50.0 and out[0].tolist() == [30.0, 40.0]


def test_infinite_gradient_scale_zero():
    g = np.array([1.0, -np.inf, -2.0, 0.0], np.float32)
    norm, out = ora.clip_grad_norm([g], 1.0)
    assert norm == math.inf
    got = out[0]
    assert got[0] == 0 and got[2] == 0 and math.copysign(1, got[2]) < 0 and np.isnan(got[1]) and got[3] == 0


def test_empty_and_none():
    norm, out = ora.clip_grad_norm([None, np.zeros(0)], 1.0)
    assert norm == 0.0
    norm, out = ora.clip_grad_norm([], 1.0)
    assert norm == 0.0


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_value_clip_hand_cases(dtype):
    g = np.array([-2.0, -0.5, 0.0, 0.5, 2.0, np.nan, np.inf, -np.inf], dtype)
    out = ora.clip_grad_value([g], -1.0, 1.0)[0]
    assert out.dtype == dtype
    assert out.tolist() == [-1.0, -0.5, 0.0, 0.5, 1.0, -1.0, 1.0, -1.0]
    # reversed bounds: max with lo first, then min with hi -> hi everywhere
    out = ora.clip_grad_value([g], 1.0, -1.0)[0]
    assert out.tolist() == [-1.0] * g.size
    # -0 against lo = +0: (-0 > +0) is false -> +0; against lo = -1: -0 kept
    z = np.array([-0.0], dtype)
    assert math.copysign(1, ora.clip_grad_value([z], 0.0, 1.0)[0][0]) > 0
    assert math.copysign(1, ora.clip_grad_value([z], -1.0, 1.0)[0][0]) < 0
    # NaN bound: each compare against NaN is false, so the bound is taken:
    # lo = NaN -> t = NaN -> (NaN < hi) false -> hi; hi = NaN -> NaN
    out = ora.clip_grad_value([np.array([0.5], dtype)], float("nan"), 1.0)[0]
    assert out[0] == 1.0
    out = ora.clip_grad_value([np.array([0.5], dtype)], -1.0, float("nan"))[0]
    assert np.isnan(out[0])


def test_value_clip_random_matches_clamp():
    rng = np.random.default_rng(23)
    g32 = rng.normal(0, 2, 5000).astype(np.float32)
    g64 = rng.normal(0, 2, 5000)
    o32, o64 = ora.clip_grad_value([g32, None, g64], -0.3, 0.7)[::2]
    # NaN-free data and lo < hi: the SSE rule is the ordinary clamp
    assert np.array_equal(o32, np.clip(g32, np.float32(-0.3), np.float32(0.7)))
    assert np.array_equal(o64, np.clip(g64, -0.3, 0.7))
