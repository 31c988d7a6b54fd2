"""Randomised row and whole-tensor reductions.

Seeded shapes in both dtypes, rows 1-1000 and widths 1-100,000 (log-uniform,
at most 4 M values), which between them take every launch form (a wave per
row up to 2048 values, a block per row above it, segmented rows with a
combine launch for few long rows), with NaN, +-Inf, +-0 and repeated maxima
planted.  Row max and argmax and the whole-tensor max and argmax must equal
the oracle's restatement of the reference's running-max chain and argmax
rule (activations.asm:888-895, main.asm:3245-3292) bit for bit; the fused
row statistics must equal the separate calls bit for bit; sums and means
must sit within the REDUCE bound of the fp64-exact sum (1e-5 * sum|x|; an
infinite or NaN exact sum must be matched by class).
"""

import ctypes

import numpy as np
import pytest

from conftest import GPU, same_bits

pytestmark = GPU

CASES = 40


def _case(rng, dt):
    rows = int(rng.choice([1, 2, 3, 5, 17, 64, 300, 1000]))
    cols = int(np.exp(rng.uniform(0, np.log(100_000))))
    cols = max(1, min(cols, 4_000_000 // rows))
    x = rng.normal(0, 3, (rows, cols)).astype(dt)
    flat = x.reshape(-1)
    specials = np.array([np.nan, np.inf, -np.inf, 0.0, -0.0], dtype=dt)
    k = int(rng.integers(0, 4)) * max(1, flat.size // 1000)
    if k:
        flat[rng.integers(0, flat.size, k)] = rng.choice(specials, k)
    if cols > 2 and rng.random() < 0.3:
        r = int(rng.integers(0, rows))
        m = np.nanmax(np.where(np.isinf(x[r]), np.nan, x[r])) if np.any(np.isfinite(x[r])) else 1.0
        x[r, int(rng.integers(0, cols))] = m  # a repeated maximum: the first occurrence wins
    return x


def _exact_sums(ora, x):
    """fp64-exact row sums for finite rows (the oracle's compensated sum,
    defined for finite data); for a row holding non-finite values, the IEEE
    value of any order of additions: NaN with a NaN or both infinities, else
    the infinity."""
    e = ora.rowsum_exact(np.where(np.isfinite(x), x, 0).astype(x.dtype))
    has_nan = np.isnan(x).any(axis=1)
    pinf, ninf = (x == np.inf).any(axis=1), (x == -np.inf).any(axis=1)
    e = np.where(pinf, np.inf, e)
    e = np.where(ninf, -np.inf, e)
    return np.where(has_nan | (pinf & ninf), np.nan, e)


def _sum_ok(g, e, bound):
    fin = np.isfinite(e)
    assert np.all(np.abs(g[fin] - e[fin]) <= bound[fin]), np.max(np.abs(g[fin] - e[fin]) - bound[fin])
    same_bits(g[~fin], e[~fin])


@pytest.mark.parametrize("dt", [np.float32, np.float64])
def test_random_row_reductions(pn, ora, dt):
    lib = pn.core._lib
    rng = np.random.default_rng(99 if dt == np.float32 else 98)
    for case in range(CASES):
        x = _case(rng, dt)
        rows, cols = x.shape
        t = pn.Tensor.from_numpy(x)
        e = _exact_sums(ora, x)
        fx = np.abs(np.where(np.isfinite(x), x, 0).astype(np.float64))
        bound = 1e-5 * fx.sum(axis=1) + np.abs(np.where(np.isfinite(e), e, 0)) * 1e-7
        s, mn, mx = (pn.Tensor.create([rows], t.dtype) for _ in range(3))
        idx = np.empty(rows, dtype=np.int64)
        assert lib.neural_reduce_sum(t._ptr, 1, s._ptr) == 0, case
        assert lib.neural_reduce_mean(t._ptr, 1, mn._ptr) == 0, case
        assert lib.neural_reduce_max(t._ptr, 1, mx._ptr) == 0, case
        assert lib.neural_reduce_argmax(t._ptr, 1, idx.ctypes.data) == 0, case
        gs = s.numpy().astype(np.float64)
        _sum_ok(gs, e, bound)
        _sum_ok(mn.numpy().astype(np.float64), e / cols, bound / cols)
        same_bits(mx.numpy(), ora.rowmax_chain(x))
        same_bits(idx, ora.rowargmax(x))
        # the fused statistics: the separate calls' bits
        s2, mn2, mx2 = (pn.Tensor.create([rows], t.dtype) for _ in range(3))
        idx2 = np.empty(rows, dtype=np.int64)
        assert lib.neural_row_stats(t._ptr, s2._ptr, mn2._ptr, mx2._ptr, idx2.ctypes.data) == 0, case
        same_bits(s2.numpy(), s.numpy())
        same_bits(mn2.numpy(), mn.numpy())
        same_bits(mx2.numpy(), mx.numpy())
        same_bits(idx2, idx)


@pytest.mark.parametrize("dt", [np.float32, np.float64])
def test_random_whole_tensor_reductions(pn, ora, dt):
    lib = pn.core._lib
    rng = np.random.default_rng(77 if dt == np.float32 else 76)
    for case in range(CASES):
        n = int(np.exp(rng.uniform(0, np.log(4_000_000))))
        x = _case(rng, dt).reshape(-1)[:n] if rng.random() < 0.5 else rng.normal(0, 1, n).astype(dt)
        n = x.size
        t = pn.Tensor.from_numpy(np.ascontiguousarray(x))
        r = ctypes.c_double()
        i = ctypes.c_int64()
        assert lib.neural_sum(t._ptr, ctypes.byref(r)) == 0, case
        e = _exact_sums(ora, x.reshape(1, -1))
        bound = 1e-5 * np.abs(np.where(np.isfinite(x), x, 0).astype(np.float64)).sum() + \
            (abs(e[0]) * 1e-7 if np.isfinite(e[0]) else 0.0)
        _sum_ok(np.array([r.value]), e, np.array([bound]))
        assert lib.neural_max(t._ptr, ctypes.byref(r)) == 0, case
        same_bits(np.array([r.value], dtype=np.float64), ora.rowmax_chain(x.reshape(1, -1)).astype(np.float64))
        assert lib.neural_argmax(t._ptr, ctypes.byref(i)) == 0, case
        assert i.value == int(ora.rowargmax(x.reshape(1, -1))[0]), (case, n)
