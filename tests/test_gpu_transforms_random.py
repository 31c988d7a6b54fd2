"""Randomised per-feature transforms (transforms.c:26-143).

Seeded cases: 1-200,000 rows of 1-3000 features (log-uniform, at most 4 M
values), features with random offsets and scales (10^U(-3, 3)), NaN, +-Inf,
+-0 and constant columns planted in some cases, buffers at an 8-byte offset
(the element-at-a-time path) in some.  Statistics: min / max bit-exact
against the oracle, mean within 1e-12 * mean|x| and variance within
1e-12 * (mean(x^2) + mean^2), non-finite by class.  The three maps
(normalize, unnormalize, min-max) with random parameters, a zero scale in
some features and eps 1e-8 or 0 must equal the oracle bit for bit.
"""

import ctypes
import math

import numpy as np

from conftest import GPU, same_bits
from test_gpu_transforms import _gpu_stats, _lib

pytestmark = GPU

CASES = 30


def _case(rng):
    nf = int(np.exp(rng.uniform(0, np.log(3000))))
    b = int(np.exp(rng.uniform(0, np.log(200_000))))
    b = max(1, min(b, 4_000_000 // nf))
    x = rng.normal(rng.normal(0, 10, nf), 10.0 ** rng.uniform(-3, 3, nf), (b, nf))
    if rng.random() < 0.4:
        for _ in range(int(rng.integers(1, 5))):
            f = int(rng.integers(0, nf))
            kind = int(rng.integers(0, 4))
            if kind == 0:
                x[rng.integers(0, b, max(1, b // 10)), f] = np.nan
            elif kind == 1:
                x[int(rng.integers(0, b)), f] = rng.choice([np.inf, -np.inf])
            elif kind == 2:
                x[:, f] = rng.choice([0.0, -0.0], b)
            else:
                x[:, f] = rng.normal()
    if rng.random() < 0.3:  # an 8-byte offset from a 16-byte boundary
        buf = np.empty(x.size + 1)
        y = buf[1:].reshape(x.shape)
        y[...] = x
        return y
    return x


def test_random_stats_and_maps(pn, ora):
    rng = np.random.default_rng(606)
    for case in range(CASES):
        x = _case(rng)
        b, nf = x.shape
        mean, std, mn, mx = _gpu_stats(x)
        _, rmean, rstd, rmn, rmx = ora.transform_stats(x)
        same_bits(mn, rmn)
        same_bits(mx, rmx)
        with np.errstate(all="ignore"):
            amean = np.abs(x).mean(axis=0)
            sq = (x * x).mean(axis=0) + rmean * rmean
        for f in range(nf):
            if not math.isfinite(rmean[f]):
                assert (math.isnan(mean[f]) and math.isnan(rmean[f])) or mean[f] == rmean[f], (case, f)
                continue
            assert abs(mean[f] - rmean[f]) <= 1e-12 * amean[f] + 1e-300, (case, x.shape, f, mean[f], rmean[f])
            if math.isfinite(sq[f]):
                assert abs(std[f] ** 2 - rstd[f] ** 2) <= 1e-12 * sq[f] + 1e-300, (case, x.shape, f)
            else:
                assert (math.isnan(std[f]) and math.isnan(rstd[f])) or std[f] == rstd[f], (case, f)
        p0 = rng.normal(0, 5, nf)
        p1 = np.abs(rng.normal(1, 0.5, nf))
        p1[rng.integers(0, nf, max(1, nf // 20))] = 0.0
        eps = 1e-8 if rng.random() < 0.7 else 0.0
        fns = [_lib().transform_normalize, _lib().transform_unnormalize, _lib().transform_minmax]
        for mode, fn in enumerate(fns):
            out = np.full((b, nf), 7.0)
            rc = fn(x.ctypes.data, out.ctypes.data, b, nf, p0.ctypes.data, p1.ctypes.data, ctypes.c_double(eps))
            assert rc == 0, (case, mode, x.shape)
            same_bits(out.reshape(-1), ora.transform_apply(mode, np.ascontiguousarray(x), p0, p1, eps)[1].reshape(-1))
