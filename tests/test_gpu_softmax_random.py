"""Randomised softmax and log-softmax rows.

Seeded shapes in both dtypes, 1-300 rows of 1-6000 values (log-uniform: the
one-wave-per-row kernels up to 4096 f32 / 2048 f64 values and 16-byte rows,
the block-per-row kernel beyond them and for other widths), N(0, 3) logits
with -Inf entries, and rows holding +Inf, NaN or only -Inf planted.  Expected
values: the reference's formula (activations.asm:761-987 intended, f64 path;
metrics_losses.c:47-64 for log-softmax) evaluated in float64 -- m = row max,
e = exp(x - m), y = e / sum e, log y = (x - m) - log(sum e) -- so a NaN or
+Inf anywhere, or a row of only -Inf, makes the row NaN, and a -Inf logit
gives 0 (softmax) or -Inf (log-softmax).  Non-finite results must match by
class; finite ones within REL32 (1e-5 relative, log-softmax + 1e-6 absolute)
for f32 and REL64 (1e-12 relative + 1e-15) for f64.
"""

import numpy as np
import pytest

from conftest import GPU, same_bits

pytestmark = GPU

CASES = 40


def _case(rng, dt):
    rows = int(rng.integers(1, 301))
    cols = int(np.exp(rng.uniform(0, np.log(6000))))
    x = rng.normal(0, 3, (rows, cols)).astype(dt)
    for _ in range(int(rng.integers(0, 4))):
        r = int(rng.integers(0, rows))
        kind = int(rng.integers(0, 4))
        if kind == 0:
            x[r, rng.integers(0, cols, max(1, cols // 4))] = -np.inf
        elif kind == 1:
            x[r, int(rng.integers(0, cols))] = np.inf
        elif kind == 2:
            x[r, int(rng.integers(0, cols))] = np.nan
        else:
            x[r, :] = -np.inf
    return x


def _expected(x):
    xd = x.astype(np.float64)
    with np.errstate(all="ignore"):
        m = np.max(xd, axis=1, keepdims=True)  # NaN if the row holds one
        d = xd - m
        e = np.exp(d)
        s = np.sum(e, axis=1, keepdims=True)
        return e / s, d - np.log(s)


@pytest.mark.parametrize("dt", [np.float32, np.float64])
def test_random_softmax_rows(pn, dt):
    lib = pn.core._lib
    rng = np.random.default_rng(55 if dt == np.float32 else 54)
    rel, floor = (1e-5, 1e-6) if dt == np.float32 else (1e-12, 1e-15)
    for case in range(CASES):
        x = _case(rng, dt)
        t = pn.Tensor.from_numpy(x)
        p, lp = pn.Tensor.create(list(x.shape), t.dtype), pn.Tensor.create(list(x.shape), t.dtype)
        assert lib.neural_softmax(p._ptr, t._ptr) == 0, case
        assert lib.neural_log_softmax(lp._ptr, t._ptr) == 0, case
        want, lwant = _expected(x)
        for got, w, fl in ((p.numpy().astype(np.float64), want, 0.0), (lp.numpy().astype(np.float64), lwant, floor)):
            fin = np.isfinite(w)
            same_bits(got[~fin], w[~fin])
            err = np.abs(got[fin] - w[fin]) - (rel * np.abs(w[fin]) + fl)
            assert np.all(err <= 0), (case, x.shape, float(err.max()))
