"""Randomised gradient clipping (optimizers.asm:1370-1620).

Seeded lists of 1-40 gradients (None entries and empty tensors included),
each of 1 to 500,000 values (log-uniform) in float32 or float64 with a
per-tensor scale 10^U(-4, 2), NaN or +-Inf planted in some lists.  Norm
clip with max_norm at a random fraction (1e-3 to 10) of the exact norm,
held to the fixed-shape tests' bounds (pre-clip norm within 1e-12 of the
fp64-exact norm; clipped float32 bit-exact when both sides' float scale
agrees, float64 within 1e-12 relative).  Value clip with a random interval
(an inverted one or a NaN bound in some cases) bit-exact.
"""

import math

import numpy as np

from conftest import GPU, same_bits
from test_gpu_clip import _check_norm_clip, _exact_norm, _tensors

pytestmark = GPU

CASES = 30


def _arrays(rng, specials):
    out = []
    for _ in range(int(rng.integers(1, 41))):
        u = rng.random()
        if u < 0.05:
            out.append(None)
            continue
        dt = np.float32 if rng.random() < 0.5 else np.float64
        n = 0 if u < 0.08 else int(np.exp(rng.uniform(0, np.log(500_000))))
        out.append(rng.normal(0, 10.0 ** rng.uniform(-4, 2), n).astype(dt))
    if specials and rng.random() < 0.3:
        full = [a for a in out if a is not None and a.size]
        if full:
            a = full[int(rng.integers(0, len(full)))]
            a[int(rng.integers(0, a.size))] = rng.choice([np.nan, np.inf, -np.inf])
    return out


def test_random_norm_clip(pn, ora):
    rng = np.random.default_rng(717)
    for case in range(CASES):
        arrays = _arrays(rng, True)
        exact = _exact_norm(arrays)
        max_norm = exact * 10.0 ** rng.uniform(-3, 1) if math.isfinite(exact) and exact > 0 else 1.0
        _check_norm_clip(pn, ora, arrays, max_norm)


def test_random_value_clip(pn, ora):
    rng = np.random.default_rng(718)
    for case in range(CASES):
        arrays = _arrays(rng, True)
        lo, hi = sorted(rng.normal(0, 0.5, 2))
        u = rng.random()
        if u < 0.1:
            lo, hi = hi, lo
        elif u < 0.15:
            hi = float("nan")
        elif u < 0.2:
            lo = float("nan")
        ts = _tensors(pn, arrays)
        pn.clip_grad_value(ts, lo, hi)
        for t, w in zip(ts, ora.clip_grad_value(arrays, lo, hi)):
            if t is not None:
                same_bits(t.numpy(), w)
