"""Randomised optimizer runs (optimizers_c.c:218-562).

Seeded cases: AdamW, Adam or SGD with random hyperparameters (lr
10^U(-5, -1), beta1 U(0.5, 0.99), beta2 U(0.9, 0.99999), eps 10^U(-12, -6),
weight decay U(0, 0.1), momentum U(0, 0.99) or 0), 1-6 parameter tensors of
1 to 300,000 values (log-uniform) in float32 and float64 mixed in one list,
2-6 steps with a fresh gradient each step (NaN / +-Inf planted in some) and
the learning rate changed between steps in some cases.  In half of the cases
the OPTS state blob is exported after a middle step and imported into a new
optimizer of the same kind, which takes the remaining steps.  Parameters and
the float64 moment buffers must equal the oracle's bit for bit.
"""

import numpy as np
import pytest

from conftest import GPU, same_bits
from test_gpu_optim import _blob_moments

pytestmark = GPU

CASES = 24


def _make(pn, kind, h):
    if kind == "adamw":
        return pn.AdamW(h["lr"], h["b1"], h["b2"], h["eps"], h["wd"])
    if kind == "adam":
        return pn.Adam(h["lr"], h["b1"], h["b2"], h["eps"])
    return pn.SGD(h["lr"], h["mom"])


def _grad(rng, n, dt):
    g = rng.normal(0, 10.0 ** rng.uniform(-5, 0), n).astype(dt)
    if n > 10 and rng.random() < 0.3:
        g[rng.integers(0, n, 3)] = rng.choice(np.array([np.nan, np.inf, -np.inf], dtype=dt), 3)
    return g


def test_random_optimizer_runs(pn, ora):
    rng = np.random.default_rng(3141)
    for case in range(CASES):
        kind = ["adamw", "adam", "sgd"][case % 3]
        h = {"lr": 10.0 ** rng.uniform(-5, -1), "b1": rng.uniform(0.5, 0.99), "b2": rng.uniform(0.9, 0.99999),
             "eps": 10.0 ** rng.uniform(-12, -6), "wd": rng.uniform(0, 0.1),
             "mom": 0.0 if rng.random() < 0.25 else rng.uniform(0, 0.99)}
        sizes = [int(np.exp(rng.uniform(0, np.log(300_000)))) for _ in range(int(rng.integers(1, 7)))]
        dts = [np.float32 if rng.random() < 0.5 else np.float64 for _ in sizes]
        params = [rng.normal(0, 0.02, n).astype(dt) for n, dt in zip(sizes, dts)]
        tps = [pn.Tensor.from_numpy(p) for p in params]
        ref = [p.copy() for p in params]
        m = [np.zeros(n) for n in sizes]
        v = [np.zeros(n) for n in sizes]
        steps = int(rng.integers(2, 7))
        swap_at = int(rng.integers(1, steps)) if rng.random() < 0.5 else None
        opt = _make(pn, kind, h)
        lr = h["lr"]
        for t in range(1, steps + 1):
            if t > 1 and rng.random() < 0.3:
                lr = 10.0 ** rng.uniform(-5, -1)
                opt.lr = lr
                assert opt.lr == lr
            grads = [_grad(rng, n, dt) for n, dt in zip(sizes, dts)]
            opt.step(tps, [pn.Tensor.from_numpy(g) for g in grads])
            for i, g in enumerate(grads):
                if kind == "adamw":
                    ora.adamw_step(ref[i], g, m[i], v[i], lr, h["b1"], h["b2"], h["eps"], h["wd"], t)
                elif kind == "adam":
                    ora.adam_step(ref[i], g, m[i], v[i], lr, h["b1"], h["b2"], h["eps"], t)
                else:
                    ora.sgd_step(ref[i], g, m[i], lr, h["mom"])
            if t == swap_at:
                blob = opt.state_bytes()
                opt = _make(pn, kind, h)
                opt.load_state_bytes(blob)
                opt.lr = lr
        for tp, r in zip(tps, ref):
            same_bits(tp.numpy(), r)
        got = _blob_moments(opt.state_bytes(), sizes, 1 if kind == "sgd" else 2)
        want = m if kind == "sgd" else m + v
        for gm, wm in zip(got, want):
            same_bits(gm, wm)
