"""Randomised activations over shapes and strided views
(activations_c.c:124-158, activations.asm:352-413).

Seeded cases in both dtypes: each activation on a 1-4 dimensional tensor of
1 to 300,000 values, input and output contiguous, permuted (a transposed
copy viewed back) or stepped (every other element of a wider tensor), with
alpha U(0, 3) for leaky_relu and elu; values N(0, 4) with +-30, +-0, NaN,
+-Inf and subnormals planted.  Expected: the oracle on the contiguous
values.  Piecewise-linear activations bit-exact; the others by the
fixed-shape tests' bounds (REL32: 1e-5 relative for float32; REL64: 1e-12
relative + 1e-15 absolute for float64), NaN / Inf by class; stepped outputs
must leave the elements between them untouched.
"""

import numpy as np

from conftest import GPU, keep, rel_close, same_bits
from test_gpu_activations import ACTS, ALPHA, EXACT
from test_gpu_broadcast_random import _view

pytestmark = GPU

CASES = 44


def _shape(rng):
    n = int(np.exp(rng.uniform(0, np.log(300_000))))
    nd = int(rng.integers(1, 5))
    dims = [1] * nd
    for i in range(nd - 1):
        dims[i] = int(rng.integers(1, max(2, int(round(n ** (1.0 / (nd - i))))) + 1))
        n = max(1, n // dims[i])
    dims[-1] = n
    return tuple(int(v) for v in rng.permutation(dims))


def _values(rng, shape, dt):
    x = rng.normal(0, 4, shape)
    flat = x.reshape(-1)
    k = max(1, flat.size // 50)
    specials = np.array([30.0, -30.0, 0.0, -0.0, np.nan, np.inf, -np.inf, 1e-310, -1e-310, 1e-40, -1e-40])
    flat[rng.integers(0, flat.size, k)] = rng.choice(specials, k)
    return x.astype(dt)


def _run(pn, lib, name, to, ti, alpha):
    import ctypes
    o, i = keep(pn.Tensor.from_torch(to)), keep(pn.Tensor.from_torch(ti))
    if name == "sigmoid":
        return lib.neural_sigmoid(o, i)
    if name in ALPHA:
        return getattr(lib, "act_" + name)(o, i, ctypes.c_double(alpha))
    return getattr(lib, "act_" + name)(o, i)


def test_random_activations(pn, ora):
    import torch
    lib = pn.core._lib
    rng = np.random.default_rng(8080)
    for case in range(CASES):
        dt = np.float32 if case % 2 == 0 else np.float64
        name = ACTS[(case // 2) % len(ACTS)]
        alpha = float(rng.uniform(0, 3))
        shape = _shape(rng)
        x = _values(rng, shape, dt)
        want = ora.act(name, np.ascontiguousarray(x).reshape(-1), alpha if name in ALPHA else 0.0).reshape(shape)
        ti, _ = _view(torch, x, int(rng.integers(0, 3)), rng)
        okind = int(rng.integers(0, 3))
        to, base = _view(torch, np.zeros(shape, dtype=dt), okind, rng)
        torch.cuda.synchronize()
        assert _run(pn, lib, name, to, ti, alpha) == 0, (case, name, shape)
        pn.synchronize()
        got = to.cpu().numpy()
        if name in EXACT:
            same_bits(got, want)
        elif dt == np.float32:
            rel_close(got, want, 1e-5, 0.0, f"{name} f32 case {case} {shape}")
        else:
            rel_close(got, want, 1e-12, 1e-15, f"{name} f64 case {case} {shape}")
        if okind == 2 and to.dim() >= 1:
            assert bool((base[..., 1::2] == 0).all()), (case, name, "stepped output wrote between its elements")
