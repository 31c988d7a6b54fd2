"""Randomised binary ops over broadcast shapes and strided views.

Seeded cases in both dtypes across add / sub / mul / div / maximum
(math_kernels.asm:66-507, 730-835, with numpy broadcasting as the intended
semantics of neural_add..div): shapes of 1-4 dims with sizes 1-7, each
operand broadcast along random dims or missing leading dims; inputs and the
output as torch tensors that are contiguous, permuted (a transposed copy
viewed back) or stepped (every other element of a wider tensor);
NaN, +-Inf, +-0 and subnormals planted.  Every result is compared bit for
bit with numpy's IEEE result in the same dtype (maximum by the reference's
rule (a > b) ? a : b, which keeps b when either is NaN); stepped outputs
must leave the elements between them untouched.
"""

import numpy as np
import pytest

from conftest import GPU, keep, same_bits

pytestmark = GPU

CASES = 60


def _ref(op, a, b):
    with np.errstate(all="ignore"):
        if op == "add":
            return a + b
        if op == "sub":
            return a - b
        if op == "mul":
            return a * b
        if op == "div":
            return a / b
        return np.where(a > b, a, b)


def _shapes(rng):
    nd = int(rng.integers(1, 5))
    out = [int(rng.integers(1, 8)) for _ in range(nd)]

    def operand():
        s = [d if rng.random() < 0.6 else 1 for d in out]
        drop = int(rng.integers(0, nd))  # missing leading dims broadcast too
        return tuple(s[drop:]) if rng.random() < 0.3 else tuple(s)

    return operand(), operand()


def _values(rng, shape, dt):
    x = rng.normal(0, 2, shape).astype(dt)
    flat = x.reshape(-1)
    specials = np.array([np.nan, np.inf, -np.inf, 0.0, -0.0, np.finfo(dt).tiny / 4], dtype=dt)
    k = int(rng.integers(0, max(1, flat.size // 4) + 1))
    if flat.size and k:
        flat[rng.integers(0, flat.size, k)] = rng.choice(specials, k)
    return x


def _view(torch, x, kind, rng):
    """A CUDA tensor whose logical values are x: contiguous, permuted, or
    stepped; also the tensor that owns the memory (for the untouched check)."""
    if kind == 1 and x.ndim >= 2:
        p = rng.permutation(x.ndim)
        base = torch.from_numpy(np.ascontiguousarray(x.transpose(p))).cuda()
        return base.permute(*np.argsort(p).tolist()), base
    if kind == 2 and x.ndim >= 1:
        wide = list(x.shape)
        wide[-1] *= 2
        base = torch.zeros(wide, dtype=torch.float32 if x.dtype == np.float32 else torch.float64, device="cuda")
        v = base[..., ::2]
        v.copy_(torch.from_numpy(x).cuda())
        return v, base
    t = torch.from_numpy(np.ascontiguousarray(x)).cuda()
    return t, t


@pytest.mark.parametrize("dt", [np.float32, np.float64])
def test_random_broadcast_and_views(pn, dt):
    torch = pytest.importorskip("torch")
    lib = pn.core._lib
    fns = {"add": lib.neural_add, "sub": lib.neural_sub, "mul": lib.neural_mul, "div": lib.neural_div,
           "max": lib.neural_maximum}
    rng = np.random.default_rng(1234 if dt == np.float32 else 4321)
    for case in range(CASES):
        sa, sb = _shapes(rng)
        a, b = _values(rng, sa, dt), _values(rng, sb, dt)
        want_shape = np.broadcast_shapes(sa, sb)
        for op, fn in fns.items():
            want = _ref(op, a, b)
            assert want.shape == want_shape
            ta, _ = _view(torch, a, int(rng.integers(0, 3)), rng)
            tb, _ = _view(torch, b, int(rng.integers(0, 3)), rng)
            okind = int(rng.integers(0, 3))
            to, base = _view(torch, np.full(want_shape, 7, dtype=dt), okind, rng)
            torch.cuda.synchronize()
            rc = fn(keep(pn.Tensor.from_torch(to)), keep(pn.Tensor.from_torch(ta)), keep(pn.Tensor.from_torch(tb)))
            assert rc == 0, (case, op, sa, sb, okind, rc)
            pn.synchronize()
            got = to.cpu().numpy()
            same_bits(got, want.astype(dt))
            if okind == 2 and to.dim() >= 1:
                assert bool((base[..., 1::2] == 0).all()), (case, op, "stepped output wrote between its elements")
