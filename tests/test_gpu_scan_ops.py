"""NaN/Inf scan + L2 norm (training_ops.asm:544-696) and 2-D tensor ops
(tensor_ops.c:15-148).

Flags are exact; the L2 norm is held to |g - e| <= 1e-5 * e with e the
sqrt of the fp64-exact sum of squares (the reference's own 4-lane fp32 norm
is reported beside it).  Tensor ops are bit-exact copies.
"""

import ctypes

import numpy as np
import pytest

from conftest import GPU, same_bits

pytestmark = GPU


def _grads(n, seed=6):
    rng = np.random.default_rng(seed)
    return rng.normal(0, 1e-3, n).astype(np.float32)


@pytest.mark.parametrize("n", [1, 3, 4, 5, 1000, 1 << 22])
def test_scan_clean(pn, ora, n):
    g = _grads(n)
    lib = pn.core._lib
    assert lib.neural_tensor_has_nan(g.ctypes.data, n) == 0
    assert lib.neural_tensor_has_inf(g.ctypes.data, n) == 0
    e = np.sqrt(ora.sumsq_exact(g))
    got = lib.neural_tensor_grad_l2_norm(g.ctypes.data, n)
    assert abs(got - e) <= 1e-5 * e
    assert abs(pn.grad_l2_norm(pn.Tensor.from_numpy(g)) - e) <= 1e-5 * e
    # reference order, reported: 4-lane fp32 (training_ops.asm:646-690)
    r = ora.l2_ref(g)
    assert abs(r - e) <= 5e-2 * e


def test_scan_injected(pn, ora):
    n = 1 << 20
    g = _grads(n)
    rng = np.random.default_rng(1)
    idx = rng.choice(n, 96, replace=False)
    lib = pn.core._lib
    for vals, want in (([np.nan], (1, 0)), ([np.inf], (0, 1)), ([-np.inf], (0, 1)), ([np.nan, -np.inf], (1, 1))):
        x = g.copy()
        for k, v in enumerate(vals):
            x[idx[k * 32:(k + 1) * 32]] = v
        hn, hi, ss = ctypes.c_int(), ctypes.c_int(), ctypes.c_double()
        assert lib.neural_scan_nan_inf_l2(x.ctypes.data, n, ctypes.byref(hn), ctypes.byref(hi), ctypes.byref(ss)) == 0
        assert (hn.value, hi.value) == want
        assert (lib.neural_tensor_has_nan(x.ctypes.data, n), lib.neural_tensor_has_inf(x.ctypes.data, n)) == want
        assert (ora.has_nan(x), ora.has_inf(x)) == want
        det = pn.NaNDetector(raise_on_detect=False)
        t = pn.Tensor.from_numpy(x)
        assert (det.has_nan(t), det.has_inf(t)) == (bool(want[0]), bool(want[1]))
        assert np.isnan(ss.value) or np.isinf(ss.value)
    assert lib.neural_tensor_has_nan(None, 5) == 0
    assert lib.neural_tensor_has_inf(g.ctypes.data, 0) == 0
    assert lib.neural_tensor_grad_l2_norm(None, 0) == 0.0


def test_detector_raises(pn):
    x = np.ones(10, dtype=np.float32)
    x[3] = np.nan
    with pytest.raises(RuntimeError):
        pn.NaNDetector().check(pn.Tensor.from_numpy(x), "grads")


def test_tensor_ops(pn, ora):
    rng = np.random.default_rng(8)
    a = rng.normal(size=12).tolist()
    b = rng.normal(size=8).tolist()
    from pyneural import tensor_ops as T
    out, r, c = T.concat_2d(a, rng.normal(size=6).tolist(), 3, 4, 3, 2, axis=1)
    rc, want, wr, wc = ora.concat_2d(np.array(a), np.array(out[4:6] + out[10:12] + out[16:18]), 3, 4, 3, 2, 1)
    assert (r, c) == (3, 6) and rc == 0
    same_bits(np.array(out), want)
    out, r, c = T.concat_2d(a, b, 3, 4, 2, 4, axis=0)
    assert (r, c) == (5, 4)
    same_bits(np.array(out), np.array(a + b))
    x = rng.normal(size=35)
    oa, ra, ca, ob, rb, cb = T.split_2d(x.tolist(), 5, 7, axis=1, split_index=3)
    rc, wa, wb, dims = ora.split_2d(x, 5, 7, 1, 3)
    assert (ra, ca, rb, cb) == dims
    same_bits(np.array(oa), wa)
    same_bits(np.array(ob), wb)
    oa, ra, ca, ob, rb, cb = T.split_2d(x.tolist(), 5, 7, axis=0, split_index=2)
    same_bits(np.array(oa + ob), x)
    out, r, c = T.pad_2d(x.tolist(), 5, 7, 1, 2, 3, 0, -1.5)
    rc, want, wr, wc = ora.pad_2d(x, 5, 7, 1, 2, 3, 0, -1.5)
    assert (r, c) == (wr, wc)
    same_bits(np.array(out), want)
    big = rng.normal(size=(300, 517))
    out, r, c = T.transpose_2d(big.ravel().tolist(), 300, 517)
    assert (r, c) == (517, 300)
    same_bits(np.array(out).reshape(517, 300), big.T)
    with pytest.raises(RuntimeError):
        T.concat_2d(a, b, 3, 4, 2, 4, axis=1)
    with pytest.raises(RuntimeError):
        T.split_2d(x.tolist(), 5, 7, axis=0, split_index=5)
    with pytest.raises(RuntimeError):
        T.pad_2d(x.tolist(), 5, 7, -1, 0, 0, 0)
