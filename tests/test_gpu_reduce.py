"""Reduction parity.

sum / mean: REDUCE tolerance |g - e| <= 1e-5 * sum|x| against the fp64-exact
value (the reference's own fp32 lane orders are reported by the CPU tests,
not gated).  max (running-max chain semantics incl. NaN restarts and zero
signs) and argmax (first index, NaN never wins, x0 NaN -> 0): bit-exact
against the oracle's restatement of activations.asm:888-895 and
main.asm:3245-3292,3598-3640.
"""

import ctypes

import numpy as np
import pytest

from conftest import GPU, keep, same_bits

pytestmark = GPU


def _sum(pn, t):
    r = ctypes.c_double()
    pn.core._check_error(pn.core._lib.neural_sum(t._ptr, ctypes.byref(r)), "sum")
    return r.value


@pytest.mark.parametrize("n", [1, 7, 8, 1000, 1 << 20, 67108864])
def test_full_sum_mean(pn, ora, n):
    rng = np.random.default_rng(0)
    x = rng.uniform(-1, 1, n).astype(np.float32)
    t = pn.Tensor.from_numpy(x)
    e = ora.sum_exact(x)
    bound = 1e-5 * float(np.sum(np.abs(x, dtype=np.float64)))
    g = _sum(pn, t)
    assert abs(g - e) <= bound
    assert _sum(pn, t) == g  # deterministic
    assert abs(t.mean() - e / n) <= bound / n
    # the reference's own 8-lane fp32 order, reported for scale
    r = ora.sum_ref(x)
    assert abs(r - e) <= 1e-3 * float(np.sum(np.abs(x)))


def test_full_sum_f64(pn, ora, rng):
    x = rng.normal(0, 1, 300001)
    g = pn.Tensor.from_numpy(x).sum()
    assert abs(g - ora.sum_exact(x)) <= 1e-12 * float(np.sum(np.abs(x)))


def _chain_cases(rng):
    cases = [rng.normal(size=1000).astype(np.float32)]
    a = rng.normal(size=777).astype(np.float32)
    a[[5, 300]] = np.nan
    cases.append(a)
    b = rng.normal(size=500).astype(np.float32)
    b[-1] = np.nan  # chain ends on NaN -> NaN
    cases.append(b)
    c = np.array([0.0, -0.0, -1.0, -0.0, -3.0], dtype=np.float32)  # ties resolve to the later zero
    cases.append(c)
    d = np.array([np.nan, 2.0, 7.0, 7.0, 1.0], dtype=np.float32)
    cases.append(d)
    e = np.full(64, -np.inf, dtype=np.float32)
    cases.append(e)
    f = rng.normal(size=3000003).astype(np.float32)
    f[1234567] = np.nan
    cases.append(f)
    return cases


def test_full_max_argmax(pn, ora, rng):
    for x in _chain_cases(rng):
        t = pn.Tensor.from_numpy(x)
        got = np.float32(t.max())
        same_bits(np.array([got]), np.array([ora.max_chain(x)], dtype=np.float32))
        assert t.argmax() == ora.argmax(x), x[:8]


def test_full_argmax_special(pn, ora):
    x = np.array([np.nan, 5.0, 9.0], dtype=np.float32)
    assert pn.Tensor.from_numpy(x).argmax() == 0
    x = np.array([1.0, 9.0, 3.0, 9.0, np.nan], dtype=np.float32)
    assert pn.Tensor.from_numpy(x).argmax() == 1
    x = np.zeros(1 << 20, dtype=np.float32)
    x[777777] = 1.0
    x[888888] = 1.0
    assert pn.Tensor.from_numpy(x).argmax() == 777777


@pytest.mark.parametrize("rows,cols", [(8192, 4096), (100, 1000), (37, 5), (3, 70000), (1, 1)])
@pytest.mark.parametrize("dt", [np.float32, np.float64])
def test_rows(pn, ora, rows, cols, dt):
    rng = np.random.default_rng(rows * 7 + cols)
    x = rng.normal(0, 3, (rows, cols)).astype(dt)
    if rows > 2 and cols > 3:
        x[1, 2] = np.nan          # NaN mid-row: chain restarts after it
        x[2, cols - 1] = np.nan   # NaN last: row max is NaN
        x[0, :] = 0.0
        x[0, 1::2] = -0.0         # zero ties: later element wins
    lib = pn.core._lib
    t = pn.Tensor.from_numpy(x)
    e = ora.rowsum_exact(x)
    bound = 1e-5 * np.sum(np.abs(x.astype(np.float64)), axis=1)
    for axis in (1, -1 if x.ndim == 1 else 1):
        out = pn.Tensor.create([rows], t.dtype)
        pn.core._check_error(lib.neural_reduce_sum(t._ptr, axis, out._ptr), "reduce_sum")
        g = out.numpy().astype(np.float64)
        ok = ~np.isnan(e)
        assert np.all(np.abs(g[ok] - e[ok]) <= bound[ok] + np.abs(e[ok]) * (6e-8 if dt == np.float32 else 0))
        assert np.array_equal(np.isnan(g), np.isnan(e))
    out = pn.Tensor.create([rows], t.dtype)
    pn.core._check_error(lib.neural_reduce_mean(t._ptr, 1, out._ptr), "reduce_mean")
    g = out.numpy().astype(np.float64)
    ok = ~np.isnan(e)
    assert np.all(np.abs(g[ok] - e[ok] / cols) <= (bound[ok] / cols) + np.abs(e[ok] / cols) * 6e-8)
    out = pn.Tensor.create([rows], t.dtype)
    pn.core._check_error(lib.neural_reduce_max(t._ptr, 1, out._ptr), "reduce_max")
    same_bits(out.numpy(), ora.rowmax_chain(x))
    idx = np.empty(rows, dtype=np.int64)
    pn.core._check_error(lib.neural_reduce_argmax(t._ptr, 1, idx.ctypes.data), "reduce_argmax")
    same_bits(idx, ora.rowargmax(x))


@pytest.mark.parametrize("rows,cols", [(8192, 4096), (1000, 3), (5, 2000)])
def test_colsum_axis0(pn, ora, rows, cols):
    rng = np.random.default_rng(cols)
    x = rng.normal(0, 1, (rows, cols)).astype(np.float32)
    out = pn.Tensor.create([cols])
    pn.core._check_error(pn.core._lib.neural_reduce_sum(keep(pn.Tensor.from_numpy(x)), 0, out._ptr), "colsum")
    e = ora.rowsum_exact(np.ascontiguousarray(x.T))
    bound = 1e-5 * np.sum(np.abs(x.astype(np.float64)), axis=0) + np.abs(e) * 6e-8
    assert np.all(np.abs(out.numpy() - e) <= bound)
    # the reference order (zero then accumulate rows) for scale
    assert np.all(np.abs(ora.colsum_ref(x) - e) <= 1e-3 * np.sum(np.abs(x), axis=0))


def test_reduce_all_axis_and_errors(pn, ora, rng):
    x = rng.uniform(-1, 1, (64, 1000)).astype(np.float32)
    t = pn.Tensor.from_numpy(x)
    out = pn.Tensor.create([1])
    pn.core._check_error(pn.core._lib.neural_reduce_sum(t._ptr, -1, out._ptr), "sum all")
    assert abs(out.numpy()[0] - ora.sum_exact(x)) <= 1e-5 * np.sum(np.abs(x)) + 1e-6
    bad = pn.Tensor.create([3])
    assert pn.core._lib.neural_reduce_sum(t._ptr, 1, bad._ptr) == pn.NeuralError.SHAPE_MISMATCH
    bad64 = pn.Tensor.create([64], pn.float64)
    assert pn.core._lib.neural_reduce_sum(t._ptr, 1, bad64._ptr) == pn.NeuralError.DTYPE_MISMATCH
    r = ctypes.c_double()
    assert pn.core._lib.neural_sum(None, ctypes.byref(r)) == pn.NeuralError.NULL_POINTER


def test_strided_reduction(pn, ora, rng):
    torch = pytest.importorskip("torch")
    a = torch.randn(300, 257, device="cuda", dtype=torch.float64)
    at = a.t()
    torch.cuda.synchronize()
    s = pn.Tensor.from_torch(at).sum()
    x = at.cpu().numpy()
    assert abs(s - ora.sum_exact(np.ascontiguousarray(x))) <= 1e-12 * np.sum(np.abs(x))
    idx = np.empty(257, dtype=np.int64)
    pn.core._check_error(pn.core._lib.neural_reduce_argmax(keep(pn.Tensor.from_torch(at)), 1, idx.ctypes.data), "am")
    same_bits(idx, ora.rowargmax(np.ascontiguousarray(x)))


def _seg_cases(rng, cols):
    """Rows long enough to be split over many blocks, with the rare cases of
    the chain (NaN restarts, a NaN as last element, zero-sign ties, Inf) placed
    at random and at both row ends."""
    rows = []
    a = rng.normal(0, 3, cols).astype(np.float32)
    rows.append(a)
    b = a.copy()
    b[rng.choice(cols, 5, replace=False)] = np.nan
    rows.append(b)
    c = a.copy()
    c[-1] = np.nan
    rows.append(c)
    d = -np.abs(a)
    d[rng.choice(cols, 40, replace=False)] = 0.0
    d[rng.choice(cols, 40, replace=False)] = -0.0
    rows.append(d)
    e = a.copy()
    e[rng.choice(cols, 3, replace=False)] = np.inf
    e[rng.choice(cols, 3, replace=False)] = -np.inf
    rows.append(e)
    f = a.copy()
    f[0] = np.nan
    rows.append(f)
    g = np.full(cols, -np.inf, dtype=np.float32)
    g[rng.choice(cols, 2, replace=False)] = np.nan
    rows.append(g)
    h = -np.abs(a)
    h[cols // 2] = -0.0
    h[cols - 1] = 0.0  # the later zero decides the sign
    rows.append(h)
    return np.stack(rows)


@pytest.mark.parametrize("cols", [1 << 20, 3 * (1 << 18) + 5])
@pytest.mark.parametrize("dt", [np.float32, np.float64])
def test_segmented_rows_special(pn, ora, cols, dt):
    rng = np.random.default_rng(cols)
    x = _seg_cases(rng, cols).astype(dt)
    rows = x.shape[0]
    lib = pn.core._lib
    t = pn.Tensor.from_numpy(x)
    out = pn.Tensor.create([rows], t.dtype)
    pn.core._check_error(lib.neural_reduce_max(t._ptr, 1, out._ptr), "reduce_max")
    same_bits(out.numpy(), ora.rowmax_chain(x))
    idx = np.empty(rows, dtype=np.int64)
    pn.core._check_error(lib.neural_reduce_argmax(t._ptr, 1, idx.ctypes.data), "reduce_argmax")
    same_bits(idx, ora.rowargmax(x))
    out = pn.Tensor.create([rows], t.dtype)
    pn.core._check_error(lib.neural_reduce_sum(t._ptr, 1, out._ptr), "reduce_sum")
    e = ora.rowsum_exact(x)
    g = out.numpy().astype(np.float64)
    fin = np.isfinite(e)
    bound = 1e-5 * np.sum(np.abs(np.where(np.isfinite(x), x, 0).astype(np.float64)), axis=1)
    assert np.all(np.abs(g[fin] - e[fin]) <= bound[fin] + np.abs(e[fin]) * 6e-8)
    same_bits(np.isnan(g), np.isnan(e))
    # every row on its own, as a 1-D tensor (one row split over the whole grid)
    for r in range(rows):
        tr = pn.Tensor.from_numpy(np.ascontiguousarray(x[r]))
        one = pn.Tensor.create([1], t.dtype)
        pn.core._check_error(lib.neural_reduce_max(tr._ptr, -1, one._ptr), "max 1-D")
        same_bits(one.numpy(), ora.rowmax_chain(x[r:r + 1]))
        got = np.array([tr.max()], dtype=dt)
        same_bits(got, np.array([ora.max_chain(x[r])], dtype=dt))
        assert tr.argmax() == ora.argmax(x[r])


def test_reduce_deterministic_large(pn, ora):
    """Same input, same grid: bitwise identical sums run to run."""
    rng = np.random.default_rng(77)
    x = rng.normal(0, 1, (3, 5_000_001)).astype(np.float32)
    t = pn.Tensor.from_numpy(x)
    outs = []
    for _ in range(3):
        o = pn.Tensor.create([3])
        pn.core._check_error(pn.core._lib.neural_reduce_sum(t._ptr, 1, o._ptr), "sum")
        outs.append(o.numpy().tobytes())
    assert outs[0] == outs[1] == outs[2]
    e = ora.rowsum_exact(x)
    assert np.all(np.abs(np.frombuffer(outs[0], np.float32) - e) <= 1e-5 * np.sum(np.abs(x), axis=1) + np.abs(e) * 6e-8)
