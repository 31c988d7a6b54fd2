"""Row softmax / log-softmax parity.

Contract: REL32 (|g - r| <= 1e-5 |r|) for f32 outputs and REL64
(|g - r| <= 1e-12 |r| + 1e-15) for f64, where r is the fp64-exact softmax
(numpy, float64 math).  The oracle's sequential-order restatement of
node_softmax / metrics_losses.c:47-64 is held to the same bound.  A NaN in a
row makes the whole row NaN, as in the reference.
"""

import numpy as np
import pytest

from conftest import GPU, rel_close

pytestmark = GPU


def _exact(x, log):
    x64 = x.astype(np.float64)
    m = np.max(np.where(np.isnan(x64), -np.inf, x64), axis=1, keepdims=True)
    e = np.exp(x64 - m)
    s = np.sum(e, axis=1, keepdims=True)
    return (x64 - m) - np.log(s) if log else e / s


def _run(pn, x, log):
    mod = pn.LogSoftmax() if log else pn.Softmax()
    return mod(pn.Tensor.from_numpy(x)).numpy()


@pytest.mark.parametrize("rows,cols", [(65536, 1024), (100, 1000), (33, 4096), (7, 5000), (9, 3), (1, 1)])
@pytest.mark.parametrize("log", [False, True])
def test_softmax_f32(pn, ora, rows, cols, log):
    rng = np.random.default_rng(rows + cols + int(log))
    x = rng.normal(0, 3, (rows, cols)).astype(np.float32)
    got = _run(pn, x, log)
    want = _exact(x, log)
    rel_close(got, want, 1e-5, 0.0, "gpu vs fp64 exact")
    if rows * cols <= 1 << 22:
        rel_close(ora.softmax_rows(x, log), want, 1e-5, 0.0, "oracle vs fp64 exact")


@pytest.mark.parametrize("rows,cols", [(4096, 1024), (50, 2048), (5, 3001)])
@pytest.mark.parametrize("log", [False, True])
def test_softmax_f64(pn, ora, rows, cols, log):
    rng = np.random.default_rng(cols)
    x = rng.normal(0, 3, (rows, cols))
    got = _run(pn, x, log)
    rel_close(got, _exact(x, log), 1e-12, 1e-15, "gpu vs fp64 exact")
    rel_close(got, ora.softmax_rows(x, log), 1e-12, 1e-15, "gpu vs oracle")


def test_softmax_special_rows(pn, ora):
    x = np.random.default_rng(5).normal(0, 3, (6, 256)).astype(np.float32)
    x[1, 17] = np.nan
    x[2, :] = -np.inf
    x[3, 5] = np.inf
    x[4, :] = 30.0
    x[5, 0] = 80.0
    for log in (False, True):
        got = _run(pn, x, log)
        want = ora.softmax_rows(x, log)
        assert np.array_equal(np.isnan(got), np.isnan(want))
        ok = ~np.isnan(want)
        rel_close(got[ok], want[ok], 1e-5, 1e-30, "special rows")
        assert np.all(np.isnan(got[1])) and np.all(np.isnan(got[2]))


def test_softmax_errors(pn):
    a = pn.Tensor.create([4, 8])
    b = pn.Tensor.create([4, 8], pn.float64)
    assert pn.core._lib.neural_softmax(b._ptr, a._ptr) == pn.NeuralError.DTYPE_MISMATCH
    c = pn.Tensor.create([5, 8])
    assert pn.core._lib.neural_softmax(c._ptr, a._ptr) == pn.NeuralError.SHAPE_MISMATCH


def test_timed_launch(pn):
    """neural_hip_time_next_launch: the events ride on the chosen launch of the
    calling thread (elapsed time > 0, outputs unchanged), are used once, can
    skip launches (the combine launch of a whole-tensor sum is skip = 1) and
    be cancelled; null events and negative skips are rejected."""
    import ctypes
    from pathlib import Path
    import torch
    hip = ctypes.CDLL(str(Path(torch.__file__).parent / "lib" / "libamdhip64.so"))
    hip.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
    hip.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
    hip.hipEventDestroy.argtypes = [ctypes.c_void_p]
    lib = pn.core._lib
    rng = np.random.default_rng(41)
    x = rng.normal(0, 3, (512, 1024)).astype(np.float32)
    tx = pn.Tensor.from_numpy(x)
    y_plain = pn.Tensor.create(tx.shape, tx.dtype)
    assert lib.neural_softmax(y_plain._ptr, tx._ptr) == 0
    s = torch.cuda.current_stream()
    lib.neural_hip_set_stream(ctypes.c_void_p(s.cuda_stream))
    ev = []
    try:
        def pair():
            e0, e1 = ctypes.c_void_p(), ctypes.c_void_p()
            assert hip.hipEventCreate(ctypes.byref(e0)) == 0 and hip.hipEventCreate(ctypes.byref(e1)) == 0
            ev.extend([e0, e1])
            return e0, e1

        def elapsed(e0, e1):
            ms = ctypes.c_float()
            assert hip.hipEventElapsedTime(ctypes.byref(ms), e0, e1) == 0
            return ms.value

        e0, e1 = pair()
        assert lib.neural_hip_time_next_launch(e0, e1, 0) == 0
        y = pn.Tensor.create(tx.shape, tx.dtype)
        assert lib.neural_softmax(y._ptr, tx._ptr) == 0
        torch.cuda.synchronize()
        assert elapsed(e0, e1) > 0.0
        assert np.array_equal(y.numpy(), y_plain.numpy())
        assert lib.neural_softmax(y._ptr, tx._ptr) == 0  # nothing armed: a plain launch
        assert np.array_equal(y.numpy(), y_plain.numpy())
        # a whole-tensor sum of 2^24 values is a segment launch and a combine launch
        big = pn.Tensor.from_numpy(rng.uniform(-1, 1, 1 << 24).astype(np.float32))
        r0 = ctypes.c_double()
        assert lib.neural_sum(big._ptr, ctypes.byref(r0)) == 0
        a0, a1 = pair()
        b0, b1 = pair()
        assert lib.neural_hip_time_next_launch(a0, a1, 0) == 0
        r1 = ctypes.c_double()
        assert lib.neural_sum(big._ptr, ctypes.byref(r1)) == 0
        assert lib.neural_hip_time_next_launch(b0, b1, 1) == 0
        r2 = ctypes.c_double()
        assert lib.neural_sum(big._ptr, ctypes.byref(r2)) == 0
        torch.cuda.synchronize()
        seg_ms, comb_ms = elapsed(a0, a1), elapsed(b0, b1)
        assert seg_ms > 0.0 and comb_ms > 0.0 and comb_ms < seg_ms, (seg_ms, comb_ms)
        assert r0.value == r1.value == r2.value
        # cancel: armed events are dropped unused
        c0, c1 = pair()
        assert lib.neural_hip_time_next_launch(c0, c1, 0) == 0
        assert lib.neural_hip_time_cancel() == 0
        assert lib.neural_softmax(y._ptr, tx._ptr) == 0
        torch.cuda.synchronize()
        ms = ctypes.c_float()
        assert hip.hipEventElapsedTime(ctypes.byref(ms), c0, c1) != 0  # never recorded
        hip.hipGetLastError()  # clear that error so the next library call does not report it
        assert lib.neural_hip_time_next_launch(None, e1, 0) == pn.NeuralError.NULL_POINTER
        assert lib.neural_hip_time_next_launch(e0, e1, -1) == pn.NeuralError.INVALID_ARGUMENT
    finally:
        lib.neural_hip_time_cancel()
        lib.neural_hip_reset_stream()
        for e in ev:
            hip.hipEventDestroy(e)
