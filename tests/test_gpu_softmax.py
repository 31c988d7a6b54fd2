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


def test_softmax_timed_launch(pn):
    """neural_hip_time_next_softmax: the events ride on the next softmax launch
    (elapsed time > 0, output unchanged), are used once, and a null event is
    rejected."""
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
    try:
        e0, e1 = ctypes.c_void_p(), ctypes.c_void_p()
        assert hip.hipEventCreate(ctypes.byref(e0)) == 0 and hip.hipEventCreate(ctypes.byref(e1)) == 0
        assert lib.neural_hip_time_next_softmax(e0, e1) == 0
        y = pn.Tensor.create(tx.shape, tx.dtype)
        assert lib.neural_softmax(y._ptr, tx._ptr) == 0
        torch.cuda.synchronize()
        ms = ctypes.c_float()
        assert hip.hipEventElapsedTime(ctypes.byref(ms), e0, e1) == 0
        assert ms.value > 0.0
        assert np.array_equal(y.numpy(), y_plain.numpy())
        assert lib.neural_softmax(y._ptr, tx._ptr) == 0  # no events pending: a plain launch
        assert np.array_equal(y.numpy(), y_plain.numpy())
        assert lib.neural_hip_time_next_softmax(None, e1) == pn.NeuralError.NULL_POINTER
        hip.hipEventDestroy(e0)
        hip.hipEventDestroy(e1)
    finally:
        lib.neural_hip_reset_stream()
