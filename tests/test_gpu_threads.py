"""Concurrent callers (ctypes releases the GIL around every library call).

Two host threads call whole-tensor reductions and the NaN/Inf/L2 scan on
different tensors at the same time; both use the shared reduction workspace
and the mapped host-result area.  Every result must equal the one the same
call returns when the process is single-threaded, and each thread's last
error must be its own.
"""

import ctypes
import threading

import numpy as np

from conftest import GPU

pytestmark = GPU

ITERS = 150


def _sum(lib, t):
    r = ctypes.c_double()
    rc = lib.neural_sum(t._ptr, ctypes.byref(r))
    return rc, r.value


def _scan(lib, t):
    n, i, s = ctypes.c_int(), ctypes.c_int(), ctypes.c_double()
    rc = lib.neural_tensor_scan(t._ptr, ctypes.byref(n), ctypes.byref(i), ctypes.byref(s))
    return rc, (n.value, i.value, s.value)


def _argmax(lib, t):
    r = ctypes.c_int64()
    rc = lib.neural_argmax(t._ptr, ctypes.byref(r))
    return rc, r.value


def test_two_threads_share_the_workspace(pn):
    lib = pn.core._lib
    rng = np.random.default_rng(77)
    a = rng.uniform(-1, 1, (1 << 23) + 3).astype(np.float32)   # many segments: the summaries are used
    b = rng.normal(0, 1e-3, 3_000_001).astype(np.float32)
    b[1_234_567] = np.inf
    ta, tb = pn.Tensor.from_numpy(a), pn.Tensor.from_numpy(b)
    want = {
        "sum_a": _sum(lib, ta), "arg_a": _argmax(lib, ta), "scan_b": _scan(lib, tb), "sum_b": _sum(lib, tb),
        "scan_a": _scan(lib, ta),
    }
    assert all(v[0] == 0 for v in want.values()), want
    assert want["scan_b"][1][:2] == (0, 1) and want["scan_a"][1][:2] == (0, 0)
    assert want["sum_a"][1] != want["sum_b"][1]
    bad = []
    bad_err = []
    start = threading.Barrier(2)

    def worker_a():
        start.wait()
        for k in range(ITERS):
            for key, fn in (("sum_a", lambda: _sum(lib, ta)), ("arg_a", lambda: _argmax(lib, ta)),
                            ("scan_a", lambda: _scan(lib, ta))):
                got = fn()
                if got != want[key]:
                    bad.append((key, k, got, want[key]))
            # an error in this thread does not show in the other thread
            if k % 10 == 0:
                small = pn.Tensor.create([3])
                if lib.neural_add(small._ptr, ta._ptr, ta._ptr) != pn.NeuralError.SHAPE_MISMATCH or \
                        lib.neural_get_last_error() != pn.NeuralError.SHAPE_MISMATCH:
                    bad_err.append(("a", k))

    def worker_b():
        start.wait()
        for k in range(ITERS):
            for key, fn in (("scan_b", lambda: _scan(lib, tb)), ("sum_b", lambda: _sum(lib, tb))):
                got = fn()
                if got != want[key]:
                    bad.append((key, k, got, want[key]))
            if lib.neural_get_last_error() != 0:
                bad_err.append(("b", k, lib.neural_get_last_error()))

    th = [threading.Thread(target=worker_a), threading.Thread(target=worker_b)]
    for t in th:
        t.start()
    for t in th:
        t.join(timeout=300)
    assert not any(t.is_alive() for t in th), "a worker thread did not finish"
    assert not bad, bad[:5]
    assert not bad_err, bad_err[:5]
