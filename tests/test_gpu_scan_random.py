"""Randomised NaN / Inf scan and gradient L2 norm (training_ops.asm:544-696).

Seeded float32 vectors of 1 to 4 M values (log-uniform) with a scale of
10^U(-6, 3), starting 0-3 values past a 16-byte boundary, with 0-3 NaN or
+-Inf planted (the first and last value included now and then).  The flags
of neural_scan_nan_inf_l2, neural_tensor_has_nan / _has_inf and the oracle
must agree exactly; on clean data the sum of squares and the norm must sit
within 1e-5 relative of the fp64-exact values.
"""

import ctypes
import math

import numpy as np

from conftest import GPU

pytestmark = GPU

CASES = 40


def test_random_scans(pn, ora):
    lib = pn.core._lib
    rng = np.random.default_rng(1001)
    for case in range(CASES):
        n = int(np.exp(rng.uniform(0, np.log(4_000_000))))
        off = int(rng.integers(0, 4))
        buf = np.empty(n + 4, dtype=np.float32)
        x = buf[off:off + n]
        x[...] = rng.normal(0, 10.0 ** rng.uniform(-6, 3), n)
        for _ in range(int(rng.integers(0, 4))):
            u = rng.random()
            i = 0 if u < 0.15 else n - 1 if u < 0.3 else int(rng.integers(0, n))
            x[i] = rng.choice([np.nan, np.inf, -np.inf])
        want = (int(np.isnan(x).any()), int(np.isinf(x).any()))
        hn, hi, ss = ctypes.c_int(), ctypes.c_int(), ctypes.c_double()
        assert lib.neural_scan_nan_inf_l2(x.ctypes.data, n, ctypes.byref(hn), ctypes.byref(hi),
                                          ctypes.byref(ss)) == 0, (case, n, off)
        assert (hn.value, hi.value) == want, (case, n, off)
        assert (lib.neural_tensor_has_nan(x.ctypes.data, n), lib.neural_tensor_has_inf(x.ctypes.data, n)) == want
        assert (ora.has_nan(np.ascontiguousarray(x)), ora.has_inf(np.ascontiguousarray(x))) == want
        if want == (0, 0):
            e2 = ora.sumsq_exact(np.ascontiguousarray(x))
            assert abs(ss.value - e2) <= 1e-5 * e2, (case, n, ss.value, e2)
            got = lib.neural_tensor_grad_l2_norm(x.ctypes.data, n)
            assert abs(got - math.sqrt(e2)) <= 1e-5 * math.sqrt(e2), (case, n)
        else:
            assert not math.isfinite(ss.value), (case, n, ss.value)
