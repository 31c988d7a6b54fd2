"""Randomised INT8 quantization (quantize.c:52-214).

Seeded cases in both dtypes: 1 to 2 M values (log-uniform), drawn from a
normal, Laplace or uniform law scaled by 10^U(-30, 30) and shifted by up to
+-5 scales (ranges on one side of zero), or constant; NaN, +-Inf, +-0 and
values 1e6 scales out planted in some cases (these reach the x86 cvttsd2si
rule for out-of-range conversions).  Calibration (min/max, both modes),
quantize and dequantize on host buffers, the float32 device forms on device
buffers, and percentile calibration (finite float64 data) must equal the
oracle bit for bit; quantized_matmul on random shapes and params likewise.
"""

import ctypes

import numpy as np
import pytest

from conftest import GPU, same_bits
from test_gpu_quant import _calib, _params_equal, _qp_bits, _quant

pytestmark = GPU

CASES = 40


def _case(rng, dt, specials=True):
    n = int(np.exp(rng.uniform(0, np.log(2_000_000))))
    s = 10.0 ** rng.uniform(-30, 30)
    kind = int(rng.integers(0, 4))
    if kind == 0:
        x = rng.normal(0, 1, n)
    elif kind == 1:
        x = rng.laplace(0, 1, n)
    elif kind == 2:
        x = rng.uniform(-1, 1, n)
    else:
        x = np.full(n, rng.normal())
    x = (x + rng.uniform(-5, 5)) * s
    if specials and rng.random() < 0.4:
        vals = np.array([np.nan, np.inf, -np.inf, 0.0, -0.0, 1e6 * s, -1e6 * s])
        k = int(rng.integers(1, 6))
        x[rng.integers(0, n, k)] = rng.choice(vals, k)
    with np.errstate(over="ignore"):
        return x.astype(dt)


@pytest.mark.parametrize("dt", [np.float32, np.float64])
def test_random_minmax_pipeline(pn, ora, dt):
    torch = pytest.importorskip("torch")
    lib = pn.core._lib
    rng = np.random.default_rng(808 if dt == np.float32 else 809)
    for case in range(CASES):
        x = _case(rng, dt)
        n = x.size
        for sym in (True, False):
            p = _calib(pn, x, sym)
            want = ora.calibrate(x, sym)
            _params_equal(p, want)
            q = _quant(pn, x, p)
            wq = ora.quantize(x, want)
            same_bits(q, wq)
            d = np.empty(n, dtype=dt)
            fn = lib.dequantize_tensor_f32 if dt == np.float32 else lib.dequantize_tensor
            assert fn(q.ctypes.data, d.ctypes.data, n, ctypes.byref(p)) == 0, (case, n, sym)
            same_bits(d, ora.dequantize(wq, want, dt))
        if dt == np.float32:
            # the device forms: params stay in device memory between the three calls
            xt = torch.from_numpy(x).cuda()
            qt = torch.empty(n, dtype=torch.int8, device="cuda")
            dt_ = torch.empty(n, dtype=torch.float32, device="cuda")
            pbuf = torch.zeros(5, dtype=torch.float64, device="cuda")
            torch.cuda.synchronize()
            assert lib.calibrate_minmax_f32_dev(xt.data_ptr(), n, 0, pbuf.data_ptr()) == 0
            assert lib.quantize_tensor_f32_dev(xt.data_ptr(), qt.data_ptr(), n, pbuf.data_ptr()) == 0
            assert lib.dequantize_tensor_f32_dev(qt.data_ptr(), dt_.data_ptr(), n, pbuf.data_ptr()) == 0
            pn.synchronize()
            _params_equal(pn.core.QuantParamsC.from_buffer_copy(pbuf.cpu().numpy().tobytes()), want)
            same_bits(qt.cpu().numpy(), wq)
            same_bits(dt_.cpu().numpy(), ora.dequantize(wq, want, np.float32))


def test_random_percentile(pn, ora):
    lib = pn.core._lib
    rng = np.random.default_rng(810)
    for case in range(CASES // 2):
        x = _case(rng, np.float64, specials=False)
        if rng.random() < 0.3:
            x[rng.integers(0, x.size, max(1, x.size // 10))] = rng.choice([0.0, -0.0])
        for sym in (0, 1):
            for pc in (float(rng.uniform(0, 0.5)), float(10.0 ** rng.uniform(-6, -1))):
                got = pn.core.QuantParamsC()
                assert lib.calibrate_percentile(x.ctypes.data, x.size, ctypes.c_double(pc), sym,
                                                ctypes.byref(got)) == 0
                rc, want = ora.calibrate_percentile(x, pc, sym)
                assert rc == 0
                assert _qp_bits(got) == _qp_bits(want), (case, x.size, pc, sym)


def test_random_quantized_matmul(pn, ora):
    lib = pn.core._lib
    rng = np.random.default_rng(811)
    for case in range(CASES // 2):
        m, k, n = (int(np.exp(rng.uniform(0, np.log(600)))) for _ in range(3))
        a = rng.integers(-128, 128, (m, k), dtype=np.int64).astype(np.int8)
        b = rng.integers(-128, 128, (k, n), dtype=np.int64).astype(np.int8)
        pa, pb = ora.QuantParams(), ora.QuantParams()
        pa.scale, pa.zero_point = 10.0 ** rng.uniform(-4, 0), int(rng.integers(-128, 128))
        pb.scale, pb.zero_point = 10.0 ** rng.uniform(-4, 0), int(rng.integers(-128, 128))
        qa, qb = pn.core.QuantParamsC(), pn.core.QuantParamsC()
        ctypes.memmove(ctypes.byref(qa), ctypes.byref(pa), ctypes.sizeof(qa))
        ctypes.memmove(ctypes.byref(qb), ctypes.byref(pb), ctypes.sizeof(qb))
        got = np.empty((m, n))
        assert lib.quantized_matmul(a.ctypes.data, b.ctypes.data, got.ctypes.data, m, k, n, ctypes.byref(qa),
                                    ctypes.byref(qb)) == 0, (case, m, k, n)
        rc, want = ora.quantized_matmul(a, b, m, k, n, pa, pb)
        assert rc == 0
        same_bits(got, want)
