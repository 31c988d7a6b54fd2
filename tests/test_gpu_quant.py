"""INT8 quantization parity (quantize.c:52-269).

QuantParams and int8 outputs are bit-exact against the oracle (whose
restatement is itself pinned to the reference's own quantize.c in
tests/test_oracle_vs_ref.py), including NaN / Inf / out-of-range inputs that
exercise the x86 cvttsd2si behaviour.  Dequantized values are bit-exact.
error / snr: REDUCE tolerance against the oracle's sequential sums.
"""

import ctypes

import numpy as np
import pytest

from conftest import GPU, same_bits

pytestmark = GPU


def _params_equal(got, want):
    assert got.scale == want.scale or (np.isnan(got.scale) and np.isnan(want.scale))
    assert got.zero_point == want.zero_point
    for f in ("min_val", "max_val"):
        g, w = getattr(got, f), getattr(want, f)
        assert (np.isnan(g) and np.isnan(w)) or np.float64(g).tobytes() == np.float64(w).tobytes(), (f, g, w)
    assert got.symmetric == want.symmetric


def _laplace(n, seed=5):
    rng = np.random.default_rng(seed)
    x = rng.laplace(0, 1, n).astype(np.float32)
    k = min(n, max(2, n // 1000))
    idx = rng.choice(n, size=k, replace=False)
    x[idx] = np.where(np.arange(k) % 2 == 0, 50.0, -50.0).astype(np.float32)
    return x


def _calib(pn, x, sym):
    p = pn.core.QuantParamsC()
    fn = pn.core._lib.calibrate_minmax_f32 if x.dtype == np.float32 else pn.core._lib.calibrate_minmax
    assert fn(x.ctypes.data, x.size, 1 if sym else 0, ctypes.byref(p)) == 0
    return p


def _quant(pn, x, p):
    q = np.empty(x.size, dtype=np.int8)
    fn = pn.core._lib.quantize_tensor_f32 if x.dtype == np.float32 else pn.core._lib.quantize_tensor
    assert fn(x.ctypes.data, q.ctypes.data, x.size, ctypes.byref(p)) == 0
    return q


@pytest.mark.parametrize("n", [1, 15, 17, 100003, 1 << 24])
@pytest.mark.parametrize("sym", [True, False])
def test_f32_pipeline(pn, ora, n, sym):
    x = _laplace(n)
    p = _calib(pn, x, sym)
    want_p = ora.calibrate(x, sym)
    _params_equal(p, want_p)
    q = _quant(pn, x, p)
    same_bits(q, ora.quantize(x, want_p))
    d = np.empty(n, dtype=np.float32)
    assert pn.core._lib.dequantize_tensor_f32(q.ctypes.data, d.ctypes.data, n, ctypes.byref(p)) == 0
    same_bits(d, ora.dequantize(q, want_p, np.float32))
    d64 = np.empty(n, dtype=np.float64)
    assert pn.core._lib.dequantize_tensor(q.ctypes.data, d64.ctypes.data, n, ctypes.byref(p)) == 0
    same_bits(d64, ora.dequantize(q, want_p, np.float64))
    err = pn.core._lib.quantization_error_f32(x.ctypes.data, n, ctypes.byref(p))
    e_want = ora.quant_error(x, want_p)
    assert abs(err - e_want) <= 1e-7 * abs(e_want) + 1e-300
    snr = pn.core._lib.quantization_snr_f32(x.ctypes.data, n, ctypes.byref(p))
    s_want = ora.quant_snr(x, want_p)
    assert abs(snr - s_want) <= 1e-7 * max(abs(s_want), 1.0)


def test_f64_reference_api(pn, ora, rng):
    x = rng.normal(0, 2, 50001)
    x[[3, 99]] = [1e12, -7.5]
    for sym in (True, False):
        p = _calib(pn, x, sym)
        want = ora.calibrate(x, sym)
        _params_equal(p, want)
        same_bits(_quant(pn, x, p), ora.quantize(x, want))


def test_special_values(pn, ora):
    x = np.array([0.3, np.nan, np.inf, -np.inf, 1e30, -1e30, 0.0, -0.0, 2.5, -2.5] * 7, dtype=np.float64)
    for zp in (-1, 0, 5, -128, 127):
        p = pn.core.QuantParamsC(0.5, zp, 0.0, 0.0, 0)
        q = _quant(pn, x, p)
        wp = ora.QuantParams(0.5, zp, 0.0, 0.0, 0)
        same_bits(q, ora.quantize(x, wp))
    # x0 NaN poisons calibration exactly as the sequential loop does
    y = np.array([np.nan, 1.0, -2.0], dtype=np.float32)
    p = _calib(pn, y, False)
    _params_equal(p, ora.calibrate(y, False))
    z = np.zeros(33, dtype=np.float32)
    z[5] = -0.0
    for sym in (True, False):
        _params_equal(_calib(pn, z, sym), ora.calibrate(z, sym))


def test_device_pipeline(pn, ora):
    torch = pytest.importorskip("torch")
    x = _laplace(1 << 20, seed=11)
    xt = torch.from_numpy(x).cuda()
    q = torch.empty(x.size, dtype=torch.int8, device="cuda")
    d = torch.empty(x.size, dtype=torch.float32, device="cuda")
    pbuf = torch.zeros(5, dtype=torch.float64, device="cuda")  # 40-byte QuantParams
    torch.cuda.synchronize()
    lib = pn.core._lib
    assert lib.calibrate_minmax_f32_dev(xt.data_ptr(), x.size, 0, pbuf.data_ptr()) == 0
    assert lib.quantize_tensor_f32_dev(xt.data_ptr(), q.data_ptr(), x.size, pbuf.data_ptr()) == 0
    assert lib.dequantize_tensor_f32_dev(q.data_ptr(), d.data_ptr(), x.size, pbuf.data_ptr()) == 0
    pn.synchronize()
    want_p = ora.calibrate(x, False)
    want_q = ora.quantize(x, want_p)
    same_bits(q.cpu().numpy(), want_q)
    same_bits(d.cpu().numpy(), ora.dequantize(want_q, want_p, np.float32))
    raw = pbuf.cpu().numpy().tobytes()
    got_p = pn.core.QuantParamsC.from_buffer_copy(raw)
    _params_equal(got_p, want_p)


def test_errors(pn):
    p = pn.core.QuantParamsC()
    x = np.zeros(4, dtype=np.float64)
    assert pn.core._lib.calibrate_minmax(None, 4, 1, ctypes.byref(p)) == -1
    assert pn.core._lib.calibrate_minmax(x.ctypes.data, 0, 1, ctypes.byref(p)) == -1
    assert pn.core._lib.quantize_tensor(x.ctypes.data, None, 4, ctypes.byref(p)) == -1
    assert pn.core._lib.quantization_error(x.ctypes.data, 0, ctypes.byref(p)) == -1.0


def test_quantizer_class(pn, ora):
    x = np.random.default_rng(2).normal(size=1000)
    qz = pn.Quantizer(symmetric=True)
    qz.calibrate(x.ctypes.data, x.size)
    q = np.frombuffer(bytes(qz.quantize(x.ctypes.data, x.size)), dtype=np.int8)
    same_bits(q, ora.quantize(x, ora.calibrate(x, True)))
    r = np.frombuffer(bytes(qz.dequantize(q.ctypes.data, x.size)), dtype=np.float64)
    same_bits(r, ora.dequantize(q, ora.calibrate(x, True)))
    assert qz.snr(x.ctypes.data, x.size) > 30


@pytest.mark.parametrize("first_zero", [0.0, -0.0])
def test_calibrate_zero_extremes_large(pn, ora, first_zero):
    """min (or max) is a zero in a tensor split over many blocks: the loop keeps
    the FIRST zero, so its sign decides min_val / max_val bit for bit."""
    rng = np.random.default_rng(21)
    n = (1 << 22) + 3
    x = np.abs(rng.laplace(0, 1, n)).astype(np.float32) + np.float32(0.5)
    zi = np.sort(rng.choice(n, 64, replace=False))
    x[zi] = np.where(np.arange(64) % 2 == 0, -0.0, 0.0).astype(np.float32)
    x[zi[0]] = first_zero
    for sym in (True, False):
        _params_equal(_calib(pn, x, sym), ora.calibrate(x, sym))
    y = -x  # now the max is the zero
    for sym in (True, False):
        _params_equal(_calib(pn, y, sym), ora.calibrate(y, sym))
    y[rng.choice(n, 10, replace=False)] = np.nan  # NaNs after x0 are skipped
    _params_equal(_calib(pn, y, False), ora.calibrate(y, False))
