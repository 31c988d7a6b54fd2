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


@pytest.mark.parametrize("n", [1, 3, 4, 255, 256, 257, 1027, 4 * 256 * 4 + 8, (1 << 20) + 5])
def test_f64_quantize_dequantize_sizes(pn, ora, n):
    """The double API's kernels regroup a wave's 256 elements through lane
    shuffles (16-byte accesses contiguous per instruction): every size around
    a unit (4), a wave (256) and a 4-unit tile, host and device buffers,
    bit-exact against the oracle."""
    import torch
    rng = np.random.default_rng(n)
    x = rng.laplace(0, 1, n)
    x[rng.integers(0, n, max(1, n // 100))] = 50.0
    for sym in (True, False):
        p = _calib(pn, x, sym)
        want = ora.calibrate(x, sym)
        _params_equal(p, want)
        q = _quant(pn, x, p)
        same_bits(q, ora.quantize(x, want))
        d = np.empty(n)
        assert pn.core._lib.dequantize_tensor(q.ctypes.data, d.ctypes.data, n, ctypes.byref(p)) == 0
        same_bits(d, ora.dequantize(q, want))
    # device pointers, an offset of 16 bytes (still 16-byte aligned) so the
    # wave-contiguous kernels run on a start that is not a multiple of 256
    xd = torch.from_numpy(np.concatenate([np.zeros(2), x])).cuda()
    qd = torch.zeros(n + 4, dtype=torch.int8, device="cuda")
    dd = torch.full((n + 2,), -7.0, dtype=torch.float64, device="cuda")
    assert pn.core._lib.quantize_tensor(xd.data_ptr() + 16, qd.data_ptr() + 4, n, ctypes.byref(p)) == 0
    assert pn.core._lib.dequantize_tensor(qd.data_ptr() + 4, dd.data_ptr() + 16, n, ctypes.byref(p)) == 0
    torch.cuda.synchronize()
    qh, dh = qd.cpu().numpy(), dd.cpu().numpy()
    same_bits(qh[4:], ora.quantize(x, want))
    assert not qh[:4].any()
    same_bits(dh[2:], ora.dequantize(qh[4:].copy(), want))
    assert (dh[:2] == -7.0).all()


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


# ---- quantized_matmul (quantize.c:191-214) on the matrix cores ---------------------

def _qmm_params(ora, za, zb):
    pa, pb = ora.QuantParams(), ora.QuantParams()
    pa.scale, pa.zero_point = 0.0123, za
    pb.scale, pb.zero_point = 3.7e-3, zb
    return pa, pb


@pytest.mark.parametrize("m,k,n", [(1, 1, 1), (3, 5, 7), (128, 128, 128), (130, 257, 129), (64, 4096, 64),
                                   (257, 33, 1000), (300, 1000, 500), (256, 64, 260), (512, 192, 3)])
@pytest.mark.parametrize("za,zb", [(0, 0), (-128, 127), (17, -3)])
def test_quantized_matmul_bit_exact(pn, ora, m, k, n, za, zb):
    rng = np.random.default_rng(m + 7 * k + 13 * n + za + 1000)
    a = rng.integers(-128, 128, (m, k), dtype=np.int64).astype(np.int8)
    b = rng.integers(-128, 128, (k, n), dtype=np.int64).astype(np.int8)
    pa, pb = _qmm_params(ora, za, zb)
    got = np.empty((m, n))
    lib = pn.core._lib
    qa, qb = pn.core.QuantParamsC(), pn.core.QuantParamsC()
    ctypes.memmove(ctypes.byref(qa), ctypes.byref(pa), ctypes.sizeof(qa))
    ctypes.memmove(ctypes.byref(qb), ctypes.byref(pb), ctypes.sizeof(qb))
    assert lib.quantized_matmul(a.ctypes.data, b.ctypes.data, got.ctypes.data, m, k, n, ctypes.byref(qa),
                                ctypes.byref(qb)) == 0
    rc, want = ora.quantized_matmul(a, b, m, k, n, pa, pb)
    assert rc == 0
    same_bits(got.reshape(-1), want.reshape(-1))


def test_quantized_matmul_device_wrap_and_errors(pn, ora):
    import torch
    lib = pn.core._lib
    # device pointers
    rng = np.random.default_rng(5)
    m, k, n = 200, 3000, 150
    a = rng.integers(-128, 128, (m, k), dtype=np.int64).astype(np.int8)
    b = rng.integers(-128, 128, (k, n), dtype=np.int64).astype(np.int8)
    pa, pb = _qmm_params(ora, -5, 9)
    qa, qb = pn.core.QuantParamsC(), pn.core.QuantParamsC()
    ctypes.memmove(ctypes.byref(qa), ctypes.byref(pa), ctypes.sizeof(qa))
    ctypes.memmove(ctypes.byref(qb), ctypes.byref(pb), ctypes.sizeof(qb))
    da, db = torch.from_numpy(a).cuda(), torch.from_numpy(b).cuda()
    dc = torch.empty(m, n, dtype=torch.float64, device="cuda")
    torch.cuda.synchronize()
    assert lib.quantized_matmul(da.data_ptr(), db.data_ptr(), dc.data_ptr(), m, k, n, ctypes.byref(qa),
                                ctypes.byref(qb)) == 0
    torch.cuda.synchronize()
    same_bits(dc.cpu().numpy().reshape(-1), ora.quantized_matmul(a, b, m, k, n, pa, pb)[1].reshape(-1))
    # A in the padded shape (256 x 128) used in place, or copied when it sits
    # at an address that is not 16-byte aligned; B at an odd address (byte
    # loads in the transpose) or aligned with N a multiple of 4 (4-byte loads)
    m3, k3, n3 = 256, 128, 12
    a3 = rng.integers(-128, 128, (m3, k3), dtype=np.int64).astype(np.int8)
    b3 = rng.integers(-128, 128, (k3, n3), dtype=np.int64).astype(np.int8)
    want3 = ora.quantized_matmul(a3, b3, m3, k3, n3, pa, pb)[1].reshape(-1)
    for off in (0, 1):
        ha = np.zeros(m3 * k3 + 16, dtype=np.int8)
        hb = np.zeros(k3 * n3 + 16, dtype=np.int8)
        ha[off:off + m3 * k3] = a3.reshape(-1)
        hb[off:off + k3 * n3] = b3.reshape(-1)
        da3, db3 = torch.from_numpy(ha).cuda(), torch.from_numpy(hb).cuda()
        dc3 = torch.empty(m3, n3, dtype=torch.float64, device="cuda")
        torch.cuda.synchronize()
        assert lib.quantized_matmul(da3.data_ptr() + off, db3.data_ptr() + off, dc3.data_ptr(), m3, k3, n3,
                                    ctypes.byref(qa), ctypes.byref(qb)) == 0
        torch.cuda.synchronize()
        same_bits(dc3.cpu().numpy().reshape(-1), want3)
    # a sum past int32 wraps mod 2^32, as in the compiled reference
    k2 = 40_000
    a2 = np.full((3, k2), -128, dtype=np.int8)
    a2[1, ::3] = 100
    b2 = np.full((k2, 5), 127, dtype=np.int8)
    b2[::7, 2] = -77
    p1, p2 = _qmm_params(ora, 127, -128)
    q1, q2 = pn.core.QuantParamsC(), pn.core.QuantParamsC()
    ctypes.memmove(ctypes.byref(q1), ctypes.byref(p1), ctypes.sizeof(q1))
    ctypes.memmove(ctypes.byref(q2), ctypes.byref(p2), ctypes.sizeof(q2))
    got = np.empty((3, 5))
    assert lib.quantized_matmul(a2.ctypes.data, b2.ctypes.data, got.ctypes.data, 3, k2, 5, ctypes.byref(q1),
                                ctypes.byref(q2)) == 0
    same_bits(got.reshape(-1), ora.quantized_matmul(a2, b2, 3, k2, 5, p1, p2)[1].reshape(-1))
    # the Python layer (reference quantize.py:195-223): ctypes arrays in, ctypes float64 array out
    ca = (ctypes.c_int8 * (m * k)).from_buffer_copy(a.tobytes())
    cb = (ctypes.c_int8 * (k * n)).from_buffer_copy(b.tobytes())
    P = pn.QuantParams(scale=pa.scale, zero_point=pa.zero_point)
    Q = pn.QuantParams(scale=pb.scale, zero_point=pb.zero_point)
    out = pn.quantized_matmul(ca, cb, m, k, n, P, Q)
    same_bits(np.frombuffer(out, dtype=np.float64), ora.quantized_matmul(a, b, m, k, n, pa, pb)[1].reshape(-1))
    # errors (0 / -1 like the reference)
    assert lib.quantized_matmul(None, b.ctypes.data, got.ctypes.data, m, k, n, ctypes.byref(qa), ctypes.byref(qb)) == -1
    assert lib.quantized_matmul(a.ctypes.data, b.ctypes.data, got.ctypes.data, 0, k, n, ctypes.byref(qa),
                                ctypes.byref(qb)) == -1
    assert lib.quantized_matmul(a.ctypes.data, b.ctypes.data, got.ctypes.data, m, k, n, None, ctypes.byref(qb)) == -1


def test_quantized_matmul_long_k_and_size_limit(pn, ora):
    """K past 65535 16-byte units (the B pass loops over its K units) is
    computed like the reference; M beyond 65535 row tiles (8,388,480) is
    refused with -1 and NEURAL_ERR_TENSOR_TOO_LARGE before any access."""
    import torch
    lib = pn.core._lib
    rng = np.random.default_rng(33)
    m, k, n = 2, (1 << 20) + 17, 3
    a = rng.integers(-128, 128, (m, k), dtype=np.int8)
    b = rng.integers(-128, 128, (k, n), dtype=np.int8)
    pa, pb = ora.QuantParams(), ora.QuantParams()
    pa.scale, pa.zero_point, pb.scale, pb.zero_point = 0.01, 3, 0.02, -5
    qa, qb = pn.core.QuantParamsC(), pn.core.QuantParamsC()
    ctypes.memmove(ctypes.byref(qa), ctypes.byref(pa), ctypes.sizeof(qa))
    ctypes.memmove(ctypes.byref(qb), ctypes.byref(pb), ctypes.sizeof(qb))
    got = np.empty((m, n))
    assert lib.quantized_matmul(a.ctypes.data, b.ctypes.data, got.ctypes.data, m, k, n, ctypes.byref(qa),
                                ctypes.byref(qb)) == 0
    same_bits(got.reshape(-1), ora.quantized_matmul(a, b, m, k, n, pa, pb)[1].reshape(-1))
    dummy = torch.zeros(16, dtype=torch.int8, device="cuda")
    big_m = 65535 * 128 + 1
    assert lib.quantized_matmul(dummy.data_ptr(), dummy.data_ptr(), dummy.data_ptr(), big_m, 1, 1, ctypes.byref(qa),
                                ctypes.byref(qb)) == -1
    assert lib.neural_get_last_error() == pn.NeuralError.TENSOR_TOO_LARGE


# ---- calibrate_percentile (quantize.c:89-132): radix select on the device -----------

def _qp_bits(p):
    return (np.float64(p.scale).view(np.uint64), p.zero_point, np.float64(p.min_val).view(np.uint64),
            np.float64(p.max_val).view(np.uint64), p.symmetric)


@pytest.mark.parametrize("sym", [0, 1])
def test_calibrate_percentile_bit_exact(pn, ora, sym):
    lib = pn.core._lib
    rng = np.random.default_rng(23)
    zeros = np.where(rng.random(3000) < 0.5, -0.0, 0.0)
    cases = [rng.normal(0, 3, 100_003), rng.integers(-5, 6, 5000).astype(np.float64), np.array([2.5]),
             np.array([1.0, -1.0]), np.concatenate([zeros, rng.normal(0, 1, 60)]),
             np.concatenate([-np.abs(rng.normal(0, 1, 40)), zeros, np.abs(rng.normal(0, 1, 40))]),
             rng.permutation(np.concatenate([zeros, rng.normal(0, 1, 200)])),
             np.array([np.inf, -np.inf, 1e308, -1e308, 5e-324, -5e-324, 0.0, -0.0] * 50),
             rng.laplace(0, 1, 1 << 20)]
    for x in cases:
        for p in [0.01, 0.05, 0.25, 0.5, 0.0, -1.0, 0.7, 1e-9]:
            got = pn.core.QuantParamsC()
            assert lib.calibrate_percentile(x.ctypes.data, x.size, ctypes.c_double(p), sym, ctypes.byref(got)) == 0
            rc, want = ora.calibrate_percentile(x, p, sym)
            assert rc == 0
            assert _qp_bits(got) == _qp_bits(want), (x.size, p, got.min_val, want.min_val)


def test_calibrate_percentile_device_python_and_errors(pn, ora):
    import torch
    lib = pn.core._lib
    rng = np.random.default_rng(29)
    x = rng.normal(0, 1, (1 << 24) + 17)
    x[::1000] = 0.0
    x[5::1000] = -0.0
    xd = torch.from_numpy(x).cuda()
    torch.cuda.synchronize()
    for p in [0.001, 0.3]:
        got = pn.core.QuantParamsC()
        assert lib.calibrate_percentile(xd.data_ptr(), x.size, ctypes.c_double(p), 0, ctypes.byref(got)) == 0
        assert _qp_bits(got) == _qp_bits(ora.calibrate_percentile(x, p, 0)[1])
    # a selected rank inside a long run of mixed-sign zeros (device pointer)
    z = np.where(rng.random(1 << 20) < 0.5, -0.0, 0.0)
    zd = torch.from_numpy(z).cuda()
    torch.cuda.synchronize()
    for p in [0.01, 0.2, 0.45]:
        got = pn.core.QuantParamsC()
        assert lib.calibrate_percentile(zd.data_ptr(), z.size, ctypes.c_double(p), 0, ctypes.byref(got)) == 0
        assert _qp_bits(got) == _qp_bits(ora.calibrate_percentile(z, p, 0)[1])
    # the Python Quantizer (reference quantize.py:76-105)
    q = pn.Quantizer(symmetric=False, percentile=0.02)
    params = q.calibrate(x.ctypes.data, x.size)
    want = ora.calibrate_percentile(x, 0.02, 0)[1]
    assert (params.scale, params.zero_point, params.min_val, params.max_val) == \
        (want.scale, want.zero_point, want.min_val, want.max_val)
    # errors: NULL, n <= 0, NaN percentile (the reference indexes out of bounds there)
    got = pn.core.QuantParamsC()
    assert lib.calibrate_percentile(None, 10, ctypes.c_double(0.01), 0, ctypes.byref(got)) == -1
    assert lib.calibrate_percentile(x.ctypes.data, 0, ctypes.c_double(0.01), 0, ctypes.byref(got)) == -1
    assert lib.calibrate_percentile(x.ctypes.data, 10, ctypes.c_double(float("nan")), 0, ctypes.byref(got)) == -1


def test_calibrate_percentile_ordered_and_duplicate_inputs(pn, ora):
    """Inputs whose matches come in long runs (sorted, reversed) or never
    thin out (few distinct values), where copying the matching keys out of the
    data overflows a block's region or never starts."""
    import torch
    lib = pn.core._lib
    rng = np.random.default_rng(31)
    base = rng.normal(0, 1, (1 << 23) + 3)
    cases = [np.sort(base), np.sort(base)[::-1].copy(), rng.integers(0, 3, 1 << 22).astype(np.float64),
             np.full(70_001, -1.5), np.concatenate([np.sort(base[: 1 << 20]), rng.normal(0, 1, 1 << 20)])]
    for x in cases:
        xd = torch.from_numpy(x).cuda()
        torch.cuda.synchronize()
        for p in [0.01, 0.1, 0.5]:
            for sym in (0, 1):
                got = pn.core.QuantParamsC()
                assert lib.calibrate_percentile(xd.data_ptr(), x.size, ctypes.c_double(p), sym, ctypes.byref(got)) == 0
                assert _qp_bits(got) == _qp_bits(ora.calibrate_percentile(x, p, sym)[1]), (x.size, p, sym)


def test_calibrate_percentile_full_size_vs_stable_sort(pn):
    """64 M doubles (the size the library is measured at): the selected order
    statistics equal a stable device sort's elements at lo = (int64)(n p) and
    hi = (int64)(n (1 - p)) bit for bit -- a stable sort keeps equal values
    (+0 / -0 included) in input order, as the reference's qsort (glibc's
    merge sort) does -- and the affine parameters follow from them."""
    import torch
    lib = pn.core._lib
    n = 1 << 26
    g = torch.Generator(device="cuda")
    g.manual_seed(37)
    # N(1, 3) with 2% +0 and 2% -0: the zeros fill sorted ranks ~[0.355, 0.395] n,
    # so p = 0.37 selects a zero (its sign: input order) and a positive value
    x = torch.randn(n, device="cuda", dtype=torch.float64, generator=g) * 3 + 1
    x[torch.randperm(n, device="cuda", generator=g)[: n // 50]] = 0.0
    x[torch.randperm(n, device="cuda", generator=g)[: n // 50]] = -0.0
    srt = torch.sort(x, stable=True).values
    torch.cuda.synchronize()
    assert float(srt[int(n * 0.37)]) == 0.0
    for p in (0.001, 0.01, 0.3, 0.37):
        lo, hi = int(n * p), int(n * (1.0 - p))
        got = pn.core.QuantParamsC()
        assert lib.calibrate_percentile(x.data_ptr(), n, ctypes.c_double(p), 0, ctypes.byref(got)) == 0
        want_lo, want_hi = float(srt[lo]), float(srt[hi])
        assert np.float64(got.min_val).view(np.uint64) == np.float64(want_lo).view(np.uint64), (p, got.min_val, want_lo)
        assert np.float64(got.max_val).view(np.uint64) == np.float64(want_hi).view(np.uint64), (p, got.max_val, want_hi)
        scale = (want_hi - want_lo) / 255.0
        assert got.scale == scale


def test_quantized_matmul_full_size_vs_exact_f64(pn):
    """4096^3 (the size the product is measured at): every inner sum
    sum_k (A - za)(B - zb) is an integer below 2^31 here (|terms| <= 255 * 255,
    K = 4096: < 2.7e8), so a float64 device product of the shifted operands is
    exact in any summation order; C must equal that sum * (sa * sb) bit for
    bit, as quantize.c:191-214 forms it."""
    import torch
    lib = pn.core._lib
    m = k = n = 4096
    g = torch.Generator(device="cuda")
    g.manual_seed(43)
    a = torch.randint(-128, 128, (m, k), dtype=torch.int8, device="cuda", generator=g)
    b = torch.randint(-128, 128, (k, n), dtype=torch.int8, device="cuda", generator=g)
    c = torch.empty(m, n, dtype=torch.float64, device="cuda")
    pa, pb = pn.core.QuantParamsC(), pn.core.QuantParamsC()
    pa.scale, pa.zero_point, pb.scale, pb.zero_point = 0.013, -7, 0.37, 11
    torch.cuda.synchronize()
    assert lib.quantized_matmul(a.data_ptr(), b.data_ptr(), c.data_ptr(), m, k, n, ctypes.byref(pa),
                                ctypes.byref(pb)) == 0
    torch.cuda.synchronize()
    exact = torch.matmul(a.double() - pa.zero_point, (b.double() - pb.zero_point).contiguous())
    want = exact * (pa.scale * pb.scale)
    assert torch.equal(c, want)
