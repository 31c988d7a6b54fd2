"""Pin the oracle to the reference's own C, compiled unchanged from the
reference tree into oracle/_ref/libneural_ref.so (oracle/Makefile).

Bit-for-bit on random and special inputs: activations_c.c (all ten act_*,
f32 and f64 tensors), quantize.c (calibrate_minmax, quantize_tensor,
dequantize_tensor, quantization_error/_snr, including NaN / Inf / huge
values), optimizers_c.c (SGD / Adam / AdamW steps, f32 and f64, and the
OPTS blob), tensor_ops.c (concat / split / pad / transpose and their -1
argument checks) and the log-softmax of metrics_losses.c:47-64 (through
label_smoothing_ce_forward with smoothing 0, which returns exactly
-log_softmax[target]).
"""

import ctypes

import numpy as np
import pytest

from conftest import same_bits

ACT_ALPHA = {"leaky_relu": 0.01, "elu": 1.0}
ACTS = ["tanh", "gelu", "leaky_relu", "elu", "selu", "swish", "mish", "hardswish", "softplus", "hardtanh"]


class TensorC(ctypes.Structure):
    """The 40-byte prefix of the reference descriptor (activations_c.c:36-43)."""
    _fields_ = [("data", ctypes.c_void_p), ("ndim", ctypes.c_int64), ("shape", ctypes.POINTER(ctypes.c_int64)),
                ("stride", ctypes.c_void_p), ("dtype", ctypes.c_int32), ("flags", ctypes.c_int32)]


def tensor_c(arr, keep):
    shape = (ctypes.c_int64 * arr.ndim)(*arr.shape)
    keep.append(shape)
    return TensorC(arr.ctypes.data, arr.ndim, shape, None, 0 if arr.dtype == np.float32 else 1, 0)


@pytest.fixture(scope="module")
def ref(ora):
    r = ora.ref()
    if r is None:
        pytest.skip("oracle/_ref not built (reference sources absent)")
    return r


def act_inputs(dt):
    rng = np.random.default_rng(44)
    x = rng.normal(0, 4, 200000)
    x[rng.choice(x.size, 2000, replace=False)] = 30.0
    x[rng.choice(x.size, 2000, replace=False)] = -30.0
    x[:14] = [0.0, -0.0, 3.0, -3.0, 1.0, -1.0, 1e-310, -700.0, 710.0, -1e-5, np.nan, np.inf, -np.inf, 20.0]
    return x.astype(dt)


@pytest.mark.parametrize("name", ACTS)
@pytest.mark.parametrize("dt", [np.float32, np.float64])
def test_activations_bit_exact(ora, ref, name, dt):
    x = act_inputs(dt)
    out = np.empty_like(x)
    keep = []
    ti, to = tensor_c(x, keep), tensor_c(out, keep)
    fn = getattr(ref, "act_" + name)
    if name in ACT_ALPHA:
        fn.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_double]
        assert fn(ctypes.addressof(to), ctypes.addressof(ti), ACT_ALPHA[name]) == 0
    else:
        fn.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        assert fn(ctypes.addressof(to), ctypes.addressof(ti)) == 0
    same_bits(ora.act(name, x, ACT_ALPHA.get(name, 0.0)), out)


def _ref_params(ref, x, sym):
    p = ora_qp()
    ref.calibrate_minmax.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_void_p]
    assert ref.calibrate_minmax(x.ctypes.data, x.size, 1 if sym else 0, ctypes.byref(p)) == 0
    return p


def ora_qp():
    import ora
    return ora.QuantParams()


def _params_bytes(p):
    return bytes(memoryview(p))


def quant_inputs():
    rng = np.random.default_rng(5)
    x = rng.laplace(0, 1, 100000)
    x[rng.choice(x.size, 100, replace=False)] = 50.0
    x[rng.choice(x.size, 100, replace=False)] = -50.0
    return x


@pytest.mark.parametrize("sym", [True, False])
def test_quantize_bit_exact(ora, ref, sym):
    x = quant_inputs()
    rp = _ref_params(ref, x, sym)
    op = ora.calibrate(x, sym)
    assert _params_bytes(rp)[:12] == _params_bytes(op)[:12]  # scale + zero_point
    assert (rp.min_val, rp.max_val, rp.symmetric) == (op.min_val, op.max_val, op.symmetric)
    # f32 input widened to double gives the same params as the double API
    x32 = x.astype(np.float32)
    p32 = ora.calibrate(x32, sym)
    rp32 = _ref_params(ref, x32.astype(np.float64), sym)
    assert (p32.scale, p32.zero_point, p32.min_val, p32.max_val) == (rp32.scale, rp32.zero_point, rp32.min_val,
                                                                     rp32.max_val)
    q = np.empty(x.size, dtype=np.int8)
    ref.quantize_tensor.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p]
    assert ref.quantize_tensor(x.ctypes.data, q.ctypes.data, x.size, ctypes.byref(rp)) == 0
    same_bits(ora.quantize(x, op), q)
    d = np.empty(x.size)
    ref.dequantize_tensor.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p]
    assert ref.dequantize_tensor(q.ctypes.data, d.ctypes.data, x.size, ctypes.byref(rp)) == 0
    same_bits(ora.dequantize(q, op), d)
    ref.quantization_error.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p]
    ref.quantization_snr.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p]
    assert ora.quant_error(x, op) == ref.quantization_error(x.ctypes.data, x.size, ctypes.byref(rp))
    assert ora.quant_snr(x, op) == ref.quantization_snr(x.ctypes.data, x.size, ctypes.byref(rp))


def test_quantize_special_values_bit_exact(ora, ref):
    """NaN, +-Inf and values beyond int32 after scaling: the reference's
    (int32_t)round() is x86 cvttsd2si (INT32_MIN), then a wrapping add."""
    x = np.array([0.3, np.nan, np.inf, -np.inf, 1e30, -1e30, 0.0, -0.0, 2.5, -2.5, 3.5, -3.5, 1e9, -1e9])
    ref.quantize_tensor.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p]
    for zp in (-128, -1, 0, 1, 127):
        for scale in (0.5, 1e-3, 7.0):
            p = ora_qp()
            p.scale, p.zero_point = scale, zp
            q = np.empty(x.size, dtype=np.int8)
            assert ref.quantize_tensor(x.ctypes.data, q.ctypes.data, x.size, ctypes.byref(p)) == 0
            same_bits(ora.quantize(x, p), q)
    for data in ([np.nan, 1.0, -2.0], [5.0, 5.0, 5.0], [0.0, -0.0, 0.0], [-0.0, 0.0], [1e-40, -1e-40],
                 [3.0, np.nan, -7.0, np.inf]):
        a = np.array(data)
        for sym in (True, False):
            rp, op = _ref_params(ref, a, sym), ora.calibrate(a, sym)
            for f in ("scale", "min_val", "max_val"):
                rv, ov = getattr(rp, f), getattr(op, f)
                assert (np.isnan(rv) and np.isnan(ov)) or np.float64(rv).tobytes() == np.float64(ov).tobytes()
            assert rp.zero_point == op.zero_point and rp.symmetric == op.symmetric


@pytest.mark.parametrize("kind", ["sgd", "adam", "adamw"])
@pytest.mark.parametrize("dt", [np.float32, np.float64])
def test_optimizers_bit_exact(ora, ref, kind, dt):
    rng = np.random.default_rng(6)
    n = 10007
    p = rng.normal(0, 0.02, n).astype(dt)
    g = rng.normal(0, 1e-3, n).astype(dt)
    g[[3, 50, 900]] = [np.nan, np.inf, -np.inf]
    rp = p.copy()
    keep = []
    tp, tg = tensor_c(rp, keep), tensor_c(g, keep)
    lr, b1, b2, eps, wd, mom = 1e-3, 0.9, 0.999, 1e-8, 0.01, 0.9
    h = {"sgd": lambda: ref.opt_sgd_create(lr, mom), "adam": lambda: ref.opt_adam_create(lr, b1, b2, eps),
         "adamw": lambda: ref.opt_adamw_create(lr, b1, b2, eps, wd)}[kind]()
    pp = (ctypes.c_void_p * 1)(ctypes.addressof(tp))
    gp = (ctypes.c_void_p * 1)(ctypes.addressof(tg))
    op = p.copy()
    m, v = np.zeros(n), np.zeros(n)
    for t in range(1, 5):
        assert ref.opt_step(h, pp, gp, 1) == 0
        if kind == "sgd":
            ora.sgd_step(op, g, m, lr, mom)
        elif kind == "adam":
            ora.adam_step(op, g, m, v, lr, b1, b2, eps, t)
        else:
            ora.adamw_step(op, g, m, v, lr, b1, b2, eps, wd, t)
    same_bits(op, rp)
    nb = ref.opt_state_bytes(h)
    buf = (ctypes.c_uint8 * nb)()
    assert ref.opt_state_export(h, buf, nb) == 0
    blob = bytes(buf)
    off = 88
    same_bits(np.frombuffer(blob[off:off + 8 * n], dtype=np.float64), m)
    if kind != "sgd":
        same_bits(np.frombuffer(blob[off + 8 * n:off + 16 * n], dtype=np.float64), v)
    ref.opt_free(h)


def test_log_softmax_through_ce(ora, ref):
    rng = np.random.default_rng(7)
    K = 37
    x = rng.normal(0, 3, (4, K))
    x[1, 5] = 40.0
    got = ora.softmax_rows(x, log=True)
    fn = ref.label_smoothing_ce_forward
    fn.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64, ctypes.c_double, ctypes.c_void_p]
    for i in range(4):
        row = np.ascontiguousarray(x[i:i + 1])
        for c in range(K):
            tgt = np.array([c], dtype=np.int64)
            loss = ctypes.c_double()
            assert fn(row.ctypes.data, tgt.ctypes.data, 1, K, 0.0, ctypes.byref(loss)) == 0
            assert np.float64(-loss.value).tobytes() == np.float64(got[i, c]).tobytes()


def test_tensor_ops_bit_exact(ora, ref):
    rng = np.random.default_rng(8)
    d = ctypes.c_double
    i64 = ctypes.c_int64
    P = ctypes.c_void_p
    ref.tensor_concat_2d.argtypes = [P, P, i64, i64, i64, i64, i64, P, P, P]
    ref.tensor_split_2d.argtypes = [P, i64, i64, i64, i64, P, P, P, P, P, P]
    ref.tensor_pad_2d.argtypes = [P, i64, i64, i64, i64, i64, i64, d, P, P, P]
    ref.tensor_transpose2d_array.argtypes = [P, i64, i64, P]
    a, b = rng.normal(size=12), rng.normal(size=6)
    for (ra, ca, rb, cb, ax) in [(3, 4, 3, 2, 1), (3, 4, 2, 4, 0), (2, 6, 3, 2, 1), (0, 4, 3, 4, 0), (3, 4, 3, 4, 2)]:
        bb = rng.normal(size=max(rb * cb, 1))
        aa = rng.normal(size=max(ra * ca, 1))
        out = np.zeros(64)
        r, c = i64(), i64()
        rc = ref.tensor_concat_2d(aa.ctypes.data, bb.ctypes.data, ra, ca, rb, cb, ax, out.ctypes.data,
                                  ctypes.byref(r), ctypes.byref(c))
        orc, oo, orr, occ = ora.concat_2d(aa, bb, ra, ca, rb, cb, ax)
        assert rc == orc
        if rc == 0:
            assert (r.value, c.value) == (orr, occ)
            same_bits(oo, out[: r.value * c.value])
    x = rng.normal(size=35)
    for ax, sp in [(0, 2), (1, 3), (0, 0), (1, 7), (2, 1)]:
        oa, ob = np.zeros(35), np.zeros(35)
        dims = [i64() for _ in range(4)]
        rc = ref.tensor_split_2d(x.ctypes.data, 5, 7, ax, sp, oa.ctypes.data, ob.ctypes.data,
                                 *[ctypes.byref(q) for q in dims])
        orc, wa, wb, odims = ora.split_2d(x, 5, 7, ax, sp)
        assert rc == orc
        if rc == 0:
            assert tuple(q.value for q in dims) == odims
            same_bits(wa, oa[: wa.size])
            same_bits(wb, ob[: wb.size])
    for pads in [(1, 2, 3, 0), (0, 0, 0, 0), (-1, 0, 0, 0)]:
        R, C = 5 + max(pads[0], 0) + pads[1], 7 + pads[2] + pads[3]
        out = np.zeros(max(R * C, 1))
        r, c = i64(), i64()
        rc = ref.tensor_pad_2d(x.ctypes.data, 5, 7, *pads, -1.5, out.ctypes.data, ctypes.byref(r), ctypes.byref(c))
        orc, oo, orr, occ = ora.pad_2d(x, 5, 7, *pads, -1.5)
        assert rc == orc
        if rc == 0:
            same_bits(oo, out[: R * C])
    out = np.zeros(35)
    assert ref.tensor_transpose2d_array(x.ctypes.data, 5, 7, out.ctypes.data) == 0
    rc, oo = ora.transpose_2d(x, 5, 7)
    same_bits(oo, out)


@pytest.mark.parametrize("m,k,n", [(1, 1, 1), (3, 5, 7), (16, 64, 9), (33, 130, 17)])
@pytest.mark.parametrize("za,zb", [(0, 0), (-128, 127), (17, -3)])
def test_quantized_matmul_matches_reference(ora, m, k, n, za, zb):
    """ora_quantized_matmul against quantize.c:191-214 compiled unchanged."""
    if ora.ref() is None:
        pytest.skip("reference C build (oracle/_ref) absent")
    rng = np.random.default_rng(m * 1000 + k + n)
    a = rng.integers(-128, 128, (m, k), dtype=np.int64).astype(np.int8)
    b = rng.integers(-128, 128, (k, n), dtype=np.int64).astype(np.int8)
    pa, pb = ora.QuantParams(), ora.QuantParams()
    pa.scale, pa.zero_point = 0.0123, za
    pb.scale, pb.zero_point = 3.7e-3, zb
    rc, got = ora.quantized_matmul(a, b, m, k, n, pa, pb)
    rc2, want = ora.quantized_matmul(a, b, m, k, n, pa, pb, use_ref=True)
    assert rc == 0 and rc2 == 0
    assert np.array_equal(got.view(np.uint64), want.view(np.uint64))
    # the closed form in exact integers when nothing overflows int32
    acc = (a.astype(np.int64) - za) @ (b.astype(np.int64) - zb)
    assert np.array_equal(got, acc.astype(np.float64) * (pa.scale * pb.scale))


def test_quantized_matmul_wraps_like_reference(ora):
    """A sum past int32 wraps mod 2^32 in the compiled reference and in the oracle."""
    if ora.ref() is None:
        pytest.skip("reference C build (oracle/_ref) absent")
    k = 40_000  # 40,000 x 255 x 255 > 2^31
    a = np.full((2, k), -128, dtype=np.int8)
    b = np.full((k, 3), 127, dtype=np.int8)
    pa, pb = ora.QuantParams(), ora.QuantParams()
    pa.scale, pa.zero_point = 1.0, 127
    pb.scale, pb.zero_point = 1.0, -128
    _, got = ora.quantized_matmul(a, b, 2, k, 3, pa, pb)
    _, want = ora.quantized_matmul(a, b, 2, k, 3, pa, pb, use_ref=True)
    assert np.array_equal(got, want)
    exact = -255 * 255 * k
    wrapped = (exact + 2 ** 31) % 2 ** 32 - 2 ** 31
    assert got[0, 0] == float(wrapped) and exact != wrapped
    # errors
    assert ora.quantized_matmul(a, b, 0, k, 3, pa, pb)[0] == -1


def _qp_tuple(p):
    return (np.float64(p.scale).view(np.uint64), p.zero_point, np.float64(p.min_val).view(np.uint64),
            np.float64(p.max_val).view(np.uint64), p.symmetric)


@pytest.mark.parametrize("sym", [0, 1])
def test_calibrate_percentile_matches_reference(ora, sym):
    """ora_calibrate_percentile against quantize.c:89-132 compiled unchanged,
    incl. percentiles outside [0, 0.5], ties and runs of +-0 at the selected ranks."""
    if ora.ref() is None:
        pytest.skip("reference C build (oracle/_ref) absent")
    rng = np.random.default_rng(17)
    zeros = np.where(rng.random(2000) < 0.5, -0.0, 0.0)
    cases = [rng.normal(0, 3, 100_003), rng.integers(-5, 6, 5000).astype(np.float64), np.array([2.5]),
             np.array([1.0, -1.0]), np.concatenate([zeros, rng.normal(0, 1, 50)]),
             np.concatenate([-np.abs(rng.normal(0, 1, 30)), zeros, np.abs(rng.normal(0, 1, 30))]),
             # infinite range: zero point from (int32)round(inf/inf), x86 INT32_MIN clamped to -128
             np.array([np.inf, -np.inf, 1e308, -1e308, 5e-324, -5e-324, 0.0, -0.0] * 50)]
    for x in cases:
        for p in [0.01, 0.05, 0.25, 0.5, 0.0, -1.0, 0.7, 1e-9]:
            rc, got = ora.calibrate_percentile(x, p, sym)
            rc2, want = ora.calibrate_percentile(x, p, sym, use_ref=True)
            assert rc == 0 and rc2 == 0
            assert _qp_tuple(got) == _qp_tuple(want), (x.size, p)
    assert ora.calibrate_percentile(np.ones(3), float("nan"), sym)[0] == -1


def _f32_quant_inputs(rng):
    """cfg4-shaped float32 data: Laplace(0,1), +-50 outliers (both signs, so
    min = -50 and max = +50 exactly), signed zeros and float32 denormals."""
    x = rng.laplace(0, 1, 100003).astype(np.float32)
    x[rng.choice(x.size, 120, replace=False)] = 50.0
    x[rng.choice(x.size, 120, replace=False)] = -50.0
    x[1:7] = [0.0, -0.0, 1e-45, -1e-45, 1.1754944e-38, -3.0e-39]
    return x


def _ref_call_f64(ref, name, *args):
    f = getattr(ref, name)
    f.argtypes = [ctypes.c_void_p] * 2 + [ctypes.c_int64, ctypes.c_void_p] if name in (
        "quantize_tensor", "dequantize_tensor") else [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p]
    return f(*args)


@pytest.mark.parametrize("sym", [True, False])
def test_f32_quant_variants_match_reference_on_widened_input(ora, ref, sym):
    """ora_calibrate_minmax_f32 / ora_quantize_f32 / ora_dequantize_f32 /
    ora_quant_error_f32 / ora_quant_snr_f32 against the reference's
    quantize.c:52-84,144-174,222-269 (compiled unchanged) run on the same
    values widened to double, which is exact: the reference API is
    double-in, double-out; the f32 entry points read floats and write
    (float) of the double result."""
    x32 = _f32_quant_inputs(np.random.default_rng(50 + sym))
    x64 = x32.astype(np.float64)
    rp = _ref_params(ref, x64, sym)
    op = ora.calibrate(x32, sym)
    assert _params_bytes(op) [:12] == _params_bytes(rp)[:12]
    assert (op.min_val, op.max_val, op.symmetric) == (rp.min_val, rp.max_val, rp.symmetric)
    # what the mathematics fixes: +-50 both present
    if sym:
        assert op.scale == 50.0 / 127.0 and op.zero_point == 0 and (op.min_val, op.max_val) == (-50.0, 50.0)
    else:
        assert op.scale == 100.0 / 255.0 and (op.min_val, op.max_val) == (-50.0, 50.0)
        v = -128.0 - (-50.0) / op.scale                    # C round(): half away from zero
        assert op.zero_point == int(np.copysign(np.floor(abs(v) + 0.5), v))
    q_ref = np.empty(x32.size, dtype=np.int8)
    assert _ref_call_f64(ref, "quantize_tensor", x64.ctypes.data, q_ref.ctypes.data, x64.size, ctypes.byref(rp)) == 0
    same_bits(ora.quantize(x32, op), q_ref)
    d_ref = np.empty(x32.size)
    assert _ref_call_f64(ref, "dequantize_tensor", q_ref.ctypes.data, d_ref.ctypes.data, x64.size,
                         ctypes.byref(rp)) == 0
    same_bits(ora.dequantize(q_ref, op, np.float32), d_ref.astype(np.float32))
    ref.quantization_error.restype = ctypes.c_double
    ref.quantization_snr.restype = ctypes.c_double
    e_ref = _ref_call_f64(ref, "quantization_error", x64.ctypes.data, x64.size, ctypes.byref(rp))
    s_ref = _ref_call_f64(ref, "quantization_snr", x64.ctypes.data, x64.size, ctypes.byref(rp))
    assert ora.quant_error(x32, op) == e_ref
    assert ora.quant_snr(x32, op) == s_ref
    # the error is bounded by the step: |x - deq(q(x))| <= scale/2 inside the range
    assert 0.0 < e_ref <= (op.scale / 2) ** 2


def test_f32_quant_variants_special_values_match_reference(ora, ref):
    """NaN, +-Inf, values whose scaled magnitude passes 2^31 (x86 cvttsd2si
    gives INT32_MIN, then the int32 add wraps), ties at .5, float32 extremes:
    the f32 variants equal the reference's double path on the widened
    values, for every zero point and several scales."""
    x32 = np.array([0.3, np.nan, np.inf, -np.inf, 3.4e38, -3.4e38, 0.0, -0.0, 2.5, -2.5, 3.5, -3.5, 1e9, -1e9,
                    1e-45, 50.0, -50.0, 127.5, -128.5], dtype=np.float32)
    x64 = x32.astype(np.float64)
    for zp in (-128, -1, 0, 1, 127):
        for scale in (0.5, 1e-3, 7.0, 50.0 / 127.0):
            p = ora_qp()
            p.scale, p.zero_point = scale, zp
            q = np.empty(x32.size, dtype=np.int8)
            assert _ref_call_f64(ref, "quantize_tensor", x64.ctypes.data, q.ctypes.data, x64.size,
                                 ctypes.byref(p)) == 0
            same_bits(ora.quantize(x32, p), q)
            d = np.empty(x32.size)
            assert _ref_call_f64(ref, "dequantize_tensor", q.ctypes.data, d.ctypes.data, x64.size,
                                 ctypes.byref(p)) == 0
            same_bits(ora.dequantize(q, p, np.float32), d.astype(np.float32))
            ref.quantization_error.restype = ctypes.c_double
            ref.quantization_snr.restype = ctypes.c_double
            for fn, name in ((ora.quant_error, "quantization_error"), (ora.quant_snr, "quantization_snr")):
                want = _ref_call_f64(ref, name, x64.ctypes.data, x64.size, ctypes.byref(p))
                got = fn(x32, p)
                assert (np.isnan(want) and np.isnan(got)) or want == got, (name, zp, scale, got, want)
            # finite-only inputs give a finite error that both sides agree on
            fin32 = x32[np.isfinite(x32)].copy()
            fin64 = fin32.astype(np.float64)
            want = _ref_call_f64(ref, "quantization_error", fin64.ctypes.data, fin64.size, ctypes.byref(p))
            assert ora.quant_error(fin32, p) == want
    # dequantize of every int8 code for an affine map: (float)((q - zp) * scale)
    qs = np.arange(-128, 128, dtype=np.int8)
    p = ora_qp()
    p.scale, p.zero_point = 0.0123, -7
    want = ((qs.astype(np.float64) + 7.0) * 0.0123).astype(np.float32)
    same_bits(ora.dequantize(qs, p, np.float32), want)
