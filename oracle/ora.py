"""
ctypes/numpy wrapper of the CPU oracle (liboracle.so) and of the reference's
own C compiled unchanged (_ref/libneural_ref.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, as the checker.  The product (libneural_hip.so,
pyneural) never loads it.
"""

import ctypes
import os
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ORACLE_SO = HERE / "liboracle.so"
CPU_SO = HERE / "libcpu_baseline.so"
REF_SO = HERE / "_ref" / "libneural_ref.so"

ADD, SUB, MUL, DIV, MAX = 0, 1, 2, 3, 4
ACTS = ["tanh", "gelu", "leaky_relu", "elu", "selu", "swish", "mish", "hardswish", "softplus", "hardtanh", "sigmoid"]
ACT_CODE = {name: i for i, name in enumerate(ACTS)}


class QuantParams(ctypes.Structure):
    _fields_ = [("scale", ctypes.c_double), ("zero_point", ctypes.c_int32), ("min_val", ctypes.c_double),
                ("max_val", ctypes.c_double), ("symmetric", ctypes.c_int)]


_lib = None
_ref = None


def lib():
    global _lib
    if _lib is None:
        if not ORACLE_SO.exists():
            raise RuntimeError(f"{ORACLE_SO} missing: run `make -C oracle`")
        _lib = ctypes.CDLL(str(ORACLE_SO))
        _lib.ora_sum_ref_f32.restype = ctypes.c_float
        _lib.ora_sum_ref_f64.restype = ctypes.c_double
        for n in ("ora_sum_exact_f32", "ora_sum_exact_f64", "ora_max_chain_f64", "ora_quant_error",
                  "ora_quant_snr", "ora_quant_error_f32", "ora_quant_snr_f32", "ora_bias_correction",
                  "ora_sumsq_exact_f32"):
            getattr(_lib, n).restype = ctypes.c_double
        _lib.ora_max_chain_f32.restype = ctypes.c_float
        _lib.ora_l2_ref_f32.restype = ctypes.c_float
        _lib.ora_argmax_f32.restype = ctypes.c_int64
        _lib.ora_argmax_f64.restype = ctypes.c_int64
        _lib.ora_bias_correction.argtypes = [ctypes.c_double, ctypes.c_int64]
    return _lib


def ref():
    """The reference's C (activations_c.c, quantize.c, optimizers_c.c,
    tensor_ops.c, metrics_losses.c, transforms.c) built by oracle/Makefile;
    None if absent."""
    global _ref
    if _ref is None and REF_SO.exists():
        _ref = ctypes.CDLL(str(REF_SO))
        _ref.quantization_error.restype = ctypes.c_double
        _ref.quantization_snr.restype = ctypes.c_double
        _ref.opt_sgd_create.restype = ctypes.c_void_p
        _ref.opt_adam_create.restype = ctypes.c_void_p
        _ref.opt_adamw_create.restype = ctypes.c_void_p
        _ref.opt_state_bytes.restype = ctypes.c_int64
        for n in ("opt_sgd_create", "opt_adam_create", "opt_adamw_create"):
            getattr(_ref, n).argtypes = [ctypes.c_double] * {"opt_sgd_create": 2, "opt_adam_create": 4,
                                                            "opt_adamw_create": 5}[n]
        _ref.opt_step.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64]
        _ref.opt_free.argtypes = [ctypes.c_void_p]
        _ref.opt_state_bytes.argtypes = [ctypes.c_void_p]
        _ref.opt_state_export.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64]
    return _ref


_cpu = None


def cpu():
    """The reference's host SIMD loops (cpu_baseline.c): AVX-256 ew_add /
    ew_mul / reduce_sum, the AVX-512 simd.asm path, the SSE L2 norm and the
    node_relu pass structure, for bench.py's CPU baseline."""
    global _cpu
    if _cpu is None:
        if not CPU_SO.exists():
            raise RuntimeError(f"{CPU_SO} missing: run `make -C oracle`")
        c = ctypes.CDLL(str(CPU_SO))
        P, I64 = ctypes.c_void_p, ctypes.c_int64
        for n in ("cpu_ew_add_avx", "cpu_ew_mul_avx", "cpu_simd_add_avx512", "cpu_simd_mul_avx512"):
            getattr(c, n).argtypes = [P, P, P, I64]
            getattr(c, n).restype = None
        for n in ("cpu_reduce_sum_avx", "cpu_simd_sum_avx512"):
            getattr(c, n).argtypes = [P, I64]
            getattr(c, n).restype = ctypes.c_float
        c.cpu_l2_sse.argtypes = [P, ctypes.c_uint64]
        c.cpu_l2_sse.restype = ctypes.c_float
        c.cpu_relu_node.argtypes = [P, P, I64]
        c.cpu_relu_node.restype = ctypes.c_int
        _cpu = c
    return _cpu


def cpu_binary(name, a, b, out=None):
    """cpu_ew_add_avx / cpu_ew_mul_avx / cpu_simd_add_avx512 / cpu_simd_mul_avx512."""
    out = np.empty_like(a) if out is None else out
    getattr(cpu(), name)(a.ctypes.data, b.ctypes.data, out.ctypes.data, a.size)
    return out


def cpu_sum(name, x):
    """cpu_reduce_sum_avx / cpu_simd_sum_avx512 (float result)."""
    return getattr(cpu(), name)(x.ctypes.data, x.size)


def cpu_l2(x):
    return cpu().cpu_l2_sse(x.ctypes.data, x.size)


def cpu_relu_node(x, out=None):
    out = np.empty_like(x) if out is None else out
    assert cpu().cpu_relu_node(x.ctypes.data, out.ctypes.data, x.size) == 0
    return out


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def _f64(x):
    return ctypes.c_double(float(x))


# ---- elementwise ----------------------------------------------------------------

def ew(op, a, b):
    out = np.empty_like(a)
    fn = lib().ora_ew_f32 if a.dtype == np.float32 else lib().ora_ew_f64
    fn(ctypes.c_int(op), _p(a), _p(b), _p(out), ctypes.c_int64(a.size))
    return out


def scalar(op, a, s):
    out = np.empty_like(a)
    fn = lib().ora_scalar_f32 if a.dtype == np.float32 else lib().ora_scalar_f64
    fn(ctypes.c_int(op), _p(a), _f64(s), _p(out), ctypes.c_int64(a.size))
    return out


def neg(a):
    out = np.empty_like(a)
    (lib().ora_neg_f32 if a.dtype == np.float32 else lib().ora_neg_f64)(_p(a), _p(out), ctypes.c_int64(a.size))
    return out


def relu(a):
    out = np.empty_like(a)
    (lib().ora_relu_f32 if a.dtype == np.float32 else lib().ora_relu_f64)(_p(a), _p(out), ctypes.c_int64(a.size))
    return out


def bias_add(x, b):
    rows, cols = x.shape
    out = np.empty_like(x)
    fn = lib().ora_bias_add_f32 if x.dtype == np.float32 else lib().ora_bias_add_f64
    fn(_p(x), _p(b), _p(out), ctypes.c_int64(rows), ctypes.c_int64(cols))
    return out


# ---- reductions -------------------------------------------------------------------

def sum_ref(x):
    f = lib().ora_sum_ref_f32 if x.dtype == np.float32 else lib().ora_sum_ref_f64
    return f(_p(x), ctypes.c_int64(x.size))


def sum_exact(x):
    f = lib().ora_sum_exact_f32 if x.dtype == np.float32 else lib().ora_sum_exact_f64
    return f(_p(x), ctypes.c_int64(x.size))


def rowsum_ref(x):
    rows, cols = x.shape
    out = np.empty(rows, dtype=x.dtype)
    f = lib().ora_rowsum_ref_f32 if x.dtype == np.float32 else lib().ora_rowsum_ref_f64
    f(_p(x), ctypes.c_int64(rows), ctypes.c_int64(cols), _p(out))
    return out


def rowsum_exact(x):
    rows, cols = x.shape
    out = np.empty(rows, dtype=np.float64)
    f = lib().ora_rowsum_exact_f32 if x.dtype == np.float32 else lib().ora_rowsum_exact_f64
    f(_p(x), ctypes.c_int64(rows), ctypes.c_int64(cols), _p(out))
    return out


def colsum_ref(x):
    rows, cols = x.shape
    out = np.empty(cols, dtype=x.dtype)
    f = lib().ora_colsum_ref_f32 if x.dtype == np.float32 else lib().ora_colsum_ref_f64
    f(_p(x), ctypes.c_int64(rows), ctypes.c_int64(cols), _p(out))
    return out


def max_chain(x):
    f = lib().ora_max_chain_f32 if x.dtype == np.float32 else lib().ora_max_chain_f64
    return f(_p(x), ctypes.c_int64(x.size))


def rowmax_chain(x):
    rows, cols = x.shape
    out = np.empty(rows, dtype=x.dtype)
    f = lib().ora_rowmax_chain_f32 if x.dtype == np.float32 else lib().ora_rowmax_chain_f64
    f(_p(x), ctypes.c_int64(rows), ctypes.c_int64(cols), _p(out))
    return out


def argmax(x):
    f = lib().ora_argmax_f32 if x.dtype == np.float32 else lib().ora_argmax_f64
    return f(_p(x), ctypes.c_int64(x.size))


def rowargmax(x):
    rows, cols = x.shape
    out = np.empty(rows, dtype=np.int64)
    f = lib().ora_rowargmax_f32 if x.dtype == np.float32 else lib().ora_rowargmax_f64
    f(_p(x), ctypes.c_int64(rows), ctypes.c_int64(cols), _p(out))
    return out


def softmax_rows(x, log=False):
    rows, cols = x.shape
    out = np.empty_like(x)
    name = ("ora_log_softmax_rows_" if log else "ora_softmax_rows_") + ("f32" if x.dtype == np.float32 else "f64")
    getattr(lib(), name)(_p(x), ctypes.c_int64(rows), ctypes.c_int64(cols), _p(out))
    return out


# ---- activations ---------------------------------------------------------------------

def act(name, x, alpha=0.0):
    out = np.empty_like(x)
    f = lib().ora_act_f32 if x.dtype == np.float32 else lib().ora_act_f64
    f(ctypes.c_int(ACT_CODE[name]), _p(x), _p(out), ctypes.c_int64(x.size), _f64(alpha))
    return out


# ---- quantization ---------------------------------------------------------------------

def calibrate(x, symmetric):
    p = QuantParams()
    f = lib().ora_calibrate_minmax_f32 if x.dtype == np.float32 else lib().ora_calibrate_minmax
    rc = f(_p(x), ctypes.c_int64(x.size), ctypes.c_int(1 if symmetric else 0), ctypes.byref(p))
    assert rc == 0
    return p


def quantize(x, p):
    out = np.empty(x.size, dtype=np.int8)
    f = lib().ora_quantize_f32 if x.dtype == np.float32 else lib().ora_quantize
    assert f(_p(x), _p(out), ctypes.c_int64(x.size), ctypes.byref(p)) == 0
    return out


def dequantize(q, p, dtype=np.float64):
    out = np.empty(q.size, dtype=dtype)
    f = lib().ora_dequantize_f32 if dtype == np.float32 else lib().ora_dequantize
    assert f(_p(q), _p(out), ctypes.c_int64(q.size), ctypes.byref(p)) == 0
    return out


def calibrate_percentile(x, percentile, symmetric, use_ref=False):
    """QuantParams from calibrate_percentile (quantize.c:89-132) on float64 x;
    use_ref: the reference's own quantize.c.  Returns (rc, params)."""
    x = np.ascontiguousarray(x, dtype=np.float64)
    p = QuantParams()
    f = ref().calibrate_percentile if use_ref else lib().ora_calibrate_percentile
    f.restype = ctypes.c_int
    f.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_double, ctypes.c_int, ctypes.POINTER(QuantParams)]
    rc = f(_p(x), x.size, percentile, 1 if symmetric else 0, ctypes.byref(p))
    return rc, p


def quantized_matmul(a, b, m, k, n, pa, pb, use_ref=False):
    """C [m x n] float64 of int8 a [m x k] and b [k x n] (quantize.c:191-214);
    use_ref: the reference's own quantize.c (oracle/_ref)."""
    a = np.ascontiguousarray(a, dtype=np.int8)
    b = np.ascontiguousarray(b, dtype=np.int8)
    c = np.empty(m * n, dtype=np.float64)
    f = ref().quantized_matmul if use_ref else lib().ora_quantized_matmul
    f.restype = ctypes.c_int
    f.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64,
                  ctypes.POINTER(QuantParams), ctypes.POINTER(QuantParams)]
    rc = f(_p(a), _p(b), _p(c), m, k, n, ctypes.byref(pa), ctypes.byref(pb))
    return rc, c.reshape(m, n)


def quant_error(x, p):
    f = lib().ora_quant_error_f32 if x.dtype == np.float32 else lib().ora_quant_error
    return f(_p(x), ctypes.c_int64(x.size), ctypes.byref(p))


def quant_snr(x, p):
    f = lib().ora_quant_snr_f32 if x.dtype == np.float32 else lib().ora_quant_snr
    return f(_p(x), ctypes.c_int64(x.size), ctypes.byref(p))


# ---- optimizers ------------------------------------------------------------------------

def bias_correction(beta, t):
    return lib().ora_bias_correction(beta, t)


def adamw_step(p, g, m, v, lr, b1, b2, eps, wd, t):
    """In-place AdamW step number t (1-based) on numpy buffers."""
    bc1, bc2 = bias_correction(b1, t), bias_correction(b2, t)
    n = ctypes.c_int64(p.size)
    args = [_f64(lr), _f64(b1), _f64(b2), _f64(eps), _f64(wd), _f64(bc1), _f64(bc2)]
    f = lib().ora_adamw_f32 if p.dtype == np.float32 else lib().ora_adamw_f64
    f(_p(p), _p(g), _p(m), _p(v), n, *args)


def adam_step(p, g, m, v, lr, b1, b2, eps, t):
    bc1, bc2 = bias_correction(b1, t), bias_correction(b2, t)
    n = ctypes.c_int64(p.size)
    args = [_f64(lr), _f64(b1), _f64(b2), _f64(eps), _f64(bc1), _f64(bc2)]
    f = lib().ora_adam_f32 if p.dtype == np.float32 else lib().ora_adam_f64
    f(_p(p), _p(g), _p(m), _p(v), n, *args)


def sgd_step(p, g, vel, lr, mom):
    f = lib().ora_sgd_f32 if p.dtype == np.float32 else lib().ora_sgd_f64
    f(_p(p), _p(g), _p(vel), ctypes.c_int64(p.size), _f64(lr), _f64(mom))


# ---- scans ------------------------------------------------------------------------------

def has_nan(x):
    return lib().ora_has_nan_f32(_p(x), ctypes.c_uint64(x.size))


def has_inf(x):
    return lib().ora_has_inf_f32(_p(x), ctypes.c_uint64(x.size))


def l2_ref(x):
    return lib().ora_l2_ref_f32(_p(x), ctypes.c_uint64(x.size))


def sumsq_exact(x):
    return lib().ora_sumsq_exact_f32(_p(x), ctypes.c_uint64(x.size))


# ---- tensor ops ------------------------------------------------------------------------------

def concat_2d(a, b, ra, ca, rb, cb, axis):
    out = np.zeros((ra + rb) * (ca + cb), dtype=np.float64)
    r, c = ctypes.c_int64(), ctypes.c_int64()
    rc = lib().ora_concat_2d(_p(a), _p(b), ctypes.c_int64(ra), ctypes.c_int64(ca), ctypes.c_int64(rb),
                             ctypes.c_int64(cb), ctypes.c_int64(axis), _p(out), ctypes.byref(r), ctypes.byref(c))
    return rc, out[: r.value * c.value] if rc == 0 else None, r.value, c.value


def transpose_2d(a, rows, cols):
    out = np.zeros(rows * cols, dtype=np.float64)
    rc = lib().ora_transpose_2d(_p(a), ctypes.c_int64(rows), ctypes.c_int64(cols), _p(out))
    return rc, out


def pad_2d(a, rows, cols, pt, pb, pl, pr, value):
    R, C = rows + pt + pb, cols + pl + pr
    out = np.zeros(max(R * C, 1), dtype=np.float64)
    r, c = ctypes.c_int64(), ctypes.c_int64()
    rc = lib().ora_pad_2d(_p(a), ctypes.c_int64(rows), ctypes.c_int64(cols), ctypes.c_int64(pt),
                          ctypes.c_int64(pb), ctypes.c_int64(pl), ctypes.c_int64(pr), _f64(value), _p(out),
                          ctypes.byref(r), ctypes.byref(c))
    return rc, out[: R * C], r.value, c.value


def split_2d(a, rows, cols, axis, split):
    oa = np.zeros(rows * cols, dtype=np.float64)
    ob = np.zeros(rows * cols, dtype=np.float64)
    ra, ca, rb, cb = (ctypes.c_int64() for _ in range(4))
    rc = lib().ora_split_2d(_p(a), ctypes.c_int64(rows), ctypes.c_int64(cols), ctypes.c_int64(axis),
                            ctypes.c_int64(split), _p(oa), _p(ob), ctypes.byref(ra), ctypes.byref(ca),
                            ctypes.byref(rb), ctypes.byref(cb))
    return rc, oa[: ra.value * ca.value], ob[: rb.value * cb.value], (ra.value, ca.value, rb.value, cb.value)


def build_info():
    return {"oracle": str(ORACLE_SO), "ref": str(REF_SO) if REF_SO.exists() else None,
            "pid": os.getpid()}


# ---- cross-entropy losses -------------------------------------------------------------

def ls_ce_forward(logits, targets, smoothing, use_ref=False):
    """Label-smoothed CE forward (metrics_losses.c:28-77); use_ref runs the
    reference's own compiled C."""
    b, k = logits.shape
    x = np.ascontiguousarray(logits, dtype=np.float64)
    t = np.ascontiguousarray(targets, dtype=np.int64)
    out = ctypes.c_double()
    f = getattr(ref() if use_ref else lib(), "label_smoothing_ce_forward" if use_ref else "ora_ls_ce_forward")
    rc = f(_p(x), _p(t), ctypes.c_int64(b), ctypes.c_int64(k), ctypes.c_double(smoothing), ctypes.byref(out))
    return rc, out.value


def ls_ce_backward(logits, targets, smoothing, use_ref=False):
    b, k = logits.shape
    x = np.ascontiguousarray(logits, dtype=np.float64)
    t = np.ascontiguousarray(targets, dtype=np.int64)
    g = np.zeros((b, k), dtype=np.float64)
    f = getattr(ref() if use_ref else lib(), "label_smoothing_ce_backward" if use_ref else "ora_ls_ce_backward")
    rc = f(_p(x), _p(t), ctypes.c_int64(b), ctypes.c_int64(k), ctypes.c_double(smoothing), _p(g))
    return rc, g


def ce_loss(logits, target_values):
    """cross_entropy_loss intended semantics (losses.asm:315-613): targets as
    values of the logits' dtype, truncated to an index."""
    b, k = logits.shape
    x = np.ascontiguousarray(logits)
    t = np.ascontiguousarray(target_values, dtype=x.dtype)
    out = ctypes.c_double()
    f = lib().ora_ce_loss_f32 if x.dtype == np.float32 else lib().ora_ce_loss_f64
    rc = f(_p(x), _p(t), ctypes.c_int64(b), ctypes.c_int64(k), ctypes.byref(out))
    return rc, out.value



# ---- gradient clipping -------------------------------------------------------------

def _grad_lists(arrays):
    outs = [None if a is None else np.array(a, copy=True, order="C") for a in arrays]
    n = len(outs)
    ptrs = (ctypes.c_void_p * max(n, 1))(*[None if a is None else a.ctypes.data for a in outs])
    dts = (ctypes.c_int * max(n, 1))(*[1 if (a is not None and a.dtype == np.float64) else 0 for a in outs])
    ns = (ctypes.c_int64 * max(n, 1))(*[0 if a is None else a.size for a in outs])
    return outs, ptrs, dts, ns, n


def clip_grad_norm(arrays, max_norm):
    """clip_grad_norm_ (optimizers.asm:1370-1516) on copies of float32/float64
    arrays (None entries skipped).  Returns (pre-clip norm, clipped copies)."""
    outs, ptrs, dts, ns, n = _grad_lists(arrays)
    f = lib().ora_clip_grad_norm
    f.restype = ctypes.c_double
    f.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_double]
    norm = f(ptrs, dts, ns, n, max_norm)
    return norm, outs


def clip_grad_value(arrays, lo, hi):
    """clip_grad_value_ (optimizers.asm:1527-1620) on copies; returns them."""
    outs, ptrs, dts, ns, n = _grad_lists(arrays)
    f = lib().ora_clip_grad_value
    f.restype = None
    f.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_double,
                  ctypes.c_double]
    f(ptrs, dts, ns, n, lo, hi)
    return outs


# ---- dropout ---------------------------------------------------------------------

def glibc_rand(seed, n, skip=0):
    """Restatement of glibc's rand() stream after srand(seed) (TYPE_3:
    r[i] = r[i-31] + r[i-3] mod 2^32 after a Park-Miller fill and 310
    discards; output r >> 1), draws skip .. skip + n - 1, as uint32."""
    s = seed & 0xFFFFFFFF
    s = s if s != 0 else 1
    r = np.zeros(344 + skip + n, dtype=np.uint64)
    r[0] = s
    w = s if s < 2 ** 31 else s - 2 ** 32
    for i in range(1, 31):
        hi = int(w / 127773)
        lo = w - hi * 127773
        w = 16807 * lo - 2836 * hi
        if w < 0:
            w += 2147483647
        r[i] = w
    r[31:34] = r[0:3]
    m = np.uint64(0xFFFFFFFF)
    for i in range(34, 344 + skip + n):
        r[i] = (r[i - 31] + r[i - 3]) & m
    return (r[344 + skip:] >> np.uint64(1)).astype(np.uint32)


def srand(seed):
    lib().ora_srand(ctypes.c_uint(seed & 0xFFFFFFFF))


def dropout_forward(x, p):
    """dropout_forward with the C library's rand() from its current state."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty_like(x)
    mask = np.empty(x.size, dtype=np.uint8)
    f = lib().ora_dropout_forward
    f.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint64, ctypes.c_float]
    rc = f(_p(x), _p(out), _p(mask), x.size, p)
    return rc, out, mask


def dropout_backward(go, mask, p):
    go = np.ascontiguousarray(go, dtype=np.float32)
    mask = np.ascontiguousarray(mask, dtype=np.uint8)
    gi = np.empty_like(go)
    f = lib().ora_dropout_backward
    f.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint64, ctypes.c_float]
    rc = f(_p(go), _p(gi), _p(mask), go.size, p)
    return rc, gi


def rand_n(n):
    """The C library's rand(), n calls from its current state, as uint32."""
    out = np.empty(n, dtype=np.uint32)
    f = lib().ora_rand_n
    f.argtypes = [ctypes.c_uint64, ctypes.c_void_p]
    f.restype = None
    f(n, _p(out))
    return out


def glibc_window(seed, skip, n):
    """rand() values skip .. skip + n - 1 after srand(seed), from the C
    restatement with the jump x^skip mod (x^31 - x^28 - 1)."""
    out = np.empty(n, dtype=np.uint32)
    f = lib().ora_glibc_window
    f.argtypes = [ctypes.c_uint32, ctypes.c_uint64, ctypes.c_uint64, ctypes.c_void_p]
    f.restype = None
    f(seed & 0xFFFFFFFF, skip, n, _p(out))
    return out


def dropout_window(seed, skip, x, p):
    """dropout_forward on draws skip .. skip + x.size - 1 after srand(seed)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty_like(x)
    mask = np.empty(x.size, dtype=np.uint8)
    f = lib().ora_dropout_window
    f.argtypes = [ctypes.c_uint32, ctypes.c_uint64, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint64,
                  ctypes.c_float]
    assert f(seed & 0xFFFFFFFF, skip, _p(x), _p(out), _p(mask), x.size, p) == 0
    return out, mask


def add_relu(a, b):
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    c = np.empty_like(a)
    f = lib().ora_add_relu_f32
    f.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64]
    f(_p(a), _p(b), _p(c), a.size)
    return c


# ---- per-feature transforms ----------------------------------------------------------

def transform_stats(data, use_ref=False):
    """transform_compute_stats (transforms.c:27-62) on a [batch, features]
    float64 array; use_ref runs the reference's own compiled C.  Returns
    (rc, mean, std, min, max)."""
    x = np.ascontiguousarray(data, dtype=np.float64)
    b, nf = x.shape
    outs = [np.zeros(nf) for _ in range(4)]
    f = ref().transform_compute_stats if use_ref else lib().ora_transform_stats
    rc = f(_p(x), ctypes.c_int64(b), ctypes.c_int64(nf), *[_p(o) for o in outs])
    return (rc, *outs)


def transform_apply(mode, data, p0, p1, eps, use_ref=False):
    """mode 0 normalize, 1 unnormalize, 2 min-max (transforms.c:68-143)."""
    x = np.ascontiguousarray(data, dtype=np.float64)
    b, nf = x.shape
    a0 = np.ascontiguousarray(p0, dtype=np.float64)
    a1 = np.ascontiguousarray(p1, dtype=np.float64)
    out = np.zeros_like(x)
    if use_ref:
        f = getattr(ref(), ["transform_normalize", "transform_unnormalize", "transform_minmax"][mode])
        rc = f(_p(x), _p(out), ctypes.c_int64(b), ctypes.c_int64(nf), _p(a0), _p(a1), ctypes.c_double(eps))
    else:
        rc = lib().ora_transform_apply(ctypes.c_int(mode), _p(x), _p(out), ctypes.c_int64(b), ctypes.c_int64(nf),
                                       _p(a0), _p(a1), ctypes.c_double(eps))
    return rc, out
