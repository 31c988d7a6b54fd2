#!/usr/bin/env python3
"""Regenerate the golden fixtures in this directory.

Vectors for the reference's C paths come from the reference's own C compiled
unchanged into oracle/_ref/libneural_ref.so (activations_c.c, quantize.c,
optimizers_c.c, tensor_ops.c, metrics_losses.c).  Vectors for the asm paths
(nasm is not available, so they cannot be built) come from the oracle's
restatement, which tests/test_oracle_closed_forms.py pins to IEEE closed forms
and brute force.  Seeded, small (<= 2 K elements per array), compressed npz,
no pickles.

    python tests/golden/make_golden.py        (needs `make -C oracle` first)
"""

import ctypes
import json
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
sys.path.insert(0, str(ROOT / "oracle"))
import ora  # noqa: E402

ACTS = ["tanh", "gelu", "leaky_relu", "elu", "selu", "swish", "mish", "hardswish", "softplus", "hardtanh"]
ALPHA = {"leaky_relu": 0.01, "elu": 1.0}
PCTS = (0.01, 0.3, 0.45)
QMM_PARAMS = ((0.02, -3), (0.5, 5))  # (scale, zero_point) of A and B, affine


class TensorC(ctypes.Structure):
    _fields_ = [("data", ctypes.c_void_p), ("ndim", ctypes.c_int64), ("shape", ctypes.POINTER(ctypes.c_int64)),
                ("stride", ctypes.c_void_p), ("dtype", ctypes.c_int32), ("flags", ctypes.c_int32)]


def tc(arr, keep):
    shape = (ctypes.c_int64 * arr.ndim)(*arr.shape)
    keep.append(shape)
    return TensorC(arr.ctypes.data, arr.ndim, shape, None, 0 if arr.dtype == np.float32 else 1, 0)


def act_input(dt):
    rng = np.random.default_rng(100)
    x = rng.normal(0, 4, 1024)
    x[rng.choice(1024, 20, replace=False)] = 30.0
    x[rng.choice(1024, 20, replace=False)] = -30.0
    x[:10] = [0.0, -0.0, 3.0, -3.0, 1.0, -1.0, 1e-310, -700.0, 20.0, -1e-5]
    return x.astype(dt)


def main():
    ref = ora.ref()
    if ref is None:
        sys.exit("oracle/_ref/libneural_ref.so missing: run `make -C oracle` with the reference tree mounted")
    out = {}
    keep = []
    # activations (activations_c.c)
    for dt, tag in ((np.float32, "f32"), (np.float64, "f64")):
        x = act_input(dt)
        for name in ACTS:
            y = np.empty_like(x)
            fn = getattr(ref, "act_" + name)
            ti, to = tc(x, keep), tc(y, keep)
            if name in ALPHA:
                fn.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_double]
                assert fn(ctypes.addressof(to), ctypes.addressof(ti), ALPHA[name]) == 0
            else:
                fn.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
                assert fn(ctypes.addressof(to), ctypes.addressof(ti)) == 0
            out[f"act_{name}_{tag}_y"] = y
        out[f"act_{tag}_x"] = x
    # quantization (quantize.c)
    rng = np.random.default_rng(101)
    xq = rng.laplace(0, 1, 2048)
    xq[[5, 77]] = [50.0, -50.0]
    xq[[9, 10, 11]] = [np.nan, np.inf, -np.inf]
    xq_clean = xq.copy()
    xq_clean[[9, 10, 11]] = 0.25
    out["quant_x"] = xq
    out["quant_x_clean"] = xq_clean
    P = ctypes.c_void_p
    ref.calibrate_minmax.argtypes = [P, ctypes.c_int64, ctypes.c_int, P]
    ref.quantize_tensor.argtypes = [P, P, ctypes.c_int64, P]
    ref.dequantize_tensor.argtypes = [P, P, ctypes.c_int64, P]
    for sym in (1, 0):
        p = ora.QuantParams()
        assert ref.calibrate_minmax(xq_clean.ctypes.data, xq_clean.size, sym, ctypes.byref(p)) == 0
        q = np.empty(xq.size, dtype=np.int8)
        assert ref.quantize_tensor(xq.ctypes.data, q.ctypes.data, xq.size, ctypes.byref(p)) == 0
        d = np.empty(xq.size)
        assert ref.dequantize_tensor(q.ctypes.data, d.ctypes.data, q.size, ctypes.byref(p)) == 0
        tag = "sym" if sym else "aff"
        out[f"quant_{tag}_params"] = np.array([p.scale, p.zero_point, p.min_val, p.max_val, p.symmetric])
        out[f"quant_{tag}_q"] = q
        out[f"quant_{tag}_dq"] = d
    # float32 quantization (calibrate_minmax_f32 / quantize_tensor_f32 /
    # dequantize_tensor_f32 / quantization_error_f32 / _snr_f32): the
    # reference's double path run on the float32 values widened to double
    # (exact); the dequantized fixture is (float) of the reference's double.
    rng32 = np.random.default_rng(105)
    xq32 = rng32.laplace(0, 1, 2048).astype(np.float32)
    xq32[[3, 64]] = [50.0, -50.0]
    xq32[[8, 13, 21, 34, 55, 89, 144]] = [np.nan, np.inf, -np.inf, 0.0, -0.0, 1e-45, 3.4e38]
    xq32_clean = xq32.copy()
    xq32_clean[[8, 13, 21, 144]] = [0.5, -0.5, 1.5, -1.5]
    out["quant32_x"], out["quant32_x_clean"] = xq32, xq32_clean
    w, wc = xq32.astype(np.float64), xq32_clean.astype(np.float64)
    ref.quantization_error.argtypes = [P, ctypes.c_int64, P]
    ref.quantization_snr.argtypes = [P, ctypes.c_int64, P]
    for sym in (1, 0):
        p = ora.QuantParams()
        assert ref.calibrate_minmax(wc.ctypes.data, wc.size, sym, ctypes.byref(p)) == 0
        q = np.empty(w.size, dtype=np.int8)
        assert ref.quantize_tensor(w.ctypes.data, q.ctypes.data, w.size, ctypes.byref(p)) == 0
        d = np.empty(w.size)
        assert ref.dequantize_tensor(q.ctypes.data, d.ctypes.data, q.size, ctypes.byref(p)) == 0
        tag = "sym" if sym else "aff"
        out[f"quant32_{tag}_params"] = np.array([p.scale, p.zero_point, p.min_val, p.max_val, p.symmetric])
        out[f"quant32_{tag}_q"] = q
        out[f"quant32_{tag}_dq"] = d.astype(np.float32)
        out[f"quant32_{tag}_err_snr"] = np.array([ref.quantization_error(wc.ctypes.data, wc.size, ctypes.byref(p)),
                                                  ref.quantization_snr(wc.ctypes.data, wc.size, ctypes.byref(p))])
    # percentile calibration (quantize.c:89-132): sorted, 500 negatives, 300
    # mixed-sign zeros, 1200 positives with integer ties; at p = 0.3 the low
    # rank (600) falls inside the zeros, so min_val carries the sign of the
    # zero that input order puts there (a -0 with this seed)
    rng = np.random.default_rng(106)
    xp = rng.permutation(np.concatenate([-np.abs(rng.normal(0, 2, 500)), np.where(rng.random(300) < 0.5, -0.0, 0.0),
                                         np.abs(rng.normal(0, 2, 1100)), rng.integers(1, 4, 100).astype(np.float64)]))
    out["pct_x"] = xp
    rows = []
    for pc in PCTS:
        for sym in (1, 0):
            rc, p = ora.calibrate_percentile(xp, pc, sym, use_ref=True)
            assert rc == 0
            rows.append([p.scale, p.zero_point, p.min_val, p.max_val, p.symmetric])
    out["pct_params"] = np.array(rows)
    # int8 product (quantize.c:191-214), affine zero points on both sides
    qa = rng.integers(-128, 128, (7, 37)).astype(np.int8)
    qb = rng.integers(-128, 128, (37, 5)).astype(np.int8)
    out["qmm_a"], out["qmm_b"] = qa, qb
    pa, pb = ora.QuantParams(), ora.QuantParams()
    (pa.scale, pa.zero_point), (pb.scale, pb.zero_point) = QMM_PARAMS
    rc, cq = ora.quantized_matmul(qa, qb, 7, 37, 5, pa, pb, use_ref=True)
    assert rc == 0
    out["qmm_c"] = cq
    # optimizers (optimizers_c.c): three steps
    for dt, tag in ((np.float32, "f32"), (np.float64, "f64")):
        rng = np.random.default_rng(102)
        p0 = rng.normal(0, 0.02, 1024).astype(dt)
        g = rng.normal(0, 1e-3, 1024).astype(dt)
        g[[1, 2, 3]] = [np.nan, np.inf, -np.inf]
        out[f"opt_{tag}_p0"], out[f"opt_{tag}_g"] = p0, g
        for kind in ("sgd", "adam", "adamw"):
            p = p0.copy()
            tp, tg = tc(p, keep), tc(g, keep)
            h = {"sgd": lambda: ref.opt_sgd_create(1e-2, 0.9),
                 "adam": lambda: ref.opt_adam_create(1e-3, 0.9, 0.999, 1e-8),
                 "adamw": lambda: ref.opt_adamw_create(1e-3, 0.9, 0.999, 1e-8, 0.01)}[kind]()
            pp = (ctypes.c_void_p * 1)(ctypes.addressof(tp))
            gp = (ctypes.c_void_p * 1)(ctypes.addressof(tg))
            for _ in range(3):
                assert ref.opt_step(h, pp, gp, 1) == 0
            nb = ref.opt_state_bytes(h)
            buf = (ctypes.c_uint8 * nb)()
            assert ref.opt_state_export(h, buf, nb) == 0
            out[f"opt_{kind}_{tag}_p"] = p
            out[f"opt_{kind}_{tag}_blob"] = np.frombuffer(bytes(buf), dtype=np.uint8)
            ref.opt_free(h)
    # log-softmax (metrics_losses.c:47-64) through the CE loss with smoothing 0
    rng = np.random.default_rng(103)
    xs = rng.normal(0, 3, (3, 19))
    ls = np.empty_like(xs)
    fn = ref.label_smoothing_ce_forward
    fn.argtypes = [P, P, ctypes.c_int64, ctypes.c_int64, ctypes.c_double, P]
    for i in range(3):
        row = np.ascontiguousarray(xs[i:i + 1])
        for c in range(19):
            t = np.array([c], dtype=np.int64)
            loss = ctypes.c_double()
            assert fn(row.ctypes.data, t.ctypes.data, 1, 19, 0.0, ctypes.byref(loss)) == 0
            ls[i, c] = -loss.value
    out["logsoftmax_x"], out["logsoftmax_y"] = xs, ls
    # tensor ops (tensor_ops.c)
    a = rng.normal(size=12)
    b = rng.normal(size=6)
    o = np.zeros(18)
    r, c = ctypes.c_int64(), ctypes.c_int64()
    ref.tensor_concat_2d.argtypes = [P, P] + [ctypes.c_int64] * 5 + [P, P, P]
    assert ref.tensor_concat_2d(a.ctypes.data, b.ctypes.data, 3, 4, 3, 2, 1, o.ctypes.data, ctypes.byref(r),
                                ctypes.byref(c)) == 0
    out["concat_a"], out["concat_b"], out["concat_axis1"] = a, b, o
    ref.tensor_transpose2d_array.argtypes = [P, ctypes.c_int64, ctypes.c_int64, P]
    tt = np.zeros(12)
    assert ref.tensor_transpose2d_array(a.ctypes.data, 3, 4, tt.ctypes.data) == 0
    out["transpose_3x4"] = tt
    # asm paths from the pinned oracle
    rng = np.random.default_rng(104)
    ea = rng.uniform(-1, 1, 1031).astype(np.float32)
    eb = rng.uniform(-1, 1, 1031).astype(np.float32)
    eb[::97] = 0.0
    out["ew_a"], out["ew_b"] = ea, eb
    for name, code in (("add", ora.ADD), ("sub", ora.SUB), ("mul", ora.MUL), ("div", ora.DIV), ("max", ora.MAX)):
        out[f"ew_{name}"] = ora.ew(code, ea, eb)
    out["relu"] = ora.relu(ea)
    rx = rng.normal(0, 3, (16, 64)).astype(np.float32)
    rx[3, 7] = np.nan
    rx[5, 63] = np.nan
    out["rows_x"] = rx
    out["rows_max"] = ora.rowmax_chain(rx)
    out["rows_argmax"] = ora.rowargmax(rx)
    out["rows_sum_exact"] = ora.rowsum_exact(rx)
    out["sum_ref_f32"] = np.array([ora.sum_ref(ea)], dtype=np.float32)
    out["l2_ref_f32"] = np.array([ora.l2_ref(ea)], dtype=np.float32)
    sx = rng.normal(0, 3, (8, 256)).astype(np.float32)
    out["softmax_x"], out["softmax_y"] = sx, ora.softmax_rows(sx)
    np.savez_compressed(HERE / "golden_vectors.npz", **out)
    meta = {"generator": "tests/golden/make_golden.py", "arrays": len(out),
            "reference_c": ["src/c/activations_c.c", "src/c/quantize.c", "src/c/optimizers_c.c",
                            "src/c/tensor_ops.c", "src/c/metrics_losses.c"],
            "oracle_pinned": ["ew_*", "relu", "rows_*", "sum_ref_f32", "l2_ref_f32", "softmax_y"]}
    (HERE / "golden_vectors.json").write_text(json.dumps(meta, indent=1) + "\n")
    print(f"wrote {len(out)} arrays to {HERE / 'golden_vectors.npz'}")


if __name__ == "__main__":
    main()
