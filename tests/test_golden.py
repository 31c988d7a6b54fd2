"""Golden fixtures (tests/golden/golden_vectors.npz, made by make_golden.py from
the reference's own C and the pinned oracle).

CPU: the oracle reproduces every fixture bit for bit.
GPU: libneural_hip.so reproduces the bit-exact fixtures bit for bit and the
transcendental ones within REL32 / REL64.
"""

import ctypes
from pathlib import Path

import numpy as np
import pytest

from conftest import GPU, rel_close, same_bits

G = np.load(Path(__file__).resolve().parent / "golden" / "golden_vectors.npz", allow_pickle=False)
ACTS = ["tanh", "gelu", "leaky_relu", "elu", "selu", "swish", "mish", "hardswish", "softplus", "hardtanh"]
ALPHA = {"leaky_relu": 0.01, "elu": 1.0}
EXACT_ACTS = {"leaky_relu", "hardswish", "hardtanh"}


def _params(ora, arr):
    p = ora.QuantParams()
    p.scale, p.zero_point, p.min_val, p.max_val, p.symmetric = arr[0], int(arr[1]), arr[2], arr[3], int(arr[4])
    return p


PCTS = (0.01, 0.3, 0.45)                 # as in make_golden.py
QMM_PARAMS = ((0.02, -3), (0.5, 5))


def _pct_rows(calib):
    """[scale, zero_point, min_val, max_val, symmetric] rows in fixture order;
    calib(percentile, symmetric) -> (rc, params)."""
    rows = []
    for pc in PCTS:
        for sym in (1, 0):
            rc, p = calib(pc, sym)
            assert rc == 0
            rows.append([p.scale, p.zero_point, p.min_val, p.max_val, p.symmetric])
    return np.array(rows)


def _qmm_params(cls):
    pa, pb = cls(), cls()
    (pa.scale, pa.zero_point), (pb.scale, pb.zero_point) = QMM_PARAMS
    pa.symmetric = pb.symmetric = 0
    return pa, pb


# ---- CPU: oracle vs fixtures ------------------------------------------------------------

@pytest.mark.parametrize("tag", ["f32", "f64"])
def test_oracle_activations(ora, tag):
    x = G[f"act_{tag}_x"]
    for name in ACTS:
        same_bits(ora.act(name, x, ALPHA.get(name, 0.0)), G[f"act_{name}_{tag}_y"])


def test_oracle_quant_opt_misc(ora):
    for tag in ("sym", "aff"):
        want_p = G[f"quant_{tag}_params"]
        p = ora.calibrate(G["quant_x_clean"], tag == "sym")
        assert [p.scale, p.zero_point, p.min_val, p.max_val, p.symmetric] == want_p.tolist()
        same_bits(ora.quantize(G["quant_x"], p), G[f"quant_{tag}_q"])
        same_bits(ora.dequantize(G[f"quant_{tag}_q"], p), G[f"quant_{tag}_dq"])
    for tag in ("f32", "f64"):
        for kind in ("sgd", "adam", "adamw"):
            p, g = G[f"opt_{tag}_p0"].copy(), G[f"opt_{tag}_g"]
            m, v = np.zeros(p.size), np.zeros(p.size)
            for t in (1, 2, 3):
                if kind == "sgd":
                    ora.sgd_step(p, g, m, 1e-2, 0.9)
                elif kind == "adam":
                    ora.adam_step(p, g, m, v, 1e-3, 0.9, 0.999, 1e-8, t)
                else:
                    ora.adamw_step(p, g, m, v, 1e-3, 0.9, 0.999, 1e-8, 0.01, t)
            same_bits(p, G[f"opt_{kind}_{tag}_p"])
            blob = G[f"opt_{kind}_{tag}_blob"].tobytes()
            same_bits(np.frombuffer(blob[88:88 + 8 * p.size], dtype=np.float64), m)
    same_bits(_pct_rows(lambda pc, sym: ora.calibrate_percentile(G["pct_x"], pc, sym)), G["pct_params"])
    pa, pb = _qmm_params(ora.QuantParams)
    rc, c = ora.quantized_matmul(G["qmm_a"], G["qmm_b"], 7, 37, 5, pa, pb)
    assert rc == 0
    same_bits(c, G["qmm_c"])
    same_bits(ora.softmax_rows(G["logsoftmax_x"], log=True), G["logsoftmax_y"])
    a, b = G["ew_a"], G["ew_b"]
    for name, code in (("add", ora.ADD), ("sub", ora.SUB), ("mul", ora.MUL), ("div", ora.DIV), ("max", ora.MAX)):
        same_bits(ora.ew(code, a, b), G[f"ew_{name}"])
    same_bits(ora.relu(a), G["relu"])
    same_bits(ora.rowmax_chain(G["rows_x"]), G["rows_max"])
    same_bits(ora.rowargmax(G["rows_x"]), G["rows_argmax"])
    assert np.float32(ora.sum_ref(a)) == G["sum_ref_f32"][0]
    assert np.float32(ora.l2_ref(a)) == G["l2_ref_f32"][0]
    same_bits(ora.softmax_rows(G["softmax_x"]), G["softmax_y"])


# ---- GPU: library vs fixtures -------------------------------------------------------------

@GPU
@pytest.mark.parametrize("tag", ["f32", "f64"])
def test_gpu_activations_golden(pn, tag):
    x = G[f"act_{tag}_x"]
    t = pn.Tensor.from_numpy(x)
    for name in ACTS:
        out = pn.Tensor.create(t.shape, t.dtype)
        fn = getattr(pn.core._lib, "act_" + name)
        rc = fn(out._ptr, t._ptr, ctypes.c_double(ALPHA[name])) if name in ALPHA else fn(out._ptr, t._ptr)
        assert rc == 0
        want = G[f"act_{name}_{tag}_y"]
        if name in EXACT_ACTS:
            same_bits(out.numpy(), want)
        elif tag == "f32":
            rel_close(out.numpy(), want, 1e-5, 0.0, name)
        else:
            rel_close(out.numpy(), want, 1e-12, 1e-15, name)


@GPU
def test_gpu_quant_opt_golden(pn):
    lib = pn.core._lib
    for tag in ("sym", "aff"):
        x = G["quant_x_clean"]
        p = pn.core.QuantParamsC()
        assert lib.calibrate_minmax(x.ctypes.data, x.size, 1 if tag == "sym" else 0, ctypes.byref(p)) == 0
        assert [p.scale, p.zero_point, p.min_val, p.max_val, p.symmetric] == G[f"quant_{tag}_params"].tolist()
        xq = G["quant_x"]
        q = np.empty(xq.size, dtype=np.int8)
        assert lib.quantize_tensor(xq.ctypes.data, q.ctypes.data, xq.size, ctypes.byref(p)) == 0
        same_bits(q, G[f"quant_{tag}_q"])
        d = np.empty(xq.size)
        assert lib.dequantize_tensor(q.ctypes.data, d.ctypes.data, q.size, ctypes.byref(p)) == 0
        same_bits(d, G[f"quant_{tag}_dq"])
    x = G["pct_x"]

    def calib(pc, sym):
        p = pn.core.QuantParamsC()
        return lib.calibrate_percentile(x.ctypes.data, x.size, ctypes.c_double(pc), sym, ctypes.byref(p)), p
    same_bits(_pct_rows(calib), G["pct_params"])
    pa, pb = _qmm_params(pn.core.QuantParamsC)
    c = np.empty((7, 5))
    assert lib.quantized_matmul(G["qmm_a"].ctypes.data, G["qmm_b"].ctypes.data, c.ctypes.data, 7, 37, 5,
                                ctypes.byref(pa), ctypes.byref(pb)) == 0
    same_bits(c, G["qmm_c"])
    for tag in ("f32", "f64"):
        for kind, opt in (("sgd", pn.SGD(1e-2, 0.9)), ("adam", pn.Adam(1e-3, 0.9, 0.999, 1e-8)),
                          ("adamw", pn.AdamW(1e-3, 0.9, 0.999, 1e-8, 0.01))):
            p, g = pn.Tensor.from_numpy(G[f"opt_{tag}_p0"]), pn.Tensor.from_numpy(G[f"opt_{tag}_g"])
            for _ in range(3):
                opt.step([p], [g])
            same_bits(p.numpy(), G[f"opt_{kind}_{tag}_p"])
            assert opt.state_bytes() == G[f"opt_{kind}_{tag}_blob"].tobytes()


def test_oracle_quant_f32_golden(ora):
    """The oracle's float32 quantization functions reproduce the fixtures the
    reference's quantize.c made from the widened values."""
    for tag in ("sym", "aff"):
        p = ora.calibrate(G["quant32_x_clean"], tag == "sym")
        assert [p.scale, p.zero_point, p.min_val, p.max_val, p.symmetric] == G[f"quant32_{tag}_params"].tolist()
        same_bits(ora.quantize(G["quant32_x"], p), G[f"quant32_{tag}_q"])
        same_bits(ora.dequantize(G[f"quant32_{tag}_q"], p, np.float32), G[f"quant32_{tag}_dq"])
        want_e, want_s = G[f"quant32_{tag}_err_snr"].tolist()
        assert ora.quant_error(G["quant32_x_clean"], p) == want_e
        assert ora.quant_snr(G["quant32_x_clean"], p) == want_s


@GPU
def test_gpu_quant_f32_golden(pn):
    """The float32 entry points reproduce the fixtures quantize.c made from
    the widened values: parameters, int8 codes and dequantized floats bit for
    bit; error and SNR within 1e-12 relative (tree order vs the reference's
    sequential double sum)."""
    lib = pn.core._lib
    for tag in ("sym", "aff"):
        xc = G["quant32_x_clean"]
        p = pn.core.QuantParamsC()
        assert lib.calibrate_minmax_f32(xc.ctypes.data, xc.size, 1 if tag == "sym" else 0, ctypes.byref(p)) == 0
        assert [p.scale, p.zero_point, p.min_val, p.max_val, p.symmetric] == G[f"quant32_{tag}_params"].tolist()
        x = G["quant32_x"]
        q = np.empty(x.size, dtype=np.int8)
        assert lib.quantize_tensor_f32(x.ctypes.data, q.ctypes.data, x.size, ctypes.byref(p)) == 0
        same_bits(q, G[f"quant32_{tag}_q"])
        d = np.empty(x.size, dtype=np.float32)
        assert lib.dequantize_tensor_f32(q.ctypes.data, d.ctypes.data, q.size, ctypes.byref(p)) == 0
        same_bits(d, G[f"quant32_{tag}_dq"])
        want_e, want_s = G[f"quant32_{tag}_err_snr"].tolist()
        rel_close([lib.quantization_error_f32(xc.ctypes.data, xc.size, ctypes.byref(p))], [want_e], 1e-12, 0.0, "err")
        rel_close([lib.quantization_snr_f32(xc.ctypes.data, xc.size, ctypes.byref(p))], [want_s], 1e-12, 0.0, "snr")


@GPU
def test_gpu_misc_golden(pn):
    lib = pn.core._lib
    ls = pn.LogSoftmax()(pn.Tensor.from_numpy(G["logsoftmax_x"])).numpy()
    rel_close(ls, G["logsoftmax_y"], 1e-12, 1e-15, "log_softmax")
    a, b = pn.Tensor.from_numpy(G["ew_a"]), pn.Tensor.from_numpy(G["ew_b"])
    for name in ("add", "sub", "mul", "div"):
        out = pn.Tensor.create(a.shape, a.dtype)
        assert getattr(lib, "neural_" + name)(out._ptr, a._ptr, b._ptr) == 0
        same_bits(out.numpy(), G[f"ew_{name}"])
    out = pn.Tensor.create(a.shape, a.dtype)
    assert lib.neural_maximum(out._ptr, a._ptr, b._ptr) == 0
    same_bits(out.numpy(), G["ew_max"])
    same_bits(pn.ReLU()(a).numpy(), G["relu"])
    rx = pn.Tensor.from_numpy(G["rows_x"])
    mx = pn.Tensor.create([16])
    assert lib.neural_reduce_max(rx._ptr, 1, mx._ptr) == 0
    same_bits(mx.numpy(), G["rows_max"])
    idx = np.empty(16, dtype=np.int64)
    assert lib.neural_reduce_argmax(rx._ptr, 1, idx.ctypes.data) == 0
    same_bits(idx, G["rows_argmax"])
    sm = pn.Softmax()(pn.Tensor.from_numpy(G["softmax_x"])).numpy()
    rel_close(sm, G["softmax_y"], 1e-5, 0.0, "softmax")
    out, r, c = pn.tensor_ops.concat_2d(G["concat_a"].tolist(), G["concat_b"].tolist(), 3, 4, 3, 2, axis=1)
    same_bits(np.array(out), G["concat_axis1"])
    out, r, c = pn.tensor_ops.transpose_2d(G["concat_a"].tolist(), 3, 4)
    same_bits(np.array(out), G["transpose_3x4"])
