"""Maximum sizes: every index path past 2^31 elements (one MI355X holds these
tensors many times over).  Elementwise results are compared on the device with
torch's IEEE-exact ops; reductions with torch's float64 sums under the REDUCE
bound (1e-5 * sum|x|) and exactly for max / argmax (planted past 2^31);
quantize, dequantize, AdamW and dropout windows (the first and last elements)
bit for bit against the CPU oracle run on the same window -- elementwise
functions, so a window's results do not depend on the rest.  Dropout runs
three calls in a row past 2^32 draws, where the apply kernels switch to 64-bit
draw indices (the third call on keep bits made by the second); its
windows come from the oracle's jump-ahead of the glibc stream (pinned against
rand() itself in test_oracle_dropout.py).

Peak device memory of one test: ~60 GB (AdamW: f32 params and grads, f64
moments).
"""

import ctypes
import math

import numpy as np
import pytest

from conftest import GPU, same_bits

pytestmark = GPU

N = (1 << 31) + 5   # elements: every flat index past int32
W = 1 << 20         # window checked against the oracle at each end


@pytest.fixture
def lib(pn):
    """The library on torch's stream, so its kernels are ordered with the
    torch ops that make inputs and check outputs."""
    import torch
    pn.set_stream(torch.cuda.current_stream().cuda_stream)
    yield pn.core._lib
    torch.cuda.synchronize()
    pn.set_stream(None)
    torch.cuda.empty_cache()
    pn.core._lib.neural_hip_empty_cache()


def _uniform(n, seed, lo=-1.0, hi=1.0, dtype=None):
    import torch
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    return torch.empty(n, device="cuda", dtype=dtype or torch.float32).uniform_(lo, hi, generator=g)


def _ends(t):
    """The first and last W elements as numpy arrays."""
    return t[:W].cpu().numpy(), t[-W:].cpu().numpy()


def test_elementwise_past_int32(pn, lib):
    import torch
    a, b = _uniform(N, 1), _uniform(N, 2)
    out = torch.empty_like(a)
    ta, tb, to = pn.Tensor.from_torch(a), pn.Tensor.from_torch(b), pn.Tensor.from_torch(out)
    torch.cuda.synchronize()
    pn.core._check_error(lib.neural_add(to._ptr, ta._ptr, tb._ptr), "add")
    assert torch.equal(out, a + b)
    pn.core._check_error(lib.neural_mul(to._ptr, ta._ptr, tb._ptr), "mul")
    assert torch.equal(out, a * b)
    pn.core._check_error(lib.neural_relu(to._ptr, ta._ptr), "relu")
    assert torch.equal(out, torch.clamp_min(a, 0.0))
    # row-broadcast bias add over [2^21 + 1, 1024] (2^31 + 1024 elements)
    del ta, tb, to, a, b, out
    rows, cols = (1 << 21) + 1, 1024
    x = _uniform(rows * cols, 11).view(rows, cols)
    bias = _uniform(cols, 12)
    y = torch.empty_like(x)
    tx, tbias, ty = pn.Tensor.from_torch(x), pn.Tensor.from_torch(bias), pn.Tensor.from_torch(y)
    pn.core._check_error(lib.neural_bias_add(ty._ptr, tx._ptr, tbias._ptr), "bias_add")
    assert torch.equal(y, x + bias)


def test_reductions_past_int32(pn, lib):
    import torch
    a = _uniform(N, 3)
    a[(1 << 31) + 3] = 2.0   # the maximum, first at an index past 2^31
    a[(1 << 31) + 4] = 2.0   # a tie after it
    ta = pn.Tensor.from_torch(a)
    torch.cuda.synchronize()
    s, m, i = ctypes.c_double(), ctypes.c_double(), ctypes.c_int64()
    pn.core._check_error(lib.neural_sum(ta._ptr, ctypes.byref(s)), "sum")
    pn.core._check_error(lib.neural_max(ta._ptr, ctypes.byref(m)), "max")
    pn.core._check_error(lib.neural_argmax(ta._ptr, ctypes.byref(i)), "argmax")
    exact = torch.sum(a, dtype=torch.float64).item()
    bound = 1e-5 * torch.linalg.vector_norm(a, 1, dtype=torch.float64).item()
    assert abs(s.value - exact) <= bound, (s.value, exact)
    assert m.value == 2.0 and i.value == (1 << 31) + 3
    # per-row sums and argmax over [2^20 + 3, 2048] (2^31 + 6144 elements)
    del ta, a
    rows, cols = (1 << 20) + 3, 2048
    x = _uniform(rows * cols, 13).view(rows, cols)
    x.view(-1)[(1 << 31) + 3] = 2.0   # row 2^20, column 3; a tie in column 4
    x.view(-1)[(1 << 31) + 4] = 2.0
    tx = pn.Tensor.from_torch(x)
    rs = torch.empty(rows, device="cuda")
    ri = torch.empty(rows, dtype=torch.int64, device="cuda")
    trs = pn.Tensor.from_torch(rs)
    pn.core._check_error(lib.neural_reduce_sum(tx._ptr, 1, trs._ptr), "row sum")
    pn.core._check_error(lib.neural_reduce_argmax(tx._ptr, 1, ctypes.c_void_p(ri.data_ptr())), "row argmax")
    torch.cuda.synchronize()
    ex = torch.sum(x, dim=1, dtype=torch.float64)
    bnd = 1e-5 * torch.sum(x.abs(), dim=1, dtype=torch.float64)
    assert bool(((rs.double() - ex).abs() <= bnd).all())
    assert torch.equal(ri, torch.argmax(x, dim=1))


def test_softmax_past_int32(pn, lib):
    import torch
    rows, cols = (1 << 21) + 1, 1024
    s = (_uniform(rows * cols, 4) * 6.0).view(rows, cols)
    p = torch.empty_like(s)
    lp = torch.empty_like(s)
    ts, tp, tl = pn.Tensor.from_torch(s), pn.Tensor.from_torch(p), pn.Tensor.from_torch(lp)
    torch.cuda.synchronize()
    pn.core._check_error(lib.neural_softmax(tp._ptr, ts._ptr), "softmax")
    pn.core._check_error(lib.neural_log_softmax(tl._ptr, ts._ptr), "log_softmax")
    torch.cuda.synchronize()
    pick = torch.tensor([0, 1, 12345, (1 << 20) + 7, rows - 2, rows - 1], device="cuda")
    want = torch.softmax(s[pick].double(), dim=1)
    assert bool(((p[pick].double() - want).abs() <= 1e-5 * want).all())
    lwant = torch.log_softmax(s[pick].double(), dim=1)
    assert bool(((lp[pick].double() - lwant).abs() <= 1e-5 * lwant.abs() + 1e-6).all())
    sums = torch.sum(p, dim=1, dtype=torch.float64)
    assert bool(((sums - 1.0).abs() < 1e-5).all())


@pytest.mark.parametrize("symmetric", [0, 1])
def test_quantize_past_int32(pn, ora, lib, symmetric):
    import torch
    x = _uniform(N, 5)
    x[(1 << 31) + 1] = -50.0
    x[N - 2] = 50.0
    q8 = torch.empty(N, dtype=torch.int8, device="cuda")
    dq = torch.empty_like(x)
    pbuf = torch.zeros(5, dtype=torch.float64, device="cuda")
    torch.cuda.synchronize()
    assert lib.calibrate_minmax_f32_dev(x.data_ptr(), N, symmetric, pbuf.data_ptr()) == 0
    assert lib.quantize_tensor_f32_dev(x.data_ptr(), q8.data_ptr(), N, pbuf.data_ptr()) == 0
    assert lib.dequantize_tensor_f32_dev(q8.data_ptr(), dq.data_ptr(), N, pbuf.data_ptr()) == 0
    torch.cuda.synchronize()
    got = ora.QuantParams.from_buffer_copy(pbuf.cpu().numpy().tobytes())
    # calibration depends only on min and max: the oracle on a 3-element array
    # with the same extremes gives the same parameters
    want = ora.calibrate(np.array([0.25, -50.0, 50.0], dtype=np.float32), symmetric)
    assert (got.scale, got.zero_point, got.min_val, got.max_val, got.symmetric) == \
        (want.scale, want.zero_point, want.min_val, want.max_val, want.symmetric)
    for xs, qs, ds in zip(_ends(x), _ends(q8), _ends(dq)):
        same_bits(qs, ora.quantize(xs, want))
        same_bits(ds, ora.dequantize(qs, want, np.float32))


def test_adamw_past_int32(pn, ora, lib):
    import torch
    p = _uniform(N, 6, -0.05, 0.05)
    g = _uniform(N, 7, -1e-3, 1e-3)
    p0 = [w.copy() for w in _ends(p)]
    g1 = [w.copy() for w in _ends(g)]
    tp, tg = pn.Tensor.from_torch(p), pn.Tensor.from_torch(g)
    torch.cuda.synchronize()
    hp = dict(lr=1e-3, b1=0.9, b2=0.999, eps=1e-8, wd=0.01)
    opt = pn.AdamW(hp["lr"], hp["b1"], hp["b2"], hp["eps"], hp["wd"])
    opt.step([tp], [tg])
    g.mul_(-0.5).add_(2e-4)          # a second, different gradient
    g2 = [w.copy() for w in _ends(g)]
    opt.step([tp], [tg])
    torch.cuda.synchronize()
    for got, pw, ga, gb in zip(_ends(p), p0, g1, g2):
        m = np.zeros(W)
        v = np.zeros(W)
        ora.adamw_step(pw, ga, m, v, hp["lr"], hp["b1"], hp["b2"], hp["eps"], hp["wd"], 1)
        ora.adamw_step(pw, gb, m, v, hp["lr"], hp["b1"], hp["b2"], hp["eps"], hp["wd"], 2)
        same_bits(got, pw)
    del opt


def test_scan_past_int32(pn, lib):
    import torch
    g = _uniform(N, 8, -1e-3, 1e-3)
    tg = pn.Tensor.from_torch(g)
    torch.cuda.synchronize()
    hn, hi, ss = ctypes.c_int(), ctypes.c_int(), ctypes.c_double()
    pn.core._check_error(lib.neural_tensor_scan(tg._ptr, ctypes.byref(hn), ctypes.byref(hi), ctypes.byref(ss)), "scan")
    exact = torch.linalg.vector_norm(g, dtype=torch.float64).item() ** 2
    assert (hn.value, hi.value) == (0, 0)
    assert abs(ss.value - exact) <= 1e-5 * exact
    l2 = lib.neural_tensor_grad_l2_norm(g.data_ptr(), N)
    assert abs(l2 - math.sqrt(exact)) <= 1e-5 * math.sqrt(exact)
    g[N - 2] = float("inf")
    g[(1 << 31) + 1] = float("nan")
    torch.cuda.synchronize()
    pn.core._check_error(lib.neural_tensor_scan(tg._ptr, ctypes.byref(hn), ctypes.byref(hi), ctypes.byref(ss)), "scan")
    assert (hn.value, hi.value) == (1, 1)
    assert lib.neural_tensor_has_nan(g.data_ptr(), N) == 1
    assert lib.neural_tensor_has_inf(g.data_ptr(), N) == 1


@pytest.mark.parametrize("n", [N, (1 << 32) + 7])
def test_dropout_past_int32(pn, ora, lib, n):
    import torch
    x = _uniform(n, 9)
    out = torch.empty_like(x)
    mask = torch.empty(n, dtype=torch.uint8, device="cuda")
    torch.cuda.synchronize()
    seed = 2024
    assert lib.neural_dropout_seed(ctypes.c_uint32(seed)) == 0
    # three calls in a row: the second makes the third's keep bits during its
    # apply pass, and the third uses them (and makes the next ones)
    for call in range(3):
        assert lib.neural_dropout_forward(x.data_ptr(), out.data_ptr(), mask.data_ptr(), n, ctypes.c_float(0.3)) == 0
        torch.cuda.synchronize()
        if call == 1:
            continue
        for start in (0, n - W):
            xs = x[start:start + W].cpu().numpy()
            wout, wmask = ora.dropout_window(seed, call * n + start, xs, 0.3)
            same_bits(mask[start:start + W].cpu().numpy(), wmask)
            same_bits(out[start:start + W].cpu().numpy(), wout)
    assert lib.neural_dropout_draws() == 3 * n
    # the stream continues past the calls
    nxt = torch.empty(1000, device="cuda")
    m2 = torch.empty(1000, dtype=torch.uint8, device="cuda")
    assert lib.neural_dropout_forward(x.data_ptr(), nxt.data_ptr(), m2.data_ptr(), 1000, ctypes.c_float(0.3)) == 0
    torch.cuda.synchronize()
    same_bits(m2.cpu().numpy(), ora.dropout_window(seed, 3 * n, x[:1000].cpu().numpy(), 0.3)[1])
    # backward over the whole mask (the third call's)
    gi = torch.empty_like(x)
    assert lib.neural_dropout_backward(x.data_ptr(), gi.data_ptr(), mask.data_ptr(), n, ctypes.c_float(0.3)) == 0
    torch.cuda.synchronize()
    for start in (0, n - W):
        _, want = ora.dropout_backward(x[start:start + W].cpu().numpy(), mask[start:start + W].cpu().numpy(), 0.3)
        same_bits(gi[start:start + W].cpu().numpy(), want)
