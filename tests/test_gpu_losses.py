"""Cross-entropy parity (metrics_losses.c:28-125, losses.asm:315-613).

label_smoothing_ce_forward / _backward / _fused against the oracle's
restatement (itself bit-exact against the reference's own C, see
tests/test_oracle_losses.py) and, where the reference build travelled with
the tree, against that C directly.  The loss is a sum over rows and classes
accumulated here in a fixed tree instead of the reference's index order:
|g - r| <= 1e-12 * sum|terms| / B.  Gradients: 1e-12 relative + 2e-15 / B
absolute (softmax - target cancels).  neural_cross_entropy_loss: f64 against
the oracle (same bound), f32 against the fp64 closed form at 2e-6 relative
+ 2e-7 absolute (p_target is rounded to float, as in the reference; near 1 that
rounding is absolute in the loss; the reference's sequential float sums are
reported, not gated).
"""

import ctypes
import math

import numpy as np
import pytest

from conftest import GPU, rel_close

pytestmark = GPU


def _case(b, k, seed, special=False):
    rng = np.random.default_rng(seed)
    x = rng.normal(0, 3, (b, k))
    t = rng.integers(0, k, b).astype(np.int64)
    if special and b >= 5 and k >= 4:
        x[0, 1] = np.inf
        x[1, 2] = -np.inf
        x[2, 0] = np.nan
        x[3, k - 1] = np.nan
        x[4, :] = -np.inf
    return x, t


def _bound(x, t, a):
    """sum over rows/classes of |st * log_soft| / B, the scale of the loss sum."""
    b, k = x.shape
    m = np.max(np.where(np.isnan(x), -np.inf, x), axis=1, keepdims=True)
    with np.errstate(all="ignore"):
        lsm = (x - m) - np.log(np.exp(x - m).sum(axis=1, keepdims=True))
    st = np.full((b, k), a / k)
    st[np.arange(b), t] += 1 - a
    with np.errstate(all="ignore"):
        v = np.abs(st * lsm)
    return float(np.nansum(np.where(np.isfinite(v), v, 0))) / b


def _ls_gpu(pn, x, t, a, mode):
    lib = pn.core._lib
    b, k = x.shape
    loss = ctypes.c_double()
    g = np.full((b, k), np.nan)
    if mode == "fwd":
        rc = lib.label_smoothing_ce_forward(x.ctypes.data, t.ctypes.data, b, k, a, ctypes.byref(loss))
    elif mode == "bwd":
        rc = lib.label_smoothing_ce_backward(x.ctypes.data, t.ctypes.data, b, k, a, g.ctypes.data)
    else:
        rc = lib.label_smoothing_ce_fused(x.ctypes.data, t.ctypes.data, b, k, a, ctypes.byref(loss), g.ctypes.data)
    return rc, loss.value, g


def _loss_close(got, want, bound, tol=1e-12):
    if math.isnan(want):
        assert math.isnan(got)
    elif math.isinf(want):
        assert got == want
    else:
        assert abs(got - want) <= tol * bound + 1e-300, (got, want, bound)


@pytest.mark.parametrize("b,k", [(1, 1), (3, 5), (17, 10), (64, 1000), (5, 4096), (300, 2049), (1024, 64)])
@pytest.mark.parametrize("a", [0.0, 0.1, 1.0])
def test_ls_ce_vs_oracle(pn, ora, b, k, a):
    x, t = _case(b, k, b * 31 + k)
    rc, want_l = ora.ls_ce_forward(x, t, a)
    assert rc == 0
    want_g = ora.ls_ce_backward(x, t, a)[1]
    bound = _bound(x, t, a)
    rc, gl, _ = _ls_gpu(pn, x, t, a, "fwd")
    assert rc == 0
    _loss_close(gl, want_l, bound)
    rc, _, gg = _ls_gpu(pn, x, t, a, "bwd")
    assert rc == 0
    rel_close(gg, want_g, 1e-12, 2e-15 / b, "ls_ce grad")
    rc, fl, fg = _ls_gpu(pn, x, t, a, "fused")
    assert rc == 0
    # the forward's exp comes from its LDS table (~3 ulp), the fused kernel's
    # from the library (it keeps every e for the gradient): the row sums can
    # differ in their last bits, so the losses agree to well inside the bar
    _loss_close(fl, gl, bound, tol=1e-13)
    # backward and fused share the exp, the sums and the gradient formula
    assert np.array_equal(fg.view(np.uint64), gg.view(np.uint64))
    if ora.ref() is not None:  # the reference's own C, when it travelled with the tree
        _loss_close(gl, ora.ls_ce_forward(x, t, a, use_ref=True)[1], bound)


def test_ls_ce_special_values(pn, ora):
    x, t = _case(6, 9, 5, special=True)
    for a in (0.0, 0.3, 1.0):
        want_l = ora.ls_ce_forward(x, t, a)[1]
        want_g = ora.ls_ce_backward(x, t, a)[1]
        rc, gl, gg = _ls_gpu(pn, x, t, a, "fused")
        assert rc == 0
        _loss_close(gl, want_l, _bound(x, t, a))
        rel_close(gg, want_g, 1e-12, 2e-15 / 6, "ls_ce grad special")


def test_ls_ce_errors(pn):
    lib = pn.core._lib
    x = np.zeros((2, 3))
    loss = ctypes.c_double()
    for t, a in [(np.array([0, 3]), 0.1), (np.array([-1, 0]), 0.1), (np.array([0, 1]), -0.1),
                 (np.array([0, 1]), 1.5), (np.array([0, 1]), float("nan"))]:
        t = t.astype(np.int64)
        assert lib.label_smoothing_ce_forward(x.ctypes.data, t.ctypes.data, 2, 3, a, ctypes.byref(loss)) == -1
    t = np.array([0, 1], dtype=np.int64)
    assert lib.label_smoothing_ce_forward(None, t.ctypes.data, 2, 3, 0.1, ctypes.byref(loss)) == -1
    assert lib.label_smoothing_ce_forward(x.ctypes.data, t.ctypes.data, 0, 3, 0.1, ctypes.byref(loss)) == -1
    assert lib.label_smoothing_ce_backward(x.ctypes.data, t.ctypes.data, 2, 3, 0.1, None) == -1
    # still usable after an error
    assert lib.label_smoothing_ce_forward(x.ctypes.data, t.ctypes.data, 2, 3, 0.1, ctypes.byref(loss)) == 0
    assert abs(loss.value - math.log(3.0)) < 1e-15


def test_ls_ce_device_pointers_and_f32(pn, ora):
    torch = pytest.importorskip("torch")
    b, k = 4096, 1000
    x, t = _case(b, k, 77)
    xt = torch.from_numpy(x).cuda()
    tt = torch.from_numpy(t).cuda()
    g = torch.empty_like(xt)
    loss = ctypes.c_double()
    torch.cuda.synchronize()
    lib = pn.core._lib
    assert lib.label_smoothing_ce_fused(xt.data_ptr(), tt.data_ptr(), b, k, 0.1, ctypes.byref(loss), g.data_ptr()) == 0
    pn.synchronize()
    want_l = ora.ls_ce_forward(x, t, 0.1)[1]
    want_g = ora.ls_ce_backward(x, t, 0.1)[1]
    _loss_close(loss.value, want_l, _bound(x, t, 0.1))
    rel_close(g.cpu().numpy(), want_g, 1e-12, 2e-15 / b, "device grad")
    # f32 logits: the reference formula on the exactly widened values, grad rounded to float
    x32 = x.astype(np.float32)
    x32t = torch.from_numpy(x32).cuda()
    g32 = torch.empty_like(x32t)
    torch.cuda.synchronize()
    assert lib.label_smoothing_ce_fused_f32(x32t.data_ptr(), tt.data_ptr(), b, k, 0.1, ctypes.byref(loss),
                                            g32.data_ptr()) == 0
    pn.synchronize()
    xw = x32.astype(np.float64)
    want_l = ora.ls_ce_forward(xw, t, 0.1)[1]
    want_g = ora.ls_ce_backward(xw, t, 0.1)[1].astype(np.float32)
    assert abs(loss.value - want_l) <= 2e-7 * _bound(xw, t, 0.1)
    rel_close(g32.cpu().numpy(), want_g, 1e-5, 2e-7 / b, "f32 grad")


@pytest.mark.parametrize("dt", [np.float32, np.float64])
@pytest.mark.parametrize("b,k", [(1, 2), (100, 10), (1000, 1000), (33, 5000)])
def test_cross_entropy_loss(pn, ora, dt, b, k):
    rng = np.random.default_rng(b + k)
    x = rng.normal(0, 3, (b, k)).astype(dt)
    tv = rng.integers(0, k, b).astype(dt)
    got = pn.CrossEntropyLoss()(pn.Tensor.from_numpy(x), pn.Tensor.from_numpy(tv))
    rc, want = ora.ce_loss(x, tv)
    assert rc == 0
    xd = x.astype(np.float64)
    m = xd.max(axis=1, keepdims=True)
    p = np.exp(xd - m) / np.exp(xd - m).sum(axis=1, keepdims=True)
    exact = float(np.mean(-np.log(p[np.arange(b), tv.astype(np.int64)] + 1e-7)))
    if dt == np.float64:
        assert abs(got - want) <= 1e-12 * abs(want)
    else:
        # p_target is a float: near 1 its rounding (6e-8) is absolute in the loss
        assert abs(got - exact) <= 2e-6 * abs(exact) + 2e-7
        assert abs(want - exact) <= 1e-3 * abs(exact) + 2e-7  # the reference's float order, reported


def test_cross_entropy_loss_errors(pn):
    lib = pn.core._lib
    x = pn.Tensor.from_numpy(np.zeros((4, 3), dtype=np.float32))
    loss = ctypes.c_double()
    bad = pn.Tensor.from_numpy(np.array([0, 1, 3, 0], dtype=np.float32))
    assert lib.neural_cross_entropy_loss(x._ptr, bad._ptr, ctypes.byref(loss)) == pn.NeuralError.INVALID_ARGUMENT
    nan = pn.Tensor.from_numpy(np.array([0, np.nan, 1, 0], dtype=np.float32))
    assert lib.neural_cross_entropy_loss(x._ptr, nan._ptr, ctypes.byref(loss)) == pn.NeuralError.INVALID_ARGUMENT
    f64 = pn.Tensor.from_numpy(np.zeros(4))
    assert lib.neural_cross_entropy_loss(x._ptr, f64._ptr, ctypes.byref(loss)) == pn.NeuralError.DTYPE_MISMATCH
    short = pn.Tensor.from_numpy(np.zeros(3, dtype=np.float32))
    assert lib.neural_cross_entropy_loss(x._ptr, short._ptr, ctypes.byref(loss)) == pn.NeuralError.SHAPE_MISMATCH
    assert lib.neural_cross_entropy_loss(None, short._ptr, ctypes.byref(loss)) == pn.NeuralError.NULL_POINTER
    ok = pn.Tensor.from_numpy(np.array([0, 1.9, 2, 0], dtype=np.float32))  # 1.9 truncates to class 1
    assert lib.neural_cross_entropy_loss(x._ptr, ok._ptr, ctypes.byref(loss)) == 0
    assert abs(loss.value - (-math.log(1.0 / 3.0 + 1e-7))) < 1e-6


def test_label_smoothing_module(pn, ora):
    m = pn.LabelSmoothingCrossEntropy(num_classes=4, smoothing=0.2)
    logits = [0.5, -1.0, 2.0, 0.0, 1.0, 1.0, -2.0, 3.0]
    got = m(logits, [2, 3])
    want = ora.ls_ce_forward(np.array(logits).reshape(2, 4), np.array([2, 3]), 0.2)[1]
    assert abs(got - want) <= 1e-14 * abs(want)
    g = (ctypes.c_double * 8)()
    m.backward_f64(ctypes.cast(g, ctypes.c_void_p))
    rel_close(np.frombuffer(g, dtype=np.float64).reshape(2, 4),
              ora.ls_ce_backward(np.array(logits).reshape(2, 4), np.array([2, 3]), 0.2)[1], 1e-12, 1e-15, "module")


def test_label_smoothing_module_device_loss(pn):
    """The module's _dev methods: the host forms' loss and gradient, the loss
    read from device memory after one synchronisation; a host pointer raises."""
    torch = pytest.importorskip("torch")
    m = pn.LabelSmoothingCrossEntropy(num_classes=37, smoothing=0.15)
    x, t = _case(300, 37, 5)
    xt, tt = torch.from_numpy(x).cuda(), torch.from_numpy(t).cuda()
    g1, g2 = torch.empty_like(xt), torch.empty_like(xt)
    loss = torch.zeros(2, dtype=torch.float64, device="cuda")
    torch.cuda.synchronize()
    want = m.forward_backward_f64(xt.data_ptr(), tt.data_ptr(), 300, g1.data_ptr())
    m.forward_f64_dev(xt.data_ptr(), tt.data_ptr(), 300, loss.data_ptr())
    m.forward_backward_f64_dev(xt.data_ptr(), tt.data_ptr(), 300, g2.data_ptr(), loss.data_ptr() + 8)
    pn.synchronize()
    assert loss.cpu().tolist() == [want, want]
    assert torch.equal(g1, g2)
    with pytest.raises(pn.NeuralException):
        m.forward_f64_dev(x.ctypes.data, tt.data_ptr(), 300, loss.data_ptr())


@pytest.mark.parametrize("k", [1000, 1024])
def test_ls_ce_loss_left_in_device_memory(pn, k):
    """The _dev forms (no reference counterpart): the host-returning forms'
    loss and gradient bits, the loss stored in device memory; three calls
    queue without waiting; a target out of range gives a NaN loss and does
    not reach the next host-returning call; argument errors return -1."""
    torch = pytest.importorskip("torch")
    from conftest import same_bits
    lib = pn.core._lib
    b = 4096
    x, t = _case(b, k, 91)  # finite logits: a NaN loss below can only come from the bad target
    xt, tt = torch.from_numpy(x).cuda(), torch.from_numpy(t).cuda()
    x32t = xt.float()
    g_host, g_dev = torch.empty_like(xt), torch.full_like(xt, 7.0)
    g32_host, g32_dev = torch.empty_like(x32t), torch.full_like(x32t, 7.0)
    losses = torch.full((4,), 7.0, dtype=torch.float64, device="cuda")
    torch.cuda.synchronize()
    want = [ctypes.c_double() for _ in range(3)]
    assert lib.label_smoothing_ce_forward(xt.data_ptr(), tt.data_ptr(), b, k, 0.1, ctypes.byref(want[0])) == 0
    assert lib.label_smoothing_ce_fused(xt.data_ptr(), tt.data_ptr(), b, k, 0.1, ctypes.byref(want[1]),
                                        g_host.data_ptr()) == 0
    assert lib.label_smoothing_ce_fused_f32(x32t.data_ptr(), tt.data_ptr(), b, k, 0.1, ctypes.byref(want[2]),
                                            g32_host.data_ptr()) == 0
    pn.synchronize()
    assert all(math.isfinite(w.value) for w in want)
    p = losses.data_ptr()
    assert lib.label_smoothing_ce_forward_dev(xt.data_ptr(), tt.data_ptr(), b, k, 0.1, p) == 0
    assert lib.label_smoothing_ce_fused_dev(xt.data_ptr(), tt.data_ptr(), b, k, 0.1, p + 8, g_dev.data_ptr()) == 0
    assert lib.label_smoothing_ce_fused_f32_dev(x32t.data_ptr(), tt.data_ptr(), b, k, 0.1, p + 16,
                                                g32_dev.data_ptr()) == 0
    pn.synchronize()
    got = losses.cpu().numpy()
    same_bits(got[:3], np.array([w.value for w in want]))
    assert got[3] == 7.0  # nothing written past the three losses
    same_bits(g_dev.cpu().numpy(), g_host.cpu().numpy())
    same_bits(g32_dev.cpu().numpy(), g32_host.cpu().numpy())
    # a target out of range: a NaN loss, and the next host-returning call is clean
    t2 = t.copy()
    t2[17] = k
    tt2 = torch.from_numpy(t2).cuda()
    torch.cuda.synchronize()
    assert lib.label_smoothing_ce_forward_dev(xt.data_ptr(), tt2.data_ptr(), b, k, 0.1, p) == 0
    pn.synchronize()
    assert math.isnan(losses[0].item())
    again = ctypes.c_double()
    assert lib.label_smoothing_ce_forward(xt.data_ptr(), tt.data_ptr(), b, k, 0.1, ctypes.byref(again)) == 0
    same_bits(np.array(again.value), np.array(want[0].value))
    # argument errors: host memory, misalignment, NULL, sizes, smoothing
    assert lib.label_smoothing_ce_forward_dev(x.ctypes.data, tt.data_ptr(), b, k, 0.1, p) == -1
    assert lib.label_smoothing_ce_forward_dev(xt.data_ptr(), t.ctypes.data, b, k, 0.1, p) == -1
    host_loss = np.zeros(1)
    assert lib.label_smoothing_ce_forward_dev(xt.data_ptr(), tt.data_ptr(), b, k, 0.1, host_loss.ctypes.data) == -1
    assert lib.label_smoothing_ce_forward_dev(xt.data_ptr(), tt.data_ptr(), b, k, 0.1, p + 4) == -1
    assert lib.label_smoothing_ce_forward_dev(xt.data_ptr(), tt.data_ptr(), b, k, 0.1, None) == -1
    assert lib.label_smoothing_ce_fused_dev(xt.data_ptr(), tt.data_ptr(), b, k, 0.1, p, None) == -1
    assert lib.label_smoothing_ce_forward_dev(xt.data_ptr(), tt.data_ptr(), 0, k, 0.1, p) == -1
    assert lib.label_smoothing_ce_forward_dev(xt.data_ptr(), tt.data_ptr(), b, k, 1.5, p) == -1
    pn.synchronize()
    assert math.isnan(losses[0].item()) and losses[3].item() == 7.0  # untouched by the refused calls
