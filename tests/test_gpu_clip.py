"""Gradient clipping parity (optimizers.asm:1370-1620) through the C-ABI.

The global-norm clip is compared with the oracle's clip_grad_norm_
restatement: the pre-clip norm within 1e-12 relative of the fp64-exact norm
(the device sums in a tree, the reference sequentially; all terms are >= 0);
clipped f32 gradients bit-exact (the float scale of both sides agrees, which
the test checks), clipped f64 gradients within REL64 (the double scale
follows the norm's last bits).  The value clip is bit-exact.  Threshold, NaN
and Inf cases, None entries, more tensors than one launch carries, the
optimizer-handle entry points and a cfg5-sized (100 M f32) run are covered.
"""

import ctypes
import math

import numpy as np
import pytest

from conftest import GPU, rel_close, same_bits

pytestmark = GPU


def _tensors(pn, arrays):
    return [None if a is None else pn.Tensor.from_numpy(a) for a in arrays]


def _exact_norm(arrays):
    return math.sqrt(math.fsum(math.fsum((a.astype(np.float64).ravel() ** 2).tolist()) for a in arrays if a is not None))


def _check_norm_clip(pn, ora, arrays, max_norm):
    ts = _tensors(pn, arrays)
    norm = pn.clip_grad_norm(ts, max_norm)
    onorm, want = ora.clip_grad_norm(arrays, max_norm)
    exact = _exact_norm(arrays)
    if math.isfinite(exact):
        assert abs(norm - exact) <= 1e-12 * exact, (norm, exact)
    else:
        assert (math.isnan(norm) and math.isnan(exact)) or norm == exact
    clipped = norm > max_norm
    assert clipped == (onorm > max_norm) or abs(norm - max_norm) <= 1e-12 * norm
    for a, t, w in zip(arrays, ts, want):
        if a is None:
            continue
        got = t.numpy().reshape(-1)
        if not clipped:
            same_bits(got, a.reshape(-1))
        elif a.dtype == np.float32 and np.float32(max_norm / norm) == np.float32(max_norm / onorm):
            same_bits(got, w.reshape(-1))
        else:
            rel_close(got, w.reshape(-1), 1e-12, 1e-300, "clipped f64")
    return norm


@pytest.mark.parametrize("frac", [0.25, 0.999, 2.0])
def test_norm_clip_mixed_list(pn, ora, frac):
    rng = np.random.default_rng(31)
    arrays = [rng.normal(0, 1e-2, 300_001).astype(np.float32), None,
              rng.normal(0, 1.0, 4099), np.zeros(0, np.float32),
              rng.normal(0, 5, 3).astype(np.float32), rng.normal(0, 1, (65536 + 5,)),
              rng.normal(0, 1, (64, 129)).astype(np.float32)]
    max_norm = frac * _exact_norm(arrays)
    _check_norm_clip(pn, ora, arrays, max_norm)


def test_norm_clip_exact_threshold(pn, ora):
    a = np.array([3.0, 4.0])
    b = np.array([0.0, 0.0], np.float32)
    assert _check_norm_clip(pn, ora, [a, b], 5.0) == 5.0
    t = pn.Tensor.from_numpy(np.array([3.0, 4.0]))
    pn.clip_grad_norm([t], 2.5)
    assert t.numpy().tolist() == [1.5, 2.0]
    t = pn.Tensor.from_numpy(np.array([3.0, -4.0]))
    assert pn.clip_grad_norm([t], -5.0) == 5.0
    assert t.numpy().tolist() == [-3.0, 4.0]


def test_norm_clip_nan_inf(pn, ora):
    rng = np.random.default_rng(32)
    g = rng.normal(0, 1, 10_000).astype(np.float32)
    g[123] = np.nan
    _check_norm_clip(pn, ora, [g, rng.normal(0, 1, 100)], 1.0)
    h = rng.normal(0, 1, 5000).astype(np.float32)
    h[7] = -np.inf
    ts = _tensors(pn, [h])
    assert pn.clip_grad_norm(ts, 1.0) == math.inf
    _, want = ora.clip_grad_norm([h], 1.0)
    same_bits(ts[0].numpy(), want[0])
    # NaN max_norm: the compare is unordered, nothing is clipped
    k = np.array([30.0, 40.0])
    tk = pn.Tensor.from_numpy(k)
    assert pn.clip_grad_norm([tk], float("nan")) == 50.0
    assert tk.numpy().tolist() == [30.0, 40.0]


def test_norm_clip_many_tensors(pn, ora):
    # more tensors than one launch's argument list holds, both dtypes
    rng = np.random.default_rng(33)
    arrays = []
    for i in range(150):
        n = int(rng.integers(1, 3000))
        arrays.append(rng.normal(0, 1, n).astype(np.float32 if i % 3 else np.float64))
    _check_norm_clip(pn, ora, arrays, 0.5 * _exact_norm(arrays))


def test_norm_clip_unaligned_and_host_buffers(pn, ora):
    import torch
    rng = np.random.default_rng(34)
    # device buffer 4 bytes past an aligned base: the kernels' scalar path
    base = torch.from_numpy(rng.normal(0, 1, 10_001).astype(np.float32)).cuda()
    view = base[1:]
    arr = view.cpu().numpy()
    torch.cuda.synchronize()
    t = pn.Tensor.from_torch(view)
    norm = pn.clip_grad_norm([t], 1.0)
    onorm, want = ora.clip_grad_norm([arr], 1.0)
    assert abs(norm - onorm) <= 1e-12 * onorm
    same_bits(view.cpu().numpy(), want[0])
    # caller host buffer (kept host-authoritative): clipped in place
    h = rng.normal(0, 1, 3001)
    th = pn.Tensor.from_numpy_zero_copy(h)
    h0 = h.copy()
    pn.clip_grad_norm([th], 2.0)
    _, want = ora.clip_grad_norm([h0], 2.0)
    rel_close(h, want[0], 1e-12, 1e-300, "host buffer")


def test_norm_clip_no_norm_requested(pn, ora):
    rng = np.random.default_rng(35)
    a = rng.normal(0, 1, 200_000).astype(np.float32)
    t = pn.Tensor.from_numpy(a)
    arr = (ctypes.c_void_p * 1)(t._ptr)
    from pyneural.core import _lib
    assert _lib.neural_clip_grad_norm_list(arr, 1, ctypes.c_double(1.0), None) == 0
    onorm, want = ora.clip_grad_norm([a], 1.0)
    got = t.numpy()
    rel_close(got, want[0], 2.4e-7, 0.0, "clip without norm readback")


@pytest.mark.parametrize("dt", [np.float32, np.float64])
def test_value_clip_bit_exact(pn, ora, dt, rng):
    from conftest import special_f32, special_f64
    make = special_f32 if dt == np.float32 else special_f64
    arrays = [make(100_003, rng), None, make(7, rng), make(65536 * 2 + 1, rng)]
    for lo, hi in [(-0.3, 0.7), (0.0, 1.0), (1.0, -1.0), (-0.1, float("nan")), (float("nan"), 0.2)]:
        ts = _tensors(pn, arrays)
        pn.clip_grad_value(ts, lo, hi)
        want = ora.clip_grad_value(arrays, lo, hi)
        for t, w in zip(ts, want):
            if t is not None:
                same_bits(t.numpy(), w)


def test_handle_entry_points(pn, ora):
    rng = np.random.default_rng(36)
    p = [rng.normal(0, 0.02, 5000).astype(np.float32), rng.normal(0, 0.02, 77)]
    g = [rng.normal(0, 1, 5000).astype(np.float32), rng.normal(0, 1, 77)]
    tp, tg = _tensors(pn, p), _tensors(pn, g)
    opt = pn.AdamW(1e-3)
    opt.clip_grad_norm(1.0)  # before any step: nothing known, nothing done
    same_bits(tg[0].numpy(), g[0])
    opt.step(tp, tg)
    opt.clip_grad_norm(1.0)
    _, want = ora.clip_grad_norm(g, 1.0)
    for t, w in zip(tg, want):
        rel_close(t.numpy(), w, 2.4e-7 if w.dtype == np.float32 else 1e-12, 0.0, "handle clip")
    opt.clip_grad_value(-0.01, 0.01)
    want = ora.clip_grad_value([t.numpy() for t in tg], -0.01, 0.01)
    same_bits(tg[0].numpy(), want[0])
    from pyneural.core import _lib
    assert _lib.neural_clip_grad_norm(None, ctypes.c_double(1.0)) == 1


def test_errors(pn):
    import torch
    from pyneural.core import _lib
    nc = pn.Tensor.from_torch(torch.ones(4, 6, device="cuda").t())
    torch.cuda.synchronize()
    assert not nc.is_contiguous
    arr = (ctypes.c_void_p * 1)(nc._ptr)
    assert _lib.neural_clip_grad_norm_list(arr, 1, ctypes.c_double(1.0), None) == 3
    assert _lib.neural_clip_grad_value_list(arr, 1, ctypes.c_double(0.0), ctypes.c_double(1.0)) == 3
    assert _lib.neural_clip_grad_norm_list(None, 2, ctypes.c_double(1.0), None) == 1
    t = pn.Tensor.from_numpy(np.ones(8, np.float32))
    arr = (ctypes.c_void_p * 1)(t._ptr)
    assert _lib.neural_clip_grad_norm_list(arr, -1, ctypes.c_double(1.0), None) == 3
    assert _lib.neural_clip_grad_norm_list(arr, 0, ctypes.c_double(1.0), None) == 0
    norm = ctypes.c_double(-1.0)
    assert _lib.neural_clip_grad_norm_list(None, 0, ctypes.c_double(1.0), ctypes.byref(norm)) == 0
    assert norm.value == 0.0
    # at most 16384 non-empty tensors per call (the sum pass's partials);
    # NULL entries do not count
    big = torch.ones(16385, device="cuda")
    views = [pn.Tensor.from_torch(big[i:i + 1]) for i in range(16385)]
    torch.cuda.synchronize()
    arr = (ctypes.c_void_p * 16386)(*([v._ptr for v in views[:16384]] + [None, views[16384]._ptr]))
    assert _lib.neural_clip_grad_norm_list(arr, 16386, ctypes.c_double(1e30), ctypes.byref(norm)) == 3
    assert _lib.neural_clip_grad_norm_list(arr, 16385, ctypes.c_double(1e30), ctypes.byref(norm)) == 0
    assert norm.value == 128.0  # sqrt(16384 ones)


def test_cfg5_scale(pn, ora):
    # 100 M f32 gradients (cfg5): size-independent properties -- the norm
    # against the fused scan's sum of squares, the clipped norm equal to
    # max_norm, and one common scale factor.
    n = 100_000_000
    rng = np.random.default_rng(6)
    g = rng.normal(0, 1e-3, n).astype(np.float32)
    t = pn.Tensor.from_numpy(g)
    _, _, ss = pn.training._scan(t)
    max_norm = 0.5 * math.sqrt(ss)
    norm = pn.clip_grad_norm([t], max_norm)
    assert abs(norm - math.sqrt(ss)) <= 1e-12 * norm
    _, _, ss2 = pn.training._scan(t)
    assert abs(math.sqrt(ss2) - max_norm) <= 2e-7 * max_norm
    got = t.numpy()
    sf = np.float32(max_norm / norm)
    idx = rng.choice(n, 100_000, replace=False)
    same_bits(got[idx], g[idx] * sf)
