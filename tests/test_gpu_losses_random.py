"""Randomised label-smoothed cross-entropy (metrics_losses.c:28-125).

Seeded cases: 1-2000 rows of 1-8000 classes (log-uniform, at most 4 M
logits), with the widths that fill a one-wave-per-row kernel exactly
(64 lanes x 1, 2, 4, 8 or 16 vectors of 16 bytes) picked a quarter of the
time, so every kernel form runs: the wave kernels with and without a ragged
tail and the block-per-row kernel beyond them.  Smoothing is 0, 1 or uniform
in (0, 1); N(0, 3) logits with +Inf, -Inf, NaN or a row of only -Inf planted
in some cases.  Forward, backward and fused (host pointers, float64) are held
to the bounds of the fixed-shape tests: loss |g - r| <= 1e-12 * sum|terms| / B
against the oracle, gradient 1e-12 relative + 2e-15 / B; the fused gradient's
bits equal the backward's, the fused loss within 1e-13 * sum|terms| / B of
the forward's (whose exp comes from a table, ~3 ulp).  The float32 fused
form on device pointers is held to 2e-7 * sum|terms| / B for the loss and
1e-5 relative + 2e-7 / B for the gradient against the oracle on the widened
logits.  The _dev forms must give the host-returning forms' loss and
gradient bits, each against the same mode.
"""

import ctypes

import numpy as np
import pytest

from conftest import GPU, rel_close, same_bits
from test_gpu_losses import _bound, _loss_close, _ls_gpu

pytestmark = GPU

CASES = 30


def _case(rng, f32):
    vn = 4 if f32 else 2
    if rng.random() < 0.25:
        k = 64 * vn * int(rng.choice([1, 2, 4, 8, 16]))
    else:
        k = int(np.exp(rng.uniform(0, np.log(8000))))
    b = int(np.exp(rng.uniform(0, np.log(2000))))
    b = max(1, min(b, 4_000_000 // k))
    x = rng.normal(0, 3, (b, k))
    t = rng.integers(0, k, b).astype(np.int64)
    if rng.random() < 0.3:
        for _ in range(int(rng.integers(1, 4))):
            r = int(rng.integers(0, b))
            kind = int(rng.integers(0, 4))
            if kind == 0:
                x[r, int(rng.integers(0, k))] = np.inf
            elif kind == 1:
                x[r, rng.integers(0, k, max(1, k // 4))] = -np.inf
            elif kind == 2:
                x[r, int(rng.integers(0, k))] = np.nan
            else:
                x[r, :] = -np.inf
    u = rng.random()
    a = 0.0 if u < 0.15 else 1.0 if u < 0.25 else float(rng.uniform(0, 1))
    return x, t, a


def test_random_ls_ce_f64(pn, ora):
    torch = pytest.importorskip("torch")
    lib = pn.core._lib
    rng = np.random.default_rng(2024)
    for case in range(CASES):
        x, t, a = _case(rng, False)
        b, k = x.shape
        rc, want_l = ora.ls_ce_forward(x, t, a)
        assert rc == 0
        want_g = ora.ls_ce_backward(x, t, a)[1]
        bound = _bound(x, t, a)
        rc, gl, _ = _ls_gpu(pn, x, t, a, "fwd")
        assert rc == 0, (case, b, k, a)
        _loss_close(gl, want_l, bound)
        rc, _, gg = _ls_gpu(pn, x, t, a, "bwd")
        assert rc == 0, (case, b, k, a)
        rel_close(gg, want_g, 1e-12, 2e-15 / b, f"grad case {case} {b}x{k} a={a}")
        rc, fl, fg = _ls_gpu(pn, x, t, a, "fused")
        assert rc == 0
        _loss_close(fl, gl, bound, tol=1e-13)  # the forward's exp is its LDS table's
        same_bits(fg, gg)
        # the _dev forms on device copies: the host forms' bits
        xt, tt = torch.from_numpy(x).cuda(), torch.from_numpy(t).cuda()
        gd = torch.full_like(xt, 7.0)
        losses = torch.full((2,), 7.0, dtype=torch.float64, device="cuda")
        torch.cuda.synchronize()
        p = losses.data_ptr()
        assert lib.label_smoothing_ce_forward_dev(xt.data_ptr(), tt.data_ptr(), b, k, a, p) == 0
        assert lib.label_smoothing_ce_fused_dev(xt.data_ptr(), tt.data_ptr(), b, k, a, p + 8, gd.data_ptr()) == 0
        pn.synchronize()
        same_bits(losses.cpu().numpy(), np.array([gl, fl]))
        same_bits(gd.cpu().numpy(), gg)


def test_random_ls_ce_f32(pn, ora):
    torch = pytest.importorskip("torch")
    lib = pn.core._lib
    rng = np.random.default_rng(4048)
    for case in range(CASES):
        x, t, a = _case(rng, True)
        b, k = x.shape
        x32 = x.astype(np.float32)
        xw = x32.astype(np.float64)
        rc, want_l = ora.ls_ce_forward(xw, t, a)
        assert rc == 0
        want_g = ora.ls_ce_backward(xw, t, a)[1].astype(np.float32)
        xt, tt = torch.from_numpy(x32).cuda(), torch.from_numpy(t).cuda()
        g, gd = torch.empty_like(xt), torch.full_like(xt, 7.0)
        dl = torch.full((1,), 7.0, dtype=torch.float64, device="cuda")
        loss = ctypes.c_double()
        torch.cuda.synchronize()
        assert lib.label_smoothing_ce_fused_f32(xt.data_ptr(), tt.data_ptr(), b, k, a, ctypes.byref(loss),
                                                g.data_ptr()) == 0, (case, b, k, a)
        assert lib.label_smoothing_ce_fused_f32_dev(xt.data_ptr(), tt.data_ptr(), b, k, a, dl.data_ptr(),
                                                    gd.data_ptr()) == 0
        pn.synchronize()
        _loss_close(loss.value, want_l, _bound(xw, t, a), tol=2e-7)
        gh = g.cpu().numpy()
        rel_close(gh, want_g, 1e-5, 2e-7 / b, f"f32 grad case {case} {b}x{k} a={a}")
        same_bits(dl.cpu().numpy(), np.array([loss.value]))
        same_bits(gd.cpu().numpy(), gh)
