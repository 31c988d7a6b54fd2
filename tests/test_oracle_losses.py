"""CPU checks of the oracle's cross-entropy restatements.

ora_ls_ce_forward/backward (metrics_losses.c:28-125) are pinned bit-exact
against the reference's own metrics_losses.c compiled unchanged
(oracle/_ref/libneural_ref.so), including the -1 argument checks and
non-finite logits.  ora_ce_loss_* (losses.asm:315-613, intended semantics)
are pinned by hand-derived values (the +1e-7 guard, truncation of the target
value) and by the fp64 closed form of -log(softmax[target] + 1e-7).
"""

import math

import numpy as np
import pytest

import ora


def _ref_or_skip():
    if ora.ref() is None:
        pytest.skip("reference C build (oracle/_ref) absent")


def _cases():
    rng = np.random.default_rng(11)
    out = []
    for b, k in [(1, 1), (3, 5), (17, 10), (64, 1000), (5, 4096)]:
        x = rng.normal(0, 3, (b, k))
        t = rng.integers(0, k, b)
        out.append((x, t))
    x = rng.normal(0, 3, (6, 9))
    x[0, 3] = np.inf
    x[1, 2] = -np.inf
    x[2, 0] = np.nan
    x[3, 5] = np.nan
    x[4, :] = -np.inf
    out.append((x, rng.integers(0, 9, 6)))
    return out


@pytest.mark.parametrize("smoothing", [0.0, 0.1, 0.37, 1.0])
def test_ls_ce_matches_reference_c(smoothing):
    _ref_or_skip()
    for x, t in _cases():
        rc_o, lo = ora.ls_ce_forward(x, t, smoothing)
        rc_r, lr = ora.ls_ce_forward(x, t, smoothing, use_ref=True)
        assert rc_o == rc_r == 0
        assert np.float64(lo).tobytes() == np.float64(lr).tobytes() or (math.isnan(lo) and math.isnan(lr))
        rc_o, go = ora.ls_ce_backward(x, t, smoothing)
        rc_r, gr = ora.ls_ce_backward(x, t, smoothing, use_ref=True)
        assert rc_o == rc_r == 0
        gn, rn = np.isnan(go), np.isnan(gr)
        assert np.array_equal(gn, rn)
        assert np.array_equal(go[~gn].view(np.uint64), gr[~rn].view(np.uint64))


def test_ls_ce_argument_checks():
    _ref_or_skip()
    x = np.zeros((2, 3))
    for t, s in [(np.array([0, 3]), 0.1), (np.array([-1, 0]), 0.1), (np.array([0, 1]), -0.1), (np.array([0, 1]), 1.5)]:
        assert ora.ls_ce_forward(x, t, s)[0] == ora.ls_ce_forward(x, t, s, use_ref=True)[0] == -1
        assert ora.ls_ce_backward(x, t, s)[0] == ora.ls_ce_backward(x, t, s, use_ref=True)[0] == -1


def test_ls_ce_closed_form():
    """Independent of either C: smoothing 0 gives -mean(log_softmax[target]);
    the gradient rows sum to 0 and equal (softmax - smoothed one-hot)/B."""
    rng = np.random.default_rng(3)
    x = rng.normal(0, 2, (7, 13))
    t = rng.integers(0, 13, 7)
    m = x.max(axis=1, keepdims=True)
    lsm = (x - m) - np.log(np.exp(x - m).sum(axis=1, keepdims=True))
    assert abs(ora.ls_ce_forward(x, t, 0.0)[1] - (-lsm[np.arange(7), t].mean())) < 1e-13
    a = 0.2
    st = np.full((7, 13), a / 13)
    st[np.arange(7), t] += 1 - a
    assert abs(ora.ls_ce_forward(x, t, a)[1] - (-(st * lsm).sum(axis=1).mean())) < 1e-13
    g = ora.ls_ce_backward(x, t, a)[1]
    assert np.allclose(g, (np.exp(lsm) - st) / 7, rtol=0, atol=1e-16)
    assert np.all(np.abs(g.sum(axis=1)) < 1e-16)


def test_ce_loss_hand_values():
    # two equal logits: p = 1/2 -> -log(0.5 + 1e-7)
    x = np.array([[0.0, 0.0]], dtype=np.float64)
    assert ora.ce_loss(x, np.array([0.0]))[1] == -math.log(0.5 + 1e-7)
    # p_t ~ e^-20: the 1e-7 guard dominates (without it the loss would be ~20)
    x = np.array([[0.0, 20.0]], dtype=np.float64)
    p = math.exp(-20.0) / (1.0 + math.exp(-20.0))
    got = ora.ce_loss(x, np.array([0.0]))[1]
    assert abs(got - (-math.log(p + 1e-7))) < 1e-15 and got < 16.2
    # the target value is truncated, not rounded: 1.7 -> class 1
    x = np.array([[1.0, 2.0, 3.0]], dtype=np.float32)
    e = np.exp(np.array([1.0, 2.0, 3.0]) - 3.0)
    want = -math.log(e[1] / e.sum() + 1e-7)
    assert abs(ora.ce_loss(x, np.array([1.7], dtype=np.float32))[1] - want) < 1e-6
    # out-of-range target
    assert ora.ce_loss(x, np.array([3.0], dtype=np.float32))[0] == -1
    assert ora.ce_loss(x, np.array([-1.0], dtype=np.float32))[0] == -1


@pytest.mark.parametrize("dt,tol", [(np.float64, 1e-13), (np.float32, 2e-6)])
def test_ce_loss_closed_form(dt, tol):
    rng = np.random.default_rng(5)
    x = rng.normal(0, 3, (300, 37)).astype(dt)
    t = rng.integers(0, 37, 300)
    xd = x.astype(np.float64)
    m = xd.max(axis=1, keepdims=True)
    p = np.exp(xd - m) / np.exp(xd - m).sum(axis=1, keepdims=True)
    want = np.mean(-np.log(p[np.arange(300), t] + 1e-7))
    rc, got = ora.ce_loss(x, t.astype(dt))
    assert rc == 0 and abs(got - want) <= tol * abs(want)
