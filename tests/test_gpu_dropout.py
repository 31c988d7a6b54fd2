"""Dropout parity (training_ops.asm:718-858) through the C-ABI.

The device stream is compared with the C library's rand() itself: after
neural_dropout_seed(s) and ora.srand(s), every forward call's mask and output
must equal the oracle's (which calls rand() once per element, as the
reference does) bit for bit -- across consecutive calls (the stream
continues), for lengths around the 31-draw period and the 248-draw segment,
for p on the threshold's rounding edge, and for host, device and unaligned
buffers.  The backward is compared bit for bit with its closed form.
"""

import ctypes

import numpy as np
import pytest

from conftest import GPU, same_bits

pytestmark = GPU


def _lib():
    from pyneural.core import _lib
    return _lib


def _fwd_host(x, p):
    out = np.empty_like(x)
    mask = np.empty(x.size, np.uint8)
    rc = _lib().neural_dropout_forward(x.ctypes.data, out.ctypes.data, mask.ctypes.data, x.size, ctypes.c_float(p))
    assert rc == 0
    return out, mask


@pytest.mark.parametrize("seed", [1, 77, 2 ** 31 + 5])
def test_stream_across_calls(pn, ora, seed):
    rng = np.random.default_rng(seed & 0xFFFF)
    assert _lib().neural_dropout_seed(ctypes.c_uint32(seed)) == 0
    ora.srand(seed)
    total = 0
    # around the 31-draw period, the 372-draw thread segment, the 23,808-draw
    # wave group and the 93 stream values carried between calls
    for n in [1, 5, 30, 31, 32, 92, 93, 94, 371, 372, 373, 744, 23_807, 23_808, 23_809, 100_003, 7,
              65_536 * 3 + 1]:
        x = rng.normal(0, 1, n).astype(np.float32)
        p = 0.5 if n % 2 else 0.3
        out, mask = _fwd_host(x, p)
        _, wout, wmask = ora.dropout_forward(x, p)
        same_bits(mask, wmask)
        same_bits(out, wout)
        total += n
    assert _lib().neural_dropout_draws() == total


@pytest.mark.parametrize("p", [0.0, 0.5, 0.1, 0.9, 1.0 / 3.0, 1.0, float("nan"), -0.25, 1.5])
def test_probabilities(pn, ora, p):
    rng = np.random.default_rng(3)
    x = rng.normal(0, 2, 50_000).astype(np.float32)
    x[::97] = np.nan
    _lib().neural_dropout_seed(ctypes.c_uint32(12))
    ora.srand(12)
    out, mask = _fwd_host(x, p)
    _, wout, wmask = ora.dropout_forward(x, p)
    same_bits(mask, wmask)
    same_bits(out, wout)


def test_device_and_unaligned_buffers(pn, ora):
    import torch
    rng = np.random.default_rng(4)
    n = 1_000_003
    x = rng.normal(0, 1, n + 1).astype(np.float32)
    xd = torch.from_numpy(x).cuda()
    od = torch.empty(n + 1, device="cuda")
    md = torch.empty(n + 4, dtype=torch.uint8, device="cuda")
    torch.cuda.synchronize()
    _lib().neural_dropout_seed(ctypes.c_uint32(5))
    ora.srand(5)
    # aligned device buffers
    assert _lib().neural_dropout_forward(xd.data_ptr(), od.data_ptr(), md.data_ptr(), n, ctypes.c_float(0.4)) == 0
    _, wout, wmask = ora.dropout_forward(x[:n], 0.4)
    same_bits(od.cpu().numpy()[:n], wout)
    same_bits(md.cpu().numpy()[:n], wmask)
    # element 1 onwards: 4-byte offset input/output, 1-byte offset mask
    assert _lib().neural_dropout_forward(xd.data_ptr() + 4, od.data_ptr() + 4, md.data_ptr() + 1, n,
                                         ctypes.c_float(0.4)) == 0
    _, wout, wmask = ora.dropout_forward(x[1:], 0.4)
    same_bits(od.cpu().numpy()[1:], wout)
    same_bits(md.cpu().numpy()[1:n + 1], wmask)


def test_large_stream(pn, ora):
    # 64 M draws in one call (270 K segments) then a short continuation
    n = 1 << 26
    x = np.ones(n, np.float32)
    _lib().neural_dropout_seed(ctypes.c_uint32(2024))
    ora.srand(2024)
    out, mask = _fwd_host(x, 0.25)
    _, wout, wmask = ora.dropout_forward(x, 0.25)
    same_bits(mask, wmask)
    same_bits(out, wout)
    out, mask = _fwd_host(x[:1000], 0.25)
    _, wout, wmask = ora.dropout_forward(x[:1000], 0.25)
    same_bits(mask, wmask)
    # a length that is not a multiple of the segment or the wave group
    m = (1 << 23) + 1003
    out, mask = _fwd_host(x[:m], 0.6)
    _, wout, wmask = ora.dropout_forward(x[:m], 0.6)
    same_bits(mask, wmask)
    same_bits(out, wout)


def test_repeated_calls_made_ahead(pn, ora):
    """A call that repeats the previous call's draws and threshold makes the
    next call's keep bits during its apply pass; the next call with the same
    (n, p) uses them, also after a change of stream (which synchronises the
    old stream).  Every path around that is checked
    against the C library's rand(): streaks of identical calls (with tails of
    1-3 elements and a single-vector call), a change of p or n inside a streak,
    alternating sizes, p = 0 and p = 1 streaks, a reseed inside a streak, an
    unaligned call that takes made-ahead bits, and a change of stream."""
    import torch
    lib = _lib()
    rng = np.random.default_rng(11)
    lib.neural_dropout_seed(ctypes.c_uint32(31337))
    ora.srand(31337)
    total = [0]

    def call(x, p, dev=None):
        if dev is None:
            out, mask = _fwd_host(x, p)
        else:
            xd, od, md, off = dev
            n = x.size
            assert lib.neural_dropout_forward(xd.data_ptr() + 4 * off, od.data_ptr() + 4 * off, md.data_ptr() + off,
                                              n, ctypes.c_float(p)) == 0
            out, mask = od.cpu().numpy()[off:off + n], md.cpu().numpy()[off:off + n]
        _, wout, wmask = ora.dropout_forward(x, p)
        same_bits(mask, wmask)
        same_bits(out, wout)
        total[0] += x.size

    xs = {n: rng.normal(0, 1, n).astype(np.float32) for n in (4, 5, 1000, 71_431, 1 << 20, 23_808 * 3 + 7)}
    for n in (4, 5, 1000, 71_431, 23_808 * 3 + 7, 1 << 20):
        for _ in range(4):
            call(xs[n], 0.5)
    for p in (0.5, 0.5, 0.25, 0.25, 0.25, 0.5, 0.5):          # p changes inside streaks
        call(xs[1 << 20], p)
    for n in (1000, 71_431, 1000, 71_431, 1000, 1000, 1000):   # alternating sizes, then a streak
        call(xs[n], 0.3)
    for p in (0.0, 0.0, 0.0, 1.0, 1.0, 1.0):                    # keep everything / nothing
        call(xs[71_431], p)
    call(xs[71_431], 0.7)
    call(xs[71_431], 0.7)                                       # makes bits ahead
    lib.neural_dropout_seed(ctypes.c_uint32(99))               # ... which the reseed drops
    ora.srand(99)
    total[0] = 0                                                # draws count from the last seed
    call(xs[71_431], 0.7)
    call(xs[71_431], 0.7)
    call(xs[71_431], 0.7)
    # device buffers: an aligned streak, then an unaligned call with the same
    # (n, p), which uses the bits made ahead and makes none
    n = 71_431
    xd = torch.from_numpy(np.concatenate([xs[n], xs[n]])).cuda()
    od = torch.empty(2 * n, device="cuda")
    md = torch.empty(2 * n, dtype=torch.uint8, device="cuda")
    torch.cuda.synchronize()
    call(xs[n], 0.4, (xd, od, md, 0))
    call(xs[n], 0.4, (xd, od, md, 0))
    call(xs[n], 0.4, (xd, od, md, 0))
    call(np.concatenate([xs[n], xs[n]])[1:n + 1], 0.4, (xd, od, md, 1))
    call(xs[n], 0.4, (xd, od, md, 0))
    call(xs[n], 0.4, (xd, od, md, 0))
    # a change of stream inside a streak
    s = torch.cuda.Stream()
    try:
        call(xs[n], 0.4, (xd, od, md, 0))                       # makes bits ahead on the library's stream
        lib.neural_hip_set_stream(ctypes.c_void_p(s.cuda_stream))
        with torch.cuda.stream(s):
            call(xs[n], 0.4, (xd, od, md, 0))
            call(xs[n], 0.4, (xd, od, md, 0))
            call(xs[n], 0.4, (xd, od, md, 0))
            torch.cuda.synchronize()
    finally:
        lib.neural_hip_reset_stream()
    call(xs[n], 0.4, (xd, od, md, 0))
    call(xs[n], 0.4, (xd, od, md, 0))
    assert lib.neural_dropout_draws() == total[0]


def test_backward(pn, ora):
    rng = np.random.default_rng(6)
    n = 300_007
    go = rng.normal(0, 1, n).astype(np.float32)
    go[::101] = np.inf
    mask = rng.integers(0, 4, n).astype(np.uint8)  # any nonzero byte keeps
    for p in [0.5, 0.2, 0.0]:
        gi = np.empty_like(go)
        assert _lib().neural_dropout_backward(go.ctypes.data, gi.ctypes.data, mask.ctypes.data, n,
                                              ctypes.c_float(p)) == 0
        _, want = ora.dropout_backward(go, mask, p)
        same_bits(gi, want)


def test_module(pn, ora):
    rng = np.random.default_rng(7)
    x = rng.normal(0, 1, (64, 257)).astype(np.float32)
    t = pn.Tensor.from_numpy(x)
    pn.dropout_seed(9)
    ora.srand(9)
    drop = pn.Dropout(0.3)
    y = drop(t)
    _, wout, wmask = ora.dropout_forward(x.reshape(-1), 0.3)
    same_bits(y.numpy().reshape(-1), wout)
    same_bits(drop.mask(), wmask)
    g = rng.normal(0, 1, x.shape).astype(np.float32)
    gi = drop.backward(pn.Tensor.from_numpy(g))
    _, wg = ora.dropout_backward(g.reshape(-1), wmask, 0.3)
    same_bits(gi.numpy().reshape(-1), wg)
    drop.eval()
    same_bits(drop(t).numpy(), x)
    drop.train()
    drop.p = 1.0
    before = _lib().neural_dropout_draws()
    assert not drop(t).numpy().any()
    assert _lib().neural_dropout_draws() == before  # p == 1 takes no draws
    with pytest.raises(ValueError):
        pn.Dropout(1.5)


def test_errors(pn):
    lib = _lib()
    buf = np.zeros(4, np.float32)
    m = np.zeros(4, np.uint8)
    assert lib.neural_dropout_forward(None, buf.ctypes.data, m.ctypes.data, 4, ctypes.c_float(0.5)) == 1
    assert lib.neural_dropout_backward(buf.ctypes.data, buf.ctypes.data, None, 4, ctypes.c_float(0.5)) == 1
    assert lib.neural_dropout_forward(buf.ctypes.data, buf.ctypes.data, m.ctypes.data, 0, ctypes.c_float(0.5)) == 0
