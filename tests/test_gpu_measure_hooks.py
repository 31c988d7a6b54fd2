"""The library's measurement entry points (no reference counterpart): the
launch-span timer, the launch counter and the float4 stream copy that the
bench uses as its bandwidth reference.

The span timer must bracket every launch of a multi-launch call (a
whole-tensor sum of 2^24 values is a segment launch and a combine launch), so
the span is at least each of its kernels; the counter must count the launches
a call makes; the copy must copy, and reject what it cannot take.
"""

import ctypes
from pathlib import Path

import numpy as np

from conftest import GPU

pytestmark = GPU


def _hip():
    import torch
    hip = ctypes.CDLL(str(Path(torch.__file__).parent / "lib" / "libamdhip64.so"))
    hip.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
    hip.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
    hip.hipEventDestroy.argtypes = [ctypes.c_void_p]
    return hip


def test_launch_span_and_count(pn):
    import torch
    hip = _hip()
    lib = pn.core._lib
    rng = np.random.default_rng(7)
    big = pn.Tensor.from_numpy(rng.uniform(-1, 1, 1 << 24).astype(np.float32))
    rows = pn.Tensor.from_numpy(rng.normal(0, 1, (256, 1024)).astype(np.float32))
    rout = pn.Tensor.create([256])
    r = ctypes.c_double()
    assert lib.neural_sum(big._ptr, ctypes.byref(r)) == 0
    want = r.value
    # launches per call: two for the whole-tensor sum, one for a row sum
    c0 = lib.neural_hip_launch_count()
    assert lib.neural_sum(big._ptr, ctypes.byref(r)) == 0
    c1 = lib.neural_hip_launch_count()
    assert lib.neural_reduce_sum(rows._ptr, 1, rout._ptr) == 0
    c2 = lib.neural_hip_launch_count()
    assert (c1 - c0, c2 - c1) == (2, 1)
    s = torch.cuda.current_stream()
    lib.neural_hip_set_stream(ctypes.c_void_p(s.cuda_stream))
    ev = []
    try:
        def pair():
            e0, e1 = ctypes.c_void_p(), ctypes.c_void_p()
            assert hip.hipEventCreate(ctypes.byref(e0)) == 0 and hip.hipEventCreate(ctypes.byref(e1)) == 0
            ev.extend([e0, e1])
            return e0, e1

        def elapsed(e0, e1):
            ms = ctypes.c_float()
            assert hip.hipEventElapsedTime(ctypes.byref(ms), e0, e1) == 0
            return ms.value

        spans, segs, combs = [], [], []
        for _ in range(5):
            a, b, c = pair(), pair(), pair()
            assert lib.neural_hip_time_launches(a[0], a[1], 0, 2) == 0
            assert lib.neural_sum(big._ptr, ctypes.byref(r)) == 0 and r.value == want
            assert lib.neural_hip_time_launches(b[0], b[1], 0, 1) == 0
            assert lib.neural_sum(big._ptr, ctypes.byref(r)) == 0 and r.value == want
            assert lib.neural_hip_time_launches(c[0], c[1], 1, 1) == 0
            assert lib.neural_sum(big._ptr, ctypes.byref(r)) == 0 and r.value == want
            torch.cuda.synchronize()
            spans.append(elapsed(*a))
            segs.append(elapsed(*b))
            combs.append(elapsed(*c))
        span, seg, comb = np.median(spans), np.median(segs), np.median(combs)
        # the span holds both kernels (and the gap between them)
        assert span > seg and span > comb, (span, seg, comb)
        assert span >= 0.9 * (seg + comb), (span, seg, comb)
        # a span counts launches, not calls: count = 3 brackets the sum's two
        # launches and the next row sum's one, then the timer is spent
        d = pair()
        assert lib.neural_hip_time_launches(d[0], d[1], 0, 3) == 0
        assert lib.neural_sum(big._ptr, ctypes.byref(r)) == 0
        assert lib.neural_reduce_sum(rows._ptr, 1, rout._ptr) == 0
        assert lib.neural_reduce_sum(rows._ptr, 1, rout._ptr) == 0  # nothing armed any more
        torch.cuda.synchronize()
        assert elapsed(*d) >= 0.9 * span, (elapsed(*d), span)
        assert lib.neural_hip_time_launches(a[0], a[1], 0, 0) == pn.NeuralError.INVALID_ARGUMENT
        assert lib.neural_hip_time_launches(a[0], a[1], -1, 1) == pn.NeuralError.INVALID_ARGUMENT
        assert lib.neural_hip_time_launches(None, a[1], 0, 1) == pn.NeuralError.NULL_POINTER
    finally:
        lib.neural_hip_time_cancel()
        lib.neural_hip_reset_stream()
        for e in ev:
            hip.hipEventDestroy(e)


def test_stream_copy(pn):
    import torch
    lib = pn.core._lib
    for n in (4, 1000, (1 << 22) + 12, 1 << 26):
        src = torch.randn(n, device="cuda")
        full = torch.full((n + 64,), 7.0, device="cuda")  # 64 values past the copy stay untouched
        torch.cuda.synchronize()
        assert lib.neural_hip_stream_copy(ctypes.c_void_p(full.data_ptr()), ctypes.c_void_p(src.data_ptr()),
                                          4 * n) == 0
        torch.cuda.synchronize()
        assert torch.equal(src, full[:n])
        assert torch.all(full[n:] == 7.0)
    src = torch.randn(1024, device="cuda")
    dst = torch.zeros_like(src)
    host = np.zeros(1024, dtype=np.float32)
    bad = pn.NeuralError.INVALID_ARGUMENT
    d, s_ = ctypes.c_void_p(dst.data_ptr()), ctypes.c_void_p(src.data_ptr())
    assert lib.neural_hip_stream_copy(d, s_, 4 * 1024 - 4) == bad                       # not a multiple of 16
    assert lib.neural_hip_stream_copy(ctypes.c_void_p(dst.data_ptr() + 4), s_, 1024) == bad  # unaligned
    assert lib.neural_hip_stream_copy(ctypes.c_void_p(host.ctypes.data), s_, 1024) == bad     # host memory
    assert lib.neural_hip_stream_copy(None, s_, 1024) == pn.NeuralError.NULL_POINTER
    torch.cuda.synchronize()
    assert torch.all(dst == 0.0)
