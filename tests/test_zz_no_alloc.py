"""calibrate_minmax_f32_dev_noalloc: the allocation-free variant of
calibrate_minmax_f32_dev (segment summaries in a static per-GPU device
buffer).  Its QuantParams must equal the allocating entry point's bit for
bit, on consecutive calls whose second input is smaller (the buffer keeps
the previous call's summaries), for the symmetric and affine modes, and on
inputs small enough to need no summaries at all."""

import ctypes

import numpy as np
import pytest

from conftest import GPU

pytestmark = GPU


def _params_dev(torch):
    return torch.zeros(5, dtype=torch.float64, device="cuda")  # 40 bytes: one QuantParams


def _bytes(t):
    """The QuantParams fields (scale, zero_point | min_val, max_val,
    symmetric) without the two 4-byte padding holes, which no kernel writes."""
    b = t.cpu().numpy().tobytes()
    return b[0:12] + b[16:36]


def _alloc_stats(lib):
    """(allocator requests, hipMalloc calls) the library has made so far."""
    a, m = ctypes.c_ulonglong(), ctypes.c_ulonglong()
    assert lib.neural_hip_alloc_stats(ctypes.byref(a), ctypes.byref(m)) == 0
    return a.value, m.value


@pytest.mark.parametrize("sym", [1, 0])
def test_noalloc_matches_allocating_entry_point(pn, sym):
    import torch
    lib = pn.core._lib
    g = torch.Generator(device="cuda")
    g.manual_seed(9 + sym)
    sizes = [(1 << 24) + 5, (1 << 20) + 3, 4099, 1]   # each call smaller than the one before
    big = torch.empty(sizes[0], device="cuda")
    big.exponential_(generator=g)
    big *= torch.randint(0, 2, (sizes[0],), device="cuda", generator=g).float() * 2 - 1
    big[123] = 50.0
    big[sizes[0] - 7] = -50.0
    big[sizes[1] - 2] = -0.0
    for n in sizes:
        x = big[:n]
        want, got = _params_dev(torch), _params_dev(torch)
        got.fill_(np.nan)
        assert lib.calibrate_minmax_f32_dev(x.data_ptr(), n, sym, want.data_ptr()) == 0
        torch.cuda.synchronize()
        before = _alloc_stats(lib)
        assert lib.calibrate_minmax_f32_dev_noalloc(x.data_ptr(), n, sym, got.data_ptr()) == 0
        torch.cuda.synchronize()
        assert _alloc_stats(lib) == before, f"the allocation-free entry point allocated (n = {n})"
        assert _bytes(got) == _bytes(want), (n, sym, got.cpu(), want.cpu())
    # a second round over the same sizes in reverse order: the buffer holds the
    # previous (smaller) call's summaries
    for n in sizes[::-1]:
        x = big[:n]
        want, got = _params_dev(torch), _params_dev(torch)
        assert lib.calibrate_minmax_f32_dev(x.data_ptr(), n, sym, want.data_ptr()) == 0
        assert lib.calibrate_minmax_f32_dev_noalloc(x.data_ptr(), n, sym, got.data_ptr()) == 0
        torch.cuda.synchronize()
        assert _bytes(got) == _bytes(want), (n, sym)


def test_noalloc_rejects_host_buffers(pn):
    import torch
    lib = pn.core._lib
    x = np.linspace(-1, 1, 1000).astype(np.float32)
    p = torch.zeros(5, dtype=torch.float64, device="cuda")
    assert lib.calibrate_minmax_f32_dev_noalloc(x.ctypes.data, x.size, 1, p.data_ptr()) == -1
    assert lib.neural_get_last_error() == pn.NeuralError.INVALID_ARGUMENT
    xd = torch.from_numpy(x).cuda()
    assert lib.calibrate_minmax_f32_dev_noalloc(xd.data_ptr(), 0, 1, p.data_ptr()) == -1
    assert lib.calibrate_minmax_f32_dev_noalloc(None, 10, 1, p.data_ptr()) == -1
    assert lib.neural_get_last_error() == pn.NeuralError.NULL_POINTER
    assert lib.calibrate_minmax_f32_dev_noalloc(xd.data_ptr(), x.size, 1, p.data_ptr()) == 0
