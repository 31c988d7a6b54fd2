"""Launch grids past HIP's limit of 2^32 work-items per grid dimension (2^24
blocks of 256 lanes).  The row kernels (softmax / log-softmax, the CE losses),
the column sums, the per-feature statistics and the 2-D transpose cap their
grids and step through the remaining rows, columns, features or tiles; these
cases sit just past the point where one block (or wave) per item would need
more blocks than a launch can have, and check the items that only the second
pass of the loop reaches.

Expected values: softmax and log-softmax from torch in float64 (REL32 with
the same floors as the other softmax tests); CE from the formula of
label_smoothing_ce_forward (metrics_losses.c:47-64) in float64; column sums of
one row, statistics of one row and the transpose are exact closed forms.

Peak device memory of one test: ~64 GB (the column sum: a 16 GiB row, its
16 GiB result and 32 GiB of float64 partials).
"""

import ctypes

import numpy as np
import pytest

from conftest import GPU

pytestmark = GPU

WAVE_ROWS = 4 * ((1 << 24) - 1)   # rows one launch of row-per-wave blocks can cover
BLOCK_ROWS = (1 << 24) - 1        # rows one launch of row-per-block blocks can cover


@pytest.fixture
def lib(pn):
    import torch
    pn.set_stream(torch.cuda.current_stream().cuda_stream)
    yield pn.core._lib
    torch.cuda.synchronize()
    pn.set_stream(None)
    torch.cuda.empty_cache()
    pn.core._lib.neural_hip_empty_cache()


def _normal(shape, seed, dtype):
    import torch
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    return torch.randn(*shape, device="cuda", dtype=dtype, generator=g) * 3.0


def _softmax_case(pn, lib, rows, cols, dtype, seed):
    import torch
    s = _normal((rows, cols), seed, dtype)
    p, lp = torch.empty_like(s), torch.empty_like(s)
    ts, tp, tl = pn.Tensor.from_torch(s), pn.Tensor.from_torch(p), pn.Tensor.from_torch(lp)
    torch.cuda.synchronize()
    pn.core._check_error(lib.neural_softmax(tp._ptr, ts._ptr), "softmax")
    pn.core._check_error(lib.neural_log_softmax(tl._ptr, ts._ptr), "log_softmax")
    torch.cuda.synchronize()
    f32 = dtype == torch.float32
    rel, floor = (1e-5, 1e-6) if f32 else (1e-12, 1e-14)
    # the first rows, rows around each launch-size boundary, the last rows
    pick = torch.tensor([0, 1, BLOCK_ROWS - 1, BLOCK_ROWS, BLOCK_ROWS + 1, rows // 2]
                        + ([WAVE_ROWS - 1, WAVE_ROWS, WAVE_ROWS + 1] if rows > WAVE_ROWS else [])
                        + [rows - 2, rows - 1], device="cuda")
    want = torch.softmax(s[pick].double(), dim=1)
    assert bool(((p[pick].double() - want).abs() <= rel * want).all())
    lwant = torch.log_softmax(s[pick].double(), dim=1)
    assert bool(((lp[pick].double() - lwant).abs() <= rel * lwant.abs() + floor).all())
    # every row: a softmax row sums to 1, and exp of the log-softmax row does too
    sums = torch.sum(p, dim=1, dtype=torch.float64)
    assert bool(((sums - 1.0).abs() < rel).all())
    lsums = torch.sum(torch.exp(lp.double()), dim=1)
    assert bool(((lsums - 1.0).abs() < rel).all())


def test_softmax_wave_rows_past_grid(pn, lib):
    import torch
    # f32 rows of 4 (one wave per row), f64 rows of 2
    _softmax_case(pn, lib, WAVE_ROWS + 4100, 4, torch.float32, 11)
    _softmax_case(pn, lib, WAVE_ROWS + 4100, 2, torch.float64, 12)


def test_softmax_block_rows_past_grid(pn, lib):
    import torch
    # rows of 3 values are not 16-byte vectors: one block per row
    _softmax_case(pn, lib, BLOCK_ROWS + 4100, 3, torch.float32, 13)


def test_ce_rows_past_grid(pn, lib):
    import torch
    b, k, a = WAVE_ROWS + 4100, 2, 0.1
    x = _normal((b, k), 14, torch.float32)
    g = torch.Generator(device="cuda")
    g.manual_seed(15)
    t = torch.randint(0, k, (b,), device="cuda", generator=g, dtype=torch.int64)
    grad = torch.empty_like(x)
    loss = ctypes.c_double()
    torch.cuda.synchronize()
    assert lib.label_smoothing_ce_fused_f32(x.data_ptr(), t.data_ptr(), b, k, a, ctypes.byref(loss),
                                            grad.data_ptr()) == 0
    torch.cuda.synchronize()
    xd = x.double()
    y = torch.full_like(xd, a / k)
    y.scatter_add_(1, t.view(-1, 1), torch.full((b, 1), 1.0 - a, device="cuda", dtype=torch.float64))
    lsm = torch.log_softmax(xd, dim=1)
    want = float(-(y * lsm).sum(dim=1).mean())
    assert abs(loss.value - want) <= 1e-6 * abs(want), (loss.value, want)
    # gradient rows that only the second pass over the grid reaches, and the first rows
    for lo, hi in ((0, 4096), (WAVE_ROWS - 8, b)):
        gw = (torch.exp(lsm[lo:hi]) - y[lo:hi]) / b
        assert bool(((grad[lo:hi].double() - gw).abs() <= 1e-5 * gw.abs() + 1e-7 / b).all()), (lo, hi)
    del xd, y, lsm


def test_column_sum_past_grid(pn, lib):
    import torch
    # [1, 2^32 + 1000] f32: column sums of a single row are the row itself,
    # its column means the row divided by 1
    n = (1 << 32) + 1000
    x = _normal((1, n), 16, torch.float32)
    out = torch.empty(n, device="cuda")
    tx, to = pn.Tensor.from_torch(x), pn.Tensor.from_torch(out)
    torch.cuda.synchronize()
    pn.core._check_error(lib.neural_reduce_sum(tx._ptr, 0, to._ptr), "reduce_sum axis 0")
    torch.cuda.synchronize()
    assert torch.equal(out, x[0])
    out.zero_()
    torch.cuda.synchronize()
    pn.core._check_error(lib.neural_reduce_mean(tx._ptr, 0, to._ptr), "reduce_mean axis 0")
    torch.cuda.synchronize()
    assert torch.equal(out, x[0])


def test_feature_stats_past_grid(pn, lib):
    # one row of 2^24 + 100 features: mean = min = max = x, std = 0
    f = (1 << 24) + 100
    rng = np.random.default_rng(17)
    x = rng.normal(0, 3, f)
    outs = [np.full(f, 7.0) for _ in range(4)]
    assert lib.transform_compute_stats(x.ctypes.data, 1, f, *[o.ctypes.data for o in outs]) == 0
    mean, std, mn, mx = outs
    assert np.array_equal(mean, x) and np.array_equal(mn, x) and np.array_equal(mx, x)
    assert np.all(std == 0.0)


@pytest.mark.parametrize("rows,cols", [(3_000_000, 3), (1, 3_000_000)])
def test_transpose_past_grid(pn, lib, rows, cols):
    # more than 65535 tiles of 32 along one dimension
    x = np.random.default_rng(18).normal(0, 1, (rows, cols))
    out = np.full((cols, rows), 7.0)
    assert lib.tensor_transpose2d_array(x.ctypes.data, rows, cols, out.ctypes.data) == 0
    assert np.array_equal(out, x.T)
