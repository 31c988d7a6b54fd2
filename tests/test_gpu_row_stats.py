"""The fused row-statistics entry points (no counterpart in the reference).

neural_row_stats and neural_bias_add_row_stats must give, bit for bit, what
the stand-alone calls give on the same rows: neural_reduce_sum / _mean /
_max (axis = last dim), neural_reduce_argmax and neural_bias_add.  Those are
pinned against the oracle by test_gpu_reduce.py and test_gpu_elementwise.py;
the max chain and argmax are also checked against the oracle here.  Shapes
cover every grid the reductions use: one wave per row (cols <= 2048), one
block per row, segmented rows (few long rows: the fused bias entry takes its
two-call route there), unaligned rows (no 16-byte vectors) and single
elements.
"""

import ctypes

import numpy as np
import pytest

from conftest import GPU, same_bits

pytestmark = GPU

SHAPES = [(8192, 4096), (1000, 1000), (513, 1023), (300, 2049), (5000, 2048), (3, 70000), (37, 5), (1, 1)]


def _rows(rows, cols, dt, seed):
    rng = np.random.default_rng(seed)
    x = rng.normal(0, 3, (rows, cols)).astype(dt)
    if rows > 4 and cols > 3:
        x[1, 2] = np.nan            # NaN mid-row: the max chain restarts after it
        x[2, cols - 1] = np.nan     # NaN last: row max NaN
        x[0, :] = 0.0
        x[0, 1::2] = -0.0           # zero ties: the later zero wins the chain
        x[3, :] = 7.0               # argmax ties: the first index
        x[4, cols // 2] = np.inf
        x[4, 0] = -np.inf
    return x


def _separate(pn, t, rows):
    """sum, mean, max, argmax of t's rows from the four stand-alone calls."""
    lib = pn.core._lib
    outs = [pn.Tensor.create([rows], t.dtype) for _ in range(3)]
    pn.core._check_error(lib.neural_reduce_sum(t._ptr, 1, outs[0]._ptr), "reduce_sum")
    pn.core._check_error(lib.neural_reduce_mean(t._ptr, 1, outs[1]._ptr), "reduce_mean")
    pn.core._check_error(lib.neural_reduce_max(t._ptr, 1, outs[2]._ptr), "reduce_max")
    idx = np.empty(rows, dtype=np.int64)
    pn.core._check_error(lib.neural_reduce_argmax(t._ptr, 1, idx.ctypes.data), "reduce_argmax")
    return [o.numpy() for o in outs] + [idx]


def _fused_outputs(pn, rows, dtype):
    outs = [pn.Tensor.create([rows], dtype) for _ in range(3)]
    idx = np.full(rows, -7, dtype=np.int64)
    return outs, idx


@pytest.mark.parametrize("rows,cols", SHAPES)
@pytest.mark.parametrize("dt", [np.float32, np.float64])
def test_row_stats_equal_separate_calls(pn, ora, rows, cols, dt):
    x = _rows(rows, cols, dt, rows * 31 + cols)
    t = pn.Tensor.from_numpy(x)
    want = _separate(pn, t, rows)
    outs, idx = _fused_outputs(pn, rows, t.dtype)
    rc = pn.core._lib.neural_row_stats(t._ptr, outs[0]._ptr, outs[1]._ptr, outs[2]._ptr, idx.ctypes.data)
    pn.core._check_error(rc, "neural_row_stats")
    for got, w in zip([o.numpy() for o in outs] + [idx], want):
        same_bits(got, w)
    same_bits(outs[2].numpy(), ora.rowmax_chain(x))
    same_bits(idx, ora.rowargmax(x))


@pytest.mark.parametrize("rows,cols", SHAPES)
@pytest.mark.parametrize("dt", [np.float32, np.float64])
def test_bias_add_row_stats_equal_separate_calls(pn, ora, rows, cols, dt):
    x = _rows(rows, cols, dt, rows * 17 + cols)
    rng = np.random.default_rng(cols)
    b = rng.normal(0, 3, cols).astype(dt)
    if cols > 6:
        b[5] = -0.0
        b[6] = np.inf
    lib = pn.core._lib
    tx, tb = pn.Tensor.from_numpy(x), pn.Tensor.from_numpy(b)
    y_ref = pn.Tensor.create([rows, cols], tx.dtype)
    pn.core._check_error(lib.neural_bias_add(y_ref._ptr, tx._ptr, tb._ptr), "bias_add")
    want = _separate(pn, y_ref, rows)
    y = pn.Tensor.create([rows, cols], tx.dtype)
    outs, idx = _fused_outputs(pn, rows, tx.dtype)
    rc = lib.neural_bias_add_row_stats(y._ptr, tx._ptr, tb._ptr, outs[0]._ptr, outs[1]._ptr, outs[2]._ptr,
                                       idx.ctypes.data)
    pn.core._check_error(rc, "neural_bias_add_row_stats")
    same_bits(y.numpy(), y_ref.numpy())
    same_bits(y.numpy(), x + b)
    for got, w in zip([o.numpy() for o in outs] + [idx], want):
        same_bits(got, w)
    yv = x + b
    same_bits(outs[2].numpy(), ora.rowmax_chain(yv))
    same_bits(idx, ora.rowargmax(yv))


@pytest.mark.parametrize("cols", [300, 4096])
@pytest.mark.parametrize("dt", [np.float32, np.float64])
def test_bias_add_row_stats_in_place(pn, ora, cols, dt):
    """out == in (the in-place bias add of a linear layer): rows whose maximum
    after the add is a zero (signed zeros mixed), rows with NaN before and
    after the zeros, and rows with +-Inf give the two separate calls' bits."""
    rows = 64
    rng = np.random.default_rng(cols + 3)
    b = rng.normal(0, 3, cols).astype(dt)
    b[7] = -0.0
    x = (-np.abs(rng.normal(0, 3, (rows, cols))) - b).astype(dt)  # x + b <= 0 (rounded)
    for r in range(0, rows, 4):
        z = rng.choice(np.arange(8, cols), size=5, replace=False)
        x[r, z] = -b[z]                                # +0 after the add: the row's maximum is 0
        x[r, 7] = -0.0                                 # -0 + -0 = -0: zeros of both signs tie
        if r % 8 == 0:
            x[r, z[2]] = np.nan                        # NaN: the chain restarts after it
        x[r + 1, rng.integers(0, cols)] = np.inf
        x[r + 2, rng.integers(0, cols)] = -np.inf
        x[r + 3, cols - 1] = np.nan                    # NaN last: row max NaN
    y_ref = x + b
    lib = pn.core._lib
    want = _separate(pn, pn.Tensor.from_numpy(y_ref), rows)
    t = pn.Tensor.from_numpy(x)
    tb = pn.Tensor.from_numpy(b)
    outs, idx = _fused_outputs(pn, rows, t.dtype)
    rc = lib.neural_bias_add_row_stats(t._ptr, t._ptr, tb._ptr, outs[0]._ptr, outs[1]._ptr, outs[2]._ptr,
                                       idx.ctypes.data)
    pn.core._check_error(rc, "neural_bias_add_row_stats in place")
    same_bits(t.numpy(), y_ref)
    for got, w in zip([o.numpy() for o in outs] + [idx], want):
        same_bits(got, w)
    same_bits(outs[2].numpy(), ora.rowmax_chain(y_ref))
    same_bits(idx, ora.rowargmax(y_ref))


def test_row_stats_subsets_and_device_indices(pn, ora):
    """Any subset of the outputs; argmax into device memory; repeated calls
    give the same bits."""
    import torch

    rows, cols = 4096, 1024
    x = _rows(rows, cols, np.float32, 5)
    t = pn.Tensor.from_numpy(x)
    want = _separate(pn, t, rows)
    lib = pn.core._lib
    mean = pn.Tensor.create([rows])
    pn.core._check_error(lib.neural_row_stats(t._ptr, None, mean._ptr, None, None), "mean only")
    same_bits(mean.numpy(), want[1])
    didx = torch.full((rows,), -1, dtype=torch.int64, device="cuda")
    torch.cuda.synchronize()  # the fill runs on torch's stream, the library's kernels on its own
    mx = pn.Tensor.create([rows])
    for _ in range(2):
        rc = lib.neural_row_stats(t._ptr, None, None, mx._ptr, ctypes.c_void_p(didx.data_ptr()))
        pn.core._check_error(rc, "max + device argmax")
        torch.cuda.synchronize()
        same_bits(mx.numpy(), want[2])
        same_bits(didx.cpu().numpy(), want[3])


def test_row_stats_errors(pn):
    lib = pn.core._lib
    E = pn.NeuralError
    t = pn.Tensor.from_numpy(np.ones((4, 8), dtype=np.float32))
    s = pn.Tensor.create([4])
    idx = np.empty(4, dtype=np.int64)
    assert lib.neural_row_stats(None, s._ptr, None, None, None) == E.NULL_POINTER
    assert lib.neural_row_stats(t._ptr, None, None, None, None) == E.NULL_POINTER
    s5 = pn.Tensor.create([5])
    assert lib.neural_row_stats(t._ptr, s5._ptr, None, None, None) == E.SHAPE_MISMATCH
    d = pn.Tensor.create([4], pn.NeuralDtype.FLOAT64)
    assert lib.neural_row_stats(t._ptr, None, d._ptr, None, None) == E.DTYPE_MISMATCH
    empty_cols = pn.Tensor.create([4, 0])
    assert lib.neural_row_stats(empty_cols._ptr, None, None, None, idx.ctypes.data) == E.INVALID_ARGUMENT
    y = pn.Tensor.create([4, 8])
    b = pn.Tensor.from_numpy(np.ones(8, dtype=np.float32))
    assert lib.neural_bias_add_row_stats(y._ptr, t._ptr, None, s._ptr, None, None, None) == E.NULL_POINTER
    bad_b = pn.Tensor.from_numpy(np.ones(7, dtype=np.float32))
    assert lib.neural_bias_add_row_stats(y._ptr, t._ptr, bad_b._ptr, s._ptr, None, None, None) == E.SHAPE_MISMATCH
    bad_y = pn.Tensor.create([4, 9])
    assert lib.neural_bias_add_row_stats(bad_y._ptr, t._ptr, b._ptr, s._ptr, None, None, None) == E.SHAPE_MISMATCH
    assert lib.neural_bias_add_row_stats(y._ptr, t._ptr, b._ptr, None, None, None, None) == E.NULL_POINTER
    # rows == 0: nothing to do
    zero_rows = pn.Tensor.create([0, 8])
    z = pn.Tensor.create([0])
    assert lib.neural_row_stats(zero_rows._ptr, z._ptr, None, None, None) == 0


def test_tensor_methods(pn):
    """pyneural's Tensor.row_stats / Tensor.bias_add_row_stats."""
    x = _rows(64, 300, np.float32, 9)
    b = np.random.default_rng(1).normal(0, 1, 300).astype(np.float32)
    t = pn.Tensor.from_numpy(x)
    s, m, mx, idx = t.row_stats()
    want = _separate(pn, t, 64)
    for got, w in zip([s.numpy(), m.numpy(), mx.numpy(), idx], want):
        same_bits(got, w)
    y, s, m, mx, idx = t.bias_add_row_stats(pn.Tensor.from_numpy(b))
    same_bits(y.numpy(), x + b)
    want = _separate(pn, pn.Tensor.from_numpy(x + b), 64)
    for got, w in zip([s.numpy(), m.numpy(), mx.numpy(), idx], want):
        same_bits(got, w)
