"""NaN bits through the ops that only move, select or flip the sign of values.

The comparisons elsewhere take NaNs by class.  Here the bits themselves are
held: negation is a sign-bit XOR that also flips a NaN's sign and keeps its
payload (ew_neg, math_kernels.asm:843-945); maximum returns b whenever
a > b is false, so a NaN in either operand comes out as b's exact bits
(vmaxps, math_kernels.asm:730-835); tensor copy and the 2-D tensor ops move
bits unchanged (neural_api.asm:905-967, tensor_ops.c:15-148).  Quiet and
signalling NaNs of both signs with assorted payloads, in both dtypes.
"""

import ctypes

import numpy as np
import pytest

from conftest import GPU

pytestmark = GPU


def _nans(dt, n, rng):
    if dt == np.float32:
        u, exp, quiet, mant = np.uint32, 0x7F800000, 0x00400000, 0x003FFFFF
    else:
        u, exp, quiet, mant = np.uint64, 0x7FF0000000000000, 0x0008000000000000, 0x0007FFFFFFFFFFFF
    bits = rng.integers(1, mant, n, dtype=np.int64).astype(u)
    bits |= u(exp)
    bits[rng.random(n) < 0.5] |= u(quiet)
    sign = u(1) << u(31 if dt == np.float32 else 63)
    bits[rng.random(n) < 0.5] |= sign
    return bits.view(dt), u, sign


@pytest.mark.parametrize("dt", [np.float32, np.float64])
def test_nan_bits_moved_selected_negated(pn, dt):
    lib = pn.core._lib
    rng = np.random.default_rng(404)
    n = 4099
    x, u, sign = _nans(dt, n, rng)
    vals = rng.normal(0, 1, n).astype(dt)
    mixed = np.where(rng.random(n) < 0.5, x, vals)  # NaNs among ordinary values
    ta = pn.Tensor.from_numpy(mixed)
    # negation: every element's bits XOR the sign bit
    out = pn.Tensor.create([n], ta.dtype)
    assert lib.neural_neg(out._ptr, ta._ptr) == 0
    assert np.array_equal(out.numpy().view(u), mixed.view(u) ^ sign)
    # maximum: (a > b) ? a : b, bit for bit, NaNs on either side
    other, _, _ = _nans(dt, n, rng)
    b = np.where(rng.random(n) < 0.5, other, rng.normal(0, 1, n).astype(dt))
    tb = pn.Tensor.from_numpy(b)
    assert lib.neural_maximum(out._ptr, ta._ptr, tb._ptr) == 0
    with np.errstate(invalid="ignore"):
        want = np.where(mixed > b, mixed, b)
    assert np.array_equal(out.numpy().view(u), want.view(u))
    # copy
    assert lib.neural_tensor_copy(out._ptr, ta._ptr) == 0
    assert np.array_equal(out.numpy().view(u), mixed.view(u))


def test_nan_bits_through_2d_tensor_ops(pn):
    lib = pn.core._lib
    rng = np.random.default_rng(405)
    r, c = 37, 53
    x, u, _ = _nans(np.float64, r * c, rng)
    x = np.where(rng.random(r * c) < 0.5, x, rng.normal(0, 1, r * c)).reshape(r, c)
    out = np.zeros(r * c)
    assert lib.tensor_transpose2d_array(x.ctypes.data, r, c, out.ctypes.data) == 0
    assert np.array_equal(out.view(u), np.ascontiguousarray(x.T).reshape(-1).view(u))
    dims = [ctypes.c_int64() for _ in range(2)]
    cat = np.zeros(2 * r * c)
    assert lib.tensor_concat_2d(x.ctypes.data, x.ctypes.data, r, c, r, c, 1, cat.ctypes.data,
                                ctypes.byref(dims[0]), ctypes.byref(dims[1])) == 0
    assert np.array_equal(cat.view(u), np.concatenate([x, x], axis=1).reshape(-1).view(u))
