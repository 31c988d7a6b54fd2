"""Empty tensors (a zero dimension) through the tensor entry points.

Elementwise, broadcast, softmax, activation, fill / copy and scan calls on an
empty tensor succeed and write nothing.  Reductions: a sum over no elements
is 0 and a mean 0 / 0 = NaN; rows of zero length in a [3, 0] tensor give 3
results.  A maximum or argmax of nothing has no value and is refused
(INVALID_ARGUMENT)."""

import ctypes

import numpy as np

from conftest import GPU

pytestmark = GPU


def test_empty_tensors(pn):
    lib = pn.core._lib
    bad = pn.NeuralError.INVALID_ARGUMENT
    for dt in (pn.NeuralDtype.FLOAT32, pn.NeuralDtype.FLOAT64):
        def T(*shape):
            return pn.Tensor.create(list(shape), dt)

        e, e2, e3 = T(0), T(0), T(0)
        m, mo, b5 = T(0, 5), T(0, 5), T(5)
        z, zo = T(3, 0), T(3, 0)
        one, r3 = T(1), T(3)
        assert lib.neural_add(e3._ptr, e._ptr, e2._ptr) == 0
        assert lib.neural_mul(e3._ptr, e._ptr, e2._ptr) == 0
        assert lib.neural_relu(e2._ptr, e._ptr) == 0
        assert lib.neural_bias_add(mo._ptr, m._ptr, b5._ptr) == 0
        assert lib.neural_softmax(mo._ptr, m._ptr) == 0
        assert lib.neural_log_softmax(mo._ptr, m._ptr) == 0
        assert lib.neural_softmax(zo._ptr, z._ptr) == 0
        assert lib.act_gelu(e2._ptr, e._ptr) == 0
        assert lib.neural_tensor_fill(e._ptr, ctypes.c_double(1.0)) == 0
        assert lib.neural_tensor_copy(e2._ptr, e._ptr) == 0
        hn, hi, ss = ctypes.c_int(7), ctypes.c_int(7), ctypes.c_double(7.0)
        assert lib.neural_tensor_scan(e._ptr, ctypes.byref(hn), ctypes.byref(hi), ctypes.byref(ss)) == 0
        assert (hn.value, hi.value, ss.value) == (0, 0, 0.0)
        s = ctypes.c_double(-1.0)
        assert lib.neural_sum(e._ptr, ctypes.byref(s)) == 0 and s.value == 0.0
        # whole-tensor sum / mean of nothing
        assert lib.neural_tensor_fill(one._ptr, ctypes.c_double(5.0)) == 0
        assert lib.neural_reduce_sum(e._ptr, -1, one._ptr) == 0
        assert one.numpy().tolist() == [0.0]
        assert lib.neural_reduce_mean(e._ptr, -1, one._ptr) == 0
        assert np.isnan(one.numpy()[0])
        # rows of zero length: 3 sums of 0, 3 means of NaN
        assert lib.neural_tensor_fill(r3._ptr, ctypes.c_double(5.0)) == 0
        assert lib.neural_reduce_sum(z._ptr, 1, r3._ptr) == 0
        assert r3.numpy().tolist() == [0.0, 0.0, 0.0]
        assert lib.neural_reduce_mean(z._ptr, 1, r3._ptr) == 0
        assert np.all(np.isnan(r3.numpy()))
        # columns of a [3, 0] tensor: none, so an empty output; the 5 columns
        # of a [0, 5] tensor are empty: 5 sums of 0, 5 means of NaN
        assert lib.neural_reduce_sum(z._ptr, 0, T(0)._ptr) == 0
        assert lib.neural_reduce_sum(m._ptr, 0, b5._ptr) == 0
        assert b5.numpy().tolist() == [0.0] * 5
        assert lib.neural_reduce_mean(m._ptr, 0, b5._ptr) == 0
        assert np.all(np.isnan(b5.numpy()))
        # no maximum of nothing
        assert lib.neural_reduce_max(e._ptr, -1, one._ptr) == bad
        assert lib.neural_reduce_max(z._ptr, 1, r3._ptr) == bad
        i = ctypes.c_int64()
        assert lib.neural_argmax(e._ptr, ctypes.byref(i)) == bad
