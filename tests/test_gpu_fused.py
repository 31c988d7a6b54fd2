"""Fused epilogues: add + ReLU (vec_add_relu_fusion, fusion.asm:200-226) and
bias add + activation (nn_layers.asm:472-539 then activations_c.c).

add_relu is bit-exact against the oracle's restatement (flat and with a
broadcast bias).  bias_add_act must equal the library's own two-pass
composition (neural_bias_add, then the activation) bit for bit, and the
oracle's composition exactly for the piecewise activations and within the
activation tolerances (REL32 / REL64 + 1e-15) for the transcendental ones.
"""

import ctypes

import numpy as np
import pytest

from conftest import GPU, rel_close, same_bits

pytestmark = GPU

EXACT = {"none", "relu", "leaky_relu", "hardswish", "hardtanh"}
NAMES = ["none", "relu", "sigmoid", "tanh", "gelu", "leaky_relu", "elu", "selu", "swish", "mish", "hardswish",
         "softplus", "hardtanh"]


def test_add_relu_flat_and_broadcast(pn, ora):
    rng = np.random.default_rng(1)
    a = rng.normal(0, 1, (257, 1024)).astype(np.float32)
    b = rng.normal(0, 1, (257, 1024)).astype(np.float32)
    a[0, :8] = [np.nan, -0.0, 0.0, np.inf, -np.inf, 1e-45, -1e-45, 3.0]
    b[0, :8] = [1.0, 0.0, -0.0, -np.inf, 1.0, 0.0, 0.0, -3.0]
    got = pn.add_relu(pn.Tensor.from_numpy(a), pn.Tensor.from_numpy(b)).numpy()
    same_bits(got.reshape(-1), ora.add_relu(a.reshape(-1), b.reshape(-1)))
    bias = rng.normal(0, 1, 1024).astype(np.float32)
    got = pn.add_relu(pn.Tensor.from_numpy(a), pn.Tensor.from_numpy(bias)).numpy()
    same_bits(got.reshape(-1), ora.add_relu(a.reshape(-1), np.tile(bias, 257)))
    # f64 follows the same rule in double
    a64, b64 = a.astype(np.float64), b.astype(np.float64)
    got = pn.add_relu(pn.Tensor.from_numpy(a64), pn.Tensor.from_numpy(b64)).numpy()
    s = a64 + b64
    same_bits(got, np.where(s > 0, s, 0.0))


def test_vec_add_relu_fusion_raw(pn, ora):
    from pyneural.core import _lib
    rng = np.random.default_rng(2)
    for n in [1, 3, 1000, 1 << 20]:
        a = rng.normal(0, 1, n).astype(np.float32)
        b = rng.normal(0, 1, n).astype(np.float32)
        c = np.full(n, 7.0, np.float32)
        _lib.vec_add_relu_fusion(a.ctypes.data, b.ctypes.data, c.ctypes.data, n)
        same_bits(c, ora.add_relu(a, b))
    c = np.full(4, 7.0, np.float32)
    _lib.vec_add_relu_fusion(a.ctypes.data, b.ctypes.data, c.ctypes.data, 0)
    _lib.vec_add_relu_fusion(a.ctypes.data, b.ctypes.data, c.ctypes.data, -5)
    assert (c == 7.0).all()


def _two_pass(pn, x, b, name, alpha):
    from pyneural.core import _lib
    tx, tb = pn.Tensor.from_numpy(x), pn.Tensor.from_numpy(b)
    mid = pn.Tensor.create(x.shape, tx.dtype)
    assert _lib.neural_bias_add(mid._ptr, tx._ptr, tb._ptr) == 0
    if name == "none":
        return mid.numpy()
    out = pn.Tensor.create(x.shape, tx.dtype)
    fn = {"relu": _lib.neural_relu, "sigmoid": _lib.neural_sigmoid}.get(name)
    if fn is not None:
        assert fn(out._ptr, mid._ptr) == 0
    elif name in ("leaky_relu", "elu"):
        assert getattr(_lib, "act_" + name)(out._ptr, mid._ptr, ctypes.c_double(alpha)) == 0
    else:
        assert getattr(_lib, "act_" + name)(out._ptr, mid._ptr) == 0
    return out.numpy()


@pytest.mark.parametrize("dt", [np.float32, np.float64])
@pytest.mark.parametrize("name", NAMES)
def test_bias_add_act(pn, ora, name, dt):
    rng = np.random.default_rng(NAMES.index(name) + 10)
    x = rng.normal(0, 4, (129, 512)).astype(dt)
    b = rng.normal(0, 1, 512).astype(dt)
    x[0, :6] = [30.0, -30.0, np.nan, np.inf, -np.inf, 0.0]
    alpha = {"leaky_relu": 0.01, "elu": 1.0}.get(name, 0.0)
    got = pn.bias_add_act(pn.Tensor.from_numpy(x), pn.Tensor.from_numpy(b), name,
                          alpha if alpha else None).numpy()
    same_bits(got, _two_pass(pn, x, b, name, alpha))
    mid = ora.bias_add(x, b).reshape(x.shape)
    if name == "none":
        want = mid
    elif name == "relu":
        want = ora.relu(mid.reshape(-1)).reshape(x.shape)
    else:
        want = ora.act(name, mid.reshape(-1), alpha).reshape(x.shape)
    if name in EXACT:
        same_bits(got, want)
    elif dt == np.float32:
        rel_close(got, want, 1e-5, 0.0, name)
    else:
        rel_close(got, want, 1e-12, 1e-15, name)


def test_bias_add_act_errors(pn):
    from pyneural.core import _lib
    x = pn.Tensor.from_numpy(np.ones((4, 8), np.float32))
    b = pn.Tensor.from_numpy(np.ones(7, np.float32))
    out = pn.Tensor.create((4, 8))
    assert _lib.neural_bias_add_act(out._ptr, x._ptr, b._ptr, 1, ctypes.c_double(0)) == 4
    b = pn.Tensor.from_numpy(np.ones(8, np.float32))
    assert _lib.neural_bias_add_act(out._ptr, x._ptr, b._ptr, 99, ctypes.c_double(0)) == 3
    assert _lib.neural_bias_add_act(None, x._ptr, b._ptr, 1, ctypes.c_double(0)) == 1
