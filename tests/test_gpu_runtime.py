"""Tensor runtime on the GPU: memory model, views, error codes, determinism.

Reference behaviour: neural_api.asm:392-967,2293-2426 (create / from_buffer /
copy / fill / reshape / buffer_info), tensor.asm:7-31 (descriptor layout).
"""

import ctypes

import numpy as np
import pytest

from conftest import GPU, keep, same_bits

pytestmark = GPU


def test_roundtrip_and_map(pn, rng):
    x = rng.normal(size=(17, 33)).astype(np.float32)
    t = pn.Tensor.from_numpy(x)
    same_bits(t.numpy(), x)
    # zero-copy view of the host mirror: writes are seen by the next call
    v = t.numpy_zero_copy()
    same_bits(v, x)
    v[0, 0] = 42.0
    y = (t + t).numpy()
    assert y[0, 0] == 84.0
    # reference-style memmove through neural_tensor_data()
    p = pn.core._lib.neural_tensor_data(t._ptr)
    z = np.arange(17 * 33, dtype=np.float32)
    ctypes.memmove(p, z.ctypes.data, z.nbytes)
    same_bits(pn.ReLU()(t).numpy().ravel(), z)


def test_from_buffer_host_is_authoritative(pn):
    arr = np.linspace(-1, 1, 1000, dtype=np.float64)
    t = pn.Tensor.from_numpy_zero_copy(arr)
    out = pn.Tensor.create([1000], pn.float64)
    pn.core._check_error(pn.core._lib.neural_relu(out._ptr, t._ptr), "relu")
    same_bits(out.numpy(), np.where(arr > 0, arr, 0.0))
    arr[:] = 2.0  # later host writes are picked up by the next call
    pn.core._check_error(pn.core._lib.neural_add(t._ptr, t._ptr, t._ptr), "add")  # in place, written back
    assert np.all(arr == 4.0)
    # the caller keeps ownership (the reference frees it: neural_api.asm:2393)
    del t
    assert arr[0] == 4.0


def test_from_buffer_strides_and_info(pn):
    base = np.arange(24, dtype=np.float32).reshape(4, 6)
    view = base[:, ::2]
    shape = (ctypes.c_uint64 * 2)(4, 3)
    strides = (ctypes.c_int64 * 2)(24, 8)
    ptr = pn.core._lib.neural_tensor_from_buffer(view.ctypes.data, shape, 2, 0, strides)
    t = pn.Tensor(ptr)
    t._keep = base
    assert not t.is_contiguous
    assert t.strides == (24, 8)
    same_bits(t.numpy(), np.ascontiguousarray(view))
    c = pn.Tensor.create([4, 3])
    pn.core._check_error(pn.core._lib.neural_scalar_mul(c._ptr, t._ptr, ctypes.c_double(2.0)), "smul")
    same_bits(c.numpy(), view * 2)
    info = pn.core.NeuralBufferInfo()
    assert pn.core._lib.neural_buffer_info(c._ptr, ctypes.byref(info)) == 0
    assert info.itemsize == 4 and info.ndim == 2 and info.format == b"f"


def test_reshape_view_shares_storage(pn, rng):
    x = rng.normal(size=24).astype(np.float32)
    t = pn.Tensor.from_numpy(x)
    v = t.reshape([4, 6])
    assert v.shape == (4, 6)
    pn.core._check_error(pn.core._lib.neural_scalar_add(v._ptr, v._ptr, ctypes.c_double(1.0)), "sadd")
    same_bits(t.numpy(), x + np.float32(1.0))
    assert pn.core._lib.neural_tensor_reshape(t._ptr, (ctypes.c_uint64 * 1)(5), 1) is None
    assert pn.get_last_error() == pn.NeuralError.SHAPE_MISMATCH


def test_create_errors(pn):
    lib = pn.core._lib
    shape = (ctypes.c_uint64 * 1)(4)
    assert lib.neural_tensor_create(shape, 1, 7) is None
    assert lib.neural_get_last_error() == pn.NeuralError.INVALID_DTYPE
    assert lib.neural_tensor_create(None, 1, 0) is None
    assert lib.neural_get_last_error() == pn.NeuralError.NULL_POINTER
    huge = (ctypes.c_uint64 * 1)(1 << 46)  # 256 TiB: device allocation must fail cleanly
    assert lib.neural_tensor_create(huge, 1, 0) is None
    assert lib.neural_get_last_error() == pn.NeuralError.OUT_OF_MEMORY
    assert pn.get_error_message(4).startswith("tensor shapes")


def test_determinism(pn):
    x = np.random.default_rng(2).normal(size=1 << 22).astype(np.float32)
    t = pn.Tensor.from_numpy(x)
    assert len({t.sum() for _ in range(5)}) == 1


def test_torch_stream_interop(pn):
    torch = pytest.importorskip("torch")
    s = torch.cuda.current_stream()
    pn.set_stream(s.cuda_stream)
    try:
        a = torch.randn(1 << 20, device="cuda")
        b = torch.randn(1 << 20, device="cuda")
        out = torch.empty_like(a)
        assert pn.core._lib.neural_add(keep(pn.Tensor.from_torch(out)), keep(pn.Tensor.from_torch(a)),
                                       keep(pn.Tensor.from_torch(b))) == 0
        same_bits(out.cpu().numpy(), a.cpu().numpy() + b.cpu().numpy())  # stream-ordered, no explicit sync
    finally:
        pn.set_stream(None)
