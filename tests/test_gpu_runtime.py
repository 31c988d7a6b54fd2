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


def test_raw_pointer_into_tensor_mirror(pn):
    """The reference's Python hands neural_tensor_data() pointers to the
    raw-pointer entry points (training.py:43-79).  Such a pointer resolves to
    the tensor's device copy, under the rule every kernel follows: host
    writes made through the pointer after neural_tensor_data() are seen by the
    next call, device writes made after the pointer was handed out are seen
    too (the reference has one copy of the data), partial ranges work, and an
    output written through a mirror pointer lands both in the host mirror and
    on the device."""
    lib = pn.core._lib
    n = 1 << 20
    t = pn.Tensor.from_numpy(np.linspace(-1, 1, n, dtype=np.float32))
    p = lib.neural_tensor_data(t._ptr)
    assert lib.neural_tensor_has_nan(p, n) == 0 and lib.neural_tensor_has_inf(p, n) == 0
    # a host write through a freshly fetched pointer (as the reference's
    # tensor.py writes: neural_tensor_data() makes the host copy
    # authoritative), then the raw call
    p = lib.neural_tensor_data(t._ptr)
    bad = np.array([np.nan], dtype=np.float32)
    ctypes.memmove(p + 4 * 777, bad.ctypes.data, 4)
    assert lib.neural_tensor_has_nan(p, n) == 1
    assert lib.neural_tensor_has_nan(p + 4 * 778, n - 778) == 0   # range after the NaN
    assert lib.neural_tensor_has_nan(p + 4 * 700, 100) == 1       # range around it
    # the NaN reached the device copy: a kernel sees it without another upload
    r = pn.Tensor.create([n])
    pn.core._check_error(lib.neural_relu(r._ptr, t._ptr), "relu")
    assert r.numpy()[777] == 0.0
    # a device write after the pointer was handed out: the old pointer sees it
    pn.core._check_error(lib.neural_tensor_fill(t._ptr, ctypes.c_double(float("inf"))), "fill")
    assert lib.neural_tensor_has_inf(p, n) == 1 and lib.neural_tensor_has_nan(p, n) == 0
    want_norm = np.float32(np.sqrt(np.float64(n) * 4.0))
    pn.core._check_error(lib.neural_tensor_fill(t._ptr, ctypes.c_double(2.0)), "fill")
    assert np.float32(lib.neural_tensor_grad_l2_norm(p, n)) == want_norm
    # an output through a mirror pointer: host mirror and device copy agree
    c = pn.Tensor.create([n])
    pc = lib.neural_tensor_data(c._ptr)
    a = np.arange(n, dtype=np.float32)
    b = np.full(n, 0.5, dtype=np.float32)
    assert lib.simd_add_f32(pc, a.ctypes.data, b.ctypes.data, n) == 0
    host_view = np.ctypeslib.as_array(ctypes.cast(pc, ctypes.POINTER(ctypes.c_float)), shape=(n,))
    same_bits(host_view.copy(), a + b)
    same_bits(c.numpy(), a + b)
    s = pn.Tensor.create([n])
    pn.core._check_error(lib.neural_add(s._ptr, c._ptr, c._ptr), "add")
    same_bits(s.numpy(), (a + b) * 2)
    # host buffers that are not mirrors (below, between and above the live
    # mirrors' addresses) are staged as before
    for m in (7, 1000, 1 << 16, 3 << 20):
        x = np.ones(m, dtype=np.float32)
        x[m // 2] = np.nan
        assert lib.neural_tensor_has_nan(x.ctypes.data, m) == 1
        y = np.empty(m, dtype=np.float32)
        assert lib.simd_add_f32(y.ctypes.data, x.ctypes.data, x.ctypes.data, m) == 0
        same_bits(y, x + x)


def test_shape_limits(pn):
    """Shapes whose element count, byte size or strided span does not fit
    int64 are refused with TENSOR_TOO_LARGE before anything is allocated (a
    wrapped count would size a buffer smaller than the kernels index); a
    tensor larger than the device is OUT_OF_MEMORY; the library keeps working
    afterwards."""
    import torch
    lib = pn.core._lib
    E = pn.NeuralError

    def create(*shape, dtype=0):
        arr = (ctypes.c_uint64 * len(shape))(*shape)
        return lib.neural_tensor_create(arr, len(shape), dtype)

    assert not create(1 << 40, 1 << 40) and lib.neural_get_last_error() == E.TENSOR_TOO_LARGE
    assert not create(1 << 32, 1 << 32, 4) and lib.neural_get_last_error() == E.TENSOR_TOO_LARGE
    assert not create(1 << 63) and lib.neural_get_last_error() == E.TENSOR_TOO_LARGE
    assert not create(1 << 62, dtype=1) and lib.neural_get_last_error() == E.TENSOR_TOO_LARGE  # bytes overflow
    assert not create(1 << 38) and lib.neural_get_last_error() == E.OUT_OF_MEMORY              # 1 TiB of f32
    buf = torch.zeros(16, device="cuda")
    torch.cuda.synchronize()
    shp = (ctypes.c_uint64 * 1)(4)
    bad_stride = (ctypes.c_int64 * 1)(1 << 62)
    assert not lib.neural_tensor_from_buffer(ctypes.c_void_p(buf.data_ptr()), shp, 1, 0, bad_stride)
    assert lib.neural_get_last_error() == E.TENSOR_TOO_LARGE
    t = pn.Tensor.from_numpy(np.arange(16, dtype=np.float32))
    wrap = (ctypes.c_uint64 * 2)(1 << 32, 1 << 32)   # 2^64 wraps to 0 in int64 arithmetic
    assert not lib.neural_tensor_reshape(t._ptr, wrap, 2)
    assert lib.neural_get_last_error() == E.SHAPE_MISMATCH
    ok = (ctypes.c_uint64 * 2)(4, 4)
    v = lib.neural_tensor_reshape(t._ptr, ok, 2)
    assert v
    lib.neural_tensor_free(v)
    u = pn.Tensor.from_numpy(np.ones(8, dtype=np.float32))
    same_bits(u.numpy(), np.ones(8, dtype=np.float32))


def test_raw_counts_beyond_limit(pn):
    """Raw-pointer entry points refuse element counts whose byte size could
    wrap (n = 2^62 + 1: times 4 or 8 it would wrap to a few bytes, so a
    staging buffer of that size would meet kernels indexing 2^62 elements)
    before staging anything, with their usual error returns; products of two
    dimensions that overflow likewise."""
    lib = pn.core._lib
    E = pn.NeuralError
    big = (1 << 62) + 1
    buf = np.zeros(64, dtype=np.float64)
    p = buf.ctypes.data
    out8 = np.zeros(64, dtype=np.int8)
    assert lib.neural_tensor_has_nan(p, big) == 0 and lib.neural_get_last_error() == E.TENSOR_TOO_LARGE
    assert lib.simd_add_f32(p, p, p, big) == E.TENSOR_TOO_LARGE
    assert lib.simd_sum_f32(p, big) == 0.0 and lib.neural_get_last_error() == E.TENSOR_TOO_LARGE
    qp = pn.core.QuantParamsC()
    assert lib.calibrate_minmax(p, big, 1, ctypes.byref(qp)) == -1
    assert lib.quantize_tensor(p, out8.ctypes.data, big, ctypes.byref(qp)) == -1
    assert lib.neural_dropout_forward(p, p, out8.ctypes.data, big, ctypes.c_float(0.5)) == E.TENSOR_TOO_LARGE
    loss = ctypes.c_double()
    tgt = np.zeros(64, dtype=np.int64)
    assert lib.label_smoothing_ce_forward(p, tgt.ctypes.data, 1 << 40, 1 << 40, 0.1, ctypes.byref(loss)) == -1
    assert lib.tensor_transpose2d_array(p, 1 << 40, 1 << 40, p) == -1
    assert lib.transform_compute_stats(p, 1 << 40, 1 << 40, p, None, None, None) == -1
    # the library still works
    x = np.arange(64, dtype=np.float32)
    assert lib.simd_sum_f32(x.ctypes.data, 64) == float(x.sum())
