"""Elementwise / broadcast parity: libneural_hip.so vs the CPU oracle, bit-exact.

Reference: math_kernels.asm:66-945 (ew_*), activations.asm:153-171 (ReLU),
nn_layers.asm:472-539 (bias add), simd.asm:190-540.
"""

import ctypes

import numpy as np
import pytest

from conftest import GPU, fmaf_exact, keep, rel_close, same_bits, special_f32, special_f64

pytestmark = GPU

SIZES = [1, 3, 7, 8, 9, 4099, 1 << 20]
OPS = [("add", 0), ("sub", 1), ("mul", 2), ("div", 3), ("maximum", 4)]


def _binary(pn, name, ta, tb):
    out = pn.Tensor.create(ta.shape, ta.dtype)
    fn = getattr(pn.core._lib, "neural_" + name)
    pn.core._check_error(fn(out._ptr, ta._ptr, tb._ptr), name)
    return out


@pytest.mark.parametrize("n", SIZES)
@pytest.mark.parametrize("name,code", OPS)
@pytest.mark.parametrize("dt", [np.float32, np.float64])
def test_binary_flat(pn, ora, rng, n, name, code, dt):
    gen = special_f32 if dt == np.float32 else special_f64
    a, b = gen(n, rng), gen(n, rng)
    got = _binary(pn, name, pn.Tensor.from_numpy(a), pn.Tensor.from_numpy(b)).numpy()
    same_bits(got, ora.ew(code, a, b))


def test_reference_unit_values(pn):
    """tests.asm:337-405,470-519: 3+2=5, 3-2=1, 3*2=6, relu(-1)=0."""
    a = pn.Tensor.create([8]).fill(3.0)
    b = pn.Tensor.create([8]).fill(2.0)
    assert (a + b).numpy()[0] == 5.0
    assert (a - b).numpy()[0] == 1.0
    assert (a * b).numpy()[0] == 6.0
    r = pn.ReLU()(pn.Tensor.from_numpy(np.array([-1, 0, 1, 2], dtype=np.float32))).numpy()
    assert r.tolist() == [0.0, 0.0, 1.0, 2.0]


@pytest.mark.parametrize("dt", [np.float32, np.float64])
def test_scalar_neg_relu(pn, ora, rng, dt):
    gen = special_f32 if dt == np.float32 else special_f64
    a = gen(100003, rng)
    ta = pn.Tensor.from_numpy(a)
    lib = pn.core._lib
    for s in (0.1, -3.7, 1e-40, 1e300):
        for fn, code in ((lib.neural_scalar_add, 0), (lib.neural_scalar_mul, 2)):
            out = pn.Tensor.create(ta.shape, ta.dtype)
            pn.core._check_error(fn(out._ptr, ta._ptr, ctypes.c_double(s)), "scalar")
            same_bits(out.numpy(), ora.scalar(0 if code == 0 else 2, a, s))
    same_bits((-ta).numpy(), ora.neg(a))
    r = pn.ReLU()(ta).numpy()
    same_bits(r, ora.relu(a))
    # NaN -> +0 and -0 -> +0 exactly (maxss x, 0)
    z = r[np.isnan(a) | (a == 0)]
    assert np.all(z.view(np.uint32 if dt == np.float32 else np.uint64) == 0)


@pytest.mark.parametrize("rows,cols", [(8192, 4096), (7, 12), (33, 1000), (5, 3)])
@pytest.mark.parametrize("dt", [np.float32, np.float64])
def test_bias_add(pn, ora, rng, rows, cols, dt):
    x = rng.normal(0, 3, (rows, cols)).astype(dt)
    b = rng.normal(0, 3, cols).astype(dt)
    out = pn.Tensor.create(x.shape, x.dtype)
    pn.core._check_error(pn.core._lib.neural_bias_add(out._ptr, keep(pn.Tensor.from_numpy(x)),
                                                     keep(pn.Tensor.from_numpy(b))), "bias_add")
    same_bits(out.numpy(), ora.bias_add(x, b))
    # same through neural_add broadcasting
    same_bits((pn.Tensor.from_numpy(x) + pn.Tensor.from_numpy(b)).numpy(), x + b)


@pytest.mark.parametrize("sa,sb", [
    ((4, 1, 6, 5), (3, 1, 5)),
    ((2, 3, 4, 5), (2, 1, 4, 1)),
    ((6, 1), (1, 7)),
    ((3, 4, 5), (5,)),
    ((2, 3, 4, 5, 6), (5, 6)),
])
def test_broadcast_nd(pn, rng, sa, sb):
    a = rng.normal(0, 1, sa).astype(np.float32)
    b = rng.normal(0, 1, sb).astype(np.float32)
    want = a / b
    out = pn.Tensor.create(want.shape, pn.float32)
    pn.core._check_error(pn.core._lib.neural_div(out._ptr, keep(pn.Tensor.from_numpy(a)),
                                                keep(pn.Tensor.from_numpy(b))), "div")
    same_bits(out.numpy(), want)


def test_broadcast_shape_errors(pn):
    a = pn.Tensor.create([3, 4])
    b = pn.Tensor.create([5])
    out = pn.Tensor.create([3, 4])
    assert pn.core._lib.neural_add(out._ptr, a._ptr, b._ptr) == pn.NeuralError.SHAPE_MISMATCH
    c = pn.Tensor.create([3, 4], pn.float64)
    assert pn.core._lib.neural_add(out._ptr, a._ptr, c._ptr) == pn.NeuralError.DTYPE_MISMATCH
    assert pn.core._lib.neural_add(None, a._ptr, a._ptr) == pn.NeuralError.NULL_POINTER


def test_strided_views_torch(pn, rng):
    torch = pytest.importorskip("torch")
    a = torch.randn(64, 96, device="cuda")
    b = torch.randn(96, 64, device="cuda")
    at = a.t()  # non-contiguous [96, 64]
    out = torch.empty(96, 64, device="cuda")
    torch.cuda.synchronize()  # torch's stream vs the library's stream
    rc = pn.core._lib.neural_mul(keep(pn.Tensor.from_torch(out)), keep(pn.Tensor.from_torch(at)),
                                 keep(pn.Tensor.from_torch(b)))
    assert rc == 0
    pn.synchronize()
    want = (at.cpu().numpy() * b.cpu().numpy()).astype(np.float32)
    same_bits(out.cpu().numpy(), want)
    # strided output view
    big = torch.zeros(96, 128, device="cuda")
    view = big[:, ::2]
    torch.cuda.synchronize()
    assert pn.core._lib.neural_add(keep(pn.Tensor.from_torch(view)), keep(pn.Tensor.from_torch(at)),
                                   keep(pn.Tensor.from_torch(b))) == 0
    pn.synchronize()
    same_bits(big.cpu().numpy()[:, ::2], (at.cpu().numpy() + b.cpu().numpy()).astype(np.float32))
    assert np.all(big.cpu().numpy()[:, 1::2] == 0)


def test_fill_copy_ones(pn, rng):
    t = pn.Tensor.ones([5, 7], pn.float64)
    assert np.all(t.numpy() == 1.0)
    z = pn.Tensor.zeros([1 << 20])
    assert not np.any(z.numpy())
    f = pn.Tensor.create([1000]).fill(0.1)
    assert np.all(f.numpy() == np.float32(0.1))
    x = rng.normal(size=(33, 17)).astype(np.float32)
    c = pn.Tensor.from_numpy(x).copy()
    same_bits(c.numpy(), x)
    bad = pn.Tensor.create([33, 17], pn.float64)
    assert pn.core._lib.neural_tensor_copy(bad._ptr, c._ptr) == pn.NeuralError.DTYPE_MISMATCH
    bad2 = pn.Tensor.create([10])
    assert pn.core._lib.neural_tensor_copy(bad2._ptr, c._ptr) == pn.NeuralError.SHAPE_MISMATCH


@pytest.mark.parametrize("n", [1, 15, 1 << 18])
def test_simd_raw_pointers(pn, ora, rng, n):
    lib = pn.core._lib
    a = rng.uniform(-1, 1, n).astype(np.float32)
    b = rng.uniform(-1, 1, n).astype(np.float32)
    c = rng.uniform(-1, 1, n).astype(np.float32)
    out = np.empty_like(a)
    assert lib.simd_add_f32(out.ctypes.data, a.ctypes.data, b.ctypes.data, n) == 0
    same_bits(out, ora.ew(ora.ADD, a, b))
    assert lib.simd_mul_f32(out.ctypes.data, a.ctypes.data, b.ctypes.data, n) == 0
    same_bits(out, ora.ew(ora.MUL, a, b))
    assert lib.simd_fma_f32(out.ctypes.data, a.ctypes.data, b.ctypes.data, c.ctypes.data, n) == 0
    same_bits(out, fmaf_exact(a, b, c))  # one rounding of the exact a*b + c
    e = float(np.sum(a.astype(np.float64) * b.astype(np.float64)))
    assert abs(lib.simd_dot_f32(a.ctypes.data, b.ctypes.data, n) - e) <= 1e-5 * float(np.sum(np.abs(a * b))) + 1e-30
    s = ora.sum_exact(a)
    assert abs(lib.simd_sum_f32(a.ctypes.data, n) - s) <= 1e-5 * float(np.sum(np.abs(a))) + 1e-30


def test_device_pointer_raw(pn, rng):
    torch = pytest.importorskip("torch")
    a = torch.rand(1 << 16, device="cuda")
    b = torch.rand(1 << 16, device="cuda")
    out = torch.empty_like(a)
    torch.cuda.synchronize()
    assert pn.core._lib.simd_add_f32(out.data_ptr(), a.data_ptr(), b.data_ptr(), a.numel()) == 0
    pn.synchronize()
    same_bits(out.cpu().numpy(), (a.cpu().numpy() + b.cpu().numpy()))


def test_unaligned_and_empty(pn, ora, rng):
    torch = pytest.importorskip("torch")
    base = torch.randn(4099, device="cuda")
    base2 = torch.randn(4101, device="cuda")
    a, b = base[1:], base2[3:]  # 4098 elements each, not 16-byte aligned
    out = torch.empty(4098, device="cuda")
    torch.cuda.synchronize()
    assert pn.core._lib.neural_sub(keep(pn.Tensor.from_torch(out)), keep(pn.Tensor.from_torch(a)),
                                   keep(pn.Tensor.from_torch(b))) == 0
    pn.synchronize()
    same_bits(out.cpu().numpy(), ora.ew(ora.SUB, a.cpu().numpy(), b.cpu().numpy()))
    e = pn.Tensor.create([0])
    assert pn.core._lib.neural_add(e._ptr, e._ptr, e._ptr) == 0
    assert e.numpy().shape == (0,)
