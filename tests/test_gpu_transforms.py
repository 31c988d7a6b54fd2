"""Per-feature transforms (transforms.c:26-143) through the C-ABI.

The three maps are bit-exact against the oracle (itself bit-exact against
the reference's transforms.c).  Statistics: min / max bit-exact, including
which zero sign comes first, NaN-skipping and the +-1e308 start values;
mean within 1e-12 of mean(|x|) and the variance within 1e-12 of
mean(x^2) + mean^2 (the device sums in a tree, the reference in one
sequential pass); NaN columns give NaN mean / std on both sides.
"""

import math

import numpy as np
import pytest

from conftest import GPU, same_bits

pytestmark = GPU


def _lib():
    from pyneural.core import _lib
    return _lib


def _shapes():
    rng = np.random.default_rng(21)
    xs = [rng.normal(0, 3, (1000, 7)), rng.normal(5, 0.1, (333, 64)), np.full((5, 3), 2.5),
          rng.normal(0, 1, (1, 9)), rng.normal(1, 2, (4096, 2)), rng.normal(0, 1, (100, 1)),
          rng.normal(0, 1, (50, 1000)), rng.normal(-3, 4, (200_000, 16)), rng.normal(0, 1, (3000, 65))]
    x = rng.normal(0, 1, (64, 12))
    x[3, 0] = np.nan
    x[:, 1] = np.nan
    x[5, 2], x[9, 2] = np.inf, -np.inf
    x[:, 3] = 0.0
    x[4, 3] = -0.0
    x[:, 4] = -0.0
    x[7, 4] = 0.0
    x[:, 5] = np.inf
    x[:, 6] = 1e308
    x[2, 7] = 1.5e308
    x[:, 8] = -np.inf
    xs.append(x)
    z = np.zeros((257, 3))
    z[100:, 0] = -0.0
    z[:200, 1] = -0.0
    xs.append(z)
    return xs


def _gpu_stats(x):
    b, nf = x.shape
    outs = [np.full(nf, 7.0) for _ in range(4)]
    rc = _lib().transform_compute_stats(x.ctypes.data, b, nf, *[o.ctypes.data for o in outs])
    assert rc == 0
    return outs


def test_stats(pn, ora):
    for x in _shapes():
        x = np.ascontiguousarray(x)
        mean, std, mn, mx = _gpu_stats(x)
        _, rmean, rstd, rmn, rmx = ora.transform_stats(x)
        same_bits(mn, rmn)
        same_bits(mx, rmx)
        with np.errstate(all="ignore"):
            amean = np.abs(x).mean(axis=0)
            sq = (x * x).mean(axis=0) + rmean * rmean
        for f in range(x.shape[1]):
            if math.isnan(rmean[f]) or math.isinf(rmean[f]):
                assert (math.isnan(mean[f]) and math.isnan(rmean[f])) or mean[f] == rmean[f], (f, mean[f], rmean[f])
                continue
            assert abs(mean[f] - rmean[f]) <= 1e-12 * amean[f] + 1e-300, (x.shape, f, mean[f], rmean[f])
            if math.isfinite(sq[f]):
                assert abs(std[f] ** 2 - rstd[f] ** 2) <= 1e-12 * sq[f] + 1e-300, (x.shape, f, std[f], rstd[f])
            else:
                assert (math.isnan(std[f]) and math.isnan(rstd[f])) or std[f] == rstd[f]


@pytest.mark.parametrize("mode", [0, 1, 2])
def test_maps_bit_exact(pn, ora, mode):
    rng = np.random.default_rng(mode + 30)
    fn = [_lib().transform_normalize, _lib().transform_unnormalize, _lib().transform_minmax][mode]
    import ctypes
    for x in _shapes():
        x = np.ascontiguousarray(x)
        b, nf = x.shape
        p0 = rng.normal(0, 1, nf)
        p1 = np.abs(rng.normal(1, 0.5, nf))
        p1[0] = 0.0
        for eps in [1e-8, 0.0]:
            out = np.empty_like(x)
            assert fn(x.ctypes.data, out.ctypes.data, b, nf, p0.ctypes.data, p1.ctypes.data, ctypes.c_double(eps)) == 0
            _, want = ora.transform_apply(mode, x, p0, p1, eps)
            same_bits(out.reshape(-1), want.reshape(-1))


def test_unaligned_and_device(pn, ora):
    import ctypes
    import torch
    rng = np.random.default_rng(40)
    buf = rng.normal(0, 1, 1 + 4096 * 8)
    x = buf[1:].reshape(4096, 8)  # 8-byte offset: the element-at-a-time path
    mean = rng.normal(0, 1, 8)
    std = np.abs(rng.normal(1, 0.2, 8))
    out = np.empty((4096, 8))
    assert _lib().transform_normalize(x.ctypes.data, out.ctypes.data, 4096, 8, mean.ctypes.data, std.ctypes.data,
                                      ctypes.c_double(1e-8)) == 0
    same_bits(out, ora.transform_apply(0, x, mean, std, 1e-8)[1])
    xd = torch.from_numpy(np.ascontiguousarray(x)).cuda()
    od = torch.empty_like(xd)
    md, sd = torch.from_numpy(mean).cuda(), torch.from_numpy(std).cuda()
    torch.cuda.synchronize()
    assert _lib().transform_normalize(xd.data_ptr(), od.data_ptr(), 4096, 8, md.data_ptr(), sd.data_ptr(),
                                      ctypes.c_double(1e-8)) == 0
    same_bits(od.cpu().numpy(), out)


def test_python_layer(pn, ora):
    rng = np.random.default_rng(41)
    x = rng.normal(2, 3, (500, 6))
    flat = x.reshape(-1).tolist()
    norm = pn.Normalize()
    y = norm(flat, 6)  # list in, list out, fitted on first use
    assert isinstance(y, list) and len(y) == x.size
    _, rmean, rstd, _, _ = ora.transform_stats(x)
    want = ora.transform_apply(0, x, norm.mean, norm.std, 1e-8)[1]
    same_bits(np.array(y), want.reshape(-1))
    back = norm.inverse(y, 6)
    assert np.allclose(back, flat, rtol=1e-13, atol=1e-12)
    t = pn.Tensor.from_numpy(x)
    ty = norm(t, 6)
    assert isinstance(ty, pn.Tensor)
    same_bits(ty.numpy().reshape(-1), want.reshape(-1))
    mm = pn.MinMaxScale()
    z = mm(x, 6)
    assert isinstance(z, np.ndarray) and z.min() >= 0.0 and z.max() <= 1.0
    comp = pn.Compose([pn.Normalize(), pn.MinMaxScale()])
    out = comp(x, 6)
    assert out.shape == x.shape
    stats = pn.compute_stats(flat, 6)
    assert stats["min"] == list(x.min(axis=0)) and stats["max"] == list(x.max(axis=0))
    with pytest.raises(ValueError):
        pn.compute_stats(flat[:-1], 6)


def test_errors(pn):
    import ctypes
    lib = _lib()
    x = np.ones((4, 3))
    o = np.ones(3)
    assert lib.transform_compute_stats(None, 4, 3, o.ctypes.data, None, None, None) == -1
    assert lib.transform_compute_stats(x.ctypes.data, 0, 3, o.ctypes.data, None, None, None) == -1
    assert lib.transform_compute_stats(x.ctypes.data, 4, 3, None, None, None, None) == 0
    assert lib.transform_normalize(x.ctypes.data, x.ctypes.data, 4, 3, None, o.ctypes.data,
                                   ctypes.c_double(1e-8)) == -1
    assert lib.transform_minmax(x.ctypes.data, x.ctypes.data, 4, -1, o.ctypes.data, o.ctypes.data,
                                ctypes.c_double(1e-8)) == -1
