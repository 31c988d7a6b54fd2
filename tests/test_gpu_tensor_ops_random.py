"""Randomised 2-D tensor ops (tensor_ops.c:15-148) through the C-ABI.

Seeded shapes of 1-1500 rows and columns (log-uniform) on host buffers and,
for half of the cases, device buffers: concat along either axis, split at a
random index (the edges included), pad with random margins and value, and
transpose.  Results must equal numpy's concatenate / slicing / pad /
transpose bit for bit (these ops move values and nothing else), and the
returned dimensions must be numpy's; the oracle's restatement must agree.
"""

import ctypes

import numpy as np

from conftest import GPU, same_bits

pytestmark = GPU

CASES = 30


def _dim(rng):
    return int(np.exp(rng.uniform(0, np.log(1500))))


def _vals(rng, r, c):
    x = rng.normal(0, 1, (r, c))
    x[rng.random((r, c)) < 0.01] = np.nan
    return x


def _buf(torch, x, dev):
    """(pointer, holder) of a float64 buffer with x's values on the host or the device."""
    if dev:
        t = torch.from_numpy(np.ascontiguousarray(x)).cuda()
        return t.data_ptr(), t
    a = np.ascontiguousarray(x)
    return a.ctypes.data, a


def _back(h, n):
    return (h.cpu().numpy() if hasattr(h, "cpu") else h).reshape(-1)[:n]


def test_random_tensor_ops(pn, ora):
    import torch
    lib = pn.core._lib
    rng = np.random.default_rng(5150)
    d = [ctypes.c_int64() for _ in range(4)]
    for case in range(CASES):
        dev = rng.random() < 0.5
        # concat
        axis = int(rng.integers(0, 2))
        ra, ca = _dim(rng), _dim(rng)
        rb, cb = (_dim(rng), ca) if axis == 0 else (ra, _dim(rng))
        a, b = _vals(rng, ra, ca), _vals(rng, rb, cb)
        want = np.concatenate([a, b], axis=axis)
        pa, ha = _buf(torch, a, dev)
        pb, hb = _buf(torch, b, dev)
        po, ho = _buf(torch, np.full((ra + rb) * (ca + cb), 7.0), dev)
        torch.cuda.synchronize()
        assert lib.tensor_concat_2d(pa, pb, ra, ca, rb, cb, axis, po, ctypes.byref(d[0]), ctypes.byref(d[1])) == 0
        pn.synchronize()
        assert (d[0].value, d[1].value) == want.shape, (case, axis)
        same_bits(_back(ho, want.size), want.reshape(-1))
        rc, wo, wr, wc = ora.concat_2d(a.reshape(-1), b.reshape(-1), ra, ca, rb, cb, axis)
        assert rc == 0 and (wr, wc) == want.shape
        same_bits(wo[:want.size], want.reshape(-1))
        # split, the edges (0 and the full extent are refused by the reference) included
        r, c = _dim(rng) + 1, _dim(rng) + 1
        x = _vals(rng, r, c)
        axis = int(rng.integers(0, 2))
        ext = r if axis == 0 else c
        s = int(rng.choice([1, ext - 1, int(rng.integers(1, ext))]))
        wa, wb = (x[:s], x[s:]) if axis == 0 else (x[:, :s], x[:, s:])
        px, hx = _buf(torch, x, dev)
        p1, h1 = _buf(torch, np.full(r * c, 7.0), dev)
        p2, h2 = _buf(torch, np.full(r * c, 7.0), dev)
        torch.cuda.synchronize()
        assert lib.tensor_split_2d(px, r, c, axis, s, p1, p2, *[ctypes.byref(v) for v in d]) == 0, (case, r, c, s)
        pn.synchronize()
        assert (d[0].value, d[1].value, d[2].value, d[3].value) == wa.shape + wb.shape
        same_bits(_back(h1, wa.size), wa.reshape(-1))
        same_bits(_back(h2, wb.size), wb.reshape(-1))
        # pad
        r, c = _dim(rng), _dim(rng)
        x = _vals(rng, r, c)
        pads = [int(rng.integers(0, 40)) for _ in range(4)]
        v = float(rng.normal())
        want = np.pad(x, ((pads[0], pads[1]), (pads[2], pads[3])), constant_values=v)
        px, hx = _buf(torch, x, dev)
        po, ho = _buf(torch, np.full(want.size, 7.0), dev)
        torch.cuda.synchronize()
        assert lib.tensor_pad_2d(px, r, c, *pads, ctypes.c_double(v), po, ctypes.byref(d[0]),
                                 ctypes.byref(d[1])) == 0, (case, r, c, pads)
        pn.synchronize()
        assert (d[0].value, d[1].value) == want.shape
        same_bits(_back(ho, want.size), want.reshape(-1))
        rc, wo, wr, wc = ora.pad_2d(x.reshape(-1), r, c, *pads, v)
        assert rc == 0
        same_bits(wo[:want.size], want.reshape(-1))
        # transpose
        r, c = _dim(rng), _dim(rng)
        x = _vals(rng, r, c)
        px, hx = _buf(torch, x, dev)
        po, ho = _buf(torch, np.full(r * c, 7.0), dev)
        torch.cuda.synchronize()
        assert lib.tensor_transpose2d_array(px, r, c, po) == 0, (case, r, c)
        pn.synchronize()
        same_bits(_back(ho, r * c), np.ascontiguousarray(x.T).reshape(-1))
