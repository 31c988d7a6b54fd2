"""Optimizer parity (optimizers_c.c:218-562).

Params and the float64 m / v (or velocity) buffers are bit-exact against the
oracle after several steps, for f32 and f64 params, including NaN / Inf
gradients.  The OPTS state blob matches the reference's own optimizers_c.c
byte for byte (oracle/_ref, when built), and round-trips through import.
"""

import ctypes

import numpy as np
import pytest

from conftest import GPU, same_bits

pytestmark = GPU

LR, B1, B2, EPS, WD = 1e-3, 0.9, 0.999, 1e-8, 0.01


def _data(n, dt, seed, inject=False):
    rng = np.random.default_rng(seed)
    p = rng.normal(0, 0.02, n).astype(dt)
    g = rng.normal(0, 1e-3, n).astype(dt)
    if inject and n > 200:
        idx = rng.choice(n, 96, replace=False)
        g[idx[:32]] = np.nan
        g[idx[32:64]] = np.inf
        g[idx[64:]] = -np.inf
    return p, g


def _blob_moments(blob, sizes, nbuf):
    off = 80 + 8 * len(sizes)
    out = []
    for _ in range(nbuf):
        for s in sizes:
            out.append(np.frombuffer(blob[off: off + 8 * s], dtype=np.float64).copy())
            off += 8 * s
    return out


@pytest.mark.parametrize("kind", ["adamw", "adam", "sgd"])
@pytest.mark.parametrize("dt", [np.float32, np.float64])
@pytest.mark.parametrize("n", [5, 4099, 1 << 20])
def test_steps_bit_exact(pn, ora, kind, dt, n):
    p, g = _data(n, dt, seed=n, inject=True)
    p2, g2 = _data(77, dt, seed=n + 1)
    tp, tg = pn.Tensor.from_numpy(p), pn.Tensor.from_numpy(g)
    tp2, tg2 = pn.Tensor.from_numpy(p2), pn.Tensor.from_numpy(g2)
    if kind == "adamw":
        opt = pn.AdamW(LR, B1, B2, EPS, WD)
    elif kind == "adam":
        opt = pn.Adam(LR, B1, B2, EPS)
    else:
        opt = pn.SGD(0.01, 0.9)
    rp, rp2 = p.copy(), p2.copy()
    m, v = np.zeros(n), np.zeros(n)
    m2, v2 = np.zeros(77), np.zeros(77)
    for t in range(1, 4):
        opt.step([tp, tp2], [tg, tg2])
        if kind == "adamw":
            ora.adamw_step(rp, g, m, v, LR, B1, B2, EPS, WD, t)
            ora.adamw_step(rp2, g2, m2, v2, LR, B1, B2, EPS, WD, t)
        elif kind == "adam":
            ora.adam_step(rp, g, m, v, LR, B1, B2, EPS, t)
            ora.adam_step(rp2, g2, m2, v2, LR, B1, B2, EPS, t)
        else:
            ora.sgd_step(rp, g, m, 0.01, 0.9)
            ora.sgd_step(rp2, g2, m2, 0.01, 0.9)
    same_bits(tp.numpy(), rp)
    same_bits(tp2.numpy(), rp2)
    blob = opt.state_bytes()
    if kind == "sgd":
        got_m, got_m2 = _blob_moments(blob, [n, 77], 1)
        same_bits(got_m, m)
        same_bits(got_m2, m2)
    else:
        gm, gm2, gv, gv2 = _blob_moments(blob, [n, 77], 2)
        same_bits(gm, m)
        same_bits(gv, v)
        same_bits(gm2, m2)
        same_bits(gv2, v2)


def test_adamw_cfg5_ten_steps(pn, ora):
    """cfg5's AdamW as BASELINE specifies it (params N(0, 0.02), grads
    N(0, 1e-3) with 32 NaN, 32 +Inf and 32 -Inf injected, lr 1e-3, wd 0.01),
    on 4 M f32 parameters: after step t = 10 (9 prior steps, a fresh gradient
    each step) params and the f64 moments equal the oracle's bit for bit."""
    n = 1 << 22
    rng = np.random.default_rng(6)
    p = rng.normal(0, 0.02, n).astype(np.float32)
    tp = pn.Tensor.from_numpy(p)
    opt = pn.AdamW(LR, B1, B2, EPS, WD)
    rp = p.copy()
    m, v = np.zeros(n), np.zeros(n)
    for t in range(1, 11):
        g = rng.normal(0, 1e-3, n).astype(np.float32)
        idx = rng.choice(n, 96, replace=False)
        g[idx[:32]] = np.nan
        g[idx[32:64]] = np.inf
        g[idx[64:]] = -np.inf
        tg = pn.Tensor.from_numpy(g)
        opt.step([tp], [tg])
        ora.adamw_step(rp, g, m, v, LR, B1, B2, EPS, WD, t)
    same_bits(tp.numpy(), rp)
    gm, gv = _blob_moments(opt.state_bytes(), [n], 2)
    same_bits(gm, m)
    same_bits(gv, v)


def test_state_roundtrip_and_reference_blob(pn, ora):
    p, g = _data(1000, np.float32, 3)
    tp, tg = pn.Tensor.from_numpy(p), pn.Tensor.from_numpy(g)
    opt = pn.AdamW(LR, B1, B2, EPS, WD)
    opt.step([tp], [tg])
    opt.step([tp], [tg])
    blob = opt.state_bytes()
    assert len(blob) == 80 + 8 + 2 * 8 * 1000
    hdr = np.frombuffer(blob[:16], dtype=np.uint32)
    assert hdr[0] == 0x5354504F and hdr[1] == 1
    # resume: a fresh optimizer loaded from the blob continues identically
    opt2 = pn.AdamW(0.5, 0.5, 0.5, 0.5, 0.5)
    opt2.load_state_bytes(blob)
    assert opt2.lr == LR
    tq = pn.Tensor.from_numpy(tp.numpy())
    opt.step([tp], [tg])
    opt2.step([tq], [tg])
    same_bits(tq.numpy(), tp.numpy())
    assert opt2.state_bytes() == opt.state_bytes()

    ref = ora.ref()
    if ref is None:
        pytest.skip("oracle/_ref not built")

    class TensorC(ctypes.Structure):
        _fields_ = [("data", ctypes.c_void_p), ("ndim", ctypes.c_int64), ("shape", ctypes.POINTER(ctypes.c_int64)),
                    ("stride", ctypes.c_void_p), ("dtype", ctypes.c_int32), ("flags", ctypes.c_int32)]

    rp = p.copy()
    shape = (ctypes.c_int64 * 1)(1000)
    tpc = TensorC(rp.ctypes.data, 1, shape, None, 0, 0)
    tgc = TensorC(g.ctypes.data, 1, shape, None, 0, 0)
    h = ref.opt_adamw_create(LR, B1, B2, EPS, WD)
    pp = (ctypes.c_void_p * 1)(ctypes.addressof(tpc))
    gp = (ctypes.c_void_p * 1)(ctypes.addressof(tgc))
    for _ in range(3):
        assert ref.opt_step(h, pp, gp, 1) == 0
    nb = ref.opt_state_bytes(h)
    buf = (ctypes.c_uint8 * nb)()
    assert ref.opt_state_export(h, buf, nb) == 0
    assert bytes(buf) == opt.state_bytes(), "OPTS blob differs from the reference optimizers_c.c"
    same_bits(tp.numpy(), rp)
    ref.opt_free(h)


def test_step_errors(pn):
    opt = pn.Adam()
    a, b = pn.Tensor.create([10]), pn.Tensor.create([10])
    opt.step([a], [b])
    lib = pn.core._lib
    arr = (ctypes.c_void_p * 2)(a._ptr, b._ptr)
    assert lib.opt_step(opt._ptr, arr, arr, 2) == pn.NeuralError.INVALID_ARGUMENT
    assert lib.opt_step(opt._ptr, arr, arr, -1) == pn.NeuralError.INVALID_ARGUMENT
    assert lib.opt_step(None, arr, arr, 1) == pn.NeuralError.NULL_POINTER
    c = pn.Tensor.create([11])
    arr1 = (ctypes.c_void_p * 1)(c._ptr)
    assert lib.opt_step(opt._ptr, arr1, arr1, 1) == pn.NeuralError.SHAPE_MISMATCH
    bad = bytearray(opt.state_bytes())
    bad[0] ^= 0xFF
    with pytest.raises(pn.NeuralException):
        opt.load_state_bytes(bytes(bad))
    sgd = pn.SGD()
    with pytest.raises(pn.NeuralException):
        sgd.load_state_bytes(opt.state_bytes())  # type mismatch -> INVALID_ARGUMENT


def test_state_import_overflowing_counts(pn):
    """Blobs whose counts overflow int64 byte sizes (n_params = 2^61, a
    parameter of 2^61 + 1 values) or run past the blob end come back as error
    codes, as the reference's calloc failure does (optimizers_c.c:480-562),
    never as an abort; the optimizer stays usable afterwards."""
    import struct

    lib = pn.core._lib
    E = pn.NeuralError
    opt = pn.AdamW()
    a, g = pn.Tensor.create([6]), pn.Tensor.create([6])
    opt.step([a], [g])
    good = opt.state_bytes()
    hdr = bytearray(good[:80])

    def blob(n_params, sizes, tail=b""):
        h = bytearray(hdr)
        struct.pack_into("<q", h, 16, n_params)
        return bytes(h) + b"".join(struct.pack("<q", s) for s in sizes) + tail

    def imp(b):
        buf = ctypes.create_string_buffer(b, len(b))
        return lib.opt_state_import(opt._ptr, buf, len(b))

    assert imp(blob(1 << 61, [])) == E.OUT_OF_MEMORY
    assert imp(blob((1 << 60) + 1, [])) == E.OUT_OF_MEMORY
    assert imp(blob((1 << 63) - 1, [])) == E.OUT_OF_MEMORY
    assert imp(blob(1 << 40, [])) == E.INVALID_ARGUMENT       # fits int64, runs past the blob
    assert imp(blob(1, [(1 << 61) + 1], b"\0" * 8)) == E.OUT_OF_MEMORY
    assert imp(blob(2, [6, (1 << 62) + 3], b"\0" * 64)) == E.OUT_OF_MEMORY
    assert imp(blob(1, [1 << 40], b"\0" * 8)) == E.INVALID_ARGUMENT
    assert imp(blob(1, [-1], b"")) == E.INVALID_ARGUMENT
    # a good blob still loads and the optimizer still steps
    assert imp(good) == 0
    assert opt.state_bytes() == good
    opt.step([a], [g])
