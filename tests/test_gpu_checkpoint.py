"""Checkpoint save / resume with device-resident parameters and moments.

A run that saves after k AdamW steps, reloads into fresh tensors and a fresh
optimizer, and continues must end bit-identical to the uninterrupted run
(params and the OPTS blob).  The file's tensor records carry the parameters'
raw bytes, and its state blob is the optimizer's export; when the reference's
C optimizer is built (oracle/_ref) the blob equals the reference's own blob
after the same steps, so the file is the one the reference would write.
Shape and dtype mismatches raise as in the reference.
"""

import ctypes
import struct

import numpy as np
import pytest

from conftest import GPU, same_bits

pytestmark = GPU

LR, B1, B2, EPS, WD = 1e-3, 0.9, 0.999, 1e-8, 0.01


def _setup(pn, seed):
    rng = np.random.default_rng(seed)
    shapes = [((256, 129), np.float32), ((129,), np.float32), ((33, 7), np.float64), ((1,), np.float32)]
    params = [rng.normal(0, 0.02, s).astype(d) for s, d in shapes]
    grads = [[rng.normal(0, 1e-3, s).astype(d) for s, d in shapes] for _ in range(6)]
    return params, grads


def _run(pn, params, grads, steps, opt=None, tp=None):
    tp = tp or [pn.Tensor.from_numpy(p) for p in params]
    opt = opt or pn.AdamW(LR, B1, B2, EPS, WD)
    for g in grads[:steps]:
        opt.step(tp, [pn.Tensor.from_numpy(x) for x in g])
    return opt, tp


@pytest.mark.parametrize("kind", ["adamw", "sgd"])
def test_resume_bit_identical(pn, tmp_path, kind):
    params, grads = _setup(pn, 41)
    make = (lambda: pn.AdamW(LR, B1, B2, EPS, WD)) if kind == "adamw" else (lambda: pn.SGD(0.01, 0.9))
    full_opt, full_tp = _run(pn, params, grads, 6, opt=make())
    opt, tp = _run(pn, params, grads, 3, opt=make())
    path = tmp_path / "run.ckpt"
    pn.save_checkpoint(path, tp, opt, epoch=3, best_loss=0.75, lr=opt.lr)
    zeros = [np.zeros_like(p) for p in params]
    tp2 = [pn.Tensor.from_numpy(z) for z in zeros]
    opt2 = make()
    info = pn.load_checkpoint(path, tp2, opt2, strict_optimizer=True)
    assert info["epoch"] == 3 and info["best_loss"] == 0.75 and info["optimizer_type"] == (3 if kind == "adamw" else 1)
    for a, b in zip(tp, tp2):
        same_bits(b.numpy(), a.numpy())
    assert opt2.state_bytes() == opt.state_bytes()
    _run(pn, params, grads[3:], 3, opt=opt2, tp=tp2)
    for a, b in zip(full_tp, tp2):
        same_bits(b.numpy(), a.numpy())
    assert opt2.state_bytes() == full_opt.state_bytes()


def test_file_records(pn, tmp_path):
    params, grads = _setup(pn, 42)
    opt, tp = _run(pn, params, grads, 2)
    path = tmp_path / "rec.ckpt"
    pn.save_checkpoint(path, tp, opt, epoch=2, lr=opt.lr)
    data = path.read_bytes()
    assert data[:8] == b"NEURCKPT" and struct.unpack_from("<II", data, 8) == (3, len(params))
    blob_len = struct.unpack_from("<Q", data, 80)[0]
    blob = data[88: 88 + blob_len]
    assert blob == opt.state_bytes()
    off = 88 + blob_len
    for t in tp:
        ndim = struct.unpack_from("<I", data, off)[0]
        shape = struct.unpack_from(f"<{ndim}Q", data, off + 4)
        dtype = struct.unpack_from("<I", data, off + 4 + 8 * ndim)[0]
        off += 8 + 8 * ndim
        arr = t.numpy()
        assert shape == arr.shape and dtype == (0 if arr.dtype == np.float32 else 1)
        assert data[off: off + arr.nbytes] == arr.tobytes()
        off += arr.nbytes
    assert off == len(data)


def test_blob_matches_reference_c(pn, ora, tmp_path):
    # the state blob inside the file equals the one the reference's
    # optimizers_c.c exports after the same steps on the same data
    ref = ora.ref()
    if ref is None:
        pytest.skip("reference C build (oracle/_ref) absent")

    class TensorC(ctypes.Structure):
        _fields_ = [("data", ctypes.c_void_p), ("ndim", ctypes.c_int64), ("shape", ctypes.POINTER(ctypes.c_int64)),
                    ("stride", ctypes.c_void_p), ("dtype", ctypes.c_int32), ("flags", ctypes.c_int32)]

    params, grads = _setup(pn, 44)
    opt, tp = _run(pn, params, grads, 4)
    path = tmp_path / "r.ckpt"
    pn.save_checkpoint(path, tp, opt, lr=opt.lr)
    data = path.read_bytes()
    blob = data[88: 88 + struct.unpack_from("<Q", data, 80)[0]]

    rp = [p.copy().reshape(-1) for p in params]
    keep = []
    h = ref.opt_adamw_create(LR, B1, B2, EPS, WD)

    def arr(ts):
        out = (ctypes.c_void_p * len(ts))()
        for i, a in enumerate(ts):
            shape = (ctypes.c_int64 * 1)(a.size)
            t = TensorC(a.ctypes.data, 1, shape, None, 0 if a.dtype == np.float32 else 1, 0)
            keep.extend([shape, t])
            out[i] = ctypes.addressof(t)
        return out

    pp = arr(rp)
    for g in grads[:4]:
        gg = [x.reshape(-1) for x in g]
        keep.append(gg)
        assert ref.opt_step(h, pp, arr(gg), len(gg)) == 0
    nb = ref.opt_state_bytes(h)
    buf = (ctypes.c_uint8 * nb)()
    assert ref.opt_state_export(h, buf, nb) == 0
    ref.opt_free(h)
    assert bytes(buf) == blob
    for a, b in zip(tp, rp):
        same_bits(a.numpy().reshape(-1), b)


def test_shape_and_dtype_mismatch(pn, tmp_path):
    params, grads = _setup(pn, 43)
    tp = [pn.Tensor.from_numpy(p) for p in params]
    path = tmp_path / "m.ckpt"
    pn.save_checkpoint(path, tp)
    wrong = [pn.Tensor.from_numpy(p) for p in params]
    wrong[2] = pn.Tensor.from_numpy(params[2].astype(np.float32))
    with pytest.raises(ValueError, match="shape mismatch"):
        pn.load_checkpoint(path, wrong)
    wrong[2] = pn.Tensor.from_numpy(params[2].reshape(7, 33))
    with pytest.raises(ValueError, match="shape mismatch"):
        pn.load_checkpoint(path, wrong)
    with pytest.raises(ValueError, match="count mismatch"):
        pn.load_checkpoint(path, tp[:2])
    data = path.read_bytes()
    path.write_bytes(data[:-3])
    with pytest.raises(IOError, match="tensor data"):
        pn.load_checkpoint(path, [pn.Tensor.from_numpy(p) for p in params])
