"""
Checkpoint save / resume (reference ``pyneural/checkpoint.py``): the NEURCKPT
binary format, version 3, with versions 1 and 2 still readable.

Layout, little-endian (reference checkpoint.py:4-35):

    "NEURCKPT" | u32 version (3) | u32 num_tensors
    u32 epoch | f64 best_loss | f64 lr
    v2+: u8 has_optimizer | u8 opt_type (0 none, 1 sgd, 2 adam, 3 adamw) | u16 0
         f64 momentum | f64 beta1 | f64 beta2 | f64 epsilon | f64 weight_decay
    v3:  u64 blob_size | the optimizer's OPTS state blob (hyper-parameters, step
         count and the float64 moments, optimizers_c.c:391-562)
    per tensor: u32 ndim | ndim x u64 shape | u32 dtype (0 f32, 1 f64) | raw data

Parameters and optimizer moments live in HBM here: each parameter comes down
with one device-to-host copy straight into a write buffer and goes back with
one host-to-device copy; the moments travel inside the state blob
(opt_state_export / opt_state_import).  Files are byte-compatible with the
reference's: the blob layout is the reference's and the tensors are raw
little-endian IEEE data.

``model`` is anything with ``parameters()`` (the reference's Module) or a
plain sequence of Tensors.
"""

from __future__ import annotations

import ctypes
import struct
from pathlib import Path

import numpy as np

from .core import _lib, NeuralDtype

MAGIC = b"NEURCKPT"
VERSION = 3

OPT_NONE = 0
OPT_SGD = 1
OPT_ADAM = 2
OPT_ADAMW = 3

_OPT_NAMES = {OPT_SGD: "sgd", OPT_ADAM: "adam", OPT_ADAMW: "adamw"}


def _params(model):
    if hasattr(model, "parameters"):
        return list(model.parameters())
    return list(model)


def _optimizer_payload(optimizer):
    """(opt_type, momentum, beta1, beta2, epsilon, weight_decay) keyed on the
    optimizer's class name, as checkpoint.py:56-76 of the reference."""
    if optimizer is None:
        return OPT_NONE, 0.0, 0.0, 0.0, 0.0, 0.0
    name = optimizer.__class__.__name__.lower()
    momentum = float(getattr(optimizer, "momentum", 0.0))
    beta1 = float(getattr(optimizer, "beta1", 0.0))
    beta2 = float(getattr(optimizer, "beta2", 0.0))
    epsilon = float(getattr(optimizer, "epsilon", 0.0))
    weight_decay = float(getattr(optimizer, "weight_decay", 0.0))
    if name == "sgd":
        return OPT_SGD, momentum, 0.0, 0.0, 0.0, 0.0
    if name == "adam":
        return OPT_ADAM, 0.0, beta1, beta2, epsilon, 0.0
    if name == "adamw":
        return OPT_ADAMW, 0.0, beta1, beta2, epsilon, weight_decay
    return OPT_NONE, 0.0, 0.0, 0.0, 0.0, 0.0


def _apply_optimizer_payload(optimizer, opt_type, payload) -> None:
    """Set the hyper-parameter attributes the optimizer object exposes."""
    if optimizer is None or opt_type == OPT_NONE:
        return
    for attr, value in zip(("momentum", "beta1", "beta2", "epsilon", "weight_decay"), payload):
        if hasattr(optimizer, attr):
            setattr(optimizer, attr, value)


def _export_state(optimizer):
    """The optimizer's OPTS blob as a ctypes buffer (empty bytes when there is
    none); the moments come down from the device inside opt_state_export."""
    if optimizer is None or not getattr(optimizer, "_ptr", None):
        return b""
    nbytes = int(_lib.opt_state_bytes(optimizer._ptr))
    if nbytes <= 0:
        return b""
    buf = (ctypes.c_uint8 * nbytes)()
    if int(_lib.opt_state_export(optimizer._ptr, ctypes.cast(buf, ctypes.c_void_p), nbytes)) != 0:
        return b""
    return buf


def _import_state(optimizer, blob) -> None:
    """Load an OPTS blob into the optimizer handle.  As in the reference
    (checkpoint.py:108-120), a blob the handle refuses is ignored."""
    if not blob or optimizer is None or not getattr(optimizer, "_ptr", None):
        return
    buf = (ctypes.c_uint8 * len(blob)).from_buffer(blob)
    _lib.opt_state_import(optimizer._ptr, ctypes.cast(buf, ctypes.c_void_p), len(blob))


def _tensor_meta(tensor):
    ndim = int(_lib.neural_tensor_ndim(tensor._ptr))
    shape_ptr = _lib.neural_tensor_shape(tensor._ptr)
    shape = tuple(int(shape_ptr[i]) for i in range(ndim))
    dtype = int(_lib.neural_tensor_dtype(tensor._ptr))
    return ndim, shape, dtype


def _elem_size(dtype: int) -> int:
    return 4 if dtype == NeuralDtype.FLOAT32 else 8


def _write_tensor(f, tensor) -> None:
    ndim, shape, dtype = _tensor_meta(tensor)
    f.write(struct.pack("<I", ndim))
    for s in shape:
        f.write(struct.pack("<Q", s))
    f.write(struct.pack("<I", dtype))
    src = tensor if tensor.is_contiguous else tensor.contiguous()
    nbytes = int(_lib.neural_tensor_bytes(src._ptr))
    if nbytes:
        buf = np.empty(nbytes, dtype=np.uint8)
        rc = _lib.neural_tensor_download(src._ptr, buf.ctypes.data, nbytes)
        if rc != 0:
            raise IOError(f"tensor download failed (error {rc})")
        f.write(memoryview(buf))


def _read_tensor_into(f, tensor) -> None:
    raw = f.read(4)
    if len(raw) < 4:
        raise IOError("Truncated checkpoint: expected ndim")
    ndim = struct.unpack("<I", raw)[0]
    shape = []
    for _ in range(ndim):
        raw = f.read(8)
        if len(raw) < 8:
            raise IOError("Truncated checkpoint: expected shape")
        shape.append(struct.unpack("<Q", raw)[0])
    raw = f.read(4)
    if len(raw) < 4:
        raise IOError("Truncated checkpoint: expected dtype")
    dtype = struct.unpack("<I", raw)[0]
    t_ndim, t_shape, t_dtype = _tensor_meta(tensor)
    if t_ndim != ndim or t_shape != tuple(shape) or t_dtype != dtype:
        raise ValueError(
            f"Checkpoint shape mismatch: file has ({ndim}, {shape}, dtype={dtype}) "
            f"but model has ({t_ndim}, {t_shape}, dtype={t_dtype})")
    numel = 1
    for s in shape:
        numel *= s
    total = numel * _elem_size(dtype)
    if total == 0:
        return
    buf = np.empty(total, dtype=np.uint8)
    got = f.readinto(memoryview(buf))
    if got < total:
        raise IOError("Truncated checkpoint: expected tensor data")
    if not tensor.is_contiguous:
        raise ValueError("checkpoint load needs contiguous parameter tensors")
    rc = _lib.neural_tensor_upload(tensor._ptr, buf.ctypes.data, total)
    if rc != 0:
        raise IOError(f"tensor upload failed (error {rc})")


def save_checkpoint(filepath, model, optimizer=None, epoch: int = 0, best_loss: float = float("inf"),
                    lr: float = 0.0) -> None:
    """Write parameters, training metadata and optimizer state (reference
    checkpoint.py:196-240)."""
    params = _params(model)
    with open(filepath, "wb") as f:
        f.write(MAGIC)
        f.write(struct.pack("<I", VERSION))
        f.write(struct.pack("<I", len(params)))
        f.write(struct.pack("<I", epoch))
        f.write(struct.pack("<d", best_loss))
        f.write(struct.pack("<d", lr))
        opt_type, momentum, beta1, beta2, epsilon, weight_decay = _optimizer_payload(optimizer)
        f.write(struct.pack("<BBH", 1 if opt_type != OPT_NONE else 0, opt_type, 0))
        f.write(struct.pack("<ddddd", momentum, beta1, beta2, epsilon, weight_decay))
        blob = _export_state(optimizer)
        f.write(struct.pack("<Q", len(blob)))
        if len(blob):
            f.write(memoryview(blob))
        for p in params:
            _write_tensor(f, p)


def load_checkpoint(filepath, model, optimizer=None, strict_optimizer: bool = False) -> dict:
    """Read a v1/v2/v3 checkpoint into existing parameters (and optimizer);
    returns {'epoch', 'best_loss', 'lr', 'optimizer_type'} (reference
    checkpoint.py:243-349, same checks and exceptions)."""
    path = Path(filepath)
    if not path.exists():
        raise FileNotFoundError(f"Checkpoint not found: {filepath}")
    params = _params(model)
    with open(filepath, "rb") as f:
        magic = f.read(8)
        if magic != MAGIC:
            raise ValueError(f"Invalid checkpoint magic: {magic!r} (expected {MAGIC!r})")
        ver = struct.unpack("<I", f.read(4))[0]
        if ver not in (1, 2, VERSION):
            raise ValueError(f"Unsupported checkpoint version {ver} (expected 1, 2, or {VERSION})")
        num_tensors = struct.unpack("<I", f.read(4))[0]
        if num_tensors != len(params):
            raise ValueError(f"Parameter count mismatch: checkpoint has {num_tensors}, model has {len(params)}")
        epoch = struct.unpack("<I", f.read(4))[0]
        best_loss = struct.unpack("<d", f.read(8))[0]
        lr = struct.unpack("<d", f.read(8))[0]

        optimizer_type = OPT_NONE
        blob = bytearray()
        if ver >= 2:
            hdr = f.read(4)
            if len(hdr) < 4:
                raise IOError("Truncated checkpoint: expected optimizer header")
            has_optimizer, optimizer_type, _ = struct.unpack("<BBH", hdr)
            vals = f.read(40)
            if len(vals) < 40:
                raise IOError("Truncated checkpoint: expected optimizer payload")
            payload = struct.unpack("<ddddd", vals)
            if has_optimizer and optimizer is not None:
                if strict_optimizer:
                    cls = optimizer.__class__.__name__.lower()
                    expected = _OPT_NAMES.get(optimizer_type, "unknown")
                    if expected != "unknown" and cls != expected:
                        raise ValueError(f"Optimizer type mismatch: checkpoint={expected}, provided={cls}")
                _apply_optimizer_payload(optimizer, optimizer_type, payload)
        if ver >= 3:
            raw = f.read(8)
            if len(raw) < 8:
                raise IOError("Truncated checkpoint: expected optimizer state blob size")
            blob_size = struct.unpack("<Q", raw)[0]
            if blob_size > 0:
                blob = bytearray(blob_size)
                if f.readinto(blob) < blob_size:
                    raise IOError("Truncated checkpoint: expected optimizer state blob")

        if optimizer is not None and hasattr(optimizer, "lr"):
            optimizer.lr = lr
        if optimizer is not None and blob:
            _import_state(optimizer, blob)

        for p in params:
            _read_tensor_into(f, p)

    return {"epoch": epoch, "best_loss": best_loss, "lr": lr, "optimizer_type": optimizer_type}
