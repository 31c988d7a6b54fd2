"""
Checkpoints in the NEURCKPT container (the reference's
``pyneural/checkpoint.py``: written as version 3, versions 1 and 2 read).

Byte layout, little-endian (documented at checkpoint.py:4-35 of the
reference; kept so that files move between the two implementations):

    "NEURCKPT" | u32 version | u32 tensor count | u32 epoch | f64 best_loss | f64 lr
    v2+: u8 has_optimizer | u8 kind (0 none, 1 sgd, 2 adam, 3 adamw) | u16 0
         f64 x 5: momentum, beta1, beta2, epsilon, weight_decay (zeros where
         the kind has no such field)
    v3:  u64 blob length | the OPTS state blob of opt_state_export
         (optimizers_c.c:391-562: hyper-parameters, step count, f64 moments)
    per tensor: u32 ndim | ndim x u64 shape | u32 dtype (0 f32, 1 f64) | raw data

Here the parameters and the moments live in device memory.  Every tensor
goes through one host staging buffer that is reused for the whole file (a
device-to-host copy into it, then one write; on load one read into it, then
one host-to-device copy), and the moments travel inside the state blob.

``model`` is anything with ``parameters()`` or a plain sequence of Tensors.
"""

from __future__ import annotations

import struct
from pathlib import Path

import numpy as np

from .core import _lib, NeuralDtype, NeuralException

MAGIC = b"NEURCKPT"
VERSION = 3

OPT_NONE = 0
OPT_SGD = 1
OPT_ADAM = 2
OPT_ADAMW = 3

_PREFIX = struct.Struct("<8sIIIdd")  # magic, version, count, epoch, best_loss, lr
_OPT_HEAD = struct.Struct("<BBH")
_OPT_FIELDS = ("momentum", "beta1", "beta2", "epsilon", "weight_decay")
_OPT_VALUES = struct.Struct("<" + "d" * len(_OPT_FIELDS))
_U64 = struct.Struct("<Q")
_U32 = struct.Struct("<I")

# optimizer kind <- lower-cased class name, and the payload fields it records
_KINDS = {
    "sgd": (OPT_SGD, ("momentum",)),
    "adam": (OPT_ADAM, ("beta1", "beta2", "epsilon")),
    "adamw": (OPT_ADAMW, ("beta1", "beta2", "epsilon", "weight_decay")),
}
_KIND_NAMES = {code: name for name, (code, _) in _KINDS.items()}


def _parameter_list(model) -> list:
    return list(model.parameters()) if hasattr(model, "parameters") else list(model)


def _describe_optimizer(optimizer):
    """(kind code, payload values) for the optimizer object."""
    entry = _KINDS.get(type(optimizer).__name__.lower()) if optimizer is not None else None
    if entry is None:
        return OPT_NONE, (0.0,) * len(_OPT_FIELDS)
    code, recorded = entry
    return code, tuple(float(getattr(optimizer, f, 0.0)) if f in recorded else 0.0 for f in _OPT_FIELDS)


class _Staging:
    """One growable host buffer shared by every tensor of a file."""

    def __init__(self):
        self._buf = np.empty(0, dtype=np.uint8)

    def view(self, nbytes: int) -> np.ndarray:
        if self._buf.size < nbytes:
            self._buf = np.empty(max(nbytes, 2 * self._buf.size), dtype=np.uint8)
        return self._buf[:nbytes]


class _Source:
    """Sequential reads that name what was missing when the file ends early."""

    def __init__(self, f):
        self._f = f

    def unpack(self, fmt: struct.Struct, what: str) -> tuple:
        raw = self._f.read(fmt.size)
        if len(raw) < fmt.size:
            raise IOError(f"checkpoint truncated in the {what}")
        return fmt.unpack(raw)

    def fill(self, buf, what: str) -> None:
        if self._f.readinto(memoryview(buf)) < len(buf):
            raise IOError(f"checkpoint truncated in the {what}")


def _tensor_header(tensor):
    ndim = int(_lib.neural_tensor_ndim(tensor._ptr))
    dims = _lib.neural_tensor_shape(tensor._ptr)
    return tuple(int(dims[k]) for k in range(ndim)), int(_lib.neural_tensor_dtype(tensor._ptr))


def _itemsize(dtype: int) -> int:
    return 4 if dtype == NeuralDtype.FLOAT32 else 8


def _dump_tensor(f, tensor, staging: _Staging) -> None:
    shape, dtype = _tensor_header(tensor)
    f.write(_U32.pack(len(shape)) + b"".join(_U64.pack(s) for s in shape) + _U32.pack(dtype))
    dense = tensor if tensor.is_contiguous else tensor.contiguous()
    nbytes = int(_lib.neural_tensor_bytes(dense._ptr))
    if nbytes == 0:
        return
    buf = staging.view(nbytes)
    rc = _lib.neural_tensor_download(dense._ptr, buf.ctypes.data, nbytes)
    if rc != 0:
        raise IOError(f"device-to-host copy of a parameter failed (error {rc})")
    f.write(memoryview(buf))


def _restore_tensor(src: _Source, index: int, tensor, staging: _Staging) -> None:
    (ndim,) = src.unpack(_U32, "tensor header")
    shape = tuple(src.unpack(_U64, "tensor shape")[0] for _ in range(ndim))
    (dtype,) = src.unpack(_U32, "tensor dtype")
    have_shape, have_dtype = _tensor_header(tensor)
    if (shape, dtype) != (have_shape, have_dtype):
        raise ValueError(f"tensor {index}: shape mismatch (file {list(shape)} dtype {dtype}, "
                         f"model {list(have_shape)} dtype {have_dtype})")
    nbytes = int(np.prod(shape, dtype=np.int64)) * _itemsize(dtype)
    if nbytes == 0:
        return
    buf = staging.view(nbytes)
    src.fill(buf, "tensor data")
    if not tensor.is_contiguous:
        raise ValueError(f"tensor {index}: loading needs a contiguous parameter")
    rc = _lib.neural_tensor_upload(tensor._ptr, buf.ctypes.data, nbytes)
    if rc != 0:
        raise IOError(f"host-to-device copy of parameter {index} failed (error {rc})")


def _optimizer_blob(optimizer) -> bytes:
    """The optimizer's OPTS state blob, or b"" when it has none or its export
    fails: the checkpoint is then written without moments, as the reference
    does (checkpoint.py:99-114)."""
    export = getattr(optimizer, "state_bytes", None)
    if export is None or not getattr(optimizer, "_ptr", None):
        return b""
    try:
        return export()
    except NeuralException:
        return b""


def save_checkpoint(filepath, model, optimizer=None, epoch: int = 0, best_loss: float = float("inf"),
                    lr: float = 0.0) -> None:
    """Write the parameters, the training position and the optimizer state
    (the interface of the reference's checkpoint.py:196-240)."""
    params = _parameter_list(model)
    kind, payload = _describe_optimizer(optimizer)
    blob = _optimizer_blob(optimizer)
    staging = _Staging()
    with open(filepath, "wb") as f:
        f.write(_PREFIX.pack(MAGIC, VERSION, len(params), epoch, best_loss, lr))
        f.write(_OPT_HEAD.pack(int(kind != OPT_NONE), kind, 0) + _OPT_VALUES.pack(*payload))
        f.write(_U64.pack(len(blob)))
        f.write(blob)
        for p in params:
            _dump_tensor(f, p, staging)


def load_checkpoint(filepath, model, optimizer=None, strict_optimizer: bool = False) -> dict:
    """Read a version 1, 2 or 3 checkpoint into existing parameters (and the
    optimizer); returns {'epoch', 'best_loss', 'lr', 'optimizer_type'} (the
    interface of the reference's checkpoint.py:243-349)."""
    if not Path(filepath).exists():
        raise FileNotFoundError(f"no checkpoint at {filepath}")
    params = _parameter_list(model)
    staging = _Staging()
    with open(filepath, "rb") as f:
        src = _Source(f)
        magic, version, count, epoch, best_loss, lr = src.unpack(_PREFIX, "file header")
        if magic != MAGIC:
            raise ValueError(f"not a NEURCKPT file (magic {magic!r})")
        if version not in (1, 2, VERSION):
            raise ValueError(f"checkpoint version {version} cannot be read (versions 1 to {VERSION})")
        if count != len(params):
            raise ValueError(f"parameter count mismatch: the file holds {count}, the model has {len(params)}")
        kind = OPT_NONE
        blob = b""
        if version >= 2:
            present, kind, _ = src.unpack(_OPT_HEAD, "optimizer header")
            payload = src.unpack(_OPT_VALUES, "optimizer payload")
            if present and optimizer is not None:
                stored = _KIND_NAMES.get(kind)
                given = type(optimizer).__name__.lower()
                if strict_optimizer and stored is not None and stored != given:
                    raise ValueError(f"Optimizer type mismatch: the checkpoint holds {stored}, got {given}")
                if kind != OPT_NONE:
                    for field, value in zip(_OPT_FIELDS, payload):
                        if hasattr(optimizer, field):
                            setattr(optimizer, field, value)
        if version >= 3:
            (size,) = src.unpack(_U64, "optimizer state blob size")
            if size:
                data = bytearray(size)
                src.fill(data, "optimizer state blob")
                blob = bytes(data)
        if optimizer is not None:
            if hasattr(optimizer, "lr"):
                optimizer.lr = lr
            load = getattr(optimizer, "load_state_bytes", None)
            if blob and load is not None and getattr(optimizer, "_ptr", None):
                try:
                    load(blob)
                except NeuralException:
                    pass  # a blob the handle refuses is skipped, as the reference does
        for index, p in enumerate(params):
            _restore_tensor(src, index, p, staging)
    return {"epoch": epoch, "best_loss": best_loss, "lr": lr, "optimizer_type": kind}
