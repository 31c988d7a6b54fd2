"""
Per-feature data transforms (reference ``pyneural/transforms.py:1-247``):
compute_stats, Normalize (z-score), MinMaxScale and Compose, over row-major
[batch, features] float64 data.

Inputs may be what the reference takes (a flat list of floats, returned as a
list) or a NumPy array (returned as an array) or a float64 Tensor (stays in
device memory; returned as a Tensor).  Each call is one library call:
transform_compute_stats / transform_normalize / transform_unnormalize /
transform_minmax (transforms.c:26-143).  The image-augmentation helpers of the
reference module (ToTensor, random flips and crops) are plain Python list
operations and are not part of this library.
"""

from __future__ import annotations

import ctypes
from typing import List, Optional, Sequence

import numpy as np

from .core import _lib, NeuralDtype
from .tensor import Tensor


class _Data:
    """The caller's data as a device or host float64 buffer, and how to give
    results back in the caller's form."""

    def __init__(self, data, num_features: int):
        self.kind = "tensor" if isinstance(data, Tensor) else ("array" if isinstance(data, np.ndarray) else "list")
        if self.kind == "tensor":
            if data.dtype != NeuralDtype.FLOAT64:
                raise TypeError("transforms work on float64 tensors")
            self.tensor = data.contiguous()
            self.shape = data.shape
            n = data.numel
        else:
            self.array = np.ascontiguousarray(data, dtype=np.float64)
            self.shape = self.array.shape
            n = self.array.size
        if n == 0 or num_features <= 0:
            raise ValueError("data must be non-empty and num_features > 0")
        if n % num_features:
            raise ValueError(f"data length {n} not divisible by num_features {num_features}")
        self.batch = n // num_features
        self.nf = num_features

    def ptr(self) -> int:
        return self.tensor.device_ptr if self.kind == "tensor" else self.array.ctypes.data

    def new_output(self):
        if self.kind == "tensor":
            out = Tensor.create(self.shape, NeuralDtype.FLOAT64)
            return out, out.device_ptr
        out = np.empty(self.shape, dtype=np.float64)
        return out, out.ctypes.data

    def give(self, out):
        if self.kind == "list":
            return out.reshape(-1).tolist()
        return out


def _vec(values, nf: int) -> np.ndarray:
    v = np.ascontiguousarray(values, dtype=np.float64).reshape(-1)
    if v.size != nf:
        raise ValueError(f"expected {nf} per-feature values, got {v.size}")
    return v


def compute_stats(data, num_features: int) -> dict:
    """Per-feature mean, population std, min and max (transforms.c:26-62).
    Returns lists for list input, arrays otherwise."""
    d = _Data(data, num_features)
    outs = [np.zeros(d.nf) for _ in range(4)]
    rc = _lib.transform_compute_stats(d.ptr(), d.batch, d.nf, *[o.ctypes.data for o in outs])
    if rc != 0:
        raise RuntimeError("transform_compute_stats failed")
    if d.kind == "list":
        outs = [o.tolist() for o in outs]
    return {"mean": outs[0], "std": outs[1], "min": outs[2], "max": outs[3]}


def _apply(fn, name, data, num_features, p0, p1, eps):
    d = _Data(data, num_features)
    a0, a1 = _vec(p0, d.nf), _vec(p1, d.nf)
    out, optr = d.new_output()
    rc = fn(d.ptr(), optr, d.batch, d.nf, a0.ctypes.data, a1.ctypes.data, ctypes.c_double(eps))
    if rc != 0:
        raise RuntimeError(f"{name} failed")
    return d.give(out)


class Normalize:
    """Z-score normalisation (x - mean) / (std + eps) per feature; mean / std
    are fitted on the first call when not given."""

    def __init__(self, mean: Optional[List[float]] = None, std: Optional[List[float]] = None, eps: float = 1e-8):
        self.mean = mean
        self.std = std
        self.eps = eps
        self._fitted = mean is not None and std is not None

    def fit(self, data, num_features: int) -> "Normalize":
        stats = compute_stats(data, num_features)
        self.mean, self.std = stats["mean"], stats["std"]
        self._fitted = True
        return self

    def __call__(self, data, num_features: int):
        if not self._fitted:
            self.fit(data, num_features)
        return _apply(_lib.transform_normalize, "transform_normalize", data, num_features, self.mean, self.std,
                      self.eps)

    def inverse(self, data, num_features: int):
        if not self._fitted:
            raise RuntimeError("Cannot inverse before fitting")
        return _apply(_lib.transform_unnormalize, "transform_unnormalize", data, num_features, self.mean, self.std,
                      self.eps)

    def __repr__(self) -> str:
        return f"Normalize(fitted={self._fitted}, eps={self.eps})"


class MinMaxScale:
    """Min-max scaling (x - min) / (max - min + eps) per feature; min / max are
    fitted on the first call when not given."""

    def __init__(self, min_val: Optional[List[float]] = None, max_val: Optional[List[float]] = None,
                 eps: float = 1e-8):
        self.min_val = min_val
        self.max_val = max_val
        self.eps = eps
        self._fitted = min_val is not None and max_val is not None

    def fit(self, data, num_features: int) -> "MinMaxScale":
        stats = compute_stats(data, num_features)
        self.min_val, self.max_val = stats["min"], stats["max"]
        self._fitted = True
        return self

    def __call__(self, data, num_features: int):
        if not self._fitted:
            self.fit(data, num_features)
        return _apply(_lib.transform_minmax, "transform_minmax", data, num_features, self.min_val, self.max_val,
                      self.eps)

    def __repr__(self) -> str:
        return f"MinMaxScale(fitted={self._fitted}, eps={self.eps})"


class Compose:
    """Chain transforms: each is called as t(data, num_features)."""

    def __init__(self, transforms: Sequence):
        self.transforms = list(transforms)

    def __call__(self, data, num_features: int):
        for t in self.transforms:
            data = t(data, num_features)
        return data

    def __repr__(self) -> str:
        inner = ", ".join(repr(t) for t in self.transforms)
        return f"Compose([{inner}])"
