"""
2-D float64 utilities over flat row-major sequences: concat, split, pad and
transpose (the interface of the reference's ``pyneural/tensor_ops.py:29-137``
over ``tensor_ops.c:15-148``).

Every function marshals its input once into a contiguous float64 numpy
buffer, lets the library's copy kernels fill preallocated float64 outputs,
and hands back plain Python lists with the output dimensions.  A rejected
argument (the library returns -1) raises RuntimeError naming the entry point
and its arguments.
"""

from __future__ import annotations

import ctypes
from typing import List, Sequence, Tuple

import numpy as np

from .core import _lib

_Dims = ctypes.c_int64


def _as_f64(values: Sequence[float]) -> np.ndarray:
    buf = np.ascontiguousarray(np.asarray(values, dtype=np.float64).ravel())
    return buf if buf.size else np.zeros(1)  # a valid address even when empty


def _scratch(n: int) -> np.ndarray:
    return np.empty(max(int(n), 1), dtype=np.float64)


def _ptr(buf: np.ndarray) -> ctypes.c_void_p:
    return ctypes.c_void_p(buf.ctypes.data)


def _invoke(entry: str, *args) -> None:
    rc = getattr(_lib, entry)(*args)
    if rc != 0:
        shown = ", ".join(str(a.value) if isinstance(a, (ctypes.c_int64, ctypes.c_double)) else
                          (str(a) if isinstance(a, (int, float)) else "<buffer>") for a in args)
        raise RuntimeError(f"{entry}({shown}) rejected its arguments (returned {rc})")


def _take(buf: np.ndarray, r: _Dims, c: _Dims) -> Tuple[List[float], int, int]:
    rows, cols = int(r.value), int(c.value)
    return buf[: rows * cols].tolist(), rows, cols


def concat_2d(a: List[float], b: List[float], rows_a: int, cols_a: int, rows_b: int, cols_b: int,
              axis: int = 0) -> Tuple[List[float], int, int]:
    """Join a [rows_a, cols_a] and b [rows_b, cols_b] along rows (axis 0) or
    columns (axis 1).  Returns (values, rows, cols)."""
    src_a, src_b = _as_f64(a), _as_f64(b)
    dst = _scratch((rows_a + rows_b) * (cols_a + cols_b))
    r, c = _Dims(), _Dims()
    _invoke("tensor_concat_2d", _ptr(src_a), _ptr(src_b), rows_a, cols_a, rows_b, cols_b, axis, _ptr(dst),
            ctypes.byref(r), ctypes.byref(c))
    return _take(dst, r, c)


def split_2d(data: List[float], rows: int, cols: int, axis: int, split_index: int):
    """Cut a [rows, cols] array before row (axis 0) or column (axis 1)
    `split_index`.  Returns (first, rows, cols, second, rows, cols)."""
    src = _as_f64(data)
    first, second = _scratch(rows * cols), _scratch(rows * cols)
    dims = [_Dims() for _ in range(4)]
    _invoke("tensor_split_2d", _ptr(src), rows, cols, axis, split_index, _ptr(first), _ptr(second),
            *[ctypes.byref(d) for d in dims])
    return _take(first, dims[0], dims[1]) + _take(second, dims[2], dims[3])


def pad_2d(data: List[float], in_rows: int, in_cols: int, pad_top: int = 0, pad_bottom: int = 0,
           pad_left: int = 0, pad_right: int = 0, pad_value: float = 0.0) -> Tuple[List[float], int, int]:
    """Surround a [in_rows, in_cols] array with `pad_value`.  Returns
    (values, rows, cols)."""
    src = _as_f64(data)
    dst = _scratch((in_rows + pad_top + pad_bottom) * (in_cols + pad_left + pad_right))
    r, c = _Dims(), _Dims()
    _invoke("tensor_pad_2d", _ptr(src), in_rows, in_cols, pad_top, pad_bottom, pad_left, pad_right,
            float(pad_value), _ptr(dst), ctypes.byref(r), ctypes.byref(c))
    return _take(dst, r, c)


def transpose_2d(data: List[float], rows: int, cols: int) -> Tuple[List[float], int, int]:
    """[rows, cols] -> [cols, rows].  Returns (values, cols, rows)."""
    src = _as_f64(data)
    dst = _scratch(rows * cols)
    _invoke("tensor_transpose2d_array", _ptr(src), rows, cols, _ptr(dst))
    return dst[: rows * cols].tolist(), cols, rows
