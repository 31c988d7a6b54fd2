"""
2-D float64 tensor utilities (reference ``pyneural/tensor_ops.py``): concat,
split, pad, transpose over flat row-major Python lists, backed by the
library's copy kernels.
"""

from __future__ import annotations

import ctypes
from typing import List, Tuple

from .core import _lib


def _make_f64(values: List[float]):
    return (ctypes.c_double * max(len(values), 1))(*values)


def _to_list(arr, n: int) -> List[float]:
    return [float(arr[i]) for i in range(n)]


def concat_2d(a: List[float], b: List[float], rows_a: int, cols_a: int, rows_b: int, cols_b: int,
              axis: int = 0) -> Tuple[List[float], int, int]:
    a_arr, b_arr = _make_f64(a), _make_f64(b)
    out_arr = (ctypes.c_double * max((rows_a + rows_b) * (cols_a + cols_b), 1))()
    out_rows, out_cols = ctypes.c_int64(), ctypes.c_int64()
    rc = _lib.tensor_concat_2d(ctypes.cast(a_arr, ctypes.c_void_p), ctypes.cast(b_arr, ctypes.c_void_p),
                               rows_a, cols_a, rows_b, cols_b, axis, ctypes.cast(out_arr, ctypes.c_void_p),
                               ctypes.byref(out_rows), ctypes.byref(out_cols))
    if rc != 0:
        raise RuntimeError("tensor_concat_2d failed")
    return _to_list(out_arr, out_rows.value * out_cols.value), out_rows.value, out_cols.value


def split_2d(data: List[float], rows: int, cols: int, axis: int, split_index: int):
    in_arr = _make_f64(data)
    out_a = (ctypes.c_double * max(rows * cols, 1))()
    out_b = (ctypes.c_double * max(rows * cols, 1))()
    ra, ca, rb, cb = ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int64()
    rc = _lib.tensor_split_2d(ctypes.cast(in_arr, ctypes.c_void_p), rows, cols, axis, split_index,
                              ctypes.cast(out_a, ctypes.c_void_p), ctypes.cast(out_b, ctypes.c_void_p),
                              ctypes.byref(ra), ctypes.byref(ca), ctypes.byref(rb), ctypes.byref(cb))
    if rc != 0:
        raise RuntimeError("tensor_split_2d failed")
    return (_to_list(out_a, ra.value * ca.value), ra.value, ca.value,
            _to_list(out_b, rb.value * cb.value), rb.value, cb.value)


def pad_2d(data: List[float], in_rows: int, in_cols: int, pad_top: int = 0, pad_bottom: int = 0,
           pad_left: int = 0, pad_right: int = 0, pad_value: float = 0.0) -> Tuple[List[float], int, int]:
    in_arr = _make_f64(data)
    R, C = in_rows + pad_top + pad_bottom, in_cols + pad_left + pad_right
    out_arr = (ctypes.c_double * max(R * C, 1))()
    out_rows, out_cols = ctypes.c_int64(), ctypes.c_int64()
    rc = _lib.tensor_pad_2d(ctypes.cast(in_arr, ctypes.c_void_p), in_rows, in_cols, pad_top, pad_bottom,
                            pad_left, pad_right, float(pad_value), ctypes.cast(out_arr, ctypes.c_void_p),
                            ctypes.byref(out_rows), ctypes.byref(out_cols))
    if rc != 0:
        raise RuntimeError("tensor_pad_2d failed")
    return _to_list(out_arr, out_rows.value * out_cols.value), out_rows.value, out_cols.value


def transpose_2d(data: List[float], rows: int, cols: int) -> Tuple[List[float], int, int]:
    in_arr = _make_f64(data)
    out_arr = (ctypes.c_double * max(rows * cols, 1))()
    rc = _lib.tensor_transpose2d_array(ctypes.cast(in_arr, ctypes.c_void_p), rows, cols,
                                       ctypes.cast(out_arr, ctypes.c_void_p))
    if rc != 0:
        raise RuntimeError("tensor_transpose2d_array failed")
    return _to_list(out_arr, rows * cols), cols, rows
