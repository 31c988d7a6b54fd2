"""
Tensor wrapper over the opaque NeuralTensor of libneural_hip.so.

Same public surface as the reference ``pyneural/tensor.py`` (create / zeros /
ones / from_numpy / from_numpy_zero_copy / numpy / tolist / fill / copy /
arithmetic operators / array interface).  Data lives in device memory:
``numpy()`` and ``from_numpy()`` move bytes with explicit downloads/uploads,
and the zero-copy array interface maps the host mirror (valid until the next
library call that uses the tensor).  ``from_torch`` wraps a device tensor's
memory in place.
"""

import ctypes
from typing import List, Sequence, Union

from .core import _lib, NeuralError, NeuralDtype, NeuralException, NeuralBufferInfo, _check_error

try:
    import numpy as np
    HAS_NUMPY = True
except ImportError:  # pragma: no cover
    HAS_NUMPY = False


def _shape_arr(shape):
    return (ctypes.c_uint64 * max(len(shape), 1))(*shape)


def _dtype_code(dtype) -> int:
    """NeuralDtype code from a code, a numpy dtype or a numpy scalar type."""
    if isinstance(dtype, int):
        return dtype
    if HAS_NUMPY:
        dt = np.dtype(dtype)
        if dt == np.float32:
            return NeuralDtype.FLOAT32
        if dt == np.float64:
            return NeuralDtype.FLOAT64
    raise ValueError(f"unsupported dtype {dtype!r} (float32 or float64)")


class Tensor:
    """Multi-dimensional float32/float64 array resident on the GPU."""

    def __init__(self, ptr, owns_data: bool = True):
        if ptr is None or ptr == 0:
            raise NeuralException(NeuralError.NULL_POINTER, "Null tensor pointer")
        self._ptr = ptr
        self._owns_data = owns_data

    def __del__(self):
        if getattr(self, "_ptr", None) and self._owns_data:
            _lib.neural_tensor_free(self._ptr)
            self._ptr = None

    # ---- construction -------------------------------------------------------
    @classmethod
    def _wrap(cls, ptr):
        if ptr is None or ptr == 0:
            raise NeuralException(_lib.neural_get_last_error())
        return cls(ptr)

    @classmethod
    def create(cls, shape: Sequence[int], dtype: int = NeuralDtype.FLOAT32) -> "Tensor":
        shape = tuple(int(s) for s in shape)
        return cls._wrap(_lib.neural_tensor_create(_shape_arr(shape), len(shape), _dtype_code(dtype)))

    @classmethod
    def zeros(cls, shape: Sequence[int], dtype: int = NeuralDtype.FLOAT32) -> "Tensor":
        shape = tuple(int(s) for s in shape)
        return cls._wrap(_lib.neural_tensor_zeros(_shape_arr(shape), len(shape), _dtype_code(dtype)))

    @classmethod
    def ones(cls, shape: Sequence[int], dtype: int = NeuralDtype.FLOAT32) -> "Tensor":
        shape = tuple(int(s) for s in shape)
        return cls._wrap(_lib.neural_tensor_ones(_shape_arr(shape), len(shape), _dtype_code(dtype)))

    @classmethod
    def from_numpy(cls, arr: "np.ndarray") -> "Tensor":
        """Copy a NumPy array to a new device tensor (non-float dtypes become float32)."""
        if arr.dtype == np.float64:
            dtype, arr = NeuralDtype.FLOAT64, np.ascontiguousarray(arr, dtype=np.float64)
        else:
            dtype, arr = NeuralDtype.FLOAT32, np.ascontiguousarray(arr, dtype=np.float32)
        t = cls.create(arr.shape, dtype)
        if arr.nbytes:
            _check_error(_lib.neural_tensor_upload(t._ptr, arr.ctypes.data, arr.nbytes), "upload")
        return t

    @classmethod
    def from_numpy_zero_copy(cls, arr: "np.ndarray") -> "Tensor":
        """Wrap a C-contiguous float32/float64 array without copying."""
        if arr.dtype == np.float32:
            dtype = NeuralDtype.FLOAT32
        elif arr.dtype == np.float64:
            dtype = NeuralDtype.FLOAT64
        else:
            raise ValueError(f"Unsupported dtype {arr.dtype}. Must be float32 or float64.")
        if not arr.flags["C_CONTIGUOUS"]:
            raise ValueError("Array must be C-contiguous for zero-copy. Use np.ascontiguousarray() first.")
        ptr = _lib.neural_tensor_from_buffer(arr.ctypes.data, _shape_arr(arr.shape), arr.ndim, dtype, None)
        t = cls._wrap(ptr)
        t._numpy_ref = arr
        return t

    @classmethod
    def from_torch(cls, t) -> "Tensor":
        """Wrap a float32/float64 torch tensor in place (device or host memory),
        honouring its strides."""
        import torch
        if t.dtype == torch.float32:
            dtype, es = NeuralDtype.FLOAT32, 4
        elif t.dtype == torch.float64:
            dtype, es = NeuralDtype.FLOAT64, 8
        else:
            raise ValueError(f"Unsupported dtype {t.dtype}")
        strides = (ctypes.c_int64 * max(t.dim(), 1))(*[s * es for s in t.stride()])
        ptr = _lib.neural_tensor_from_buffer(t.data_ptr(), _shape_arr(tuple(t.shape)), t.dim(), dtype, strides)
        w = cls._wrap(ptr)
        w._torch_ref = t
        return w

    @classmethod
    def from_list(cls, data: List, dtype: int = NeuralDtype.FLOAT32) -> "Tensor":
        arr = np.array(data, dtype=np.float32 if dtype == NeuralDtype.FLOAT32 else np.float64)
        return cls.from_numpy(arr)

    # ---- properties ------------------------------------------------------------
    @property
    def shape(self) -> tuple:
        nd = _lib.neural_tensor_ndim(self._ptr)
        if nd == 0:
            return ()
        sp = _lib.neural_tensor_shape(self._ptr)
        return tuple(int(sp[i]) for i in range(nd))

    @property
    def ndim(self) -> int:
        return int(_lib.neural_tensor_ndim(self._ptr))

    @property
    def dtype(self) -> int:
        return int(_lib.neural_tensor_dtype(self._ptr))

    @property
    def numel(self) -> int:
        return int(_lib.neural_tensor_numel(self._ptr))

    @property
    def nbytes(self) -> int:
        return int(_lib.neural_tensor_bytes(self._ptr))

    @property
    def strides(self) -> tuple:
        """Strides in bytes."""
        sp = _lib.neural_tensor_stride(self._ptr)
        return tuple(int(sp[i]) for i in range(self.ndim))

    @property
    def is_contiguous(self) -> bool:
        return _lib.neural_tensor_is_contiguous(self._ptr) == 1

    @property
    def data_ptr(self) -> int:
        """Host pointer to the data (maps the host mirror)."""
        return _lib.neural_tensor_data(self._ptr)

    @property
    def device_ptr(self) -> int:
        """Device address of element 0."""
        return _lib.neural_tensor_device_data(self._ptr)

    @property
    def __array_interface__(self) -> dict:
        info = NeuralBufferInfo()
        _check_error(_lib.neural_buffer_info(self._ptr, ctypes.byref(info)), "buffer_info")
        return {
            "version": 3,
            "data": (info.data, False),
            "shape": self.shape,
            "typestr": "<f4" if self.dtype == NeuralDtype.FLOAT32 else "<f8",
            "strides": self.strides,
        }

    def numpy_zero_copy(self) -> "np.ndarray":
        """View of the host mirror; valid until the next library call that
        uses this tensor."""
        return np.asarray(self)

    # ---- data movement ---------------------------------------------------------
    def numpy(self) -> "np.ndarray":
        np_dtype = np.float32 if self.dtype == NeuralDtype.FLOAT32 else np.float64
        if not self.is_contiguous:
            return self.contiguous().numpy()
        out = np.empty(self.shape, dtype=np_dtype)
        if out.nbytes:
            _check_error(_lib.neural_tensor_download(self._ptr, out.ctypes.data, out.nbytes), "download")
        return out

    def tolist(self) -> List:
        return self.numpy().tolist()

    def fill(self, value: float) -> "Tensor":
        _check_error(_lib.neural_tensor_fill(self._ptr, ctypes.c_double(value)), "fill")
        return self

    def copy(self) -> "Tensor":
        new = Tensor.create(self.shape, self.dtype)
        _check_error(_lib.neural_tensor_copy(new._ptr, self._ptr), "copy")
        return new

    def contiguous(self) -> "Tensor":
        if self.is_contiguous:
            return self
        ptr = _lib.neural_tensor_make_contiguous(self._ptr)
        return Tensor._wrap(ptr)

    def reshape(self, shape: Sequence[int]) -> "Tensor":
        shape = tuple(int(s) for s in shape)
        ptr = _lib.neural_tensor_reshape(self._ptr, _shape_arr(shape), len(shape))
        v = Tensor._wrap(ptr)
        v._base = self
        return v

    def detach(self) -> "Tensor":
        d = Tensor(self._ptr, owns_data=False)
        d._requires_grad = False
        d._grad_fn = None
        d._base = self
        return d

    def detach_(self) -> "Tensor":
        self._requires_grad = False
        self._grad_fn = None
        return self

    @property
    def requires_grad(self) -> bool:
        return getattr(self, "_requires_grad", False)

    @requires_grad.setter
    def requires_grad(self, value: bool) -> None:
        self._requires_grad = value

    @property
    def grad(self):
        return getattr(self, "_grad", None)

    @grad.setter
    def grad(self, value):
        self._grad = value

    # ---- reductions (new) ---------------------------------------------------------
    def sum(self) -> float:
        r = ctypes.c_double()
        _check_error(_lib.neural_sum(self._ptr, ctypes.byref(r)), "sum")
        return r.value

    def mean(self) -> float:
        r = ctypes.c_double()
        _check_error(_lib.neural_mean(self._ptr, ctypes.byref(r)), "mean")
        return r.value

    def max(self) -> float:
        r = ctypes.c_double()
        _check_error(_lib.neural_max(self._ptr, ctypes.byref(r)), "max")
        return r.value

    def argmax(self) -> int:
        r = ctypes.c_int64()
        _check_error(_lib.neural_argmax(self._ptr, ctypes.byref(r)), "argmax")
        return r.value

    def _row_outputs(self):
        if not self.shape or self.shape[-1] <= 0:
            raise NeuralException(NeuralError.INVALID_ARGUMENT, "row statistics need a non-empty last dimension")
        rows = self.numel // self.shape[-1]
        return [Tensor.create([rows], self.dtype) for _ in range(3)], np.empty(rows, dtype=np.int64)

    def row_stats(self):
        """(sum, mean, max, argmax) of every row over the last dimension from one
        read of the tensor (neural_row_stats; no counterpart in the reference):
        three Tensors of `rows` values and an int64 numpy array, equal bit for
        bit to the separate row reductions."""
        (s, m, mx), idx = self._row_outputs()
        _check_error(_lib.neural_row_stats(self._ptr, s._ptr, m._ptr, mx._ptr, idx.ctypes.data), "row_stats")
        return s, m, mx, idx

    def bias_add_row_stats(self, bias: "Tensor"):
        """(self + bias, and that result's row sum, mean, max, argmax) in one
        pass (neural_bias_add_row_stats; no counterpart in the reference)."""
        out = Tensor.create(self.shape, self.dtype)
        (s, m, mx), idx = self._row_outputs()
        rc = _lib.neural_bias_add_row_stats(out._ptr, self._ptr, bias._ptr, s._ptr, m._ptr, mx._ptr, idx.ctypes.data)
        _check_error(rc, "bias_add_row_stats")
        return out, s, m, mx, idx

    # ---- arithmetic (tensor.py:627-665 of the reference) ----------------------------
    def _binary(self, other, fn, label):
        if not isinstance(other, Tensor):
            raise TypeError(f"Cannot {label} Tensor and {type(other)}")
        result = Tensor.create(self.shape, self.dtype)
        _check_error(fn(result._ptr, self._ptr, other._ptr), label)
        return result

    def __add__(self, other):
        return self._binary(other, _lib.neural_add, "add")

    def __sub__(self, other):
        return self._binary(other, _lib.neural_sub, "sub")

    def __mul__(self, other):
        return self._binary(other, _lib.neural_mul, "mul")

    def __truediv__(self, other):
        return self._binary(other, _lib.neural_div, "div")

    def __neg__(self):
        result = Tensor.create(self.shape, self.dtype)
        _check_error(_lib.neural_neg(result._ptr, self._ptr), "neg")
        return result

    def __matmul__(self, other):
        raise NeuralException(NeuralError.NOT_IMPLEMENTED, "matmul is outside this library's hot path")

    def __repr__(self) -> str:
        return f"Tensor(shape={self.shape}, dtype={'float32' if self.dtype == 0 else 'float64'})"

    def __str__(self) -> str:
        return str(self.numpy())


def zeros(shape: Sequence[int], dtype: int = NeuralDtype.FLOAT32) -> Tensor:
    return Tensor.zeros(shape, dtype)


def ones(shape: Sequence[int], dtype: int = NeuralDtype.FLOAT32) -> Tensor:
    return Tensor.ones(shape, dtype)


def tensor(data: Union[List, "np.ndarray"], dtype: int = NeuralDtype.FLOAT32) -> Tensor:
    if HAS_NUMPY and isinstance(data, np.ndarray):
        return Tensor.from_numpy(data)
    return Tensor.from_list(data, dtype)
