"""
INT8 quantization (reference ``pyneural/quantize.py``): ``QuantParams``,
``Quantizer`` (calibrate / quantize / dequantize / error / snr).  Pointers are
ctypes float64 (or, via the ``*_f32`` dtype switch, float32) arrays or raw
addresses -- host or device; the library stages host buffers through HBM.
"""

import ctypes

from . import core
from .core import QuantParamsC, NeuralException, NeuralError


class QuantParams:
    """Python-side view of quantization parameters."""

    def __init__(self, scale: float = 1.0, zero_point: int = 0, min_val: float = 0.0,
                 max_val: float = 0.0, symmetric: bool = True):
        self.scale = scale
        self.zero_point = zero_point
        self.min_val = min_val
        self.max_val = max_val
        self.symmetric = symmetric

    def _to_c(self) -> QuantParamsC:
        p = QuantParamsC()
        p.scale = self.scale
        p.zero_point = self.zero_point
        p.min_val = self.min_val
        p.max_val = self.max_val
        p.symmetric = 1 if self.symmetric else 0
        return p

    @classmethod
    def _from_c(cls, p: QuantParamsC) -> "QuantParams":
        return cls(scale=p.scale, zero_point=p.zero_point, min_val=p.min_val, max_val=p.max_val,
                   symmetric=bool(p.symmetric))

    def __repr__(self):
        mode = "symmetric" if self.symmetric else "affine"
        return (f"QuantParams({mode}, scale={self.scale:.6g}, "
                f"zp={self.zero_point}, range=[{self.min_val:.4g}, {self.max_val:.4g}])")


class Quantizer:
    """INT8 quantizer with min/max or percentile calibration (quantize.py:60-105).

    Args:
        symmetric: symmetric (zero_point 0) or affine quantization.
        percentile: when > 0, calibrate on the [p, 1 - p] order statistics
            (calibrate_percentile, float64 data only; NOT_IMPLEMENTED with
            float32=True).
        float32: inputs are float32 arrays (the library's *_f32 entry points)
            instead of the reference's float64.
    """

    def __init__(self, symmetric: bool = True, percentile: float = 0.0, float32: bool = False):
        self.symmetric = symmetric
        self.percentile = percentile
        self.float32 = float32
        self.params = None

    def _fn(self, name):
        return getattr(core._lib, name + ("_f32" if self.float32 else ""))

    def calibrate(self, data_ptr, n: int) -> QuantParams:
        c_params = QuantParamsC()
        if self.percentile > 0.0:
            if self.float32:
                raise NeuralException(NeuralError.NOT_IMPLEMENTED, "percentile calibration of float32 data")
            rc = core._lib.calibrate_percentile(ctypes.cast(data_ptr, ctypes.c_void_p), ctypes.c_int64(n),
                                                ctypes.c_double(self.percentile), 1 if self.symmetric else 0,
                                                ctypes.byref(c_params))
        else:
            rc = self._fn("calibrate_minmax")(ctypes.cast(data_ptr, ctypes.c_void_p), ctypes.c_int64(n),
                                              1 if self.symmetric else 0, ctypes.byref(c_params))
        if rc != 0:
            raise RuntimeError("Calibration failed")
        self.params = QuantParams._from_c(c_params)
        return self.params

    def quantize(self, data_ptr, n: int) -> ctypes.Array:
        if self.params is None:
            raise RuntimeError("Must calibrate before quantizing")
        out = (ctypes.c_int8 * n)()
        c_params = self.params._to_c()
        rc = self._fn("quantize_tensor")(ctypes.cast(data_ptr, ctypes.c_void_p), ctypes.cast(out, ctypes.c_void_p),
                                         ctypes.c_int64(n), ctypes.byref(c_params))
        if rc != 0:
            raise RuntimeError("Quantization failed")
        return out

    def dequantize(self, int8_ptr, n: int) -> ctypes.Array:
        if self.params is None:
            raise RuntimeError("Must calibrate before dequantizing")
        out = (ctypes.c_float * n)() if self.float32 else (ctypes.c_double * n)()
        c_params = self.params._to_c()
        rc = self._fn("dequantize_tensor")(ctypes.cast(int8_ptr, ctypes.c_void_p), ctypes.cast(out, ctypes.c_void_p),
                                           ctypes.c_int64(n), ctypes.byref(c_params))
        if rc != 0:
            raise RuntimeError("Dequantization failed")
        return out

    def error(self, original_ptr, n: int) -> float:
        if self.params is None:
            raise RuntimeError("Must calibrate first")
        c_params = self.params._to_c()
        return self._fn("quantization_error")(ctypes.cast(original_ptr, ctypes.c_void_p), ctypes.c_int64(n),
                                              ctypes.byref(c_params))

    def snr(self, original_ptr, n: int) -> float:
        if self.params is None:
            raise RuntimeError("Must calibrate first")
        c_params = self.params._to_c()
        return self._fn("quantization_snr")(ctypes.cast(original_ptr, ctypes.c_void_p), ctypes.c_int64(n),
                                            ctypes.byref(c_params))

    def __repr__(self):
        mode = "symmetric" if self.symmetric else "affine"
        calib = "calibrated" if self.params else "uncalibrated"
        return f"Quantizer({mode}, {calib})"


def quantized_matmul(a_int8, b_int8, m: int, k: int, n: int, params_a: QuantParams,
                     params_b: QuantParams) -> ctypes.Array:
    """C[M,N] = dequant(A[M,K]) @ dequant(B[K,N]) (reference quantize.py:195-223,
    quantize.c:191-214): the inner sum in int32, then scaled to float64, on the
    matrix cores.  a_int8 / b_int8 are ctypes int8 arrays (or anything with a
    buffer, e.g. numpy int8 arrays); returns a ctypes float64 array of m*n."""
    c_out = (ctypes.c_double * (m * n))()
    pa = params_a._to_c()
    pb = params_b._to_c()
    rc = core._lib.quantized_matmul(_buf_ptr(a_int8), _buf_ptr(b_int8), ctypes.addressof(c_out), ctypes.c_int64(m),
                               ctypes.c_int64(k), ctypes.c_int64(n), ctypes.byref(pa), ctypes.byref(pb))
    if rc != 0:
        raise RuntimeError("Quantized matmul failed")
    return c_out


def _buf_ptr(a) -> int:
    """Address of a ctypes array, a numpy array or an integer address."""
    if isinstance(a, int):
        return a
    if hasattr(a, "ctypes"):
        return a.ctypes.data
    return ctypes.addressof(a)
