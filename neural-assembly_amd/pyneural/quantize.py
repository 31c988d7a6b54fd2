"""
INT8 quantization: calibration, quantize / dequantize, error and SNR, and
the int8 product -- the interface of the reference's
``pyneural/quantize.py:23-223`` over ``quantize.c``.

Data pointers are whatever the reference accepts (a ctypes array or pointer,
or an integer address) and may point to host or device memory: the library
stages host buffers through HBM.  ``Quantizer(float32=True)`` switches to the
library's float32 entry points (``*_f32``), which read float32 data and
produce exactly what the double entry points produce for the same values.
"""

import ctypes
from dataclasses import dataclass

from . import core
from .core import QuantParamsC, NeuralException, NeuralError


@dataclass
class QuantParams:
    """Scale, zero point and calibrated range of one tensor (the 40-byte C
    struct of quantize.c:39-45 on the Python side)."""

    scale: float = 1.0
    zero_point: int = 0
    min_val: float = 0.0
    max_val: float = 0.0
    symmetric: bool = True

    def _to_c(self) -> QuantParamsC:
        return QuantParamsC(float(self.scale), int(self.zero_point), float(self.min_val), float(self.max_val),
                            int(bool(self.symmetric)))

    @classmethod
    def _from_c(cls, raw: QuantParamsC) -> "QuantParams":
        return cls(raw.scale, raw.zero_point, raw.min_val, raw.max_val, bool(raw.symmetric))

    def __repr__(self):
        kind = "symmetric" if self.symmetric else "affine"
        return (f"QuantParams({kind}: scale {self.scale:.6g}, zero point {self.zero_point}, "
                f"calibrated on [{self.min_val:.4g}, {self.max_val:.4g}])")


def _addr(p) -> ctypes.c_void_p:
    """A C pointer for a ctypes array / pointer, a numpy array or an address."""
    if p is None or isinstance(p, int):
        return ctypes.c_void_p(p)
    if hasattr(p, "ctypes"):
        return ctypes.c_void_p(p.ctypes.data)
    if isinstance(p, ctypes.c_void_p):
        return p
    return ctypes.cast(p, ctypes.c_void_p)


class Quantizer:
    """Calibrate once, then quantize / dequantize / measure.

    symmetric:  zero point 0 and a range of +-max|x|; otherwise affine.
    percentile: when > 0, calibrate on the order statistics at p and 1 - p
                (calibrate_percentile; float64 data only).
    float32:    the data are float32 (the library's *_f32 entry points).
    """

    def __init__(self, symmetric: bool = True, percentile: float = 0.0, float32: bool = False):
        self.symmetric = symmetric
        self.percentile = percentile
        self.float32 = float32
        self.params = None

    def _entry(self, base: str):
        return getattr(core._lib, base + "_f32" if self.float32 else base)

    def _calibrated(self, action: str) -> QuantParamsC:
        if self.params is None:
            raise RuntimeError(f"Quantizer.{action} called before calibrate()")
        return self.params._to_c()

    def calibrate(self, data_ptr, n: int) -> QuantParams:
        raw = QuantParamsC()
        mode = int(bool(self.symmetric))
        if self.percentile > 0.0:
            if self.float32:
                raise NeuralException(NeuralError.NOT_IMPLEMENTED, "percentile calibration of float32 data")
            rc = core._lib.calibrate_percentile(_addr(data_ptr), ctypes.c_int64(n), ctypes.c_double(self.percentile),
                                                mode, ctypes.byref(raw))
        else:
            rc = self._entry("calibrate_minmax")(_addr(data_ptr), ctypes.c_int64(n), mode, ctypes.byref(raw))
        if rc != 0:
            raise RuntimeError(f"calibration of {n} values failed")
        self.params = QuantParams._from_c(raw)
        return self.params

    def quantize(self, data_ptr, n: int) -> ctypes.Array:
        """int8 codes of n values, as a ctypes int8 array."""
        raw = self._calibrated("quantize")
        codes = (ctypes.c_int8 * n)()
        if self._entry("quantize_tensor")(_addr(data_ptr), _addr(codes), ctypes.c_int64(n), ctypes.byref(raw)) != 0:
            raise RuntimeError(f"quantization of {n} values failed")
        return codes

    def dequantize(self, int8_ptr, n: int) -> ctypes.Array:
        """Reconstructed values of n codes: a ctypes float64 array (float32
        with float32=True)."""
        raw = self._calibrated("dequantize")
        values = ((ctypes.c_float if self.float32 else ctypes.c_double) * n)()
        if self._entry("dequantize_tensor")(_addr(int8_ptr), _addr(values), ctypes.c_int64(n), ctypes.byref(raw)) != 0:
            raise RuntimeError(f"dequantization of {n} codes failed")
        return values

    def error(self, original_ptr, n: int) -> float:
        """Mean squared error of quantize -> dequantize."""
        raw = self._calibrated("error")
        return self._entry("quantization_error")(_addr(original_ptr), ctypes.c_int64(n), ctypes.byref(raw))

    def snr(self, original_ptr, n: int) -> float:
        """Signal-to-noise ratio of quantize -> dequantize in dB."""
        raw = self._calibrated("snr")
        return self._entry("quantization_snr")(_addr(original_ptr), ctypes.c_int64(n), ctypes.byref(raw))

    def __repr__(self):
        state = "calibrated" if self.params is not None else "not calibrated"
        return f"Quantizer({'symmetric' if self.symmetric else 'affine'}, {state})"


def quantized_matmul(a_int8, b_int8, m: int, k: int, n: int, params_a: QuantParams,
                     params_b: QuantParams) -> ctypes.Array:
    """C[m, n] = dequant(A[m, k]) @ dequant(B[k, n]) with the inner sums in
    int32 (quantize.c:191-214), as a ctypes float64 array of m * n values.
    A and B are int8 buffers (ctypes arrays, numpy arrays or addresses)."""
    out = (ctypes.c_double * (m * n))()
    pa, pb = params_a._to_c(), params_b._to_c()
    rc = core._lib.quantized_matmul(_addr(a_int8), _addr(b_int8), _addr(out), ctypes.c_int64(m), ctypes.c_int64(k),
                                    ctypes.c_int64(n), ctypes.byref(pa), ctypes.byref(pb))
    if rc != 0:
        raise RuntimeError(f"quantized_matmul of [{m}x{k}] by [{k}x{n}] failed")
    return out
