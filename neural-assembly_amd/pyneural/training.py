"""
Training-step checks (reference ``pyneural/training.py:25-79``): NaN/Inf
detection and the gradient L2 norm.  Both use one fused device scan of the
tensor (``neural_tensor_scan``) instead of the reference's host pointer
round trip.
"""

import ctypes
import math

from .core import _lib, _check_error


def _scan(tensor):
    has_nan, has_inf, ss = ctypes.c_int(), ctypes.c_int(), ctypes.c_double()
    _check_error(_lib.neural_tensor_scan(tensor._ptr, ctypes.byref(has_nan), ctypes.byref(has_inf),
                                         ctypes.byref(ss)), "scan")
    return bool(has_nan.value), bool(has_inf.value), ss.value


class NaNDetector:
    """Detect NaN or Inf values in tensor data."""

    def __init__(self, raise_on_detect: bool = True):
        self.raise_on_detect = raise_on_detect
        self.nan_count = 0
        self.inf_count = 0

    def has_nan(self, tensor) -> bool:
        return _scan(tensor)[0]

    def has_inf(self, tensor) -> bool:
        return _scan(tensor)[1]

    def check(self, tensor, name: str = "tensor") -> None:
        nan, inf, _ = _scan(tensor)
        if nan:
            self.nan_count += 1
            if self.raise_on_detect:
                raise RuntimeError(f"NaN detected in {name}")
        if inf:
            self.inf_count += 1
            if self.raise_on_detect:
                raise RuntimeError(f"Inf detected in {name}")

    def reset_counts(self) -> None:
        self.nan_count = 0
        self.inf_count = 0


def grad_l2_norm(tensor) -> float:
    """L2 norm of a tensor's data, rounded to float32 as the reference returns."""
    _, _, ss = _scan(tensor)
    return float(ctypes.c_float(math.sqrt(ss)).value)
