"""
Training-step checks (reference ``pyneural/training.py:25-79``): NaN/Inf
detection and the gradient L2 norm.  Both use one fused device scan of the
tensor (``neural_tensor_scan``) instead of the reference's host pointer
round trip.  Gradient clipping over a gradient list (the work the reference's
Trainer asks of ``neural_clip_grad_norm``, training.py:267-271;
optimizers.asm:1370-1620) runs as three device launches for the whole list.
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


def _grad_array(grads):
    grads = list(grads)
    arr = (ctypes.c_void_p * max(len(grads), 1))(*[g._ptr if g is not None else None for g in grads])
    return arr, len(grads)


def clip_grad_norm(grads, max_norm: float) -> float:
    """Scale every gradient by max_norm / norm when the global L2 norm exceeds
    max_norm (clip_grad_norm_, optimizers.asm:1370-1516).  Returns the norm
    before clipping.  None entries are skipped."""
    arr, n = _grad_array(grads)
    norm = ctypes.c_double()
    _check_error(_lib.neural_clip_grad_norm_list(arr, n, ctypes.c_double(max_norm), ctypes.byref(norm)),
                 "clip_grad_norm")
    return norm.value


def clip_grad_value(grads, min_val: float, max_val: float) -> None:
    """Clamp every gradient element to [min_val, max_val] with the reference's
    maxsd/minsd rules (clip_grad_value_, optimizers.asm:1527-1620)."""
    arr, n = _grad_array(grads)
    _check_error(_lib.neural_clip_grad_value_list(arr, n, ctypes.c_double(min_val), ctypes.c_double(max_val)),
                 "clip_grad_value")
