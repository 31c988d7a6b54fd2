"""
Extended activation modules (reference ``pyneural/activations.py``): each
allocates the output tensor and calls one ``act_*`` kernel of
libneural_hip.so (formulas of activations_c.c:124-158, double math).
"""

from __future__ import annotations

import ctypes

from .core import _lib, _check_error
from .nn import Module
from .tensor import Tensor


def _act(fn, x: Tensor, label: str, *extra) -> Tensor:
    out = Tensor.create(x.shape, x.dtype)
    _check_error(fn(out._ptr, x._ptr, *extra), label)
    return out


class GELU(Module):
    """0.5*x*(1 + tanh(0.7978845608028654*(x + 0.044715*x^3)))."""

    def forward(self, x: Tensor) -> Tensor:
        return _act(_lib.act_gelu, x, "gelu")

    def __repr__(self) -> str:
        return "GELU()"


class LeakyReLU(Module):
    """x if x >= 0 else alpha*x (alpha default 0.01)."""

    def __init__(self, alpha: float = 0.01):
        super().__init__()
        self.alpha = alpha

    def forward(self, x: Tensor) -> Tensor:
        return _act(_lib.act_leaky_relu, x, "leaky_relu", ctypes.c_double(self.alpha))

    def __repr__(self) -> str:
        return f"LeakyReLU(alpha={self.alpha})"


class ELU(Module):
    """x if x > 0 else alpha*(exp(x) - 1) (alpha default 1.0)."""

    def __init__(self, alpha: float = 1.0):
        super().__init__()
        self.alpha = alpha

    def forward(self, x: Tensor) -> Tensor:
        return _act(_lib.act_elu, x, "elu", ctypes.c_double(self.alpha))

    def __repr__(self) -> str:
        return f"ELU(alpha={self.alpha})"


class SELU(Module):
    """lambda*x if x > 0 else lambda*alpha*(exp(x) - 1)."""

    def forward(self, x: Tensor) -> Tensor:
        return _act(_lib.act_selu, x, "selu")

    def __repr__(self) -> str:
        return "SELU()"


class Swish(Module):
    """x / (1 + exp(-x))."""

    def forward(self, x: Tensor) -> Tensor:
        return _act(_lib.act_swish, x, "swish")

    def __repr__(self) -> str:
        return "Swish()"


class Mish(Module):
    """x * tanh(log(1 + exp(x)))."""

    def forward(self, x: Tensor) -> Tensor:
        return _act(_lib.act_mish, x, "mish")

    def __repr__(self) -> str:
        return "Mish()"


class HardSwish(Module):
    """0 if x <= -3, x if x >= 3, else x*(x+3)/6."""

    def forward(self, x: Tensor) -> Tensor:
        return _act(_lib.act_hardswish, x, "hardswish")

    def __repr__(self) -> str:
        return "HardSwish()"


class Softplus(Module):
    """log(1 + exp(x))."""

    def forward(self, x: Tensor) -> Tensor:
        return _act(_lib.act_softplus, x, "softplus")

    def __repr__(self) -> str:
        return "Softplus()"


class HardTanh(Module):
    """clamp(x, -1, 1)."""

    def forward(self, x: Tensor) -> Tensor:
        return _act(_lib.act_hardtanh, x, "hardtanh")

    def __repr__(self) -> str:
        return "HardTanh()"
