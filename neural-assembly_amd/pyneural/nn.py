"""
Activation modules of the reference ``pyneural/nn.py`` that sit on the hot
path: ReLU (nn.py:118-133 -> neural_relu), Sigmoid, Softmax (nn.py:152-173 ->
neural_softmax over the last dim) and Tanh (nn.py:176-190 -> act_tanh), plus
LogSoftmax (rows, formula of metrics_losses.c:47-64).  Each allocates the
output and makes one library call.
"""

from .core import _lib, _check_error
from .tensor import Tensor


class Module:
    """Minimal module base: ``m(x)`` calls ``m.forward(x)``."""

    def __init__(self):
        self.training = True

    def __call__(self, *args, **kwargs):
        return self.forward(*args, **kwargs)

    def forward(self, *args, **kwargs):  # pragma: no cover
        raise NotImplementedError

    def parameters(self):
        return []

    def train(self, mode: bool = True):
        self.training = mode
        return self

    def eval(self):
        return self.train(False)


def _unary(fn, x: Tensor, label: str) -> Tensor:
    out = Tensor.create(x.shape, x.dtype)
    _check_error(fn(out._ptr, x._ptr), label)
    return out


class ReLU(Module):
    """y = max(0, x) (NaN and -0 map to +0, as maxss x, 0 does)."""

    def forward(self, x: Tensor) -> Tensor:
        return _unary(_lib.neural_relu, x, "relu")

    def __repr__(self):
        return "ReLU()"


class Sigmoid(Module):
    """y = 1 / (1 + exp(-x)), double math."""

    def forward(self, x: Tensor) -> Tensor:
        return _unary(_lib.neural_sigmoid, x, "sigmoid")

    def __repr__(self):
        return "Sigmoid()"


class Softmax(Module):
    """Row softmax over the last dimension."""

    def __init__(self, dim: int = -1):
        super().__init__()
        self.dim = dim

    def forward(self, x: Tensor) -> Tensor:
        if self.dim not in (-1, x.ndim - 1):
            raise ValueError("Softmax runs over the last dimension only")
        return _unary(_lib.neural_softmax, x, "softmax")

    def __repr__(self):
        return f"Softmax(dim={self.dim})"


class LogSoftmax(Module):
    """Row log-softmax over the last dimension."""

    def __init__(self, dim: int = -1):
        super().__init__()
        self.dim = dim

    def forward(self, x: Tensor) -> Tensor:
        if self.dim not in (-1, x.ndim - 1):
            raise ValueError("LogSoftmax runs over the last dimension only")
        return _unary(_lib.neural_log_softmax, x, "log_softmax")

    def __repr__(self):
        return f"LogSoftmax(dim={self.dim})"


class Tanh(Module):
    """y = tanh(x), double math."""

    def forward(self, x: Tensor) -> Tensor:
        return _unary(_lib.act_tanh, x, "tanh")

    def __repr__(self):
        return "Tanh()"
