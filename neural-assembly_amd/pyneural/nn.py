"""
Activation modules of the reference ``pyneural/nn.py`` that sit on the hot
path: ReLU (nn.py:118-133 -> neural_relu), Sigmoid, Softmax (nn.py:152-173 ->
neural_softmax over the last dim) and Tanh (nn.py:176-190 -> act_tanh), plus
LogSoftmax (rows, formula of metrics_losses.c:47-64).  Each allocates the
output and makes one library call.  Loss modules: CrossEntropyLoss
(nn.py:629-654 -> neural_cross_entropy_loss) and LabelSmoothingCrossEntropy
(nn.py:657-751 -> label_smoothing_ce_forward / _backward).
"""

import ctypes

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


class CrossEntropyLoss(Module):
    """Cross-entropy of softmax(prediction) against class indices held as values
    of the prediction's dtype (reference nn.py:629-654)."""

    def forward(self, prediction: Tensor, target: Tensor) -> float:
        loss = ctypes.c_double()
        _check_error(_lib.neural_cross_entropy_loss(prediction._ptr, target._ptr, ctypes.byref(loss)),
                     "cross_entropy_loss")
        return loss.value

    def __repr__(self) -> str:
        return "CrossEntropyLoss()"


class LabelSmoothingCrossEntropy(Module):
    """Label-smoothed cross-entropy on raw double*/int64* buffers (reference
    nn.py:657-751): smoothed target (1 - a) * one_hot + a / K.  Pointers may be
    host memory (staged to the GPU for the call) or device memory."""

    def __init__(self, num_classes: int, smoothing: float = 0.1):
        super().__init__()
        if not (0.0 <= smoothing <= 1.0):
            raise ValueError(f"smoothing must be in [0, 1], got {smoothing}")
        if num_classes < 1:
            raise ValueError(f"num_classes must be >= 1, got {num_classes}")
        self.smoothing = smoothing
        self.num_classes = num_classes
        self._cached_logits = None
        self._cached_targets = None
        self._cached_batch_size = None

    def forward_f64(self, logits_ptr, targets_ptr, batch_size):
        loss = ctypes.c_double()
        rc = _lib.label_smoothing_ce_forward(logits_ptr, targets_ptr, batch_size, self.num_classes,
                                             self.smoothing, ctypes.byref(loss))
        _check_error(rc, "label_smoothing_ce_forward")
        self._cached_logits, self._cached_targets, self._cached_batch_size = logits_ptr, targets_ptr, batch_size
        return loss.value

    def backward_f64(self, grad_out_ptr, logits_ptr=None, targets_ptr=None, batch_size=None):
        lp = logits_ptr if logits_ptr is not None else self._cached_logits
        tp = targets_ptr if targets_ptr is not None else self._cached_targets
        bs = batch_size if batch_size is not None else self._cached_batch_size
        if lp is None or tp is None or bs is None:
            raise RuntimeError("backward called before forward; provide explicit pointers")
        rc = _lib.label_smoothing_ce_backward(lp, tp, bs, self.num_classes, self.smoothing, grad_out_ptr)
        _check_error(rc, "label_smoothing_ce_backward")

    def forward_backward_f64(self, logits_ptr, targets_ptr, batch_size, grad_out_ptr):
        """Both in one pass over the logits (label_smoothing_ce_fused)."""
        loss = ctypes.c_double()
        rc = _lib.label_smoothing_ce_fused(logits_ptr, targets_ptr, batch_size, self.num_classes, self.smoothing,
                                           ctypes.byref(loss), grad_out_ptr)
        _check_error(rc, "label_smoothing_ce_fused")
        return loss.value

    def forward(self, logits_list, targets_list):
        bs = len(targets_list)
        nc = self.num_classes
        logits_arr = (ctypes.c_double * (bs * nc))(*logits_list)
        targets_arr = (ctypes.c_int64 * bs)(*targets_list)
        return self.forward_f64(ctypes.cast(logits_arr, ctypes.c_void_p), ctypes.cast(targets_arr, ctypes.c_void_p),
                                bs)

    def __call__(self, logits, targets):
        return self.forward(logits, targets)

    def __repr__(self) -> str:
        return f"LabelSmoothingCrossEntropy(num_classes={self.num_classes}, smoothing={self.smoothing})"

