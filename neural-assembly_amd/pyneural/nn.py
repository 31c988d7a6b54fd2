"""
Activation modules of the reference ``pyneural/nn.py`` that sit on the hot
path: ReLU (nn.py:118-133 -> neural_relu), Sigmoid, Softmax (nn.py:152-173 ->
neural_softmax over the last dim) and Tanh (nn.py:176-190 -> act_tanh), plus
LogSoftmax (rows, formula of metrics_losses.c:47-64).  Each allocates the
output and makes one library call.  Loss modules: CrossEntropyLoss
(nn.py:629-654 -> neural_cross_entropy_loss) and LabelSmoothingCrossEntropy
(nn.py:657-751 -> label_smoothing_ce_forward / _backward).  Dropout
(nn.py:193-301 -> neural_dropout_forward / _backward) keeps its mask in device
memory.  Fused epilogues: add_relu (vec_add_relu_fusion, fusion.asm:200-226)
and bias_add_act (bias add of nn_layers.asm:472-539 followed by an
activation, one pass).
"""

import ctypes

import numpy as np

from .core import _lib, _check_error, NeuralDtype
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

    def forward_f64_dev(self, logits_ptr, targets_ptr, batch_size, loss_ptr):
        """Addition without a reference counterpart: device pointers only; the
        mean loss goes into the double at loss_ptr (device memory) and the
        call returns without waiting for it (label_smoothing_ce_forward_dev).
        A target outside [0, K) makes that loss NaN."""
        rc = _lib.label_smoothing_ce_forward_dev(logits_ptr, targets_ptr, batch_size, self.num_classes,
                                                 self.smoothing, loss_ptr)
        _check_error(rc, "label_smoothing_ce_forward_dev")
        self._cached_logits, self._cached_targets, self._cached_batch_size = logits_ptr, targets_ptr, batch_size

    def forward_backward_f64_dev(self, logits_ptr, targets_ptr, batch_size, grad_out_ptr, loss_ptr):
        """forward_backward_f64 with the loss left in device memory, as
        forward_f64_dev (label_smoothing_ce_fused_dev)."""
        rc = _lib.label_smoothing_ce_fused_dev(logits_ptr, targets_ptr, batch_size, self.num_classes,
                                               self.smoothing, loss_ptr, grad_out_ptr)
        _check_error(rc, "label_smoothing_ce_fused_dev")

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



class Dropout(Module):
    """Inverted dropout: in training, each element is zeroed with probability
    ``p`` and the rest are scaled by ``1 / (1 - p)``; identity in eval mode.
    Draws come from the library's copy of the C library's rand() stream (see
    ``dropout_seed``), one per element, as the reference's kernel draws them.
    float32 tensors only (the reference kernel reads float data)."""

    def __init__(self, p: float = 0.5):
        super().__init__()
        if not 0.0 <= p <= 1.0:
            raise ValueError(f"Dropout probability must be in [0, 1], got {p}")
        self.p = p
        self._mask = None  # device bytes, held in a float32 tensor of ceil(n / 4) words
        self._numel = 0

    @staticmethod
    def _mask_buffer(numel: int) -> Tensor:
        return Tensor.zeros([max((numel + 3) // 4, 1)], NeuralDtype.FLOAT32)

    def forward(self, x: Tensor) -> Tensor:
        if not self.training or self.p == 0.0:
            out = Tensor.create(x.shape, x.dtype)
            _check_error(_lib.neural_tensor_copy(out._ptr, x._ptr), "dropout (identity)")
            return out
        numel = x.numel
        if self.p == 1.0:  # all dropped, no draws taken (reference nn.py:241-249)
            self._mask, self._numel = self._mask_buffer(numel), numel
            return Tensor.zeros(x.shape, x.dtype)
        if x.dtype != NeuralDtype.FLOAT32:
            raise TypeError("dropout works on float32 tensors")
        src = x.contiguous()
        out = Tensor.create(x.shape, x.dtype)
        mask = self._mask_buffer(numel)
        _check_error(_lib.neural_dropout_forward(src.device_ptr, out.device_ptr, mask.device_ptr, numel,
                                                 ctypes.c_float(self.p)), "dropout forward")
        self._mask, self._numel = mask, numel
        return out

    def backward(self, grad_output: Tensor) -> Tensor:
        if self._mask is None:
            raise RuntimeError("Dropout.backward called before forward")
        go = grad_output.contiguous()
        gi = Tensor.create(grad_output.shape, grad_output.dtype)
        _check_error(_lib.neural_dropout_backward(go.device_ptr, gi.device_ptr, self._mask.device_ptr, self._numel,
                                                  ctypes.c_float(self.p)), "dropout backward")
        return gi

    def mask(self) -> "np.ndarray":
        """The last forward's keep mask (uint8, one byte per element)."""
        if self._mask is None:
            return np.zeros(0, dtype=np.uint8)
        return self._mask.numpy().view(np.uint8)[: self._numel].copy()

    def __repr__(self) -> str:
        return f"Dropout(p={self.p})"


def dropout_seed(seed: int) -> None:
    """Position the dropout stream as srand(seed) positions the C library's
    rand() (the stream starts as srand(1))."""
    _check_error(_lib.neural_dropout_seed(ctypes.c_uint32(seed & 0xFFFFFFFF)), "dropout seed")


def add_relu(a: Tensor, b: Tensor) -> Tensor:
    """max(0, a + b) in one pass (b broadcasts, e.g. a [.., C] bias)."""
    out = Tensor.create(a.shape, a.dtype)
    _check_error(_lib.neural_add_relu(out._ptr, a._ptr, b._ptr), "add_relu")
    return out


ACTIVATIONS = {"none": 0, "relu": 1, "sigmoid": 2, "tanh": 3, "gelu": 4, "leaky_relu": 5, "elu": 6, "selu": 7,
               "swish": 8, "mish": 9, "hardswish": 10, "softplus": 11, "hardtanh": 12}


def bias_add_act(x: Tensor, bias: Tensor, activation: str = "relu", alpha: float = None) -> Tensor:
    """act(x + bias) for x [.., C] and bias [C] in one pass; equal bit for bit
    to the bias add followed by the activation.  alpha defaults to 0.01 for
    leaky_relu and 1.0 for elu (the reference's defaults)."""
    code = ACTIVATIONS[activation]
    if alpha is None:
        alpha = 0.01 if activation == "leaky_relu" else 1.0
    out = Tensor.create(x.shape, x.dtype)
    _check_error(_lib.neural_bias_add_act(out._ptr, x._ptr, bias._ptr, code, ctypes.c_double(alpha)),
                 "bias_add_act")
    return out
