"""
Optimizers (reference ``pyneural/optim.py``): SGD, Adam, AdamW over lists of
param/grad tensors, with the opaque OPTS state blob for checkpoints.  Moments
are float64 and live on the GPU; one fused kernel per parameter per step.
"""

import ctypes
from typing import List

from .core import _lib, NeuralException, _check_error
from .tensor import Tensor


class Optimizer:
    def __init__(self):
        self._ptr = None

    def __del__(self):
        if getattr(self, "_ptr", None):
            _lib.opt_free(self._ptr)
            self._ptr = None

    def step(self, params: List[Tensor], grads: List[Tensor]) -> None:
        raise NotImplementedError

    def zero_grad(self, grads: List[Tensor]) -> None:
        for g in grads:
            g.fill(0.0)

    @property
    def lr(self) -> float:
        return _lib.opt_get_lr(self._ptr)

    @lr.setter
    def lr(self, value: float):
        _lib.opt_set_lr(self._ptr, ctypes.c_double(value))

    def _do_step(self, params: List[Tensor], grads: List[Tensor], label: str):
        if len(params) != len(grads):
            raise ValueError("params and grads must have same length")
        n = len(params)
        pp = (ctypes.c_void_p * max(n, 1))(*[p._ptr for p in params])
        gp = (ctypes.c_void_p * max(n, 1))(*[g._ptr for g in grads])
        _check_error(_lib.opt_step(self._ptr, pp, gp, n), label)
        # The handle clips the gradients of its latest step (neural_clip_grad_*);
        # keep those tensors alive while it may touch them.
        self._last_grads = list(grads)

    def clip_grad_norm(self, max_norm: float) -> None:
        """Clip the gradients of the latest step by their global L2 norm
        (neural_clip_grad_norm, optimizers.asm:1370-1516)."""
        _check_error(_lib.neural_clip_grad_norm(self._ptr, ctypes.c_double(max_norm)), "clip_grad_norm")

    def clip_grad_value(self, min_val: float, max_val: float) -> None:
        """Clamp the gradients of the latest step to [min_val, max_val]
        (neural_clip_grad_value, optimizers.asm:1527-1620)."""
        _check_error(_lib.neural_clip_grad_value(self._ptr, ctypes.c_double(min_val), ctypes.c_double(max_val)),
                     "clip_grad_value")

    def state_bytes(self) -> bytes:
        if not self._ptr:
            return b""
        nbytes = int(_lib.opt_state_bytes(self._ptr))
        if nbytes <= 0:
            return b""
        buf = (ctypes.c_uint8 * nbytes)()
        _check_error(_lib.opt_state_export(self._ptr, ctypes.cast(buf, ctypes.c_void_p), nbytes),
                     "optimizer state export")
        return bytes(buf)

    def load_state_bytes(self, blob: bytes) -> None:
        if not blob:
            return
        if not self._ptr:
            raise ValueError("optimizer handle is not initialized")
        nbytes = len(blob)
        buf = (ctypes.c_uint8 * nbytes).from_buffer_copy(blob)
        _check_error(_lib.opt_state_import(self._ptr, ctypes.cast(buf, ctypes.c_void_p), nbytes),
                     "optimizer state import")

    def save_state(self, filepath: str) -> None:
        with open(filepath, "wb") as f:
            f.write(self.state_bytes())

    def load_state(self, filepath: str) -> None:
        with open(filepath, "rb") as f:
            self.load_state_bytes(f.read())


class SGD(Optimizer):
    def __init__(self, learning_rate: float = 0.01, momentum: float = 0.0):
        super().__init__()
        self.learning_rate = learning_rate
        self.momentum = momentum
        self._ptr = _lib.opt_sgd_create(ctypes.c_double(learning_rate), ctypes.c_double(momentum))
        if not self._ptr:
            raise NeuralException(0, "Failed to create SGD optimizer")

    def step(self, params, grads) -> None:
        self._do_step(params, grads, "sgd step")

    def __repr__(self) -> str:
        return f"SGD(lr={self.learning_rate}, momentum={self.momentum})"


class Adam(Optimizer):
    def __init__(self, learning_rate: float = 0.001, beta1: float = 0.9, beta2: float = 0.999,
                 epsilon: float = 1e-8):
        super().__init__()
        self.learning_rate, self.beta1, self.beta2, self.epsilon = learning_rate, beta1, beta2, epsilon
        self._ptr = _lib.opt_adam_create(ctypes.c_double(learning_rate), ctypes.c_double(beta1),
                                         ctypes.c_double(beta2), ctypes.c_double(epsilon))
        if not self._ptr:
            raise NeuralException(0, "Failed to create Adam optimizer")

    def step(self, params, grads) -> None:
        self._do_step(params, grads, "adam step")

    def __repr__(self) -> str:
        return f"Adam(lr={self.learning_rate}, betas=({self.beta1}, {self.beta2}), eps={self.epsilon})"


class AdamW(Optimizer):
    def __init__(self, learning_rate: float = 0.001, beta1: float = 0.9, beta2: float = 0.999,
                 epsilon: float = 1e-8, weight_decay: float = 0.01):
        super().__init__()
        self.learning_rate, self.beta1, self.beta2 = learning_rate, beta1, beta2
        self.epsilon, self.weight_decay = epsilon, weight_decay
        self._ptr = _lib.opt_adamw_create(ctypes.c_double(learning_rate), ctypes.c_double(beta1),
                                          ctypes.c_double(beta2), ctypes.c_double(epsilon),
                                          ctypes.c_double(weight_decay))
        if not self._ptr:
            raise NeuralException(0, "Failed to create AdamW optimizer")

    def step(self, params, grads) -> None:
        self._do_step(params, grads, "adamw step")

    def __repr__(self) -> str:
        return (f"AdamW(lr={self.learning_rate}, betas=({self.beta1}, {self.beta2}), "
                f"eps={self.epsilon}, wd={self.weight_decay})")
