"""
SGD, Adam and AdamW over lists of parameter / gradient tensors -- the
interface of the reference's ``pyneural/optim.py:16-237`` over the C
optimizer handle of ``optimizers_c.c:135-562``.

One handle owns the float64 moments (on the GPU here) and the step counter;
``opt_step`` updates every parameter with one fused kernel each.  The state
blob is the OPTS format of ``opt_state_export`` (checkpoints embed it).

Each concrete optimizer only names its C constructor and the order of the
hyper-parameters it takes; construction, stepping, clipping and the state
blob are shared.  The handle is released by a finalizer, so an optimizer that
failed half-way through construction never frees an invalid pointer.
"""

import ctypes
import weakref
from pathlib import Path
from typing import Iterable, List

from .core import _lib, NeuralException, _check_error, get_last_error
from .tensor import Tensor


def _addresses(tensors: List[Tensor]):
    """A C array of the tensors' descriptor addresses (length >= 1)."""
    return (ctypes.c_void_p * max(len(tensors), 1))(*[t._ptr for t in tensors])


class Optimizer:
    """Owner of one C optimizer handle."""

    _ctor = ""           # C constructor
    _hyper = ()          # its double arguments, in order (attribute names)

    def __init__(self):
        self._ptr = None
        self._latest_grads: List[Tensor] = []

    def _open(self, **hyper) -> None:
        for name, value in hyper.items():
            setattr(self, name, value)
        args = [ctypes.c_double(float(hyper[name])) for name in self._hyper]
        handle = getattr(_lib, self._ctor)(*args)
        if not handle:
            raise NeuralException(get_last_error(), f"{self._ctor} returned no optimizer handle")
        self._ptr = handle
        weakref.finalize(self, _lib.opt_free, handle)

    # ---- stepping ------------------------------------------------------------------

    def step(self, params: List[Tensor], grads: List[Tensor]) -> None:
        """One update of every parameter from its gradient (same order)."""
        params, grads = list(params), list(grads)
        if len(params) != len(grads):
            raise ValueError(f"{type(self).__name__}.step got {len(params)} parameters and {len(grads)} gradients")
        rc = _lib.opt_step(self._ptr, _addresses(params), _addresses(grads), len(params))
        _check_error(rc, f"{type(self).__name__}.step")
        # the handle's clip entry points act on the gradients of its latest
        # step: keep those tensors alive while it may touch them
        self._latest_grads = grads

    def zero_grad(self, grads: Iterable[Tensor]) -> None:
        for g in grads:
            g.fill(0.0)

    @property
    def lr(self) -> float:
        return _lib.opt_get_lr(self._ptr)

    @lr.setter
    def lr(self, value: float):
        _lib.opt_set_lr(self._ptr, ctypes.c_double(value))

    # ---- gradient clipping of the latest step ---------------------------------------

    def clip_grad_norm(self, max_norm: float) -> None:
        """Scale the gradients of the latest step so that their global L2
        norm is at most max_norm (neural_clip_grad_norm,
        optimizers.asm:1370-1516)."""
        _check_error(_lib.neural_clip_grad_norm(self._ptr, ctypes.c_double(max_norm)), "clip_grad_norm")

    def clip_grad_value(self, min_val: float, max_val: float) -> None:
        """Clamp the gradients of the latest step to [min_val, max_val]
        (neural_clip_grad_value, optimizers.asm:1527-1620)."""
        rc = _lib.neural_clip_grad_value(self._ptr, ctypes.c_double(min_val), ctypes.c_double(max_val))
        _check_error(rc, "clip_grad_value")

    # ---- the OPTS state blob ----------------------------------------------------------

    def state_bytes(self) -> bytes:
        """The handle's state as the OPTS blob (b"" without a handle)."""
        if not self._ptr:
            return b""
        size = int(_lib.opt_state_bytes(self._ptr))
        if size <= 0:
            return b""
        blob = bytearray(size)
        view = (ctypes.c_char * size).from_buffer(blob)
        _check_error(_lib.opt_state_export(self._ptr, ctypes.addressof(view), size), "opt_state_export")
        return bytes(blob)

    def load_state_bytes(self, blob: bytes) -> None:
        """Replace the handle's state with an OPTS blob (empty: no change)."""
        if not blob:
            return
        if not self._ptr:
            raise ValueError(f"{type(self).__name__} has no C optimizer handle to load state into")
        data = bytearray(blob)
        view = (ctypes.c_char * len(data)).from_buffer(data)
        _check_error(_lib.opt_state_import(self._ptr, ctypes.addressof(view), len(data)), "opt_state_import")

    def save_state(self, filepath: str) -> None:
        Path(filepath).write_bytes(self.state_bytes())

    def load_state(self, filepath: str) -> None:
        self.load_state_bytes(Path(filepath).read_bytes())

    def __repr__(self) -> str:
        shown = ", ".join(f"{name}={getattr(self, name)}" for name in self._hyper)
        return f"{type(self).__name__}({shown})"


class SGD(Optimizer):
    """SGD with momentum (optimizers_c.c:218-249)."""

    _ctor = "opt_sgd_create"
    _hyper = ("learning_rate", "momentum")

    def __init__(self, learning_rate: float = 0.01, momentum: float = 0.0):
        super().__init__()
        self._open(learning_rate=learning_rate, momentum=momentum)


class Adam(Optimizer):
    """Adam (optimizers_c.c:251-293)."""

    _ctor = "opt_adam_create"
    _hyper = ("learning_rate", "beta1", "beta2", "epsilon")

    def __init__(self, learning_rate: float = 0.001, beta1: float = 0.9, beta2: float = 0.999,
                 epsilon: float = 1e-8):
        super().__init__()
        self._open(learning_rate=learning_rate, beta1=beta1, beta2=beta2, epsilon=epsilon)


class AdamW(Optimizer):
    """AdamW, decoupled weight decay (optimizers_c.c:295-348)."""

    _ctor = "opt_adamw_create"
    _hyper = ("learning_rate", "beta1", "beta2", "epsilon", "weight_decay")

    def __init__(self, learning_rate: float = 0.001, beta1: float = 0.9, beta2: float = 0.999,
                 epsilon: float = 1e-8, weight_decay: float = 0.01):
        super().__init__()
        self._open(learning_rate=learning_rate, beta1=beta1, beta2=beta2, epsilon=epsilon,
                   weight_decay=weight_decay)
