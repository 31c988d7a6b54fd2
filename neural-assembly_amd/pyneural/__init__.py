"""
pyneural -- drop-in Python API for libneural_hip.so, the MI355X (gfx950)
implementation of Neural-Assembly's tensor hot path.

Public names follow the reference package for this path: Tensor, zeros,
ones, tensor; nn.ReLU/Sigmoid/Softmax/Tanh, nn.CrossEntropyLoss /
LabelSmoothingCrossEntropy, nn.Dropout (+ dropout_seed), fused add_relu /
bias_add_act; activations.*; Quantizer /
QuantParams; optim.SGD/Adam/AdamW; training.NaNDetector / grad_l2_norm /
clip_grad_norm / clip_grad_value; save_checkpoint / load_checkpoint;
transforms.Normalize / MinMaxScale / Compose / compute_stats; tensor_ops.*.
"""

from .core import (NeuralError, NeuralDtype, NeuralException, init, shutdown, version, get_last_error,
                   get_error_message, clear_error, set_stream, synchronize, device_info)
from .tensor import Tensor, zeros, ones, tensor
from . import nn, activations, optim, quantize, training, tensor_ops, checkpoint, transforms
from .nn import (ReLU, Sigmoid, Softmax, LogSoftmax, Tanh, CrossEntropyLoss, LabelSmoothingCrossEntropy, Dropout,
                 dropout_seed, add_relu, bias_add_act)
from .activations import GELU, LeakyReLU, ELU, SELU, Swish, Mish, HardSwish, Softplus, HardTanh
from .optim import SGD, Adam, AdamW
from .quantize import Quantizer, QuantParams, quantized_matmul
from .training import NaNDetector, grad_l2_norm, clip_grad_norm, clip_grad_value
from .checkpoint import save_checkpoint, load_checkpoint
from .transforms import Normalize, MinMaxScale, Compose, compute_stats

float32 = NeuralDtype.FLOAT32
float64 = NeuralDtype.FLOAT64

__version__ = "1.0.0"
