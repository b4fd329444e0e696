"""oxitorch_amd.nn: the hot-path subset of the reference `oxitorch.nn`
(python/oxitorch/nn/__init__.py): functional norms, activations, softmax
family, cross-entropy and embedding, plus their Module wrappers."""

from .module import Module, Parameter, Sequential
from . import functional
from .functional import (
    cross_entropy,
    embedding,
    gelu,
    layer_norm,
    leaky_relu,
    log_softmax,
    mse_loss,
    relu,
    rms_norm,
    sigmoid,
    silu,
    softmax,
    tanh,
)
from .layers import GELU, Embedding, LayerNorm, LeakyReLU, ReLU, RMSNorm, SiLU, Sigmoid, Softmax, Tanh
# outside the device hot path: each raises NotImplementedError when called
from .functional import bmm, conv2d, dropout, linear, max_pool2d
from .layers import Conv2d, Dropout, Linear, MaxPool2d

__all__ = [
    "Module", "Parameter", "Sequential", "functional", "cross_entropy", "embedding", "gelu", "layer_norm",
    "leaky_relu", "log_softmax", "mse_loss", "relu", "rms_norm", "sigmoid", "silu", "softmax", "tanh",
    "GELU", "Embedding", "LayerNorm", "LeakyReLU", "ReLU", "RMSNorm", "SiLU", "Sigmoid", "Softmax", "Tanh",
    "bmm", "conv2d", "dropout", "linear", "max_pool2d", "Conv2d", "Dropout", "Linear", "MaxPool2d",
]
