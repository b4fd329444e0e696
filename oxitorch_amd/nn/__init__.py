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
from .layers import GELU, Embedding, LayerNorm, ReLU, RMSNorm, SiLU, Sigmoid, Softmax, Tanh

__all__ = [
    "Module", "Parameter", "Sequential", "functional", "cross_entropy", "embedding", "gelu", "layer_norm",
    "leaky_relu", "log_softmax", "mse_loss", "relu", "rms_norm", "sigmoid", "silu", "softmax", "tanh",
    "GELU", "Embedding", "LayerNorm", "ReLU", "RMSNorm", "SiLU", "Sigmoid", "Softmax", "Tanh",
]
