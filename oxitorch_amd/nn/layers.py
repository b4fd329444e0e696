"""Module wrappers of the hot-path functions (python/oxitorch/nn/layers.py:94-196):
parameter initialisation follows the reference (norm weights one, biases
zero, embedding rows standard-normal * 0.05 from `default_rng(seed)`)."""

import numpy as np

from . import functional as F
from .module import Module, Parameter


class LayerNorm(Module):
    """F.layer_norm with its own weight (ones) and bias (zeros) of
    `normalized_shape`; `seed` is accepted for the reference's signature and
    unused (the initial values are constants)."""

    def __init__(self, normalized_shape, eps=1e-5, seed=None):
        self.eps = eps
        self.weight = Parameter(F._native_from_numpy(np.ones(normalized_shape, dtype=np.float32), True))
        self.bias = Parameter(F._native_from_numpy(np.zeros(normalized_shape, dtype=np.float32), True))

    def forward(self, x):
        return F.layer_norm(x, self.weight.tensor, self.bias.tensor, self.eps)


class RMSNorm(Module):
    """F.rms_norm with its own weight (ones) of `normalized_shape`; `seed`
    as in LayerNorm."""

    def __init__(self, normalized_shape, eps=1e-6, seed=None):
        self.eps = eps
        self.weight = Parameter(F._native_from_numpy(np.ones(normalized_shape, dtype=np.float32), True))

    def forward(self, x):
        return F.rms_norm(x, self.weight.tensor, self.eps)


class Embedding(Module):
    """F.embedding over its own (num_embeddings, embedding_dim) table, drawn
    as standard normals * 0.05 from default_rng(seed); forward takes a flat
    sequence of int ids."""

    def __init__(self, num_embeddings, embedding_dim, seed=None):
        rng = np.random.default_rng(seed)
        w = rng.standard_normal((num_embeddings, embedding_dim)) * 0.05
        self.weight = Parameter(F._native_from_numpy(w.astype(np.float32), True))
        self.num_embeddings = num_embeddings
        self.embedding_dim = embedding_dim

    def forward(self, indices):
        return F.embedding(indices, self.weight.tensor)


class _Activation(Module):
    """A parameterless module that applies one F.* activation."""

    def __init__(self, fn):
        self._fn = fn

    def forward(self, x):
        return self._fn(x)


def ReLU():
    return _Activation(F.relu)


def GELU(approximate="tanh"):
    return _Activation(lambda x: F.gelu(x, approximate))


def SiLU():
    return _Activation(F.silu)


def Tanh():
    return _Activation(F.tanh)


def Sigmoid():
    return _Activation(F.sigmoid)


def LeakyReLU(negative_slope=0.01):
    return _Activation(lambda x: F.leaky_relu(x, negative_slope))


def _outside_layer(name, what):
    def layer(*args, **kwargs):
        raise NotImplementedError(f"nn.{name} ({what}) is outside this build's device hot path")
    layer.__name__ = name
    return layer


# layers.py:20-92,134-164 of the reference: not part of this build
Linear = _outside_layer("Linear", "SGEMM")
Conv2d = _outside_layer("Conv2d", "im2col + GEMM")
MaxPool2d = _outside_layer("MaxPool2d", "window gather + max")
Dropout = _outside_layer("Dropout", "host RNG masks")


class Softmax(Module):
    """F.softmax along `dim`."""

    def __init__(self, dim=-1):
        self.dim = dim

    def forward(self, x):
        return F.softmax(x, self.dim)
