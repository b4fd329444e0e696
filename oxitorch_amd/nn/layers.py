"""Module wrappers of the hot-path functions (python/oxitorch/nn/layers.py:94-196):
parameter initialisation follows the reference (norm weights one, biases
zero, embedding rows standard-normal * 0.05 from `default_rng(seed)`)."""

import numpy as np

from . import functional as F
from .module import Module, Parameter


class LayerNorm(Module):
    """LayerNorm over the last dim with learned affine."""

    def __init__(self, normalized_shape, eps=1e-5, seed=None):
        self.eps = eps
        self.weight = Parameter(F._native_from_numpy(np.ones(normalized_shape, dtype=np.float32), True))
        self.bias = Parameter(F._native_from_numpy(np.zeros(normalized_shape, dtype=np.float32), True))

    def forward(self, x):
        return F.layer_norm(x, self.weight.tensor, self.bias.tensor, self.eps)


class RMSNorm(Module):
    """RMSNorm over the last dim (scale only)."""

    def __init__(self, normalized_shape, eps=1e-6, seed=None):
        self.eps = eps
        self.weight = Parameter(F._native_from_numpy(np.ones(normalized_shape, dtype=np.float32), True))

    def forward(self, x):
        return F.rms_norm(x, self.weight.tensor, self.eps)


class Embedding(Module):
    """Lookup table: rows of `weight` selected by integer indices."""

    def __init__(self, num_embeddings, embedding_dim, seed=None):
        rng = np.random.default_rng(seed)
        w = rng.standard_normal((num_embeddings, embedding_dim)) * 0.05
        self.weight = Parameter(F._native_from_numpy(w.astype(np.float32), True))
        self.num_embeddings = num_embeddings
        self.embedding_dim = embedding_dim

    def forward(self, indices):
        return F.embedding(indices, self.weight.tensor)


class _Activation(Module):
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


class Softmax(Module):
    def __init__(self, dim=-1):
        self.dim = dim

    def forward(self, x):
        return F.softmax(x, self.dim)
