"""Float64 closed forms for the hot-path functions -- TEST INFRASTRUCTURE.

These are the textbook formulas, evaluated in float64. They arbitrate where
the reference's own sequential-f32 rounding is larger than the parity
tolerance (long column sums, heavy embedding segments), define the exact
norm VJPs and exact-erf GELU that the reference does not have, and pin the
f32 restatement in refcpu.c.
"""

from __future__ import annotations

import numpy as np
from scipy.special import erf

SQRT_2_OVER_PI = np.sqrt(2.0 / np.pi)


def _d(a):
    return np.asarray(a, dtype=np.float64)


# ---- norms -------------------------------------------------------------------

def rms_norm_fwd(x, w, eps=1e-6):
    x = _d(x)
    inv = 1.0 / np.sqrt((x * x).mean(-1, keepdims=True) + eps)
    return x * inv * _d(w), inv[..., 0]


def rms_norm_bwd_exact(x, w, g, eps=1e-6):
    """Full derivative of y = x*inv*w with inv = (mean(x^2)+eps)^-1/2."""
    x, w, g = _d(x), _d(w), _d(g)
    H = x.shape[-1]
    inv = 1.0 / np.sqrt((x * x).mean(-1, keepdims=True) + eps)
    xh = x * inv
    gw = g * w
    dx = inv * (gw - xh * (gw * xh).sum(-1, keepdims=True) / H)
    dw = (g * xh).reshape(-1, H).sum(0)
    return dx, dw


def rms_norm_bwd_refgraph(x, w, g, eps=1e-6):
    """The reference graph's VJP (inv detached) in float64: dx = g*w*inv."""
    x, w, g = _d(x), _d(w), _d(g)
    H = x.shape[-1]
    inv = 1.0 / np.sqrt((x * x).mean(-1, keepdims=True) + eps)
    return g * w * inv, (g * x * inv).reshape(-1, H).sum(0)


def layer_norm_fwd(x, w, b, eps=1e-5):
    x = _d(x)
    mu = x.mean(-1, keepdims=True)
    var = ((x - mu) ** 2).mean(-1, keepdims=True)
    inv = 1.0 / np.sqrt(var + eps)
    return (x - mu) * inv * _d(w) + _d(b), mu[..., 0], inv[..., 0]


def layer_norm_bwd_exact(x, w, g, eps=1e-5):
    x, w, g = _d(x), _d(w), _d(g)
    H = x.shape[-1]
    mu = x.mean(-1, keepdims=True)
    inv = 1.0 / np.sqrt(((x - mu) ** 2).mean(-1, keepdims=True) + eps)
    xh = (x - mu) * inv
    gw = g * w
    dx = inv * (gw - gw.mean(-1, keepdims=True) - xh * (gw * xh).mean(-1, keepdims=True))
    return dx, (g * xh).reshape(-1, H).sum(0), g.reshape(-1, H).sum(0)


def layer_norm_bwd_refgraph(x, w, g, eps=1e-5):
    """Reference graph VJP (inv detached): dx = inv*gw - mean(inv*gw)."""
    x, w, g = _d(x), _d(w), _d(g)
    H = x.shape[-1]
    mu = x.mean(-1, keepdims=True)
    inv = 1.0 / np.sqrt(((x - mu) ** 2).mean(-1, keepdims=True) + eps)
    gc = g * w * inv
    dx = gc - gc.mean(-1, keepdims=True)
    return dx, (g * (x - mu) * inv).reshape(-1, H).sum(0), g.reshape(-1, H).sum(0)


# ---- activations -------------------------------------------------------------

def gelu_tanh(x):
    x = _d(x)
    return 0.5 * x * (1.0 + np.tanh(SQRT_2_OVER_PI * (x + 0.044715 * x ** 3)))


def gelu_tanh_grad(x):
    x = _d(x)
    u = SQRT_2_OVER_PI * (x + 0.044715 * x ** 3)
    t = np.tanh(u)
    du = SQRT_2_OVER_PI * (1.0 + 3 * 0.044715 * x * x)
    return 0.5 * (1.0 + t) + 0.5 * x * (1.0 - t * t) * du


def gelu_erf(x):
    x = _d(x)
    return 0.5 * x * (1.0 + erf(x / np.sqrt(2.0)))


def gelu_erf_grad(x):
    x = _d(x)
    return 0.5 * (1.0 + erf(x / np.sqrt(2.0))) + x * np.exp(-0.5 * x * x) / np.sqrt(2.0 * np.pi)


def silu(x):
    x = _d(x)
    return x / (1.0 + np.exp(-x))


def silu_grad(x):
    x = _d(x)
    s = 1.0 / (1.0 + np.exp(-x))
    return s + x * s * (1.0 - s)


# ---- softmax family ------------------------------------------------------------

def softmax(x, dim=-1):
    x = _d(x)
    z = x - x.max(dim, keepdims=True)
    e = np.exp(z)
    return e / e.sum(dim, keepdims=True)


def log_softmax(x, dim=-1):
    x = _d(x)
    z = x - x.max(dim, keepdims=True)
    return z - np.log(np.exp(z).sum(dim, keepdims=True))


def softmax_bwd(x, g, dim=-1):
    y = softmax(x, dim)
    g = _d(g)
    return y * (g - (g * y).sum(dim, keepdims=True))


def log_softmax_bwd(x, g, dim=-1):
    g = _d(g)
    return g - softmax(x, dim) * g.sum(dim, keepdims=True)


def cross_entropy(logits, targets):
    ls = log_softmax(logits, -1)
    t = np.asarray(targets, dtype=np.int64)
    return float(-ls[np.arange(len(t)), t].mean())


def cross_entropy_grad(logits, targets, gloss=1.0):
    p = softmax(logits, -1)
    t = np.asarray(targets, dtype=np.int64)
    p[np.arange(len(t)), t] -= 1.0
    return p * (gloss / len(t))


# ---- embedding -----------------------------------------------------------------

def embedding_grad(g, ids, V):
    """dW[v] = sum over positions p with ids[p] == v of g[p], in float64."""
    g = _d(g).reshape(len(ids), -1)
    dW = np.zeros((V, g.shape[1]), np.float64)
    np.add.at(dW, np.asarray(ids, dtype=np.int64), g)
    return dW
