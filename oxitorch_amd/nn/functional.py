"""Functional API of the hot path, same signatures as the reference
python/oxitorch/nn/functional.py:182-293.

Where the reference composes each F.* from several graph ops, this module
calls one fused device node (one kernel forward, one kernel backward), whose
values and gradients match the composition within the parity tolerances.
Inputs the fused nodes do not take (a weight that is not a (H,) vector,
for instance) fall back to the reference's composition of graph ops, still
on the device.
"""

from __future__ import annotations

import numpy as np

from .. import _native


def _native_from_numpy(arr, requires_grad=False):
    """Build a graph-connected tensor from a numpy array (default device)."""
    return _native.from_numpy(np.ascontiguousarray(arr, dtype=np.float32), requires_grad)


# ---- activations (functional.py:182-208) ---------------------------------------

def relu(x):
    return x.apply("relu")


def sigmoid(x):
    return x.apply("sigmoid")


def tanh(x):
    return x.apply("tanh")


def gelu(x, approximate="tanh"):
    """GELU. `approximate='tanh'` is the reference's F.gelu
    0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))); `'none'` is the exact
    0.5 x (1 + erf(x / sqrt 2)), which the reference does not have."""
    return _native.gelu(x, approximate)


def silu(x):
    """Sigmoid-weighted linear unit, elementwise: each value times its own
    logistic sigmoid. One device node with its VJP."""
    return _native.silu(x)


def leaky_relu(x, negative_slope=0.01):
    return x.apply("relu") + (x * float(negative_slope)).apply("neg").apply("relu").apply("neg")


# ---- softmax family (functional.py:211-222) -------------------------------------

def softmax(x, dim=-1):
    """Probabilities along `dim`: exponentials of x shifted by the largest
    value of its slice (so no exponential overflows), divided by their sum.
    One device node; the reference composes it from max, exp and sum nodes."""
    return _native.softmax(x, dim)


def log_softmax(x, dim=-1):
    """Log-probabilities along `dim`: x shifted by its slice maximum, minus the
    log of the shifted exponentials' sum. One device node."""
    return _native.log_softmax(x, dim)


# ---- normalization (functional.py:227-240) ----------------------------------------

def _is_vec(t, H):
    return t is not None and len(t.shape) == 1 and t.shape[0] == H


def layer_norm(x, weight, bias, eps=1e-5, vjp=None):
    """Normalizes each last-dim row to zero mean and unit variance (eps added
    to the variance), then scales by `weight` and shifts by `bias`.

    `vjp` selects the x-gradient: "ref" (default, or OXI_NORM_VJP) reproduces
    the reference graph, where `.apply("rsqrt")` detaches the inverse std;
    "exact" is the full derivative.

    When the output feeds only a gelu, silu, or last-dim softmax/log_softmax,
    backward runs both VJPs as one device pass (the same values, bit for bit;
    OXI_FUSE_NORM_ACT=0 turns it off)."""
    H = x.shape[-1]
    if _is_vec(weight, H) and _is_vec(bias, H):
        return _native.layer_norm(x, weight, bias, eps, vjp)
    mu = x.mean(-1, True)
    centered = x - mu
    var = (centered * centered).mean(-1, True)
    inv = (var + float(eps)).apply("rsqrt")
    return centered * inv * weight + bias


def rms_norm(x, weight, eps=1e-6, vjp=None):
    """Divides each last-dim row by its root mean square (eps added to the mean
    square) and scales by `weight`; `vjp` as in layer_norm."""
    if _is_vec(weight, x.shape[-1]):
        return _native.rms_norm(x, weight, eps, vjp)
    ms = (x * x).mean(-1, True)
    inv = (ms + float(eps)).apply("rsqrt")
    return x * inv * weight


# ---- embedding (functional.py:245-247) -----------------------------------------------

def embedding(indices, weight):
    """Rows of the `(num_embeddings, dim)` table `weight` picked by `indices`:
    a flat sequence of ints as the reference takes them, or a numpy integer
    array of any shape (read in C order)."""
    if isinstance(indices, np.ndarray):
        indices = indices.ravel()
    return _native.embedding(indices, weight)


# ---- losses (functional.py:270-293) -----------------------------------------------------

def mse_loss(pred, target):
    diff = pred - target
    return (diff * diff).mean()


def cross_entropy(logits, targets):
    """Mean cross-entropy; `targets` is a flat list of int class indices.

    Fused: the forward reads each row once (its log-sum-exp and picked
    log-probability, NaN where the reference's sum(onehot * log_softmax)
    is); when the logits require grad it also writes the gradient that
    backward() with its implicit seed of 1 hands them, and any other
    upstream gradient g runs one backward pass writing
    (softmax - onehot) * g / n. The argument checks mirror the reference's: a batch-size mismatch raises
    ValueError mentioning the targets, and class ids follow numpy indexing
    (negatives wrap, out-of-range raises IndexError)."""
    n, classes = logits.shape
    t = np.asarray(targets)
    if t.size and t.dtype.kind not in "iu":
        # the reference indexes its one-hot with them (functional.py:288-289)
        if isinstance(targets, np.ndarray):
            raise IndexError("arrays used as indices must be of integer (or boolean) type")
        raise IndexError("only integers, slices (`:`), ellipsis (`...`), numpy.newaxis (`None`) and integer or "
                         "boolean arrays are valid indices")
    t = t.astype(np.int64).ravel()
    if len(t) != n:
        raise ValueError(f"{len(t)} targets for batch of {n}")
    bad = (t >= classes) | (t < -classes)
    if bad.any():
        raise IndexError(f"index {int(t[bad][0])} is out of bounds for axis 1 with size {classes}")
    t = np.where(t < 0, t + classes, t)
    return _native.cross_entropy(logits, t)


def _outside(what):
    def op(*args, **kwargs):
        raise NotImplementedError(f"{what} is outside this build's device hot path")
    op.__name__ = what.split(" ")[0]
    op.__doc__ = f"The reference's {what}: not part of this build; raises NotImplementedError."
    return op


# The reference's GEMM, convolution, pooling and dropout entry points
# (functional.py:23-47,49-55,104-148,150-181,255-268) are outside the device
# hot path; calling one says so instead of failing on a missing name.
linear = _outside("linear (SGEMM)")
bmm = _outside("bmm (batched GEMM)")
conv2d = _outside("conv2d (im2col + GEMM)")
max_pool2d = _outside("max_pool2d")
dropout = _outside("dropout")
