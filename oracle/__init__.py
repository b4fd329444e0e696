"""CPU oracle for the oxitorch layer-kernel hot path -- TEST INFRASTRUCTURE.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this package, and only as the checker (never as the measured or shipped path).
`oxitorch_amd` never imports it.

Two parts:
  * `ref` -- numpy wrappers over librefcpu.so, a plain-C restatement of the
    reference's CPU algorithms in f32 with the reference's rounding order
    (refcpu.c cites the reference file:line of each function);
  * `closed_form` -- float64 closed forms (the arbiter for long reductions
    and for the exact VJPs the reference lacks).

Parity status of every function is listed in `PINS` (filled by the tests in
tests/test_oracle.py, which check each function against the reference's
known-answer tests, the closed forms, finite differences and invariants).
"""

from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "librefcpu.so"

_f = ctypes.POINTER(ctypes.c_float)
_i64 = ctypes.POINTER(ctypes.c_int64)
_lib = None


def build() -> Path:
    """Compile refcpu.c with the committed Makefile."""
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB


def lib():
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        _lib = ctypes.CDLL(str(LIB))
    return _lib


def _fp(a: np.ndarray):
    assert a.dtype == np.float32 and a.flags.c_contiguous
    return a.ctypes.data_as(_f)


def _ip(a: np.ndarray):
    assert a.dtype == np.int64 and a.flags.c_contiguous
    return a.ctypes.data_as(_i64)


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


class ref:
    """f32 restatement of the reference CPU path (librefcpu.so)."""

    @staticmethod
    def rms_norm_fwd(x, w, eps=1e-6):
        x = _f32(x)
        w = _f32(w)
        H = x.shape[-1]
        rows = x.size // H if H else 0
        y = np.empty_like(x)
        inv = np.empty(rows, np.float32)
        lib().ref_rms_norm_fwd(_fp(x), _fp(w), _fp(y), _fp(inv), ctypes.c_int64(rows), ctypes.c_int64(H),
                               ctypes.c_float(eps))
        return y, inv

    @staticmethod
    def rms_norm_bwd(x, w, inv, g):
        x, w, inv, g = _f32(x), _f32(w), _f32(inv), _f32(g)
        H = x.shape[-1]
        lead = np.ascontiguousarray(x.shape[:-1], dtype=np.int64)
        dx = np.empty_like(x)
        dw = np.empty(H, np.float32)
        lib().ref_rms_norm_bwd(_fp(x), _fp(w), _fp(inv), _fp(g), _fp(dx), _fp(dw), _ip(lead),
                               ctypes.c_int(len(lead)), ctypes.c_int64(H))
        return dx, dw

    @staticmethod
    def layer_norm_fwd(x, w, b, eps=1e-5):
        x, w, b = _f32(x), _f32(w), _f32(b)
        H = x.shape[-1]
        rows = x.size // H if H else 0
        y = np.empty_like(x)
        mean = np.empty(rows, np.float32)
        inv = np.empty(rows, np.float32)
        lib().ref_layer_norm_fwd(_fp(x), _fp(w), _fp(b), _fp(y), _fp(mean), _fp(inv), ctypes.c_int64(rows),
                                 ctypes.c_int64(H), ctypes.c_float(eps))
        return y, mean, inv

    @staticmethod
    def layer_norm_bwd(x, w, mean, inv, g):
        x, w, mean, inv, g = map(_f32, (x, w, mean, inv, g))
        H = x.shape[-1]
        lead = np.ascontiguousarray(x.shape[:-1], dtype=np.int64)
        dx = np.empty_like(x)
        dw = np.empty(H, np.float32)
        db = np.empty(H, np.float32)
        lib().ref_layer_norm_bwd(_fp(x), _fp(w), _fp(mean), _fp(inv), _fp(g), _fp(dx), _fp(dw), _fp(db), _ip(lead),
                                 ctypes.c_int(len(lead)), ctypes.c_int64(H))
        return dx, dw, db

    @staticmethod
    def _map1(fn, x):
        x = _f32(x)
        y = np.empty_like(x)
        getattr(lib(), fn)(_fp(x), _fp(y), ctypes.c_int64(x.size))
        return y

    @staticmethod
    def _map2(fn, x, g):
        x, g = _f32(x), _f32(g)
        y = np.empty_like(x)
        getattr(lib(), fn)(_fp(x), _fp(g), _fp(y), ctypes.c_int64(x.size))
        return y

    @staticmethod
    def gelu_tanh_fwd(x):
        return ref._map1("ref_gelu_tanh_fwd", x)

    @staticmethod
    def gelu_tanh_bwd(x, g):
        return ref._map2("ref_gelu_tanh_bwd", x, g)

    @staticmethod
    def gelu_erf_fwd(x):
        return ref._map1("ref_gelu_erf_fwd", x)

    @staticmethod
    def gelu_erf_bwd(x, g):
        return ref._map2("ref_gelu_erf_bwd", x, g)

    @staticmethod
    def silu_fwd(x):
        return ref._map1("ref_silu_fwd", x)

    @staticmethod
    def silu_bwd(x, g):
        return ref._map2("ref_silu_bwd", x, g)

    @staticmethod
    def _oli(shape, dim):
        dim = dim % len(shape)
        outer = int(np.prod(shape[:dim], dtype=np.int64))
        inner = int(np.prod(shape[dim + 1:], dtype=np.int64))
        return outer, shape[dim], inner

    @staticmethod
    def softmax_fwd(x, dim=-1):
        x = _f32(x)
        o, l, i = ref._oli(x.shape, dim)
        y = np.empty_like(x)
        lib().ref_softmax_fwd(_fp(x), _fp(y), ctypes.c_int64(o), ctypes.c_int64(l), ctypes.c_int64(i))
        return y

    @staticmethod
    def softmax_bwd(x, g, dim=-1):
        x, g = _f32(x), _f32(g)
        o, l, i = ref._oli(x.shape, dim)
        dx = np.empty_like(x)
        lib().ref_softmax_bwd(_fp(x), _fp(g), _fp(dx), ctypes.c_int64(o), ctypes.c_int64(l), ctypes.c_int64(i))
        return dx

    @staticmethod
    def log_softmax_fwd(x, dim=-1):
        x = _f32(x)
        o, l, i = ref._oli(x.shape, dim)
        y = np.empty_like(x)
        lib().ref_log_softmax_fwd(_fp(x), _fp(y), ctypes.c_int64(o), ctypes.c_int64(l), ctypes.c_int64(i))
        return y

    @staticmethod
    def log_softmax_bwd(x, g, dim=-1):
        x, g = _f32(x), _f32(g)
        o, l, i = ref._oli(x.shape, dim)
        dx = np.empty_like(x)
        lib().ref_log_softmax_bwd(_fp(x), _fp(g), _fp(dx), ctypes.c_int64(o), ctypes.c_int64(l),
                                  ctypes.c_int64(i))
        return dx

    @staticmethod
    def cross_entropy_fwd(logits, targets):
        logits = _f32(logits)
        t = np.ascontiguousarray(targets, dtype=np.int64)
        n, c = logits.shape
        loss = np.zeros(1, np.float32)
        lib().ref_cross_entropy_fwd(_fp(logits), _ip(t), _fp(loss), ctypes.c_int64(n), ctypes.c_int64(c))
        return float(loss[0])

    @staticmethod
    def cross_entropy_bwd(logits, targets, gloss=1.0):
        logits = _f32(logits)
        t = np.ascontiguousarray(targets, dtype=np.int64)
        n, c = logits.shape
        d = np.empty_like(logits)
        lib().ref_cross_entropy_bwd(_fp(logits), _ip(t), ctypes.c_float(gloss), _fp(d), ctypes.c_int64(n),
                                    ctypes.c_int64(c))
        return d

    @staticmethod
    def index_select(src, dim, idx):
        src = _f32(src)
        idx = np.ascontiguousarray(idx, dtype=np.int64)
        o, l, i = ref._oli(src.shape, dim)
        shape = list(src.shape)
        shape[dim % src.ndim] = len(idx)
        out = np.empty(shape, np.float32)
        rc = lib().ref_index_select(_fp(src), ctypes.c_int64(o), ctypes.c_int64(l), ctypes.c_int64(i), _ip(idx),
                                    ctypes.c_int64(len(idx)), _fp(out))
        if rc:
            raise IndexError("index out of range")
        return out

    @staticmethod
    def index_select_bwd(g, full_shape, dim, idx):
        g = _f32(g)
        idx = np.ascontiguousarray(idx, dtype=np.int64)
        o, l, i = ref._oli(tuple(full_shape), dim)
        grad = np.empty(full_shape, np.float32)
        lib().ref_index_select_bwd(_fp(g), ctypes.c_int64(o), ctypes.c_int64(l), ctypes.c_int64(i), _ip(idx),
                                   ctypes.c_int64(len(idx)), _fp(grad))
        return grad

    KINDS = {"sum": 0, "mean": 1, "max": 2, "min": 3, "argmax": 4, "argmin": 5, "norm": 6}

    @staticmethod
    def reduce(kind, x, dim):
        x = _f32(x)
        dim = dim % x.ndim
        shape = np.ascontiguousarray(x.shape, dtype=np.int64)
        out = np.empty(x.shape[:dim] + x.shape[dim + 1:], np.float32)
        rc = lib().ref_reduce(ctypes.c_int(ref.KINDS[kind]), _fp(x), _ip(shape), ctypes.c_int(x.ndim),
                              ctypes.c_int(dim), _fp(out))
        if rc:
            raise ValueError("cannot reduce over a zero-length dim")
        return out

    UNARY = ["neg", "abs", "sqrt", "rsqrt", "exp", "log", "log2", "log10", "sin", "cos", "tanh", "relu",
             "sigmoid", "floor", "ceil", "round", "sign", "square", "reciprocal"]
    BINARY = ["add", "sub", "mul", "div", "pow", "min", "max", "eq", "ne", "lt", "le", "gt", "ge"]

    @staticmethod
    def unary(name, x):
        x = _f32(x)
        y = np.empty_like(x)
        lib().ref_unary(ctypes.c_int(ref.UNARY.index(name)), _fp(x), _fp(y), ctypes.c_int64(x.size))
        return y

    @staticmethod
    def binary(name, a, b):
        a, b = _f32(a), _f32(b)
        shape = np.broadcast_shapes(a.shape, b.shape)
        av = np.broadcast_to(a, shape)
        bv = np.broadcast_to(b, shape)
        as_ = np.ascontiguousarray([s // 4 for s in av.strides], dtype=np.int64)
        bs_ = np.ascontiguousarray([s // 4 for s in bv.strides], dtype=np.int64)
        y = np.empty(shape, np.float32)
        shp = np.ascontiguousarray(shape, dtype=np.int64)
        lib().ref_binary(ctypes.c_int(ref.BINARY.index(name)), _fp(a), _ip(as_), _fp(b), _ip(bs_), _fp(y),
                         _ip(shp), ctypes.c_int(len(shape)))
        return y


    @staticmethod
    def scatter_dim0(base, idx, values):
        """Tensor::scatter_dim0: rows idx[p] of `base` replaced by values[p]
        in order (last write wins)."""
        base, values = _f32(base), _f32(values)
        idx = np.ascontiguousarray(idx, dtype=np.int64)
        rows = base.shape[0]
        inner = int(np.prod(base.shape[1:], dtype=np.int64))
        out = np.empty_like(base)
        rc = lib().ref_scatter_dim0(_fp(base), ctypes.c_int64(rows), ctypes.c_int64(inner), _ip(idx),
                                    ctypes.c_int64(len(idx)), _fp(values), _fp(out))
        if rc:
            raise IndexError("index out of range")
        return out

    @staticmethod
    def scatter_dim0_bwd(g, idx, n_values_shape):
        """(gbase, gvalues) of scatter_dim0 for upstream g (base's shape)."""
        g = _f32(g)
        idx = np.ascontiguousarray(idx, dtype=np.int64)
        rows = g.shape[0]
        inner = int(np.prod(g.shape[1:], dtype=np.int64))
        gb = np.empty_like(g)
        gv = np.empty(n_values_shape, np.float32)
        lib().ref_scatter_dim0_bwd(_fp(g), ctypes.c_int64(rows), ctypes.c_int64(inner), _ip(idx),
                                   ctypes.c_int64(len(idx)), _fp(gb), _fp(gv))
        return gb, gv

    @staticmethod
    def _bcast_elem_strides(a, shape):
        v = np.broadcast_to(a, shape)
        return np.ascontiguousarray([s // 4 for s in v.strides], dtype=np.int64)

    @staticmethod
    def _rm_bcast_strides(own_shape, shape):
        """Row-major strides of `own_shape`, expanded to `shape` with 0 on
        broadcast (size-1 or missing) dims (aops::masked_select's flat strides)."""
        rm = [1] * len(own_shape)
        for d in range(len(own_shape) - 2, -1, -1):
            rm[d] = rm[d + 1] * own_shape[d + 1]
        off = len(shape) - len(own_shape)
        out = [0 if d < off or own_shape[d - off] == 1 else rm[d - off] for d in range(len(shape))]
        return np.ascontiguousarray(out, dtype=np.int64)

    @staticmethod
    def masked_select(x, mask):
        """Tensor::masked_select over the broadcast of x and mask."""
        x, mask = _f32(x), _f32(mask)
        shape = np.broadcast_shapes(x.shape, mask.shape)
        n = int(np.prod(shape, dtype=np.int64))
        out = np.empty(max(n, 1), np.float32)
        lib().ref_masked_select.restype = ctypes.c_int64
        cnt = lib().ref_masked_select(_fp(x), _ip(ref._bcast_elem_strides(x, shape)), _fp(mask),
                                      _ip(ref._bcast_elem_strides(mask, shape)),
                                      _ip(np.ascontiguousarray(shape, dtype=np.int64)), ctypes.c_int(len(shape)),
                                      _fp(out))
        return out[:cnt].copy()

    @staticmethod
    def masked_select_bwd(x_shape, mask, g):
        """Gradient of x for masked_select(x, mask) with upstream g."""
        mask, g = _f32(mask), _f32(g)
        x_shape = tuple(x_shape)
        shape = np.broadcast_shapes(x_shape, mask.shape)
        gx = np.empty(x_shape, np.float32)
        lib().ref_masked_select_bwd(_fp(mask), _ip(ref._rm_bcast_strides(mask.shape, shape)),
                                    _ip(np.ascontiguousarray(shape, dtype=np.int64)), ctypes.c_int(len(shape)),
                                    _fp(g), _fp(gx), _ip(ref._rm_bcast_strides(x_shape, shape)),
                                    ctypes.c_int64(gx.size))
        return gx

    @staticmethod
    def sgd_step(p, g, buf, lr, momentum=0.0, nesterov=False):
        """One Sgd step; `buf` (momentum state, updated in place) may be None
        when momentum == 0. Returns the new parameter values."""
        p, g = _f32(p), _f32(g)
        out = np.empty_like(p)
        bp = _fp(buf) if buf is not None else None
        lib().ref_sgd_step(_fp(p), _fp(g), bp, _fp(out), ctypes.c_int64(p.size), ctypes.c_float(lr),
                           ctypes.c_float(momentum), ctypes.c_int(int(nesterov)))
        return out

    @staticmethod
    def adamw_step(p, g, m, v, t, lr, beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=1e-2, decoupled=True):
        """One AdamW/Adam step at per-parameter step t (m, v updated in place).
        Returns the new parameter values."""
        p, g = _f32(p), _f32(g)
        out = np.empty_like(p)
        lib().ref_adamw_step(_fp(p), _fp(g), _fp(m), _fp(v), _fp(out), ctypes.c_int64(p.size), ctypes.c_float(lr),
                             ctypes.c_float(beta1), ctypes.c_float(beta2), ctypes.c_float(eps),
                             ctypes.c_float(weight_decay), ctypes.c_int(int(decoupled)), ctypes.c_int64(t))
        return out


from . import closed_form  # noqa: E402  (float64 arbiter)

__all__ = ["ref", "closed_form", "build", "lib"]
