"""ctypes binding of liboxihip's C-ABI (include/oxihip.h).

This is the thin Python-side FFI a host binds to reach the MI355X kernels:
`DeviceArray` owns an HBM buffer from the library's caching allocator, and
each launcher takes DeviceArrays and plain sizes. Status codes are mapped to
exceptions exactly as the reference maps OxitorchError variants
(crates/oxi-bindings/src/error.rs:22-32): invalid argument / shape mismatch ->
ValueError, not implemented -> NotImplementedError, out of bounds / other ->
RuntimeError, each carrying the library's message.

There is no CPU fallback: if liboxihip.so is missing, importing this module
raises.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
LIB_PATH = Path(os.environ.get("OXIHIP_LIB", _HERE / "liboxihip.so"))

if not LIB_PATH.exists():
    raise ImportError(
        f"liboxihip.so not found at {LIB_PATH}: build it with `python -m oxitorch_amd.build lib` "
        "(the device path has no CPU fallback)"
    )

lib = ctypes.CDLL(str(LIB_PATH))

c_i64 = ctypes.c_int64
c_int = ctypes.c_int
c_float = ctypes.c_float
c_size = ctypes.c_size_t
vp = ctypes.c_void_p
P_i64 = ctypes.POINTER(ctypes.c_int64)

# status codes (oxi_status)
OK, INVALID_ARGUMENT, SHAPE_MISMATCH, NOT_IMPLEMENTED, OUT_OF_BOUNDS, OTHER = range(6)

UNARY = ["neg", "abs", "sqrt", "rsqrt", "exp", "log", "log2", "log10", "sin", "cos", "tanh", "relu", "sigmoid",
         "floor", "ceil", "round", "sign", "square", "reciprocal", "identity"]
BINARY = ["add", "sub", "mul", "div", "pow", "min", "max", "eq", "ne", "lt", "le", "gt", "ge"]
REDUCE = ["sum", "mean", "max", "min", "argmax", "argmin", "norm"]
NORM_VJP = {"ref": 0, "exact": 1}
GELU = {"tanh": 0, "none": 1, "erf": 1}
ACT = {"none": -1, "gelu_tanh": 0, "gelu_erf": 1, "silu": 2, "softmax": 3, "log_softmax": 4}

_SIGS = {
    "oxi_hip_init": [c_int],
    "oxi_hip_device_count": [ctypes.POINTER(c_int)],
    "oxi_hip_current_device": [ctypes.POINTER(c_int)],
    "oxi_hip_default_device": [ctypes.POINTER(c_int)],
    "oxi_hip_alloc": [c_size, ctypes.POINTER(vp)],
    "oxi_hip_free": [vp],
    "oxi_hip_empty_cache": [],
    "oxi_hip_memory_stats": [ctypes.POINTER(c_size), ctypes.POINTER(c_size)],
    "oxi_hip_memcpy_h2d": [vp, vp, c_size],
    "oxi_hip_memcpy_d2h": [vp, vp, c_size],
    "oxi_hip_memcpy_d2d": [vp, vp, c_size],
    "oxi_hip_host_alloc": [c_size, ctypes.POINTER(vp)],
    "oxi_hip_host_free": [vp],
    "oxi_hip_upload": [vp, vp, c_size],
    "oxi_hip_memcpy_h2d_async": [vp, vp, c_size],
    "oxi_hip_download": [vp, vp, c_size],
    "oxi_hip_sync": [],
    "oxi_hip_stream": [ctypes.POINTER(vp)],
    "oxi_hip_event_create": [ctypes.POINTER(vp)],
    "oxi_hip_event_record": [vp],
    "oxi_hip_event_elapsed_ms": [vp, vp, ctypes.POINTER(c_float)],
    "oxi_hip_event_destroy": [vp],
    "oxi_hip_debug_fail_alloc_after": [c_int],
    "oxi_hip_device_props": [vp],
    "oxi_fill": [vp, c_i64, c_float],
    "oxi_unary": [c_int, vp, P_i64, vp, P_i64, P_i64, c_int],
    "oxi_binary": [c_int, vp, P_i64, vp, P_i64, vp, P_i64, P_i64, c_int],
    "oxi_gelu_fwd": [vp, P_i64, vp, P_i64, P_i64, c_int, c_int],
    "oxi_gelu_bwd": [vp, P_i64, vp, P_i64, vp, P_i64, P_i64, c_int, c_int],
    "oxi_silu_fwd": [vp, P_i64, vp, P_i64, P_i64, c_int],
    "oxi_silu_bwd": [vp, P_i64, vp, P_i64, vp, P_i64, P_i64, c_int],
    "oxi_rms_norm_fwd": [vp, vp, vp, vp, c_i64, c_i64, c_float],
    "oxi_rms_norm_bwd": [vp, vp, vp, vp, vp, vp, c_i64, c_i64, c_int],
    "oxi_layer_norm_fwd": [vp, vp, vp, vp, vp, vp, c_i64, c_i64, c_float],
    "oxi_layer_norm_bwd": [vp, vp, vp, vp, vp, vp, vp, vp, c_i64, c_i64, c_int],
    "oxi_layer_norm_bwd_noalloc": [vp, vp, vp, vp, vp, vp, vp, vp, c_i64, c_i64, c_int],
    "oxi_rms_norm_act_bwd": [vp, vp, vp, vp, c_int, vp, vp, vp, c_i64, c_i64, c_int],
    "oxi_layer_norm_act_bwd": [vp, vp, vp, vp, vp, vp, c_int, vp, vp, vp, vp, c_i64, c_i64, c_int],
    "oxi_rms_norm_bwd_lead_sum": [vp, vp, vp, vp, c_int, vp, vp, vp, vp, c_i64, c_i64, c_i64, c_int],
    "oxi_layer_norm_bwd_lead_sum": [vp, vp, vp, vp, vp, vp, c_int, vp, vp, vp, vp, vp, c_i64, c_i64, c_i64, c_int],
    "oxi_softmax_fwd": [vp, vp, c_i64, c_i64, c_i64],
    "oxi_softmax_bwd": [vp, vp, vp, c_i64, c_i64, c_i64],
    "oxi_log_softmax_fwd": [vp, vp, c_i64, c_i64, c_i64],
    "oxi_log_softmax_bwd": [vp, vp, vp, c_i64, c_i64, c_i64],
    "oxi_cross_entropy_fwd": [vp, vp, vp, vp, c_i64, c_i64],
    "oxi_cross_entropy_bwd": [vp, vp, vp, vp, vp, c_i64, c_i64],
    "oxi_cross_entropy_fwd_grad": [vp, vp, vp, vp, vp, c_i64, c_i64],
    "oxi_index_select": [vp, c_i64, c_i64, c_i64, vp, c_i64, vp],
    "oxi_batch_gather": [vp, c_int, c_i64, vp, c_i64],
    "oxi_index_select_bwd": [vp, c_i64, c_i64, c_i64, vp, c_i64, vp],
    "oxi_index_select_bwd_plan": [vp, c_i64, c_i64, ctypes.POINTER(vp)],
    "oxi_index_select_bwd_apply": [vp, vp, c_i64, c_i64, vp],
    "oxi_index_select_bwd_plan_free": [vp],
    "oxi_embedding_fwd": [vp, vp, c_i64, c_i64, c_i64, vp],
    "oxi_embedding_bwd": [vp, vp, c_i64, c_i64, c_i64, vp],
    "oxi_reduce": [c_int, vp, P_i64, P_i64, c_int, c_int, vp],
    "oxi_scatter_rows": [vp, c_i64, c_i64, vp, c_i64, vp, vp],
    "oxi_scatter_rows_bwd": [vp, c_i64, c_i64, vp, c_i64, vp, vp],
    "oxi_masked_select": [vp, P_i64, vp, P_i64, P_i64, c_int, ctypes.POINTER(vp), ctypes.POINTER(c_i64), vp],
    "oxi_masked_select_record_bytes": [P_i64, c_int, ctypes.POINTER(c_i64)],
    "oxi_masked_select_bwd": [vp, P_i64, c_int, vp, c_i64, vp, P_i64, c_i64],
    "oxi_sgd_step": [vp, vp, vp, vp, c_i64, c_float, c_float, c_int],
    "oxi_adamw_step": [vp, vp, vp, vp, vp, c_i64, c_float, c_float, c_float, c_float, c_float, c_int, c_i64],
    "oxi_sgd_step_multi": [vp, c_int, c_float, c_float, c_int],
    "oxi_adamw_step_multi": [vp, c_int, c_float, c_float, c_float, c_float, c_float, c_int],
}

for _name, _args in _SIGS.items():
    _fn = getattr(lib, _name)
    _fn.argtypes = _args
    _fn.restype = c_int
lib.oxi_hip_last_error.argtypes = []
lib.oxi_hip_last_error.restype = ctypes.c_char_p

DECLARED = sorted(list(_SIGS) + ["oxi_hip_last_error"])


class OxiError(RuntimeError):
    pass


def last_error() -> str:
    return lib.oxi_hip_last_error().decode("utf-8", "replace")


def check(rc: int) -> None:
    if rc == OK:
        return
    msg = last_error()
    if rc in (INVALID_ARGUMENT, SHAPE_MISMATCH):
        raise ValueError(msg)
    if rc == NOT_IMPLEMENTED:
        raise NotImplementedError(msg)
    raise RuntimeError(msg)


def call(name: str, *args) -> None:
    check(getattr(lib, name)(*args))


def device_count() -> int:
    n = c_int(0)
    check(lib.oxi_hip_device_count(ctypes.byref(n)))
    return n.value


def init(device: int = 0) -> None:
    check(lib.oxi_hip_init(device))


def sync() -> None:
    check(lib.oxi_hip_sync())


def memory_stats() -> tuple[int, int]:
    a, b = c_size(0), c_size(0)
    check(lib.oxi_hip_memory_stats(ctypes.byref(a), ctypes.byref(b)))
    return a.value, b.value


def _i64arr(vals) -> ctypes.Array:
    vals = [int(v) for v in vals]
    return (ctypes.c_int64 * max(1, len(vals)))(*vals)


class DeviceArray:
    """An HBM buffer of fp32 or int64 elements with a shape (row-major)."""

    __slots__ = ("ptr", "shape", "dtype", "nbytes", "__weakref__")

    def __init__(self, shape, dtype=np.float32):
        self.shape = tuple(int(s) for s in shape)
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape, dtype=np.int64)) * self.dtype.itemsize
        p = vp()
        check(lib.oxi_hip_alloc(self.nbytes, ctypes.byref(p)))
        self.ptr = p.value

    @classmethod
    def adopt(cls, ptr, shape, dtype=np.float32) -> "DeviceArray":
        """Wraps a block that liboxihip allocated (freed with oxi_hip_free)."""
        d = cls.__new__(cls)
        d.shape = tuple(int(s) for s in shape)
        d.dtype = np.dtype(dtype)
        d.nbytes = int(np.prod(d.shape, dtype=np.int64)) * d.dtype.itemsize
        d.ptr = ptr
        return d

    @classmethod
    def from_numpy(cls, a: np.ndarray) -> "DeviceArray":
        a = np.ascontiguousarray(a)
        d = cls(a.shape, a.dtype)
        if d.nbytes:
            check(lib.oxi_hip_memcpy_h2d(d.ptr, a.ctypes.data, d.nbytes))
        return d

    def numpy(self) -> np.ndarray:
        out = np.empty(self.shape, self.dtype)
        if self.nbytes:
            check(lib.oxi_hip_memcpy_d2h(out.ctypes.data, self.ptr, self.nbytes))
        return out

    @property
    def size(self) -> int:
        return int(np.prod(self.shape, dtype=np.int64))

    def free(self) -> None:
        if self.ptr:
            lib.oxi_hip_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class DeviceProps(ctypes.Structure):
    """oxi_device_props"""
    _fields_ = [("compute_units", ctypes.c_int32), ("memory_clock_khz", ctypes.c_int32),
                ("memory_bus_bits", ctypes.c_int32), ("l2_bytes", ctypes.c_int32), ("hbm_bytes", ctypes.c_int64),
                ("arch", ctypes.c_char * 64)]


def device_props() -> dict:
    p = DeviceProps()
    call("oxi_hip_device_props", ctypes.byref(p))
    return {"compute_units": p.compute_units, "memory_clock_khz": p.memory_clock_khz,
            "memory_bus_bits": p.memory_bus_bits, "l2_bytes": p.l2_bytes, "hbm_bytes": p.hbm_bytes,
            "arch": p.arch.decode()}


def row_major_strides(shape):
    st = [1] * len(shape)
    for d in range(len(shape) - 2, -1, -1):
        st[d] = st[d + 1] * shape[d + 1]
    return st


# ---- launchers (DeviceArray in, DeviceArray out) -----------------------------

def unary(name: str, x: DeviceArray, out: DeviceArray | None = None, x_strides=None, shape=None) -> DeviceArray:
    shape = tuple(shape or x.shape)
    out = out or DeviceArray(shape)
    xs = x_strides or row_major_strides(shape)
    call("oxi_unary", UNARY.index(name), x.ptr, _i64arr(xs), out.ptr, _i64arr(row_major_strides(shape)),
         _i64arr(shape), len(shape))
    return out


def binary(name: str, a: DeviceArray, b: DeviceArray, a_strides, b_strides, shape,
           out: DeviceArray | None = None) -> DeviceArray:
    shape = tuple(shape)
    out = out or DeviceArray(shape)
    call("oxi_binary", BINARY.index(name), a.ptr, _i64arr(a_strides), b.ptr, _i64arr(b_strides), out.ptr,
         _i64arr(row_major_strides(shape)), _i64arr(shape), len(shape))
    return out


def gelu_fwd(x: DeviceArray, approximate="tanh", out=None, x_strides=None, shape=None) -> DeviceArray:
    shape = tuple(shape or x.shape)
    out = out or DeviceArray(shape)
    call("oxi_gelu_fwd", x.ptr, _i64arr(x_strides or row_major_strides(shape)), out.ptr,
         _i64arr(row_major_strides(shape)), _i64arr(shape), len(shape), GELU[approximate])
    return out


def gelu_bwd(x: DeviceArray, g: DeviceArray, approximate="tanh", out=None, x_strides=None, g_strides=None,
             shape=None) -> DeviceArray:
    shape = tuple(shape or x.shape)
    out = out or DeviceArray(shape)
    rm = row_major_strides(shape)
    call("oxi_gelu_bwd", x.ptr, _i64arr(x_strides or rm), g.ptr, _i64arr(g_strides or rm), out.ptr, _i64arr(rm),
         _i64arr(shape), len(shape), GELU[approximate])
    return out


def silu_fwd(x: DeviceArray, out=None, x_strides=None, shape=None) -> DeviceArray:
    shape = tuple(shape or x.shape)
    out = out or DeviceArray(shape)
    rm = row_major_strides(shape)
    call("oxi_silu_fwd", x.ptr, _i64arr(x_strides or rm), out.ptr, _i64arr(rm), _i64arr(shape), len(shape))
    return out


def silu_bwd(x: DeviceArray, g: DeviceArray, out=None, x_strides=None, g_strides=None, shape=None) -> DeviceArray:
    shape = tuple(shape or x.shape)
    out = out or DeviceArray(shape)
    rm = row_major_strides(shape)
    call("oxi_silu_bwd", x.ptr, _i64arr(x_strides or rm), g.ptr, _i64arr(g_strides or rm), out.ptr, _i64arr(rm),
         _i64arr(shape), len(shape))
    return out


def _rows(x: DeviceArray):
    H = x.shape[-1] if x.shape else 1
    return (x.size // H if H else 0), H


def rms_norm_fwd(x: DeviceArray, w: DeviceArray, eps=1e-6):
    rows, H = _rows(x)
    y = DeviceArray(x.shape)
    rstd = DeviceArray((rows,))
    call("oxi_rms_norm_fwd", x.ptr, w.ptr, y.ptr, rstd.ptr, rows, H, eps)
    return y, rstd


def rms_norm_bwd(x, w, rstd, g, mode="ref", need_dx=True, need_dw=True):
    rows, H = _rows(x)
    dx = DeviceArray(x.shape) if need_dx else None
    dw = DeviceArray((H,)) if need_dw else None
    call("oxi_rms_norm_bwd", x.ptr, w.ptr, rstd.ptr, g.ptr, dx.ptr if dx else None, dw.ptr if dw else None, rows, H,
         NORM_VJP[mode])
    return dx, dw


def layer_norm_fwd(x: DeviceArray, w: DeviceArray | None, b: DeviceArray | None, eps=1e-5):
    rows, H = _rows(x)
    y = DeviceArray(x.shape)
    mean = DeviceArray((rows,))
    rstd = DeviceArray((rows,))
    call("oxi_layer_norm_fwd", x.ptr, w.ptr if w else None, b.ptr if b else None, y.ptr, mean.ptr, rstd.ptr, rows,
         H, eps)
    return y, mean, rstd


def layer_norm_bwd(x, w, mean, rstd, g, mode="ref", need_dx=True, need_dw=True, need_db=True):
    rows, H = _rows(x)
    dx = DeviceArray(x.shape) if need_dx else None
    dw = DeviceArray((H,)) if need_dw else None
    db = DeviceArray((H,)) if need_db else None
    call("oxi_layer_norm_bwd", x.ptr, w.ptr if w else None, mean.ptr, rstd.ptr, g.ptr, dx.ptr if dx else None,
         dw.ptr if dw else None, db.ptr if db else None, rows, H, NORM_VJP[mode])
    return dx, dw, db


def rms_norm_bwd_lead_sum(x, w, rstd, g, lead, act="none", mode="ref", need_dy=True, need_dw=True):
    """The rms VJP (or rms + act VJP) over (lead, T) rows that also sums dx
    over the leading dim; returns (dy, dx, dw, dx_sum)."""
    rows, H = _rows(x)
    dy = DeviceArray(x.shape) if need_dy and act != "none" else None
    dx = DeviceArray(x.shape)
    dw = DeviceArray((H,)) if need_dw else None
    ds = DeviceArray((rows // lead, H))
    call("oxi_rms_norm_bwd_lead_sum", x.ptr, w.ptr if w else None, rstd.ptr, g.ptr, ACT[act], dy.ptr if dy else None,
         dx.ptr, dw.ptr if dw else None, ds.ptr, lead, rows, H, NORM_VJP[mode])
    return dy, dx, dw, ds


def layer_norm_bwd_lead_sum(x, w, b, mean, rstd, g, lead, act="none", mode="ref", need_dy=True, need_dw=True,
                            need_db=True):
    """The layer_norm VJP (or layer_norm + act VJP) over (lead, T) rows that
    also sums dx over the leading dim; returns (dy, dx, dw, db, dx_sum)."""
    rows, H = _rows(x)
    dy = DeviceArray(x.shape) if need_dy and act != "none" else None
    dx = DeviceArray(x.shape)
    dw = DeviceArray((H,)) if need_dw else None
    db = DeviceArray((H,)) if need_db else None
    ds = DeviceArray((rows // lead, H))
    call("oxi_layer_norm_bwd_lead_sum", x.ptr, w.ptr if w else None, b.ptr if b else None, mean.ptr, rstd.ptr, g.ptr,
         ACT[act], dy.ptr if dy else None, dx.ptr, dw.ptr if dw else None, db.ptr if db else None, ds.ptr, lead, rows,
         H, NORM_VJP[mode])
    return dy, dx, dw, db, ds


NOALLOC_SCRATCH_BYTES = 16 << 20  # OXI_NOALLOC_SCRATCH_BYTES


def layer_norm_bwd_noalloc(x, w, mean, rstd, g, dx, dw, db, mode="ref"):
    """oxi_layer_norm_bwd_noalloc into caller-provided outputs (DeviceArrays
    or None); the call itself allocates nothing."""
    rows, H = _rows(x)
    call("oxi_layer_norm_bwd_noalloc", x.ptr, w.ptr if w else None, mean.ptr, rstd.ptr, g.ptr,
         dx.ptr if dx else None, dw.ptr if dw else None, db.ptr if db else None, rows, H, NORM_VJP[mode])


def rms_norm_act_bwd(x, w, rstd, g, act, mode="ref", need_dy=True, need_dx=True, need_dw=True):
    """VJP of act(rms_norm(x)) in one pass; returns (dy, dx, dw). `act` is a key of ACT."""
    rows, H = _rows(x)
    dy = DeviceArray(x.shape) if need_dy else None
    dx = DeviceArray(x.shape) if need_dx else None
    dw = DeviceArray((H,)) if need_dw else None
    call("oxi_rms_norm_act_bwd", x.ptr, w.ptr if w else None, rstd.ptr, g.ptr, ACT[act], dy.ptr if dy else None,
         dx.ptr if dx else None, dw.ptr if dw else None, rows, H, NORM_VJP[mode])
    return dy, dx, dw


def layer_norm_act_bwd(x, w, b, mean, rstd, g, act, mode="ref", need_dy=True, need_dx=True, need_dw=True,
                       need_db=True):
    """VJP of act(layer_norm(x)) in one pass; returns (dy, dx, dw, db). `act` is a key of ACT."""
    rows, H = _rows(x)
    dy = DeviceArray(x.shape) if need_dy else None
    dx = DeviceArray(x.shape) if need_dx else None
    dw = DeviceArray((H,)) if need_dw else None
    db = DeviceArray((H,)) if need_db else None
    call("oxi_layer_norm_act_bwd", x.ptr, w.ptr if w else None, b.ptr if b else None, mean.ptr, rstd.ptr, g.ptr,
         ACT[act], dy.ptr if dy else None, dx.ptr if dx else None, dw.ptr if dw else None, db.ptr if db else None,
         rows, H, NORM_VJP[mode])
    return dy, dx, dw, db


def _oli(shape, dim):
    dim = dim % len(shape)
    outer = int(np.prod(shape[:dim], dtype=np.int64))
    inner = int(np.prod(shape[dim + 1:], dtype=np.int64))
    return outer, shape[dim], inner


def softmax_fwd(x: DeviceArray, dim=-1, log=False) -> DeviceArray:
    y = DeviceArray(x.shape)
    call("oxi_log_softmax_fwd" if log else "oxi_softmax_fwd", x.ptr, y.ptr, *_oli(x.shape, dim))
    return y


def softmax_bwd(y: DeviceArray, g: DeviceArray, dim=-1, log=False) -> DeviceArray:
    dx = DeviceArray(y.shape)
    call("oxi_log_softmax_bwd" if log else "oxi_softmax_bwd", y.ptr, g.ptr, dx.ptr, *_oli(y.shape, dim))
    return dx


def cross_entropy_fwd(logits: DeviceArray, targets: DeviceArray):
    n, c = logits.shape
    loss = DeviceArray((1,))
    lse = DeviceArray((n,))
    call("oxi_cross_entropy_fwd", logits.ptr, targets.ptr, loss.ptr, lse.ptr, n, c)
    return loss, lse


def cross_entropy_fwd_grad(logits: DeviceArray, targets: DeviceArray):
    """Loss, lse and the gradient for an upstream 1 in one pass (oxi_cross_entropy_fwd_grad)."""
    n, c = logits.shape
    loss = DeviceArray((1,))
    lse = DeviceArray((n,))
    d = DeviceArray((n, c))
    call("oxi_cross_entropy_fwd_grad", logits.ptr, targets.ptr, loss.ptr, lse.ptr, d.ptr, n, c)
    return loss, lse, d


def cross_entropy_bwd(logits: DeviceArray, targets: DeviceArray, lse: DeviceArray, gloss: DeviceArray):
    n, c = logits.shape
    d = DeviceArray((n, c))
    call("oxi_cross_entropy_bwd", logits.ptr, targets.ptr, lse.ptr, gloss.ptr, d.ptr, n, c)
    return d


def index_select(src: DeviceArray, dim: int, idx: DeviceArray) -> DeviceArray:
    o, l, i = _oli(src.shape, dim)
    shape = list(src.shape)
    shape[dim % len(shape)] = idx.size
    out = DeviceArray(shape)
    call("oxi_index_select", src.ptr, o, l, i, idx.ptr, idx.size, out.ptr)
    return out


def index_select_bwd(g: DeviceArray, full_shape, dim: int, idx: DeviceArray) -> DeviceArray:
    o, l, i = _oli(tuple(full_shape), dim)
    grad = DeviceArray(full_shape)
    call("oxi_index_select_bwd", g.ptr, o, l, i, idx.ptr, idx.size, grad.ptr)
    return grad


class BwdPlan:
    """The id sort of an index_select VJP, queued on the library's second
    stream (oxi_index_select_bwd_plan); freed with the object."""

    def __init__(self, idx: DeviceArray, length: int):
        p = vp()
        call("oxi_index_select_bwd_plan", idx.ptr, idx.size, length, ctypes.byref(p))
        self.ptr = p.value

    def apply(self, g: DeviceArray, full_shape, dim: int) -> DeviceArray:
        o, _, i = _oli(tuple(full_shape), dim)
        grad = DeviceArray(full_shape)
        call("oxi_index_select_bwd_apply", self.ptr, g.ptr, o, i, grad.ptr)
        return grad

    def free(self):
        if self.ptr:
            lib.oxi_index_select_bwd_plan_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def embedding_fwd(W: DeviceArray, ids: DeviceArray) -> DeviceArray:
    V, D = W.shape
    out = DeviceArray((ids.size, D))
    call("oxi_embedding_fwd", W.ptr, ids.ptr, ids.size, V, D, out.ptr)
    return out


def embedding_bwd(g: DeviceArray, ids: DeviceArray, V: int) -> DeviceArray:
    D = g.shape[-1]
    dW = DeviceArray((V, D))
    call("oxi_embedding_bwd", g.ptr, ids.ptr, ids.size, V, D, dW.ptr)
    return dW


def reduce(kind: str, x: DeviceArray, dim: int, x_strides=None, shape=None) -> DeviceArray:
    shape = tuple(shape or x.shape)
    dim = dim % len(shape)
    out = DeviceArray(shape[:dim] + shape[dim + 1:])
    call("oxi_reduce", REDUCE.index(kind), x.ptr, _i64arr(x_strides or row_major_strides(shape)), _i64arr(shape),
         len(shape), dim, out.ptr)
    return out


def sgd_step(p: DeviceArray, g: DeviceArray, buf: DeviceArray | None, lr, momentum=0.0, nesterov=False,
             out: DeviceArray | None = None) -> DeviceArray:
    """One SGD step over a flat parameter; `buf` is updated in place. `out`
    defaults to a new array; pass `p` to update in place."""
    out = out if out is not None else DeviceArray(p.shape)
    call("oxi_sgd_step", p.ptr, g.ptr, buf.ptr if buf is not None else None, out.ptr, p.size, lr, momentum,
         int(bool(nesterov)))
    return out


def adamw_step(p: DeviceArray, g: DeviceArray, m: DeviceArray, v: DeviceArray, t: int, lr, beta1=0.9, beta2=0.999,
               eps=1e-8, weight_decay=1e-2, decoupled=True, out: DeviceArray | None = None) -> DeviceArray:
    """One Adam/AdamW step at step count `t`; `m`, `v` are updated in place."""
    out = out if out is not None else DeviceArray(p.shape)
    call("oxi_adamw_step", p.ptr, g.ptr, m.ptr, v.ptr, out.ptr, p.size, lr, beta1, beta2, eps, weight_decay,
         int(bool(decoupled)), t)
    return out


def scatter_rows(base: DeviceArray, idx: DeviceArray, values: DeviceArray) -> DeviceArray:
    """Tensor::scatter_dim0 on a contiguous base: rows idx[p] <- values[p], last write wins."""
    rows = base.shape[0]
    inner = int(np.prod(base.shape[1:], dtype=np.int64))
    out = DeviceArray(base.shape)
    call("oxi_scatter_rows", base.ptr, rows, inner, idx.ptr, idx.size, values.ptr, out.ptr)
    return out


def scatter_rows_bwd(g: DeviceArray, idx: DeviceArray, values_shape, need_base=True, need_values=True):
    rows = g.shape[0]
    inner = int(np.prod(g.shape[1:], dtype=np.int64))
    gb = DeviceArray(g.shape) if need_base else None
    gv = DeviceArray(values_shape) if need_values else None
    call("oxi_scatter_rows_bwd", g.ptr, rows, inner, idx.ptr, idx.size, gb.ptr if gb else None, gv.ptr if gv else None)
    return gb, gv


def broadcast_elem_strides(shape, grid):
    """Row-major element strides of a contiguous `shape`, expanded to `grid`
    with 0 on broadcast (missing or size-1) dims."""
    rm = row_major_strides(shape)
    lead = len(grid) - len(shape)
    return [0 if d < lead or shape[d - lead] == 1 else rm[d - lead] for d in range(len(grid))]


def masked_select_record(grid) -> DeviceArray:
    """A device buffer for the record of a selection over `grid`."""
    nb = c_i64(0)
    call("oxi_masked_select_record_bytes", _i64arr(grid), len(grid), ctypes.byref(nb))
    return DeviceArray((nb.value,), np.uint8)


def masked_select(x: DeviceArray, mask: DeviceArray, record: DeviceArray | None = None) -> DeviceArray:
    """Tensor::masked_select over the broadcast of contiguous x and mask; the
    record (for the VJP) goes to `record` when given."""
    grid = tuple(np.broadcast_shapes(x.shape, mask.shape))
    out, cnt = vp(), c_i64(0)
    call("oxi_masked_select", x.ptr, _i64arr(broadcast_elem_strides(x.shape, grid)), mask.ptr,
         _i64arr(broadcast_elem_strides(mask.shape, grid)), _i64arr(grid), len(grid), ctypes.byref(out),
         ctypes.byref(cnt), record.ptr if record is not None else None)
    return DeviceArray.adopt(out.value, (cnt.value,))


def masked_select_bwd(record: DeviceArray, x_shape, mask_shape, g: DeviceArray) -> DeviceArray:
    grid = tuple(np.broadcast_shapes(tuple(x_shape), tuple(mask_shape)))
    gx = DeviceArray(x_shape)
    call("oxi_masked_select_bwd", record.ptr, _i64arr(grid), len(grid), g.ptr, g.size, gx.ptr,
         _i64arr(broadcast_elem_strides(tuple(x_shape), grid)), gx.size)
    return gx


class BatchColumn(ctypes.Structure):
    """oxi_batch_column"""
    _fields_ = [("src", vp), ("dst", vp), ("inner", c_i64)]


def batch_gather(columns, idx: DeviceArray, n: int | None = None) -> list:
    """gather_columns: the rows `idx` of every (len, ...) column, one launch
    per 8 columns; returns the new (n, ...) device arrays."""
    n = idx.size if n is None else n
    length = columns[0].shape[0] if columns else 0
    outs = [DeviceArray((n,) + tuple(c.shape[1:])) for c in columns]
    arr = (BatchColumn * max(1, len(columns)))()
    for k, (c, o) in enumerate(zip(columns, outs)):
        arr[k] = BatchColumn(c.ptr, o.ptr, int(np.prod(c.shape[1:], dtype=np.int64)))
    call("oxi_batch_gather", ctypes.cast(arr, vp), len(columns), length, idx.ptr, n)
    return outs


class SgdSlice(ctypes.Structure):
    """oxi_sgd_slice"""
    _fields_ = [("p", vp), ("g", vp), ("buf", vp), ("p_out", vp), ("n", c_i64)]


class AdamWSlice(ctypes.Structure):
    """oxi_adamw_slice"""
    _fields_ = [("p", vp), ("g", vp), ("m", vp), ("v", vp), ("p_out", vp), ("n", c_i64), ("t", c_i64)]


def slice_array(cls, rows):
    """A ctypes array of `cls` built from tuples of field values."""
    arr = (cls * max(1, len(rows)))()
    for i, r in enumerate(rows):
        arr[i] = cls(*r)
    return arr


class Timer:
    """HIP events on the library stream (the stream every kernel runs on)."""

    def __init__(self):
        self.a, self.b = vp(), vp()
        check(lib.oxi_hip_event_create(ctypes.byref(self.a)))
        check(lib.oxi_hip_event_create(ctypes.byref(self.b)))

    def start(self):
        check(lib.oxi_hip_event_record(self.a))

    def stop(self) -> float:
        check(lib.oxi_hip_event_record(self.b))
        ms = c_float(0.0)
        check(lib.oxi_hip_event_elapsed_ms(self.a, self.b, ctypes.byref(ms)))
        return ms.value

    def __del__(self):
        try:
            lib.oxi_hip_event_destroy(self.a)
            lib.oxi_hip_event_destroy(self.b)
        except Exception:
            pass
