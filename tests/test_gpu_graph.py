"""HIP graph capture of a step of C-ABI calls that allocate nothing.

The norm forwards and the elementwise kernels take no workspace, and
oxi_layer_norm_bwd_noalloc keeps its column partials in the library's fixed
device scratch. A caller can therefore capture a whole step of these calls
on the library stream (oxi_hip_stream) into a hipGraph and replay it. Config
2's step is captured once: layer_norm -> exact-erf gelu forward, the gelu
VJP, then the LayerNorm VJP through the no-alloc entry point. It is replayed
four times. Between replays the test uploads new inputs into the captured
buffers and runs the same step eagerly through the allocating entry points,
with host synchronisations in between. Every replay's outputs must equal the
eager step's bit for bit. A second step captures the other workspace-free
families the same way: a norm forward, softmax forward and VJP, a dim
reduction and an AdamW step. No call inside the capture allocates, copies,
clears memory or waits.
"""

import ctypes
import sys

import numpy as np
import pytest

from conftest import rng

pytestmark = pytest.mark.gpu

CAPTURE_MODE_RELAXED = 2  # hipStreamCaptureModeRelaxed


def say(*a):
    print("[case]", *a, flush=True)
    sys.stdout.flush()


def _runtime():
    """The HIP runtime liboxihip is linked against (same soname, same instance)."""
    rt = ctypes.CDLL("libamdhip64.so.7")
    vp = ctypes.c_void_p
    rt.hipStreamBeginCapture.argtypes = [vp, ctypes.c_int]
    rt.hipStreamEndCapture.argtypes = [vp, ctypes.POINTER(vp)]
    rt.hipGraphInstantiate.argtypes = [ctypes.POINTER(vp), vp, vp, ctypes.c_char_p, ctypes.c_size_t]
    rt.hipGraphLaunch.argtypes = [vp, vp]
    rt.hipGraphExecDestroy.argtypes = [vp]
    rt.hipGraphDestroy.argtypes = [vp]
    for f in ("hipStreamBeginCapture", "hipStreamEndCapture", "hipGraphInstantiate", "hipGraphLaunch",
              "hipGraphExecDestroy", "hipGraphDestroy"):
        getattr(rt, f).restype = ctypes.c_int
    return rt


def test_c2_step_replayed_from_a_hip_graph(hip):
    R, H = 2048, 4096
    say("hip graph: C2 step", (R, H))
    rt = _runtime()
    A = hip.DeviceArray
    x, g = A((R, H)), A((R, H))
    r = rng(31)
    w = hip.DeviceArray.from_numpy((r.standard_normal(H, dtype=np.float32) * 0.02 + 1).astype(np.float32))
    b = hip.DeviceArray.from_numpy((r.standard_normal(H, dtype=np.float32) * 0.02).astype(np.float32))

    def outputs():
        return dict(y=A((R, H)), mean=A((R,)), rstd=A((R,)), a=A((R, H)), dh=A((R, H)), dx=A((R, H)),
                    dw=A((H,)), db=A((H,)))

    G, E = outputs(), outputs()  # the graph's outputs, the eager step's
    rm = hip._i64arr([H, 1])
    shape = hip._i64arr([R, H])
    gelu = hip.GELU["none"]

    def step(o, noalloc):
        hip.call("oxi_layer_norm_fwd", x.ptr, w.ptr, b.ptr, o["y"].ptr, o["mean"].ptr, o["rstd"].ptr, R, H,
                 ctypes.c_float(1e-5))
        hip.call("oxi_gelu_fwd", o["y"].ptr, rm, o["a"].ptr, rm, shape, 2, gelu)
        hip.call("oxi_gelu_bwd", o["y"].ptr, rm, g.ptr, rm, o["dh"].ptr, rm, shape, 2, gelu)
        hip.call("oxi_layer_norm_bwd_noalloc" if noalloc else "oxi_layer_norm_bwd", x.ptr, w.ptr, o["mean"].ptr,
                 o["rstd"].ptr, o["dh"].ptr, o["dx"].ptr, o["dw"].ptr, o["db"].ptr, R, H, 0)

    stream = ctypes.c_void_p()
    hip.check(hip.lib.oxi_hip_stream(ctypes.byref(stream)))
    hip.sync()
    graph, exe = ctypes.c_void_p(), ctypes.c_void_p()
    assert rt.hipStreamBeginCapture(stream, CAPTURE_MODE_RELAXED) == 0
    try:
        step(G, noalloc=True)
    finally:
        rc_end = rt.hipStreamEndCapture(stream, ctypes.byref(graph))  # the stream never stays capturing
    assert rc_end == 0 and graph.value
    try:
        assert rt.hipGraphInstantiate(ctypes.byref(exe), graph, None, None, 0) == 0
        for k in range(4):
            say("hip graph replay", k)
            rk = rng(100 + k)
            xs = (rk.standard_normal((R, H), dtype=np.float32) * (1 + k)).astype(np.float32)
            gs = rk.standard_normal((R, H), dtype=np.float32)
            hip.check(hip.lib.oxi_hip_memcpy_h2d(x.ptr, xs.ctypes.data, x.nbytes))
            hip.check(hip.lib.oxi_hip_memcpy_h2d(g.ptr, gs.ctypes.data, g.nbytes))
            step(E, noalloc=False)
            hip.sync()
            assert rt.hipGraphLaunch(exe, stream) == 0
            hip.sync()
            for name in G:
                got, want = G[name].numpy(), E[name].numpy()
                bad = np.flatnonzero(got.view(np.uint32) != want.view(np.uint32))
                assert bad.size == 0, f"replay {k}: {name} differs from the eager step at {bad.size} elements"
            assert np.isfinite(E["dx"].numpy()).all()
    finally:
        if exe.value:
            rt.hipGraphExecDestroy(exe)
        rt.hipGraphDestroy(graph)


def test_norm_softmax_reduce_optimizer_step_replayed_from_a_hip_graph(hip):
    """The other workspace-free families in one captured step: rms_norm
    forward, softmax forward and VJP over the rows, the column sum of the
    VJP (a dim reduction), and an AdamW step on a parameter with that sum as
    its gradient (m and v updated in place, reset to the same state before
    each replay and each eager step). Every replay equals the eager step bit
    for bit, the updated moments included."""
    R, H = 1024, 768
    say("hip graph: rms_norm, softmax, reduce, adamw", (R, H))
    rt = _runtime()
    A = hip.DeviceArray
    r = rng(32)
    x, g = A((R, H)), A((R, H))
    w = hip.DeviceArray.from_numpy((r.standard_normal(H, dtype=np.float32) * 0.02 + 1).astype(np.float32))
    P = hip.DeviceArray.from_numpy(r.standard_normal(H, dtype=np.float32))
    m0 = (r.standard_normal(H, dtype=np.float32) * 0.01).astype(np.float32)
    v0 = np.abs(r.standard_normal(H, dtype=np.float32) * 0.01).astype(np.float32)

    def outputs():
        return dict(y=A((R, H)), rstd=A((R,)), p=A((R, H)), dp=A((R, H)), s=A((H,)), m=A((H,)), v=A((H,)),
                    Pn=A((H,)))

    G, E = outputs(), outputs()
    rm = hip._i64arr([H, 1])
    shape = hip._i64arr([R, H])
    SUM = hip.REDUCE.index("sum")

    def step(o):
        hip.call("oxi_rms_norm_fwd", x.ptr, w.ptr, o["y"].ptr, o["rstd"].ptr, R, H, ctypes.c_float(1e-6))
        hip.call("oxi_softmax_fwd", o["y"].ptr, o["p"].ptr, R, H, 1)
        hip.call("oxi_softmax_bwd", o["p"].ptr, g.ptr, o["dp"].ptr, R, H, 1)
        hip.call("oxi_reduce", SUM, o["dp"].ptr, rm, shape, 2, 0, o["s"].ptr)
        hip.call("oxi_adamw_step", P.ptr, o["s"].ptr, o["m"].ptr, o["v"].ptr, o["Pn"].ptr, H, 1e-3, 0.9, 0.999,
                 1e-8, 1e-2, 1, 3)

    def reset(o):
        hip.check(hip.lib.oxi_hip_memcpy_h2d(o["m"].ptr, m0.ctypes.data, o["m"].nbytes))
        hip.check(hip.lib.oxi_hip_memcpy_h2d(o["v"].ptr, v0.ctypes.data, o["v"].nbytes))

    stream = ctypes.c_void_p()
    hip.check(hip.lib.oxi_hip_stream(ctypes.byref(stream)))
    hip.sync()
    graph, exe = ctypes.c_void_p(), ctypes.c_void_p()
    assert rt.hipStreamBeginCapture(stream, CAPTURE_MODE_RELAXED) == 0
    try:
        step(G)
    finally:
        rc_end = rt.hipStreamEndCapture(stream, ctypes.byref(graph))
    assert rc_end == 0 and graph.value
    try:
        assert rt.hipGraphInstantiate(ctypes.byref(exe), graph, None, None, 0) == 0
        for k in range(4):
            say("hip graph replay", k)
            rk = rng(200 + k)
            xs = (rk.standard_normal((R, H), dtype=np.float32) * (1 + k)).astype(np.float32)
            gs = rk.standard_normal((R, H), dtype=np.float32)
            hip.check(hip.lib.oxi_hip_memcpy_h2d(x.ptr, xs.ctypes.data, x.nbytes))
            hip.check(hip.lib.oxi_hip_memcpy_h2d(g.ptr, gs.ctypes.data, g.nbytes))
            reset(E)
            step(E)
            reset(G)
            hip.sync()
            assert rt.hipGraphLaunch(exe, stream) == 0
            hip.sync()
            for name in G:
                got, want = G[name].numpy(), E[name].numpy()
                bad = np.flatnonzero(got.view(np.uint32) != want.view(np.uint32))
                assert bad.size == 0, f"replay {k}: {name} differs from the eager step at {bad.size} elements"
            assert not np.array_equal(E["m"].numpy(), m0), "the step must move the first moment"
    finally:
        if exe.value:
            rt.hipGraphExecDestroy(exe)
        rt.hipGraphDestroy(graph)
