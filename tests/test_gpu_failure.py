"""Allocation failures inside the entry points, injected from the host with
oxi_hip_debug_fail_alloc_after (no kernel is made to fail): each one surfaces
as a RuntimeError that names the call site and carries the allocator's
message, returns every block it took, and leaves the library working, so the
next call gives the bits of a run that never failed.

Every allocation of a call is failed in turn (the first, the second, ...)
until the call makes fewer, so the sweep covers each allocation site of the
embedding VJP's sort plan and its apply, the norm VJP's column partials, and
masked_select's count, record and output blocks; then the same for one whole
forward + backward of the config-5 chain through the host core."""

import gc
import os
import sys

import numpy as np
import pytest

from conftest import rng

pytestmark = pytest.mark.gpu

INJECTED = "injected by oxi_hip_debug_fail_alloc_after"


def say(*a):
    print("[case]", *a, flush=True)
    sys.stdout.flush()


def same_bits(got, want, what):
    got = np.ascontiguousarray(got, dtype=np.float32)
    want = np.ascontiguousarray(want, dtype=np.float32)
    assert got.shape == want.shape, f"{what}: shape {got.shape} vs {want.shape}"
    bad = np.flatnonzero(got.view(np.uint32) != want.view(np.uint32))
    assert bad.size == 0, f"{what}: {bad.size} of {got.size} differ after a failed call; first at {bad[0]}"


def _attempt(hip, k, call):
    """Runs `call` with the k-th device allocation failing; returns the
    RuntimeError's message, or None when the call made fewer than k."""
    hip.lib.oxi_hip_debug_fail_alloc_after(k)
    try:
        call()
    except RuntimeError as e:
        assert type(e) is RuntimeError or isinstance(e, hip.OxiError), f"{type(e).__name__}: {e}"
        return str(e)
    finally:
        hip.lib.oxi_hip_debug_fail_alloc_after(0)
    return None


def sweep(hip, what, call, recover, site, limit=16):
    """Fails each allocation of `call` in turn. After every failure: the
    message names `site` and the injection, the bytes in use are back to
    what they were before the call, and `recover()` (a clean call checked
    against a clean run) passes. Returns how many allocations `call` makes."""
    hip.sync()
    base = hip.memory_stats()[0]
    for k in range(1, limit + 1):
        say(what, "- allocation", k, "fails")
        msg = _attempt(hip, k, call)
        hip.sync()
        if msg is None:
            return k - 1
        assert INJECTED in msg and site in msg, f"{what}, allocation {k}: {msg!r}"
        assert hip.memory_stats()[0] == base, f"{what}, allocation {k}: blocks not returned"
        recover()
    raise AssertionError(f"{what}: more than {limit} allocations")


def test_index_select_bwd_plan_and_apply(hip):
    """oxi_index_select_bwd_plan (its sort workspace) and
    oxi_index_select_bwd_apply (end tiles and partial rows) on a C4-shaped
    id list with duplicates; a plan whose apply failed is applied again."""
    from oxitorch_amd.capi import DeviceArray, BwdPlan

    r = rng(5)
    V, D, n = 5000, 256, 8192
    ids = r.integers(0, V, n)
    ids[:64] = 17  # one long key: the owner path of the apply
    idx = DeviceArray.from_numpy(ids.astype(np.int64))
    g = DeviceArray.from_numpy(r.standard_normal((n, D), dtype=np.float32))
    grad = DeviceArray((V, D))

    clean = BwdPlan(idx, V).apply(g, (V, D), 0).numpy()

    def plan_fails():
        BwdPlan(idx, V)

    def plan_recovers():
        same_bits(BwdPlan(idx, V).apply(g, (V, D), 0).numpy(), clean, "plan, then apply")

    made = sweep(hip, "index_select_bwd_plan", plan_fails, plan_recovers, "index_select_bwd: sort workspace")
    assert made == 1, made

    plan = BwdPlan(idx, V)

    def apply_fails():
        hip.call("oxi_index_select_bwd_apply", plan.ptr, g.ptr, 1, D, grad.ptr)

    def apply_recovers():
        hip.call("oxi_index_select_bwd_apply", plan.ptr, g.ptr, 1, D, grad.ptr)
        same_bits(grad.numpy(), clean, "apply of a plan whose apply failed")

    made = sweep(hip, "index_select_bwd_apply", apply_fails, apply_recovers, "index_select_bwd: apply workspace")
    assert made == 2, made

    def oneshot():
        hip.call("oxi_index_select_bwd", g.ptr, 1, V, D, idx.ptr, n, grad.ptr)

    def oneshot_recovers():
        oneshot()
        same_bits(grad.numpy(), clean, "one-shot index_select_bwd")

    made = sweep(hip, "index_select_bwd", oneshot, oneshot_recovers, "index_select_bwd:")
    assert made == 3, made


@pytest.mark.parametrize("kind", ["layer_norm", "rms_norm", "layer_norm_lead_sum"])
def test_norm_vjp_workspace(hip, kind):
    """The norm VJP's column partials (dw/db need them) at a C1 shape; the
    lead-sum variant on (16, 64, 768) rows."""
    from oxitorch_amd.capi import DeviceArray, NORM_VJP, ACT

    r = rng(9)
    lead, T, H = 16, 64, 768
    rows = lead * T
    xa = r.standard_normal((rows, H), dtype=np.float32)
    x = DeviceArray.from_numpy(xa)
    w = DeviceArray.from_numpy(r.standard_normal(H, dtype=np.float32))
    b = DeviceArray.from_numpy(r.standard_normal(H, dtype=np.float32))
    g = DeviceArray.from_numpy(r.standard_normal((rows, H), dtype=np.float32))
    if kind == "rms_norm":
        _, rstd = hip.rms_norm_fwd(x, w)
        mean = None
    else:
        _, mean, rstd = hip.layer_norm_fwd(x, w, b)
    dx, dw, db = DeviceArray((rows, H)), DeviceArray((H,)), DeviceArray((H,))
    ds = DeviceArray((T, H))
    outs = {"dx": dx, "dw": dw} if kind == "rms_norm" else {"dx": dx, "dw": dw, "db": db}
    if kind == "layer_norm_lead_sum":
        outs["dx_sum"] = ds

    def call():
        if kind == "layer_norm":
            hip.call("oxi_layer_norm_bwd", x.ptr, w.ptr, mean.ptr, rstd.ptr, g.ptr, dx.ptr, dw.ptr, db.ptr, rows, H,
                     NORM_VJP["ref"])
        elif kind == "rms_norm":
            hip.call("oxi_rms_norm_bwd", x.ptr, w.ptr, rstd.ptr, g.ptr, dx.ptr, dw.ptr, rows, H, NORM_VJP["ref"])
        else:
            hip.call("oxi_layer_norm_bwd_lead_sum", x.ptr, w.ptr, b.ptr, mean.ptr, rstd.ptr, g.ptr, ACT["none"], None,
                     dx.ptr, dw.ptr, db.ptr, ds.ptr, lead, rows, H, NORM_VJP["ref"])

    call()
    clean = {k: v.numpy() for k, v in outs.items()}

    def recover():
        call()
        for k, v in outs.items():
            same_bits(v.numpy(), clean[k], f"{kind} {k}")

    made = sweep(hip, kind + " VJP", call, recover, "norm VJP: column partials")
    assert made == 1, made


def test_masked_select(hip):
    """masked_select of a column broadcast over a 3-d mask. The record (when
    the caller passes none) fails first. The one-pass path's output, sized for
    every grid point, failing is not an error: the call takes the two-pass
    path, whose per-tile counts and exact-size output then each fail in turn.
    Then the VJP's grid-order buffer, which the broadcast x needs."""
    from oxitorch_amd.capi import DeviceArray

    r = rng(13)
    xs, ms = (96, 1), (64, 96, 128)
    x = DeviceArray.from_numpy(r.standard_normal(xs, dtype=np.float32))
    mask = DeviceArray.from_numpy((r.random(ms) > 0.4).astype(np.float32))
    clean = hip.masked_select(x, mask).numpy()
    assert clean.size > 0

    def call():
        hip.masked_select(x, mask).free()

    def recover():
        same_bits(hip.masked_select(x, mask).numpy(), clean, "masked_select")

    # one pass: the record (1), the output for every grid point (2), the
    # look-back status words (3). The output failing is not an error: the
    # call takes the two-pass path, with the same bits.
    base = hip.memory_stats()[0]
    for k, site in ((1, "masked_select: workspace"), (2, None), (3, "masked_select: look-back workspace")):
        say("masked_select one pass - allocation", k, "fails")
        hip.lib.oxi_hip_debug_fail_alloc_after(k)
        try:
            got = hip.masked_select(x, mask)
        except RuntimeError as e:
            got, msg = None, str(e)
        finally:
            hip.lib.oxi_hip_debug_fail_alloc_after(0)
        hip.sync()
        if site is None:
            assert got is not None, k
            same_bits(got.numpy(), clean, "masked_select on the two-pass path")
            got.free()
        else:
            assert got is None and INJECTED in msg and site in msg, (k, msg)
        hip.sync()
        assert hip.memory_stats()[0] == base, k
        recover()
    assert _attempt(hip, 4, call) is None  # no fourth allocation
    # two passes (OXI_MASKED_SELECT_EXACT=1): the record, the per-tile counts
    # and the exact-size output each fail in turn
    os.environ["OXI_MASKED_SELECT_EXACT"] = "1"
    try:
        made = sweep(hip, "masked_select two-pass", call, recover, "masked_select:")
    finally:
        del os.environ["OXI_MASKED_SELECT_EXACT"]
    assert made == 3, made

    grid = tuple(np.broadcast_shapes(xs, ms))
    rec = hip.masked_select_record(grid)
    same_bits(hip.masked_select(x, mask, rec).numpy(), clean, "masked_select with a record")
    g = DeviceArray.from_numpy(r.standard_normal(clean.shape, dtype=np.float32))
    want = hip.masked_select_bwd(rec, xs, ms, g).numpy()
    gx = DeviceArray(xs)

    def bwd():
        hip.call("oxi_masked_select_bwd", rec.ptr, hip._i64arr(grid), len(grid), g.ptr, g.size, gx.ptr,
                 hip._i64arr(hip.broadcast_elem_strides(xs, grid)), gx.size)

    def bwd_recovers():
        bwd()
        same_bits(gx.numpy(), want, "masked_select_bwd")

    made = sweep(hip, "masked_select_bwd", bwd, bwd_recovers, "masked_select_bwd: workspace")
    assert made == 1, made


def test_masked_select_offset_wait(hip):
    """The one pass's offset wait failing, forced from the host: with
    OXI_MSEL_SPIN_LIMIT=-1 every chunk but the first gives up its wait at
    once (no kernel spins or faults). The call reports the failed last chunk,
    returns every block it took, and oxi_hip_sync reports the guard; a grid of
    one chunk never waits, and the next call gives the clean bits."""
    from oxitorch_amd.capi import DeviceArray

    r = rng(14)
    shape = (64, 96, 128)  # 192 tiles of 4096 points: 48 chunks
    xa = r.standard_normal(shape, dtype=np.float32)
    ma = (r.random(shape) > 0.4).astype(np.float32)
    x, mask = DeviceArray.from_numpy(xa), DeviceArray.from_numpy(ma)
    clean = hip.masked_select(x, mask).numpy()
    same_bits(clean, xa[ma != 0], "masked_select")
    small_x = DeviceArray.from_numpy(xa[:1, :96, :128].copy())  # 12288 points: one chunk
    small_m = DeviceArray.from_numpy(ma[:1, :96, :128].copy())
    base = hip.memory_stats()[0]
    say("masked_select one pass - every offset wait fails")
    os.environ["OXI_MSEL_SPIN_LIMIT"] = "-1"
    try:
        with pytest.raises(RuntimeError, match="offset wait did not finish"):
            hip.masked_select(x, mask)
        with pytest.raises(RuntimeError, match="offset wait did not finish"):
            hip.sync()
        got = hip.masked_select(small_x, small_m)
        same_bits(got.numpy(), xa[:1, :96, :128][ma[:1, :96, :128] != 0], "masked_select, one chunk")
        got.free()
        hip.sync()
    finally:
        del os.environ["OXI_MSEL_SPIN_LIMIT"]
    assert hip.memory_stats()[0] == base
    same_bits(hip.masked_select(x, mask).numpy(), clean, "masked_select after the failed waits")
    hip.sync()


def _c5_step(ox, F, data):
    """One forward + backward of the config-5 chain (embedding, layer_norm,
    silu through a permute, positional add, rms_norm, softmax) on fresh
    leaves; returns the output and every leaf gradient as numpy arrays."""
    Wa, ids, lnw, lnb, rw, pos, g, (B, T, H) = data
    W, LW, LB, RW, P = (ox.from_numpy(a, True) for a in (Wa, lnw, lnb, rw, pos))
    G = ox.from_numpy(g)
    h = F.layer_norm(F.embedding(ids, W).reshape([B, T, H]), LW, LB)
    s = F.silu(h.permute([0, 2, 1]))
    y = F.softmax(F.rms_norm(s.permute([0, 2, 1]) + P, RW), -1)
    y.backward(G)
    return {"y": y.numpy(), "W": W.grad.numpy(), "lnw": LW.grad.numpy(), "lnb": LB.grad.numpy(),
            "rw": RW.grad.numpy(), "pos": P.grad.numpy()}


def test_host_core_step(hip):
    """Each allocation of one whole step through the host core fails in
    turn: a RuntimeError with the injected message reaches Python, the step's
    blocks all come back once its tensors are gone, and the next step gives
    the same bits as a step that never failed."""
    import oxitorch_amd as ox
    from oxitorch_amd.nn import functional as F

    r = rng(17)
    B, T, H, V = 4, 64, 256, 1000
    data = (r.standard_normal((V, H), dtype=np.float32), r.integers(0, V, B * T),
            *(r.standard_normal(H, dtype=np.float32) for _ in range(3)),
            r.standard_normal((1, T, H), dtype=np.float32), r.standard_normal((B, T, H), dtype=np.float32), (B, T, H))
    clean = _c5_step(ox, F, data)
    gc.collect()
    hip.sync()
    base = hip.memory_stats()[0]
    made = None
    for k in range(1, 400):
        say("C5 step through the host core - allocation", k, "fails")
        msg = _attempt(hip, k, lambda: _c5_step(ox, F, data))
        gc.collect()
        hip.sync()
        assert hip.memory_stats()[0] == base, f"allocation {k}: blocks of the failed step not returned"
        if msg is None:
            made = k - 1
            break
        assert INJECTED in msg, f"allocation {k}: {msg!r}"
        again = _c5_step(ox, F, data)
        for key, v in clean.items():
            same_bits(again[key], v, f"C5 step after allocation {k} failed: {key}")
    assert made is not None and made > 10, made
