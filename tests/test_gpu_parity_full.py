"""Full-size parity on the paths the host core takes by default.

- Config 2 through F.gelu(F.layer_norm(...), approximate="none").backward():
  the graph runs the fused layer_norm + GELU VJP by default; with the fusion
  off it runs the two VJPs. Both must agree bit for bit, and the result is
  checked against the oracle and the float64 chain over all 16384 rows.
- The fused norm + activation VJP where blocks own several rows: wide rows
  (one row per 256/512-thread block, at most 2 blocks per CU) beyond 2 x CUs
  rows, so the second register set of the double-buffered loop runs, and
  one-wave rows beyond 16 per CU, for every activation.
- Config 3's gradient on all 8192 rows (n * dlogits against the float64
  closed form, the f32 oracle beside it), through the C-ABI and through
  F.cross_entropy(...).backward().
- LayerNorm's exact VJP at config 2's 16384 rows against float64.
"""

import functools
import sys

import numpy as np
import pytest

from conftest import assert_close, assert_close_arb, assert_reduction_close, record, rng

pytestmark = pytest.mark.gpu

ACTS = ["gelu_tanh", "gelu_erf", "silu"]


def say(*a):
    print("[case]", *a, flush=True)
    sys.stdout.flush()


def D(hip, a):
    return hip.DeviceArray.from_numpy(np.ascontiguousarray(a))


def _same(a, b, what):
    assert a.shape == b.shape, what
    bad = np.flatnonzero(a.view(np.uint32) != b.view(np.uint32))
    assert bad.size == 0, f"{what}: {bad.size} of {a.size} differ, first at {bad[0]}: {a.flat[bad[0]]} vs {b.flat[bad[0]]}"


def _merge(parts):
    """One report entry from the stats of several row chunks."""
    out = {"n": sum(p["n"] for p in parts), "arbitrated": sum(p.get("arbitrated", 0) for p in parts)}
    for k in ("worst_tol", "worst_tol_f64", "ref_worst_tol_f64"):
        vals = [p[k] for p in parts if p.get(k) is not None]
        if vals:
            out[k] = max(vals)
    return out


@pytest.fixture(scope="module")
def ox(hip):
    import oxitorch_amd as ox
    return ox


@pytest.fixture(scope="module")
def F(ox):
    from oxitorch_amd.nn import functional as F
    return F


def _c2_inputs():
    """Config 2's inputs as bench.py draws them (seed 2)."""
    r = np.random.default_rng(2)
    R, H = 16384, 4096
    x = r.standard_normal((R, H), dtype=np.float32)
    w = (r.standard_normal(H, dtype=np.float32) * 0.02 + 1).astype(np.float32)
    b = (r.standard_normal(H, dtype=np.float32) * 0.02).astype(np.float32)
    g = r.standard_normal((R, H), dtype=np.float32)
    return x, w, b, g


# ---------------------------------------------------------------------------
# Config 2 through the graph, fused (the default) and unfused

def test_c2_graph_fused_and_unfused(ox, F):
    from oracle import closed_form, ref
    from oxitorch_amd import _native
    say("C2 via F.* (16384, 4096), fused and unfused norm+gelu VJP")
    x, w, b, g = _c2_inputs()
    G = ox.from_numpy(g)
    out = {}
    for fuse in (True, False):
        prev = _native.fuse_norm_act()
        _native.set_fuse_norm_act(fuse)
        try:
            n0 = _native.fused_norm_act_passes()
            X, Wt, Bt = (ox.from_numpy(a, True) for a in (x, w, b))
            y = F.gelu(F.layer_norm(X, Wt, Bt, 1e-5), approximate="none")
            y.backward(G)
            passes = _native.fused_norm_act_passes() - n0
        finally:
            _native.set_fuse_norm_act(prev)
        assert passes == (1 if fuse else 0), f"fuse={fuse}: {passes} fused passes"
        out[fuse] = [a.numpy() for a in (y, X.grad, Wt.grad, Bt.grad)]
    for name, a, c in zip(("y", "dx", "dw", "db"), out[True], out[False]):
        _same(a, c, f"C2 {name}: fused vs two VJPs")
    y, dx, dw, db = out[True]

    # the reference path in f32 over all rows, the float64 chain in row chunks
    h_ref, mu_ref, inv_ref = ref.layer_norm_fwd(x, w, b, 1e-5)
    dh_ref = ref.gelu_erf_bwd(h_ref, g)
    dx_ref, dw_ref, db_ref = ref.layer_norm_bwd(x, w, mu_ref, inv_ref, dh_ref)
    y_ref = ref.gelu_erf_fwd(h_ref)
    H = x.shape[1]
    dw64, db64 = np.zeros(H), np.zeros(H)
    sy, sdx = [], []
    for s in range(0, x.shape[0], 2048):
        sl = slice(s, s + 2048)
        h64, _, _ = closed_form.layer_norm_fwd(x[sl], w, b, 1e-5)
        dx64, dwc, dbc = closed_form.layer_norm_bwd_refgraph(x[sl], w, closed_form.gelu_erf_grad(h64) * g[sl], 1e-5)
        dw64 += dwc
        db64 += dbc
        sy.append(assert_close_arb(y[sl], y_ref[sl], closed_form.gelu_erf(h64), what=f"C2 y rows {s}+"))
        sdx.append(assert_close_arb(dx[sl], dx_ref[sl], dx64, what=f"C2 dx rows {s}+"))
    record("C2", "y via F.* vs oracle chain", _merge(sy))
    record("C2", "dx via F.*, fused VJP", _merge(sdx))
    record("C2", "dw via F.*, fused VJP", assert_reduction_close(dw, dw_ref, dw64, what="C2 dw"))
    record("C2", "db via F.*, fused VJP", assert_reduction_close(db, db_ref, db64, what="C2 db"))


# ---------------------------------------------------------------------------
# Fused norm + activation VJP where blocks own several rows

def _act_bwd(hip, y, g, act):
    if act in ("softmax", "log_softmax"):
        log = act == "log_softmax"
        return hip.softmax_bwd(hip.softmax_fwd(y, log=log), g, log=log)
    if act == "silu":
        return hip.silu_bwd(y, g)
    return hip.gelu_bwd(y, g, "tanh" if act == "gelu_tanh" else "none")


# wide rows: at most 2 blocks per CU (512 on 256 CUs), so more rows than that
# give a block 2-3 rows; one-wave rows: 16 (or 8) per block, one (or two)
# block per CU, so more than 4096 rows give a wave several
MULTI_ROW_SHAPES = [(1100, 2048), (1100, 4096), (1030, 8192), (16384, 768), (20000, 1024), (20000, 256)]


@functools.lru_cache(maxsize=None)
def _multi_row_inputs(shape):
    r = rng(sum(shape))
    H = shape[1]
    x = r.standard_normal(shape, dtype=np.float32)
    w = (r.standard_normal(H, dtype=np.float32) * 0.02 + 1).astype(np.float32)
    b = (r.standard_normal(H, dtype=np.float32) * 0.02).astype(np.float32)
    g = r.standard_normal(shape, dtype=np.float32)
    return x, w, b, g


def _check_multi_rows(hip, norm, shape, act, mode):
    x, w, b, g = _multi_row_inputs(shape)
    dx_, dw_, db_, dg = D(hip, x), D(hip, w), D(hip, b), D(hip, g)
    if norm == "layer_norm":
        y, mean, rstd = hip.layer_norm_fwd(dx_, dw_, db_, 1e-5)
        dy2 = _act_bwd(hip, y, dg, act)
        two = hip.layer_norm_bwd(dx_, dw_, mean, rstd, dy2, mode=mode)
        one = hip.layer_norm_act_bwd(dx_, dw_, db_, mean, rstd, dg, act, mode=mode)
    else:
        y, rstd = hip.rms_norm_fwd(dx_, dw_, 1e-6)
        dy2 = _act_bwd(hip, y, dg, act)
        two = hip.rms_norm_bwd(dx_, dw_, rstd, dy2, mode=mode)
        one = hip.rms_norm_act_bwd(dx_, dw_, rstd, dg, act, mode=mode)
    _same(one[0].numpy(), dy2.numpy(), "dy")
    for name, a, c in zip(("dx", "dw", "db"), one[1:], two):
        _same(a.numpy(), c.numpy(), name)
    return x, w, b, g, one


@pytest.mark.parametrize("mode", ["ref", "exact"])
@pytest.mark.parametrize("norm", ["layer_norm", "rms_norm"])
@pytest.mark.parametrize("act", ACTS)
@pytest.mark.parametrize("shape", MULTI_ROW_SHAPES)
def test_fused_vjp_blocks_with_several_rows(hip, shape, act, norm, mode):
    say("fused norm+act VJP, several rows per block", norm, shape, act, mode)
    _check_multi_rows(hip, norm, shape, act, mode)


@pytest.mark.parametrize("norm", ["layer_norm", "rms_norm"])
@pytest.mark.parametrize("act", ["softmax", "log_softmax"])
@pytest.mark.parametrize("shape", [(1100, 2048), (16384, 768), (20000, 256)])
def test_fused_softmax_vjp_blocks_with_several_rows(hip, shape, act, norm):
    say("fused norm+softmax VJP, several rows per block", norm, shape, act)
    _check_multi_rows(hip, norm, shape, act, "ref")


def test_fused_vjp_several_rows_vs_oracle(hip):
    """One multi-row wide case against the oracle directly: gelu_erf on
    layer_norm, (1100, 4096), reference VJP."""
    from oracle import closed_form, ref
    say("fused layer_norm+gelu_erf VJP (1100, 4096) vs oracle")
    x, w, b, g, (dy, dx, dw, db) = _check_multi_rows(hip, "layer_norm", (1100, 4096), "gelu_erf", "ref")
    h_ref, mu_ref, inv_ref = ref.layer_norm_fwd(x, w, b, 1e-5)
    h64, _, _ = closed_form.layer_norm_fwd(x, w, b, 1e-5)
    dy_ref = ref.gelu_erf_bwd(h_ref, g)
    dy64 = closed_form.gelu_erf_grad(h64) * g
    assert_close_arb(dy.numpy(), dy_ref, dy64, what="dy")
    dx_ref, dw_ref, db_ref = ref.layer_norm_bwd(x, w, mu_ref, inv_ref, dy_ref)
    dx64, dw64, db64 = closed_form.layer_norm_bwd_refgraph(x, w, dy64, 1e-5)
    assert_close_arb(dx.numpy(), dx_ref, dx64, what="dx")
    assert_reduction_close(dw.numpy(), dw_ref, dw64, what="dw")
    assert_reduction_close(db.numpy(), db_ref, db64, what="db")


# ---------------------------------------------------------------------------
# Config 3: the gradient on every row

def _c3_inputs():
    r = np.random.default_rng(3)
    n, c = 8192, 32000
    logits = (r.standard_normal((n, c), dtype=np.float32) * 2).astype(np.float32)
    t = r.integers(0, c, n).astype(np.int64)
    return logits, t


def test_cross_entropy_c3_all_rows(hip):
    """Both C3 paths on all 8192 rows: the one-pass forward that writes the
    gradient (what backward() seeded with 1 takes) and the forward, then the
    backward kernel from lse (any other upstream gradient)."""
    from oracle import closed_form, ref
    say("cross_entropy C3 (8192, 32000): n*dlogits on all rows, both paths")
    logits, t = _c3_inputs()
    n = logits.shape[0]
    dl, dt = D(hip, logits), D(hip, t)
    loss, lse = hip.cross_entropy_fwd(dl, dt)
    d = hip.cross_entropy_bwd(dl, dt, lse, D(hip, np.array([1.0], np.float32))).numpy()
    loss1, _, d1 = hip.cross_entropy_fwd_grad(dl, dt)
    d1 = d1.numpy()
    assert np.array_equal(loss1.numpy().view(np.uint32), loss.numpy().view(np.uint32))
    parts, parts1, tot = [], [], 0.0
    for s in range(0, n, 512):
        sl = slice(s, s + 512)
        k = logits[sl].shape[0]
        # the oracle divides by its own row count: scale both to softmax - onehot
        want = ref.cross_entropy_bwd(logits[sl], t[sl]) * k
        exact = closed_form.cross_entropy_grad(logits[sl], t[sl]) * k
        parts1.append(assert_close_arb(d1[sl] * n, want, exact, what=f"C3 one-pass n*dlogits rows {s}+"))
        parts.append(assert_close_arb(d[sl] * n, want, exact, what=f"C3 n*dlogits rows {s}+"))
        ls = closed_form.log_softmax(logits[sl])
        tot += ls[np.arange(k), t[sl]].sum()
    record("C3", "n*dlogits, one pass, all 8192 rows", _merge(parts1))
    record("C3", "n*dlogits, fwd then bwd, all 8192 rows", _merge(parts))
    l = float(loss.numpy()[0])
    err = abs(l - (-tot / n))
    assert err <= 1e-5 * abs(l)
    record("C3", "loss vs f64", {"n": 1, "worst_tol_f64": err / (1e-6 + 1e-5 * abs(tot / n)), "arbitrated": 0})
    # every row of softmax - onehot sums to zero
    for g in (d, d1):
        assert np.abs(g.astype(np.float64).sum(1) * n).max() < 1e-4


def test_cross_entropy_c3_all_rows_through_F(hip, ox, F):
    """F.cross_entropy(...).backward() takes the one-pass kernel for the
    implicit seed 1.0: its gradient equals oxi_cross_entropy_fwd_grad's bit
    for bit on every row."""
    say("cross_entropy C3 via F.*: all rows equal the C-ABI path")
    logits, t = _c3_inputs()
    dl, dt = D(hip, logits), D(hip, t)
    want = hip.cross_entropy_fwd_grad(dl, dt)[2].numpy()
    L = ox.from_numpy(logits, True)
    F.cross_entropy(L, t.tolist()).backward()
    _same(L.grad.numpy(), want, "C3 dlogits via F.* vs C-ABI")


# ---------------------------------------------------------------------------
# LayerNorm exact VJP at config 2's size

def test_layer_norm_exact_c2_rows(hip):
    from oracle import closed_form, ref
    say("layer_norm exact VJP (16384, 4096) vs float64")
    x, w, b, g = _c2_inputs()
    dxx, dw_, db_ = D(hip, x), D(hip, w), D(hip, b)
    _, mean, rstd = hip.layer_norm_fwd(dxx, dw_, db_, 1e-5)
    dx, dw, db = hip.layer_norm_bwd(dxx, dw_, mean, rstd, D(hip, g), mode="exact")
    dx, dw, db = dx.numpy(), dw.numpy(), db.numpy()
    H = x.shape[1]
    dw64, db64 = np.zeros(H), np.zeros(H)
    parts = []
    for s in range(0, x.shape[0], 2048):
        sl = slice(s, s + 2048)
        dx64, dwc, dbc = closed_form.layer_norm_bwd_exact(x[sl], w, g[sl], 1e-5)
        dw64 += dwc
        db64 += dbc
        parts.append(assert_close(dx[sl], dx64, what=f"exact dx rows {s}+"))
    record("C2", "dx, exact VJP vs f64", _merge(parts))
    _, mu_ref, inv_ref = ref.layer_norm_fwd(x, w, b, 1e-5)
    _, dw_ref, db_ref = ref.layer_norm_bwd(x, w, mu_ref, inv_ref, g)
    assert_reduction_close(dw, dw_ref, dw64, what="exact-mode dw")
    assert_reduction_close(db, db_ref, db64, what="exact-mode db")
