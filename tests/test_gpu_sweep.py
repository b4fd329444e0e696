"""Seeded sweep of row widths across the kernels' configuration boundaries.

The row kernels pick their launch shape from the row width: one-wave rows of
1 to 4 float4s per lane (H up to 1024 floats), 256-thread rows of 2, 4 or 8
float4s (up to 8192), 512-thread backward rows, and the looping kernels for
wider or unaligned rows. Each width below sits on, just past or just short of
one of those edges, or is not a multiple of 4; the row count of each case is
drawn from a fixed seed. Every case runs the norms, softmax / log_softmax and
cross-entropy forward and VJP against the CPU oracle (rtol 1e-5, atol 1e-6),
with float64 as the arbiter wherever a row sum enters: summed in another
order, the sum moves an output near zero by more than that bar (a
log-probability of -0.009 at a row's dominant element, -log(s) with s the
sum of 1026 exponentials, came out 2.95e-6 from the f32 oracle), so an
element outside it must be no further from float64 than the reference
path's own worst element. At every width the fused norm + activation VJPs
must give the node-by-node VJPs' bits, or refuse the width. The embedding
gather and its VJP get the same treatment over table widths and id
distributions: the gather bit-exact, each id's run that lies inside one
position tile bit-exact, absent rows +0, long sums against float64. Last,
seeded random shapes of rank 1 to 4 take every dim reduction over one dim of
a contiguous or permuted view, and every binary op over operands with
broadcast dims, fewer leading dims and a permuted storage order; softmax and
log_softmax over any dim; gelu and silu with x and g on permuted views.
"""

import sys

import numpy as np
import pytest

from conftest import assert_close, assert_close_arb, assert_reduction_close, rng, segmented_runs_in_one_tile

pytestmark = pytest.mark.gpu

# float4s per row at the launch-shape edges of the row kernels
_EDGES = (64, 128, 192, 256, 512, 1024, 2048)


def _widths():
    out = [4, 8, 12]
    for e in _EDGES:
        out += [4 * e - 4, 4 * e, 4 * e + 4, 4 * e + 2]
    return out


def _cases():
    r = rng(2024)
    return [(int(r.integers(1, 300)), H) for H in _widths()]


CASES = _cases()


def say(*a):
    print("[case]", *a, flush=True)
    sys.stdout.flush()


def D(hip, a):
    return hip.DeviceArray.from_numpy(np.ascontiguousarray(a))


def _data(seed, R, H):
    r = rng(seed)
    x = r.standard_normal((R, H), dtype=np.float32)
    w = (r.standard_normal(H, dtype=np.float32) * 0.02 + 1).astype(np.float32)
    b = (r.standard_normal(H, dtype=np.float32) * 0.02).astype(np.float32)
    g = r.standard_normal((R, H), dtype=np.float32)
    return x, w, b, g


@pytest.mark.parametrize("R,H", CASES, ids=[f"{R}x{H}" for R, H in CASES])
def test_sweep_rms_norm(hip, R, H):
    from oracle import ref, closed_form
    say("sweep rms_norm", R, H)
    x, w, _, g = _data(R * 7 + H, R, H)
    y, rstd = hip.rms_norm_fwd(D(hip, x), D(hip, w), 1e-6)
    y_ref, inv_ref = ref.rms_norm_fwd(x, w, 1e-6)
    y64, inv64 = closed_form.rms_norm_fwd(x, w, 1e-6)
    assert_close_arb(y.numpy(), y_ref, y64, what=f"rms y {R}x{H}")
    assert_close_arb(rstd.numpy(), inv_ref, inv64, what=f"rms rstd {R}x{H}")
    dx, dw = hip.rms_norm_bwd(D(hip, x), D(hip, w), rstd, D(hip, g), mode="ref")
    dx_ref, dw_ref = ref.rms_norm_bwd(x, w, inv_ref, g)
    assert_close(dx.numpy(), dx_ref, what=f"rms dx {R}x{H}")
    _, dw64 = closed_form.rms_norm_bwd_refgraph(x, w, g, 1e-6)
    assert_reduction_close(dw.numpy(), dw_ref, dw64, what=f"rms dw {R}x{H}")


@pytest.mark.parametrize("R,H", CASES, ids=[f"{R}x{H}" for R, H in CASES])
def test_sweep_layer_norm(hip, R, H):
    from oracle import ref, closed_form
    say("sweep layer_norm", R, H)
    x, w, b, g = _data(R * 11 + H, R, H)
    y, mean, rstd = hip.layer_norm_fwd(D(hip, x), D(hip, w), D(hip, b), 1e-5)
    y_ref, mu_ref, inv_ref = ref.layer_norm_fwd(x, w, b, 1e-5)
    y64, mu64, inv64 = closed_form.layer_norm_fwd(x, w, b, 1e-5)
    assert_close_arb(y.numpy(), y_ref, y64, what=f"ln y {R}x{H}")
    assert_close_arb(mean.numpy(), mu_ref, mu64, what=f"ln mean {R}x{H}")
    assert_close_arb(rstd.numpy(), inv_ref, inv64, what=f"ln rstd {R}x{H}")
    dx, dw, db = hip.layer_norm_bwd(D(hip, x), D(hip, w), mean, rstd, D(hip, g), mode="ref")
    dx_ref, dw_ref, db_ref = ref.layer_norm_bwd(x, w, mu_ref, inv_ref, g)
    assert_close(dx.numpy(), dx_ref, what=f"ln dx {R}x{H}")
    _, dw64, db64 = closed_form.layer_norm_bwd_refgraph(x, w, g, 1e-5)
    assert_reduction_close(dw.numpy(), dw_ref, dw64, what=f"ln dw {R}x{H}")
    assert_reduction_close(db.numpy(), db_ref, db64, what=f"ln db {R}x{H}")


@pytest.mark.parametrize("R,H", CASES, ids=[f"{R}x{H}" for R, H in CASES])
def test_sweep_softmax(hip, R, H):
    from oracle import ref, closed_form
    say("sweep softmax", R, H)
    x, _, _, g = _data(R * 13 + H, R, H)
    x = (x * 3).astype(np.float32)
    y = hip.softmax_fwd(D(hip, x), 1).numpy()
    assert_close_arb(y, ref.softmax_fwd(x, 1), closed_form.softmax(x, 1), what=f"softmax {R}x{H}")
    d = hip.softmax_bwd(D(hip, y), D(hip, g), 1).numpy()
    assert_close_arb(d, ref.softmax_bwd(x, g, 1), closed_form.softmax_bwd(x, g, 1), what=f"softmax bwd {R}x{H}")
    ly = hip.softmax_fwd(D(hip, x), 1, log=True).numpy()
    assert_close_arb(ly, ref.log_softmax_fwd(x, 1), closed_form.log_softmax(x, 1), what=f"log_softmax {R}x{H}")
    ld = hip.softmax_bwd(D(hip, ly), D(hip, g), 1, log=True).numpy()
    assert_close_arb(ld, ref.log_softmax_bwd(x, g, 1), closed_form.log_softmax_bwd(x, g, 1),
                     what=f"log_softmax bwd {R}x{H}")


@pytest.mark.parametrize("R,H", CASES, ids=[f"{R}x{H}" for R, H in CASES])
def test_sweep_cross_entropy(hip, R, H):
    """H classes: the loss of the forward and the gradient of the two-call
    path, as n * dlogits; where the class count is a multiple of 4, the same
    of the one-pass forward, whose loss and lse match the forward's bit for
    bit. Other class counts are refused by the one-pass entry point (the host
    core then takes the two calls)."""
    from oracle import ref, closed_form
    say("sweep cross_entropy", R, H)
    r = rng(R * 17 + H)
    logits = (r.standard_normal((R, H), dtype=np.float32) * 2).astype(np.float32)
    t = r.integers(0, H, R).astype(np.int64)
    dl, dt = D(hip, logits), D(hip, t)
    want_l = ref.cross_entropy_fwd(logits, t)
    exact_l = closed_form.cross_entropy(logits, t)
    loss, lse = hip.cross_entropy_fwd(dl, dt)
    losses = [("fwd", float(loss.numpy()[0]))]
    d2 = None
    if H % 4 == 0:
        loss2, lse2, d2 = hip.cross_entropy_fwd_grad(dl, dt)
        assert np.array_equal(loss.numpy(), loss2.numpy()), f"loss of the two forwards differ at {R}x{H}"
        assert np.array_equal(lse.numpy(), lse2.numpy()), f"lse of the two forwards differ at {R}x{H}"
    else:
        with pytest.raises(NotImplementedError, match="one-pass"):
            hip.cross_entropy_fwd_grad(dl, dt)
    for name, l in losses:
        assert abs(l - want_l) <= 1e-5 * abs(l) + 1e-6, f"{name} loss {R}x{H}: {l} vs oracle {want_l}"
        assert abs(l - exact_l) <= 1e-5 * abs(l) + 1e-6, f"{name} loss {R}x{H}: {l} vs float64 {exact_l}"
    d = hip.cross_entropy_bwd(dl, dt, lse, D(hip, np.ones(1, np.float32))).numpy()
    want_d = ref.cross_entropy_bwd(logits, t) * R
    exact_d = closed_form.cross_entropy_grad(logits, t) * R
    assert_close_arb(d * R, want_d, exact_d, what=f"n*dlogits (bwd) {R}x{H}")
    if d2 is not None:
        assert_close_arb(d2.numpy() * R, want_d, exact_d, what=f"n*dlogits (one pass) {R}x{H}")


FUSED_ACTS = ["gelu_tanh", "gelu_erf", "silu", "softmax", "log_softmax"]


def _act_bwd(hip, y, g, act):
    if act in ("softmax", "log_softmax"):
        log = act == "log_softmax"
        return hip.softmax_bwd(hip.softmax_fwd(y, log=log), g, log=log)
    if act == "silu":
        return hip.silu_bwd(y, g)
    return hip.gelu_bwd(y, g, "tanh" if act == "gelu_tanh" else "none")


def _same(a, b, what):
    a, b = a.numpy(), b.numpy()
    assert a.shape == b.shape, what
    bad = np.flatnonzero(a.view(np.uint32) != b.view(np.uint32))
    assert bad.size == 0, f"{what}: {bad.size} of {a.size} differ, first at {bad[0]}: {a.flat[bad[0]]} vs {b.flat[bad[0]]}"


@pytest.mark.parametrize("R,H", CASES, ids=[f"{R}x{H}" for R, H in CASES])
def test_sweep_fused_norm_act(hip, R, H):
    """The fused norm + activation VJPs give the node-by-node VJPs' bits
    (dy, dx, dw, db) at every width they take: a multiple of 4 floats up to
    8192, up to 2048 with a softmax. Other widths are refused."""
    say("sweep fused norm+act", R, H)
    x, w, b, g = _data(R * 19 + H, R, H)
    dx_, dw_, db_, dg = D(hip, x), D(hip, w), D(hip, b), D(hip, g)
    y, mean, rstd = hip.layer_norm_fwd(dx_, dw_, db_, 1e-5)
    yr, rstd_r = hip.rms_norm_fwd(dx_, dw_, 1e-6)
    for act in FUSED_ACTS:
        soft = act in ("softmax", "log_softmax")
        if H % 4 or H > (2048 if soft else 8192):
            with pytest.raises(NotImplementedError):
                hip.layer_norm_act_bwd(dx_, dw_, db_, mean, rstd, dg, act)
            with pytest.raises(NotImplementedError):
                hip.rms_norm_act_bwd(dx_, dw_, rstd_r, dg, act)
            continue
        dy2 = _act_bwd(hip, y, dg, act)
        dx2, dw2, db2 = hip.layer_norm_bwd(dx_, dw_, mean, rstd, dy2)
        dy, dx, dw, db = hip.layer_norm_act_bwd(dx_, dw_, db_, mean, rstd, dg, act)
        for name, a, c in (("dy", dy, dy2), ("dx", dx, dx2), ("dw", dw, dw2), ("db", db, db2)):
            _same(a, c, f"layer_norm+{act} {name} {R}x{H}")
        dyr2 = _act_bwd(hip, yr, dg, act)
        dxr2, dwr2 = hip.rms_norm_bwd(dx_, dw_, rstd_r, dyr2)
        dyr, dxr, dwr = hip.rms_norm_act_bwd(dx_, dw_, rstd_r, dg, act)
        for name, a, c in (("dy", dyr, dyr2), ("dx", dxr, dxr2), ("dw", dwr, dwr2)):
            _same(a, c, f"rms_norm+{act} {name} {R}x{H}")


def _exact_bwd(g, L, idx):
    """float64 scatter-add over dim 0: the arbiter for long duplicate sums."""
    keys = np.where(idx < 0, idx + L, idx)
    out = np.zeros((L,) + g.shape[1:])
    np.add.at(out, keys, g.astype(np.float64))
    return out


# (rows of the table, floats per row, ids, distribution): single-row tables,
# rows that do not vectorize, heavy duplicates (runs far longer than a
# position tile), tables much larger than the id count, rows past 1024 floats
EMB = [(1, 4, 50, "uniform"), (7, 3, 1000, "zipf"), (1000, 64, 3000, "uniform"), (50, 257, 2000, "zipf"),
       (3000, 256, 5000, "zipf"), (40000, 12, 20000, "uniform"), (10, 1028, 700, "uniform"),
       (5000, 768, 16384, "uniform"), (300, 1, 4000, "zipf"), (2, 4096, 65, "uniform")]


@pytest.mark.parametrize("V,Dm,n,dist", EMB, ids=[f"{V}x{Dm}-{n}-{d}" for V, Dm, n, d in EMB])
def test_sweep_embedding(hip, V, Dm, n, dist):
    from oracle import ref
    say("sweep embedding", V, Dm, n, dist)
    r = rng(V * 3 + Dm * 5 + n)
    W = r.standard_normal((V, Dm), dtype=np.float32)
    if dist == "zipf":
        ids = np.minimum(r.zipf(1.2, n) - 1, V - 1).astype(np.int64)
    else:
        ids = r.integers(-V, V, n).astype(np.int64)  # negative ids count from the end
    got = hip.index_select(D(hip, W), 0, D(hip, ids)).numpy()
    np.testing.assert_array_equal(got, ref.index_select(W, 0, ids))
    g = r.standard_normal((n, Dm), dtype=np.float32)
    dg, di = D(hip, g), D(hip, ids)
    dW = hip.index_select_bwd(dg, (V, Dm), 0, di).numpy()
    want32 = ref.index_select_bwd(g, (V, Dm), 0, ids)
    one = segmented_runs_in_one_tile(ids, V)
    np.testing.assert_array_equal(dW[one], want32[one])
    keys = np.where(ids < 0, ids + V, ids)
    absent = np.bincount(keys, minlength=V) == 0
    assert not dW[absent].any(), "rows of ids that never occur must be zero"
    assert_reduction_close(dW, want32, _exact_bwd(g, V, ids), what=f"embedding dW {V}x{Dm} n={n} {dist}")


# ---- dim reductions and the binary registry over random strided shapes -------------------------

def _red_cases():
    r = rng(77)
    out = []
    for _ in range(24):
        nd = int(r.integers(1, 5))
        shape = tuple(int(s) for s in r.integers(1, 41 if nd < 4 else 13, nd))
        out.append((shape, int(r.integers(0, nd)), bool(r.integers(0, 2))))
    return out


RED_CASES = _red_cases()


@pytest.mark.parametrize("shape,dim,permuted", RED_CASES,
                         ids=[f"{'x'.join(map(str, s))}-d{d}{'-perm' if p else ''}" for s, d, p in RED_CASES])
def test_sweep_reduce(hip, shape, dim, permuted):
    """Every reduction kind over one dim of a contiguous or permuted view:
    max, min, argmax and argmin bit-exact (first winner); sum, mean and norm
    against the oracle with float64 as the arbiter."""
    from oracle import ref
    say("sweep reduce", shape, dim, permuted)
    r = rng(sum(shape) * 31 + dim)
    nd = len(shape)
    if permuted and nd > 1:
        perm = tuple(int(p) for p in r.permutation(nd))
        base = r.standard_normal(tuple(shape[p] for p in perm)).astype(np.float32)  # stored layout
        view = base.transpose(np.argsort(perm))  # logical layout `shape`
    else:
        base = r.standard_normal(shape).astype(np.float32)
        view = base
    strides = [s // 4 for s in view.strides]
    x = np.ascontiguousarray(view)
    x64 = x.astype(np.float64)
    exact = {"sum": x64.sum(dim), "mean": x64.mean(dim), "norm": np.sqrt((x64 * x64).sum(dim))}
    for kind in ("sum", "mean", "max", "min", "argmax", "argmin", "norm"):
        got = hip.reduce(kind, D(hip, base), dim, x_strides=strides, shape=shape).numpy()
        want = ref.reduce(kind, x, dim)
        if kind in exact:
            assert_close_arb(got, want, exact[kind], what=f"reduce {kind} {shape} dim {dim}")
        else:
            np.testing.assert_array_equal(got, want, err_msg=f"reduce {kind} {shape} dim {dim}")


def _bin_cases():
    r = rng(91)
    out = []
    for _ in range(16):
        nd = int(r.integers(1, 5))
        shape = tuple(int(s) for s in r.integers(1, 31 if nd < 4 else 11, nd))
        a_keep = tuple(bool(k) for k in r.integers(0, 4, nd) > 0)  # False: size 1, broadcast
        b_keep = tuple(bool(k) for k in r.integers(0, 3, nd) > 0)
        b_lead = int(r.integers(0, nd))  # leading dims b does not have
        out.append((shape, a_keep, b_keep, b_lead, bool(r.integers(0, 2))))
    return out


BIN_CASES = _bin_cases()
BIN_OPS = ["add", "sub", "mul", "div", "pow", "min", "max", "eq", "ne", "lt", "le", "gt", "ge"]


@pytest.mark.parametrize("shape,a_keep,b_keep,b_lead,a_perm", BIN_CASES,
                         ids=[f"case{i}" for i in range(len(BIN_CASES))])
def test_sweep_binary(hip, shape, a_keep, b_keep, b_lead, a_perm):
    """Every binary op over broadcast operands: a with size-1 dims and
    optionally stored permuted, b with size-1 dims and fewer leading dims.
    Results bit-exact (IEEE add, sub, mul, correctly rounded div, min, max,
    comparisons) except pow, to 2e-6 relative."""
    from oracle import ref
    say("sweep binary", shape, a_keep, b_keep, b_lead, a_perm)
    r = rng(sum(shape) * 37 + b_lead)
    nd = len(shape)
    a_shape = tuple(s if k else 1 for s, k in zip(shape, a_keep))
    if a_perm and nd > 1:
        perm = tuple(int(p) for p in r.permutation(nd))
        a_base = r.standard_normal(tuple(a_shape[p] for p in perm)).astype(np.float32)
        a_view = a_base.transpose(np.argsort(perm))
    else:
        a_base = r.standard_normal(a_shape).astype(np.float32)
        a_view = a_base
    b_shape = tuple(s if k else 1 for s, k in zip(shape, b_keep))[b_lead:]
    b = r.standard_normal(b_shape).astype(np.float32)
    a_str = [s // 4 for s in np.broadcast_to(a_view, shape).strides]
    b_str = [s // 4 for s in np.broadcast_to(b, shape).strides]
    a_c = np.ascontiguousarray(a_view)
    da, db = D(hip, a_base), D(hip, b)
    for op in BIN_OPS:
        aa = np.abs(a_c) + 0.1 if op == "pow" else a_c
        dA = D(hip, np.abs(a_base) + 0.1) if op == "pow" else da
        got = hip.binary(op, dA, db, a_str, b_str, shape).numpy()
        # the output shape, also along dims that neither operand covers
        want = ref.binary(op, np.broadcast_to(aa, shape), np.broadcast_to(b, shape))
        if op == "pow":
            assert_close(got, want, rtol=2e-6, what=f"binary pow {shape}")
        else:
            np.testing.assert_array_equal(got, want, err_msg=f"binary {op} {shape}")


# ---- softmax over any dim, activations over permuted views ---------------------------------------

def _dim_cases():
    r = rng(113)
    out = []
    for _ in range(16):
        nd = int(r.integers(2, 5))
        shape = tuple(int(s) for s in r.integers(1, 70 if nd == 2 else (25 if nd == 3 else 12), nd))
        out.append((shape, int(r.integers(0, nd))))
    return out


DIM_CASES = _dim_cases()


@pytest.mark.parametrize("shape,dim", DIM_CASES, ids=[f"{'x'.join(map(str, s))}-d{d}" for s, d in DIM_CASES])
def test_sweep_softmax_any_dim(hip, shape, dim):
    """softmax / log_softmax over a leading, middle or last dim (inner > 1
    for all but the last), forward and VJP, arbitrated by float64."""
    from oracle import ref, closed_form
    say("sweep softmax dim", shape, dim)
    r = rng(sum(shape) * 41 + dim)
    x = (r.standard_normal(shape, dtype=np.float32) * 3).astype(np.float32)
    g = r.standard_normal(shape, dtype=np.float32)
    for log in (False, True):
        name = "log_softmax" if log else "softmax"
        y = hip.softmax_fwd(D(hip, x), dim, log=log).numpy()
        want = ref.log_softmax_fwd(x, dim) if log else ref.softmax_fwd(x, dim)
        exact = closed_form.log_softmax(x, dim) if log else closed_form.softmax(x, dim)
        assert_close_arb(y, want, exact, what=f"{name} {shape} dim {dim}")
        d = hip.softmax_bwd(D(hip, y), D(hip, g), dim, log=log).numpy()
        want_d = ref.log_softmax_bwd(x, g, dim) if log else ref.softmax_bwd(x, g, dim)
        exact_d = closed_form.log_softmax_bwd(x, g, dim) if log else closed_form.softmax_bwd(x, g, dim)
        assert_close_arb(d, want_d, exact_d, what=f"{name} bwd {shape} dim {dim}")


def _view(r, shape):
    """A permuted view of shape `shape`: (stored array, its element strides)."""
    nd = len(shape)
    perm = tuple(int(p) for p in r.permutation(nd))
    base = (r.standard_normal(tuple(shape[p] for p in perm), dtype=np.float32) * 3).astype(np.float32)
    view = base.transpose(np.argsort(perm))
    return base, view, [s // 4 for s in view.strides]


@pytest.mark.parametrize("shape,dim", DIM_CASES, ids=[f"{'x'.join(map(str, s))}-{i}" for i, (s, _) in enumerate(DIM_CASES)])
def test_sweep_activations_on_views(hip, shape, dim):
    """gelu (tanh, exact erf) and silu, forward and VJP, with x and g each a
    differently permuted view: tanh-GELU and SiLU against the oracle, the
    exact-erf GELU (which the reference lacks) against float64."""
    from oracle import ref, closed_form
    say("sweep activations on views", shape)
    r = rng(sum(shape) * 43 + dim)
    xb, xv, xs = _view(r, shape)
    gb, gv, gs = _view(r, shape)
    x, g = np.ascontiguousarray(xv), np.ascontiguousarray(gv)
    dxb, dgb = D(hip, xb), D(hip, gb)
    y = hip.gelu_fwd(dxb, "tanh", x_strides=xs, shape=shape).numpy()
    assert_close(y, ref.gelu_tanh_fwd(x), what=f"gelu tanh {shape}")
    d = hip.gelu_bwd(dxb, dgb, "tanh", x_strides=xs, g_strides=gs, shape=shape).numpy()
    assert_close(d, ref.gelu_tanh_bwd(x, g), what=f"gelu tanh bwd {shape}")
    y = hip.gelu_fwd(dxb, "none", x_strides=xs, shape=shape).numpy()
    assert_close(y, closed_form.gelu_erf(x), what=f"gelu erf {shape}")
    d = hip.gelu_bwd(dxb, dgb, "none", x_strides=xs, g_strides=gs, shape=shape).numpy()
    assert_close(d, closed_form.gelu_erf_grad(x) * g, what=f"gelu erf bwd {shape}")
    y = hip.silu_fwd(dxb, x_strides=xs, shape=shape).numpy()
    assert_close(y, ref.silu_fwd(x), what=f"silu {shape}")
    d = hip.silu_bwd(dxb, dgb, x_strides=xs, g_strides=gs, shape=shape).numpy()
    assert_close(d, ref.silu_bwd(x, g), what=f"silu bwd {shape}")
