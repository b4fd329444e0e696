"""The fused norm + activation VJP (oxi_layer_norm_act_bwd, oxi_rms_norm_act_bwd)
and the graph rule that uses it.

The fused pass must give exactly what the two separate VJPs give (the
activation's VJP on the norm output, then the norm's VJP on that gradient):
the kernel recomputes the norm output with the forward's arithmetic and uses
the activation's own VJP functor, so dy, dx, dw and db are compared bit for
bit with the two-step path, which the kernel parity tests pin to the oracle.
One case per norm is also checked against the oracle directly.
"""

import sys

import numpy as np
import pytest

from conftest import assert_close, assert_sum_close, rng

pytestmark = pytest.mark.gpu

ACTS = ["gelu_tanh", "gelu_erf", "silu"]


def say(*a):
    print("[case]", *a, flush=True)
    sys.stdout.flush()


def D(hip, a):
    return hip.DeviceArray.from_numpy(np.ascontiguousarray(a, dtype=np.float32))


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


def _inputs(shape, seed):
    r = rng(seed)
    H = shape[-1]
    x = r.standard_normal(shape, dtype=np.float32)
    w = (r.standard_normal(H, dtype=np.float32) * 0.02 + 1).astype(np.float32)
    b = (r.standard_normal(H, dtype=np.float32) * 0.02).astype(np.float32)
    g = r.standard_normal(shape, dtype=np.float32)
    return x, w, b, g


LN_SHAPES = [(512, 4096), (16, 768), (7, 36), (300, 1000), (5, 8192), (33, 256), (1, 4), (2, 3, 512)]


@pytest.mark.parametrize("mode", ["ref", "exact"])
@pytest.mark.parametrize("act", ACTS)
@pytest.mark.parametrize("shape", LN_SHAPES)
def test_layer_norm_act_bwd_matches_two_vjps(hip, shape, act, mode):
    say("layer_norm_act_bwd", shape, act, mode)
    x, w, b, g = _inputs(shape, 11)
    dx_, dw_, db_, dg = D(hip, x), D(hip, w), D(hip, b), D(hip, g)
    y, mean, rstd = hip.layer_norm_fwd(dx_, dw_, db_, 1e-5)
    dy2 = _act_bwd(hip, y, dg, act)
    dx2, dw2, db2 = hip.layer_norm_bwd(dx_, dw_, mean, rstd, dy2, mode=mode)
    dy, dx, dw, db = hip.layer_norm_act_bwd(dx_, dw_, db_, mean, rstd, dg, act, mode=mode)
    _same(dy, dy2, "dy")
    _same(dx, dx2, "dx")
    _same(dw, dw2, "dw")
    _same(db, db2, "db")
    # without dy (the graph's default): the same norm gradients
    none, dx3, dw3, db3 = hip.layer_norm_act_bwd(dx_, dw_, db_, mean, rstd, dg, act, mode=mode, need_dy=False)
    assert none is None
    _same(dx3, dx2, "dx without dy")
    _same(dw3, dw2, "dw without dy")
    _same(db3, db2, "db without dy")


@pytest.mark.parametrize("mode", ["ref", "exact"])
@pytest.mark.parametrize("act", ACTS)
@pytest.mark.parametrize("shape", [(4096, 768), (9, 40), (64, 1000), (3, 8192), (1, 4)])
def test_rms_norm_act_bwd_matches_two_vjps(hip, shape, act, mode):
    say("rms_norm_act_bwd", shape, act, mode)
    x, w, _, g = _inputs(shape, 12)
    dx_, dw_, dg = D(hip, x), D(hip, w), D(hip, g)
    y, rstd = hip.rms_norm_fwd(dx_, dw_, 1e-6)
    dy2 = _act_bwd(hip, y, dg, act)
    dx2, dw2 = hip.rms_norm_bwd(dx_, dw_, rstd, dy2, mode=mode)
    dy, dx, dw = hip.rms_norm_act_bwd(dx_, dw_, rstd, dg, act, mode=mode)
    _same(dy, dy2, "dy")
    _same(dx, dx2, "dx")
    _same(dw, dw2, "dw")
    none, dx3, dw3 = hip.rms_norm_act_bwd(dx_, dw_, rstd, dg, act, mode=mode, need_dy=False)
    assert none is None
    _same(dx3, dx2, "dx without dy")
    _same(dw3, dw2, "dw without dy")


SOFTMAX_SHAPES = [(512, 768), (64, 1000), (7, 36), (33, 256), (5, 2048), (1, 4), (2, 3, 512)]


@pytest.mark.parametrize("norm", ["layer_norm", "rms_norm"])
@pytest.mark.parametrize("act", ["softmax", "log_softmax"])
@pytest.mark.parametrize("shape", SOFTMAX_SHAPES)
def test_norm_softmax_bwd_matches_two_vjps(hip, shape, act, norm):
    """softmax / log_softmax over the last dim of a norm output: the fused VJP
    recomputes the softmax as the softmax kernels do, so dy is bit-identical."""
    say("norm_act_bwd softmax", norm, shape, act)
    x, w, b, g = _inputs(shape, 15)
    dx_, dw_, db_, dg = D(hip, x), D(hip, w), D(hip, b), D(hip, g)
    if norm == "layer_norm":
        y, mean, rstd = hip.layer_norm_fwd(dx_, dw_, db_, 1e-5)
        dy2 = _act_bwd(hip, y, dg, act)
        dx2, dw2, db2 = hip.layer_norm_bwd(dx_, dw_, mean, rstd, dy2)
        dy, dx, dw, db = hip.layer_norm_act_bwd(dx_, dw_, db_, mean, rstd, dg, act)
        _same(db, db2, "db")
    else:
        y, rstd = hip.rms_norm_fwd(dx_, dw_, 1e-6)
        dy2 = _act_bwd(hip, y, dg, act)
        dx2, dw2 = hip.rms_norm_bwd(dx_, dw_, rstd, dy2)
        dy, dx, dw = hip.rms_norm_act_bwd(dx_, dw_, rstd, dg, act)
    _same(dy, dy2, "dy")
    _same(dx, dx2, "dx")
    _same(dw, dw2, "dw")


def test_norm_softmax_against_oracle(hip):
    """C5's tail, rms_norm -> softmax, at a reduced row count against the oracle."""
    from oracle import closed_form, ref
    say("rms_norm_act_bwd softmax vs oracle (256, 768)")
    x, w, _, g = _inputs((256, 768), 5)
    dx_, dw_ = D(hip, x), D(hip, w)
    y, rstd = hip.rms_norm_fwd(dx_, dw_, 1e-6)
    dy, dx, dw = hip.rms_norm_act_bwd(dx_, dw_, rstd, D(hip, g), "softmax")
    yy = y.numpy().astype(np.float64)
    p = np.exp(yy - yy.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    assert_close(dy.numpy(), p * (g - (g * p).sum(-1, keepdims=True)), what="dy")
    _, inv_ref = ref.rms_norm_fwd(x, w, 1e-6)
    dx_ref, dw_ref = ref.rms_norm_bwd(x, w, inv_ref, dy.numpy())
    assert_close(dx.numpy(), dx_ref, what="dx")
    assert_close(dw.numpy(), dw_ref, rtol=1e-4, atol=1e-4, what="dw")


def test_softmax_rows_past_2048_are_not_implemented(hip):
    say("norm_act_bwd softmax, 4096-float rows")
    x, w, b, g = _inputs((3, 4096), 16)
    dx_, dw_ = D(hip, x), D(hip, w)
    _, rstd = hip.rms_norm_fwd(dx_, dw_, 1e-6)
    with pytest.raises(NotImplementedError, match="lane layout"):
        hip.rms_norm_act_bwd(dx_, dw_, rstd, D(hip, g), "softmax")


def test_layer_norm_act_bwd_without_affine_and_partial_outputs(hip):
    say("layer_norm_act_bwd no affine / NULL outputs")
    x, _, _, g = _inputs((64, 2048), 13)
    dx_, dg = D(hip, x), D(hip, g)
    y, mean, rstd = hip.layer_norm_fwd(dx_, None, None, 1e-5)
    dy2 = _act_bwd(hip, y, dg, "gelu_erf")
    dx2, _, db2 = hip.layer_norm_bwd(dx_, None, mean, rstd, dy2, need_dw=False)
    dy, dx, dw, db = hip.layer_norm_act_bwd(dx_, None, None, mean, rstd, dg, "gelu_erf", need_dw=False)
    assert dw is None
    _same(dy, dy2, "dy")
    _same(dx, dx2, "dx")
    _same(db, db2, "db")
    # only the parameter gradient, no dy and no dx
    _, _, _, db3 = hip.layer_norm_act_bwd(dx_, None, None, mean, rstd, dg, "gelu_erf", need_dy=False,
                                          need_dx=False, need_dw=False)
    _same(db3, db2, "db alone")


def test_layer_norm_gelu_fused_against_oracle(hip):
    """C2's arithmetic at a reduced row count, checked against the oracle."""
    from oracle import closed_form, ref
    say("layer_norm_act_bwd vs oracle (256, 4096)")
    x, w, b, g = _inputs((256, 4096), 2)
    dx_, dw_, db_ = D(hip, x), D(hip, w), D(hip, b)
    y, mean, rstd = hip.layer_norm_fwd(dx_, dw_, db_, 1e-5)
    dy, dx, dw, db = hip.layer_norm_act_bwd(dx_, dw_, db_, mean, rstd, D(hip, g), "gelu_erf")
    h_ref, mu_ref, inv_ref = ref.layer_norm_fwd(x, w, b, 1e-5)
    dy_np = dy.numpy()
    assert_close(dy_np, closed_form.gelu_erf_grad(y.numpy()) * g, what="dy")
    dx_ref, dw_ref, db_ref = ref.layer_norm_bwd(x, w, mu_ref, inv_ref, dy_np)
    assert_close(dx.numpy(), dx_ref, what="dx")
    assert_close(dw.numpy(), dw_ref, rtol=1e-4, atol=1e-4, what="dw")
    assert_close(db.numpy(), db_ref, rtol=1e-4, atol=1e-4, what="db")


def test_rms_norm_silu_fused_against_oracle(hip):
    from oracle import closed_form, ref
    say("rms_norm_act_bwd vs oracle (512, 768)")
    x, w, _, g = _inputs((512, 768), 3)
    dx_, dw_ = D(hip, x), D(hip, w)
    y, rstd = hip.rms_norm_fwd(dx_, dw_, 1e-6)
    dy, dx, dw = hip.rms_norm_act_bwd(dx_, dw_, rstd, D(hip, g), "silu")
    y_ref, inv_ref = ref.rms_norm_fwd(x, w, 1e-6)
    dy_np = dy.numpy()
    assert_close(dy_np, closed_form.silu_grad(y.numpy()) * g, what="dy")
    dx_ref, dw_ref = ref.rms_norm_bwd(x, w, inv_ref, dy_np)
    assert_close(dx.numpy(), dx_ref, what="dx")
    assert_close(dw.numpy(), dw_ref, rtol=1e-4, atol=1e-4, what="dw")


def test_unvectorized_rows_are_not_implemented(hip):
    say("layer_norm_act_bwd unvectorized rows")
    for H in (770, 8196):
        x, w, b, g = _inputs((3, H), 14)
        dx_, dw_, db_ = D(hip, x), D(hip, w), D(hip, b)
        _, mean, rstd = hip.layer_norm_fwd(dx_, dw_, db_, 1e-5)
        with pytest.raises(NotImplementedError, match="do not vectorize"):
            hip.layer_norm_act_bwd(dx_, dw_, db_, mean, rstd, D(hip, g), "silu")


# ---- the graph rule ------------------------------------------------------------------------

@pytest.fixture(scope="module")
def ox(hip):
    import oxitorch_amd

    return oxitorch_amd


def _run_graph(ox, native, fuse, build, shape, seed, retain=1):
    """Builds the graph with `build`, runs backward `retain` + 1 times (the
    first ones retaining), and returns the leaf grads and the intermediate's."""
    prev = native.set_fuse_norm_act(fuse)
    try:
        x, w, b, g = _inputs(shape, seed)
        tx = ox.from_numpy(x, True)
        tw = ox.from_numpy(w, True)
        tb = ox.from_numpy(b, True)
        mid, out = build(tx, tw, tb)
        seed_t = ox.from_numpy(g)
        for _ in range(retain):
            out.backward(seed_t, retain_graph=True)
        out.backward(seed_t)
        grads = [t.grad.numpy() if t.grad is not None else None for t in (tx, tw, tb, mid)]
        return grads
    finally:
        native.set_fuse_norm_act(prev)


def _graph_cases(F):
    return {
        "ln_gelu_tanh": lambda x, w, b: (lambda y: (y, F.gelu(y)))(F.layer_norm(x, w, b)),
        "ln_gelu_erf": lambda x, w, b: (lambda y: (y, F.gelu(y, approximate="none")))(F.layer_norm(x, w, b)),
        "ln_silu": lambda x, w, b: (lambda y: (y, F.silu(y)))(F.layer_norm(x, w, b)),
        "rms_silu": lambda x, w, b: (lambda y: (y, F.silu(y)))(F.rms_norm(x, w)),
        "rms_gelu": lambda x, w, b: (lambda y: (y, F.gelu(y)))(F.rms_norm(x, w)),
        "rms_softmax": lambda x, w, b: (lambda y: (y, F.softmax(y, -1)))(F.rms_norm(x, w)),
        "ln_log_softmax": lambda x, w, b: (lambda y: (y, F.log_softmax(y, -1)))(F.layer_norm(x, w, b)),
        # y feeds two edges: the rule must not fire
        "ln_gelu_plus_y": lambda x, w, b: (lambda y: (y, F.gelu(y) + y))(F.layer_norm(x, w, b)),
    }


@pytest.mark.parametrize("shape", [(64, 768), (2, 5, 1024), (16, 4096), (3, 770)])
@pytest.mark.parametrize("case", ["ln_gelu_tanh", "ln_gelu_erf", "ln_silu", "rms_silu", "rms_gelu",
                                  "rms_softmax", "ln_log_softmax", "ln_gelu_plus_y"])
def test_graph_fusion_is_invisible(ox, case, shape):
    """Leaf gradients and the norm output's gradient are the same bits with and
    without the fused pass, through two retained backward passes and a final one."""
    from oxitorch_amd import _native
    from oxitorch_amd.nn import functional as F
    say("graph fusion", case, shape)
    build = _graph_cases(F)[case]
    before = _native.fused_norm_act_passes()
    fused = _run_graph(ox, _native, True, build, shape, 21)
    ran = _native.fused_norm_act_passes() - before
    plain = _run_graph(ox, _native, False, build, shape, 21)
    assert _native.fused_norm_act_passes() - before == ran, "fusion ran while switched off"
    softmax_too_wide = "softmax" in case and shape[-1] > 2048
    expect = 0 if (case == "ln_gelu_plus_y" or shape[-1] % 4 or softmax_too_wide) else 2
    assert ran == expect, f"fused passes {ran}, expected {expect}"
    for name, a, b in zip(["x", "w", "b", "y"], fused, plain):
        if b is None:
            assert a is None, name
            continue
        assert a.shape == b.shape, name
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"{case} {shape}: {name}.grad differs"


def test_fused_intermediate_grad_is_formed_on_read(ox):
    """The fused pass leaves the norm output's gradient unwritten; reading
    .grad forms it (the activation's VJP, and the permute's in between) with
    the node-by-node values, once; clearing or zeroing it drops the recipe,
    and the next backward replaces it."""
    from oxitorch_amd import _native
    from oxitorch_amd.nn import functional as F
    say("graph fusion: deferred intermediate gradient")
    x, w, b, g = _inputs((4, 64, 768), 25)

    def run(fuse, read_twice=False):
        prev = _native.set_fuse_norm_act(fuse)
        try:
            tx, tw, tb = (ox.from_numpy(a, True) for a in (x, w, b))
            h = F.layer_norm(tx, tw, tb)
            hp = h.permute([0, 2, 1])
            y = F.silu(hp)
            y.backward(ox.from_numpy(g.transpose(0, 2, 1).copy()))
            out = {"x": tx.grad.numpy(), "hp": hp.grad.numpy(), "h": h.grad.numpy()}
            if read_twice:
                assert np.array_equal(h.grad.numpy(), out["h"]) and np.array_equal(hp.grad.numpy(), out["hp"])
                h.grad = None
                assert h.grad is None
                hp.zero_grad()
                assert not hp.grad.numpy().any()
            return out
        finally:
            _native.set_fuse_norm_act(prev)

    before = _native.fused_norm_act_passes()
    fused = run(True, read_twice=True)
    assert _native.fused_norm_act_passes() - before == 1
    plain = run(False)
    for k in ("x", "hp", "h"):
        assert np.array_equal(fused[k].view(np.uint32), plain[k].view(np.uint32)), k


def test_graph_fusion_frees_both_vjps(ox):
    from oxitorch_amd import _native
    from oxitorch_amd.nn import functional as F
    say("graph fusion: second backward")
    prev = _native.set_fuse_norm_act(True)
    try:
        x, w, b, g = _inputs((8, 256), 22)
        y = F.gelu(F.layer_norm(ox.from_numpy(x, True), ox.from_numpy(w, True), ox.from_numpy(b, True)))
        y.backward(ox.from_numpy(g))
        with pytest.raises(ValueError, match="retain_graph"):
            y.backward(ox.from_numpy(g))
    finally:
        _native.set_fuse_norm_act(prev)


def test_graph_fusion_only_param_grads(ox):
    """x without grad: the fused pass computes dw and db (and dy) only."""
    from oxitorch_amd import _native
    from oxitorch_amd.nn import functional as F
    say("graph fusion: x without grad")
    x, w, b, g = _inputs((32, 512), 23)
    outs = []
    for fuse in (True, False):
        prev = _native.set_fuse_norm_act(fuse)
        try:
            tw, tb = ox.from_numpy(w, True), ox.from_numpy(b, True)
            F.gelu(F.layer_norm(ox.from_numpy(x), tw, tb)).backward(ox.from_numpy(g))
            outs.append((tw.grad.numpy(), tb.grad.numpy()))
        finally:
            _native.set_fuse_norm_act(prev)
    for a, b_ in zip(*outs):
        assert np.array_equal(a.view(np.uint32), b_.view(np.uint32))


@pytest.mark.parametrize("vjp", ["ref", "exact"])
def test_graph_fusion_x_grad_only_and_exact_mode(ox, vjp):
    """Only x requires grad (no parameter partials), in both VJP modes."""
    from oxitorch_amd import _native
    from oxitorch_amd.nn import functional as F
    say("graph fusion: x grad only", vjp)
    x, w, b, g = _inputs((48, 2048), 24)
    outs = []
    before = _native.fused_norm_act_passes()
    for fuse in (True, False):
        prev = _native.set_fuse_norm_act(fuse)
        try:
            tx = ox.from_numpy(x, True)
            F.silu(F.layer_norm(tx, ox.from_numpy(w), ox.from_numpy(b), vjp=vjp)).backward(ox.from_numpy(g))
            outs.append(tx.grad.numpy())
        finally:
            _native.set_fuse_norm_act(prev)
    assert _native.fused_norm_act_passes() - before == 1
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))


# ---- the leading-dim sum folded into the norm VJP ------------------------------------------

# (4, 2500, 768) and (4, 1500, 512): more positions than the softmax split's
# blocks, so its blocks take several positions each. A position's dx rows
# are staged in LDS up to 56 KB ((28, 50, 512) stages exactly 56 KB): (32,
# 40, 512) and (32, 1100, 512), 64 KB, re-read dx instead, the second with
# several positions per block
LEAD_SHAPES = [(16, 1024, 768), (4, 300, 256), (8, 64, 1024), (4, 7, 36), (12, 5, 768), (16, 3, 64), (32, 40, 512),
               (4, 2500, 768), (4, 1500, 512), (32, 1100, 512), (28, 50, 512)]


@pytest.mark.parametrize("act", ["none", "silu", "gelu_erf", "gelu_tanh", "softmax", "log_softmax"])
@pytest.mark.parametrize("norm", ["rms_norm", "layer_norm"])
@pytest.mark.parametrize("lts", LEAD_SHAPES)
def test_lead_sum_matches_vjp_and_reduce(hip, lts, norm, act):
    """dy, dx and the leading-dim sum are the bits of the separate VJP(s) and
    oxi_reduce(SUM) over dim 0; dw / db are the same column sums added in
    another row order, so they agree to the sum's conditioning."""
    lead, T, H = lts
    say("lead-sum VJP", norm, lts, act)
    x, w, b, g = _inputs((lead * T, H), 31)
    dx_, dw_, db_, dg = D(hip, x), D(hip, w), D(hip, b), D(hip, g)
    if norm == "layer_norm":
        y, mean, rstd = hip.layer_norm_fwd(dx_, dw_, db_, 1e-5)
    else:
        y, rstd = hip.rms_norm_fwd(dx_, dw_, 1e-6)
    dyv = dg if act == "none" else _act_bwd(hip, y, dg, act)
    if norm == "layer_norm":
        dx2, dw2, db2 = hip.layer_norm_bwd(dx_, dw_, mean, rstd, dyv)
        dy, dx, dw, db, ds = hip.layer_norm_bwd_lead_sum(dx_, dw_, db_, mean, rstd, dg, lead, act=act)
    else:
        dx2, dw2 = hip.rms_norm_bwd(dx_, dw_, rstd, dyv)
        dy, dx, dw, ds = hip.rms_norm_bwd_lead_sum(dx_, dw_, rstd, dg, lead, act=act)
    if act != "none":
        _same(dy, dyv, "dy")
    _same(dx, dx2, "dx")
    ds2 = hip.reduce("sum", dx2, 0, shape=(lead, T, H), x_strides=(T * H, H, 1))
    assert np.array_equal(ds.numpy().reshape(T, H).view(np.uint32), ds2.numpy().reshape(T, H).view(np.uint32)), \
        "dx_sum differs from oxi_reduce over the leading dim"
    # column sums in another order: |difference| within rtol * sum|terms|
    yv, dyn = y.numpy().astype(np.float64), dyv.numpy().astype(np.float64)
    xh = (yv - b if norm == "layer_norm" else yv) / w  # the normalised input, up to rounding
    assert_sum_close(dw.numpy(), dw2.numpy(), np.abs(dyn * xh).sum(0), what="dw")
    if norm == "layer_norm":
        assert_sum_close(db.numpy(), db2.numpy(), np.abs(dyn).sum(0), what="db")


def test_lead_sum_refusals(hip):
    say("lead-sum VJP refusals")
    for (rows, H, lead, exc) in [(3 * 4, 768, 3, NotImplementedError), (1 * 5, 768, 1, NotImplementedError),
                                 (16 * 4, 2048, 16, NotImplementedError), (30, 768, 16, ValueError)]:
        x, w, _, g = _inputs((rows, H), 32)
        dx_, dw_ = D(hip, x), D(hip, w)
        _, rstd = hip.rms_norm_fwd(dx_, dw_, 1e-6)
        with pytest.raises(exc):
            hip.rms_norm_bwd_lead_sum(dx_, dw_, rstd, D(hip, g), lead)


# ---- the graph rules on config 5's chain ------------------------------------------------------

def _c5_chain(ox, F, fuse, B, T, H, V, seed):
    from oxitorch_amd import _native
    r = rng(seed)
    Wa = r.standard_normal((V, H), dtype=np.float32)
    ids = r.integers(0, V, B * T)
    lnw, lnb, rw = (r.standard_normal(H, dtype=np.float32) for _ in range(3))
    pos = r.standard_normal((1, T, H), dtype=np.float32)
    g = r.standard_normal((B, T, H), dtype=np.float32)
    prev = _native.set_fuse_norm_act(fuse)
    try:
        n0 = _native.fused_norm_act_passes()
        W, LW, LB, RW, P = (ox.from_numpy(a, True) for a in (Wa, lnw, lnb, rw, pos))
        h = F.layer_norm(F.embedding(ids, W).reshape([B, T, H]), LW, LB)
        s = F.silu(h.permute([0, 2, 1]))
        n = F.rms_norm(s.permute([0, 2, 1]) + P, RW)
        y = F.softmax(n, -1)
        y.backward(ox.from_numpy(g))
        passes = _native.fused_norm_act_passes() - n0
        out = {"y": y.numpy(), "W": W.grad.numpy(), "lnw": LW.grad.numpy(), "lnb": LB.grad.numpy(),
               "rw": RW.grad.numpy(), "pos": P.grad.numpy(), "dn": n.grad.numpy(), "n": n.numpy(),
               "dh": h.grad.numpy(),
               "rw_value": rw}
        return out, passes
    finally:
        _native.set_fuse_norm_act(prev)


@pytest.mark.parametrize("dims", [(16, 128, 768), (4, 33, 256), (16, 1024, 768)])
def test_c5_graph_fusions(ox, dims):
    """Config 5's backward with the graph fusions (layer_norm + silu through the
    permute, rms_norm + softmax with the positional gradient) against the
    reference's node-by-node order: the same bits except rms_norm's weight
    gradient, a column sum taken in another row order."""
    from oxitorch_amd.nn import functional as F
    B, T, H = dims
    say("C5 graph fusions", dims)
    fused, passes = _c5_chain(ox, F, True, B, T, H, 5000, 41)
    plain, none = _c5_chain(ox, F, False, B, T, H, 5000, 41)
    assert passes == 2 and none == 0, (passes, none)
    for k in ("y", "W", "lnw", "lnb", "pos", "dn", "dh"):
        a, b = fused[k], plain[k]
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"{dims}: {k} differs"
    # drw = sum over rows of dn * xhat (xhat = n / rw): both sums hold the same
    # terms in another order, so they differ by at most rtol * sum |terms|
    xh = fused["n"].astype(np.float64).reshape(-1, H) / fused["rw_value"]
    terms = np.abs(fused["dn"].astype(np.float64).reshape(-1, H) * xh).sum(0)
    assert_sum_close(fused["rw"], plain["rw"], terms, what="drw")
