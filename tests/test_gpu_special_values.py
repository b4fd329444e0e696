"""Special values through every floating-point op of the hot path: rows and
elements holding +-inf, NaN, +-3e38 (sums and squares that overflow), -0.0,
subnormals and all-zero rows, through the MI355X kernels (C-ABI) and the CPU
oracle (the reference's formulas in f32). The kernels must put NaN and +-inf
where the reference's own evaluation puts them; finite results are compared
at a loose tolerance, since the point here is which values come out special,
not rounding (the parity tests bound that).
"""

import sys

import numpy as np
import pytest

from conftest import rng

pytestmark = pytest.mark.gpu

INF, NAN = np.float32(np.inf), np.float32(np.nan)


def say(*a):
    print("[case]", *a, flush=True)
    sys.stdout.flush()


def D(hip, a):
    return hip.DeviceArray.from_numpy(np.ascontiguousarray(a, dtype=np.float32))


def same_specials(got, want, what, rtol=1e-4, atol=1e-5, skip=None):
    """NaN, +inf and -inf in the same places; the other values close, except
    where `skip` is set (values whose rounding the input leaves undetermined)."""
    got = np.asarray(got, np.float32)
    want = np.asarray(want, np.float32)
    assert got.shape == want.shape, f"{what}: shape {got.shape} vs {want.shape}"
    for name, f in (("NaN", np.isnan), ("+inf", np.isposinf), ("-inf", np.isneginf)):
        a, b = f(got), f(want)
        if not np.array_equal(a, b):
            i = np.flatnonzero((a != b).ravel())[0]
            raise AssertionError(f"{what}: {name} placement differs at flat {i} ({(a != b).sum()} elements): "
                                 f"got {got.ravel()[i]!r}, reference {want.ravel()[i]!r}")
    ok = np.isfinite(want)
    if skip is not None:
        ok &= ~np.asarray(skip, bool)
    scale = max(1.0, float(np.abs(want[ok]).max())) if ok.any() else 1.0
    bad = ~np.isclose(got[ok], want[ok], rtol=rtol, atol=atol * scale)
    assert not bad.any(), (f"{what}: {bad.sum()} finite values differ, e.g. got {got[ok][bad][0]!r} "
                           f"reference {want[ok][bad][0]!r}")


SPECIAL = np.array([INF, -INF, NAN, 0.0, -0.0, 3e38, -3e38, 1e-40, -1e-40, 1.0, -1.0, 10.0, -10.0, 50.0, -50.0,
                    100.0, -100.0, 1e20, -1e20, 5e-20], np.float32)


def _elementwise_inputs():
    x = np.repeat(SPECIAL, len(SPECIAL))
    g = np.tile(SPECIAL, len(SPECIAL))
    return x, g


@pytest.mark.parametrize("op", ["gelu_tanh", "gelu_erf", "silu"])
def test_activations(hip, op):
    """Every pairing of special x with special upstream g."""
    from oracle import ref
    say("special values", op)
    x, g = _elementwise_inputs()
    dx, dg = D(hip, x), D(hip, g)
    if op == "silu":
        y, gx = hip.silu_fwd(dx), hip.silu_bwd(dx, dg)
    else:
        a = "tanh" if op == "gelu_tanh" else "none"
        y, gx = hip.gelu_fwd(dx, a), hip.gelu_bwd(dx, dg, a)
    same_specials(y.numpy(), getattr(ref, op + "_fwd")(x), f"{op} forward")
    same_specials(gx.numpy(), getattr(ref, op + "_bwd")(x, g), f"{op} VJP")


def _row_cases(H):
    """(name, row) pairs: each special pattern in one row of width H."""
    r = rng(H)
    base = lambda: r.standard_normal(H, dtype=np.float32)  # noqa: E731
    cases = []
    for name in ("plain", "+inf", "-inf", "nan", "all -inf", "all zero", "3e38 pair", "1e20 element",
                 "subnormals", "-0.0 row"):
        row = base()
        if name == "+inf":
            row[H // 3] = INF
        elif name == "-inf":
            row[H // 3] = -INF
        elif name == "nan":
            row[H // 3] = NAN
        elif name == "all -inf":
            row[:] = -INF
        elif name == "all zero":
            row[:] = 0.0
        elif name == "3e38 pair":
            row[1], row[H - 2] = 3e38, -3e38
        elif name == "1e20 element":
            row[H // 2] = 1e20
        elif name == "subnormals":
            row[:] = 1e-40
        elif name == "-0.0 row":
            row[:] = -0.0
        cases.append((name, row))
    return cases


@pytest.mark.parametrize("H", [768, 4096, 1003])
def test_softmax_family(hip, H):
    """softmax / log_softmax forward and VJP, one special row at a time
    beside a plain row (the VJP with a plain upstream gradient)."""
    from oracle import ref
    r = rng(H + 1)
    for name, row in _row_cases(H):
        say("special values softmax", H, name)
        x = np.stack([r.standard_normal(H, dtype=np.float32), row])
        g = r.standard_normal(x.shape, dtype=np.float32)
        for log in (False, True):
            tag = f"{'log_' if log else ''}softmax H={H} {name}"
            y = hip.softmax_fwd(D(hip, x), log=log)
            want = (ref.log_softmax_fwd if log else ref.softmax_fwd)(x)
            same_specials(y.numpy(), want, tag + " forward")
            d = hip.softmax_bwd(y, D(hip, g), log=log).numpy()
            # the reference's max VJP adds the row's zero-sum rounding residue
            # at the argmax (its first maximum); the kernels form no residue
            arg = np.zeros(x.shape, bool)
            arg[np.arange(2), np.argmax(np.where(np.isnan(x), -np.inf, x), axis=1)] = True
            same_specials(d, (ref.log_softmax_bwd if log else ref.softmax_bwd)(x, g), tag + " VJP", skip=arg)


@pytest.mark.parametrize("H", [768, 4096, 1003])
@pytest.mark.parametrize("kind", ["rms_norm", "layer_norm"])
def test_norms(hip, kind, H):
    """Norm forward and VJP (dx, and the column sums dw/db over the two
    rows), one special row at a time beside a plain row."""
    from oracle import ref
    r = rng(H + 2)
    w = (r.standard_normal(H, dtype=np.float32) * 0.02 + 1).astype(np.float32)
    b = (r.standard_normal(H, dtype=np.float32) * 0.02).astype(np.float32)
    for name, row in _row_cases(H):
        say("special values", kind, H, name)
        x = np.stack([r.standard_normal(H, dtype=np.float32), row])
        g = r.standard_normal(x.shape, dtype=np.float32)
        tag = f"{kind} H={H} {name}"
        dxx, dw_, dg = D(hip, x), D(hip, w), D(hip, g)
        if kind == "rms_norm":
            y, rstd = hip.rms_norm_fwd(dxx, dw_)
            wy, winv = ref.rms_norm_fwd(x, w)
            same_specials(y.numpy(), wy, tag + " y")
            same_specials(rstd.numpy(), winv, tag + " rstd")
            dx, dw = hip.rms_norm_bwd(dxx, dw_, rstd, dg)
            wdx, wdw = ref.rms_norm_bwd(x, w, winv, g)
            same_specials(dx.numpy(), wdx, tag + " dx")
            same_specials(dw.numpy(), wdw, tag + " dw")
        else:
            db_ = D(hip, b)
            y, mean, rstd = hip.layer_norm_fwd(dxx, dw_, db_)
            wy, wmean, winv = ref.layer_norm_fwd(x, w, b)
            same_specials(y.numpy(), wy, tag + " y")
            # +-3e38 cancel in the mean, and which small values they absorbed
            # depends on the summation order: only its specials are determined
            same_specials(mean.numpy(), wmean, tag + " mean", skip=np.array([False, name == "3e38 pair"]))
            same_specials(rstd.numpy(), winv, tag + " rstd")
            dx, dw, db = hip.layer_norm_bwd(dxx, dw_, mean, rstd, dg)
            wdx, wdw, wdb = ref.layer_norm_bwd(x, w, wmean, winv, g)
            same_specials(dx.numpy(), wdx, tag + " dx")
            same_specials(dw.numpy(), wdw, tag + " dw")
            same_specials(db.numpy(), wdb, tag + " db")


def same_bits(got, want, what):
    """Bit for bit, any NaN matching any NaN."""
    got = np.ascontiguousarray(got, np.float32)
    want = np.ascontiguousarray(want, np.float32)
    nan = np.isnan(got)
    assert np.array_equal(nan, np.isnan(want)), f"{what}: NaN placement differs"
    diff = got.view(np.uint32)[~nan] != want.view(np.uint32)[~nan]
    assert not diff.any(), f"{what}: {diff.sum()} elements differ, e.g. {got[~nan][diff][0]!r} vs {want[~nan][diff][0]!r}"


@pytest.mark.parametrize("H", [768, 4096])
@pytest.mark.parametrize("kind", ["rms_norm", "layer_norm"])
@pytest.mark.parametrize("act", ["gelu_erf", "gelu_tanh", "silu", "softmax", "log_softmax"])
def test_fused_norm_act_matches_node_by_node(hip, kind, act, H):
    """The one-pass norm + activation VJP gives the node-by-node kernels'
    bits (dy, dx, dw, db) on rows holding special values."""
    r = rng(H + 3)
    w = D(hip, (r.standard_normal(H, dtype=np.float32) * 0.02 + 1).astype(np.float32))
    b = D(hip, (r.standard_normal(H, dtype=np.float32) * 0.02).astype(np.float32))
    for name, row in _row_cases(H):
        say("special values fused", kind, act, H, name)
        x = D(hip, np.stack([r.standard_normal(H, dtype=np.float32), row]))
        g = D(hip, r.standard_normal((2, H), dtype=np.float32))
        if kind == "rms_norm":
            h, rstd = hip.rms_norm_fwd(x, w)
        else:
            h, mean, rstd = hip.layer_norm_fwd(x, w, b)
        if act in ("softmax", "log_softmax"):
            dh = hip.softmax_bwd(hip.softmax_fwd(h, log=act == "log_softmax"), g, log=act == "log_softmax")
        elif act == "silu":
            dh = hip.silu_bwd(h, g)
        else:
            dh = hip.gelu_bwd(h, g, "tanh" if act == "gelu_tanh" else "none")
        tag = f"{kind}+{act} H={H} {name}"
        if act in ("softmax", "log_softmax") and H > 1024:
            # the fused softmax VJP takes one-wave rows; wider ones are refused
            # before any launch and the graph runs the two VJPs
            with pytest.raises(NotImplementedError, match="run the two VJPs"):
                if kind == "rms_norm":
                    hip.rms_norm_act_bwd(x, w, rstd, g, act)
                else:
                    hip.layer_norm_act_bwd(x, w, b, mean, rstd, g, act)
            continue
        if kind == "rms_norm":
            want = (dh, *hip.rms_norm_bwd(x, w, rstd, dh))
            got = hip.rms_norm_act_bwd(x, w, rstd, g, act)
        else:
            want = (dh, *hip.layer_norm_bwd(x, w, mean, rstd, dh))
            got = hip.layer_norm_act_bwd(x, w, b, mean, rstd, g, act)
        for part, a, c in zip(("dy", "dx", "dw", "db"), got, want):
            same_bits(a.numpy(), c.numpy(), f"{tag} {part}")


REGISTRY_X = np.concatenate([SPECIAL, np.array([0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 0.49999997, 8388609.0, 2.0, -3.0,
                                                 0.25, 88.8, -104.0], np.float32)])


def test_unary_registry(hip):
    """Every unary op of the registry on special and boundary inputs (half
    integers for round, exp's overflow and underflow edges, logs and roots
    of negatives and zeros)."""
    from oracle import ref
    x = REGISTRY_X
    dx = D(hip, x)
    for name in hip.UNARY:
        if name not in ref.UNARY:
            continue
        say("special values unary", name)
        same_specials(hip.unary(name, dx).numpy(), ref.unary(name, x), f"unary {name}")


def test_binary_registry(hip):
    """Every binary op of the registry on all pairs of special inputs (pow's
    special cases, min/max and comparisons with NaN, signed zeros)."""
    from oracle import ref
    a = np.repeat(REGISTRY_X, len(REGISTRY_X))
    b = np.tile(REGISTRY_X, len(REGISTRY_X))
    da, db = D(hip, a), D(hip, b)
    st = hip.row_major_strides(a.shape)
    for name in hip.BINARY:
        if name not in ref.BINARY:
            continue
        say("special values binary", name)
        same_specials(hip.binary(name, da, db, st, st, a.shape).numpy(), ref.binary(name, a, b), f"binary {name}")


@pytest.mark.parametrize("kind", ["rms_norm", "layer_norm"])
@pytest.mark.parametrize("act", ["none", "softmax", "log_softmax", "silu", "gelu_tanh"])
def test_lead_sum_matches_node_by_node(hip, kind, act):
    """The norm VJP that also sums dx over the leading dim (the positional
    gradient of x + pos): dy, dx and the sum give the node-by-node kernels'
    bits (the sum is the reduce over dim 0) on (4, 8, 768) inputs with one
    special row; dw/db (another row order) the same specials."""
    lead, T, H = 4, 8, 768
    r = rng(7)
    w = D(hip, (r.standard_normal(H, dtype=np.float32) * 0.02 + 1).astype(np.float32))
    b = D(hip, (r.standard_normal(H, dtype=np.float32) * 0.02).astype(np.float32))
    for name, row in _row_cases(H):
        say("special values lead sum", kind, act, name)
        xa = r.standard_normal((lead, T, H), dtype=np.float32)
        xa[2, 5] = row
        x = D(hip, xa)
        g = D(hip, r.standard_normal((lead, T, H), dtype=np.float32))
        if kind == "rms_norm":
            h, rstd = hip.rms_norm_fwd(x, w)
        else:
            h, mean, rstd = hip.layer_norm_fwd(x, w, b)
        if act in ("softmax", "log_softmax"):
            log = act == "log_softmax"
            dh = hip.softmax_bwd(hip.softmax_fwd(h, log=log), g, log=log)
        elif act == "silu":
            dh = hip.silu_bwd(h, g)
        elif act == "gelu_tanh":
            dh = hip.gelu_bwd(h, g, "tanh")
        else:
            dh = g
        tag = f"{kind}+{act} lead sum {name}"
        if kind == "rms_norm":
            dx, dw = hip.rms_norm_bwd(x, w, rstd, dh)
            wants = {"dx": dx, "dw": dw}
            dy1, dx1, dw1, ds1 = hip.rms_norm_bwd_lead_sum(x, w, rstd, g, lead, act=act)
            gots = {"dx": dx1, "dw": dw1}
        else:
            dx, dw, db = hip.layer_norm_bwd(x, w, mean, rstd, dh)
            wants = {"dx": dx, "dw": dw, "db": db}
            dy1, dx1, dw1, db1, ds1 = hip.layer_norm_bwd_lead_sum(x, w, b, mean, rstd, g, lead, act=act)
            gots = {"dx": dx1, "dw": dw1, "db": db1}
        if act != "none":
            same_bits(dy1.numpy(), dh.numpy(), f"{tag} dy")
        same_bits(gots["dx"].numpy(), wants["dx"].numpy(), f"{tag} dx")
        same_bits(ds1.numpy().reshape(T, H), hip.reduce("sum", wants["dx"], 0).numpy().reshape(T, H), f"{tag} sum")
        for part in ("dw", "db"):
            if part in gots:
                same_specials(gots[part].numpy(), wants[part].numpy(), f"{tag} {part}")


@pytest.mark.parametrize("opt", ["sgd", "sgd_nesterov", "adamw", "adam"])
def test_optimizer_steps(hip, opt):
    """Two optimizer steps over every pairing of special parameter value and
    special gradient (the state then holds specials too): parameters and
    state as the oracle's steps leave them."""
    from oracle import ref
    say("special values", opt)
    p0 = np.repeat(REGISTRY_X, len(REGISTRY_X))
    g = np.tile(REGISTRY_X, len(REGISTRY_X))
    p, st1, st2 = p0.copy(), np.zeros_like(p0), np.zeros_like(p0)
    dp, dg, d1, d2 = D(hip, p0), D(hip, g), D(hip, st1), D(hip, st2)
    for t in (1, 2):
        if opt.startswith("sgd"):
            nest = opt == "sgd_nesterov"
            p = ref.sgd_step(p, g, st1, 0.1, momentum=0.9, nesterov=nest)
            dp = hip.sgd_step(dp, dg, d1, 0.1, momentum=0.9, nesterov=nest)
        else:
            dec = opt == "adamw"
            p = ref.adamw_step(p, g, st1, st2, t, 1e-3, weight_decay=0.01, decoupled=dec)
            dp = hip.adamw_step(dp, dg, d1, d2, t, 1e-3, weight_decay=0.01, decoupled=dec)
        same_specials(dp.numpy(), p, f"{opt} step {t} parameters")
        same_specials(d1.numpy(), st1, f"{opt} step {t} first state")
        if not opt.startswith("sgd"):
            same_specials(d2.numpy(), st2, f"{opt} step {t} second state")


def test_embedding_vjp_sums(hip):
    """Gradient rows holding NaN and +-inf summed into shared ids (and ids
    seen once): the table's rows as the oracle's position-order sums."""
    from oracle import ref
    say("special values embedding VJP")
    r = rng(31)
    V, H = 64, 96
    ids = np.array([3, 5, 3, 7, 3, 9, 5, 11, 3, 3, 12, 13] * 4, np.int64)
    g = r.standard_normal((len(ids), H), dtype=np.float32)
    g[0, 4], g[2, 4] = INF, -INF      # +inf + -inf in id 3: NaN
    g[1, 7] = NAN                     # NaN in id 5
    g[3, 9], g[15, 9] = INF, INF      # +inf twice in id 7
    g[5, :] = 3e38                    # one row, id 9, four times: overflows
    gw = hip.embedding_bwd(D(hip, g), hip.DeviceArray.from_numpy(ids), V).numpy()
    same_specials(gw, ref.index_select_bwd(g, (V, H), 0, ids), "embedding VJP")
