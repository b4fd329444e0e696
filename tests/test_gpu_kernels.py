"""Kernel-level parity: liboxihip (through its C-ABI) vs the CPU oracle.

Every test here runs the MI355X kernels and compares them with oracle.ref
(the f32 restatement of the reference CPU path) and, for long reductions and
functions the reference lacks, with oracle.closed_form (float64).
Tolerances are the north-star's: bit-exact for gathers/argmax, otherwise
rtol 1e-5 / atol 1e-6 in fp32.
"""

import sys

import numpy as np
import pytest

from conftest import (assert_close, assert_close_arb, assert_reduction_close, record, rng,
                      segmented_runs_in_one_tile)

pytestmark = pytest.mark.gpu


def say(*a):
    print("[case]", *a, flush=True)
    sys.stdout.flush()


def D(hip, a):
    return hip.DeviceArray.from_numpy(np.ascontiguousarray(a))


# ---------------------------------------------------------------------------
# RMSNorm

@pytest.mark.parametrize("shape", [(4096, 768), (7, 33), (64, 1000), (3, 5, 256), (2, 8196), (1, 4096)])
def test_rms_norm_fwd_bwd_ref(hip, shape):
    from oracle import ref, closed_form
    say("rms_norm", shape)
    r = rng(1)
    x = r.standard_normal(shape, dtype=np.float32)
    w = (r.standard_normal(shape[-1], dtype=np.float32) * 0.02 + 1).astype(np.float32)
    g = r.standard_normal(shape, dtype=np.float32)
    y, rstd = hip.rms_norm_fwd(D(hip, x), D(hip, w), 1e-6)
    y_ref, inv_ref = ref.rms_norm_fwd(x, w, 1e-6)
    assert_close(y.numpy(), y_ref, what="rms y")
    assert_close(rstd.numpy(), inv_ref, what="rms rstd")
    dx, dw = hip.rms_norm_bwd(D(hip, x), D(hip, w), rstd, D(hip, g), mode="ref")
    dx_ref, dw_ref = ref.rms_norm_bwd(x, w, inv_ref, g)
    s_dx = assert_close(dx.numpy(), dx_ref, what="rms dx(ref)")
    _, dw64 = closed_form.rms_norm_bwd_refgraph(x, w, g, 1e-6)
    s_dw = assert_reduction_close(dw.numpy(), dw_ref, dw64, what="rms dw")
    if shape == (4096, 768):  # config 1
        record("C1", "y", assert_close(y.numpy(), y_ref))
        record("C1", "dx (ref VJP)", s_dx)
        record("C1", "dw (4096-row column sums)", s_dw)


@pytest.mark.parametrize("shape", [(4096, 768), (9, 40), (5, 3000)])
def test_rms_norm_bwd_exact(hip, shape):
    from oracle import closed_form
    say("rms_norm exact", shape)
    r = rng(2)
    x = r.standard_normal(shape, dtype=np.float32)
    w = (r.standard_normal(shape[-1], dtype=np.float32) * 0.02 + 1).astype(np.float32)
    g = r.standard_normal(shape, dtype=np.float32)
    _, rstd = hip.rms_norm_fwd(D(hip, x), D(hip, w), 1e-6)
    dx, dw = hip.rms_norm_bwd(D(hip, x), D(hip, w), rstd, D(hip, g), mode="exact")
    dx64, dw64 = closed_form.rms_norm_bwd_exact(x, w, g, 1e-6)
    assert_close(dx.numpy(), dx64, what="rms dx(exact)")


# ---------------------------------------------------------------------------
# LayerNorm

@pytest.mark.parametrize("shape", [(512, 4096), (16, 768), (7, 33), (6, 1002), (3, 9000), (2, 3, 64)])
def test_layer_norm_fwd_bwd_ref(hip, shape):
    from oracle import ref, closed_form
    say("layer_norm", shape)
    r = rng(3)
    x = r.standard_normal(shape, dtype=np.float32)
    H = shape[-1]
    w = (r.standard_normal(H, dtype=np.float32) * 0.02 + 1).astype(np.float32)
    b = (r.standard_normal(H, dtype=np.float32) * 0.02).astype(np.float32)
    g = r.standard_normal(shape, dtype=np.float32)
    y, mean, rstd = hip.layer_norm_fwd(D(hip, x), D(hip, w), D(hip, b), 1e-5)
    y_ref, mu_ref, inv_ref = ref.layer_norm_fwd(x, w, b, 1e-5)
    assert_close(y.numpy(), y_ref, what="ln y")
    assert_close(mean.numpy(), mu_ref, what="ln mean")
    assert_close(rstd.numpy(), inv_ref, what="ln rstd")
    dx, dw, db = hip.layer_norm_bwd(D(hip, x), D(hip, w), mean, rstd, D(hip, g), mode="ref")
    dx_ref, dw_ref, db_ref = ref.layer_norm_bwd(x, w, mu_ref, inv_ref, g)
    assert_close(dx.numpy(), dx_ref, what="ln dx(ref)")
    _, dw64, db64 = closed_form.layer_norm_bwd_refgraph(x, w, g, 1e-5)
    assert_reduction_close(dw.numpy(), dw_ref, dw64, what="ln dw")
    assert_reduction_close(db.numpy(), db_ref, db64, what="ln db")


@pytest.mark.parametrize("shape", [(512, 4096), (5, 33), (4, 768)])
def test_layer_norm_bwd_exact(hip, shape):
    from oracle import closed_form
    say("layer_norm exact", shape)
    r = rng(4)
    x = r.standard_normal(shape, dtype=np.float32)
    H = shape[-1]
    w = (r.standard_normal(H, dtype=np.float32) * 0.02 + 1).astype(np.float32)
    b = (r.standard_normal(H, dtype=np.float32) * 0.02).astype(np.float32)
    g = r.standard_normal(shape, dtype=np.float32)
    _, mean, rstd = hip.layer_norm_fwd(D(hip, x), D(hip, w), D(hip, b), 1e-5)
    dx, _, _ = hip.layer_norm_bwd(D(hip, x), D(hip, w), mean, rstd, D(hip, g), mode="exact")
    dx64, _, _ = closed_form.layer_norm_bwd_exact(x, w, g, 1e-5)
    assert_close(dx.numpy(), dx64, what="ln dx(exact)")


def test_layer_norm_c2_full(hip):
    """Config 2 at full size: LN(affine) -> exact-erf GELU, forward + backward."""
    from oracle import ref, closed_form
    say("layer_norm+gelu C2 (16384, 4096)")
    r = rng(2)
    shape = (16384, 4096)
    x = r.standard_normal(shape, dtype=np.float32)
    w = (r.standard_normal(4096, dtype=np.float32) * 0.02 + 1).astype(np.float32)
    b = (r.standard_normal(4096, dtype=np.float32) * 0.02).astype(np.float32)
    g = r.standard_normal(shape, dtype=np.float32)
    dxx, dw_, db_ = D(hip, x), D(hip, w), D(hip, b)
    h, mean, rstd = hip.layer_norm_fwd(dxx, dw_, db_, 1e-5)
    y = hip.gelu_fwd(h, "none")
    dh = hip.gelu_bwd(h, D(hip, g), "none")
    dx, dw, db = hip.layer_norm_bwd(dxx, dw_, mean, rstd, dh, mode="ref")
    h_ref, mu_ref, inv_ref = ref.layer_norm_fwd(x, w, b, 1e-5)
    hh = h.numpy()
    record("C2", "h = layer_norm(x)", assert_close(hh, h_ref, what="C2 h"))
    record("C2", "gelu(h) vs f64", assert_close(y.numpy(), closed_form.gelu_erf(hh), what="C2 gelu(h)"))
    dh_np = dh.numpy()
    record("C2", "dh = gelu'(h) g vs f64", assert_close(dh_np, closed_form.gelu_erf_grad(hh) * g,
                                                        what="C2 gelu'(h)*g"))
    dx_ref, dw_ref, db_ref = ref.layer_norm_bwd(x, w, mu_ref, inv_ref, dh_np)
    record("C2", "dx (two VJPs)", assert_close(dx.numpy(), dx_ref, what="C2 dx"))
    _, dw64, db64 = closed_form.layer_norm_bwd_refgraph(x, w, dh_np, 1e-5)
    record("C2", "dw (16384-row sums)", assert_reduction_close(dw.numpy(), dw_ref, dw64, what="C2 dw"))
    record("C2", "db (16384-row sums)", assert_reduction_close(db.numpy(), db_ref, db64, what="C2 db"))


# ---------------------------------------------------------------------------
# Activations

@pytest.mark.parametrize("n", [4, 1, 1023, 1 << 20])
def test_gelu_tanh(hip, n):
    from oracle import ref, closed_form
    say("gelu tanh", n)
    r = rng(5)
    x = (r.standard_normal(n, dtype=np.float32) * 3).astype(np.float32)
    g = r.standard_normal(n, dtype=np.float32)
    y = hip.gelu_fwd(D(hip, x), "tanh").numpy()
    assert_close(y, ref.gelu_tanh_fwd(x), what="gelu tanh fwd vs ref")
    assert_close(y, closed_form.gelu_tanh(x), rtol=1e-5, atol=2e-6, what="gelu tanh fwd vs f64")
    d = hip.gelu_bwd(D(hip, x), D(hip, g), "tanh").numpy()
    assert_close(d, ref.gelu_tanh_bwd(x, g), what="gelu tanh bwd vs ref")


@pytest.mark.parametrize("n", [5, 4096, 1 << 20])
def test_gelu_erf(hip, n):
    from oracle import closed_form
    say("gelu erf", n)
    r = rng(6)
    x = (r.standard_normal(n, dtype=np.float32) * 3).astype(np.float32)
    g = r.standard_normal(n, dtype=np.float32)
    assert_close(hip.gelu_fwd(D(hip, x), "none").numpy(), closed_form.gelu_erf(x), what="gelu erf fwd")
    assert_close(hip.gelu_bwd(D(hip, x), D(hip, g), "none").numpy(), closed_form.gelu_erf_grad(x) * g,
                 what="gelu erf bwd")


def test_silu_contiguous(hip):
    from oracle import ref
    say("silu contiguous")
    r = rng(7)
    x = (r.standard_normal(100003, dtype=np.float32) * 4).astype(np.float32)
    g = r.standard_normal(100003, dtype=np.float32)
    assert_close(hip.silu_fwd(D(hip, x)).numpy(), ref.silu_fwd(x), what="silu fwd")
    assert_close(hip.silu_bwd(D(hip, x), D(hip, g)).numpy(), ref.silu_bwd(x, g), what="silu bwd")


@pytest.mark.parametrize("B,T,H", [(16, 1024, 768), (2, 70, 33)])
def test_silu_on_transposed_view(hip, B, T, H):
    """silu(h.permute([0,2,1])): the input is a transposed view (LDS-tiled path)."""
    from oracle import ref
    say("silu transposed", (B, T, H))
    r = rng(8)
    h = r.standard_normal((B, T, H), dtype=np.float32)
    view_shape = (B, H, T)
    view_strides = (T * H, 1, H)  # h.permute([0,2,1])
    y = hip.silu_fwd(D(hip, h), x_strides=view_strides, shape=view_shape).numpy()
    hp = np.ascontiguousarray(h.transpose(0, 2, 1))
    assert_close(y, ref.silu_fwd(hp), what="silu(view)")
    gview = r.standard_normal(view_shape, dtype=np.float32)
    d = hip.silu_bwd(D(hip, h), D(hip, gview), x_strides=view_strides, shape=view_shape).numpy()
    assert_close(d, ref.silu_bwd(hp, gview), what="silu bwd(view)")


# ---------------------------------------------------------------------------
# Softmax family

@pytest.mark.parametrize("shape,dim", [((16384, 768), -1), ((7, 33), -1), ((3, 4, 5), 1), ((2, 9000), -1),
                                       ((5, 1000), 0), ((64, 4096), -1)])
def test_softmax_log_softmax(hip, shape, dim):
    from oracle import ref, closed_form
    say("softmax", shape, dim)
    r = rng(9)
    x = (r.standard_normal(shape, dtype=np.float32) * 2).astype(np.float32)
    g = r.standard_normal(shape, dtype=np.float32)
    y = hip.softmax_fwd(D(hip, x), dim).numpy()
    assert_close(y, ref.softmax_fwd(x, dim), what="softmax")
    assert_close(y, closed_form.softmax(x, dim), what="softmax vs f64")
    d = hip.softmax_bwd(D(hip, y), D(hip, g), dim).numpy()
    assert_close_arb(d, ref.softmax_bwd(x, g, dim), closed_form.softmax_bwd(x, g, dim), what="softmax bwd")
    ly = hip.softmax_fwd(D(hip, x), dim, log=True).numpy()
    assert_close(ly, ref.log_softmax_fwd(x, dim), what="log_softmax")
    ld = hip.softmax_bwd(D(hip, ly), D(hip, g), dim, log=True).numpy()
    assert_close_arb(ld, ref.log_softmax_bwd(x, g, dim), closed_form.log_softmax_bwd(x, g, dim),
                     what="log_softmax bwd")


def test_softmax_kat_and_stability(hip):
    """Known answers of python/tests/test_nn.py:30-48."""
    say("softmax KAT")
    x = np.array([[1.0, 2.0, 3.0], [3.0, 1.0, 2.0]], np.float32)
    sm = hip.softmax_fwd(D(hip, x)).numpy()
    ref = np.exp(x) / np.exp(x).sum(-1, keepdims=True)
    assert np.allclose(sm, ref, atol=1e-6)
    big = np.array([[1000.0, 1001.0, 1002.0]], np.float32)
    ls = hip.softmax_fwd(D(hip, big), log=True).numpy()
    assert np.all(np.isfinite(ls))
    want = np.exp(np.array([1000.0, 1001.0, 1002.0]) - 1002.0)
    assert np.allclose(np.exp(ls) / np.exp(ls).sum(), want / want.sum(), atol=1e-6)


@pytest.mark.parametrize("n,c", [(2, 3), (64, 1000), (33, 31), (256, 32000)])
def test_cross_entropy(hip, n, c):
    from oracle import ref, closed_form
    say("cross_entropy", n, c)
    r = rng(10)
    logits = (r.standard_normal((n, c), dtype=np.float32) * 2).astype(np.float32)
    t = r.integers(0, c, n).astype(np.int64)
    loss, lse = hip.cross_entropy_fwd(D(hip, logits), D(hip, t))
    l = float(loss.numpy()[0])
    assert abs(l - ref.cross_entropy_fwd(logits, t)) <= 1e-5 * abs(l) + 1e-6
    assert abs(l - closed_form.cross_entropy(logits, t)) <= 1e-5 * abs(l) + 1e-6
    gl = D(hip, np.array([1.0], np.float32))
    d = hip.cross_entropy_bwd(D(hip, logits), D(hip, t), lse, gl).numpy()
    # dlogits are O(1/n): compare n * dlogits (the 1e-6 abs bound is vacuous otherwise)
    assert_close_arb(d * n, ref.cross_entropy_bwd(logits, t) * n, closed_form.cross_entropy_grad(logits, t) * n,
                     what="n*dlogits")


@pytest.mark.parametrize("n,c", [(2, 4), (64, 1000), (7, 36), (33, 8196), (256, 32000), (5, 65536), (3, 4100),
                                 (9, 8192), (4, 16388), (3, 28672), (3, 28676), (3, 32768), (3, 32772),
                                 (8192, 32000)])
def test_cross_entropy_fwd_grad_against_the_oracle(hip, n, c):
    """The forward that also writes the gradient for an upstream 1 writes the
    loss and lse of oxi_cross_entropy_fwd bit for bit, and dlogits as the
    composed log_softmax VJP forms them, (1/n)(1/s) exp(x - max) and 1/n less
    at the target: n * dlogits to the reference path's tolerance, arbitrated
    by float64, as oxi_cross_entropy_bwd(gloss = 1)'s are (every block width
    of the register-row kernel and both sides of each width's limit, C3
    included; all rows up to 2^24 elements, else 64 sampled rows)."""
    from oracle import ref, closed_form
    say("cross_entropy_fwd_grad", n, c)
    r = rng(n + c)
    logits = (r.standard_normal((n, c), dtype=np.float32) * 3).astype(np.float32)
    t = r.integers(0, c, n).astype(np.int64)
    t[0] = c - 1
    dl, dt = D(hip, logits), D(hip, t)
    loss, lse = hip.cross_entropy_fwd(dl, dt)
    d = hip.cross_entropy_bwd(dl, dt, lse, D(hip, np.ones(1, np.float32)))
    loss2, lse2, d2 = hip.cross_entropy_fwd_grad(dl, dt)
    for a, b, what in ((loss2, loss, "loss"), (lse2, lse, "lse")):
        a, b = a.numpy(), b.numpy()
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"({n}, {c}) {what} differs"
    rows = np.arange(n) if n * c <= (1 << 24) else np.sort(r.choice(n, 64, replace=False))
    want = ref.cross_entropy_bwd(logits[rows], t[rows]) * len(rows)
    exact = np.concatenate([closed_form.cross_entropy_grad(logits[rows[i:i + 16]], t[rows[i:i + 16]])
                            * len(rows[i:i + 16]) for i in range(0, len(rows), 16)])
    for what, arr in (("fwd_grad", d2), ("fwd then bwd", d)):
        assert_close_arb(arr.numpy()[rows] * n, want, exact, what=f"({n}, {c}) n*dlogits, {what}")


def _ce_special_batches(c):
    """Two-row batches, row 0 plain, row 1 special: (name, logits, targets)."""
    r = rng(c)
    out = []
    for name in ("masked logit", "masked target", "overflowing gap", "overflowing target", "all -inf", "+inf",
                 "nan"):
        x = (r.standard_normal((2, c), dtype=np.float32) * 2).astype(np.float32)
        t = np.array([3, 7], np.int64)
        row = x[1]
        if name == "masked logit":
            row[[0, c // 2, c - 1]] = -np.inf
        elif name == "masked target":
            row[7] = -np.inf
        elif name == "overflowing gap":  # x - max overflows to -inf on a non-target class
            row[5], row[c - 2] = 3e38, -3e38
        elif name == "overflowing target":
            row[5], row[7] = 3e38, -3e38
        elif name == "all -inf":
            row[:] = -np.inf
        elif name == "+inf":
            row[c // 3] = np.inf
        else:
            row[c // 3] = np.nan
        out.append((name, x, t))
    return out


@pytest.mark.parametrize("c", [1000, 1003, 65540])
def test_cross_entropy_special_values(hip, c):
    """Rows with -inf, overflowing, +inf and NaN logits give the reference's
    values: its picked log-probability is sum(onehot * log_softmax(x))
    (functional.py:287-292), so a non-target log-probability of -inf makes
    the loss NaN (0 * -inf) while the gradient stays finite; a -inf target
    gives an infinite loss; +inf, NaN and all -inf rows are NaN throughout.
    Register rows (c = 1000, with the one-pass gradient), the streaming
    kernel (1003, and 65540 float4 rows), the backward from lse."""
    from oracle import ref
    for name, x, t in _ce_special_batches(c):
        say("cross_entropy special values", c, name)
        dx, dt = D(hip, x), D(hip, t)
        loss, lse = hip.cross_entropy_fwd(dx, dt)
        paths = [("fwd then bwd", float(loss.numpy()[0]),
                  hip.cross_entropy_bwd(dx, dt, lse, D(hip, np.ones(1, np.float32))).numpy())]
        if c % 4 == 0 and c <= 65536:
            l1, _, d1 = hip.cross_entropy_fwd_grad(dx, dt)
            paths.append(("one pass", float(l1.numpy()[0]), d1.numpy()))
        want_l = ref.cross_entropy_fwd(x, t)
        want_d = ref.cross_entropy_bwd(x, t)
        for what, l, d in paths:
            tag = f"c={c} {name} {what}"
            if np.isnan(want_l):
                assert np.isnan(l), f"{tag}: loss {l}, reference NaN"
            elif np.isinf(want_l):
                assert l == want_l, f"{tag}: loss {l}, reference {want_l}"
            else:
                assert abs(l - want_l) <= 1e-5 * abs(want_l) + 1e-6, f"{tag}: loss {l} vs {want_l}"
            assert np.array_equal(np.isnan(d), np.isnan(want_d)), f"{tag}: NaN placement differs"
            assert np.array_equal(np.isinf(d), np.isinf(want_d)), f"{tag}: inf placement differs"
            ok = np.isfinite(want_d)
            # the reference adds its zero-sum residue at the argmax: compare elementwise within
            # the reference path's tolerance, n * dlogits being O(1)
            assert np.allclose(2 * d[ok], 2 * want_d[ok], rtol=1e-5, atol=1e-5), f"{tag}: dlogits differ"


def test_cross_entropy_fwd_grad_refusals(hip):
    """Rows past 65536 classes or of a class count that is not a multiple of
    4 are refused before any launch (the two-call path serves them)."""
    say("cross_entropy_fwd_grad refusals")
    for n, c in ((3, 65540), (3, 50257), (4, 10)):
        dl = D(hip, np.zeros((n, c), np.float32))
        dt = D(hip, np.zeros(n, np.int64))
        with pytest.raises(NotImplementedError, match="do not take the one-pass kernel"):
            hip.cross_entropy_fwd_grad(dl, dt)
        loss, _ = hip.cross_entropy_fwd(dl, dt)
        assert np.isclose(float(loss.numpy()[0]), np.log(c), rtol=1e-6)


def test_cross_entropy_c3_full(hip):
    """Config 3 at full size (8192, 32000): loss vs float64 over all rows, grads on a row sample."""
    from oracle import ref, closed_form
    say("cross_entropy C3 (8192, 32000)")
    r = rng(3)
    n, c = 8192, 32000
    logits = (r.standard_normal((n, c), dtype=np.float32) * 2).astype(np.float32)
    t = r.integers(0, c, n).astype(np.int64)
    dl, dt = D(hip, logits), D(hip, t)
    loss, lse = hip.cross_entropy_fwd(dl, dt)
    d = hip.cross_entropy_bwd(dl, dt, lse, D(hip, np.array([1.0], np.float32)))
    l = float(loss.numpy()[0])
    # float64 loss in row chunks
    tot = 0.0
    for s in range(0, n, 1024):
        ls = closed_form.log_softmax(logits[s:s + 1024])
        tot += ls[np.arange(ls.shape[0]), t[s:s + 1024]].sum()
    assert abs(l - (-tot / n)) <= 1e-5 * abs(l)
    rows = np.sort(r.choice(n, 64, replace=False))
    dd = d.numpy()[rows]
    want = ref.cross_entropy_bwd(logits[rows], t[rows]) * len(rows)
    exact = closed_form.cross_entropy_grad(logits[rows], t[rows]) * len(rows)
    assert_close_arb(dd * n, want, exact, what="C3 n*dlogits (sampled rows)")
    assert np.allclose(lse.numpy()[rows],
                       np.log(np.exp(logits[rows].astype(np.float64)).sum(-1)), rtol=1e-6, atol=1e-5)


# ---------------------------------------------------------------------------
# Gather / embedding

def test_index_select_kats(hip):
    """python/tests/test_smoke.py:147-149 and test_indexing_grad.py:72-89."""
    from oracle import ref
    say("index_select KAT")
    a = rng(11).standard_normal((4, 6)).astype(np.float32)
    got = hip.index_select(D(hip, a), 0, D(hip, np.array([3, 0, 2], np.int64))).numpy()
    np.testing.assert_array_equal(got, a[[3, 0, 2]])
    got = hip.index_select(D(hip, a), 1, D(hip, np.array([-1, -2], np.int64))).numpy()
    np.testing.assert_array_equal(got, a[:, [-1, -2]])
    g = np.array([[1.0, 10.0], [2.0, 20.0], [3.0, 30.0]], np.float32)
    w = hip.index_select_bwd(D(hip, g), (3, 2), 0, D(hip, np.array([1, 1, 2], np.int64))).numpy()
    np.testing.assert_array_equal(w, [[0.0, 0.0], [3.0, 30.0], [3.0, 30.0]])
    g = np.arange(1, 13, dtype=np.float32).reshape(4, 3)
    w = hip.embedding_bwd(D(hip, g), D(hip, np.array([2, 2, 0, 2], np.int64)), 4).numpy()
    want = np.zeros((4, 3), np.float32)
    want[2] = [1 + 4 + 10, 2 + 5 + 11, 3 + 6 + 12]
    want[0] = [7, 8, 9]
    np.testing.assert_array_equal(w, want)
    np.testing.assert_array_equal(ref.index_select_bwd(g, (4, 3), 0, [2, 2, 0, 2]), want)


@pytest.mark.parametrize("shape,dim,n", [((50, 8), 0, 200), ((3, 40, 5), 1, 77), ((6, 7), 1, 9),
                                         ((1000, 129), 0, 3000)])
def test_index_select_general(hip, shape, dim, n):
    from oracle import ref
    say("index_select general", shape, dim, n)
    r = rng(12)
    a = r.standard_normal(shape).astype(np.float32)
    L = shape[dim]
    idx = r.integers(-L, L, n).astype(np.int64)
    got = hip.index_select(D(hip, a), dim, D(hip, idx)).numpy()
    np.testing.assert_array_equal(got, ref.index_select(a, dim, idx))
    out_shape = list(shape)
    out_shape[dim] = n
    g = r.standard_normal(out_shape).astype(np.float32)
    grad = hip.index_select_bwd(D(hip, g), shape, dim, D(hip, idx)).numpy()
    np.testing.assert_allclose(grad, ref.index_select_bwd(g, shape, dim, idx), rtol=1e-6, atol=1e-6)


def _exact_bwd(g, shape, dim, idx):
    """float64 scatter-add: the arbiter for long duplicate sums."""
    L = shape[dim]
    keys = np.where(idx < 0, idx + L, idx)
    gm = np.moveaxis(g.astype(np.float64), dim, 0)
    out = np.zeros((L,) + gm.shape[1:])
    np.add.at(out, keys, gm)
    return np.moveaxis(out, 0, dim)


@pytest.mark.parametrize("case", ["skewed_outer", "one_key", "tile_runs", "two_hot_keys", "many_ids",
                                  "many_ids_no_long_run"])
def test_index_select_bwd_run_shapes(hip, case):
    """Runs shorter than, equal to and far longer than the VJP's position
    tiles, on the scalar path (rows not a multiple of 4 floats) with several
    outer slices, and on the vector path, below and from 65536 ids (where the
    segment kernel double-buffers its loads and the fix-up launch writes the
    zero rows, with and without long runs): values vs the oracle, long sums
    vs float64, runs inside one aligned tile bit-exact, every call
    deterministic."""
    from oracle import ref
    say("index_select_bwd runs", case)
    r = rng(21)
    if case == "skewed_outer":   # outer 4, inner 130 (scalar), 6 keys over 500 positions
        shape, dim = (4, 6, 130), 1
        idx = np.minimum(r.zipf(1.3, 500) - 1, 5).astype(np.int64)
    elif case == "one_key":      # a single key owning every position
        shape, dim = (300, 64), 0
        idx = np.full(5000, 17, np.int64)
    elif case == "tile_runs":    # runs of 10..80 positions: cut by one or several tile edges
        shape, dim = (400, 96), 0
        idx = np.repeat(r.permutation(400)[:120], r.integers(10, 81, 120)).astype(np.int64)
        r.shuffle(idx)
    elif case == "two_hot_keys":  # two hot keys plus a uniform tail, negative ids included
        shape, dim = (2000, 32), 0
        idx = np.concatenate([np.full(3000, 5), np.full(2500, -1), r.integers(-2000, 2000, 4000)]).astype(np.int64)
        r.shuffle(idx)
    elif case == "many_ids_no_long_run":  # 70000 ids over 200000 rows: no run spans three tiles,
        shape, dim = (200000, 16), 0      # so the fix-up launch only writes the zero rows
        idx = r.integers(0, 200000, 70000).astype(np.int64)
        assert np.bincount(idx).max() < 64
    else:                        # about 110k ids: runs of 1..150 positions, a hot key, negative ids
        shape, dim = (3000, 64), 0
        runs = np.repeat(r.permutation(3000)[:1200], r.integers(1, 151, 1200))
        idx = np.concatenate([runs, np.full(20000, 7), r.integers(-3000, 0, 2000)]).astype(np.int64)
        r.shuffle(idx)
        assert idx.size >= 65536
    L = shape[dim]
    out_shape = list(shape)
    out_shape[dim] = idx.size
    g = r.standard_normal(out_shape).astype(np.float32)
    dg, di = D(hip, g), D(hip, idx)
    got = hip.index_select_bwd(dg, shape, dim, di).numpy()
    again = hip.index_select_bwd(dg, shape, dim, di).numpy()
    hip.sync()
    np.testing.assert_array_equal(got, again)
    want32 = ref.index_select_bwd(g, shape, dim, idx)
    exact = _exact_bwd(g, shape, dim, idx)
    one = segmented_runs_in_one_tile(idx, L)
    gm, wm = np.moveaxis(got, dim, 0), np.moveaxis(want32, dim, 0)
    np.testing.assert_array_equal(gm[one], wm[one])
    keys = np.where(idx < 0, idx + L, idx)
    absent = np.bincount(keys, minlength=L) == 0
    np.testing.assert_array_equal(gm[absent], 0.0)
    assert_reduction_close(got, want32, exact, what=f"index_select_bwd {case}")


def test_elementwise_zero_d_operands(hip):
    """A 0-d operand has no strides: with ndim 0, NULL shape and stride arrays
    are accepted; NULL strides with ndim > 0 are refused before any launch."""
    say("elementwise 0-d")
    a, b = D(hip, np.array([3.0], np.float32)), D(hip, np.array([2.0], np.float32))
    y = hip.DeviceArray((1,))
    mul = hip.BINARY.index("mul")
    hip.call("oxi_binary", mul, a.ptr, None, b.ptr, None, y.ptr, None, None, 0)
    assert y.numpy().tolist() == [6.0]
    hip.call("oxi_unary", hip.UNARY.index("neg"), a.ptr, None, y.ptr, None, None, 0)
    assert y.numpy().tolist() == [-3.0]
    # operands sized for the shape, so that even a launch would stay in bounds
    a2, b2, y2 = D(hip, np.ones(2, np.float32)), D(hip, np.ones(2, np.float32)), hip.DeviceArray((2,))
    one, two = hip._i64arr([1]), hip._i64arr([2])
    with pytest.raises(ValueError, match="NULL input strides"):
        hip.call("oxi_binary", mul, a2.ptr, None, b2.ptr, one, y2.ptr, one, two, 1)
    with pytest.raises(ValueError, match="NULL output strides"):
        hip.call("oxi_binary", mul, a2.ptr, one, b2.ptr, one, y2.ptr, None, two, 1)


@pytest.mark.parametrize("n,V", [(16384, 50257), (16385, 50257), (1, 7), (3000, 65535), (3000, 65536),
                                 (12000, 16), (9000, 300)])
def test_index_select_bwd_sort_limits(hip, n, V):
    """Sizes around the sort's tile and table limits (16384 ids, tables of
    65535 and 65536 rows, 1 to 3 radix passes): Zipf ids with negatives
    and repeats; rows whose runs sit in one segment tile are bit-exact with
    the oracle's position-order sums, the rest within the reduction bar of
    float64; absent keys are zero; two calls agree bitwise."""
    from oracle import ref
    say("index_select_bwd sort limits", n, V)
    r = rng(n + V)
    ids = np.minimum(r.zipf(1.2, n) - 1, V - 1).astype(np.int64)
    neg = r.random(n) < 0.1
    ids[neg] -= V  # same rows, written as negatives
    Dm = 8
    g = r.standard_normal((n, Dm), dtype=np.float32)
    dg, di = D(hip, g), D(hip, ids)
    got = hip.index_select_bwd(dg, (V, Dm), 0, di).numpy()
    again = hip.index_select_bwd(dg, (V, Dm), 0, di).numpy()
    hip.sync()
    np.testing.assert_array_equal(got, again)
    keys = np.where(ids < 0, ids + V, ids)
    want32 = ref.index_select_bwd(g, (V, Dm), 0, ids)
    exact = _exact_bwd(g, (V, Dm), 0, ids)
    one = segmented_runs_in_one_tile(keys, V)
    np.testing.assert_array_equal(got[one], want32[one])
    absent = np.bincount(keys, minlength=V) == 0
    np.testing.assert_array_equal(got[absent], 0.0)
    assert_reduction_close(got, want32, exact, what=f"index_select_bwd n={n} V={V}")


@pytest.mark.parametrize("case", ["skewed_outer", "zipf_vocab", "empty"])
def test_index_select_bwd_plan_matches_one_call(hip, case):
    """The sort plan queued on the second stream, applied (twice, as a second
    backward would), equals the one-call VJP bit for bit; a plan freed
    without being applied leaves the stream usable."""
    say("index_select_bwd plan", case)
    r = rng(31)
    if case == "skewed_outer":
        shape, dim = (4, 6, 130), 1
        idx = np.minimum(r.zipf(1.3, 500) - 1, 5).astype(np.int64)
    elif case == "zipf_vocab":
        shape, dim = (50257, 64), 0
        idx = np.minimum(r.zipf(1.1, 20000) - 1, 50256).astype(np.int64)
    else:
        shape, dim = (30, 8), 0
        idx = np.zeros(0, np.int64)
    out_shape = list(shape)
    out_shape[dim] = idx.size
    g = r.standard_normal(out_shape).astype(np.float32)
    dg, di = D(hip, g), D(hip, idx) if idx.size else hip.DeviceArray((0,), np.int64)
    want = hip.index_select_bwd(dg, shape, dim, di).numpy()
    plan = hip.BwdPlan(di, shape[dim])
    first = plan.apply(dg, shape, dim).numpy()
    second = plan.apply(dg, shape, dim).numpy()
    plan.free()
    np.testing.assert_array_equal(first, want)
    np.testing.assert_array_equal(second, want)
    unused = hip.BwdPlan(di, shape[dim])
    unused.free()
    hip.sync()


@pytest.mark.parametrize("n,V", [(16384, 50257), (16385, 50257), (1, 7), (2, 1), (3000, 65535), (3000, 65536),
                                 (12000, 16), (9000, 300), (16384, 256), (5000, 257)])
def test_index_select_bwd_plan_at_sort_limits(hip, n, V):
    """The plan built on the second stream and the one-call VJP give the same
    bits around the sort's limits (tile and table sizes, 1 and 2 radix
    passes, one and two rows), with Zipf ids, repeats and negatives."""
    say("index_select_bwd plan sort", n, V)
    r = rng(7 * n + V)
    ids = np.minimum(r.zipf(1.2, n) - 1, V - 1).astype(np.int64)
    ids[r.random(n) < 0.1] -= V
    Dm = 8
    g = r.standard_normal((n, Dm), dtype=np.float32)
    dg, di = D(hip, g), D(hip, ids)
    want = hip.index_select_bwd(dg, (V, Dm), 0, di).numpy()
    plan = hip.BwdPlan(di, V)
    got = plan.apply(dg, (V, Dm), 0).numpy()
    plan.free()
    hip.sync()
    np.testing.assert_array_equal(got, want)


def _zipf_ids(seed, shape, V):
    r = rng(seed)
    return np.minimum(r.zipf(1.1, shape) - 1, V - 1).astype(np.int64)


def test_embedding_c4_full(hip):
    """Config 4: W (50257, 1024), clipped-Zipf ids (64, 2048): forward bit-exact, dW vs oracle/f64."""
    from oracle import ref, closed_form
    say("embedding C4")
    r = rng(4)
    V, Dm = 50257, 1024
    W = r.standard_normal((V, Dm), dtype=np.float32)
    ids = np.minimum(r.zipf(1.1, (64, 2048)) - 1, V - 1).astype(np.int64).ravel()
    g = r.standard_normal((ids.size, Dm), dtype=np.float32)
    dW_, dids = D(hip, W), D(hip, ids)
    out = hip.embedding_fwd(dW_, dids).numpy()
    np.testing.assert_array_equal(out, W[ids])
    record("C4", "out = W[ids] (bit-exact)", {"n": int(out.size), "worst_tol": 0.0, "arbitrated": 0})
    dg = D(hip, g)
    dW = hip.embedding_bwd(dg, dids, V).numpy()
    dW2 = hip.embedding_bwd(dg, dids, V).numpy()
    np.testing.assert_array_equal(dW, dW2)  # deterministic, bitwise
    want32 = ref.index_select_bwd(g, (V, Dm), 0, ids)
    counts = np.bincount(ids, minlength=V)
    # at C4's size the VJP cuts the sorted positions into tiles of 64: a run
    # within one tile or reaching into the next is summed by one wave in
    # position order in f32, as the reference sums it (bit-exact); a longer
    # run is summed in float64 and rounded once
    one = segmented_runs_in_one_tile(ids, V, tile=64)
    start = np.concatenate([[0], np.cumsum(counts)[:-1]])
    end = start + counts - 1
    two = (counts > 0) & ~one & (end // 64 == start // 64 + 1)
    short = one | two
    np.testing.assert_array_equal(dW[short], want32[short])
    np.testing.assert_array_equal(dW[counts == 0], 0.0)
    record("C4", f"dW rows of runs within two tiles (bit-exact; {int(two.sum())} reach the next tile)",
           {"n": int(dW[short].size), "worst_tol": 0.0, "arbitrated": 0})
    heavy = np.flatnonzero((counts > 0) & ~short)
    exact = np.zeros((heavy.size, Dm))
    for j, v in enumerate(heavy):
        exact[j] = g[ids == v].astype(np.float64).sum(0)
    # a float64 sum rounded once: within a tenth of the parity bar of the
    # exact sum, no arbitration needed
    np.testing.assert_allclose(dW[heavy], exact, rtol=1e-6, atol=1e-7)
    stats = assert_reduction_close(dW[heavy], want32[heavy], exact, what="C4 heavy dW rows")
    assert stats["arbitrated"] == 0
    record("C4", f"dW {heavy.size} rows of runs over 3+ tiles (float64 sums)", stats)
    # conservation: sum over rows of dW equals the sum of all upstream rows
    assert np.allclose(dW.astype(np.float64).sum(0), g.astype(np.float64).sum(0), rtol=1e-5, atol=1e-3)


def test_embedding_out_of_range_guard(hip):
    say("embedding guard")
    W = np.ones((5, 4), np.float32)
    ids = np.array([0, 7], np.int64)  # 7 escaped host validation
    out = hip.embedding_fwd(D(hip, W), D(hip, ids))
    with pytest.raises(RuntimeError, match="outside its valid range"):
        hip.sync()
    np.testing.assert_array_equal(out.numpy()[1], 0.0)
    hip.sync()  # the flag was cleared


# ---------------------------------------------------------------------------
# Reductions and the elementwise registry

@pytest.mark.parametrize("kind", ["sum", "mean", "max", "min", "argmax", "argmin", "norm"])
@pytest.mark.parametrize("shape,dim", [((3, 4, 5), 0), ((3, 4, 5), 1), ((3, 4, 5), 2), ((64, 300), 1),
                                       ((300, 64), 0), ((16, 8, 768), 0)])
def test_reduce(hip, kind, shape, dim):
    from oracle import ref
    say("reduce", kind, shape, dim)
    x = rng(13).standard_normal(shape).astype(np.float32)
    got = hip.reduce(kind, D(hip, x), dim).numpy()
    want = ref.reduce(kind, x, dim)
    if kind.startswith("arg"):
        np.testing.assert_array_equal(got, want)
    else:
        assert_close(got, want, rtol=2e-5, what=f"reduce {kind}")


def test_reduce_semantics_nan_ties(hip):
    """First-tie argmax (crates/oxi-tensor/src/tests.rs:188-196), NaN rules of reduce_strip."""
    say("reduce NaN/ties")
    x = np.array([[5, 7, 7], [np.nan, 1, 2], [1, np.nan, 3], [np.nan, np.nan, np.nan]] + [[2, 2, 2]] * 60, np.float32)
    am = hip.reduce("argmax", D(hip, x), 1).numpy()
    assert list(am[:5]) == [1, 0, 2, 0, 0]
    mx = hip.reduce("max", D(hip, x), 1).numpy()
    assert mx[1] == 2 and mx[2] == 3 and mx[3] == -np.inf
    xt = np.ascontiguousarray(np.tile(np.array([5, 7, 7, 1], np.float32), (64, 1)))
    np.testing.assert_array_equal(hip.reduce("argmax", D(hip, xt), 1).numpy(), 1)


@pytest.mark.parametrize("name", ["neg", "abs", "sqrt", "rsqrt", "exp", "log", "log2", "log10", "sin", "cos",
                                  "tanh", "relu", "sigmoid", "floor", "ceil", "round", "sign", "square",
                                  "reciprocal"])
def test_unary_registry(hip, name):
    from oracle import ref
    say("unary", name)
    a = rng(14).standard_normal((37, 129)).astype(np.float32)
    if name in ("sqrt", "rsqrt", "log", "log2", "log10", "reciprocal"):
        a = np.abs(a) + 0.5
    got = hip.unary(name, D(hip, a)).numpy()
    assert_close(got, ref.unary(name, a), rtol=2e-6, atol=1e-6, what=name)


@pytest.mark.parametrize("name", ["add", "sub", "mul", "div", "pow", "min", "max", "eq", "ne", "lt", "le", "gt",
                                  "ge"])
def test_binary_registry_broadcast(hip, name):
    from oracle import ref
    say("binary", name)
    r = rng(15)
    a = r.standard_normal((3, 70, 129)).astype(np.float32)
    b = r.standard_normal((70, 1)).astype(np.float32)
    if name == "pow":
        a = np.abs(a) + 0.1
    shape = (3, 70, 129)
    got = hip.binary(name, D(hip, a), D(hip, b), (70 * 129, 129, 1), (0, 1, 0), shape).numpy()
    assert_close(got, ref.binary(name, a, b), rtol=2e-6, what=name)


def test_binary_transposed_plus_broadcast(hip):
    """C5's residual add: s.permute([0,2,1]) + pos, pos (1, T, H) broadcast over batch."""
    say("binary transposed + broadcast")
    r = rng(16)
    B, T, H = 4, 130, 96
    s = r.standard_normal((B, H, T)).astype(np.float32)
    pos = r.standard_normal((1, T, H)).astype(np.float32)
    got = hip.binary("add", D(hip, s), D(hip, pos), (H * T, 1, T), (0, H, 1), (B, T, H)).numpy()
    np.testing.assert_array_equal(got, s.transpose(0, 2, 1) + pos)
