"""Pins the CPU oracle (oracle/refcpu.c + oracle/closed_form.py) before it is
trusted as the parity checker. CPU only.

Each function of the oracle is checked against at least one of:
  * the reference's own known-answer tests (python/tests/*.py, crates/*/tests.rs),
    restated here with their file:line;
  * the float64 closed form (which itself is checked against finite
    differences and invariants);
  * finite-difference gradient checks with the reference's gradcheck
    parameters (h = 1e-2, tol 1e-3 * max(1, |g|): crates/oxi-autograd/src/gradcheck.rs:30-62);
  * invariants (softmax rows sum to 1, dW conservation, ...).
The `planted` tests put a plausible mistake into a copy of an oracle function
and show that the checks above reject it.
"""

import numpy as np
import pytest

from conftest import rng
from oracle import closed_form as cf
from oracle import ref

# ---------------------------------------------------------------------------
# Known-answer tests of the reference


def test_kat_softmax_log_softmax():
    """python/tests/test_nn.py:30-48."""
    x = np.array([[1.0, 2.0, 3.0], [3.0, 1.0, 2.0]], np.float32)
    sm = ref.softmax_fwd(x)
    want = np.exp(x) / np.exp(x).sum(-1, keepdims=True)
    assert np.allclose(sm, want, atol=1e-6)
    ls = ref.log_softmax_fwd(x)
    assert np.allclose(np.exp(ls).sum(-1), 1.0, atol=1e-6)
    big = np.array([[1000.0, 1001.0, 1002.0]], np.float32)
    ls = ref.log_softmax_fwd(big)
    assert np.all(np.isfinite(ls))
    w = np.exp(np.array([1000.0, 1001.0, 1002.0]) - 1002.0)
    assert np.allclose(np.exp(ls) / np.exp(ls).sum(), w / w.sum(), atol=1e-6)


def test_kat_activations():
    """python/tests/test_nn.py:51-60 (silu, tanh-gelu at [-1, 0, 1, 2])."""
    x = np.array([-1.0, 0.0, 1.0, 2.0], np.float32)
    r = x.astype(np.float64)
    assert np.allclose(ref.silu_fwd(x), r / (1 + np.exp(-r)), atol=1e-6)
    c = np.sqrt(2 / np.pi)
    assert np.allclose(ref.gelu_tanh_fwd(x), 0.5 * r * (1 + np.tanh(c * (r + 0.044715 * r ** 3))), atol=1e-5)
    assert np.allclose(ref.unary("sigmoid", x), 1 / (1 + np.exp(-r)), atol=1e-6)
    assert np.allclose(ref.unary("tanh", x), np.tanh(r), atol=1e-6)
    assert np.allclose(ref.unary("relu", x), np.maximum(r, 0), atol=1e-7)


def test_kat_layer_norm_and_rms_values():
    """python/tests/test_nn.py:63-72 and :81-87."""
    x = np.array([[1.0, 2.0, 3.0], [4.0, 5.0, 6.0]], np.float32)
    y, _, _ = ref.layer_norm_fwd(x, np.ones(3, np.float32), np.zeros(3, np.float32), 1e-5)
    mu = x.mean(-1, keepdims=True)
    v = ((x - mu) ** 2).mean(-1, keepdims=True)
    assert np.allclose(y, (x - mu) / np.sqrt(v + 1e-5), rtol=1e-4, atol=1e-5)
    x = np.array([[1.0, -2.0, 3.0]], np.float32)
    w = np.array([1.0, 2.0, 0.5], np.float32)
    y, _ = ref.rms_norm_fwd(x, w, 1e-6)
    assert np.allclose(y, x / np.sqrt((x ** 2).mean(-1, keepdims=True) + 1e-6) * w, rtol=1e-4, atol=1e-5)


def test_kat_layer_norm_grads_nonzero():
    """python/tests/test_nn.py:73-78: weighted-sum backward gives a nonzero x grad."""
    x = np.array([[1.0, 2.0, 3.0], [4.0, 5.0, 6.0]], np.float32)
    coef = np.array([[1.0, -2.0, 0.5], [0.25, 1.0, -1.0]], np.float32)
    _, mu, inv = ref.layer_norm_fwd(x, np.ones(3, np.float32), np.zeros(3, np.float32), 1e-5)
    dx, dw, db = ref.layer_norm_bwd(x, np.ones(3, np.float32), mu, inv, coef)
    assert np.abs(dx).sum() > 1e-6
    assert np.allclose(db, coef.sum(0))


def test_kat_embedding_and_index_select():
    """python/tests/test_nn.py:90-96, test_indexing_grad.py:72-108, test_smoke.py:147-149,
    crates/oxi-tensor/src/tests.rs:346-355, crates/oxi-autograd/src/tests.rs:341-353."""
    w = np.array([[1.0, 1.0], [2.0, 2.0], [3.0, 3.0]], np.float32)
    out = ref.index_select(w, 0, [2, 0, 2])
    np.testing.assert_array_equal(out, [[3, 3], [1, 1], [3, 3]])
    g = ref.index_select_bwd(np.ones((3, 2), np.float32), (3, 2), 0, [2, 0, 2])
    np.testing.assert_array_equal(g, [[1, 1], [0, 0], [2, 2]])
    g = ref.index_select_bwd(np.array([[1, 10], [2, 20], [3, 30]], np.float32), (3, 2), 0, [1, 1, 2])
    np.testing.assert_array_equal(g, [[0, 0], [3, 30], [3, 30]])
    g = ref.index_select_bwd(np.arange(1, 13, dtype=np.float32).reshape(4, 3), (4, 3), 0, [2, 2, 0, 2])
    want = np.zeros((4, 3), np.float32)
    want[2] = [15, 18, 21]
    want[0] = [7, 8, 9]
    np.testing.assert_array_equal(g, want)
    a = np.arange(9, dtype=np.float32).reshape(3, 3)
    np.testing.assert_array_equal(ref.index_select(a, 0, [2, 1, 1]), a[[2, 1, 1]])
    np.testing.assert_array_equal(ref.index_select_bwd(np.ones((3, 3), np.float32), (3, 3), 0, [2, 1, 1]),
                                  [[0, 0, 0], [2, 2, 2], [1, 1, 1]])
    t = np.array([[1.0, 2.0], [3.0, 4.0]], np.float32)
    np.testing.assert_array_equal(ref.index_select_bwd(np.array([[5, 5], [6, 6]], np.float32), (2, 2), 0, [1, 1]),
                                  [[0, 0], [11, 11]])
    np.testing.assert_array_equal(ref.index_select(t, 0, [1, 1]), [[3, 4], [3, 4]])
    b = np.array([[1.0, 2.0], [3.0, 4.0], [5.0, 6.0]], np.float32)
    np.testing.assert_array_equal(ref.index_select(b, 0, [2, 0]), [[5, 6], [1, 2]])
    np.testing.assert_array_equal(ref.index_select(b, 0, [-1]), [[5, 6]])
    with pytest.raises(IndexError):
        ref.index_select(b, 0, [3])
    a = rng(11).standard_normal((4, 6)).astype(np.float32)
    np.testing.assert_array_equal(ref.index_select(a, 0, [3, 0, 2]), a[[3, 0, 2]])
    np.testing.assert_array_equal(ref.index_select(a, 1, [-1, -2]), a[:, [-1, -2]])
    g = ref.index_select_bwd(np.array([[1, 2, 3], [4, 5, 6]], np.float32), (3, 3), 0, [1, 1])
    np.testing.assert_array_equal(g[1], [5, 7, 9])


def test_kat_cross_entropy():
    """python/tests/test_nn.py:111-122."""
    lg = np.array([[1.0, 2.0, 3.0], [3.0, 1.0, 2.0]], np.float32)
    loss = ref.cross_entropy_fwd(lg, [2, 0])
    m = lg.max(-1, keepdims=True)
    ls = lg - m - np.log(np.exp(lg - m).sum(-1, keepdims=True))
    assert abs(loss - (-np.mean([ls[0, 2], ls[1, 0]]))) < 1e-5
    g = ref.cross_entropy_bwd(lg, [2, 0])
    want = (np.exp(ls) - np.eye(3, dtype=np.float32)[[2, 0]]) / 2
    assert np.allclose(g, want, rtol=1e-4, atol=1e-6)


def test_cross_entropy_masked_logits_follow_the_onehot_product():
    """The reference picks ls[i, t] as sum(onehot * ls) (functional.py:287-292):
    a -inf logit at a non-target class gives 0 * -inf = NaN in that sum, so
    the loss is NaN, while a -inf target alone gives +inf; the gradient's
    onehot factor stays finite either way (it is g * onehot). An oracle that
    read ls[i, t] directly would give a finite loss for the first case."""
    lg = np.array([[1.0, 2.0, 3.0, 0.5], [3.0, 1.0, 2.0, 0.0]], np.float32)
    t = [2, 0]
    base = ref.cross_entropy_fwd(lg, t)
    assert np.isfinite(base)
    masked = lg.copy()
    masked[1, 3] = -np.inf
    assert np.isnan(ref.cross_entropy_fwd(masked, t))
    g = ref.cross_entropy_bwd(masked, t)
    assert np.isfinite(g).all() and g[1, 3] == 0.0
    masked_t = lg.copy()
    masked_t[1, 0] = -np.inf
    assert ref.cross_entropy_fwd(masked_t, t) == np.inf
    # x - max overflowing to -inf acts as a -inf logit
    far = lg.copy()
    far[1, 2], far[1, 3] = 3e38, -3e38
    assert np.isnan(ref.cross_entropy_fwd(far, t))


def test_kat_reductions():
    """crates/oxi-tensor/src/ops.rs:370-381, tests.rs:180-196, python/tests/test_smoke.py:107-121."""
    d = np.array([[1.0, 2.0, 3.0, 4.0]], np.float32)
    assert ref.reduce("sum", d, 1)[0] == 10.0
    assert ref.reduce("mean", d, 1)[0] == 2.5
    assert ref.reduce("max", d, 1)[0] == 4.0
    assert ref.reduce("min", d, 1)[0] == 1.0
    assert ref.reduce("argmax", d, 1)[0] == 3.0
    assert ref.reduce("argmin", d, 1)[0] == 0.0
    assert ref.reduce("norm", np.array([[3.0, 4.0]], np.float32), 1)[0] == 5.0
    assert ref.reduce("sum", np.zeros((1, 0), np.float32), 1)[0] == 0.0
    with pytest.raises(ValueError):
        ref.reduce("max", np.zeros((1, 0), np.float32), 1)
    a = np.array([[5.0, 7.0, 7.0], [1.0, 9.0, 2.0]], np.float32)
    np.testing.assert_array_equal(ref.reduce("argmax", a, -1), [1.0, 1.0])
    np.testing.assert_array_equal(ref.reduce("argmin", a, 1), [0.0, 0.0])
    c = np.array([[1.0, 2.0], [3.0, 4.0], [5.0, 6.0]], np.float32)
    np.testing.assert_array_equal(ref.reduce("sum", c, 0), [9.0, 12.0])
    a = rng(0).standard_normal((3, 4, 5)).astype(np.float32)
    np.testing.assert_allclose(ref.reduce("sum", a, 0), a.sum(0), rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(ref.reduce("sum", a, -1), a.sum(-1), rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(ref.reduce("mean", a, 1), a.mean(1), rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(ref.reduce("max", a, 0), a.max(0))
    np.testing.assert_allclose(ref.reduce("min", a, 2), a.min(2))
    np.testing.assert_array_equal(ref.reduce("argmax", a, -1), a.argmax(-1))
    np.testing.assert_array_equal(ref.reduce("argmin", a, 1), a.argmin(1))
    np.testing.assert_allclose(ref.reduce("norm", a, -1), np.linalg.norm(a, axis=-1), rtol=1e-5, atol=1e-6)


def test_kat_registry():
    """crates/oxi-tensor/src/ops.rs:361-367 and python/tests/test_smoke.py:59-94 (rtol 1e-5, atol 1e-8)."""
    assert ref.binary("pow", np.array([2.0], np.float32), np.array([10.0], np.float32))[0] == 1024.0
    assert ref.binary("ge", np.array([2.0], np.float32), np.array([2.0], np.float32))[0] == 1.0
    assert ref.unary("relu", np.array([-3.0], np.float32))[0] == 0.0
    assert ref.unary("sigmoid", np.array([0.0], np.float32))[0] == 0.5
    a = rng(1).standard_normal((3, 4)).astype(np.float32)
    b = rng(2).standard_normal(4).astype(np.float32)
    r = np.abs(a) + 0.5
    np_un = {"neg": (a, -a), "abs": (a, np.abs(a)), "sqrt": (r, np.sqrt(r)), "exp": (a * 0.1, np.exp(a * 0.1)),
             "log": (r, np.log(r)), "sin": (a, np.sin(a)), "cos": (a, np.cos(a)), "tanh": (a, np.tanh(a)),
             "relu": (a, np.maximum(a, 0)), "sigmoid": (a, 1 / (1 + np.exp(-a))), "floor": (a, np.floor(a)),
             "ceil": (a, np.ceil(a)), "round": (a, np.round(a)), "square": (a, a * a),
             "reciprocal": (r, 1 / r)}
    for name, (inp, want) in np_un.items():
        np.testing.assert_allclose(ref.unary(name, inp), want, rtol=1e-5, atol=1e-8, err_msg=name)
    np_bin = {"add": a + b, "sub": a - b, "mul": a * b, "div": a / b, "min": np.minimum(a, b),
              "max": np.maximum(a, b), "eq": a == b, "ne": a != b, "lt": a < b, "le": a <= b, "gt": a > b,
              "ge": a >= b}
    for name, want in np_bin.items():
        np.testing.assert_allclose(ref.binary(name, a, b), want, rtol=1e-5, atol=1e-8, err_msg=name)


def test_kat_rsqrt_and_round():
    """rsqrt is `1.0 / a.sqrt()` (crates/oxi-tensor/src/ops.rs:138-141): an f32
    square root, then an f32 division, each correctly rounded, so NumPy's f32
    ops give its bits (an approximate reciprocal square root would not).
    round is f32::round (ops.rs:186-188): halves go away from zero, where
    np.round and rint go to even."""
    r = np.abs(rng(3).standard_normal(4096)).astype(np.float32) * np.float32(100)
    r = np.concatenate([r, np.array([4.0, 0.25, 1e-30, 3e38, 1.0, 2.0], np.float32)])
    want = np.float32(1.0) / np.sqrt(r)
    assert np.array_equal(ref.unary("rsqrt", r).view(np.uint32), want.view(np.uint32))
    sp = ref.unary("rsqrt", np.array([0.0, -0.0, -1.0, np.inf], np.float32))
    assert sp[0] == np.inf and sp[1] == -np.inf and np.isnan(sp[2]) and sp[3] == 0.0
    half = np.array([0.5, -0.5, 1.5, -1.5, 2.5, -2.5, 3.5, 4194304.5, 0.49999997, -0.49999997, 2.4999998,
                     -0.0, 8388609.0], np.float32)
    away = np.array([1.0, -1.0, 2.0, -2.0, 3.0, -3.0, 4.0, 4194305.0, 0.0, -0.0, 2.0, -0.0, 8388609.0], np.float32)
    got = ref.unary("round", half)
    assert np.array_equal(got.view(np.uint32), away.view(np.uint32)), got
    assert not np.array_equal(np.round(half), away)  # ties to even would fail the check above


# ---------------------------------------------------------------------------
# Oracle f32 restatement vs float64 closed forms


def test_refcpu_vs_closed_forms():
    r = rng(21)
    x = r.standard_normal((37, 96)).astype(np.float32)
    w = (r.standard_normal(96) * 0.1 + 1).astype(np.float32)
    b = (r.standard_normal(96) * 0.1).astype(np.float32)
    g = r.standard_normal((37, 96)).astype(np.float32)
    y, _ = ref.rms_norm_fwd(x, w)
    np.testing.assert_allclose(y, cf.rms_norm_fwd(x, w)[0], rtol=1e-5, atol=1e-6)
    y, mu, inv = ref.layer_norm_fwd(x, w, b)
    y64, mu64, inv64 = cf.layer_norm_fwd(x, w, b)
    np.testing.assert_allclose(y, y64, rtol=1e-5, atol=2e-6)
    dx, dw, db = ref.layer_norm_bwd(x, w, mu, inv, g)
    dx64, dw64, db64 = cf.layer_norm_bwd_refgraph(x, w, g)
    np.testing.assert_allclose(dx, dx64, rtol=1e-5, atol=2e-6)
    np.testing.assert_allclose(dw, dw64, rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(db, db64, rtol=1e-5, atol=1e-5)
    _, inv = ref.rms_norm_fwd(x, w)
    dx, dw = ref.rms_norm_bwd(x, w, inv, g)
    dx64, dw64 = cf.rms_norm_bwd_refgraph(x, w, g)
    np.testing.assert_allclose(dx, dx64, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(dw, dw64, rtol=1e-5, atol=1e-5)
    z = (r.standard_normal(5000) * 3).astype(np.float32)
    gz = r.standard_normal(5000).astype(np.float32)
    np.testing.assert_allclose(ref.gelu_tanh_fwd(z), cf.gelu_tanh(z), rtol=1e-5, atol=2e-6)
    np.testing.assert_allclose(ref.gelu_tanh_bwd(z, gz), cf.gelu_tanh_grad(z) * gz, rtol=1e-4, atol=2e-6)
    np.testing.assert_allclose(ref.gelu_erf_fwd(z), cf.gelu_erf(z), rtol=1e-5, atol=2e-6)
    np.testing.assert_allclose(ref.gelu_erf_bwd(z, gz), cf.gelu_erf_grad(z) * gz, rtol=1e-5, atol=2e-6)
    np.testing.assert_allclose(ref.silu_fwd(z), cf.silu(z), rtol=1e-5, atol=2e-6)
    np.testing.assert_allclose(ref.silu_bwd(z, gz), cf.silu_grad(z) * gz, rtol=1e-5, atol=2e-6)
    s = (r.standard_normal((40, 300)) * 2).astype(np.float32)
    gs = r.standard_normal((40, 300)).astype(np.float32)
    for dim in (-1, 0):
        np.testing.assert_allclose(ref.softmax_fwd(s, dim), cf.softmax(s, dim), rtol=1e-5, atol=1e-7)
        np.testing.assert_allclose(ref.log_softmax_fwd(s, dim), cf.log_softmax(s, dim), rtol=1e-5, atol=1e-6)
        np.testing.assert_allclose(ref.softmax_bwd(s, gs, dim), cf.softmax_bwd(s, gs, dim), rtol=1e-4, atol=1e-6)
        # the reference's max-path noise lands on the argmax: compare with a wider atol there
        np.testing.assert_allclose(ref.log_softmax_bwd(s, gs, dim), cf.log_softmax_bwd(s, gs, dim), rtol=1e-4,
                                   atol=5e-5)
    t = r.integers(0, 300, 40)
    assert abs(ref.cross_entropy_fwd(s, t) - cf.cross_entropy(s, t)) < 1e-5
    np.testing.assert_allclose(ref.cross_entropy_bwd(s, t) * 40, cf.cross_entropy_grad(s, t) * 40, rtol=1e-4,
                               atol=1e-5)
    ids = r.integers(0, 50, 400)
    ge = r.standard_normal((400, 8)).astype(np.float32)
    np.testing.assert_allclose(ref.index_select_bwd(ge, (50, 8), 0, ids), cf.embedding_grad(ge, ids, 50), rtol=1e-5,
                               atol=1e-5)


# ---------------------------------------------------------------------------
# Finite differences (gradcheck.rs parameters: h = 1e-2 in f32, tol 1e-3 * max(1, |g|))


def fd_check(f, x, analytic, weights, h=1e-2, tol=1e-3):
    """Central differences of sum(f(x) * weights), evaluated in float64."""
    x = np.asarray(x, np.float64)
    num = np.zeros_like(x)
    it = np.nditer(x, flags=["multi_index"])
    for _ in it:
        i = it.multi_index
        xp = x.copy()
        xp[i] += h
        xm = x.copy()
        xm[i] -= h
        num[i] = ((f(xp) * weights).sum() - (f(xm) * weights).sum()) / (2 * h)
    return np.all(np.abs(analytic - num) <= tol * np.maximum(1.0, np.abs(analytic)))


def test_fd_exact_norm_vjps():
    r = rng(31)
    x = r.standard_normal((3, 6))
    w = r.standard_normal(6) * 0.3 + 1
    b = r.standard_normal(6) * 0.1
    g = r.standard_normal((3, 6))
    dx, _ = cf.rms_norm_bwd_exact(x, w, g)
    assert fd_check(lambda v: cf.rms_norm_fwd(v, w)[0], x, dx, g)
    dx, _, _ = cf.layer_norm_bwd_exact(x, w, g)
    assert fd_check(lambda v: cf.layer_norm_fwd(v, w, b)[0], x, dx, g)


def test_fd_documents_reference_norm_defect():
    """The reference detaches rsqrt (bindings lib.rs:682-710): its x-grads fail FD, its w/b grads pass."""
    r = rng(32)
    x = r.standard_normal((3, 6)).astype(np.float32)
    w = (r.standard_normal(6) * 0.3 + 1).astype(np.float32)
    b = (r.standard_normal(6) * 0.1).astype(np.float32)
    g = r.standard_normal((3, 6)).astype(np.float32)
    _, mu, inv = ref.layer_norm_fwd(x, w, b)
    dx, dw, db = ref.layer_norm_bwd(x, w, mu, inv, g)
    assert not fd_check(lambda v: cf.layer_norm_fwd(v, w, b)[0], x, dx, g)
    assert fd_check(lambda v: cf.layer_norm_fwd(x, v, b)[0], w, dw, g)
    assert fd_check(lambda v: cf.layer_norm_fwd(x, w, v)[0], b, db, g)
    _, inv = ref.rms_norm_fwd(x, w)
    dx, dw = ref.rms_norm_bwd(x, w, inv, g)
    assert not fd_check(lambda v: cf.rms_norm_fwd(v, w)[0], x, dx, g)
    assert fd_check(lambda v: cf.rms_norm_fwd(x, v)[0], w, dw, g)


def test_fd_activation_softmax_ce_vjps():
    r = rng(33)
    x = (r.standard_normal((2, 7)) * 1.5).astype(np.float32)
    g = r.standard_normal((2, 7)).astype(np.float32)
    assert fd_check(cf.gelu_tanh, x, ref.gelu_tanh_bwd(x, g), g)
    assert fd_check(cf.gelu_erf, x, ref.gelu_erf_bwd(x, g), g)
    assert fd_check(cf.silu, x, ref.silu_bwd(x, g), g)
    assert fd_check(cf.softmax, x, ref.softmax_bwd(x, g), g)
    assert fd_check(cf.log_softmax, x, ref.log_softmax_bwd(x, g), g)
    t = np.array([3, 0])
    assert fd_check(lambda v: np.array(cf.cross_entropy(v, t)), x, ref.cross_entropy_bwd(x, t), 1.0)


# ---------------------------------------------------------------------------
# Invariants


def test_invariants():
    r = rng(41)
    x = (r.standard_normal((20, 333)) * 3).astype(np.float32)
    np.testing.assert_allclose(ref.softmax_fwd(x).sum(-1), 1.0, rtol=1e-5)
    np.testing.assert_allclose(np.exp(ref.log_softmax_fwd(x).astype(np.float64)).sum(-1), 1.0, rtol=1e-5)
    y, _, _ = ref.layer_norm_fwd(x, np.ones(333, np.float32), np.zeros(333, np.float32))
    np.testing.assert_allclose(y.mean(-1), 0.0, atol=1e-5)
    np.testing.assert_allclose(y.var(-1), 1.0, rtol=1e-3)
    ids = np.minimum(r.zipf(1.1, 3000) - 1, 99)
    g = r.standard_normal((3000, 5)).astype(np.float32)
    dW = ref.index_select_bwd(g, (100, 5), 0, ids)
    np.testing.assert_allclose(dW.sum(0), g.sum(0), rtol=1e-4, atol=1e-3)
    absent = np.setdiff1d(np.arange(100), ids)
    assert np.all(dW[absent] == 0)
    # CE gradient rows sum to zero
    t = r.integers(0, 333, 20)
    np.testing.assert_allclose(ref.cross_entropy_bwd(x, t).sum(-1), 0.0, atol=1e-7)


# ---------------------------------------------------------------------------
# Planted mistakes: a wrong variant of an oracle function must fail the checks


def test_planted_mistakes_are_caught():
    r = rng(51)
    x = r.standard_normal((3, 6))
    w = r.standard_normal(6) * 0.3 + 1
    b = r.standard_normal(6) * 0.1
    g = r.standard_normal((3, 6))

    def ln_exact_missing_mean_term(x, w, g, eps=1e-5):
        mu = x.mean(-1, keepdims=True)
        inv = 1.0 / np.sqrt(((x - mu) ** 2).mean(-1, keepdims=True) + eps)
        xh = (x - mu) * inv
        gw = g * w
        return inv * (gw - xh * (gw * xh).mean(-1, keepdims=True))  # dropped: - mean(gw)

    assert not fd_check(lambda v: cf.layer_norm_fwd(v, w, b)[0], x, ln_exact_missing_mean_term(x, w, g), g)

    def gelu_grad_wrong_sign(v):
        u = cf.SQRT_2_OVER_PI * (v + 0.044715 * v ** 3)
        t = np.tanh(u)
        du = cf.SQRT_2_OVER_PI * (1.0 + 3 * 0.044715 * v * v)
        return 0.5 * (1.0 + t) - 0.5 * v * (1.0 - t * t) * du

    xs = r.standard_normal(9)
    assert not fd_check(cf.gelu_tanh, xs, gelu_grad_wrong_sign(xs) * np.ones(9), np.ones(9))

    def embedding_grad_transposed_index(gg, ids, V):  # accumulates row p into row p instead of ids[p]
        out = np.zeros((V, gg.shape[1]))
        for p in range(len(ids)):
            out[p % V] += gg[p]
        return out

    ids = np.array([2, 2, 0, 2])
    gg = np.arange(12, dtype=np.float64).reshape(4, 3)
    assert not np.array_equal(embedding_grad_transposed_index(gg, ids, 4), cf.embedding_grad(gg, ids, 4))

    def softmax_bwd_missing_dot(v, gg):
        return cf.softmax(v) * gg

    xs = r.standard_normal((2, 5))
    gs = r.standard_normal((2, 5))
    assert not fd_check(cf.softmax, xs, softmax_bwd_missing_dot(xs, gs), gs)


# ---------------------------------------------------------------------------
# Optimizer steps (crates/oxi-autograd/src/optim.rs)

def _adam_f64(p, g, m, v, t, lr, b1, b2, eps, wd, decoupled):
    p, g = p.astype(np.float64), g.astype(np.float64)
    ge = g + wd * p if (not decoupled and wd != 0) else g
    m = b1 * m + (1 - b1) * ge
    v = b2 * v + (1 - b2) * ge * ge
    nxt = p - lr * (m / (1 - b1 ** t)) / (np.sqrt(v / (1 - b2 ** t)) + eps)
    if decoupled and wd != 0:
        nxt = nxt - lr * wd * p
    return nxt, m, v


def test_kat_sgd_momentum_and_nesterov():
    """crates/oxi-autograd/src/optim.rs:314-334: three momentum steps of a
    constant gradient 0.5 (lr 0.1, momentum 0.9), and one Nesterov step."""
    buf = np.zeros(1, np.float32)
    val = np.ones(1, np.float32)
    for want in (1.0 - 0.05, 0.95 - 0.095, 0.855 - 0.1355):
        val = ref.sgd_step(val, np.array([0.5], np.float32), buf, 0.1, 0.9)
        assert abs(float(val[0]) - want) < 1e-6
    buf = np.zeros(1, np.float32)
    val = ref.sgd_step(np.ones(1, np.float32), np.array([0.5], np.float32), buf, 0.1, 0.9, nesterov=True)
    assert abs(float(val[0]) - (1.0 - 0.1 * 0.95)) < 1e-6
    # no momentum: plain descent, no state
    val = ref.sgd_step(np.ones(1, np.float32), np.array([0.5], np.float32), None, 0.1, 0.0)
    assert abs(float(val[0]) - 0.95) < 1e-7


def test_kat_adamw_and_classic_adam():
    """optim.rs:366-404: two AdamW steps against the float64 closed form, and
    classic Adam folding the decay into the gradient."""
    m, v = np.zeros(1, np.float32), np.zeros(1, np.float32)
    val = np.ones(1, np.float32)
    vf, mf, vvf = np.ones(1), np.zeros(1), np.zeros(1)
    for t in (1, 2):
        val = ref.adamw_step(val, np.array([0.5], np.float32), m, v, t, 0.1, 0.9, 0.999, 1e-8, 0.1, True)
        vf, mf, vvf = _adam_f64(vf, np.array([0.5]), mf, vvf, t, 0.1, 0.9, 0.999, 1e-8, 0.1, True)
        assert abs(float(val[0]) - float(vf[0])) < 1e-5
    m, v = np.zeros(1, np.float32), np.zeros(1, np.float32)
    got = ref.adamw_step(np.ones(1, np.float32), np.array([0.5], np.float32), m, v, 1, 0.1, 0.9, 0.999, 1e-8, 0.1,
                         False)
    ge = 0.5 + 0.1 * 1.0
    want = 1.0 - 0.1 * ((0.1 * ge) / 0.1) / (np.sqrt((0.001 * ge * ge) / 0.001) + 1e-8)
    assert abs(float(got[0]) - want) < 1e-5


@pytest.mark.parametrize("decoupled", [True, False])
def test_adam_matches_float64_over_steps(decoupled):
    """Random parameters, 5 steps with fresh gradients: the f32 oracle stays
    within 1e-6 relative of the float64 closed form; a planted mistake (bias
    correction dropped from the second moment) does not."""
    r = rng(31)
    p = r.standard_normal(257).astype(np.float32)
    m, v = np.zeros_like(p), np.zeros_like(p)
    pf, mf, vf = p.astype(np.float64), np.zeros(p.size), np.zeros(p.size)
    for t in range(1, 6):
        g = r.standard_normal(p.size).astype(np.float32)
        p = ref.adamw_step(p, g, m, v, t, 1e-2, 0.9, 0.999, 1e-8, 0.05, decoupled)
        pf, mf, vf = _adam_f64(pf, g, mf, vf, t, 1e-2, 0.9, 0.999, 1e-8, 0.05, decoupled)
        assert np.allclose(p, pf, rtol=1e-6, atol=1e-7)
    # planted mistake, carried through the same recurrence: v not bias-corrected
    r = rng(31)
    q = r.standard_normal(257).astype(np.float64)
    mq, vq = np.zeros(q.size), np.zeros(q.size)
    for t in range(1, 6):
        g = r.standard_normal(q.size).astype(np.float32).astype(np.float64)
        ge = g + 0.05 * q if not decoupled else g
        mq = 0.9 * mq + 0.1 * ge
        vq = 0.999 * vq + 0.001 * ge * ge
        q = q - 1e-2 * (mq / (1 - 0.9 ** t)) / (np.sqrt(vq) + 1e-8) - (1e-2 * 0.05 * q if decoupled else 0)
    assert not np.allclose(p, q, rtol=1e-6, atol=1e-7)


def test_sgd_matches_float64_over_steps():
    r = rng(32)
    p = r.standard_normal(300).astype(np.float32)
    buf = np.zeros_like(p)
    pf, bf = p.astype(np.float64), np.zeros(p.size)
    for _ in range(4):
        g = r.standard_normal(p.size).astype(np.float32)
        p = ref.sgd_step(p, g, buf, 0.05, 0.9, nesterov=True)
        bf = 0.9 * bf + g
        pf = pf - 0.05 * (g + 0.9 * bf)
        assert np.allclose(p, pf, rtol=1e-6, atol=1e-6)
    # planted mistake, carried through the same recurrence: the Nesterov
    # update without its gradient term
    r = rng(32)
    q = r.standard_normal(300).astype(np.float64)
    bq = np.zeros(q.size)
    for _ in range(4):
        g = r.standard_normal(q.size).astype(np.float32).astype(np.float64)
        bq = 0.9 * bq + g
        q = q - 0.05 * (0.9 * bq)
    assert not np.allclose(p, q, rtol=1e-6, atol=1e-6)


# ---- scatter_dim0 and masked_select (crates/oxi-tensor/src/lib.rs:895-961,
# crates/oxi-autograd/src/ops.rs:531-667) -------------------------------------------

def test_kat_scatter_and_masked_select():
    """python/tests/test_indexing_grad.py:20-69,111-117."""
    base = np.array([[10.0, 11.0], [20.0, 21.0], [30.0, 31.0]], np.float32)
    vals = np.array([[1.0, 2.0], [3.0, 4.0], [5.0, 6.0]], np.float32)
    assert ref.scatter_dim0(base, [2, 0, 2], vals).tolist() == [[3.0, 4.0], [20.0, 21.0], [5.0, 6.0]]
    gb, gv = ref.scatter_dim0_bwd(np.ones((3, 2), np.float32), [2, 0, 2], (3, 2))
    assert gb.tolist() == [[0.0, 0.0], [1.0, 1.0], [0.0, 0.0]]
    assert gv.tolist() == [[0.0, 0.0], [1.0, 1.0], [1.0, 1.0]]
    r = rng(7)
    a = r.standard_normal((5, 3)).astype(np.float32)
    v3 = r.standard_normal((3, 3)).astype(np.float32)
    want = a.copy()
    want[[4, 1, 4]] = v3
    assert np.array_equal(ref.scatter_dim0(a, [4, 1, 4], v3), want)
    assert ref.scatter_dim0(np.ones((2, 2), np.float32), [0], np.full((1, 2), -1.0, np.float32)).tolist() == \
        [[-1.0, -1.0], [1.0, 1.0]]
    col = np.array([[7.0], [9.0]], np.float32)
    mask = np.array([[1.0, 1.0, 0.0], [0.0, 1.0, 1.0]], np.float32)
    assert ref.masked_select(col, mask).tolist() == [7.0, 7.0, 9.0, 9.0]
    assert ref.masked_select_bwd(col.shape, mask, np.array([1, 2, 3, 4], np.float32)).tolist() == [[3.0], [7.0]]
    r = rng(11)
    a = r.standard_normal((2, 3)).astype(np.float32)
    up = r.standard_normal((2, 3)).astype(np.float32)
    m = (r.standard_normal((2, 3)) > 0).astype(np.float32)
    np.testing.assert_allclose(ref.masked_select_bwd(a.shape, m, up[m > 0]), m * up, rtol=1e-4, atol=1e-5)


def _rand_ids(r, rows, n):
    ids = r.integers(-rows, rows, n)
    if n:
        ids[: n // 3] = ids[0]  # a run of duplicates: last-writer logic matters
    return ids


@pytest.mark.parametrize("shape,n", [((7,), 5), ((9, 4), 12), ((6, 3, 5), 10), ((4, 2), 0)])
def test_scatter_against_numpy_and_adjoint(shape, n):
    """Forward: numpy's fancy assignment (last write wins). VJP: the adjoint
    identity <g, S(db, dv)> = <gb, db> + <gv, dv> of the linear map S, in
    float64; a VJP that credits the first writer instead fails it."""
    r = rng(100 + n)
    rows = shape[0]
    ids = _rand_ids(r, rows, n)
    base = r.standard_normal(shape).astype(np.float32)
    vals = r.standard_normal((n,) + shape[1:]).astype(np.float32)
    want = base.copy()
    if n:
        want[ids] = vals
    got = ref.scatter_dim0(base, ids, vals)
    assert np.array_equal(got, want)
    g = r.standard_normal(shape).astype(np.float32)
    gb, gv = ref.scatter_dim0_bwd(g, ids, vals.shape)
    db = r.standard_normal(shape)
    dv = r.standard_normal(vals.shape)
    lin = ref.scatter_dim0(db.astype(np.float32), ids, dv.astype(np.float32)).astype(np.float64)
    lhs = float(np.sum(g.astype(np.float64) * lin))
    rhs = float(np.sum(gb * db.astype(np.float32).astype(np.float64)) +
                np.sum(gv * dv.astype(np.float32).astype(np.float64)))
    assert abs(lhs - rhs) <= 1e-9 * (1 + abs(lhs))
    if n:
        # planted mistake: credit the FIRST writer of each row
        bad = np.zeros_like(gv)
        seen = set()
        for p, i in enumerate(ids % rows):
            if i not in seen:
                bad[p] = g[i]
                seen.add(i)
        rhs_bad = float(np.sum(gb * db.astype(np.float32)) + np.sum(bad * dv.astype(np.float32)))
        if not np.array_equal(bad, gv):
            assert abs(lhs - rhs_bad) > 1e-6 * (1 + abs(lhs))


def test_scatter_bwd_signed_zero_and_nan():
    """gbase is g * 0 on written rows: -0 for a negative g, NaN for a NaN g."""
    g = np.array([[-1.0, np.nan], [2.0, -3.0]], np.float32)
    gb, _ = ref.scatter_dim0_bwd(g, [0], (1, 2))
    assert np.signbit(gb[0, 0]) and gb[0, 0] == 0 and np.isnan(gb[0, 1])
    assert gb[1].tolist() == [2.0, -3.0]


@pytest.mark.parametrize("xs,ms", [((3, 4), (3, 4)), ((2, 1, 5), (3, 5)), ((4,), (3, 1)), ((1,), (2, 3)),
                                   ((2, 3, 4), (4,))])
def test_masked_select_against_numpy_and_adjoint(xs, ms):
    """Forward: numpy boolean indexing of the broadcast arrays. VJP: np.add.at
    over the broadcast positions (exact here: few adds per element) and the
    adjoint identity of the linear map x -> masked_select(x, m)."""
    r = rng(200 + len(xs) + len(ms))
    x = r.standard_normal(xs).astype(np.float32)
    m = (r.random(ms) > 0.4).astype(np.float32)
    m.ravel()[0] = -0.0  # negative zero is not picked
    m.ravel()[-1] = np.nan  # NaN compares != 0: picked
    grid = np.broadcast_shapes(xs, ms)
    xb, mb = np.broadcast_to(x, grid), np.broadcast_to(m, grid)
    sel = mb != 0
    assert np.array_equal(ref.masked_select(x, m), xb[sel])
    g = r.standard_normal(int(sel.sum())).astype(np.float32)
    gx = ref.masked_select_bwd(xs, m, g)
    pos = np.broadcast_to(np.arange(x.size).reshape(xs), grid)[sel]
    want = np.zeros(x.size, np.float64)
    np.add.at(want, pos, g.astype(np.float64))
    np.testing.assert_allclose(gx.ravel(), want, rtol=1e-6, atol=1e-6)
    dx = r.standard_normal(xs).astype(np.float32)
    lhs = float(np.sum(g.astype(np.float64) * ref.masked_select(dx, m)))
    rhs = float(np.sum(gx.astype(np.float64) * dx))
    assert abs(lhs - rhs) <= 1e-5 * (1 + abs(lhs))


def test_masked_select_drops_nan_values():
    """The reference's NaN marker also drops picked NaN values of x."""
    x = np.array([1.0, np.nan, 3.0], np.float32)
    m = np.ones(3, np.float32)
    assert ref.masked_select(x, m).tolist() == [1.0, 3.0]


def test_cross_entropy_of_an_empty_batch_is_negative_zero():
    """picked.mean() over no rows goes through reduce_all, whose Mean of an
    empty strip is 0 (bindings lib.rs:126-143, ops.rs:247-249), so the loss
    is -(0.0) = -0.0, not the 0/0 of Tensor::mean_all."""
    loss = ref.cross_entropy_fwd(np.zeros((0, 5), np.float32), np.zeros(0, np.int64))
    assert loss == 0.0 and np.signbit(loss)
