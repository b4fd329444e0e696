"""The reference's own Python tests for the hot path, run through
oxitorch_amd's drop-in surface on the GPU (python/tests/test_nn.py,
test_indexing_grad.py, test_smoke.py, test_autograd.py, test_grad_mode.py),
plus the five BASELINE configs end to end through F.* and backward(),
checked against the CPU oracle."""

import sys

import numpy as np
import pytest

from conftest import (assert_close, assert_close_arb, assert_reduction_close, assert_sum_close, record, rng,
                      segmented_runs_in_one_tile)

pytestmark = pytest.mark.gpu


def say(*a):
    print("[case]", *a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def ox(hip):
    import oxitorch_amd

    return oxitorch_amd


@pytest.fixture(scope="module")
def F(ox):
    import oxitorch_amd.nn.functional as F

    return F


def _t(ox, arr, requires_grad=False):
    return ox.from_numpy(np.ascontiguousarray(arr, dtype=np.float32), requires_grad)


# ---- python/tests/test_nn.py ------------------------------------------------------------

def test_softmax_and_log_softmax_parity(ox, F):
    say("api softmax")
    x = _t(ox, [[1.0, 2.0, 3.0], [3.0, 1.0, 2.0]])
    xr = x.detach().numpy()
    sm = F.softmax(x, -1).numpy()
    assert np.allclose(sm, np.exp(xr) / np.exp(xr).sum(-1, keepdims=True), atol=1e-6)
    ls = F.log_softmax(x, -1).numpy()
    assert np.allclose(np.exp(ls).sum(-1), 1.0, atol=1e-6)


def test_log_softmax_stability_large_inputs(ox, F):
    ls = F.log_softmax(_t(ox, [[1000.0, 1001.0, 1002.0]]), -1).numpy()
    assert np.all(np.isfinite(ls))
    sm = np.exp(ls)
    sm = sm / sm.sum()
    want = np.exp(np.array([1000.0, 1001.0, 1002.0]) - 1002.0)
    assert np.allclose(sm, want / want.sum(), atol=1e-6)


def test_activations_values(ox, F):
    x = _t(ox, [-1.0, 0.0, 1.0, 2.0])
    r = x.detach().numpy()
    assert np.allclose(F.relu(x).numpy(), np.maximum(r, 0), atol=1e-7)
    assert np.allclose(F.sigmoid(x).numpy(), 1 / (1 + np.exp(-r)), atol=1e-6)
    assert np.allclose(F.tanh(x).numpy(), np.tanh(r), atol=1e-6)
    assert np.allclose(F.silu(x).numpy(), r / (1 + np.exp(-r)), atol=1e-6)
    c = np.sqrt(2 / np.pi)
    assert np.allclose(F.gelu(x).numpy(), 0.5 * r * (1 + np.tanh(c * (r + 0.044715 * r ** 3))), atol=1e-5)
    # layers.py:183-188: LeakyReLU is F.leaky_relu
    import oxitorch_amd.nn as nn
    assert np.allclose(F.leaky_relu(x, 0.2).numpy(), np.where(r > 0, r, 0.2 * r), atol=1e-7)
    assert np.array_equal(nn.LeakyReLU(0.2)(x).numpy(), F.leaky_relu(x, 0.2).numpy())


def test_layer_norm_value_and_grads(ox, F):
    x = _t(ox, [[1.0, 2.0, 3.0], [4.0, 5.0, 6.0]], requires_grad=True)
    w = _t(ox, [1.0, 1.0, 1.0], requires_grad=True)
    b = _t(ox, [0.0, 0.0, 0.0], requires_grad=True)
    out = F.layer_norm(x, w, b)
    xr = x.detach().numpy()
    mu = xr.mean(-1, keepdims=True)
    v = ((xr - mu) ** 2).mean(-1, keepdims=True)
    assert np.allclose(out.numpy(), (xr - mu) / np.sqrt(v + 1e-5), rtol=1e-4, atol=1e-5)
    coef = np.array([[1.0, -2.0, 0.5], [0.25, 1.0, -1.0]], dtype=np.float32)
    (out * _t(ox, coef)).sum().backward()
    assert x.grad is not None and w.grad is not None and b.grad is not None
    assert np.abs(x.grad.numpy()).sum() > 1e-6


def test_rms_norm_value(ox, F):
    x = _t(ox, [[1.0, -2.0, 3.0]])
    w = _t(ox, [1.0, 2.0, 0.5])
    xr = x.detach().numpy()
    ref = xr / np.sqrt((xr ** 2).mean(-1, keepdims=True) + 1e-6) * np.array([[1.0, 2.0, 0.5]])
    assert np.allclose(F.rms_norm(x, w).numpy(), ref, rtol=1e-4, atol=1e-5)


def test_embedding_lookup_and_grad(ox, F):
    w = _t(ox, [[1.0, 1.0], [2.0, 2.0], [3.0, 3.0]], requires_grad=True)
    out = F.embedding([2, 0, 2], w)
    assert np.allclose(out.numpy(), [[3, 3], [1, 1], [3, 3]], atol=1e-7)
    out.sum().backward()
    assert np.allclose(w.grad.numpy(), [[1, 1], [0, 0], [2, 2]], atol=1e-6)


def test_cross_entropy_value_and_grad(ox, F):
    logits = _t(ox, [[1.0, 2.0, 3.0], [3.0, 1.0, 2.0]], requires_grad=True)
    loss = F.cross_entropy(logits, [2, 0])
    lg = logits.detach().numpy()
    m = lg.max(-1, keepdims=True)
    ls = lg - m - np.log(np.exp(lg - m).sum(-1, keepdims=True))
    assert abs(loss.item() - (-np.mean([ls[0, 2], ls[1, 0]]))) < 1e-5
    loss.backward()
    g = (np.exp(ls) - np.eye(3, dtype=np.float32)[[2, 0]]) / 2
    assert np.allclose(logits.grad.numpy(), g, rtol=1e-4, atol=1e-6)


@pytest.mark.parametrize("c", [1000, 32000, 50257])
def test_cross_entropy_seeded_with_one_takes_the_forward_gradient(ox, F, c):
    """loss.backward() (the implicit seed 1) hands the logits the gradient
    the forward pass formed; an explicit seed, a loss used inside the graph,
    a retained second backward and rows whose class count is not a multiple
    of 4 all run the backward kernel (twice its gradient, bit for bit, when
    the loss is doubled; the retained pair adds the two). The one-pass and
    the backward kernel's gradients agree within a few ulp; a class count
    that is not a multiple of 4 takes the backward kernel both ways, bit for
    bit."""
    say("cross_entropy backward seeds", c)
    r = np.random.default_rng(c)
    n = 16
    la = (r.standard_normal((n, c), dtype=np.float32) * 2).astype(np.float32)
    t = r.integers(0, c, n)

    def grad_of(run):
        x = _t(ox, la, True)
        run(x)
        return x.grad.numpy()

    implicit = grad_of(lambda x: F.cross_entropy(x, t).backward())
    explicit = grad_of(lambda x: F.cross_entropy(x, t).backward(ox.from_numpy(np.ones((), np.float32))))
    doubled = grad_of(lambda x: (F.cross_entropy(x, t) * 2.0).backward())

    def twice(x):
        loss = F.cross_entropy(x, t)
        loss.backward(retain_graph=True)
        loss.backward()
    both = grad_of(twice)
    if c % 4:
        assert np.array_equal(implicit.view(np.uint32), explicit.view(np.uint32))
    else:
        assert np.allclose(implicit, explicit, rtol=1e-5, atol=1e-7 / n)
    assert np.array_equal((2 * explicit).view(np.uint32), doubled.view(np.uint32))
    assert np.array_equal((implicit + explicit).view(np.uint32), both.view(np.uint32))
    m = la.max(-1, keepdims=True)
    ls = la - m - np.log(np.exp(la - m).sum(-1, keepdims=True))
    want = (np.exp(ls) - np.eye(c, dtype=np.float32)[t]) / n
    assert np.allclose(implicit, want, rtol=1e-4, atol=1e-6)
    # with the one-pass forward off, backward() runs the backward kernel: the
    # bits of the explicit seed
    from oxitorch_amd import _native
    prev = _native.set_ce_one_pass(False)
    try:
        assert not _native.ce_one_pass()
        two_call = grad_of(lambda x: F.cross_entropy(x, t).backward())
    finally:
        _native.set_ce_one_pass(prev)
    assert np.array_equal(two_call.view(np.uint32), explicit.view(np.uint32))


@pytest.mark.parametrize("c", [1000, 1003])
def test_cross_entropy_masked_logits(ox, F, c):
    """A -inf logit at a non-target class: the loss is NaN, as the
    reference's sum(onehot * log_softmax) makes it, and backward() still gives
    the finite gradient (0 at the masked class), through the one-pass kernel
    (c = 1000) and the two calls (c = 1003)."""
    from oracle import ref
    say("cross_entropy masked logits via F.*", c)
    r = np.random.default_rng(c)
    la = (r.standard_normal((8, c), dtype=np.float32) * 2).astype(np.float32)
    t = r.integers(0, c, 8)
    la[3, (t[3] + 1) % c] = -np.inf
    x = _t(ox, la, True)
    loss = F.cross_entropy(x, t)
    assert np.isnan(loss.item())
    loss.backward()
    g = x.grad.numpy()
    want = ref.cross_entropy_bwd(la, t)
    assert np.isfinite(g).all() and g[3, (t[3] + 1) % c] == 0.0
    assert np.allclose(8 * g, 8 * want, rtol=1e-5, atol=1e-5)


def test_cross_entropy_rejects_wrong_batch(ox, F):
    with pytest.raises(ValueError, match="targets"):
        F.cross_entropy(_t(ox, np.zeros((2, 3))), [0, 1, 2])


def test_modules(ox):
    import oxitorch_amd.nn as nn

    ln = nn.LayerNorm(8)
    rms = nn.RMSNorm(8)
    emb = nn.Embedding(10, 8, seed=0)
    assert [n for n, _ in ln.named_parameters()] == ["weight", "bias"]
    np.testing.assert_array_equal(ln.weight.tensor.numpy(), np.ones(8, np.float32))
    h = emb([1, 2, 3])
    np.testing.assert_allclose(h.numpy(),
                               (np.random.default_rng(0).standard_normal((10, 8)) * 0.05).astype(np.float32)[[1, 2, 3]])
    y = nn.Softmax(-1)(nn.SiLU()(rms(ln(h))))
    y.sum().backward()
    assert emb.weight.grad is not None and ln.bias.grad is not None and rms.weight.grad is not None


def test_module_state_round_trip(ox):
    """python/oxitorch/nn/module.py:62-98,121-122: dotted names through lists,
    train() reaching list members, state_dict / load_state_dict with the
    reference's missing-key and shape errors, Sequential indexing."""
    import oxitorch_amd.nn as nn

    class Block(nn.Module):
        def __init__(self):
            self.norms = [nn.LayerNorm(4), nn.RMSNorm(4)]
            self.emb = nn.Embedding(6, 4, seed=1)

        def forward(self, ids):
            return self.norms[1](self.norms[0](self.emb(ids)))

    seq = nn.Sequential(Block(), nn.SiLU())
    assert seq[0] is seq.layers[0] and seq[-1] is seq.layers[1]
    names = [n for n, _ in seq.named_parameters()]
    assert names == ["layers.0.norms.0.weight", "layers.0.norms.0.bias", "layers.0.norms.1.weight",
                     "layers.0.emb.weight"]
    assert len(seq.parameters()) == 4
    seq.eval()
    assert not seq.training and not seq[0].training and not seq[0].norms[0].training and not seq[0].emb.training
    seq.train()
    assert seq[0].norms[1].training

    state = seq.state_dict()
    assert sorted(state) == sorted(names)
    r = rng(12)
    new = {k: r.standard_normal(v.shape).astype(np.float32) for k, v in state.items()}
    seq.load_state_dict(new)
    for k, p in seq.named_parameters():
        np.testing.assert_array_equal(p.tensor.numpy(), new[k])
        assert p.tensor.requires_grad
    out = seq([0, 5, 2])
    out.sum().backward()
    assert seq[0].emb.weight.grad is not None

    before = {k: v.copy() for k, v in seq.state_dict().items()}
    missing = dict(new)
    del missing["layers.0.emb.weight"]
    with pytest.raises(KeyError, match="missing key in state_dict: 'layers.0.emb.weight'"):
        seq.load_state_dict(missing)
    bad = dict(new)
    bad["layers.0.norms.1.weight"] = np.zeros(5, np.float32)
    with pytest.raises(ValueError, match=r"shape mismatch for 'layers.0.norms.1.weight': state \[5\] vs parameter \[4\]"):
        seq.load_state_dict(bad)
    # a refused load changes nothing
    for k, v in seq.state_dict().items():
        np.testing.assert_array_equal(v, before[k])


# ---- python/tests/test_indexing_grad.py ------------------------------------------------------

def test_index_select_duplicate_accumulation(ox):
    w = _t(ox, np.zeros((3, 2)), requires_grad=True)
    w.index_select(0, [1, 1, 2]).backward(_t(ox, [[1.0, 10.0], [2.0, 20.0], [3.0, 30.0]]))
    np.testing.assert_array_equal(w.grad.numpy(), [[0.0, 0.0], [3.0, 30.0], [3.0, 30.0]])


def test_embedding_duplicate_index_accumulation(ox, F):
    weight = _t(ox, np.zeros((4, 3)), requires_grad=True)
    F.embedding([2, 2, 0, 2], weight).backward(_t(ox, np.arange(1, 13, dtype=np.float32).reshape(4, 3)))
    want = np.zeros((4, 3), dtype=np.float32)
    want[2] = np.array([1, 2, 3]) + np.array([4, 5, 6]) + np.array([10, 11, 12])
    want[0] = np.array([7, 8, 9])
    np.testing.assert_array_equal(weight.grad.numpy(), want)


def test_fancy_index_getitem_backward(ox):
    a = np.arange(9, dtype=np.float32).reshape(3, 3)
    t = _t(ox, a, requires_grad=True)
    picked = t[[2, 1, 1]]
    picked.backward(_t(ox, np.ones((3, 3))))
    np.testing.assert_array_equal(picked.numpy(), a[[2, 1, 1]])
    np.testing.assert_array_equal(t.grad.numpy(), [[0, 0, 0], [2, 2, 2], [1, 1, 1]])


def test_gather_backward_accumulates_duplicates(ox):
    t = _t(ox, [[1.0, 2.0], [3.0, 4.0]], requires_grad=True)
    out = t.gather([1, 1])
    out.backward(_t(ox, [[5.0, 5.0], [6.0, 6.0]]))
    np.testing.assert_array_equal(out.numpy(), [[3.0, 4.0], [3.0, 4.0]])
    np.testing.assert_array_equal(t.grad.numpy(), [[0.0, 0.0], [11.0, 11.0]])


# ---- python/tests/test_smoke.py (hot-path part) ------------------------------------------------

def test_reduction_parity(ox):
    a = rng(0).standard_normal((3, 4, 5)).astype(np.float32)
    t = _t(ox, a)
    np.testing.assert_allclose(t.sum(0).numpy(), a.sum(0), rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(t.sum(-1).numpy(), a.sum(-1), rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(t.sum(-1, keepdim=True).numpy(), a.sum(-1, keepdims=True), rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(t.mean(1).numpy(), a.mean(1), rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(t.max(0).numpy(), a.max(0))
    np.testing.assert_allclose(t.min(2).numpy(), a.min(2))
    np.testing.assert_array_equal(t.argmax(-1).numpy(), a.argmax(-1))
    np.testing.assert_array_equal(t.argmin(1).numpy(), a.argmin(1))
    np.testing.assert_allclose(t.norm(-1, False).numpy(), np.linalg.norm(a, axis=-1), rtol=1e-5, atol=1e-6)
    assert float(t.sum()) == pytest.approx(float(a.sum()), rel=1e-5)
    assert float(t.mean()) == pytest.approx(float(a.mean()), rel=1e-5)


def test_view_and_indexing_parity(ox):
    a = rng(0).standard_normal((4, 6)).astype(np.float32)
    t = _t(ox, a)
    np.testing.assert_array_equal(t.reshape([-1, 8]).numpy(), a.reshape(-1, 8))
    np.testing.assert_array_equal(t.transpose().numpy(), a.T)
    np.testing.assert_array_equal(t.transpose().contiguous().numpy(), a.T)
    np.testing.assert_array_equal(t[::2].numpy(), a[::2])
    np.testing.assert_array_equal(t.index_select(0, [3, 0, 2]).numpy(), a[[3, 0, 2]])
    np.testing.assert_array_equal(t.index_select(1, [-1, -2]).numpy(), a[:, [-1, -2]])
    np.testing.assert_array_equal(t.gather([1, 1, 0]).numpy(), a[[1, 1, 0]])


def test_op_parity(ox):
    r = rng(1)
    a = r.standard_normal((3, 4)).astype(np.float32)
    b = r.standard_normal(4).astype(np.float32)
    ta, tb = _t(ox, a), _t(ox, b)
    for got, want in [(ta + tb, a + b), (ta - tb, a - b), (ta * tb, a * b), (ta / tb, a / b),
                      (2.0 - ta, 2.0 - a), (2.0 / (ta * ta + 1), 2.0 / (a * a + 1)), (-ta, -a),
                      (ta > tb, a > b), (ta <= tb, a <= b)]:
        np.testing.assert_allclose(got.numpy(), want, rtol=1e-5, atol=1e-6)
    for name, fn in [("exp", np.exp), ("tanh", np.tanh), ("abs", np.abs), ("floor", np.floor)]:
        np.testing.assert_allclose(ta.apply(name).numpy(), fn(a), rtol=1e-5, atol=1e-6)
    with pytest.raises(ValueError, match="unknown unary op"):
        ta.apply("frobnicate")


# ---- autograd (python/tests/test_autograd.py, test_grad_mode.py) -----------------------------

def test_autograd_semantics(ox):
    x = _t(ox, [3.0, -1.0], requires_grad=True)
    y = (x + x) * x  # diamond: crates/oxi-autograd/src/tests.rs:357-366
    y.sum().backward()
    np.testing.assert_allclose(x.grad.numpy(), [12.0, -4.0])
    y = x * x
    s = y.sum()
    s.backward(retain_graph=True)
    s.backward()
    np.testing.assert_allclose(x.grad.numpy(), [12.0 + 12.0, -4.0 - 4.0])
    with pytest.raises(ValueError, match="retain_graph"):
        s.backward()
    with pytest.raises(ValueError, match="implicitly created only for scalar"):
        (x * 2.0).backward()
    with ox.no_grad():
        z = x * 2.0
    assert not z.requires_grad
    for name, fn, d in [("exp", np.exp, np.exp), ("tanh", np.tanh, lambda v: 1 - np.tanh(v) ** 2),
                        ("sigmoid", lambda v: 1 / (1 + np.exp(-v)),
                         lambda v: (1 / (1 + np.exp(-v))) * (1 - 1 / (1 + np.exp(-v))))]:
        v = _t(ox, [0.5, -1.5], requires_grad=True)
        v.apply(name).sum().backward()
        np.testing.assert_allclose(v.grad.numpy(), d(np.array([0.5, -1.5])), rtol=1e-5)
    w = _t(ox, [1.0, 2.0, 3.0], requires_grad=True)
    w.max(0).backward()
    np.testing.assert_array_equal(w.grad.numpy(), [0, 0, 1])
    r = _t(ox, np.ones((2, 3)), requires_grad=True)
    r.apply("rsqrt").sum()  # detached (bindings lib.rs:682-710)
    assert not r.apply("rsqrt").requires_grad


def test_exact_norm_vjp_mode(ox, F):
    from oracle import closed_form
    r = rng(3)
    xa = r.standard_normal((5, 40)).astype(np.float32)
    wa = (r.standard_normal(40) * 0.1 + 1).astype(np.float32)
    ba = (r.standard_normal(40) * 0.1).astype(np.float32)
    g = r.standard_normal((5, 40)).astype(np.float32)
    x = _t(ox, xa, True)
    F.layer_norm(x, _t(ox, wa), _t(ox, ba), vjp="exact").backward(_t(ox, g))
    assert_close(x.grad.numpy(), closed_form.layer_norm_bwd_exact(xa, wa, g)[0], what="ln exact")
    x = _t(ox, xa, True)
    F.rms_norm(x, _t(ox, wa), vjp="exact").backward(_t(ox, g))
    assert_close(x.grad.numpy(), closed_form.rms_norm_bwd_exact(xa, wa, g)[0], what="rms exact")


# ---- the five BASELINE configs end to end through F.* ----------------------------------------------

def test_config1_rms_norm(ox, F):
    from oracle import ref, closed_form
    say("C1 via F.rms_norm")
    r = np.random.default_rng(1)
    xa = r.standard_normal((4096, 768), dtype=np.float32)
    wa = (r.standard_normal(768, dtype=np.float32) * 0.02 + 1).astype(np.float32)
    g = r.standard_normal((4096, 768), dtype=np.float32)
    x, w = _t(ox, xa, True), _t(ox, wa, True)
    y = F.rms_norm(x, w, 1e-6)
    y.backward(_t(ox, g))
    y_ref, inv = ref.rms_norm_fwd(xa, wa, 1e-6)
    dx_ref, dw_ref = ref.rms_norm_bwd(xa, wa, inv, g)
    assert_close(y.numpy(), y_ref, what="C1 y")
    assert_close(x.grad.numpy(), dx_ref, what="C1 dx")
    assert_reduction_close(w.grad.numpy(), dw_ref, closed_form.rms_norm_bwd_refgraph(xa, wa, g)[1], what="C1 dw")


def test_config3_cross_entropy(ox, F):
    from oracle import ref, closed_form
    say("C3 via F.cross_entropy (rows subsampled for the oracle)")
    r = np.random.default_rng(3)
    n, c = 8192, 32000
    la = (r.standard_normal((n, c), dtype=np.float32) * 2).astype(np.float32)
    t = r.integers(0, c, n)
    logits = _t(ox, la, True)
    loss = F.cross_entropy(logits, t.tolist())
    loss.backward()
    tot = 0.0
    for s in range(0, n, 1024):
        ls = closed_form.log_softmax(la[s:s + 1024])
        tot += ls[np.arange(ls.shape[0]), t[s:s + 1024]].sum()
    assert abs(loss.item() - (-tot / n)) <= 1e-5 * abs(loss.item())
    rows = np.sort(r.choice(n, 32, replace=False))
    d = logits.grad.numpy()[rows] * n
    assert_close_arb(d, ref.cross_entropy_bwd(la[rows], t[rows]) * len(rows),
                     closed_form.cross_entropy_grad(la[rows], t[rows]) * len(rows), what="C3 n*dlogits")


def test_config4_embedding(ox, F):
    from oracle import ref
    say("C4 via F.embedding")
    r = np.random.default_rng(4)
    V, D = 50257, 1024
    Wa = r.standard_normal((V, D), dtype=np.float32)
    ids = np.minimum(r.zipf(1.1, (64, 2048)) - 1, V - 1).astype(np.int64).ravel()
    g = r.standard_normal((ids.size, D), dtype=np.float32)
    W = _t(ox, Wa, True)
    out = F.embedding(ids, W)
    np.testing.assert_array_equal(out.numpy(), Wa[ids])
    out.backward(_t(ox, g))
    dW = W.grad.numpy()
    want = ref.index_select_bwd(g, (V, D), 0, ids)
    counts = np.bincount(ids, minlength=V)
    one = segmented_runs_in_one_tile(ids, V)
    np.testing.assert_array_equal(dW[one], want[one])
    heavy = np.flatnonzero(~one & (counts > 0))
    exact = np.stack([g[ids == v].astype(np.float64).sum(0) for v in heavy])
    assert_reduction_close(dW[heavy], want[heavy], exact, what="C4 heavy rows")


def _c5_oracle(ref, Wa, ids, lnw, lnb, rw, pos, g, softmax_bwd):
    e = Wa[ids].reshape(16, 1024, 768)
    h, mu, inv = ref.layer_norm_fwd(e, lnw, lnb, 1e-5)
    hp = np.ascontiguousarray(h.transpose(0, 2, 1))
    s = ref.silu_fwd(hp)
    rr = np.ascontiguousarray(s.transpose(0, 2, 1)) + pos
    n, inv2 = ref.rms_norm_fwd(rr, rw, 1e-6)
    y = ref.softmax_fwd(n)
    dn = np.asarray(softmax_bwd(n, g), np.float32)
    dr, drw = ref.rms_norm_bwd(rr, rw, inv2, dn)
    dpos = np.zeros((1, 1024, 768), np.float32)
    for b in range(16):  # unbroadcast: sequential f32 over the batch axis
        dpos[0] = dpos[0] + dr[b]
    dpos_abs = np.abs(dr.astype(np.float64)).sum(0, keepdims=True)
    ds = np.ascontiguousarray(dr.transpose(0, 2, 1))
    dhp = ref.silu_bwd(hp, ds)
    dh = np.ascontiguousarray(dhp.transpose(0, 2, 1))
    de, dlnw, dlnb = ref.layer_norm_bwd(e, lnw, mu, inv, dh)
    dW = ref.index_select_bwd(de.reshape(-1, 768), Wa.shape, 0, ids)
    # float64 sums of the oracle's own f32 terms: the arbiter for the long column sums
    xh = (e.astype(np.float64) - mu.reshape(16, 1024, 1)) * inv.reshape(16, 1024, 1)
    exact = dict(lnw=(dh * xh).reshape(-1, 768).sum(0), lnb=dh.astype(np.float64).reshape(-1, 768).sum(0),
                 rw=(dn.astype(np.float64) * rr * inv2.reshape(16, 1024, 1)).reshape(-1, 768).sum(0))
    exact["pos_abs"] = dpos_abs
    return y, dict(W=dW, lnw=dlnw, lnb=dlnb, rw=drw, pos=dpos), exact


def _c5_f64(Wa, ids, lnw, lnb, rw, pos, g):
    """The whole C5 chain in float64 closed forms (reference-graph VJPs: the
    norms' inverse std is detached, as in the reference)."""
    from oracle import closed_form as cf
    B, T, H = 16, 1024, 768
    e = Wa.astype(np.float64)[ids].reshape(B, T, H)
    h, mu, inv = cf.layer_norm_fwd(e, lnw, lnb, 1e-5)
    hp = h.transpose(0, 2, 1)
    s = cf.silu(hp)
    rr = s.transpose(0, 2, 1) + pos
    n, inv2 = cf.rms_norm_fwd(rr, rw, 1e-6)
    y = cf.softmax(n)
    dn = cf.softmax_bwd(n, g)
    dr, drw = cf.rms_norm_bwd_refgraph(rr, rw, dn, 1e-6)
    dpos = dr.sum(0, keepdims=True)
    dhp = cf.silu_grad(hp) * dr.transpose(0, 2, 1)
    de, dlnw, dlnb = cf.layer_norm_bwd_refgraph(e, lnw, dhp.transpose(0, 2, 1), 1e-5)
    dW = cf.embedding_grad(de.reshape(-1, H), ids, Wa.shape[0])
    return y, dict(W=dW, lnw=dlnw, lnb=dlnb, rw=drw, pos=dpos)


def test_config5_gpt2_chain(ox, F):
    from oracle import ref
    say("C5 chain")
    r = np.random.default_rng(5)
    V, B, T, H = 50257, 16, 1024, 768
    Wa = r.standard_normal((V, H), dtype=np.float32)
    ids = r.integers(0, V, B * T)
    lnw, lnb, rw = (r.standard_normal(H, dtype=np.float32) for _ in range(3))
    pos = r.standard_normal((1, T, H), dtype=np.float32)
    g = r.standard_normal((B, T, H), dtype=np.float32)
    W, LW, LB, RW, P = (_t(ox, a, True) for a in (Wa, lnw, lnb, rw, pos))
    h = F.layer_norm(F.embedding(ids, W).reshape([B, T, H]), LW, LB)
    s = F.silu(h.permute([0, 2, 1]))
    assert s.is_contiguous()  # forward outputs are row-major, as the reference's
    y = F.softmax(F.rms_norm(s.permute([0, 2, 1]) + P, RW), -1)
    y.backward(_t(ox, g))
    y_ref, grads, _ = _c5_oracle(ref, Wa, ids, lnw, lnb, rw, pos, g, ref.softmax_bwd)
    y64, g64 = _c5_f64(Wa, ids, lnw, lnb, rw, pos, g)
    record("C5", "y", assert_close_arb(y.numpy(), y_ref, y64, what="C5 y"))
    got = dict(W=W.grad.numpy(), lnw=LW.grad.numpy(), lnb=LB.grad.numpy(), rw=RW.grad.numpy(), pos=P.grad.numpy())
    # Ten f32 stages each round differently on the device and in the oracle;
    # where the two differ beyond tolerance the float64 chain arbitrates.
    for k in ("W", "pos"):
        record("C5", f"d{k}", assert_close_arb(got[k], grads[k], g64[k], what=f"C5 d{k}"))
    for k in ("lnw", "lnb", "rw"):  # column sums over 16384 rows
        record("C5", f"d{k} (16384-row sums)", assert_reduction_close(got[k], grads[k], g64[k], what=f"C5 d{k}"))
