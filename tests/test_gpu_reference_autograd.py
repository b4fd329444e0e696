"""The reference's own autograd and grad-mode tests, restated through
oxitorch_amd on the device (python/tests/test_autograd.py,
python/tests/test_grad_mode.py, and the scalar/apply/strided cases of
python/tests/test_nn.py and python/tests/test_smoke.py).

Matrix products are outside this build (SGEMM is not on the path), so where a
reference test multiplies by an (n, 1) weight or goes through nn.Linear the
restatement uses the equivalent broadcast product and sum; every asserted
value is the reference test's own."""

import math

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

RTOL = 1e-4
ATOL = 1e-5


@pytest.fixture(scope="module")
def ox(hip):
    import oxitorch_amd

    return oxitorch_amd


def _t(ox, arr, requires_grad=False):
    return ox.from_numpy(np.ascontiguousarray(arr, dtype=np.float32), requires_grad)


# ---- python/tests/test_autograd.py ------------------------------------------------------

def test_backward_matches_numpy_quadratic(ox):
    """test_autograd.py:19-32, with x @ w written as (x * w^T).sum(1, keepdim)."""
    x = _t(ox, [[1.0, 2.0], [3.0, 4.0]])
    w = _t(ox, [[0.5, 0.5]], requires_grad=True)  # w^T of the reference's (2, 1) weight
    b = ox.full([], 1.0, requires_grad=True)
    pred = (x * w).sum(1, keepdim=True) + b
    diff = pred - _t(ox, [[1.0], [2.0]])
    loss = (diff * diff).sum()
    loss.backward()
    xa = np.array([[1.0, 2.0], [3.0, 4.0]], dtype=np.float32)
    wa = np.array([[0.5], [0.5]], dtype=np.float32)
    da = xa @ wa + 1.0 - np.array([[1.0], [2.0]], dtype=np.float32)
    np.testing.assert_allclose(w.grad.numpy(), (2 * da * xa).sum(0, keepdims=True), rtol=RTOL, atol=ATOL)
    assert float(b.grad) == pytest.approx(float((2 * da).sum()), rel=RTOL)


def test_backward_broadcast_grad_reduces_to_param_shape(ox):
    """test_autograd.py:35-41."""
    w = _t(ox, [1.0, 2.0, 3.0], requires_grad=True)
    x = _t(ox, np.ones((4, 3)))
    (x * w).sum().backward()
    np.testing.assert_allclose(w.grad.numpy(), np.full(3, 4.0, dtype=np.float32), rtol=RTOL)


def test_grad_accumulates_over_multiple_backward_calls(ox):
    """test_autograd.py:44-49."""
    w = _t(ox, [1.0], requires_grad=True)
    x = _t(ox, [2.0])
    (x * w).sum().backward()
    (x * w).sum().backward()
    assert float(w.grad) == pytest.approx(4.0, rel=RTOL)


def test_no_grad_leaf_has_no_grad(ox):
    """test_autograd.py:52-57."""
    x = _t(ox, [1.0, 2.0])
    y = (x * x).sum()
    with pytest.raises(ValueError):
        y.backward()
    assert x.grad is None


def test_detach_and_zero_grad(ox):
    """test_autograd.py:60-67."""
    w = _t(ox, [1.0], requires_grad=True)
    y = (w * w).sum()
    y.backward()
    d = w.detach()
    assert not d.requires_grad
    w.zero_grad()
    assert w.grad is not None and float(w.grad) == 0.0


def test_sgd_training_converges(ox):
    """test_autograd.py:70-89: y = 2x + 1 fitted through the origin; xs @ w
    for a (1, 1) weight is the broadcast product xs * w."""
    xs_np = (np.arange(8, dtype=np.float32) * 0.5 - 1.5).reshape(8, 1)
    ys_np = (2.0 * xs_np + 1.0).astype(np.float32)
    fixed_point = float((2 * xs_np * ys_np).sum() / (2 * xs_np * xs_np).sum())
    w = _t(ox, [[2.5]], requires_grad=True)
    xs, ys = _t(ox, xs_np), _t(ox, ys_np)
    lr = 0.01
    for _ in range(500):
        pred = xs * w
        loss = ((pred - ys) * (pred - ys)).sum()
        loss.backward()
        g = w.grad.numpy().copy()
        w.zero_grad()
        w = _t(ox, w.detach().numpy() - lr * g, requires_grad=True)
    assert float(w) == pytest.approx(fixed_point, abs=0.02)


def test_unary_grads_via_apply(ox):
    """test_autograd.py:92-110."""
    x_np = np.array([0.3, -0.6, 1.2], dtype=np.float32)
    w_np = np.ones(3, dtype=np.float32)
    for name, np_grad in [
        ("sigmoid", lambda v: (1 / (1 + np.exp(-v))) * (1 - 1 / (1 + np.exp(-v)))),
        ("tanh", lambda v: 1 - np.tanh(v) ** 2),
        ("exp", lambda v: np.exp(v)),
        ("relu", lambda v: (v > 0).astype(np.float32)),
    ]:
        x = _t(ox, x_np, requires_grad=True)
        loss = (x.apply(name) * _t(ox, w_np)).sum()
        loss.backward()
        np.testing.assert_allclose(x.grad.numpy(), np_grad(x_np.astype(np.float64)).astype(np.float32),
                                   rtol=RTOL, atol=ATOL)


# ---- python/tests/test_grad_mode.py --------------------------------------------------------

def test_is_grad_enabled_default(ox):
    assert ox.is_grad_enabled() is True


def test_no_grad_detaches_op_results(ox):
    x = _t(ox, [1.0, 2.0], requires_grad=True)
    with ox.no_grad():
        assert ox.is_grad_enabled() is False
        y = x * x
        assert y.requires_grad is False
        assert np.allclose(y.numpy(), [1.0, 4.0])
    z = x * x
    assert z.requires_grad is True


def test_no_grad_restores_mode_on_exception(ox):
    x = _t(ox, [1.0], requires_grad=True)
    with pytest.raises(RuntimeError, match="boom"):
        with ox.no_grad():
            raise RuntimeError("boom")
    assert ox.is_grad_enabled() is True
    assert (x * x).requires_grad is True


def test_nested_enable_grad_inside_no_grad(ox):
    x = _t(ox, [3.0, -1.0], requires_grad=True)
    with ox.no_grad():
        with ox.enable_grad():
            assert ox.is_grad_enabled() is True
            z = x * x
            assert z.requires_grad is True
        assert ox.is_grad_enabled() is False
        w = x * x
        assert w.requires_grad is False
    assert ox.is_grad_enabled() is True


def test_enable_grad_inside_no_grad_backward_flows(ox):
    x = _t(ox, [2.0], requires_grad=True)
    with ox.no_grad():
        with ox.enable_grad():
            y = x * 3.0
    loss = (y * y).sum()
    loss.backward()
    assert np.allclose(x.grad.numpy(), [36.0], atol=1e-6)


def _affine(ox, seed):
    """Stand-in for nn.Linear(2, 2, seed): y = x * w + b with (2,) leaves."""
    r = np.random.default_rng(seed)
    w = _t(ox, r.standard_normal(2), requires_grad=True)
    b = _t(ox, r.standard_normal(2), requires_grad=True)
    return w, b


def test_backward_through_no_grad_output_rejected(ox):
    """test_grad_mode.py:70-78 (nn.Linear replaced by a broadcast affine map)."""
    w, b = _affine(ox, 1)
    x = _t(ox, [[1.0, 2.0]])
    with ox.no_grad():
        out = x * w + b
    with pytest.raises(ValueError, match="does not require grad"):
        out.sum().backward()
    assert w.grad is None and b.grad is None


def test_no_grad_inference_leaves_params_untouched(ox):
    """test_grad_mode.py:81-89."""
    w1, b1 = _affine(ox, 3)
    w2, b2 = _affine(ox, 4)
    x = _t(ox, [[0.5, -1.5]])
    with ox.no_grad():
        out = (x * w1 + b1).apply("relu") * w2 + b2
    assert out.requires_grad is False
    assert all(p.grad is None for p in (w1, b1, w2, b2))


def test_set_grad_enabled_manual_save_restore(ox):
    prev = ox.set_grad_enabled(False)
    try:
        assert ox.is_grad_enabled() is False
    finally:
        ox.set_grad_enabled(prev)
    assert ox.is_grad_enabled() is True


def test_default_backward_consumes_graph(ox):
    w = _t(ox, [2.0], requires_grad=True)
    loss = (w * w).sum()
    loss.backward()
    assert np.allclose(w.grad.numpy(), [4.0])
    with pytest.raises(ValueError, match="retain_graph"):
        loss.backward()


def test_retain_graph_accumulates_leaf_grads(ox):
    w = _t(ox, [2.0], requires_grad=True)
    loss = (w * w).sum()
    loss.backward(retain_graph=True)
    assert np.allclose(w.grad.numpy(), [4.0])
    loss.backward(retain_graph=True)
    assert np.allclose(w.grad.numpy(), [8.0])
    loss.backward()
    assert np.allclose(w.grad.numpy(), [12.0])


def test_retain_passes_do_not_compound_intermediates(ox):
    a = _t(ox, [3.0], requires_grad=True)
    b = (a * a).sum()
    c = (b * 2.0).sum()
    c.backward(retain_graph=True)
    first = a.grad.item()
    c.backward(retain_graph=True)
    second = a.grad.item()
    assert abs(first - 12.0) < 1e-5 and abs(second - 24.0) < 1e-5


def test_two_losses_into_one_leaf_accumulate(ox):
    w = _t(ox, [1.0, 2.0], requires_grad=True)
    l1 = (w * w).sum()
    l2 = (w * 3.0).sum()
    l1.backward(retain_graph=True)
    l2.backward()
    assert np.allclose(w.grad.numpy(), [2.0 * 1.0 + 3.0, 2.0 * 2.0 + 3.0])


# ---- python/tests/test_nn.py:133-160 and python/tests/test_smoke.py:167-176 -----------------

def test_scalar_arithmetic_autograd(ox):
    t = _t(ox, [1.0, 2.0], requires_grad=True)
    (t * 2.0 + 1.0).sum().backward()
    assert np.allclose(t.grad.numpy(), [2.0, 2.0], atol=1e-6)
    t.zero_grad()
    (2.0 - t).sum().backward()
    assert np.allclose(t.grad.numpy(), [-1.0, -1.0], atol=1e-6)
    t.zero_grad()
    (2.0 / t).sum().backward()
    assert np.allclose(t.grad.numpy(), -2.0 / np.array([1.0, 4.0]), atol=1e-6)
    t.zero_grad()
    (t**3).sum().backward()
    assert np.allclose(t.grad.numpy(), [3.0, 12.0], atol=1e-5)


def test_apply_neg_abs_are_differentiable(ox):
    t = _t(ox, [1.0, -2.0], requires_grad=True)
    t.mean().apply("neg").backward()
    assert np.allclose(t.grad.numpy(), [-0.5, -0.5], atol=1e-6)
    t.zero_grad()
    t.apply("abs").sum().backward()
    assert np.allclose(t.grad.numpy(), [1.0, -1.0], atol=1e-6)


def test_strided_op_parity(ox):
    """Ops on non-contiguous views match NumPy."""
    a = np.random.default_rng(0).standard_normal((4, 5)).astype(np.float32)
    t = _t(ox, a)
    tr = t.transpose()
    np.testing.assert_allclose(tr.apply("square").numpy(), a.T ** 2, rtol=RTOL, atol=ATOL)
    sliced = t[1:4:2]
    np.testing.assert_allclose(sliced.apply("neg").numpy(), -a[1:4:2], rtol=RTOL, atol=ATOL)
    np.testing.assert_allclose(tr.sum(0).numpy(), a.sum(1), rtol=RTOL, atol=ATOL)


def test_full_round_trip(ox):
    a = np.random.default_rng(1).standard_normal((3, 4)).astype(np.float32)
    back = _t(ox, a).numpy()
    np.testing.assert_array_equal(back, a)
    assert back.dtype == np.float32 and not math.isnan(float(back[0, 0]))
