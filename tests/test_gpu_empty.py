"""Zero-size inputs through the drop-in surface (F.* and backward()) on the
GPU, with the reference's outcomes: empty outputs and input gradients, weight
and table gradients of zeros (a sum over no rows is 0: ops.rs:247-249), a
cross-entropy of an empty batch of -0.0 (reduce_all's Mean of an empty strip
is 0, negated: bindings lib.rs:126-143), and the reference's error for a max
over a zero-length dim (lib.rs:527-531)."""

import sys

import numpy as np
import pytest

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


def T(ox, a, g=False):
    return ox.from_numpy(np.ascontiguousarray(a, dtype=np.float32), g)


def is_pos_zero(a):
    a = np.asarray(a)
    return bool(np.all(a == 0) and not np.any(np.signbit(a)))


@pytest.mark.parametrize("H", [768, 4096])
def test_norms_and_activations(ox, F, H):
    say("empty norms", H)
    x, w, b = T(ox, np.zeros((0, H)), True), T(ox, np.ones(H), True), T(ox, np.zeros(H), True)
    y = F.gelu(F.layer_norm(x, w, b), approximate="none")
    assert y.numpy().shape == (0, H)
    y.backward(T(ox, np.zeros((0, H))))
    assert x.grad.numpy().shape == (0, H)
    assert is_pos_zero(w.grad.numpy()) and w.grad.numpy().shape == (H,)
    assert is_pos_zero(b.grad.numpy())
    x2, w2 = T(ox, np.zeros((0, H)), True), T(ox, np.ones(H), True)
    z = F.silu(F.rms_norm(x2, w2))
    z.backward(T(ox, np.zeros((0, H))))
    assert z.numpy().shape == (0, H) and x2.grad.numpy().shape == (0, H)
    assert is_pos_zero(w2.grad.numpy())


def test_softmax_family(ox, F):
    say("empty softmax")
    for fn in (F.softmax, F.log_softmax):
        x = T(ox, np.zeros((0, 10)), True)
        y = fn(x, -1)
        y.backward(T(ox, np.zeros((0, 10))))
        assert y.numpy().shape == (0, 10) and x.grad.numpy().shape == (0, 10)
        with pytest.raises(ValueError, match="cannot compute max/min over a zero-length dim"):
            fn(T(ox, np.zeros((3, 0))), -1)


@pytest.mark.parametrize("c", [1000, 1003])
def test_cross_entropy_of_an_empty_batch(ox, F, c, hip):
    say("empty cross_entropy", c)
    x = T(ox, np.zeros((0, c)), True)
    loss = F.cross_entropy(x, np.zeros(0, np.int64))
    v = loss.item()
    assert v == 0.0 and np.signbit(v)
    loss.backward()
    assert x.grad.numpy().shape == (0, c)
    # the C-ABI, both forwards
    dl = hip.DeviceArray((0, c))
    dt = hip.DeviceArray((0,), np.int64)
    l1, _ = hip.cross_entropy_fwd(dl, dt)
    assert np.signbit(l1.numpy()[0]) and l1.numpy()[0] == 0.0
    if c % 4 == 0:
        l2, _, _ = hip.cross_entropy_fwd_grad(dl, dt)
        assert np.signbit(l2.numpy()[0]) and l2.numpy()[0] == 0.0


def test_embedding_with_no_ids(ox, F):
    say("empty embedding")
    W = T(ox, np.ones((10, 8)), True)
    y = F.embedding(np.zeros(0, np.int64), W)
    assert y.numpy().shape == (0, 8)
    y.sum().backward()
    assert is_pos_zero(W.grad.numpy()) and W.grad.numpy().shape == (10, 8)


def test_reductions_of_empty(ox):
    say("empty reductions")
    for g in (False, True):
        x = T(ox, np.zeros((0, 5)), g)
        assert is_pos_zero(x.sum().item()) and is_pos_zero(x.mean().item())
        assert is_pos_zero(x.sum(0).numpy()) and x.sum(0).numpy().shape == (5,)
        assert is_pos_zero(x.mean(0).numpy())
        with pytest.raises(ValueError, match="zero-length dim"):
            x.max(0)
