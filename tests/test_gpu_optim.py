"""Optimizer steps on the device: the oxi_sgd_step / oxi_adamw_step kernels
bit-exact against the CPU oracle (crates/oxi-autograd/src/optim.rs:104-137,
223-262) over several steps, sizes, alignments and special values; then the
reference's optimizer tests (python/tests/test_rust_optim.py,
test_phase4_training.py) through oxitorch_amd.optim. Models with matmul are
outside this build, so those tests use LayerNorm / Embedding models or set
gradients directly."""

import sys

import numpy as np
import pytest

from conftest import rng

pytestmark = pytest.mark.gpu


def say(*a):
    print("[case]", *a, flush=True)
    sys.stdout.flush()


def bits_equal(got, want, what):
    got = np.ascontiguousarray(got, dtype=np.float32)
    want = np.ascontiguousarray(want, dtype=np.float32)
    assert got.shape == want.shape, what
    gb, wb = got.view(np.uint32), want.view(np.uint32)
    # every NaN payload counts as one value
    gb = np.where(np.isnan(got), np.uint32(0x7FC00000), gb)
    wb = np.where(np.isnan(want), np.uint32(0x7FC00000), wb)
    bad = np.flatnonzero(gb != wb)
    if bad.size:
        i = bad[0]
        raise AssertionError(f"{what}: {bad.size} of {got.size} differ; first at {i}: got {got.ravel()[i]!r} "
                             f"want {want.ravel()[i]!r}")


@pytest.fixture(scope="module")
def oracle():
    from oracle import ref

    return ref


def _special(r, n):
    """Values that stress the update: zeros, signed zeros, tiny and denormal
    gradients, large magnitudes whose square overflows, and ordinary noise."""
    x = r.standard_normal(n).astype(np.float32)
    if n >= 16:
        x[0], x[1] = 0.0, -0.0
        x[2], x[3] = 1e-40, -3e-39  # denormal
        x[4], x[5] = 3e21, -2e20  # (1-beta2)*g*g overflows to inf for the first
        x[6] = 1e-20
    return x


class _Buf:
    """A device copy of a host array, optionally offset by one float so the
    kernels take their unaligned (scalar) path."""

    def __init__(self, hip, a, shift):
        self.shift = shift
        self.dev = hip.DeviceArray.from_numpy(np.concatenate([np.zeros(shift, np.float32), a]))
        self.n = a.size

    @property
    def ptr(self):
        return None if self.dev.ptr is None else self.dev.ptr + 4 * self.shift

    def numpy(self):
        return self.dev.numpy()[self.shift:]


SIZES = [1, 3, 4, 7, 64, 1021, 4096, 65539]


@pytest.mark.parametrize("shift", [0, 1])
@pytest.mark.parametrize("n", SIZES)
@pytest.mark.parametrize("mode", ["plain", "momentum", "nesterov"])
def test_sgd_step_matches_oracle(hip, oracle, mode, n, shift):
    say("sgd_step", mode, n, shift)
    r = rng(1000 + n + shift)
    momentum = 0.0 if mode == "plain" else 0.9
    nesterov = mode == "nesterov"
    lr = 0.05
    p = r.standard_normal(n).astype(np.float32)
    d_p = _Buf(hip, p, shift)
    d_buf = _Buf(hip, np.zeros(n, np.float32), shift)
    buf = np.zeros(n, np.float32)
    for step in range(4):
        g = _special(r, n)
        d_g = _Buf(hip, g, shift)
        want = oracle.sgd_step(p, g, buf if momentum > 0 else None, lr, momentum, nesterov)
        # in place on even steps, into a fresh output on odd ones
        if step % 2 == 0:
            out = d_p
        else:
            out = _Buf(hip, np.zeros(n, np.float32), shift)
        hip.call("oxi_sgd_step", d_p.ptr, d_g.ptr, d_buf.ptr if momentum > 0 else None, out.ptr, n, lr, momentum,
                 int(nesterov))
        bits_equal(out.numpy(), want, f"sgd {mode} n={n} step {step} params")
        if momentum > 0:
            bits_equal(d_buf.numpy(), buf, f"sgd {mode} n={n} step {step} velocity")
        p, d_p = want, out


@pytest.mark.parametrize("shift", [0, 1])
@pytest.mark.parametrize("n", SIZES)
@pytest.mark.parametrize("decoupled,wd", [(True, 0.01), (False, 0.1), (True, 0.0), (False, 0.0)])
def test_adamw_step_matches_oracle(hip, oracle, decoupled, wd, n, shift):
    say("adamw_step", decoupled, wd, n, shift)
    r = rng(2000 + n + shift)
    lr, b1, b2, eps = 1e-3, 0.9, 0.999, 1e-8
    p = r.standard_normal(n).astype(np.float32)
    m = np.zeros(n, np.float32)
    v = np.zeros(n, np.float32)
    d_p = _Buf(hip, p, shift)
    d_m = _Buf(hip, m, shift)
    d_v = _Buf(hip, v, shift)
    for t in range(1, 6):
        g = _special(r, n)
        d_g = _Buf(hip, g, shift)
        want = oracle.adamw_step(p, g, m, v, t, lr, b1, b2, eps, wd, decoupled)
        out = d_p if t % 2 else _Buf(hip, np.zeros(n, np.float32), shift)
        hip.call("oxi_adamw_step", d_p.ptr, d_g.ptr, d_m.ptr, d_v.ptr, out.ptr, n, lr, b1, b2, eps, wd,
                 int(decoupled), t)
        bits_equal(out.numpy(), want, f"adam t={t} params")
        bits_equal(d_m.numpy(), m, f"adam t={t} m")
        bits_equal(d_v.numpy(), v, f"adam t={t} v")
        p, d_p = want, out


def test_adamw_large_step_count_and_hyperparameters(hip, oracle):
    """Late steps (bias corrections near 1) and non-default betas/eps."""
    say("adamw late steps")
    r = rng(7)
    n = 10007
    p = r.standard_normal(n).astype(np.float32)
    m = (r.standard_normal(n) * 0.1).astype(np.float32)
    v = np.abs(r.standard_normal(n) * 0.01).astype(np.float32)
    g = r.standard_normal(n).astype(np.float32)
    d = [hip.DeviceArray.from_numpy(a) for a in (p, g, m, v)]
    for t, (b1, b2, eps, lr) in [(1000, (0.8, 0.99, 1e-6, 3e-4)), (123456, (0.9, 0.95, 1e-5, 1e-2))]:
        mm, vv = m.copy(), v.copy()
        want = oracle.adamw_step(p, g, mm, vv, t, lr, b1, b2, eps, 0.05, True)
        dm, dv = hip.DeviceArray.from_numpy(m), hip.DeviceArray.from_numpy(v)
        out = hip.adamw_step(d[0], d[1], dm, dv, t, lr, b1, b2, eps, 0.05, True)
        bits_equal(out.numpy(), want, f"adam t={t}")
        bits_equal(dm.numpy(), mm, f"adam t={t} m")
        bits_equal(dv.numpy(), vv, f"adam t={t} v")


def test_optimizer_steps_at_bench_size(hip, oracle):
    """The bench workload's flat size (GPT-2 small, 124,439,808 floats) in one
    launch each, bit-exact against the oracle over every element."""
    say("optim bench size")
    n = 124_439_808
    r = rng(11)
    p = r.standard_normal(n, dtype=np.float32)
    g = r.standard_normal(n, dtype=np.float32)
    m = r.standard_normal(n, dtype=np.float32) * np.float32(0.1)
    v = r.random(n, dtype=np.float32) * np.float32(0.01)
    dp, dg, dm, dv = (hip.DeviceArray.from_numpy(a) for a in (p, g, m, v))
    out = hip.adamw_step(dp, dg, dm, dv, 3, 6e-4, 0.9, 0.95, 1e-8, 0.1, True)
    want = oracle.adamw_step(p, g, m, v, 3, 6e-4, 0.9, 0.95, 1e-8, 0.1, True)
    bits_equal(out.numpy(), want, "adam bench size")
    bits_equal(dm.numpy(), m, "adam bench size m")
    bits_equal(dv.numpy(), v, "adam bench size v")
    del out, want, dm, dv, m, v
    buf = r.standard_normal(n, dtype=np.float32) * np.float32(0.1)
    dbuf = hip.DeviceArray.from_numpy(buf)
    out = hip.sgd_step(dp, dg, dbuf, 0.01, 0.9, True)
    want = oracle.sgd_step(p, g, buf, 0.01, 0.9, True)
    bits_equal(out.numpy(), want, "sgd bench size")
    bits_equal(dbuf.numpy(), buf, "sgd bench size velocity")


# sizes of a mixed parameter list: empty, tails, one float4, biases, and more
# than one launch's worth of slices (32 per launch)
MULTI_SIZES = [0, 1, 3, 4, 5, 768, 2304, 3, 65536 + 3] + [768] * 30 + [4099, 0, 100003]


@pytest.mark.parametrize("misaligned", [False, True])
def test_adamw_step_multi_matches_oracle(hip, oracle, misaligned):
    """A parameter list in one call, each slice with its own step count,
    against the oracle slice by slice; with `misaligned`, every third slice is
    offset by one float (those slices take the single-parameter path)."""
    say("adamw_step_multi", misaligned)
    r = rng(31)
    lr, b1, b2, eps, wd = 3e-3, 0.9, 0.95, 1e-8, 0.1
    host, dev = [], []
    for i, n in enumerate(MULTI_SIZES):
        shift = 1 if misaligned and i % 3 == 0 else 0
        arrs = dict(p=r.standard_normal(n).astype(np.float32), g=_special(r, n),
                    m=(r.standard_normal(n) * 0.1).astype(np.float32),
                    v=(r.random(n) * 0.01).astype(np.float32))
        host.append(arrs)
        dev.append({k: _Buf(hip, a, shift) for k, a in arrs.items()} | {"out": _Buf(hip, np.zeros(n, np.float32), shift)})
    for rep in range(2):
        ts = [1 + (i * 7 + rep) % 5 for i in range(len(MULTI_SIZES))]
        rows = [(d["p"].ptr, d["g"].ptr, d["m"].ptr, d["v"].ptr, d["out"].ptr, n, t)
                for d, n, t in zip(dev, MULTI_SIZES, ts)]
        hip.call("oxi_adamw_step_multi", hip.slice_array(hip.AdamWSlice, rows), len(rows), lr, b1, b2, eps, wd, 1)
        for i, (h, d, t) in enumerate(zip(host, dev, ts)):
            want = oracle.adamw_step(h["p"], h["g"], h["m"], h["v"], t, lr, b1, b2, eps, wd, True)
            bits_equal(d["out"].numpy(), want, f"slice {i} n={MULTI_SIZES[i]} rep {rep}")
            bits_equal(d["m"].numpy(), h["m"], f"slice {i} m rep {rep}")
            bits_equal(d["v"].numpy(), h["v"], f"slice {i} v rep {rep}")


@pytest.mark.parametrize("mode", ["plain", "momentum", "nesterov"])
def test_sgd_step_multi_matches_oracle(hip, oracle, mode):
    say("sgd_step_multi", mode)
    r = rng(32)
    momentum = 0.0 if mode == "plain" else 0.9
    nesterov = mode == "nesterov"
    host, dev = [], []
    for i, n in enumerate(MULTI_SIZES):
        shift = 1 if i % 5 == 2 else 0
        arrs = dict(p=r.standard_normal(n).astype(np.float32), g=_special(r, n),
                    buf=(r.standard_normal(n) * 0.1).astype(np.float32))
        host.append(arrs)
        dev.append({k: _Buf(hip, a, shift) for k, a in arrs.items()} | {"out": _Buf(hip, np.zeros(n, np.float32), shift)})
    rows = [(d["p"].ptr, d["g"].ptr, d["buf"].ptr if momentum > 0 else None, d["out"].ptr, n)
            for d, n in zip(dev, MULTI_SIZES)]
    hip.call("oxi_sgd_step_multi", hip.slice_array(hip.SgdSlice, rows), len(rows), 0.02, momentum, int(nesterov))
    for i, (h, d) in enumerate(zip(host, dev)):
        want = oracle.sgd_step(h["p"], h["g"], h["buf"] if momentum > 0 else None, 0.02, momentum, nesterov)
        bits_equal(d["out"].numpy(), want, f"slice {i}")
        if momentum > 0:
            bits_equal(d["buf"].numpy(), h["buf"], f"slice {i} velocity")


def test_step_multi_argument_errors(hip):
    a = hip.DeviceArray((8,))
    ok = (a.ptr, a.ptr, a.ptr, a.ptr, a.ptr, 8, 1)
    with pytest.raises(ValueError, match="slice 1: step count"):
        hip.call("oxi_adamw_step_multi", hip.slice_array(hip.AdamWSlice, [ok, ok[:6] + (0,)]), 2, 0.1, 0.9, 0.99,
                 1e-8, 0.0, 1)
    with pytest.raises(ValueError, match="slice 0 has a NULL pointer"):
        hip.call("oxi_sgd_step_multi", hip.slice_array(hip.SgdSlice, [(a.ptr, a.ptr, None, a.ptr, 8)]), 1, 0.1, 0.9,
                 0)
    with pytest.raises(ValueError, match="nesterov"):
        hip.call("oxi_sgd_step_multi", hip.slice_array(hip.SgdSlice, []), 0, 0.1, 0.0, 1)
    hip.call("oxi_adamw_step_multi", None, 0, 0.1, 0.9, 0.99, 1e-8, 0.0, 1)


def test_step_argument_errors(hip):
    with pytest.raises(ValueError, match="nesterov momentum requires momentum > 0"):
        hip.call("oxi_sgd_step", None, None, None, None, 4, 0.1, 0.0, 1)
    with pytest.raises(ValueError, match="step count"):
        hip.call("oxi_adamw_step", None, None, None, None, None, 4, 0.1, 0.9, 0.999, 1e-8, 0.0, 1, 0)
    with pytest.raises(ValueError, match="state buffer"):
        a = hip.DeviceArray((4,))
        hip.call("oxi_sgd_step", a.ptr, a.ptr, None, a.ptr, 4, 0.1, 0.9, 0)
    hip.call("oxi_adamw_step", None, None, None, None, None, 0, 0.1, 0.9, 0.999, 1e-8, 0.0, 1, 1)  # empty: no-op


# ---- the host core and oxitorch_amd.optim ------------------------------------------------

@pytest.fixture(scope="module")
def ox(hip):
    import oxitorch_amd

    return oxitorch_amd


def _t(ox, arr, requires_grad=False):
    return ox.from_numpy(np.ascontiguousarray(arr, dtype=np.float32), requires_grad)


def _ln_model(ox, seed=0, d=8):
    """y = layer_norm(x) * w + b with trainable w, b (stands in for the
    reference tests' Linear layers)."""
    import oxitorch_amd.nn as nn

    layer = nn.LayerNorm(d)
    r = rng(seed)
    layer.weight.tensor = _t(ox, 1.0 + 0.3 * r.standard_normal(d), True)
    layer.bias.tensor = _t(ox, 0.1 * r.standard_normal(d), True)
    return layer


def _ln_data(seed=0, rows=5, d=8):
    r = rng(seed + 100)
    return r.standard_normal((rows, d)).astype(np.float32), r.standard_normal((rows, d)).astype(np.float32)


def test_adamw_through_backward_matches_oracle(ox, oracle):
    """python/tests/test_rust_optim.py:33-60 with a LayerNorm model: each step
    reads the gradients backward() left on the device, and the updated
    parameters equal the oracle's step from those gradients, bit for bit."""
    import oxitorch_amd.nn.functional as F
    import oxitorch_amd.optim as op

    say("api adamw backward")
    x, y = _ln_data()
    layer = _ln_model(ox)
    lr, b1, b2, eps, wd = 0.05, 0.9, 0.999, 1e-8, 0.1
    opt = op.AdamW(layer.parameters(), lr=lr, betas=(b1, b2), eps=eps, weight_decay=wd)
    state = {name: (np.zeros(8, np.float32), np.zeros(8, np.float32)) for name in ("weight", "bias")}
    for t in range(1, 4):
        layer.zero_grad()
        F.mse_loss(layer(_t(ox, x)), _t(ox, y)).backward()
        before = {k: getattr(layer, k).tensor.numpy() for k in state}
        grads = {k: getattr(layer, k).grad.numpy() for k in state}
        opt.step()
        for k, (m, v) in state.items():
            want = oracle.adamw_step(before[k], grads[k], m, v, t, lr, b1, b2, eps, wd, True)
            bits_equal(getattr(layer, k).tensor.numpy(), want, f"{k} step {t}")


def test_sgd_momentum_through_backward_matches_oracle(ox, oracle):
    """python/tests/test_rust_optim.py:63-83, plus the Nesterov variant."""
    import oxitorch_amd.nn.functional as F
    import oxitorch_amd.optim as op

    for nesterov in (False, True):
        say("api sgd backward", nesterov)
        x, y = _ln_data(1)
        layer = _ln_model(ox, 1)
        opt = op.Sgd(layer.parameters(), lr=0.1, momentum=0.9, nesterov=nesterov)
        bufs = {k: np.zeros(8, np.float32) for k in ("weight", "bias")}
        for _ in range(3):
            layer.zero_grad()
            F.mse_loss(layer(_t(ox, x)), _t(ox, y)).backward()
            before = {k: getattr(layer, k).tensor.numpy() for k in bufs}
            grads = {k: getattr(layer, k).grad.numpy() for k in bufs}
            opt.step()
            for k, b in bufs.items():
                want = oracle.sgd_step(before[k], grads[k], b, 0.1, 0.9, nesterov)
                bits_equal(getattr(layer, k).tensor.numpy(), want, f"{k} nesterov={nesterov}")


def test_step_preserves_tensor_identity(ox):
    """python/tests/test_rust_optim.py:86-104."""
    import oxitorch_amd.nn.functional as F
    import oxitorch_amd.optim as op

    x, y = _ln_data(2)
    layer = _ln_model(ox, 2)
    weight_obj, bias_obj = layer.weight.tensor, layer.bias.tensor
    weight_before = weight_obj.numpy().copy()
    opt = op.AdamW(layer.parameters(), lr=0.05)
    for _ in range(3):
        layer.zero_grad()
        F.mse_loss(layer(_t(ox, x)), _t(ox, y)).backward()
        opt.step()
        assert layer.weight.tensor is weight_obj
        assert layer.bias.tensor is bias_obj
        assert weight_obj.requires_grad and weight_obj.grad is None  # a fresh leaf
    assert not np.allclose(weight_before, weight_obj.numpy())


def test_lazy_state_param_without_grad_gets_fresh_buffers(ox):
    """python/tests/test_rust_optim.py:107-135."""
    import oxitorch_amd.optim as op

    g = np.array([0.5, -0.5], dtype=np.float32)
    w_fresh = _t(ox, [1.0, 2.0], True)
    fresh = op.AdamW([w_fresh], lr=0.1, weight_decay=0.0)
    w_fresh.grad = _t(ox, g)
    fresh.step()
    one_step = w_fresh.numpy().copy()
    np.testing.assert_allclose(one_step, [0.9, 2.1], rtol=1e-6)  # lr * sign(g)

    w_lazy = _t(ox, [1.0, 2.0], True)
    w_other = _t(ox, [1.0, 2.0], True)
    lazy = op.AdamW([w_other, w_lazy], lr=0.1, weight_decay=0.0)
    w_other.grad = _t(ox, g)
    lazy.step()  # w_lazy has no gradient: no state, no counter advance
    assert w_lazy.numpy().tolist() == [1.0, 2.0]
    w_other.grad = _t(ox, g)
    w_lazy.grad = _t(ox, g)
    lazy.step()
    bits_equal(w_lazy.numpy(), one_step, "lazy first step")


def test_scheduler_lr_mutation_reaches_engine(ox):
    """python/tests/test_rust_optim.py:138-148."""
    import oxitorch_amd.optim as op

    w = _t(ox, [1.0], True)
    opt = op.Sgd([w], lr=0.1)
    opt.lr = 0.5
    assert opt.lr == 0.5
    w.grad = _t(ox, [1.0])
    opt.step()
    np.testing.assert_allclose(w.numpy(), [0.5], rtol=1e-6)


def test_state_survives_parameter_rebinding(ox):
    """python/tests/test_rust_optim.py:151-167."""
    import oxitorch_amd.optim as op

    g = np.array([1.0], dtype=np.float32)
    w = _t(ox, [1.0], True)
    opt = op.Sgd([w], lr=0.1, momentum=0.9)
    w.grad = _t(ox, g)
    opt.step()
    w2 = _t(ox, [0.9], True)
    opt.params = [w2]
    w2.grad = _t(ox, g)
    opt.step()  # buf = 1.9, w = 0.9 - 0.19
    np.testing.assert_allclose(w2.numpy(), [0.71], rtol=1e-5, atol=1e-7)


def test_state_size_change_is_an_error(ox):
    """optim.rs:31-51: a parameter whose size changed mid-run is rejected."""
    import oxitorch_amd.optim as op

    w = _t(ox, [1.0, 2.0], True)
    opt = op.AdamW([w], lr=0.1)
    w.grad = _t(ox, [1.0, 1.0])
    opt.step()
    w3 = _t(ox, [1.0, 2.0, 3.0], True)
    w3.grad = _t(ox, [1.0, 1.0, 1.0])
    opt.params = [w3]
    with pytest.raises(ValueError, match="optimizer state for parameter 0 has 2 elements but the parameter now has 3"):
        opt.step()


def test_adam_l2_in_grad_vs_adamw_decoupled(ox, oracle):
    """python/tests/test_phase4_training.py:72-107: Adam folds decay into the
    gradient, AdamW decays the parameter; defaults as torch's."""
    import oxitorch_amd.optim as op

    p0 = np.array([1.0, -2.0, 0.5], np.float32)
    g = np.array([0.3, 0.1, -0.2], np.float32)
    for cls, decoupled in ((op.Adam, False), (op.AdamW, True)):
        w = _t(ox, p0, True)
        opt = cls([w], lr=0.01, weight_decay=0.1)
        m, v = np.zeros(3, np.float32), np.zeros(3, np.float32)
        p = p0
        for t in (1, 2):
            w.grad = _t(ox, g)
            opt.step()
            p = oracle.adamw_step(p, g, m, v, t, 0.01, 0.9, 0.999, 1e-8, 0.1, decoupled)
            bits_equal(w.numpy(), p, f"{cls.__name__} t={t}")
    assert op.AdamW([w]).weight_decay == 1e-2
    assert op.Adam([w]).weight_decay == 0.0


def test_training_loop_reaches_solution(ox):
    """python/tests/test_rust_optim.py:170-192 with an embedding table fitted
    to random targets through a LayerNorm-free lookup."""
    import oxitorch_amd.nn as nn
    import oxitorch_amd.nn.functional as F
    import oxitorch_amd.optim as op

    r = rng(7)
    ids = r.integers(0, 16, 48)
    y = r.standard_normal((48, 8)).astype(np.float32)
    emb = nn.Embedding(16, 8, seed=0)
    opt = op.AdamW(emb.parameters(), lr=0.05)
    first = final = None
    for _ in range(150):
        opt.zero_grad()
        loss = F.mse_loss(emb(ids.tolist()), _t(ox, y))
        loss.backward()
        opt.step()
        final = float(loss.numpy())
        first = final if first is None else first
    assert np.isfinite(final)
    # the optimum puts each row at its ids' mean target: the loss floor is the
    # within-id spread of the targets
    floor = float(np.mean(np.concatenate([y[ids == k] - y[ids == k].mean(0) for k in np.unique(ids)]) ** 2))
    assert final < floor + 0.1 * (first - floor), f"loss {first} -> {final} (floor {floor})"


def test_many_parameters_one_step_matches_per_parameter_oracle(ox, oracle):
    """A GPT-2-like parameter list (70 tensors, three launches of the
    multi-slice kernel) stepped by AdamW.step() equals the oracle parameter by
    parameter, with a parameter that has no gradient on the first step."""
    import oxitorch_amd.optim as op

    say("api many params")
    r = rng(40)
    shapes = [(64, 48), (32, 48)] + [(48,), (48,), (48, 144), (144,), (48, 48), (48,)] * 11 + [(48,), (48,)]
    params = [_t(ox, r.standard_normal(s), True) for s in shapes]
    opt = op.AdamW(params, lr=0.01, betas=(0.9, 0.95), weight_decay=0.1)
    state = [(np.zeros(int(np.prod(s)), np.float32), np.zeros(int(np.prod(s)), np.float32)) for s in shapes]
    steps = [0] * len(shapes)
    for it in range(3):
        grads = []
        for i, (w, s) in enumerate(zip(params, shapes)):
            if it == 0 and i == 5:
                grads.append(None)
                continue
            g = r.standard_normal(s).astype(np.float32)
            w.grad = _t(ox, g)
            grads.append(g)
        before = [w.numpy() for w in params]
        opt.step()
        for i, (w, g) in enumerate(zip(params, grads)):
            if g is None:
                bits_equal(w.numpy(), before[i], f"param {i} without grad")
                continue
            steps[i] += 1
            m, v = state[i]
            want = oracle.adamw_step(before[i].ravel(), g.ravel(), m, v, steps[i], 0.01, 0.9, 0.95, 1e-8, 0.1, True)
            bits_equal(w.numpy().ravel(), want, f"param {i} step {it}")


def test_duplicate_parameter_is_refused(ox):
    import oxitorch_amd.optim as op

    w = _t(ox, [1.0, 2.0], True)
    w.grad = _t(ox, [1.0, 1.0])
    with pytest.raises(RuntimeError, match="Already borrowed"):
        op.Sgd([w, w], lr=0.1).step()
    np.testing.assert_array_equal(w.numpy(), [1.0, 2.0])


def test_clip_grad_norm(ox):
    """python/tests/test_phase4_training.py:188-240."""
    import oxitorch_amd.nn as nn
    import oxitorch_amd.optim as op

    def pw(arr, grad):
        p = nn.Parameter(_t(ox, arr, True))
        p.tensor.grad = _t(ox, grad)
        return p

    p = pw([[1.0, 2.0]], [[3.0, 4.0]])
    assert op.clip_grad_norm_([p], 1.0) == pytest.approx(5.0)
    np.testing.assert_allclose(p.grad.numpy(), [[0.6, 0.8]], rtol=1e-5)
    p = pw([[1.0, 2.0]], [[3.0, 4.0]])
    assert op.clip_grad_norm_([p], 10.0) == pytest.approx(5.0)
    np.testing.assert_array_equal(p.grad.numpy(), [[3.0, 4.0]])
    pa = pw(np.zeros((1, 3)), [[3.0, 0.0, 0.0]])
    pb = pw(np.zeros((1, 4)), [[0.0, 4.0, 0.0, 0.0]])
    assert op.clip_grad_norm_([pa, pb], 0.5) == pytest.approx(5.0)
    np.testing.assert_allclose(pa.grad.numpy(), [[0.3, 0.0, 0.0]], rtol=1e-5)
    np.testing.assert_allclose(pb.grad.numpy(), [[0.0, 0.4, 0.0, 0.0]], rtol=1e-5)
    p = pw(np.zeros((1, 2)), [[3.0, -4.0]])
    assert op.clip_grad_norm_([p], 1.0, norm_type=float("inf")) == pytest.approx(4.0)
    np.testing.assert_allclose(p.grad.numpy(), [[0.75, -1.0]], rtol=1e-5)
    p = pw(np.zeros((1, 2)), [[3.0, 4.0]])
    assert op.clip_grad_norm_([p], 1.0, norm_type=1.0) == pytest.approx(7.0)
    np.testing.assert_allclose(p.grad.numpy(), [[3.0 / 7.0, 4.0 / 7.0]], rtol=1e-5)
    p_with = pw(np.zeros((1, 2)), [[3.0, 4.0]])
    p_without = nn.Parameter(_t(ox, np.zeros((1, 2)), True))
    assert op.clip_grad_norm_([p_with, p_without], 1.0) == pytest.approx(5.0)


def test_clip_grad_value(ox):
    import oxitorch_amd.nn as nn
    import oxitorch_amd.optim as op

    p = nn.Parameter(_t(ox, np.zeros((1, 3)), True))
    p.tensor.grad = _t(ox, [[5.0, -5.0, 1.0]])
    op.clip_grad_value_([p], 2.0)
    np.testing.assert_array_equal(p.grad.numpy(), [[2.0, -2.0, 1.0]])
    with pytest.raises(ValueError):
        op.clip_grad_value_([p], 0.0)
