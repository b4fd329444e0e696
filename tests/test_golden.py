"""Golden fixtures (tests/golden/): the reference's known-answer tests as data,
and seeded vectors with the oracle's outputs.

CPU: the oracle passes every known-answer test and still reproduces the
committed vectors bit for bit (a change to oracle/refcpu.c that alters a
result fails here). GPU: liboxihip, through its C-ABI, passes the same
known-answer tests and matches the vectors: bit-exact for gathers and argmax,
rtol 1e-5 / atol 1e-6 otherwise (the float64 closed form arbitrates long
sums; cross-entropy gradients are compared as n * dlogits).
"""

import json
from pathlib import Path

import numpy as np
import pytest

from conftest import assert_close, assert_close_arb, assert_reduction_close

GOLDEN = Path(__file__).resolve().parent / "golden"
KATS = json.loads((GOLDEN / "kats.json").read_text())
VEC = dict(np.load(GOLDEN / "vectors.npz"))


def _a(x):
    return np.asarray(x, dtype=np.float32)


def _kat_ids():
    return [k["id"] for k in KATS]


def _check(got, want, kat, what):
    want = np.asarray(want, dtype=np.float64)
    got = np.asarray(got, dtype=np.float64)
    assert got.shape == want.shape, f"{kat['id']} {what}: shape {got.shape} vs {want.shape}"
    tol = kat["atol"] + kat["rtol"] * np.abs(want)
    assert np.all(np.abs(got - want) <= tol), f"{kat['id']} {what} ({kat['source']}): got {got} want {want}"


# ---------------------------------------------------------------------------
# the oracle against the reference's known-answer tests (CPU)

def _oracle_kat(kat):
    from oracle import ref

    op, i, e = kat["op"], kat["inputs"], kat["expected"]
    if op in ("softmax", "log_softmax"):
        y = ref.softmax_fwd(_a(i["x"])) if op == "softmax" else ref.log_softmax_fwd(_a(i["x"]))
        _check(y, e["y"], kat, "y")
    elif op in ("relu", "sigmoid", "tanh"):
        _check(ref.unary(op, _a(i["x"])), e["y"], kat, "y")
    elif op == "silu":
        _check(ref.silu_fwd(_a(i["x"])), e["y"], kat, "y")
    elif op == "gelu_tanh":
        _check(ref.gelu_tanh_fwd(_a(i["x"])), e["y"], kat, "y")
    elif op == "layer_norm":
        y, mu, inv = ref.layer_norm_fwd(_a(i["x"]), _a(i["w"]), _a(i["b"]), i["eps"])
        _check(y, e["y"], kat, "y")
        dx, dw, db = ref.layer_norm_bwd(_a(i["x"]), _a(i["w"]), mu, inv, _a(i["g"]))
        _check(dw, e["dw"], kat, "dw")
        _check(db, e["db"], kat, "db")
        assert np.abs(dx).sum() > e["dx_abs_sum_gt"]
    elif op == "rms_norm":
        y, _ = ref.rms_norm_fwd(_a(i["x"]), _a(i["w"]), i["eps"])
        _check(y, e["y"], kat, "y")
    elif op == "cross_entropy":
        lg, t = _a(i["logits"]), np.asarray(i["targets"], np.int64)
        assert abs(ref.cross_entropy_fwd(lg, t) - e["loss"]) < e["loss_atol"]
        _check(ref.cross_entropy_bwd(lg, t), e["dlogits"], kat, "dlogits")
    elif op in ("embedding", "index_select"):
        src = _a(i["W"] if op == "embedding" else i["src"])
        dim = i.get("dim", 0)
        idx = np.asarray(i["ids"] if op == "embedding" else i["idx"], np.int64)
        if "error" in e:
            with pytest.raises(IndexError):
                ref.index_select(src, dim, idx)
            return
        if "out" in e:
            _check(ref.index_select(src, dim, idx), e["out"], kat, "out")
        if "grad" in e or "dW" in e:
            _check(ref.index_select_bwd(_a(i["g"]), src.shape, dim, idx), e.get("grad", e.get("dW")), kat, "grad")
    elif op == "reduce":
        _check(ref.reduce(i["kind"], _a(i["x"]), i["dim"]), e["y"], kat, "y")
    else:
        raise AssertionError(f"unknown op {op}")


@pytest.mark.parametrize("kat", KATS, ids=_kat_ids())
def test_oracle_known_answers(kat):
    _oracle_kat(kat)


def test_oracle_reproduces_vectors():
    """Every f32 array of vectors.npz is exactly what the oracle computes now."""
    from oracle import ref

    V = VEC
    for name in ("norm_a", "norm_b"):
        x, w, g = V[f"rms_{name}/x"], V[f"rms_{name}/w"], V[f"rms_{name}/g"]
        y, inv = ref.rms_norm_fwd(x, w, 1e-6)
        dx, dw = ref.rms_norm_bwd(x, w, inv, g)
        for k, a in dict(y32=y, inv32=inv, dx32=dx, dw32=dw).items():
            np.testing.assert_array_equal(a, V[f"rms_{name}/{k}"], err_msg=f"rms {name} {k}")
        x, w, b, g = (V[f"ln_{name}/{k}"] for k in ("x", "w", "b", "g"))
        y, mu, inv = ref.layer_norm_fwd(x, w, b, 1e-5)
        dx, dw, db = ref.layer_norm_bwd(x, w, mu, inv, g)
        for k, a in dict(y32=y, mean32=mu, inv32=inv, dx32=dx, dw32=dw, db32=db).items():
            np.testing.assert_array_equal(a, V[f"ln_{name}/{k}"], err_msg=f"ln {name} {k}")
    x, g = V["act/x"], V["act/g"]
    for k, a in dict(gelu_tanh_y32=ref.gelu_tanh_fwd(x), gelu_tanh_dx32=ref.gelu_tanh_bwd(x, g),
                     gelu_erf_y32=ref.gelu_erf_fwd(x), gelu_erf_dx32=ref.gelu_erf_bwd(x, g),
                     silu_y32=ref.silu_fwd(x), silu_dx32=ref.silu_bwd(x, g)).items():
        np.testing.assert_array_equal(a, V[f"act/{k}"], err_msg=k)
    for name in ("a", "b"):
        x, g = V[f"sm_{name}/x"], V[f"sm_{name}/g"]
        for k, a in dict(y32=ref.softmax_fwd(x), dx32=ref.softmax_bwd(x, g), ly32=ref.log_softmax_fwd(x),
                         ldx32=ref.log_softmax_bwd(x, g)).items():
            np.testing.assert_array_equal(a, V[f"sm_{name}/{k}"], err_msg=f"softmax {name} {k}")
    lg, t = V["ce/logits"], V["ce/targets"]
    assert np.float32(ref.cross_entropy_fwd(lg, t)) == V["ce/loss32"][0]
    np.testing.assert_array_equal(ref.cross_entropy_bwd(lg, t), V["ce/d32"])
    W, ids, g = V["emb/W"], V["emb/ids"], V["emb/g"]
    np.testing.assert_array_equal(ref.index_select(W, 0, ids), V["emb/out32"])
    np.testing.assert_array_equal(ref.index_select_bwd(g, W.shape, 0, ids), V["emb/dW32"])
    x = V["red/x"]
    for kind in ("sum", "mean", "max", "min", "argmax", "argmin", "norm"):
        for dim in (0, 1, 2):
            np.testing.assert_array_equal(ref.reduce(kind, x, dim), V[f"red/{kind}_{dim}_32"], err_msg=f"{kind} {dim}")


def test_vectors_oracle_within_tolerance_of_float64():
    """The f32 oracle outputs stored with the vectors sit within the parity
    tolerance of the float64 closed forms stored beside them (what the device
    is held to as well)."""
    V = VEC
    for name in ("norm_a", "norm_b"):
        assert_close(V[f"rms_{name}/y32"], V[f"rms_{name}/y64"], what=f"rms {name}")
        assert_close(V[f"ln_{name}/y32"], V[f"ln_{name}/y64"], what=f"ln {name}")
    for k in ("gelu_tanh_y", "gelu_erf_y", "silu_y"):
        assert_close(V[f"act/{k}32"], V[f"act/{k}64"], what=k)
    for k in ("gelu_erf_dx", "silu_dx"):
        assert_close(V[f"act/{k}32"], V[f"act/{k}64"], what=k)
    for name in ("a", "b"):
        assert_close(V[f"sm_{name}/y32"], V[f"sm_{name}/y64"], what="softmax")
        assert_close(V[f"sm_{name}/ly32"], V[f"sm_{name}/ly64"], what="log_softmax")
    n = V["ce/logits"].shape[0]
    assert_close(V["ce/loss32"], V["ce/loss64"], what="ce loss")
    assert_close(n * V["ce/d32"], n * V["ce/d64"], what="n * dlogits")
    assert_reduction_close(V["emb/dW32"], V["emb/dW32"], V["emb/dW64"], what="dW")


# ---------------------------------------------------------------------------
# the device against the same fixtures (GPU)

def _D(hip, a):
    return hip.DeviceArray.from_numpy(np.ascontiguousarray(a))


def _device_kat(hip, kat):
    op, i, e = kat["op"], kat["inputs"], kat["expected"]
    D = lambda a: _D(hip, a)  # noqa: E731
    if op in ("softmax", "log_softmax"):
        _check(hip.softmax_fwd(D(_a(i["x"])), -1, log=op == "log_softmax").numpy(), e["y"], kat, "y")
    elif op in ("relu", "sigmoid", "tanh"):
        _check(hip.unary(op, D(_a(i["x"]))).numpy(), e["y"], kat, "y")
    elif op == "silu":
        _check(hip.silu_fwd(D(_a(i["x"]))).numpy(), e["y"], kat, "y")
    elif op == "gelu_tanh":
        _check(hip.gelu_fwd(D(_a(i["x"])), "tanh").numpy(), e["y"], kat, "y")
    elif op == "layer_norm":
        x, w = D(_a(i["x"])), D(_a(i["w"]))
        y, mu, inv = hip.layer_norm_fwd(x, w, D(_a(i["b"])), i["eps"])
        _check(y.numpy(), e["y"], kat, "y")
        dx, dw, db = hip.layer_norm_bwd(x, w, mu, inv, D(_a(i["g"])), mode="ref")
        _check(dw.numpy(), e["dw"], kat, "dw")
        _check(db.numpy(), e["db"], kat, "db")
        assert np.abs(dx.numpy()).sum() > e["dx_abs_sum_gt"]
    elif op == "rms_norm":
        y, _ = hip.rms_norm_fwd(D(_a(i["x"])), D(_a(i["w"])), i["eps"])
        _check(y.numpy(), e["y"], kat, "y")
    elif op == "cross_entropy":
        lg, t = D(_a(i["logits"])), D(np.asarray(i["targets"], np.int64))
        loss, lse = hip.cross_entropy_fwd(lg, t)
        assert abs(float(loss.numpy()[0]) - e["loss"]) < e["loss_atol"]
        d = hip.cross_entropy_bwd(lg, t, lse, D(np.ones(1, np.float32)))
        _check(d.numpy(), e["dlogits"], kat, "dlogits")
    elif op in ("embedding", "index_select"):
        src = _a(i["W"] if op == "embedding" else i["src"])
        dim = i.get("dim", 0)
        idx = D(np.asarray(i["ids"] if op == "embedding" else i["idx"], np.int64))
        if "error" in e:  # the C-ABI takes ids on the device: the kernel guard reports them
            hip.index_select(D(src), dim, idx)
            with pytest.raises(RuntimeError, match="outside its valid range"):
                hip.sync()
            return
        if "out" in e:
            _check(hip.index_select(D(src), dim, idx).numpy(), e["out"], kat, "out")
        if "grad" in e or "dW" in e:
            _check(hip.index_select_bwd(D(_a(i["g"])), src.shape, dim, idx).numpy(), e.get("grad", e.get("dW")),
                   kat, "grad")
    elif op == "reduce":
        _check(hip.reduce(i["kind"], D(_a(i["x"])), i["dim"]).numpy(), e["y"], kat, "y")
    else:
        raise AssertionError(f"unknown op {op}")
    hip.sync()


@pytest.mark.gpu
@pytest.mark.parametrize("kat", KATS, ids=_kat_ids())
def test_device_known_answers(hip, kat):
    print(f"[case] golden KAT {kat['id']}", flush=True)
    _device_kat(hip, kat)


@pytest.mark.gpu
def test_device_matches_vectors(hip):
    V = VEC
    D = lambda a: _D(hip, a)  # noqa: E731
    print("[case] golden vectors: norms", flush=True)
    for name in ("norm_a", "norm_b"):
        x, w, g = (D(V[f"rms_{name}/{k}"]) for k in ("x", "w", "g"))
        y, inv = hip.rms_norm_fwd(x, w, 1e-6)
        assert_close(y.numpy(), V[f"rms_{name}/y32"], what=f"rms {name} y")
        dx, dw = hip.rms_norm_bwd(x, w, inv, g, mode="ref")
        assert_close(dx.numpy(), V[f"rms_{name}/dx32"], what=f"rms {name} dx")
        assert_close(dw.numpy(), V[f"rms_{name}/dw32"], what=f"rms {name} dw")
        dx, _ = hip.rms_norm_bwd(x, w, inv, g, mode="exact")
        assert_close(dx.numpy(), V[f"rms_{name}/dx64_exact"], what=f"rms {name} exact dx")
        x, w, b, g = (D(V[f"ln_{name}/{k}"]) for k in ("x", "w", "b", "g"))
        y, mu, inv = hip.layer_norm_fwd(x, w, b, 1e-5)
        assert_close(y.numpy(), V[f"ln_{name}/y32"], what=f"ln {name} y")
        dx, dw, db = hip.layer_norm_bwd(x, w, mu, inv, g, mode="ref")
        assert_close(dx.numpy(), V[f"ln_{name}/dx32"], what=f"ln {name} dx")
        assert_close(dw.numpy(), V[f"ln_{name}/dw32"], what=f"ln {name} dw")
        assert_close(db.numpy(), V[f"ln_{name}/db32"], what=f"ln {name} db")
        dx, _, _ = hip.layer_norm_bwd(x, w, mu, inv, g, mode="exact")
        assert_close(dx.numpy(), V[f"ln_{name}/dx64_exact"], what=f"ln {name} exact dx")
    print("[case] golden vectors: activations", flush=True)
    x, g = D(V["act/x"]), D(V["act/g"])
    for k, got in dict(gelu_tanh_y=hip.gelu_fwd(x, "tanh"), gelu_erf_y=hip.gelu_fwd(x, "none"),
                       silu_y=hip.silu_fwd(x), gelu_tanh_dx=hip.gelu_bwd(x, g, "tanh"),
                       gelu_erf_dx=hip.gelu_bwd(x, g, "none"), silu_dx=hip.silu_bwd(x, g)).items():
        assert_close(got.numpy(), V[f"act/{k}32"], what=k)
    for k, got in dict(gelu_erf_y=hip.gelu_fwd(x, "none"), gelu_erf_dx=hip.gelu_bwd(x, g, "none"),
                       silu_y=hip.silu_fwd(x), silu_dx=hip.silu_bwd(x, g)).items():
        assert_close(got.numpy(), V[f"act/{k}64"], what=f"{k} vs float64")
    print("[case] golden vectors: softmax family", flush=True)
    for name in ("a", "b"):
        x, g = D(V[f"sm_{name}/x"]), D(V[f"sm_{name}/g"])
        y = hip.softmax_fwd(x)
        ly = hip.softmax_fwd(x, log=True)
        assert_close(y.numpy(), V[f"sm_{name}/y32"], what=f"softmax {name}")
        assert_close(ly.numpy(), V[f"sm_{name}/ly32"], what=f"log_softmax {name}")
        assert_close_arb(hip.softmax_bwd(y, g).numpy(), V[f"sm_{name}/dx32"], V[f"sm_{name}/dx64"],
                         what=f"softmax bwd {name}")
        assert_close_arb(hip.softmax_bwd(ly, g, log=True).numpy(), V[f"sm_{name}/ldx32"], V[f"sm_{name}/ldx64"],
                         what=f"log_softmax bwd {name}")
    print("[case] golden vectors: cross-entropy", flush=True)
    lg, t = D(V["ce/logits"]), D(V["ce/targets"])
    n = V["ce/logits"].shape[0]
    loss, lse = hip.cross_entropy_fwd(lg, t)
    assert_close(loss.numpy(), V["ce/loss32"], what="ce loss")
    d = hip.cross_entropy_bwd(lg, t, lse, D(np.ones(1, np.float32)))
    assert_close(n * d.numpy(), n * V["ce/d32"], what="n * dlogits")
    print("[case] golden vectors: embedding", flush=True)
    W, ids, g = D(V["emb/W"]), D(V["emb/ids"]), D(V["emb/g"])
    np.testing.assert_array_equal(hip.index_select(W, 0, ids).numpy(), V["emb/out32"])
    assert_reduction_close(hip.index_select_bwd(g, V["emb/W"].shape, 0, ids).numpy(), V["emb/dW32"],
                           V["emb/dW64"], what="dW")
    print("[case] golden vectors: reductions", flush=True)
    x = D(V["red/x"])
    for kind in ("sum", "mean", "max", "min", "argmax", "argmin", "norm"):
        for dim in (0, 1, 2):
            got = hip.reduce(kind, x, dim).numpy()
            want = V[f"red/{kind}_{dim}_32"]
            if kind in ("argmax", "argmin", "max", "min"):
                np.testing.assert_array_equal(got, want, err_msg=f"{kind} {dim}")
            else:
                assert_close(got, want, what=f"{kind} {dim}")
    hip.sync()
