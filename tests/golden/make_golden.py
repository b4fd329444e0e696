"""Writes the golden fixtures of the hot path (test infrastructure).

Two files, both data:

* kats.json -- the reference's own known-answer tests for the path, restated
  as inputs, expected outputs and tolerances, each with the reference
  file:line it comes from. The expected values are the ones those tests
  state literally, or the numpy expressions they compare against, evaluated
  here in float64.
* vectors.npz -- small seeded inputs of every hot-path function with the
  outputs of the CPU oracle (oracle/refcpu.c, the f32 restatement of the
  reference path; keys ending in "32") and of the float64 closed forms (keys
  ending in "64"). tests/test_golden.py checks that the oracle still
  reproduces them bit for bit and that the device matches them.

Usage (from the repo root): python tests/golden/make_golden.py
"""

from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def _l(a):
    return np.asarray(a, dtype=np.float64).tolist()


def kats() -> list[dict]:
    k = []
    x = np.array([[1.0, 2.0, 3.0], [3.0, 1.0, 2.0]])
    sm = np.exp(x) / np.exp(x).sum(-1, keepdims=True)
    k.append(dict(id="softmax_rows", source="python/tests/test_nn.py:30-37", op="softmax",
                  inputs=dict(x=_l(x)), expected=dict(y=_l(sm)), rtol=0.0, atol=1e-6))
    k.append(dict(id="log_softmax_rows", source="python/tests/test_nn.py:30-37", op="log_softmax",
                  inputs=dict(x=_l(x)), expected=dict(y=_l(np.log(sm))), rtol=0.0, atol=1e-6))
    big = np.array([[1000.0, 1001.0, 1002.0]])
    w = np.exp(big - 1002.0)
    k.append(dict(id="log_softmax_large", source="python/tests/test_nn.py:40-48", op="log_softmax",
                  inputs=dict(x=_l(big)), expected=dict(y=_l(np.log(w / w.sum()))), rtol=0.0, atol=1e-6))
    r = np.array([-1.0, 0.0, 1.0, 2.0])
    c = np.sqrt(2 / np.pi)
    for name, want, atol in [("relu", np.maximum(r, 0), 1e-7), ("sigmoid", 1 / (1 + np.exp(-r)), 1e-6),
                             ("tanh", np.tanh(r), 1e-6), ("silu", r / (1 + np.exp(-r)), 1e-6),
                             ("gelu_tanh", 0.5 * r * (1 + np.tanh(c * (r + 0.044715 * r ** 3))), 1e-5)]:
        k.append(dict(id=f"activation_{name}", source="python/tests/test_nn.py:51-60", op=name,
                      inputs=dict(x=_l(r)), expected=dict(y=_l(want)), rtol=0.0, atol=atol))
    x = np.array([[1.0, 2.0, 3.0], [4.0, 5.0, 6.0]])
    mu = x.mean(-1, keepdims=True)
    v = ((x - mu) ** 2).mean(-1, keepdims=True)
    coef = np.array([[1.0, -2.0, 0.5], [0.25, 1.0, -1.0]])
    xhat = (x - mu) / np.sqrt(v + 1e-5)
    k.append(dict(id="layer_norm_value_grads", source="python/tests/test_nn.py:63-78", op="layer_norm",
                  inputs=dict(x=_l(x), w=[1.0, 1.0, 1.0], b=[0.0, 0.0, 0.0], eps=1e-5, g=_l(coef)),
                  expected=dict(y=_l(xhat), dw=_l((coef * xhat).sum(0)), db=_l(coef.sum(0)), dx_abs_sum_gt=1e-6),
                  rtol=1e-4, atol=1e-5))
    x = np.array([[1.0, -2.0, 3.0]])
    w = np.array([1.0, 2.0, 0.5])
    k.append(dict(id="rms_norm_value", source="python/tests/test_nn.py:81-87", op="rms_norm",
                  inputs=dict(x=_l(x), w=_l(w), eps=1e-6),
                  expected=dict(y=_l(x / np.sqrt((x ** 2).mean(-1, keepdims=True) + 1e-6) * w)), rtol=1e-4, atol=1e-5))
    k.append(dict(id="embedding_lookup_grad", source="python/tests/test_nn.py:90-96", op="embedding",
                  inputs=dict(W=[[1.0, 1.0], [2.0, 2.0], [3.0, 3.0]], ids=[2, 0, 2], g=[[1.0, 1.0]] * 3),
                  expected=dict(out=[[3.0, 3.0], [1.0, 1.0], [3.0, 3.0]], dW=[[1.0, 1.0], [0.0, 0.0], [2.0, 2.0]]),
                  rtol=0.0, atol=0.0))
    lg = np.array([[1.0, 2.0, 3.0], [3.0, 1.0, 2.0]])
    m = lg.max(-1, keepdims=True)
    ls = lg - m - np.log(np.exp(lg - m).sum(-1, keepdims=True))
    k.append(dict(id="cross_entropy_value_grad", source="python/tests/test_nn.py:111-122", op="cross_entropy",
                  inputs=dict(logits=_l(lg), targets=[2, 0]),
                  expected=dict(loss=float(-np.mean([ls[0, 2], ls[1, 0]])),
                                dlogits=_l((np.exp(ls) - np.eye(3)[[2, 0]]) / 2), loss_atol=1e-5),
                  rtol=1e-4, atol=1e-6))
    k.append(dict(id="index_select_duplicates", source="python/tests/test_indexing_grad.py:72-76", op="index_select",
                  inputs=dict(src=[[0.0, 0.0]] * 3, dim=0, idx=[1, 1, 2], g=[[1.0, 10.0], [2.0, 20.0], [3.0, 30.0]]),
                  expected=dict(grad=[[0.0, 0.0], [3.0, 30.0], [3.0, 30.0]]), rtol=0.0, atol=0.0))
    want = np.zeros((4, 3))
    want[2] = np.array([1, 2, 3]) + np.array([4, 5, 6]) + np.array([10, 11, 12])
    want[0] = [7, 8, 9]
    k.append(dict(id="embedding_duplicates", source="python/tests/test_indexing_grad.py:79-89", op="embedding",
                  inputs=dict(W=[[0.0] * 3] * 4, ids=[2, 2, 0, 2], g=_l(np.arange(1, 13).reshape(4, 3))),
                  expected=dict(out=[[0.0] * 3] * 4, dW=_l(want)), rtol=0.0, atol=0.0))
    a = np.arange(9.0).reshape(3, 3)
    k.append(dict(id="fancy_getitem", source="python/tests/test_indexing_grad.py:92-100", op="index_select",
                  inputs=dict(src=_l(a), dim=0, idx=[2, 1, 1], g=[[1.0] * 3] * 3),
                  expected=dict(out=_l(a[[2, 1, 1]]), grad=[[0.0] * 3, [2.0] * 3, [1.0] * 3]), rtol=0.0, atol=0.0))
    k.append(dict(id="gather_duplicates", source="python/tests/test_indexing_grad.py:103-108", op="index_select",
                  inputs=dict(src=[[1.0, 2.0], [3.0, 4.0]], dim=0, idx=[1, 1], g=[[5.0, 5.0], [6.0, 6.0]]),
                  expected=dict(out=[[3.0, 4.0], [3.0, 4.0]], grad=[[0.0, 0.0], [11.0, 11.0]]), rtol=0.0, atol=0.0))
    k.append(dict(id="index_select_rows_negative", source="crates/oxi-tensor/src/tests.rs:346-355", op="index_select",
                  inputs=dict(src=[[1.0, 2.0], [3.0, 4.0], [5.0, 6.0]], dim=0, idx=[2, 0]),
                  expected=dict(out=[[5.0, 6.0], [1.0, 2.0]]), rtol=0.0, atol=0.0))
    k.append(dict(id="index_select_negative", source="crates/oxi-tensor/src/tests.rs:346-355", op="index_select",
                  inputs=dict(src=[[1.0, 2.0], [3.0, 4.0], [5.0, 6.0]], dim=0, idx=[-1]),
                  expected=dict(out=[[5.0, 6.0]]), rtol=0.0, atol=0.0))
    k.append(dict(id="index_select_out_of_range", source="crates/oxi-tensor/src/tests.rs:346-355", op="index_select",
                  inputs=dict(src=[[1.0, 2.0], [3.0, 4.0], [5.0, 6.0]], dim=0, idx=[3]),
                  expected=dict(error="index 3 out of range for dim 0 of size 3"), rtol=0.0, atol=0.0))
    k.append(dict(id="index_select_columns", source="python/tests/test_smoke.py:147-149", op="index_select",
                  inputs=dict(src=_l(np.arange(24.0).reshape(4, 6)), dim=1, idx=[-1, -2]),
                  expected=dict(out=_l(np.arange(24.0).reshape(4, 6)[:, [-1, -2]])), rtol=0.0, atol=0.0))
    t = np.array([[5.0, 7.0, 7.0], [1.0, 9.0, 2.0]])
    k.append(dict(id="argmax_first_tie", source="crates/oxi-tensor/src/tests.rs:188-196", op="reduce",
                  inputs=dict(x=_l(t), kind="argmax", dim=-1), expected=dict(y=[1.0, 1.0]), rtol=0.0, atol=0.0))
    k.append(dict(id="argmin_dim1", source="crates/oxi-tensor/src/tests.rs:188-196", op="reduce",
                  inputs=dict(x=_l(t), kind="argmin", dim=1), expected=dict(y=[0.0, 0.0]), rtol=0.0, atol=0.0))
    k.append(dict(id="duplicate_accumulation", source="crates/oxi-autograd/src/tests.rs:341-353", op="index_select",
                  inputs=dict(src=[[0.0] * 3] * 3, dim=0, idx=[1, 1], g=[[1.0, 2.0, 3.0], [4.0, 5.0, 6.0]]),
                  expected=dict(grad=[[0.0] * 3, [5.0, 7.0, 9.0], [0.0] * 3]), rtol=0.0, atol=0.0))
    return k


def vectors() -> dict[str, np.ndarray]:
    from oracle import closed_form as cf
    from oracle import ref

    r = np.random.default_rng(20261201)
    v: dict[str, np.ndarray] = {}

    def f32(*shape, scale=1.0, shift=0.0):
        return (r.standard_normal(shape, dtype=np.float32) * np.float32(scale) + np.float32(shift)).astype(np.float32)

    # norms: rows of 96 (one-wave rows) and 1040 (block rows, ragged in float4s)
    for name, (R, H) in {"norm_a": (6, 96), "norm_b": (2, 1040)}.items():
        x, g = f32(R, H), f32(R, H)
        w, b = f32(H, scale=0.02, shift=1.0), f32(H, scale=0.02)
        y, inv = ref.rms_norm_fwd(x, w, 1e-6)
        dx, dw = ref.rms_norm_bwd(x, w, inv, g)
        v.update({f"rms_{name}/x": x, f"rms_{name}/w": w, f"rms_{name}/g": g, f"rms_{name}/y32": y,
                  f"rms_{name}/inv32": inv, f"rms_{name}/dx32": dx, f"rms_{name}/dw32": dw,
                  f"rms_{name}/y64": cf.rms_norm_fwd(x, w, 1e-6)[0],
                  f"rms_{name}/dx64_exact": cf.rms_norm_bwd_exact(x, w, g, 1e-6)[0]})
        y, mu, inv = ref.layer_norm_fwd(x, w, b, 1e-5)
        dx, dw, db = ref.layer_norm_bwd(x, w, mu, inv, g)
        v.update({f"ln_{name}/x": x, f"ln_{name}/w": w, f"ln_{name}/b": b, f"ln_{name}/g": g, f"ln_{name}/y32": y,
                  f"ln_{name}/mean32": mu, f"ln_{name}/inv32": inv, f"ln_{name}/dx32": dx, f"ln_{name}/dw32": dw,
                  f"ln_{name}/db32": db, f"ln_{name}/y64": cf.layer_norm_fwd(x, w, b, 1e-5)[0],
                  f"ln_{name}/dx64_exact": cf.layer_norm_bwd_exact(x, w, g, 1e-5)[0]})
    # activations over a wide range, including the tails
    x = np.concatenate([f32(300, scale=3.0), np.array([-12.0, -6.0, -1e-4, 0.0, 1e-4, 6.0, 12.0], np.float32)])
    g = f32(x.size)
    v.update({"act/x": x, "act/g": g,
              "act/gelu_tanh_y32": ref.gelu_tanh_fwd(x), "act/gelu_tanh_dx32": ref.gelu_tanh_bwd(x, g),
              "act/gelu_erf_y32": ref.gelu_erf_fwd(x), "act/gelu_erf_dx32": ref.gelu_erf_bwd(x, g),
              "act/silu_y32": ref.silu_fwd(x), "act/silu_dx32": ref.silu_bwd(x, g),
              "act/gelu_tanh_y64": cf.gelu_tanh(x), "act/gelu_erf_y64": cf.gelu_erf(x),
              "act/gelu_erf_dx64": cf.gelu_erf_grad(x) * g.astype(np.float64),
              "act/silu_y64": cf.silu(x), "act/silu_dx64": cf.silu_grad(x) * g.astype(np.float64)})
    # softmax family, last dim of 50 and 3000
    for name, (R, C) in {"a": (5, 50), "b": (2, 3000)}.items():
        x, g = f32(R, C, scale=2.0), f32(R, C)
        v.update({f"sm_{name}/x": x, f"sm_{name}/g": g,
                  f"sm_{name}/y32": ref.softmax_fwd(x), f"sm_{name}/dx32": ref.softmax_bwd(x, g),
                  f"sm_{name}/ly32": ref.log_softmax_fwd(x), f"sm_{name}/ldx32": ref.log_softmax_bwd(x, g),
                  f"sm_{name}/y64": cf.softmax(x), f"sm_{name}/ly64": cf.log_softmax(x),
                  f"sm_{name}/dx64": cf.softmax_bwd(x, g), f"sm_{name}/ldx64": cf.log_softmax_bwd(x, g)})
    # cross-entropy, 5 rows of 1003 classes
    lg = f32(5, 1003, scale=2.0)
    t = r.integers(0, 1003, 5).astype(np.int64)
    v.update({"ce/logits": lg, "ce/targets": t,
              "ce/loss32": np.array([ref.cross_entropy_fwd(lg, t)], np.float32),
              "ce/d32": ref.cross_entropy_bwd(lg, t),
              "ce/loss64": np.array([cf.cross_entropy(lg, t)]), "ce/d64": cf.cross_entropy_grad(lg, t)})
    # embedding with duplicates and negative ids
    W = f32(37, 20)
    ids = np.concatenate([r.integers(-37, 37, 150), np.full(40, 5), np.full(30, -1)]).astype(np.int64)
    r.shuffle(ids)
    g = f32(ids.size, 20)
    v.update({"emb/W": W, "emb/ids": ids, "emb/g": g, "emb/out32": ref.index_select(W, 0, ids),
              "emb/dW32": ref.index_select_bwd(g, W.shape, 0, ids),
              "emb/dW64": cf.embedding_grad(g, np.where(ids < 0, ids + 37, ids), 37)})
    # reductions with ties and NaN
    x = np.round(f32(4, 7, 9), 1)
    x[0, 0, 3] = np.nan
    x[1, 2, :] = 0.5
    v["red/x"] = x
    for kind in ("sum", "mean", "max", "min", "argmax", "argmin", "norm"):
        for dim in (0, 1, 2):
            v[f"red/{kind}_{dim}_32"] = ref.reduce(kind, x, dim)
    return v


def main() -> None:
    import oracle

    oracle.build()
    (HERE / "kats.json").write_text(json.dumps(kats(), indent=1) + "\n")
    vec = vectors()
    np.savez_compressed(HERE / "vectors.npz", **vec)
    print(f"wrote {len(kats())} known-answer tests and {len(vec)} arrays")


if __name__ == "__main__":
    main()
