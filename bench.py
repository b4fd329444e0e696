#!/usr/bin/env python3
"""Throughput bench of the oxitorch layer-kernel hot path on one MI355X.

A "step" is one forward+backward pass of a BASELINE.json config over one batch
of synthetic, seeded input that is already resident in HBM, driven through the
liboxihip C-ABI (include/oxihip.h) in the order the host core launches it.

The default run (`--config all`) measures all five configs C1-C5 and prints
one JSON line whose headline (`value`, `ms_per_step`, `roofline`,
`cpu_baseline`) is C3, the largest config (3.15 GB per step), with a compact
block per config under `configs` and, last on the line, a `summary` of every
config in one short string each. `--config c1..c5` runs one config; `f2`
(device DataLoader batches), `f3` (masked_select + row scatter) and `f4`
(AdamW over GPT-2 small's parameters) time the rows after the path.
`--detail PATH` also writes every measurement (per-call tables, node-by-node
steps) to a JSON file.

A config's step is the launch sequence the host core runs by default: with
the graph fusions on, C2's backward is one layer_norm+gelu VJP pass and C5's
is two fused passes (rms_norm+softmax with the positional gradient,
layer_norm+silu through the permute), none of which writes the norm output's
gradient (the host core forms it if its .grad is read); C3's forward also
writes the gradient for loss.backward()'s seed 1, so its backward launches
nothing.

The main figure (`ms_per_step`, `value`) is the slower of two medians over
K steps each (after W untimed warmup steps and about a quarter of a second of
untimed steps, so that the GPU is back at its steady clocks):
- cold: every step is preceded by an untimed flush of a 512 MiB scratch buffer
  (twice the 256 MB Infinity Cache), written and then read back, so the step
  reads its inputs from HBM and the cache holds no dirty lines (`--flush
  write` fills only, which leaves the fill's dirty lines for the step to write
  back; `--flush read` only reads, which evicts nothing from the Infinity
  Cache on this GPU and so behaves like the warm step);
- warm: the steps back to back, each paying the write-back of the previous
  step's outputs.
Each step is timed alone with HIP events on the library stream (the stream
every liboxihip kernel runs on). `gbs` (and `value`) divides the HBM bytes
the step's kernels must move (each call's reads and writes; C4's gather
counted as reading each distinct row of W once; checked against the PMC
counters in profiles/pmc_traffic_<config>.md) by that time, against the
8 TB/s peak. `per_op_gbs` divides the metric's per-op algorithmic bytes
(every F.* op reading its inputs and writing its outputs once) by the same
time: the rate a step of separate ops would need, which passes the peak where
the fused passes remove traffic.

Per config:
- in_step_us: each C-ABI call's time inside the step, from HIP events around
  every call of K more steps under the graded protocol (median per call);
- roofline: the dominant call (largest in-step time) against MI355X's 8 TB/s
  HBM peak, its time from K more steps under the graded protocol with HIP
  events around that call alone (events between every call add a launch
  bubble at each, so in_step_us runs a little long); `traffic` is its HBM bytes per
  call from the committed rocprofv3 PMC summary
  profiles/pmc_traffic_<config>.md (FETCH_SIZE and WRITE_SIZE runs, scaled by
  a copy kernel's readings);
- cold_after_fill_only_ms: cold steps after a write-only flush;
- copy_floor_ms: the step's launch sequence with every call replaced by an
  identity copy moving the same number of bytes (warm): the practical floor
  for a step of that many launches and bytes on this GPU;
- unfused_ms (C2, C3, C5): the warm step without the host core's fusions;
- dropin_ms (C1-C5): the same step through the Python surface (F.* and
  backward() over the host core's graph, C4's ids a host list as the
  reference takes them), warm, with the host's time per step;
- cpu_baseline: the CPU oracle (oracle/refcpu.c, a C restatement of the
  reference CPU path) on a bounded sample of the same workload on this host.

Python's cycle collector is off around the timed loops of C-ABI calls (as in
timeit), so that no collection pass lands among them. Prints ONE JSON line on
stdout; progress goes to stderr.
"""

from __future__ import annotations

import argparse
import gc
import json
import os
import re
import sys
import time

import numpy as np

PEAK_HBM_GBS = 8000.0
SETTLE_S = 0.25  # untimed steps before a config's timed ones, in seconds
MIB = 1 << 20
ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "achieved HBM GB/s (% of MI355X peak) + rows/s, norm/softmax/embed fwd+bwd"

PROFILES = os.path.join(ROOT, "profiles")


def pmc_traffic(config):
    """HBM bytes per C-ABI call from the committed PMC summary of `config`
    (its line "traffic per C-ABI call, MiB: name=value; ..."), or {}."""
    path = os.path.join(PROFILES, f"pmc_traffic_{config}.md")
    try:
        text = open(path).read()
    except OSError:
        return {}
    m = re.search(r"^traffic per C-ABI call, MiB: (.*)$", text, re.M)
    if not m:
        return {}
    out = {}
    for item in m.group(1).split(";"):
        if "=" in item:
            k, v = item.split("=")
            out[k.strip()] = float(v) * MIB
    return out


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=3)
    p.add_argument("--config", default="all", choices=["all"] + sorted(WORKLOADS))
    p.add_argument("--cpu-seconds", type=float, default=4.0,
                   help="budget of each config's CPU-oracle baseline sample")
    p.add_argument("--no-dropin", action="store_true", help="skip the F.*/backward() timing")
    p.add_argument("--no-cold", action="store_true", help="skip the cold-cache medians")
    p.add_argument("--no-cpu", action="store_true")
    p.add_argument("--no-copy-probe", action="store_true")
    p.add_argument("--detail", default=None, help="also write every measurement to this JSON file")
    p.add_argument("--flush", default="write-read", choices=["write", "write-read", "read"],
                   help="how the cold-MALL steps evict the inputs (see Flush)")
    p.add_argument("--only-graded", action="store_true",
                   help="warmup and the K graded cold-MALL steps only (for rocprofv3 runs: every dispatch of the "
                        "run is then a warmup or in-step one)")
    return p.parse_args()


class EmbeddingPlan:
    """The host core's embedding pattern: the VJP's id sort queued on the
    library's second stream, then the forward gather (the sort overlaps the
    gather and the rest of the forward); the backward applies it. The
    previous step's plan is freed when the next forward replaces it."""

    def __init__(self, hip):
        self.hip = hip
        self.plan = self.hip.vp()

    def plan_sort(self, ids, n, V):
        """Queued before the gather, so the sort overlaps it."""
        L, c = self.hip.lib, self.hip.check
        if self.plan.value:
            c(L.oxi_index_select_bwd_plan_free(self.plan))
        c(L.oxi_index_select_bwd_plan(ids, n, V, self.hip.ctypes.byref(self.plan)))

    def forward(self, W, ids, n, V, D, out):
        self.hip.check(self.hip.lib.oxi_embedding_fwd(W, ids, n, V, D, out))

    def backward(self, g, D, dW):
        self.hip.check(self.hip.lib.oxi_index_select_bwd_apply(self.plan, g, 1, D, dW))


class Workload:
    """kernels(): [(label, launch_fn, algorithmic_bytes)] in step order."""

    name = ""
    rows = 0
    bytes_per_step = 0

    def __init__(self, hip):
        self.hip = hip
        self.D = hip.DeviceArray.from_numpy

    def st(self, vals):
        return self.hip._i64arr(vals)

    def release(self):
        """Frees the workload's device buffers (the next config reuses the HBM)."""
        emb = getattr(self, "emb", None)
        if emb is not None and emb.plan.value:
            self.hip.check(self.hip.lib.oxi_index_select_bwd_plan_free(emb.plan))
            emb.plan.value = None
        for v in list(vars(self).values()):
            if isinstance(v, self.hip.DeviceArray):
                v.free()
        self.hip.sync()


# ---------------------------------------------------------------------------

class C1(Workload):
    def __init__(self, hip):
        super().__init__(hip)
        R, H = 4096, 768
        self.R, self.H, self.rows = R, H, R
        self.name = "C1 rms_norm fwd+bwd fp32 x(4096,768)"
        r = np.random.default_rng(1)
        x = r.standard_normal((R, H), dtype=np.float32)
        w = (r.standard_normal(H, dtype=np.float32) * 0.02 + 1).astype(np.float32)
        g = r.standard_normal((R, H), dtype=np.float32)
        self.host = dict(x=x, w=w, g=g)
        self.x, self.w, self.g = self.D(x), self.D(w), self.D(g)
        A = hip.DeviceArray
        self.y, self.dx, self.rstd, self.dw = A((R, H)), A((R, H)), A((R,)), A((H,))
        self.bytes_per_step = 5 * R * H * 4

    def kernels(self):
        L, c, R, H = self.hip.lib, self.hip.check, self.R, self.H
        E4 = R * H * 4
        return [("rms_norm_fwd", lambda: c(L.oxi_rms_norm_fwd(self.x.ptr, self.w.ptr, self.y.ptr, self.rstd.ptr, R, H,
                                                              1e-6)), 2 * E4),
                ("rms_norm_bwd", lambda: c(L.oxi_rms_norm_bwd(self.x.ptr, self.w.ptr, self.rstd.ptr, self.g.ptr,
                                                              self.dx.ptr, self.dw.ptr, R, H, 0)), 3 * E4)]

    def cpu_step(self, ref, lo, hi):
        h = self.host
        y, inv = ref.rms_norm_fwd(h["x"][lo:hi], h["w"], 1e-6)
        ref.rms_norm_bwd(h["x"][lo:hi], h["w"], inv, h["g"][lo:hi])

    dropin_what = "x.grad = w.grad = None; F.rms_norm(x, w, 1e-6).backward(g)"

    def dropin(self, ox, F):
        h = self.host
        x, w, g = ox.from_numpy(h["x"], True), ox.from_numpy(h["w"], True), ox.from_numpy(h["g"])

        def step():
            x.grad = None
            w.grad = None
            F.rms_norm(x, w, 1e-6).backward(g)
        return step


class C2(Workload):
    def __init__(self, hip):
        super().__init__(hip)
        R, H = 16384, 4096
        self.R, self.H, self.rows = R, H, R
        self.name = "C2 layer_norm(affine)+erf-gelu fwd+bwd fp32 x(16384,4096)"
        r = np.random.default_rng(2)
        x = r.standard_normal((R, H), dtype=np.float32)
        w = (r.standard_normal(H, dtype=np.float32) * 0.02 + 1).astype(np.float32)
        b = (r.standard_normal(H, dtype=np.float32) * 0.02).astype(np.float32)
        g = r.standard_normal((R, H), dtype=np.float32)
        self.host = dict(x=x, w=w, b=b, g=g)
        self.x, self.w, self.b, self.g = (self.D(a) for a in (x, w, b, g))
        A = hip.DeviceArray
        self.h, self.y, self.dh, self.dx = (A((R, H)) for _ in range(4))
        self.mean, self.rstd, self.dw, self.db = A((R,)), A((R,)), A((H,)), A((H,))
        self.bytes_per_step = 10 * R * H * 4

    def unfused_kernels(self):
        L, c, R, H = self.hip.lib, self.hip.check, self.R, self.H
        st, shp = self.st((H, 1)), self.st((R, H))
        E4 = R * H * 4
        return [
            ("layer_norm_fwd", lambda: c(L.oxi_layer_norm_fwd(self.x.ptr, self.w.ptr, self.b.ptr, self.h.ptr,
                                                              self.mean.ptr, self.rstd.ptr, R, H, 1e-5)), 2 * E4),
            ("gelu_erf_fwd", lambda: c(L.oxi_gelu_fwd(self.h.ptr, st, self.y.ptr, st, shp, 2, 1)), 2 * E4),
            ("gelu_erf_bwd", lambda: c(L.oxi_gelu_bwd(self.h.ptr, st, self.g.ptr, st, self.dh.ptr, st, shp, 2, 1)),
             3 * E4),
            ("layer_norm_bwd", lambda: c(L.oxi_layer_norm_bwd(self.x.ptr, self.w.ptr, self.mean.ptr, self.rstd.ptr,
                                                              self.dh.ptr, self.dx.ptr, self.dw.ptr, self.db.ptr, R,
                                                              H, 0)), 3 * E4)]

    # The host core's default for this config: the norm output feeds only the
    # GELU, so backward runs both VJPs as one pass (oxi_layer_norm_act_bwd
    # reads x and g and writes dx; the norm output's gradient is formed only
    # if its .grad is read) and a step crosses HBM 7 E-sized times
    # (moved_bytes), not the 10 of the per-op count the metric is defined on.
    # unfused_kernels() is the path with that fusion off (OXI_FUSE_NORM_ACT=0)
    # or with other consumers of the norm output.
    unfused_what = ("layer_norm_fwd + gelu_erf_fwd, then the two VJPs node by node (gelu_erf_bwd, "
                    "layer_norm_bwd), as the host core runs them with OXI_FUSE_NORM_ACT=0")

    def kernels(self):
        L, c, R, H = self.hip.lib, self.hip.check, self.R, self.H
        E4 = R * H * 4
        return self.unfused_kernels()[:2] + [
            ("layer_norm_gelu_bwd", lambda: c(L.oxi_layer_norm_act_bwd(
                self.x.ptr, self.w.ptr, self.b.ptr, self.mean.ptr, self.rstd.ptr, self.g.ptr, 1, None,
                self.dx.ptr, self.dw.ptr, self.db.ptr, R, H, 0)), 3 * E4)]

    def cpu_step(self, ref, lo, hi):
        h = self.host
        x, g = h["x"][lo:hi], h["g"][lo:hi]
        hh, mu, inv = ref.layer_norm_fwd(x, h["w"], h["b"], 1e-5)
        ref.gelu_erf_fwd(hh)
        dh = ref.gelu_erf_bwd(hh, g)
        ref.layer_norm_bwd(x, h["w"], mu, inv, dh)

    dropin_what = ("x.grad = w.grad = b.grad = None; F.gelu(F.layer_norm(x, w, b, 1e-5), approximate='none')"
                   ".backward(g)")

    def dropin(self, ox, F):
        h = self.host
        x, w, b = (ox.from_numpy(h[k], True) for k in ("x", "w", "b"))
        g = ox.from_numpy(h["g"])

        def step():
            for t in (x, w, b):
                t.grad = None
            F.gelu(F.layer_norm(x, w, b, 1e-5), approximate="none").backward(g)
        return step


class C3(Workload):
    def __init__(self, hip):
        super().__init__(hip)
        n, c = 8192, 32000
        self.n, self.c, self.rows = n, c, n
        self.name = "C3 log_softmax+cross_entropy(mean) fwd+bwd fp32 logits(8192,32000)"
        r = np.random.default_rng(3)
        logits = (r.standard_normal((n, c), dtype=np.float32) * 2).astype(np.float32)
        t = r.integers(0, c, n).astype(np.int64)
        self.host = dict(logits=logits, t=t)
        self.logits, self.t = self.D(logits), self.D(t)
        self.gl = self.D(np.ones(1, np.float32))
        A = hip.DeviceArray
        self.loss, self.lse, self.d = A((1,)), A((n,)), A((n, c))
        self.bytes_per_step = 3 * n * c * 4

    unfused_what = ("oxi_cross_entropy_fwd, then oxi_cross_entropy_bwd: the host core's path for any upstream "
                    "gradient other than backward()'s implicit seed 1")

    def unfused_kernels(self):
        L, c, n, C = self.hip.lib, self.hip.check, self.n, self.c
        E4 = n * C * 4
        return [("cross_entropy_fwd", lambda: c(L.oxi_cross_entropy_fwd(self.logits.ptr, self.t.ptr, self.loss.ptr,
                                                                        self.lse.ptr, n, C)), E4),
                ("cross_entropy_bwd", lambda: c(L.oxi_cross_entropy_bwd(self.logits.ptr, self.t.ptr, self.lse.ptr,
                                                                        self.gl.ptr, self.d.ptr, n, C)), 2 * E4)]

    # The host core's default for loss.backward(): the forward pass holds each
    # row in registers and also writes the gradient for the seed 1, so the
    # step reads the logits once and writes dlogits once (moved bytes 2 E),
    # against the per-op count of 3 E the metric is defined on.
    def kernels(self):
        L, c, n, C = self.hip.lib, self.hip.check, self.n, self.c
        E4 = n * C * 4
        return [("cross_entropy_fwd_grad", lambda: c(L.oxi_cross_entropy_fwd_grad(
            self.logits.ptr, self.t.ptr, self.loss.ptr, self.lse.ptr, self.d.ptr, n, C)), 2 * E4)]

    dropin_what = "logits.grad = None; F.cross_entropy(logits, targets).backward(), targets a numpy int64 array"

    def dropin(self, ox, F):
        h = self.host
        x = ox.from_numpy(h["logits"], True)
        t = h["t"]

        def step():
            x.grad = None
            F.cross_entropy(x, t).backward()
        return step

    def cpu_step(self, ref, lo, hi):
        h = self.host
        ref.cross_entropy_fwd(h["logits"][lo:hi], h["t"][lo:hi])
        ref.cross_entropy_bwd(h["logits"][lo:hi], h["t"][lo:hi])


class C4(Workload):
    def __init__(self, hip):
        super().__init__(hip)
        V, Dm = 50257, 1024
        self.V, self.Dm = V, Dm
        self.name = "C4 embedding fwd+bwd fp32 W(50257,1024) ids(64,2048) clipped Zipf(1.1)"
        r = np.random.default_rng(4)
        W = r.standard_normal((V, Dm), dtype=np.float32)
        ids = np.minimum(r.zipf(1.1, (64, 2048)) - 1, V - 1).astype(np.int64).ravel()
        g = r.standard_normal((ids.size, Dm), dtype=np.float32)
        self.n = ids.size
        self.rows = ids.size
        self.host = dict(W=W, ids=ids, g=g)
        self.W, self.ids, self.g = self.D(W), self.D(ids), self.D(g)
        A = hip.DeviceArray
        self.out, self.dW = A((self.n, Dm)), A((V, Dm))
        idb = self.n * 8
        self.fwd_bytes = idb + 2 * self.n * Dm * 4
        self.bwd_bytes = idb + self.n * Dm * 4 + V * Dm * 4
        self.bytes_per_step = self.fwd_bytes + self.bwd_bytes
        # the clipped Zipf ids name few distinct rows: counting each row of W
        # the gather reads once gives the bytes HBM has to deliver at least
        self.unique_rows = int(np.unique(ids).size)
        self.fwd_bytes_unique = idb + self.unique_rows * Dm * 4 + self.n * Dm * 4

    def kernels(self):
        L, c = self.hip.lib, self.hip.check
        ep = self.emb = getattr(self, "emb", None) or EmbeddingPlan(self.hip)
        return [("embedding_bwd_plan", lambda: ep.plan_sort(self.ids.ptr, self.n, self.V), 0),
                # HBM bytes: each distinct row of W once (repeats come from the caches)
                ("embedding_fwd", lambda: ep.forward(self.W.ptr, self.ids.ptr, self.n, self.V, self.Dm,
                                                     self.out.ptr), self.fwd_bytes_unique),
                ("embedding_bwd", lambda: ep.backward(self.g.ptr, self.Dm, self.dW.ptr), self.bwd_bytes)]

    def cpu_step(self, ref, lo, hi):
        h = self.host
        ids = h["ids"][lo:hi]
        ref.index_select(h["W"], 0, ids)
        ref.index_select_bwd(h["g"][lo:hi], h["W"].shape, 0, ids)

    dropin_what = ("W.grad = None; F.embedding(ids, W).backward(g), ids a host list of 131072 ints as the reference "
                   "takes them (functional.py:245-247)")

    def dropin(self, ox, F):
        h = self.host
        W = ox.from_numpy(h["W"], True)
        g = ox.from_numpy(h["g"])
        ids = h["ids"].tolist()

        def step():
            W.grad = None
            F.embedding(ids, W).backward(g)
        return step

    def dropin_array(self, ox, F):
        """The same step with the ids as a numpy int64 array (no list conversion)."""
        h = self.host
        W = ox.from_numpy(h["W"], True)
        g = ox.from_numpy(h["g"])
        ids = h["ids"]

        def step():
            W.grad = None
            F.embedding(ids, W).backward(g)
        return step


class C5(Workload):
    """GPT-2-small non-GEMM chain, launched as the host core launches it:
    emb -> layer_norm -> silu(permuted view) -> + pos (broadcast) -> rms_norm
    -> softmax, then the full backward."""

    def __init__(self, hip):
        super().__init__(hip)
        V, B, T, H = 50257, 16, 1024, 768
        self.V, self.B, self.T, self.H = V, B, T, H
        R = B * T
        self.rows = R
        self.name = "C5 GPT-2-small non-GEMM chain fwd+bwd fp32 16x1024x768"
        r = np.random.default_rng(5)
        W = r.standard_normal((V, H), dtype=np.float32)
        ids = r.integers(0, V, R).astype(np.int64)
        lnw, lnb, rw = (r.standard_normal(H, dtype=np.float32) for _ in range(3))
        pos = r.standard_normal((1, T, H), dtype=np.float32)
        g = r.standard_normal((B, T, H), dtype=np.float32)
        self.host = dict(W=W, ids=ids, lnw=lnw, lnb=lnb, rw=rw, pos=pos, g=g)
        for k, v in self.host.items():
            setattr(self, k, self.D(v))
        A = hip.DeviceArray
        E = R * H
        self.e, self.h, self.s, self.r, self.n, self.y = (A((E,)) for _ in range(6))
        self.dn, self.dr, self.dh, self.de = (A((E,)) for _ in range(4))
        self.mu, self.rs1, self.rs2 = A((R,)), A((R,)), A((R,))
        self.dlnw, self.dlnb, self.drw, self.dpos, self.dW = A((H,)), A((H,)), A((H,)), A((T * H,)), A((V, H))
        E4, P4, VH4, ID = E * 4, T * H * 4, V * H * 4, R * 8
        self.op_bytes = dict(embedding_bwd_plan=0, embedding_fwd=ID + 2 * E4, layer_norm_fwd=2 * E4, silu_fwd=2 * E4, add_fwd=2 * E4 + P4,
                             rms_norm_fwd=2 * E4, softmax_fwd=2 * E4, softmax_bwd=3 * E4, rms_norm_bwd=3 * E4,
                             pos_grad_reduce=E4 + P4, silu_bwd=3 * E4, layer_norm_bwd=3 * E4,
                             embedding_bwd=ID + E4 + VH4)
        self.bytes_per_step = 26 * E4 + VH4 + 2 * P4 + 2 * ID
        # the default backward's fused passes: rms_norm + softmax VJP with the
        # positional gradient (read r, g; write dr, dpos), layer_norm + silu
        # VJP through the permute (read e, dr; write de). Neither writes the
        # norm output's gradient: the host core forms it when .grad is read.
        self.op_bytes.update(rms_norm_softmax_pos_bwd=3 * E4 + P4, layer_norm_silu_bwd=3 * E4)

    def unfused_kernels(self):
        L, c = self.hip.lib, self.hip.check
        V, B, T, H = self.V, self.B, self.T, self.H
        R = B * T
        st = self.st
        tview_shape, tview_strides = st((B, H, T)), st((T * H, 1, H))   # h.permute([0,2,1])
        rm_bht = st((H * T, T, 1))
        sview = st((H * T, 1, T))                                        # s.permute([0,2,1])
        pos_b = st((0, H, 1))
        rm_bth, shp_bth = st((T * H, H, 1)), st((B, T, H))
        b = self.op_bytes
        ep = self.emb = getattr(self, "emb", None) or EmbeddingPlan(self.hip)
        ops = [
            ("embedding_bwd_plan", lambda: ep.plan_sort(self.ids.ptr, R, V)),
            ("embedding_fwd", lambda: ep.forward(self.W.ptr, self.ids.ptr, R, V, H, self.e.ptr)),
            ("layer_norm_fwd", lambda: c(L.oxi_layer_norm_fwd(self.e.ptr, self.lnw.ptr, self.lnb.ptr, self.h.ptr,
                                                              self.mu.ptr, self.rs1.ptr, R, H, 1e-5))),
            ("silu_fwd", lambda: c(L.oxi_silu_fwd(self.h.ptr, tview_strides, self.s.ptr, rm_bht, tview_shape, 3))),
            ("add_fwd", lambda: c(L.oxi_binary(0, self.s.ptr, sview, self.pos.ptr, pos_b, self.r.ptr, rm_bth,
                                               shp_bth, 3))),
            ("rms_norm_fwd", lambda: c(L.oxi_rms_norm_fwd(self.r.ptr, self.rw.ptr, self.n.ptr, self.rs2.ptr, R, H,
                                                          1e-6))),
            ("softmax_fwd", lambda: c(L.oxi_softmax_fwd(self.n.ptr, self.y.ptr, R, H, 1))),
            ("softmax_bwd", lambda: c(L.oxi_softmax_bwd(self.y.ptr, self.g.ptr, self.dn.ptr, R, H, 1))),
            ("rms_norm_bwd", lambda: c(L.oxi_rms_norm_bwd(self.r.ptr, self.rw.ptr, self.rs2.ptr, self.dn.ptr,
                                                          self.dr.ptr, self.drw.ptr, R, H, 0))),
            ("pos_grad_reduce", lambda: c(L.oxi_reduce(0, self.dr.ptr, rm_bth, shp_bth, 3, 0, self.dpos.ptr))),
            # silu VJP: x and g are both the permuted view; dx keeps that layout
            ("silu_bwd", lambda: c(L.oxi_silu_bwd(self.h.ptr, tview_strides, self.dr.ptr, tview_strides, self.dh.ptr,
                                                  tview_strides, tview_shape, 3))),
            ("layer_norm_bwd", lambda: c(L.oxi_layer_norm_bwd(self.e.ptr, self.lnw.ptr, self.mu.ptr, self.rs1.ptr,
                                                              self.dh.ptr, self.de.ptr, self.dlnw.ptr, self.dlnb.ptr,
                                                              R, H, 0))),
            ("embedding_bwd", lambda: ep.backward(self.de.ptr, H, self.dW.ptr)),
        ]
        return [(k, f, b[k]) for k, f in ops]

    # The host core's default backward for the chain: softmax over the last
    # dim of the rms_norm output and the positional table's gradient (the sum
    # of dr over the batch) in one pass, then silu on the permuted
    # layer_norm output and the layer_norm VJP in one pass. unfused_kernels()
    # is the node-by-node order (OXI_FUSE_NORM_ACT=0).
    unfused_what = ("the chain node by node, as the host core runs it with OXI_FUSE_NORM_ACT=0: softmax_bwd, "
                    "rms_norm_bwd, the positional gradient as a column sum over the batch, silu_bwd, layer_norm_bwd")

    def kernels(self):
        L, c, R, H = self.hip.lib, self.hip.check, self.rows, self.H
        b = self.op_bytes
        out = []
        for name, fn, nbytes in self.unfused_kernels():
            if name in ("softmax_bwd", "pos_grad_reduce", "silu_bwd"):
                continue
            if name == "rms_norm_bwd":
                out.append(("rms_norm_softmax_pos_bwd", lambda: c(L.oxi_rms_norm_bwd_lead_sum(
                    self.r.ptr, self.rw.ptr, self.rs2.ptr, self.g.ptr, 3, None, self.dr.ptr, self.drw.ptr,
                    self.dpos.ptr, self.B, R, H, 0)), b["rms_norm_softmax_pos_bwd"]))
                continue
            if name == "layer_norm_bwd":
                out.append(("layer_norm_silu_bwd", lambda: c(L.oxi_layer_norm_act_bwd(
                    self.e.ptr, self.lnw.ptr, self.lnb.ptr, self.mu.ptr, self.rs1.ptr, self.dr.ptr, 2, None,
                    self.de.ptr, self.dlnw.ptr, self.dlnb.ptr, R, H, 0)), b["layer_norm_silu_bwd"]))
                continue
            out.append((name, fn, nbytes))
        return out

    def cpu_step(self, ref, lo, hi):
        # the whole chain on the CPU oracle (batch rows lo..hi of 16)
        h = self.host
        B0, B1 = lo // self.T, max(lo // self.T + 1, hi // self.T)
        ids = h["ids"][B0 * self.T:B1 * self.T]
        nb = B1 - B0
        e = ref.index_select(h["W"], 0, ids).reshape(nb, self.T, self.H)
        hh, mu, inv = ref.layer_norm_fwd(e, h["lnw"], h["lnb"], 1e-5)
        hp = np.ascontiguousarray(hh.transpose(0, 2, 1))
        s = ref.silu_fwd(hp)
        rr = np.ascontiguousarray(s.transpose(0, 2, 1)) + h["pos"]
        n, inv2 = ref.rms_norm_fwd(rr, h["rw"], 1e-6)
        ref.softmax_fwd(n)
        g = h["g"][B0:B1]
        dn = ref.softmax_bwd(n, g)
        dr, _ = ref.rms_norm_bwd(rr, h["rw"], inv2, dn)
        dr.sum(0)
        dhp = ref.silu_bwd(hp, np.ascontiguousarray(dr.transpose(0, 2, 1)))
        de, _, _ = ref.layer_norm_bwd(e, h["lnw"], mu, inv, np.ascontiguousarray(dhp.transpose(0, 2, 1)))
        ref.index_select_bwd(de.reshape(-1, self.H), h["W"].shape, 0, ids)

    dropin_what = ("leaf grads = None; F.softmax(F.rms_norm(F.silu(F.layer_norm(F.embedding(ids, W).reshape(...), "
                   "lnw, lnb).permute([0,2,1])).permute([0,2,1]) + pos, rw), -1).backward(g), ids a host list "
                   "as the reference takes them")

    def dropin(self, ox, F):
        h = self.host
        B, T, H = self.B, self.T, self.H
        W, lnw, lnb, rw, pos = (ox.from_numpy(h[k], True) for k in ("W", "lnw", "lnb", "rw", "pos"))
        g = ox.from_numpy(h["g"])
        ids = h["ids"].tolist()

        def step():
            for t in (W, lnw, lnb, rw, pos):
                t.grad = None
            e = F.embedding(ids, W).reshape([B, T, H])
            s = F.silu(F.layer_norm(e, lnw, lnb, 1e-5).permute([0, 2, 1]))
            F.softmax(F.rms_norm(s.permute([0, 2, 1]) + pos, rw, 1e-6), -1).backward(g)
        return step


def gpt2_small_param_shapes(V=50257, T=1024, H=768, L=12):
    """Parameter shapes of GPT-2 small with tied embeddings: 148 tensors,
    124,439,808 floats."""
    block = [(H,), (H,), (H, 3 * H), (3 * H,), (H, H), (H,), (H,), (H,), (H, 4 * H), (4 * H,), (4 * H, H), (H,)]
    return [(V, H), (T, H)] + block * L + [(H,), (H,)]


class F4(Workload):
    """One AdamW step (decoupled decay) over every parameter of GPT-2 small,
    one tensor per parameter as a model holds them, through the multi-slice
    entry point the host core calls; new values ping-pong between two
    buffers per parameter."""

    cpu_full = True

    def __init__(self, hip):
        super().__init__(hip)
        self.shapes = gpt2_small_param_shapes()
        sizes = [int(np.prod(s)) for s in self.shapes]
        self.sizes = sizes
        N = sum(sizes)
        self.rows = N
        self.name = f"F4 AdamW step, GPT-2 small parameters ({len(sizes)} tensors, {N:,} fp32)"
        r = np.random.default_rng(44)
        flat = {k: r.standard_normal(N, dtype=np.float32) for k in ("p", "g")}
        flat["m"] = r.standard_normal(N, dtype=np.float32) * np.float32(0.01)
        flat["v"] = r.random(N, dtype=np.float32) * np.float32(1e-4)
        self.host = flat
        A = hip.DeviceArray
        self.dev = []
        off = 0
        for n in sizes:
            d = {k: self.D(flat[k][off:off + n]) for k in ("p", "g", "m", "v")}
            d["q"] = A((n,))
            self.dev.append(d)
            off += n
        self.hyper = (6e-4, 0.9, 0.95, 1e-8, 0.1, 1)
        t = 10
        fwd = [(d["p"].ptr, d["g"].ptr, d["m"].ptr, d["v"].ptr, d["q"].ptr, n, t) for d, n in zip(self.dev, sizes)]
        back = [(d["q"].ptr, d["g"].ptr, d["m"].ptr, d["v"].ptr, d["p"].ptr, n, t) for d, n in zip(self.dev, sizes)]
        self.tables = [hip.slice_array(hip.AdamWSlice, fwd), hip.slice_array(hip.AdamWSlice, back)]
        self.flip = 0
        self.bytes_per_step = 28 * N  # read p, g, m, v; write p', m, v

    def _multi(self):
        L, c = self.hip.lib, self.hip.check
        c(L.oxi_adamw_step_multi(self.tables[self.flip], len(self.sizes), *self.hyper))
        self.flip ^= 1

    def kernels(self):
        return [("adamw_step_multi", self._multi, self.bytes_per_step)]

    def per_tensor(self):
        """The same step with one oxi_adamw_step launch per parameter."""
        L, c = self.hip.lib, self.hip.check
        lr, b1, b2, eps, wd, dec = self.hyper

        def run():
            for d, n in zip(self.dev, self.sizes):
                c(L.oxi_adamw_step(d["p"].ptr, d["g"].ptr, d["m"].ptr, d["v"].ptr, d["q"].ptr, n, lr, b1, b2, eps, wd,
                                   dec, 10))
        return [("adamw_step_per_tensor", run, self.bytes_per_step)]

    def cpu_step(self, ref, lo, hi):
        h = self.host
        m, v = h["m"][lo:hi].copy(), h["v"][lo:hi].copy()
        ref.adamw_step(h["p"][lo:hi], h["g"][lo:hi], m, v, 10, *self.hyper)


class F2(Workload):
    """The input pipeline: shuffled batches of 8192 rows from an MNIST-shaped
    dataset (60000 x 784 features + labels, fp32) resident in HBM, drawn
    through the host core's DataLoader (one device gather of all columns per
    batch, the epoch's order uploaded once). Side figures: 256 MiB host->device
    and device->host through the pinned staging ring and through plain
    waiting copies."""

    def __init__(self, hip):
        super().__init__(hip)
        import oxitorch_amd as ox
        from oxitorch_amd import _native

        N, D, B = 60000, 784, 8192
        self.N, self.Dm, self.B = N, D, B
        self.name = ("F2 device DataLoader, MNIST-shaped (60000,784)+labels fp32, shuffled batches of 8192 rows, "
                     "num_workers=4")
        r = np.random.default_rng(22)
        x = r.standard_normal((N, D), dtype=np.float32)
        y = r.integers(0, 10, N).astype(np.float32)
        self.host = dict(x=x, y=y)
        # four host threads compute the coming epochs' orders (the only host work)
        self.loader = _native.DataLoader([ox.from_numpy(x), ox.from_numpy(y)], batch_size=B, shuffle=True,
                                         drop_last=True, seed=5, num_workers=4)
        self.it = iter(self.loader)
        self.rows = B
        self.perm = np.random.RandomState(5).permutation(N)
        # per batch: each row read and written once per column, plus its id
        self.bytes_per_step = 2 * B * (D + 1) * 4 + 2 * B * 8
        self.keep = None

    def _batch(self):
        try:
            self.keep = next(self.it)
        except StopIteration:
            self.it = iter(self.loader)
            self.keep = next(self.it)

    def kernels(self):
        return [("loader_batch", self._batch, self.bytes_per_step)]

    def side_figures(self):
        """PCIe rates of 256 MiB copies (GB/s)."""
        hip = self.hip
        nb = 256 << 20
        a = np.random.default_rng(1).integers(0, 255, nb, dtype=np.uint8)
        back = np.empty_like(a)
        d = hip.DeviceArray((nb,), np.uint8)
        out = {}
        for label, fn in [("upload_staged", lambda: hip.call("oxi_hip_upload", d.ptr, a.ctypes.data, nb)),
                          ("h2d_waiting_copy", lambda: hip.call("oxi_hip_memcpy_h2d", d.ptr, a.ctypes.data, nb)),
                          ("download_staged", lambda: hip.call("oxi_hip_download", back.ctypes.data, d.ptr, nb)),
                          ("d2h_waiting_copy", lambda: hip.call("oxi_hip_memcpy_d2h", back.ctypes.data, d.ptr, nb))]:
            fn()
            hip.sync()
            t0 = time.perf_counter()
            for _ in range(5):
                fn()
            hip.sync()
            out[label] = round(5 * nb / (time.perf_counter() - t0) / 1e9, 2)
        assert np.array_equal(back, a)
        d.free()
        return out

    def cpu_step(self, ref, lo, hi):
        # the reference's worker path: host index_select of the batch rows
        h = self.host
        ids = self.perm[lo % self.N:lo % self.N + (hi - lo)]
        ref.index_select(h["x"], 0, ids)
        ref.index_select(h["y"].reshape(-1, 1), 0, ids)


class F3(Workload):
    """The remaining indexing ops, fwd+bwd: masked_select over x (16384, 4096)
    with a density-0.5 mask of the same shape, and the last-write-wins row
    scatter of 16384 rows (with repeats) into a (50257, 768) table."""

    cpu_full = True

    def __init__(self, hip):
        super().__init__(hip)
        R, H = 16384, 4096
        V, D, n = 50257, 768, 16384
        self.R, self.H, self.V, self.Dm, self.n = R, H, V, D, n
        self.name = "F3 masked_select (16384,4096) p=0.5 + scatter_dim0 16384 rows into (50257,768), fwd+bwd fp32"
        r = np.random.default_rng(33)
        x = r.standard_normal((R, H), dtype=np.float32)
        m = (r.random((R, H), dtype=np.float32) < 0.5).astype(np.float32)
        base = r.standard_normal((V, D), dtype=np.float32)
        ids = r.integers(0, V, n).astype(np.int64)
        vals = r.standard_normal((n, D), dtype=np.float32)
        gs = r.standard_normal((V, D), dtype=np.float32)
        self.count = int((m != 0).sum())
        gm = r.standard_normal(self.count, dtype=np.float32)
        self.host = dict(x=x, m=m, base=base, ids=ids, vals=vals, gs=gs, gm=gm)
        for k, v in self.host.items():
            setattr(self, "d_" + k, self.D(v))
        A = hip.DeviceArray
        self.gx = A((R, H))
        self.out_s, self.gb, self.gv = A((V, D)), A((V, D)), A((n, D))
        self.rows = R + n
        E = R * H
        # masked_select moves x and the mask in, the picks and its record (one
        # bit per element) out; its VJP reads the record and the upstream
        # gradient and writes grad_x
        self.op_bytes = dict(masked_select_fwd=8 * E + 4 * self.count + E // 8,
                             masked_select_bwd=E // 8 + 4 * self.count + 4 * E,
                             scatter_rows_fwd=8 * V * D + 8 * n, scatter_rows_bwd=8 * V * D + 4 * n * D + 8 * n)
        self.bytes_per_step = sum(self.op_bytes.values())
        st = hip._i64arr
        self.s_x, self.s_shape = st((H, 1)), st((R, H))
        self.picked = None
        self.record = hip.masked_select_record((R, H))

    def _msel(self):
        L, c = self.hip.lib, self.hip.check
        out, cnt = self.hip.vp(), self.hip.c_i64(0)
        c(L.oxi_masked_select(self.d_x.ptr, self.s_x, self.d_m.ptr, self.s_x, self.s_shape, 2,
                              self.hip.ctypes.byref(out), self.hip.ctypes.byref(cnt), self.record.ptr))
        if self.picked:
            c(L.oxi_hip_free(self.picked))
        self.picked = out.value

    def kernels(self):
        L, c = self.hip.lib, self.hip.check
        V, D, n, b = self.V, self.Dm, self.n, self.op_bytes
        return [
            ("masked_select_fwd", self._msel, b["masked_select_fwd"]),
            ("masked_select_bwd", lambda: c(L.oxi_masked_select_bwd(
                self.record.ptr, self.s_shape, 2, self.d_gm.ptr, self.count, self.gx.ptr, self.s_x,
                self.R * self.H)), b["masked_select_bwd"]),
            ("scatter_rows_fwd", lambda: c(L.oxi_scatter_rows(self.d_base.ptr, V, D, self.d_ids.ptr, n,
                                                              self.d_vals.ptr, self.out_s.ptr)),
             b["scatter_rows_fwd"]),
            ("scatter_rows_bwd", lambda: c(L.oxi_scatter_rows_bwd(self.d_gs.ptr, V, D, self.d_ids.ptr, n,
                                                                  self.gb.ptr, self.gv.ptr)), b["scatter_rows_bwd"]),
        ]

    def cpu_step(self, ref, lo, hi):
        h = self.host
        ref.masked_select(h["x"], h["m"])
        ref.masked_select_bwd(h["x"].shape, h["m"], h["gm"])
        ref.scatter_dim0(h["base"], h["ids"], h["vals"])
        ref.scatter_dim0_bwd(h["gs"], h["ids"], h["vals"].shape)


WORKLOADS = {"c1": C1, "c2": C2, "c3": C3, "c4": C4, "c5": C5, "f2": F2, "f3": F3, "f4": F4}


# ---------------------------------------------------------------------------

class _NoGC:
    """Python's cycle collector off around a timed loop of C-ABI calls (as
    timeit does): a collection pass started by the objects earlier
    measurements left would otherwise land in a few hundred microseconds of
    timed launches. The F.* step is timed with the collector on, as a user
    runs it."""

    def __enter__(self):
        gc.collect()
        self.was = gc.isenabled()
        gc.disable()

    def __exit__(self, *exc):
        if self.was:
            gc.enable()


class Events:
    """A pool of HIP events recorded on the library stream in sequence; the
    times between consecutive records, read once the stream has passed the
    last one."""

    def __init__(self, hip, n):
        self.hip = hip
        self.ev = []
        for _ in range(n):
            e = hip.vp()
            hip.check(hip.lib.oxi_hip_event_create(hip.ctypes.byref(e)))
            self.ev.append(e)
        self.k = 0

    def record(self):
        self.hip.check(self.hip.lib.oxi_hip_event_record(self.ev[self.k]))
        self.k += 1

    def ms(self, i, j):
        """Milliseconds from record i to record j (waits for record j)."""
        out = self.hip.c_float(0.0)
        self.hip.check(self.hip.lib.oxi_hip_event_elapsed_ms(self.ev[i], self.ev[j], self.hip.ctypes.byref(out)))
        return out.value

    def free(self):
        for e in self.ev:
            self.hip.lib.oxi_hip_event_destroy(e)
        self.ev = []


def time_steps(hip, kernels, steps, host=None):
    """Warm device time per step over `steps` back-to-back steps (HIP events
    on the library stream around the run); `host`, when given, receives the
    host's issue time per step (a host that issues slower than the device
    runs leaves the device idle)."""
    t = hip.Timer()
    hip.sync()
    with _NoGC():
        t.start()
        h0 = time.perf_counter()
        for _ in range(steps):
            for _, fn, _ in kernels:
                fn()
        h1 = time.perf_counter()
        ms = t.stop()
    hip.sync()
    if host is not None:
        host.append((h1 - h0) * 1e3 / steps)
    return ms / steps


def time_calls(hip, kernels, reps):
    """Each C-ABI call of the step timed alone: two untimed launches (a
    repeated call can take a path the first does not, e.g. a plan applied a
    second time, and a kernel's first launch loads its code), then `reps`
    back-to-back launches between two events on the library stream (its
    inputs stay in the Infinity Cache: a warm figure, not the in-step one)."""
    t = hip.Timer()
    out = {}
    for label, fn, nbytes in kernels:
        fn()
        fn()
        hip.sync()
        with _NoGC():
            t.start()
            for _ in range(reps):
                fn()
            avg = t.stop() / reps
        out[label] = {"ms": avg, "bytes": nbytes, "gbs": nbytes / (avg * 1e-3) / 1e9 if nbytes else None}
    hip.sync()
    return out


FLUSH_BYTES = 512 << 20  # twice the 256 MB Infinity Cache


class Flush:
    """Evicts a step's inputs from the Infinity Cache (and the L2s) before it
    is timed, so that the step reads them from HBM. mode "write": a 512 MiB
    fill, which leaves the cache full of the fill's dirty lines, whose
    write-back the step then pays; "write-read": the fill, then a column sum
    that reads the 512 MiB back (writing 4 MiB), which leaves clean lines of
    the scratch buffer; "read": the column sum alone."""

    ROWS = 128

    def __init__(self, hip, mode="write-read", buf=None):
        self.hip = hip
        self.mode = mode
        n = FLUSH_BYTES // 4
        self.own = buf is None
        self.buf = hip.DeviceArray((n,)) if buf is None else buf
        self.out = hip.DeviceArray((n // self.ROWS,))
        self.shape = hip._i64arr((self.ROWS, n // self.ROWS))
        self.strides = hip._i64arr((n // self.ROWS, 1))
        if self.own:
            hip.check(hip.lib.oxi_fill(self.buf.ptr, n, 0.0))

    def __call__(self):
        L, c = self.hip.lib, self.hip.check
        if self.mode in ("write", "write-read"):
            c(L.oxi_fill(self.buf.ptr, FLUSH_BYTES // 4, 0.0))
        if self.mode in ("read", "write-read"):
            c(L.oxi_reduce(0, self.buf.ptr, self.strides, self.shape, 2, 0, self.out.ptr))

    def free(self):
        if self.own:
            self.buf.free()
        self.out.free()


def time_graded(hip, kernels, steps, flush, per_call, only=None):
    """`steps` steps, each after an untimed flush() (a no-op for warm steps),
    timed alone with HIP events on the library stream. With per_call, events
    also sit between the step's calls. Returns (step times in ms, {call: [ms
    per step]}). With `only` (a call's index), the two events of each step
    bracket that call alone, and the step times are that call's times."""
    n = len(kernels)
    marks = (n + 1) if per_call else 2
    ev = Events(hip, steps * marks)
    hip.sync()
    with _NoGC():
        for _ in range(steps):
            flush()
            if only is None:
                ev.record()
            for i, (_, fn, _) in enumerate(kernels):
                if i == only:
                    ev.record()
                fn()
                if per_call or (i == n - 1 if only is None else i == only):
                    ev.record()
    hip.sync()
    step_ms, calls = [], {label: [] for label, _, _ in kernels}
    for s in range(steps):
        base = s * marks
        step_ms.append(ev.ms(base, base + marks - 1))
        if per_call:
            for i, (label, _, _) in enumerate(kernels):
                calls[label].append(ev.ms(base + i, base + i + 1))
    ev.free()
    return step_ms, calls


def median(v):
    v = sorted(v)
    n = len(v)
    return v[n // 2] if n % 2 else 0.5 * (v[n // 2 - 1] + v[n // 2])


def same_bytes_copy(hip, kernels, steps):
    """The step's launch sequence with each call that moves data replaced by
    one identity copy (oxi_unary IDENTITY, the flat float4 kernel) reading
    half and writing half of that call's algorithmic bytes: what a step of
    this many launches and bytes costs when every launch is a plain copy."""
    sizes = [b for _, _, b in kernels if b > 0]
    nmax = max(sizes) // 8
    a, b = hip.DeviceArray((nmax,)), hip.DeviceArray((nmax,))
    hip.check(hip.lib.oxi_fill(a.ptr, nmax, 1.0))
    one = hip._i64arr((1,))
    calls = []
    for nbytes in sizes:
        shape = hip._i64arr((nbytes // 8,))
        calls.append(("copy", lambda shape=shape: hip.check(hip.lib.oxi_unary(19, a.ptr, one, b.ptr, one, shape, 1)),
                      nbytes))
    for _ in range(2):
        for _, fn, _ in calls:
            fn()
    ms = time_steps(hip, calls, steps)
    a.free()
    b.free()
    moved = sum(8 * (n // 8) for n in sizes)
    return {"ms_per_step": round(ms, 5), "gbs": round(moved / (ms * 1e-3) / 1e9, 1), "launches": len(calls)}


def copy_probe(hip, nbytes=1 << 30):
    """STREAM-style copy rates (read + write bytes) on this GPU."""
    a = hip.DeviceArray((nbytes // 4,))
    b = hip.DeviceArray((nbytes // 4,))
    hip.check(hip.lib.oxi_fill(a.ptr, nbytes // 4, 1.0))
    t = hip.Timer()
    res = {}
    for label, fn in [("hip_memcpy_d2d", lambda: hip.check(hip.lib.oxi_hip_memcpy_d2d(b.ptr, a.ptr, nbytes))),
                      ("oxi_copy_kernel", lambda: hip.unary("identity", a, out=b))]:
        fn()
        hip.sync()
        t.start()
        for _ in range(5):
            fn()
        ms = t.stop() / 5
        res[label] = round(2 * nbytes / (ms * 1e-3) / 1e9, 1)
    a.free()
    b.free()
    return res


def _cpu_threads():
    """Host threads for the threaded baseline: the box's CPU share (at most 16)."""
    return max(1, min(os.cpu_count() or 1, 16))


def cpu_threaded(wl, ref, budget_s, threads):
    """Row chunks of the same workload on `threads` host threads (the oracle's
    C calls release the GIL); returns (rows, seconds)."""
    from concurrent.futures import ThreadPoolExecutor

    chunk = max(1, min(wl.rows // threads, 1024))
    t0 = time.perf_counter()
    done = 0
    with ThreadPoolExecutor(max_workers=threads) as pool:
        while time.perf_counter() - t0 < budget_s:
            starts = [((done + k * chunk) % wl.rows) for k in range(threads)]
            list(pool.map(lambda lo: wl.cpu_step(ref, lo, min(lo + chunk, wl.rows)), starts))
            done += sum(min(lo + chunk, wl.rows) - lo for lo in starts)
    return done, time.perf_counter() - t0


def cpu_baseline(wl, budget_s):
    from oracle import ref  # the checker/baseline, never the measured product

    full = isinstance(wl, (C4, C5)) or getattr(wl, "cpu_full", False)
    if full:
        # a dense dW per call makes row samples unrepresentative (C4, C5), and
        # per-call overhead would swamp small element ranges (F4): time the
        # full workload once
        t0 = time.perf_counter()
        wl.cpu_step(ref, 0, wl.rows)
        done = wl.rows
    else:
        rows = min(wl.rows, 64)
        t0 = time.perf_counter()
        wl.cpu_step(ref, 0, rows)
        dt = time.perf_counter() - t0
        target = max(rows, min(wl.rows, int(rows * (budget_s / max(dt, 1e-6)) * 0.8)))
        chunk = min(wl.rows, 4096)
        t0 = time.perf_counter()
        done = 0
        while done < target and time.perf_counter() - t0 < budget_s:
            n = min(chunk, target - done)
            lo = done % wl.rows
            wl.cpu_step(ref, lo, min(lo + n, wl.rows))
            done += min(n, wl.rows - lo)
    el = time.perf_counter() - t0
    bytes_per_row = wl.bytes_per_step / wl.rows
    one = {"value": round(done * bytes_per_row / el / 1e9, 4), "rows_per_s": round(done / el, 1),
           "sample": f"{done} of {wl.rows} rows, {el:.2f} s"}
    out = {
        "value": one["value"],
        "unit": "GB/s",
        "rows_per_s": one["rows_per_s"],
        "cores": 1,
        "kind": "port",
        "sample": f"{done} of {wl.rows} rows of the same workload, fwd+bwd through oracle/refcpu.c "
                  f"(single thread), {el:.2f} s; GB/s scaled by the same algorithmic bytes per row",
    }
    threads = _cpu_threads()
    if threads > 1 and not full:
        # row-parallel like the reference's rayon row reductions (its
        # elementwise passes run on one thread, so this is the faster of the two)
        n, secs = cpu_threaded(wl, ref, budget_s, threads)
        out["single_thread"] = one
        out["value"] = round(n * bytes_per_row / secs / 1e9, 4)
        out["rows_per_s"] = round(n / secs, 1)
        out["cores"] = threads
        out["sample"] = (f"row chunks of the same workload on {threads} host threads through oracle/refcpu.c, "
                         f"{n} rows in {secs:.2f} s (single thread: {one['sample']}); GB/s scaled by the same "
                         "algorithmic bytes per row")
        out["note"] = ("an upper bound on the reference: it parallelises whole rows, where the reference runs its "
                       "elementwise passes on one thread (iterate.rs:21) and its column sums serially "
                       "(lib.rs:549-558); single_thread is the other bound")
    return out


def _calls_json(per):
    return {k: {"avg_ms": round(v["ms"], 5), "gbs": None if v["gbs"] is None else round(v["gbs"], 1)}
            for k, v in per.items()}


# the kernels each C-ABI call launches (rocprofv3 names), to read a call's
# in-step time off a kernel trace
CALL_KERNELS = {
    "rms_norm_fwd": "norm_fwd_k (rms)", "layer_norm_fwd": "norm_fwd_k (layer)",
    "rms_norm_bwd": "norm_bwd_k", "layer_norm_gelu_bwd": "norm_bwd_k (+ gelu)",
    "rms_norm_softmax_pos_bwd": "norm_bwd_k (+ softmax, positional sum)",
    "layer_norm_silu_bwd": "norm_bwd_k (+ silu)",
    "cross_entropy_fwd_grad": "ce_fwd_rows_k", "embedding_fwd": "gather_k",
    "embedding_bwd": "seg_wave_k + seg_fixup_k", "embedding_bwd_plan": "sort_hist_k + sort_scatter_k (side stream)",
    "silu_fwd": "map_regt_k (silu)", "add_fwd": "map_regt_k (add)", "softmax_fwd": "sm_fwd_k",
    "gelu_erf_fwd": "map_flat_vec_k (gelu)", "masked_select_fwd": "masked-select kernels",
}


def roofline(in_step, nbytes, traffic, source):
    """The dominant call (largest in-step time among the calls that move
    data) against the HBM peak, its time the median of its in-step times."""
    dom = max((k for k in in_step if nbytes[k] > 0), key=lambda k: in_step[k])
    ms = in_step[dom]
    gbs = nbytes[dom] / (ms * 1e-3) / 1e9
    return {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
            "frac": round(gbs / PEAK_HBM_GBS, 4), "traffic": traffic.get(dom),
            "kernel": dom, "kernels": CALL_KERNELS.get(dom, dom), "algorithmic_bytes": nbytes[dom],
            "avg_launch_ms": round(ms, 5), "traffic_source": source if dom in traffic else None,
            "timing": "HIP events around the call inside each cold-MALL step, median of K"}


def time_dropin(hip, wl, steps, warmup, hbm, make=None):
    """The step through the Python surface (F.* and backward() over the host
    core's graph): device time per step (events on the library stream around
    `steps` steps, so host gaps count) and the host's time per step."""
    import oxitorch_amd as ox
    from oxitorch_amd.nn import functional as F

    step = (make or wl.dropin)(ox, F)
    for _ in range(max(warmup, 1)):
        step()
    hip.sync()
    # enough steps for about 0.2 s, so that the host settles into its
    # steady state (a few steps time the first ones only)
    t0 = time.perf_counter()
    for _ in range(3):
        step()
    hip.sync()
    est = (time.perf_counter() - t0) / 3
    steps = max(steps, min(2000, int(0.2 / max(est, 1e-6))))
    t = hip.Timer()
    t.start()
    h0 = time.perf_counter()
    for _ in range(steps):
        step()
    h1 = time.perf_counter()
    ms = t.stop() / steps
    hip.sync()
    return {"what": wl.dropin_what, "steps": steps, "ms_per_step": round(ms, 5),
            "host_ms_per_step": round((h1 - h0) * 1e3 / steps, 5), "gbs": round(hbm / (ms * 1e-3) / 1e9, 2)}


def _rate(nbytes, ms):
    gbs = nbytes / (ms * 1e-3) / 1e9
    return round(gbs, 2), round(100.0 * gbs / PEAK_HBM_GBS, 2)


def run_config(hip, key, args, flush):
    """Everything measured for one config; returns (compact block, detail).

    W untimed warmup steps and about SETTLE_S s of untimed steps, then K
    cold and K warm timed steps (the main figure is the slower median),
    then K steps with per-call events under the graded protocol, then the
    other measurements."""
    log(f"[{key}] building workload")
    wl = WORKLOADS[key](hip)
    kernels = wl.kernels()
    nbytes = {label: b for label, _, b in kernels}
    hbm = sum(nbytes.values())
    traffic = pmc_traffic(key)
    for _ in range(max(args.warmup, 1)):
        for _, fn, _ in kernels:
            fn()
    hip.sync()
    # untimed steps for about SETTLE_S more: the host work before a config
    # (building it, the previous config's CPU baseline) leaves the GPU idle
    # for seconds, and a few warmup steps do not bring it back to its steady
    # clocks (default runs had measured C2's warm step 8-30 us slower than
    # runs of C2 alone)
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < SETTLE_S:
        for _, fn, _ in kernels:
            fn()
        hip.sync()
    # cold: each step after a flush (inputs from HBM, a clean cache); warm:
    # back-to-back steps, each also paying the previous step's write-backs
    log(f"[{key}] timing {args.steps} cold-MALL steps")
    cold_steps, _ = time_graded(hip, kernels, args.steps, flush, per_call=False)
    log(f"[{key}] timing {args.steps} warm steps")
    warm_steps, _ = time_graded(hip, kernels, args.steps, lambda: None, per_call=False)
    cms, wms = median(cold_steps), median(warm_steps)
    graded = "cold" if cms >= wms else "warm"
    ms = max(cms, wms)
    gbs, pct = _rate(hbm, ms)
    op_gbs, op_pct = _rate(wl.bytes_per_step, ms)
    cg, cp = _rate(hbm, cms)
    wg, wp = _rate(hbm, wms)
    block = {"workload": wl.name, "ms_per_step": round(ms, 5), "graded": graded, "gbs": gbs, "pct_of_peak": pct,
             "per_op_gbs": op_gbs, "per_op_pct_of_peak": op_pct, "rows_per_s": round(wl.rows / (ms * 1e-3), 1),
             "rows_per_step": wl.rows, "hbm_bytes_per_step": hbm, "per_op_bytes_per_step": wl.bytes_per_step,
             "cold": {"ms_per_step": round(cms, 5), "gbs": cg, "pct_of_peak": cp,
                      "range_ms": [round(min(cold_steps), 5), round(max(cold_steps), 5)]},
             "warm": {"ms_per_step": round(wms, 5), "gbs": wg, "pct_of_peak": wp,
                      "range_ms": [round(min(warm_steps), 5), round(max(warm_steps), 5)]}}
    detail = {"cold_steps_ms": [round(v, 5) for v in cold_steps], "warm_steps_ms": [round(v, 5) for v in warm_steps]}
    if args.only_graded:
        wl.release()
        return block, detail
    log(f"[{key}] timing each call inside {args.steps} {graded} steps")
    _, calls = time_graded(hip, kernels, args.steps, flush if graded == "cold" else (lambda: None), per_call=True)
    in_step = {k: median(v) for k, v in calls.items()}
    block["in_step_us"] = {k: round(v * 1e3, 1) for k, v in in_step.items()}
    block["roofline"] = roofline(in_step, nbytes, traffic, f"profiles/pmc_traffic_{key}.md")
    # the dominant call again, with events around it alone: events between
    # every call add a launch bubble at each and shift the step's timing
    dom = block["roofline"]["kernel"]
    idx = [label for label, _, _ in kernels].index(dom)
    log(f"[{key}] timing {dom} alone inside {args.steps} {graded} steps")
    alone, _ = time_graded(hip, kernels, args.steps, flush if graded == "cold" else (lambda: None), per_call=False,
                           only=idx)
    block["roofline"] = roofline({dom: median(alone)}, nbytes, traffic, f"profiles/pmc_traffic_{key}.md")
    block["roofline"]["timing"] = (f"HIP events around this call alone inside each {graded} step (the graded "
                                   "protocol), median of K; the call is the one with the largest in_step_us")
    host_ms = []
    time_steps(hip, kernels, args.steps, host_ms)
    block["warm"]["host_issue_ms_per_step"] = round(host_ms[0], 5)
    # the flush of the survey's protocol as written: a 512 MiB fill alone
    # leaves the cache full of its own dirty lines, whose write-back the step
    # then pays
    wflush = Flush(hip, "write", flush.buf)
    ws_steps, _ = time_graded(hip, kernels, args.steps, wflush, per_call=False)
    block["cold_after_fill_only_ms"] = round(median(ws_steps), 5)
    reps = max(5, min(args.steps, 20))
    detail["calls_alone_warm"] = _calls_json(time_calls(hip, kernels, reps))
    if hasattr(wl, "unfused_kernels"):
        uk = wl.unfused_kernels()
        for _ in range(max(args.warmup, 1)):
            for _, fn, _ in uk:
                fn()
        hip.sync()
        log(f"[{key}] timing the node-by-node backward")
        ums = time_steps(hip, uk, args.steps)
        ubytes = sum(b for _, _, b in uk)
        block["unfused_ms"] = round(ums, 5)
        detail["unfused"] = {"what": wl.unfused_what, "ms_per_step": round(ums, 5),
                             "algorithmic_bytes_per_step": ubytes, "gbs": _rate(ubytes, ums)[0],
                             "calls_alone_warm": _calls_json(time_calls(hip, uk, reps))}
    log(f"[{key}] same-bytes copy floor")
    cf = same_bytes_copy(hip, kernels, args.steps)
    block["copy_floor_ms"] = cf["ms_per_step"]
    detail["same_bytes_copy"] = cf
    if hasattr(wl, "side_figures"):
        block["pcie_gbs"] = wl.side_figures()
    if hasattr(wl, "per_tensor"):
        alt = wl.per_tensor()
        ms_alt = time_steps(hip, alt, max(3, min(args.steps, 10)))
        block["per_tensor_launches_ms"] = round(ms_alt, 5)
    if hasattr(wl, "dropin") and not args.no_dropin:
        log(f"[{key}] timing the F.*/backward() step")
        d = time_dropin(hip, wl, max(3, min(args.steps, 10)), args.warmup, hbm)
        block["dropin_ms"] = d["ms_per_step"]
        block["dropin_host_ms"] = d["host_ms_per_step"]
        detail["dropin"] = d
        if hasattr(wl, "dropin_array"):
            d2 = time_dropin(hip, wl, max(3, min(args.steps, 10)), args.warmup, hbm, make=wl.dropin_array)
            d2["what"] = "the same with the ids as a numpy int64 array"
            block["dropin_array_ms"] = d2["ms_per_step"]
            detail["dropin_array"] = d2
    if isinstance(wl, C4):
        block["distinct_ids"] = wl.unique_rows  # the rows of W the gather's HBM bytes count
    block["cpu_baseline"] = None
    if not args.no_cpu and args.cpu_seconds > 0:
        log(f"[{key}] timing the CPU oracle baseline")
        block["cpu_baseline"] = cpu_baseline(wl, args.cpu_seconds)
    wl.release()
    return block, detail


def summary_line(b):
    """One short string per config for the end of the line."""
    out = (f"graded ({b['graded']}) {b['ms_per_step'] * 1e3:.1f}us {b['pct_of_peak']:.1f}% moved "
           f"({b['per_op_pct_of_peak']:.1f}% per-op); cold {b['cold']['ms_per_step'] * 1e3:.1f}us, "
           f"warm {b['warm']['ms_per_step'] * 1e3:.1f}us")
    if "roofline" in b:
        r = b["roofline"]
        out += f"; dominant {r['kernel']} {r['avg_launch_ms'] * 1e3:.1f}us frac {r['frac']:.3f} in-step"
    if "dropin_ms" in b:
        out += f"; F.* {b['dropin_ms'] * 1e3:.1f}us"
    cb = b.get("cpu_baseline")
    if cb:
        out += f"; cpu {cb['value']:.2f} GB/s ({cb['cores']} thr)"
    return out


HEADLINE = "c3"
ALL = ["c1", "c2", "c3", "c4", "c5"]


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU (asked for --gpus {args.gpus}); the row-sharded multi-GPU "
              "path is not built", file=sys.stderr)
        sys.exit(2)
    from oxitorch_amd import capi as hip

    if hip.device_count() == 0:
        print("bench.py: no HIP device visible", file=sys.stderr)
        sys.exit(1)
    hip.init(0)
    keys = ALL if args.config == "all" else [args.config]
    flush = Flush(hip, args.flush)
    blocks, details = {}, {}
    for k in keys:
        blocks[k], details[k] = run_config(hip, k, args, flush)
    flush.free()
    head_key = HEADLINE if args.config == "all" else args.config
    head = blocks[head_key]
    line = {
        "metric": METRIC,
        "value": head["gbs"],
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded inputs of the configs' shapes and distributions)",
        "config": {"workload": head["workload"], "headline": head_key,
                   "why": ("the largest config (3.15 GB per step); every config is under configs and summary"
                           if args.config == "all" else "selected with --config"),
                   "protocol": ("the graded step is the slower of two medians over K steps: cold (before each "
                                f"step a 512 MiB scratch buffer is flushed with mode {args.flush!r}, so the inputs "
                                "come from HBM and the cache holds no dirty lines) and warm (back-to-back steps, "
                                "each paying the previous step's write-backs)"),
                   "rows_per_step": head["rows_per_step"]},
        "roofline": head.get("roofline"),
        "cpu_baseline": head.get("cpu_baseline"),
    }
    props = hip.device_props()
    # HBM3E moves 4 bits per pin per reported memory clock (8 Gb/s per pin at
    # 2 GHz), so clock x 4 x bus width is the interface peak the props imply
    line["device"] = {"arch": props["arch"], "compute_units": props["compute_units"],
                      "peak_from_props_gbs": round(props["memory_clock_khz"] * 1e3 * 4 * props["memory_bus_bits"]
                                                   / 8 / 1e9, 1), "peak_datasheet_gbs": PEAK_HBM_GBS}
    if not args.no_copy_probe and not args.only_graded:
        log("copy probe")
        line["stream_copy_gbs"] = copy_probe(hip)
    line["gbs_definitions"] = ("gbs/pct_of_peak: HBM bytes the step's kernels move (checked against rocprofv3 "
                               "FETCH_SIZE + WRITE_SIZE) over the graded step time; per_op: the metric's per-op "
                               "algorithmic bytes over the same time; roofline: the dominant call's in-step time "
                               "under the graded protocol, events around it alone; cold_after_fill_only_ms: cold steps after a 512 MiB fill "
                               "alone, which leaves its dirty lines for the step to write back")
    # the other configs' blocks in short (the headline's block and the detail
    # file keep everything), so that the whole line stays within a driver's
    # tail of its output
    for k, blk in blocks.items():
        details[k]["block"] = dict(blk)
        if k == head_key:
            continue
        cb = blk.get("cpu_baseline")
        if cb:
            blk["cpu_baseline"] = {"value": cb["value"], "unit": cb["unit"], "cores": cb["cores"],
                                   "kind": cb["kind"],
                                   "single_thread": (cb.get("single_thread") or {}).get("value", cb["value"])}
        r = blk.get("roofline")
        if r:
            blk["roofline"] = {key: r[key] for key in ("kernel", "avg_launch_ms", "achieved", "frac", "traffic")}
        for key in ("rows_per_step", "hbm_bytes_per_step", "per_op_bytes_per_step", "per_op_gbs"):
            blk.pop(key, None)
        for key in ("cold", "warm"):
            if key in blk:
                blk[key].pop("range_ms", None)
    line["configs"] = blocks
    line["summary"] = {k: summary_line(b) for k, b in blocks.items()}
    if args.detail:
        with open(args.detail, "w") as f:
            json.dump({"line": line, "detail": details}, f, indent=1)
    print(json.dumps(line, separators=(",", ":")), flush=True)


if __name__ == "__main__":
    main()
