"""Shared pytest configuration.

`gpu` tests need a HIP device (MI355X); they call the product through the
liboxihip C-ABI and check it against the CPU oracle under oracle/.
"""

import os
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

RTOL = 1e-5
ATOL = 1e-6


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device; runs the liboxihip kernels")


# ---- parity report -------------------------------------------------------------------------
# The config tests record, per compared quantity, the device's worst error in
# units of the tolerance (atol + rtol*|want|) against the f32 oracle and
# against float64, and how many elements only the float64 arbiter admitted.
# The table is printed at the end of the session and written as JSON lines
# to $OXI_PARITY_REPORT when set.

PARITY = []


def record(config, what, stats):
    """Adds one compared quantity of `config` to the session's parity report."""
    PARITY.append(dict(config=config, what=what, **stats))
    return stats


def pytest_terminal_summary(terminalreporter):
    if not PARITY:
        return
    tr = terminalreporter
    tr.section("parity report (worst error in tolerance units; arbitrated = elements admitted by float64 only)")
    for r in PARITY:
        tr.write_line(f"{r['config']:4s} {r['what']:28s} n={r['n']:<11d} vs_oracle={_fmt(r.get('worst_tol'))} "
                      f"vs_f64={_fmt(r.get('worst_tol_f64'))} ref_vs_f64={_fmt(r.get('ref_worst_tol_f64'))} "
                      f"arbitrated={r.get('arbitrated', 0)}")
    path = os.environ.get("OXI_PARITY_REPORT")
    if path:
        import json
        with open(path, "w") as f:
            for r in PARITY:
                f.write(json.dumps(r) + "\n")


def _fmt(v):
    return "-" if v is None else f"{v:.3g}"


def _worst(got, want, rtol, atol):
    if got.size == 0:
        return 0.0
    return float((np.abs(got - want) / (atol + rtol * np.abs(want))).max())


@pytest.fixture(scope="session")
def hip():
    """The liboxihip ctypes binding with device 0 initialised (fails loudly if absent)."""
    from oxitorch_amd import capi

    if capi.device_count() == 0:
        pytest.fail("no HIP device visible: gpu tests must run on the MI355X box")
    capi.init(0)
    return capi


def assert_close(got, want, rtol=RTOL, atol=ATOL, what=""):
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    assert got.shape == want.shape, f"{what}: shape {got.shape} vs {want.shape}"
    err = np.abs(got - want)
    tol = atol + rtol * np.abs(want)
    bad = ~(err <= tol) & ~(np.isnan(got) & np.isnan(want))  # NaN must meet NaN
    if bad.any():
        i = np.flatnonzero(bad.ravel())[0]
        raise AssertionError(
            f"{what}: {bad.sum()} of {bad.size} elements outside rtol={rtol} atol={atol}; "
            f"first at flat {i}: got {got.ravel()[i]!r} want {want.ravel()[i]!r}; max err {err.max():.3e}"
        )
    fin = ~np.isnan(want)
    return {"n": int(got.size), "worst_tol": float((err[fin] / tol[fin]).max()) if fin.any() else 0.0,
            "arbitrated": 0}


def assert_reduction_close(got, ref32, exact64, rtol=RTOL, atol=ATOL, what=""):
    """Parity for long reductions (column sums, heavy embedding segments).

    Elements within rtol/atol of the float64 arbiter pass. For the rest, the
    reference's own sequential-f32 result must be at least as far from the
    arbiter in the worst case: the device result is then no less accurate than
    the reference path it replaces.
    """
    got = np.asarray(got, dtype=np.float64)
    ref32 = np.asarray(ref32, dtype=np.float64)
    exact64 = np.asarray(exact64, dtype=np.float64)
    tol = atol + rtol * np.abs(exact64)
    e_got = np.abs(got - exact64) / tol
    e_ref = np.abs(ref32 - exact64) / tol
    worst = float(e_got.max()) if e_got.size else 0.0
    stats = {"n": int(got.size), "worst_tol": _worst(got, ref32, rtol, atol), "worst_tol_f64": worst,
             "ref_worst_tol_f64": float(e_ref.max()) if e_ref.size else 0.0, "arbitrated": int((e_got > 1.0).sum())}
    if worst <= 1.0:
        return stats
    assert worst <= max(1.0, e_ref.max()), (
        f"{what}: device error {worst:.3g} x tolerance exceeds the reference path's own "
        f"worst error {e_ref.max():.3g} x tolerance against the float64 arbiter"
    )
    return stats


def assert_close_arb(got, ref32, exact64, rtol=RTOL, atol=ATOL, what=""):
    """Parity with the reference path, arbitrated by float64 where they differ.

    An element passes if it is within rtol/atol of the f32 reference path or of
    the float64 evaluation. The remaining elements must be no further from the
    float64 evaluation (in units of the tolerance) than the reference path's own
    worst element is: the device result is then no less accurate than the path
    it replaces. Where this matters: the reference's composed softmax-family
    VJPs add a mathematically-zero max-path term whose f32 rounding noise lands
    on the argmax element, and long chains of f32 ops round differently in any
    two evaluation orders.
    """
    got = np.asarray(got, dtype=np.float64)
    ref32 = np.asarray(ref32, dtype=np.float64)
    exact64 = np.asarray(exact64, dtype=np.float64)
    assert got.shape == ref32.shape == exact64.shape, f"{what}: shapes differ"
    tol_ex = atol + rtol * np.abs(exact64)
    ok = (np.abs(got - ref32) <= atol + rtol * np.abs(ref32)) | (np.abs(got - exact64) <= tol_ex)
    e_f64 = np.abs(got - exact64) / tol_ex
    stats = {"n": int(got.size), "worst_tol": _worst(got, ref32, rtol, atol),
             "worst_tol_f64": float(e_f64.max()) if e_f64.size else 0.0,
             "ref_worst_tol_f64": float((np.abs(ref32 - exact64) / tol_ex).max()) if got.size else 0.0,
             "arbitrated": int((~ok).sum())}
    if ok.all():
        return stats
    worst_got = e_f64[~ok].max()
    worst_ref = stats["ref_worst_tol_f64"]
    if worst_got > worst_ref:
        i = np.flatnonzero(~ok.ravel())[0]
        raise AssertionError(
            f"{what}: {(~ok).sum()} of {ok.size} elements outside both tolerances, worst {worst_got:.3g} x tol "
            f"from float64 vs the reference path's worst {worst_ref:.3g} x tol; first at flat {i}: got "
            f"{got.ravel()[i]!r} ref {ref32.ravel()[i]!r} f64 {exact64.ravel()[i]!r}")
    return stats


def assert_sum_close(got, ref32, abs_sum, rtol=RTOL, atol=ATOL, what=""):
    """Parity for short sums with cancellation: |got - ref| <= atol + rtol * sum|terms|.

    Any f32 evaluation order of a sum has an error bounded by a multiple of
    eps * sum|terms|; relative to |sum| that bound is unbounded when the
    terms cancel, so the tolerance is taken relative to the sum's condition.
    """
    got = np.asarray(got, dtype=np.float64)
    ref32 = np.asarray(ref32, dtype=np.float64)
    abs_sum = np.asarray(abs_sum, dtype=np.float64)
    err = np.abs(got - ref32)
    bad = err > atol + rtol * abs_sum
    assert not bad.any(), f"{what}: {bad.sum()} elements outside rtol*sum|terms|; max err {err.max():.3e}"


def segmented_runs_in_one_tile(ids, V, tile=16):
    """Keys whose stably-sorted run of positions lies inside one aligned
    `tile`-position block. The embedding VJP cuts the sorted positions into
    aligned tiles of 16, 32 or 64, so such a run lies inside one of its tiles:
    its row is summed in position order in f32 in one pass, exactly as the
    reference does, and must match bitwise."""
    keys = np.where(np.asarray(ids) < 0, np.asarray(ids) + V, np.asarray(ids))
    counts = np.bincount(keys, minlength=V)
    start = np.concatenate([[0], np.cumsum(counts)[:-1]])
    end = start + counts - 1
    return (counts > 0) & (start // tile == end // tile)


def rng(seed):
    return np.random.default_rng(seed)
