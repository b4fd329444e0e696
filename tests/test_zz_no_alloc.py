"""oxi_layer_norm_bwd_noalloc: the allocation-free variant of the LayerNorm VJP.

It keeps its column partials in a fixed device scratch array instead of a
workspace, with the same kernels and launch shapes as oxi_layer_norm_bwd, so
its outputs must equal that entry point's bit for bit. Each case runs two
calls in a row, the second on a smaller input, so a stale partial left in the
shared array by the first call would show. The caching allocator's counters
must not move across a call (nothing allocated, nothing freed).
"""

import numpy as np
import pytest

from conftest import rng

pytestmark = pytest.mark.gpu


def _inputs(hip, seed, R, H):
    r = rng(seed)
    x = r.standard_normal((R, H), dtype=np.float32)
    w = (r.standard_normal(H, dtype=np.float32) * 0.02 + 1).astype(np.float32)
    b = (r.standard_normal(H, dtype=np.float32) * 0.02).astype(np.float32)
    g = r.standard_normal((R, H), dtype=np.float32)
    D = hip.DeviceArray.from_numpy
    xd, wd, bd, gd = D(x), D(w), D(b), D(g)
    _, mean, rstd = hip.layer_norm_fwd(xd, wd, bd, 1e-5)
    return xd, wd, mean, rstd, gd


def _noalloc(hip, xd, wd, mean, rstd, gd, mode):
    R, H = xd.shape
    dx, dw, db = hip.DeviceArray((R, H)), hip.DeviceArray((H,)), hip.DeviceArray((H,))
    hip.sync()
    before = hip.memory_stats()
    hip.layer_norm_bwd_noalloc(xd, wd, mean, rstd, gd, dx, dw, db, mode=mode)
    after = hip.memory_stats()
    hip.sync()
    assert after == before, f"allocator moved during the call: {before} -> {after}"
    return dx.numpy(), dw.numpy(), db.numpy()


# (first call, second smaller call): one-wave rows (16 rows per block), wide
# rows (one row per 512-thread block, 2 blocks per CU), rows that do not
# vectorize (one 256-thread block per row, partials accumulated in place)
CASES = [((4096, 768), (1000, 768)),
         ((16384, 4096), (777, 4096)),
         ((2048, 1024), (300, 256)),
         ((3000, 770), (129, 770))]


@pytest.mark.parametrize("mode", ["ref", "exact"])
@pytest.mark.parametrize("first,second", CASES)
def test_noalloc_matches_layer_norm_bwd(hip, first, second, mode):
    for k, (R, H) in enumerate((first, second)):
        print(f"noalloc case {R}x{H} mode={mode} call {k}", flush=True)
        xd, wd, mean, rstd, gd = _inputs(hip, 100 + 7 * k + R % 13, R, H)
        want = hip.layer_norm_bwd(xd, wd, mean, rstd, gd, mode=mode)
        got = _noalloc(hip, xd, wd, mean, rstd, gd, mode)
        for name, a, b in zip(("dx", "dw", "db"), got, want):
            assert np.array_equal(a, b.numpy()), f"{name} of call {k} ({R}x{H}, {mode}) differs from oxi_layer_norm_bwd"


def test_noalloc_partial_outputs_and_empty(hip):
    """dw only (db NULL), dx only, and zero rows (dw/db filled with zeros)."""
    R, H = 512, 768
    xd, wd, mean, rstd, gd = _inputs(hip, 7, R, H)
    _, dw_ref, _ = hip.layer_norm_bwd(xd, wd, mean, rstd, gd)
    dw = hip.DeviceArray((H,))
    hip.layer_norm_bwd_noalloc(xd, wd, mean, rstd, gd, None, dw, None)
    assert np.array_equal(dw.numpy(), dw_ref.numpy())
    dx_ref, _, _ = hip.layer_norm_bwd(xd, wd, mean, rstd, gd, need_dw=False, need_db=False)
    dx = hip.DeviceArray((R, H))
    hip.layer_norm_bwd_noalloc(xd, wd, mean, rstd, gd, dx, None, None)
    assert np.array_equal(dx.numpy(), dx_ref.numpy())
    e = hip.DeviceArray((0, H))
    dw0, db0 = hip.DeviceArray((H,)), hip.DeviceArray((H,))
    hip.check(hip.lib.oxi_fill(dw0.ptr, H, 5.0))
    hip.check(hip.lib.oxi_fill(db0.ptr, H, 5.0))
    hip.check(hip.lib.oxi_layer_norm_bwd_noalloc(e.ptr, wd.ptr, mean.ptr, rstd.ptr, e.ptr, None, dw0.ptr, db0.ptr,
                                                 0, H, 0))
    assert not dw0.numpy().any() and not db0.numpy().any()


def test_noalloc_refuses_rows_beyond_the_scratch(hip):
    """Rows of 12288 floats (past the register-row widths: one 256-thread
    block per CU) need 2 x 256 x 12288 x 4 bytes (24 MiB) of partials on a
    256-CU device: refused before any launch, with the limit in the message."""
    props = hip.device_props()
    R, H = 2 * 2 * props["compute_units"], 12288
    need = 2 * min(R, props["compute_units"]) * H * 4
    assert need > hip.NOALLOC_SCRATCH_BYTES
    x = hip.DeviceArray((R, H))
    stats = hip.DeviceArray((R,))
    dw = hip.DeviceArray((H,))
    with pytest.raises(ValueError, match="scratch"):
        hip.check(hip.lib.oxi_layer_norm_bwd_noalloc(x.ptr, None, stats.ptr, stats.ptr, x.ptr, None, dw.ptr, None,
                                                     R, H, 0))
