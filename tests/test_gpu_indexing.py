"""Row scatter (last write wins) and boolean-mask selection on the device,
forward and VJP, bit-exact against the CPU oracle (crates/oxi-tensor/src/
lib.rs:895-961, crates/oxi-autograd/src/ops.rs:531-667); then the reference's
own tests for them (python/tests/test_indexing_grad.py) through
oxitorch_amd."""

import ctypes
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
    assert got.shape == want.shape, f"{what}: shape {got.shape} vs {want.shape}"
    gb = np.where(np.isnan(got), np.uint32(0x7FC00000), got.view(np.uint32))
    wb = np.where(np.isnan(want), np.uint32(0x7FC00000), want.view(np.uint32))
    bad = np.flatnonzero(gb != wb)
    if bad.size:
        i = bad[0]
        raise AssertionError(f"{what}: {bad.size} of {got.size} differ; first at {i}: got {got.ravel()[i]!r} "
                             f"want {want.ravel()[i]!r}")


@pytest.fixture(scope="module")
def oracle():
    from oracle import ref

    return ref


def _ids(r, rows, n, dup=True):
    ids = r.integers(-rows, rows, n).astype(np.int64)
    if dup and n > 2:
        ids[: n // 3] = ids[0]
        ids[-1] = ids[1]
    return ids


SCATTER_CASES = [((7,), 5), ((9, 4), 12), ((6, 3, 5), 10), ((4, 2), 0), ((1000, 768), 3000), ((50257, 64), 20000),
                 ((300, 13), 1000), ((1, 8), 4)]


@pytest.mark.parametrize("shape,n", SCATTER_CASES)
def test_scatter_rows_matches_oracle(hip, oracle, shape, n):
    say("scatter_rows", shape, n)
    r = rng(10 + n)
    rows = shape[0]
    inner = int(np.prod(shape[1:], dtype=np.int64))
    ids = _ids(r, rows, n)
    base = r.standard_normal(shape).astype(np.float32)
    vals = r.standard_normal((n,) + shape[1:]).astype(np.float32)
    d_base, d_vals, d_ids = (hip.DeviceArray.from_numpy(a) for a in (base, vals, ids))
    out = hip.scatter_rows(d_base, d_ids, d_vals)
    bits_equal(out.numpy(), oracle.scatter_dim0(base, ids, vals), f"scatter {shape} n={n}")
    g = r.standard_normal(shape).astype(np.float32)
    g.ravel()[:3] = [-1.0, np.nan, -0.0][: min(3, g.size)]
    want_b, want_v = oracle.scatter_dim0_bwd(g, ids, vals.shape)
    d_g = hip.DeviceArray.from_numpy(g)
    gb, gv = hip.scatter_rows_bwd(d_g, d_ids, vals.shape)
    bits_equal(gb.numpy(), want_b, f"scatter bwd base {shape}")
    bits_equal(gv.numpy(), want_v, f"scatter bwd values {shape}")
    # one output at a time
    gb1, none = hip.scatter_rows_bwd(d_g, d_ids, vals.shape, need_values=False)
    assert none is None
    bits_equal(gb1.numpy(), want_b, "scatter bwd base only")
    none, gv1 = hip.scatter_rows_bwd(d_g, d_ids, vals.shape, need_base=False)
    bits_equal(gv1.numpy(), want_v, "scatter bwd values only")
    del inner


def test_scatter_rows_unaligned_operands(hip, oracle):
    """Pointers off 16-byte alignment take the scalar path."""
    say("scatter_rows unaligned")
    r = rng(3)
    rows, inner, n = 50, 8, 40
    ids = _ids(r, rows, n)
    base = r.standard_normal(rows * inner + 1).astype(np.float32)
    vals = r.standard_normal(n * inner + 1).astype(np.float32)
    d_base, d_vals, d_ids = (hip.DeviceArray.from_numpy(a) for a in (base, vals, ids))
    out = hip.DeviceArray((rows * inner + 1,))
    hip.call("oxi_scatter_rows", d_base.ptr + 4, rows, inner, d_ids.ptr, n, d_vals.ptr + 4, out.ptr + 4)
    want = oracle.scatter_dim0(base[1:].reshape(rows, inner), ids, vals[1:].reshape(n, inner))
    bits_equal(out.numpy()[1:].reshape(rows, inner), want, "unaligned scatter")


def test_scatter_rows_argument_errors(hip):
    with pytest.raises(ValueError, match="negative size"):
        hip.call("oxi_scatter_rows", None, -1, 4, None, 0, None, None)
    with pytest.raises(ValueError, match="empty tensor"):
        hip.call("oxi_scatter_rows", None, 0, 4, None, 3, None, None)
    with pytest.raises(ValueError, match="NULL"):
        hip.call("oxi_scatter_rows", None, 4, 4, None, 0, None, None)


def _grid_strides(shape, grid):
    from oxitorch_amd.capi import broadcast_elem_strides

    return broadcast_elem_strides(shape, grid)


MASK_CASES = [((3, 4), (3, 4), 0.5), ((2, 1, 5), (3, 5), 0.6), ((4,), (3, 1), 0.5), ((1,), (2, 3), 0.5),
              ((2, 3, 4), (4,), 0.5), ((4097,), (4097,), 0.3), ((16384, 4096), (16384, 4096), 0.5),
              ((1000, 1), (1000, 777), 0.1), ((64, 1, 33), (1, 50, 33), 0.9), ((5,), (5,), 0.0), ((3,), (3,), 1.0),
              # hundreds of 4096-point tiles with no pick or all picked
              ((1200000,), (1200000,), 0.0), ((1200000,), (1200000,), 0.00002), ((700, 3000), (700, 3000), 1.0)]


@pytest.fixture(params=["one_pass", "two_pass"])
def msel_path(request):
    """The one-pass path (default: x read once, the output sized for every
    grid point) and the two-pass path (OXI_MASKED_SELECT_EXACT=1)."""
    import os
    if request.param == "two_pass":
        os.environ["OXI_MASKED_SELECT_EXACT"] = "1"
    yield request.param
    os.environ.pop("OXI_MASKED_SELECT_EXACT", None)


@pytest.mark.parametrize("xs,ms,density", MASK_CASES)
def test_masked_select_matches_oracle(hip, oracle, xs, ms, density, msel_path):
    say("masked_select", msel_path, xs, ms, density)
    r = rng(20 + len(xs) * 7 + len(ms))
    x = r.standard_normal(xs, dtype=np.float32)
    m = (r.random(ms, dtype=np.float32) < density).astype(np.float32)
    if m.size > 2:
        m.ravel()[0] = -0.0
        m.ravel()[1] = np.nan
    if x.size > 3:
        x.ravel()[3] = np.nan  # dropped when picked
    d_x, d_m = hip.DeviceArray.from_numpy(x), hip.DeviceArray.from_numpy(m)
    grid = np.broadcast_shapes(xs, ms)
    rec = hip.masked_select_record(grid)
    got = hip.masked_select(d_x, d_m, rec)
    want = oracle.masked_select(x, m)
    assert got.shape == want.shape, (got.shape, want.shape)
    if want.size:
        bits_equal(got.numpy(), want, f"masked_select {xs} {ms}")
    else:
        assert got.ptr is None
    # VJP from the forward's record: its picks exclude NaN values of x, so
    # compare with the oracle's VJP on a mask that skips those points
    g = r.standard_normal(want.size, dtype=np.float32)
    gx = hip.masked_select_bwd(rec, xs, ms, hip.DeviceArray.from_numpy(g) if g.size else hip.DeviceArray((0,)))
    nanpos = np.broadcast_to(np.isnan(x), grid)
    mb = np.broadcast_to(m, grid).copy()
    mb[nanpos] = 0.0
    want_gx = oracle.masked_select_bwd(xs, mb, g)
    bits_equal(gx.numpy(), want_gx, f"masked_select bwd {xs} {ms}")
    got.free()


@pytest.mark.parametrize("density,exact", [(0.1, True), (0.3, True), (0.6, False)])
def test_masked_select_output_memory(hip, oracle, density, exact):
    """The one pass's output: picks that fill at most a third of the grid
    move into a buffer of their own size (the allocator's 512-byte or 2 MiB
    rounding aside), denser ones keep the grid-sized buffer; the bits are the
    oracle's either way."""
    say("masked_select output memory", density)
    r = rng(31)
    shape = (1024, 2048)  # 8 MiB of x: the grid-sized buffer is 8 MiB
    x = r.standard_normal(shape, dtype=np.float32)
    m = (r.random(shape, dtype=np.float32) < density).astype(np.float32)
    dx, dm = hip.DeviceArray.from_numpy(x), hip.DeviceArray.from_numpy(m)
    hip.sync()
    base = hip.memory_stats()[0]
    got = hip.masked_select(dx, dm)
    held = hip.memory_stats()[0] - base
    bits_equal(got.numpy(), oracle.masked_select(x, m), f"masked_select density {density}")
    picks = 4 * got.size
    grid = 4 * x.size
    if exact:
        assert picks * 3 <= grid and held <= picks + (2 << 20), (held, picks)
    else:
        assert picks * 3 > grid and held >= grid, (held, grid)
    got.free()


def test_masked_select_strided_operands(hip, oracle, msel_path):
    """A transposed x and a broadcast column mask, through explicit strides."""
    say("masked_select strided")
    r = rng(5)
    base = r.standard_normal((300, 200), dtype=np.float32)
    x = base.T  # (200, 300) view
    m = (r.random((200, 1), dtype=np.float32) < 0.5).astype(np.float32)
    grid = (200, 300)
    d_base, d_m = hip.DeviceArray.from_numpy(base), hip.DeviceArray.from_numpy(m)
    out, cnt = ctypes.c_void_p(), ctypes.c_int64(0)
    rec = hip.masked_select_record(grid)
    hip.call("oxi_masked_select", d_base.ptr, hip._i64arr([1, 200]), d_m.ptr, hip._i64arr([1, 0]),
             hip._i64arr(grid), 2, ctypes.byref(out), ctypes.byref(cnt), rec.ptr)
    got = hip.DeviceArray.adopt(out.value, (cnt.value,))
    want = oracle.masked_select(np.ascontiguousarray(x), m)
    bits_equal(got.numpy(), want, "strided masked_select")
    g = r.standard_normal(want.size, dtype=np.float32)
    gx = hip.DeviceArray((200, 300))
    hip.call("oxi_masked_select_bwd", rec.ptr, hip._i64arr(grid), 2, hip.DeviceArray.from_numpy(g).ptr, g.size,
             gx.ptr, hip._i64arr([300, 1]), 200 * 300)
    bits_equal(gx.numpy(), oracle.masked_select_bwd((200, 300), m, g), "strided masked_select bwd")


def test_masked_select_bwd_checks(hip):
    """A count that differs from the record's raises the device guard
    (reported by the next sync) and reads no gradient beyond it; strides that
    do not describe x are refused before any launch."""
    x = hip.DeviceArray.from_numpy(np.ones((4,), np.float32))
    m = hip.DeviceArray.from_numpy(np.ones((4,), np.float32))
    rec = hip.masked_select_record((4,))
    picks = hip.masked_select(x, m, rec)
    assert picks.shape == (4,)
    g = hip.DeviceArray.from_numpy(np.ones((3,), np.float32))
    gx = hip.DeviceArray((4,))
    hip.call("oxi_masked_select_bwd", rec.ptr, hip._i64arr([4]), 1, g.ptr, 3, gx.ptr, hip._i64arr([1]), 4)
    with pytest.raises(RuntimeError, match="guard|out of range|index"):
        hip.sync()
    hip.sync()  # the flag is cleared once reported
    assert gx.numpy().tolist() == [1.0, 1.0, 1.0, 0.0]
    with pytest.raises(ValueError, match="do not describe"):
        hip.call("oxi_masked_select_bwd", rec.ptr, hip._i64arr([4]), 1, g.ptr, 4, gx.ptr, hip._i64arr([2]), 4)


# ---- python/tests/test_indexing_grad.py through oxitorch_amd -----------------------

@pytest.fixture(scope="module")
def ox(hip):
    import oxitorch_amd

    return oxitorch_amd


def _t(ox, arr, requires_grad=False):
    return ox.from_numpy(np.ascontiguousarray(arr, dtype=np.float32), requires_grad)


def test_scatter_grads_last_write_wins(ox):
    """test_indexing_grad.py:20-32."""
    base = _t(ox, [[10.0, 11.0], [20.0, 21.0], [30.0, 31.0]], True)
    vals = _t(ox, [[1.0, 2.0], [3.0, 4.0], [5.0, 6.0]], True)
    out = base.scatter([2, 0, 2], vals)
    out.sum().backward()
    np.testing.assert_array_equal(out.numpy(), [[3.0, 4.0], [20.0, 21.0], [5.0, 6.0]])
    np.testing.assert_array_equal(base.grad.numpy(), [[0.0, 0.0], [1.0, 1.0], [0.0, 0.0]])
    np.testing.assert_array_equal(vals.grad.numpy(), [[0.0, 0.0], [1.0, 1.0], [1.0, 1.0]])


def test_scatter_forward_matches_numpy(ox):
    """test_indexing_grad.py:35-42."""
    r = np.random.default_rng(7)
    a = r.standard_normal((5, 3)).astype(np.float32)
    vals = r.standard_normal((3, 3)).astype(np.float32)
    out = _t(ox, a, True).scatter([4, 1, 4], _t(ox, vals))
    want = a.copy()
    want[[4, 1, 4]] = vals
    np.testing.assert_array_equal(out.numpy(), want)


def test_masked_select_broadcast_accumulation(ox):
    """test_indexing_grad.py:45-54."""
    col = _t(ox, [[7.0], [9.0]], True)
    mask = _t(ox, [[1.0, 1.0, 0.0], [0.0, 1.0, 1.0]])
    picked = col.masked_select(mask)
    assert picked.numpy().shape == (4,)
    picked.backward(_t(ox, [1.0, 2.0, 3.0, 4.0]))
    np.testing.assert_array_equal(picked.numpy(), [7.0, 7.0, 9.0, 9.0])
    np.testing.assert_array_equal(col.grad.numpy(), [[3.0], [7.0]])


def test_masked_select_grad_matches_dense_multiply(ox):
    """test_indexing_grad.py:57-69."""
    r = np.random.default_rng(11)
    a = r.standard_normal((2, 3)).astype(np.float32)
    up = r.standard_normal((2, 3)).astype(np.float32)
    mask = (r.standard_normal((2, 3)) > 0).astype(np.float32)
    x = _t(ox, a, True)
    picked = x.masked_select(_t(ox, mask))
    picked.backward(_t(ox, up[mask > 0]))
    np.testing.assert_allclose(x.grad.numpy(), mask * up, rtol=1e-4, atol=1e-5)


def test_detached_scatter_still_works(ox):
    """test_indexing_grad.py:111-117."""
    out = _t(ox, np.ones((2, 2))).scatter([0], _t(ox, np.full((1, 2), -1.0)))
    np.testing.assert_array_equal(out.numpy(), [[-1.0, -1.0], [1.0, 1.0]])
    assert out.grad is None
    sel = _t(ox, [1.0, 2.0, 3.0]).masked_select(_t(ox, [0.0, 1.0, 1.0]))
    assert sel.numpy().tolist() == [2.0, 3.0] and not sel.requires_grad


def test_scatter_and_masked_select_errors(ox):
    """Argument checks of Tensor::scatter_dim0 / masked_select, before any
    device work, with the reference's messages."""
    base = _t(ox, np.zeros((3, 2)), True)
    with pytest.raises(RuntimeError, match="index 3 out of range for dim 0 of size 3"):
        base.scatter([3], _t(ox, np.zeros((1, 2))))
    with pytest.raises(ValueError, match=r"shape mismatch: \[1, 3\] vs \[1, 2\]"):
        base.scatter([0], _t(ox, np.zeros((1, 3))))
    with pytest.raises(ValueError):
        base.masked_select(_t(ox, np.ones((4,))))
    empty = _t(ox, np.zeros((0, 3))).masked_select(_t(ox, np.ones((0, 3))))
    assert empty.numpy().shape == (0,)
