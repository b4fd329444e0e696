"""The reference tensor engine's unit tests (crates/oxi-tensor/src/tests.rs),
restated through the Python surface they back (the PyTensor methods of
crates/oxi-bindings/src/lib.rs:454-742) with every op on the device.
Matrix products (SGEMM is outside this build) are left out."""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ox(hip):
    import oxitorch_amd

    return oxitorch_amd


def _t(ox, arr, shape=None):
    a = np.asarray(arr, dtype=np.float32)
    if shape is not None:
        a = a.reshape(shape)
    return ox.from_numpy(np.ascontiguousarray(a))


def _v(t):
    return np.asarray(t.numpy(), dtype=np.float32).ravel().tolist()


# ---- broadcasting and the registries (tests.rs:72-164) ---------------------------------

def test_add_broadcasts_row_vector(ox):
    a = _t(ox, [1, 2, 3, 4, 5, 6], (2, 3))
    row = _t(ox, [10, 20, 30], (3,))
    assert _v(a + row) == [11, 22, 33, 14, 25, 36]


def test_add_broadcasts_column_vector_and_scalar(ox):
    a = _t(ox, [1, 2, 3, 4, 5, 6], (2, 3))
    col = _t(ox, [100, 200], (2, 1))
    assert _v(a + col) == [101, 102, 103, 204, 205, 206]
    s = ox.full([], 1.0)
    assert _v(a + s) == [2, 3, 4, 5, 6, 7]
    assert tuple((s + a).shape) == (2, 3), "commutes"


def test_add_broadcast_incompatible_shapes_error(ox):
    with pytest.raises(ValueError, match="shape mismatch"):
        ox.zeros([2, 3]) + ox.zeros([4, 3])


def test_binary_ops(ox):
    a, b = _t(ox, [8, 9]), _t(ox, [2, 3])
    assert _v(a - b) == [6, 6]
    assert _v(a * b) == [16, 27]
    assert _v(a / b) == [4, 3]
    assert _v(a ** b) == [64, 729]


def test_comparison_ops_produce_0_or_1(ox):
    a, b = _t(ox, [1, 2, 3]), _t(ox, [2, 2, 1])
    assert _v(a < b) == [1, 0, 0]
    assert _v(a <= b) == [1, 1, 0]
    assert _v(a == b) == [0, 1, 0]
    assert _v(a != b) == [1, 0, 1]
    assert _v(a > b) == [0, 0, 1]
    assert _v(a >= b) == [0, 1, 1]


def test_unary_ops_fast_and_strided_paths_agree(ox):
    base = _t(ox, range(6), (2, 3))
    t = base.transpose()
    assert not t.is_contiguous()
    for name in ["neg", "abs", "sqrt", "exp", "relu", "sigmoid", "square"]:
        fast = base.apply(name)
        slow = t.contiguous().transpose().apply(name)
        assert _v(fast) == _v(slow), f"unary {name} disagrees between contiguous and strided paths"


def test_unknown_unary_name_rejected(ox):
    with pytest.raises(ValueError):
        _t(ox, [1.0]).apply("frob")


def test_scalar_helpers(ox):
    a = _t(ox, [1, 2])
    assert _v(a + 10.0) == [11, 12]
    assert _v(a * 3.0) == [3, 6]


# ---- reductions (tests.rs:168-225) ----------------------------------------------------------

def test_reduce_last_dim_rows(ox):
    a = _t(ox, [1, 2, 3, 10, 20, 30], (2, 3))
    s = a.sum(-1)
    assert tuple(s.shape) == (2,) and _v(s) == [6, 60]
    m = a.max(-1, keepdim=True)
    assert tuple(m.shape) == (2, 1) and _v(m) == [3, 30]


def test_reduce_inner_dim_columns(ox):
    s = _t(ox, [1, 2, 3, 4, 5, 6], (3, 2)).sum(0)
    assert tuple(s.shape) == (2,) and _v(s) == [9, 12]


def test_reduce_argmax_argmin_first_tie_and_negative(ox):
    a = _t(ox, [5, 7, 7, 1, 9, 2], (2, 3))
    assert _v(a.argmax(-1)) == [1, 1]
    assert _v(a.argmin(1)) == [0, 0]


def test_reduce_3d_middle_dim(ox):
    s = _t(ox, range(1, 9), (2, 2, 2)).sum(1)
    assert tuple(s.shape) == (2, 2) and _v(s) == [4, 6, 12, 14]


def test_reduce_mean_norm_and_all(ox):
    a = _t(ox, [1, 2, 3, 4], (2, 2))
    assert _v(a.mean()) == [2.5]
    assert _v(a.sum()) == [10.0]
    n = _v(a.norm(-1))
    assert abs(n[0] - 5 ** 0.5) < 1e-6 and abs(n[1] - 5.0) < 1e-6


def test_reduce_errors(ox):
    e = ox.zeros([0, 3])
    with pytest.raises(ValueError):
        e.max(0)
    assert _v(e.sum(0)) == [0, 0, 0]  # sum of empty = 0
    # normalize_dim: InvalidArgument (layout.rs:162-176) -> ValueError
    with pytest.raises(ValueError, match="dim 5 out of range for 2-D tensor"):
        ox.zeros([2, 2]).sum(5)


# ---- views (tests.rs:229-336) ----------------------------------------------------------------

def test_narrow_with_step_and_negatives(ox):
    base = _t(ox, range(1, 7))
    assert _v(base.narrow(0, 0, 6, 2)) == [1, 3, 5]
    assert _v(base.narrow(0, -3, 6, 1)) == [4, 5, 6]
    # a step <= 0 is NotImplemented in the reference (layout.rs:129-133)
    with pytest.raises(NotImplementedError, match="negative slice steps"):
        base.narrow(0, 0, 6, 0)


def test_views_share_values(ox):
    base = _t(ox, [1, 2, 3, 4])
    v = base.narrow(0, 1, 3, 1)
    assert tuple(v.shape) == (2,) and _v(v) == [2, 3]


def test_select_drops_dim(ox):
    base = _t(ox, [1, 2, 3, 4, 5, 6], (2, 3))
    r1 = base.select(0, 1)
    assert tuple(r1.shape) == (3,) and _v(r1) == [4, 5, 6]
    assert _v(base.select(1, -2)) == [2, 5]
    # OutOfBounds (lib.rs:645-650) -> RuntimeError
    with pytest.raises(RuntimeError, match="index 2 out of range for dim 0 of size 2"):
        base.select(0, 2)


def test_reshape_views_and_copies(ox):
    base = _t(ox, range(1, 7), (2, 3))
    assert _v(base.reshape([3, 2])) == _v(base)
    assert tuple(base.reshape([-1]).shape) == (6,)
    assert tuple(base.reshape([6, -1]).shape) == (6, 1)
    with pytest.raises(ValueError):
        base.reshape([])  # N > 1 elements to [] is an error
    assert ox.full([], 7.0).reshape([]).numel() == 1
    with pytest.raises(ValueError):
        base.reshape([4, 2])
    with pytest.raises(ValueError):
        base.reshape([-1, -1])
    t = base.transpose()  # (3, 2), non-contiguous: reshape copies
    assert _v(t.reshape([6])) == _v(t)


def test_permute_and_transpose_are_views(ox):
    base = _t(ox, range(24), (2, 3, 4))
    p = base.permute([2, 0, 1])
    assert tuple(p.shape) == (4, 2, 3) and not p.is_contiguous()
    pv = _v(p)
    for i in range(4):
        for j in range(2):
            for k in range(3):
                assert pv[i * 6 + j * 3 + k] == j * 12 + k * 4 + i
    with pytest.raises(ValueError):
        base.permute([0, 0, 1])
    with pytest.raises(ValueError):
        base.permute([0, 1])
    assert _v(_t(ox, [1, 2, 3, 4], (2, 2)).transpose()) == [1, 3, 2, 4]
    with pytest.raises(ValueError):
        ox.zeros([2, 2, 2]).transpose()


def test_broadcast_to_zero_strides(ox):
    row = _t(ox, [1, 2, 3], (1, 3))
    big = row.broadcast_to([2, 3])
    assert tuple(big.shape) == (2, 3) and _v(big) == [1, 2, 3, 1, 2, 3]
    assert row.broadcast_to([4, 3]).numel() == 12
    with pytest.raises(ValueError):
        row.broadcast_to([2, 4])


def test_contiguous_materializes(ox):
    base = _t(ox, range(1, 7), (2, 3))
    t = base.transpose()
    c = t.contiguous()
    assert c.is_contiguous() and _v(c) == _v(t)
    assert base.contiguous().is_contiguous()


# ---- fancy indexing (tests.rs:340-405) --------------------------------------------------------

def test_index_select_rows_and_negative(ox):
    base = _t(ox, [1, 2, 3, 4, 5, 6], (3, 2))
    picked = base.index_select(0, [2, 0])
    assert tuple(picked.shape) == (2, 2) and _v(picked) == [5, 6, 1, 2]
    assert _v(base.index_select(0, [-1])) == [5, 6]
    with pytest.raises(RuntimeError, match="out of range"):
        base.index_select(0, [3])


def test_gather_dim0(ox):
    base = _t(ox, range(1, 7), (2, 3))
    rows = base.gather([1, 1, 0])
    assert tuple(rows.shape) == (3, 3) and _v(rows) == [4, 5, 6, 4, 5, 6, 1, 2, 3]
    with pytest.raises(RuntimeError, match="out of range"):
        base.gather([2])


def test_scatter_dim0_roundtrip_with_gather(ox):
    base = _t(ox, [1, 2, 3, 4], (2, 2))
    vals = _t(ox, [9, 8], (1, 2))
    out = base.scatter([1], vals)
    assert _v(out) == [1, 2, 9, 8]
    assert _v(out.gather([1])) == [9, 8]
    with pytest.raises(RuntimeError, match="out of range"):
        base.scatter([5], vals)
    with pytest.raises(ValueError):
        base.scatter([0], ox.zeros([2, 2]))


def test_masked_select_basic_and_broadcast(ox):
    base = _t(ox, [1, 2, 3, 4, 5, 6], (2, 3))
    mask = _t(ox, [1, 0, 1, 0, 1, 0], (2, 3))
    assert _v(base.masked_select(mask)) == [1, 3, 5]
    row_mask = _t(ox, [1, 0, 0], (3,))
    assert _v(base.masked_select(row_mask)) == [1, 4]


def test_scalar_tensors_have_zero_dims(ox):
    s = ox.full([], 3.5)
    assert tuple(s.shape) == () and s.numel() == 1 and float(s) == 3.5
    assert _v(s * s) == [12.25]
    assert _v(s.apply("neg")) == [-3.5]
