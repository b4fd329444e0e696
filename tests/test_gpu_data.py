"""The input pipeline on the device: staged transfers (oxi_hip_upload /
download / h2d_async) bit-exact round trips, and the tensor-column loader,
whose batches must equal NumPy's gather of the columns in the reference's
epoch order (RandomState(seed + epoch).permutation, crates/oxi-data); then
the reference's own loader tests (python/tests/test_data.py) through
oxitorch_amd.utils.data."""

import ctypes
import sys

import numpy as np
import pytest

from conftest import rng

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def oracle():
    from oracle import ref

    return ref


def say(*a):
    print("[case]", *a, flush=True)
    sys.stdout.flush()


# ---- staged transfers ----------------------------------------------------------------

@pytest.mark.parametrize("nbytes", [4, 100, 4096, 1 << 20, 40 << 20, 100 << 20])
def test_upload_download_round_trip(hip, nbytes):
    say("upload/download", nbytes)
    r = rng(nbytes % 1000)
    a = r.integers(0, 256, nbytes, dtype=np.uint8)
    d = hip.DeviceArray((nbytes,), np.uint8)
    hip.call("oxi_hip_upload", d.ptr, a.ctypes.data, nbytes)
    a_copy = a.copy()
    a[:] = 0  # the source may be reused as soon as the call returns
    back = np.empty(nbytes, np.uint8)
    hip.call("oxi_hip_download", back.ctypes.data, d.ptr, nbytes)
    assert np.array_equal(back, a_copy)
    assert np.array_equal(d.numpy(), a_copy)  # the waiting d2h path agrees


def test_many_small_uploads_wrap_the_ring(hip):
    """2048 uploads of 64 KiB (128 MiB through a 64 MiB ring) queued without
    waiting, each into its own device slot, then checked at once."""
    say("ring wrap")
    n, sz = 2048, 64 << 10
    dev = hip.DeviceArray((n * sz,), np.uint8)
    want = np.empty((n, sz), np.uint8)
    buf = np.empty(sz, np.uint8)
    for i in range(n):
        buf[:] = (i * 7 + np.arange(sz)) % 251
        want[i] = buf
        hip.call("oxi_hip_upload", dev.ptr + i * sz, buf.ctypes.data, sz)
    assert np.array_equal(dev.numpy().reshape(n, sz), want)


@pytest.mark.parametrize("offset", [0, 1, 4, 8, 12, 15])
def test_small_uploads_any_alignment(hip, offset):
    """Uploads up to 1 MiB are copied by a kernel: destinations at every
    offset mod 16, sizes around the 16-byte vector width and the 1 MiB limit,
    interleaved with DMA uploads, and the bytes either side left alone."""
    say("small uploads at offset", offset)
    sizes = [1, 3, 15, 16, 17, 255, 4096 + 5, (1 << 20) - 1, 1 << 20, (1 << 20) + 1, 3 << 20]
    total = sum(sizes) + 64 * len(sizes) + 64
    dev = hip.DeviceArray((total,), np.uint8)
    fill = np.full(total, 0xA5, np.uint8)
    hip.call("oxi_hip_upload", dev.ptr, fill.ctypes.data, total)
    want = fill.copy()
    r = rng(offset)
    at = offset
    for sz in sizes:
        a = r.integers(0, 256, sz, dtype=np.uint8)
        hip.call("oxi_hip_upload", dev.ptr + at, a.ctypes.data, sz)
        want[at:at + sz] = a
        a[:] = 0
        at += sz + 64
    assert np.array_equal(dev.numpy(), want)


def test_pinned_async_copy(hip):
    say("pinned h2d_async")
    nbytes = 8 << 20
    p = ctypes.c_void_p()
    hip.call("oxi_hip_host_alloc", nbytes, ctypes.byref(p))
    try:
        host = np.ctypeslib.as_array((ctypes.c_uint8 * nbytes).from_address(p.value))
        host[:] = np.arange(nbytes) % 253
        d = hip.DeviceArray((nbytes,), np.uint8)
        hip.call("oxi_hip_memcpy_h2d_async", d.ptr, p.value, nbytes)
        hip.sync()
        assert np.array_equal(d.numpy(), np.arange(nbytes) % 253)
    finally:
        hip.call("oxi_hip_host_free", p.value)


# ---- the device loader -----------------------------------------------------------------

@pytest.fixture(scope="module")
def ox(hip):
    import oxitorch_amd

    return oxitorch_amd


def _t(ox, arr, requires_grad=False):
    return ox.from_numpy(np.ascontiguousarray(arr, dtype=np.float32), requires_grad)


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.mark.parametrize("n,bs,drop,workers", [(1000, 64, False, 0), (1000, 64, True, 0), (257, 300, True, 0),
                                               (4096, 1024, False, 0), (1000, 64, False, 3), (4096, 1024, True, 8)])
def test_device_loader_matches_numpy_gather(ox, n, bs, drop, workers):
    """Five epochs: each batch of each column equals the NumPy gather of the
    epoch's RandomState(seed + epoch) order, bit for bit, however many epochs'
    orders the host threads compute ahead."""
    from oxitorch_amd import _native

    say("device loader", n, bs, drop, workers)
    r = rng(n + bs)
    x = r.standard_normal((n, 3, 4), dtype=np.float32)
    y = np.arange(n, dtype=np.float32)
    loader = _native.DataLoader([_t(ox, x), _t(ox, y)], batch_size=bs, shuffle=True, drop_last=drop, seed=1234,
                                num_workers=workers)
    assert loader.n == n and loader.batch_size == bs
    for epoch in range(5):
        order = np.random.RandomState(1234 + epoch).permutation(n)
        plan = _native._epoch_plan(n, bs, drop)
        got = list(iter(loader))
        assert len(got) == len(plan)
        for (start, length), (bx, by) in zip(plan, got):
            rows = order[start:start + length]
            assert np.array_equal(_bits(bx.numpy()), _bits(x[rows]))
            assert np.array_equal(_bits(by.numpy()), _bits(y[rows]))
            assert not bx.requires_grad and bx.device.startswith("hip")


def test_batch_gather_all_column_kinds(hip, oracle):
    """One launch per 8 columns: float4 rows, unaligned scalar rows, short
    rows and 1-D columns, 11 columns in all; negative ids wrap; every column
    equals the oracle's index_select bit for bit."""
    say("batch_gather")
    r = rng(91)
    n_rows = 3001
    shapes = [(n_rows, 784), (n_rows,), (n_rows, 66), (n_rows, 3, 4), (n_rows, 64), (n_rows, 1), (n_rows, 130),
              (n_rows, 7), (n_rows, 256), (n_rows,), (n_rows, 2, 40)]
    cols = [r.standard_normal(sh, dtype=np.float32) for sh in shapes]
    ids = r.integers(-n_rows, n_rows, 1000).astype(np.int64)
    d_cols = [hip.DeviceArray.from_numpy(c) for c in cols]
    outs = hip.batch_gather(d_cols, hip.DeviceArray.from_numpy(ids))
    hip.sync()
    for c, o in zip(cols, outs):
        want = oracle.index_select(c.reshape(n_rows, -1), 0, ids).reshape((len(ids),) + c.shape[1:])
        assert np.array_equal(_bits(o.numpy()), _bits(want)), c.shape
    # an out-of-range id writes zeros and raises the guard
    bad = ids.copy()
    bad[5] = n_rows
    outs = hip.batch_gather(d_cols[:2], hip.DeviceArray.from_numpy(bad))
    with pytest.raises(RuntimeError, match="guard|out of range|index"):
        hip.sync()
    hip.sync()
    assert not outs[0].numpy()[5].any() and outs[1].numpy()[5] == 0.0
    with pytest.raises(ValueError, match="NULL"):
        hip.call("oxi_batch_gather", None, 2, n_rows, None, 4)


def test_device_loader_sequential_and_unseeded_shuffle(ox):
    """Without shuffle, or shuffled without a seed, the native loader walks
    rows in order (bindings data.rs:216-227)."""
    from oxitorch_amd import _native

    x = np.arange(10, dtype=np.float32)
    for kw in ({}, {"shuffle": True}):
        got = [b[0].numpy().tolist() for b in _native.DataLoader([_t(ox, x)], batch_size=4, **kw)]
        assert got == [[0, 1, 2, 3], [4, 5, 6, 7], [8, 9]]


def test_host_columns_are_uploaded_once(ox):
    from oxitorch_amd import _native

    x = np.arange(12, dtype=np.float32).reshape(6, 2)
    host = ox.from_numpy(x, device="cpu")
    batches = list(_native.DataLoader([host], batch_size=4))
    assert batches[0][0].device.startswith("hip")
    assert np.array_equal(np.concatenate([b[0].numpy() for b in batches]), x)


# ---- python/tests/test_data.py through oxitorch_amd.utils.data --------------------------

@pytest.fixture()
def tiny(ox):
    from oxitorch_amd.utils.data import TensorDataset

    x = ox.from_numpy(np.arange(24, dtype=np.float32).reshape(12, 2))
    y = ox.from_numpy(np.arange(12, dtype=np.float32))
    return TensorDataset(x, y)


def _labels(loader):
    return [b[1].numpy().tolist() for b in loader]


def test_sequential_batches_and_len(tiny):
    """test_data.py:32-51."""
    from oxitorch_amd.utils.data import DataLoader

    assert _labels(DataLoader(tiny, batch_size=5)) == [[0, 1, 2, 3, 4], [5, 6, 7, 8, 9], [10, 11]]
    assert len(DataLoader(tiny, batch_size=5)) == 3
    assert len(DataLoader(tiny, batch_size=5, drop_last=True)) == 2
    assert len(DataLoader(tiny, batch_size=12)) == 1
    assert _labels(DataLoader(tiny, batch_size=5, drop_last=True)) == [[0, 1, 2, 3, 4], [5, 6, 7, 8, 9]]
    assert len(_labels(DataLoader(tiny, batch_size=1))) == 12
    assert _labels(DataLoader(tiny, batch_size=12)) == [list(range(12))]


def test_columns_keep_trailing_dims(ox):
    """test_data.py:53-58."""
    from oxitorch_amd.utils.data import DataLoader, TensorDataset

    imgs = ox.from_numpy(np.arange(24, dtype=np.float32).reshape(6, 1, 2, 2))
    batch = next(iter(DataLoader(TensorDataset(imgs), batch_size=6)))
    assert tuple(batch[0].shape) == (6, 1, 2, 2)


@pytest.mark.parametrize("workers", [0, 1, 4])
def test_worker_parity_with_inline_path(tiny, workers):
    """test_data.py:63-67."""
    from oxitorch_amd.utils.data import DataLoader

    assert _labels(DataLoader(tiny, batch_size=3, num_workers=workers)) == _labels(DataLoader(tiny, batch_size=3))


def test_shuffle_epochs_differ_but_are_reproducible(tiny):
    """test_data.py:70-94, and the order is NumPy's RandomState(seed + epoch)."""
    from oxitorch_amd.utils.data import DataLoader

    shuffled = _labels(DataLoader(tiny, batch_size=3, shuffle=True, seed=1, num_workers=2))
    assert shuffled != _labels(DataLoader(tiny, batch_size=3))
    assert sorted(x for b in shuffled for x in b) == list(range(12))
    loader = DataLoader(tiny, batch_size=4, shuffle=True, seed=42, num_workers=2)
    e0, e1 = _labels(loader), _labels(loader)
    assert e0 != e1
    assert _labels(DataLoader(tiny, batch_size=4, shuffle=True, seed=42, num_workers=2)) == e0
    flat = [x for b in e1 for x in b]
    assert flat == np.random.RandomState(43).permutation(12).astype(float).tolist()
    for workers in (2, 3):
        seen = [x for b in DataLoader(tiny, batch_size=4, shuffle=True, seed=7, num_workers=workers) for x in
                b[1].numpy().tolist()]
        assert sorted(seen) == list(range(12))


def test_batch_tensors_are_leaf_constants_and_empty_rejected(ox, tiny):
    """test_data.py:97-108."""
    from oxitorch_amd import _native
    from oxitorch_amd.utils.data import DataLoader

    batch = next(iter(DataLoader(tiny, batch_size=4, num_workers=2)))
    assert batch[0].requires_grad is False and batch[1].requires_grad is False
    with pytest.raises(Exception):
        _native.DataLoader([ox.from_numpy(np.zeros((0, 2), dtype=np.float32))])


def test_per_item_paths_are_refused(ox, tiny):
    """The reference's per-item path (python/oxitorch/utils/data.py:112-170:
    map-style datasets fetched item by item, samplers, custom collation) is
    not part of the device build: it is refused with a message, not run on
    the host."""
    from oxitorch_amd.utils.data import DataLoader

    class NumpyDS:
        def __len__(self):
            return 7

        def __getitem__(self, i):
            return np.full((3,), float(i), dtype=np.float32), float(i)

    with pytest.raises(NotImplementedError, match="TensorDataset"):
        DataLoader(NumpyDS(), batch_size=4)
    for kw in ({"sampler": [0, 1]}, {"batch_sampler": [[0, 1]]}, {"collate_fn": list}):
        with pytest.raises(NotImplementedError, match="device"):
            DataLoader(tiny, batch_size=2, **kw)
    with pytest.raises(ValueError, match="batch_size"):
        DataLoader(tiny, batch_size=0)


def test_training_through_the_loader(ox):
    """test_data.py:294-335 without a GEMM: an embedding table fitted by AdamW
    to targets streamed by the device loader; a seeded run is reproducible."""
    import oxitorch_amd.nn as nn
    import oxitorch_amd.nn.functional as F
    import oxitorch_amd.optim as op
    from oxitorch_amd.utils.data import DataLoader, TensorDataset

    r = rng(9)
    ids = r.integers(0, 32, 512).astype(np.float32)
    table = r.standard_normal((32, 8)).astype(np.float32)
    tgt = (table[ids.astype(np.int64)] + 0.05 * r.standard_normal((512, 8))).astype(np.float32)

    def run():
        emb = nn.Embedding(32, 8, seed=0)
        opt = op.AdamW(emb.parameters(), lr=0.05)
        loader = DataLoader(TensorDataset(ox.from_numpy(ids), ox.from_numpy(tgt)), batch_size=64, shuffle=True,
                            seed=11)
        losses = []
        for _ in range(6):
            for bi, bt in loader:
                opt.zero_grad()
                loss = F.mse_loss(emb(bi.numpy().astype(np.int64).tolist()), bt)
                loss.backward()
                opt.step()
                losses.append(float(loss.numpy()))
        return losses, emb.weight.tensor.numpy()

    l1, w1 = run()
    l2, w2 = run()
    assert l1[-1] < 0.2 * l1[0]
    assert l1 == l2 and np.array_equal(w1, w2)
