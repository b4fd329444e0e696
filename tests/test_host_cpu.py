"""Host-side logic, no GPU: the C-ABI library loads and exports every symbol
include/oxihip.h declares; status codes map to the reference's exceptions;
shape algebra, views and argument validation of the host core behave as the
reference's (crates/oxi-tensor/src/{layout.rs,lib.rs}, crates/oxi-bindings)."""

import re
import subprocess
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]


def declared_symbols():
    text = (ROOT / "include" / "oxihip.h").read_text()
    return sorted(set(re.findall(r"^\s*(?:int|const char\*)\s+(oxi_[a-z0-9_]+)\s*\(", text, re.M)))


def test_liboxihip_exports_every_declared_symbol():
    from oxitorch_amd import capi

    names = declared_symbols()
    assert len(names) >= 40
    for n in names:
        assert hasattr(capi.lib, n), f"liboxihip.so does not export {n}"
    assert sorted(capi.DECLARED) == names, "capi signature table out of sync with include/oxihip.h"
    out = subprocess.run(["nm", "-D", "--defined-only", str(capi.LIB_PATH)], capture_output=True, text=True).stdout
    exported = set(re.findall(r" T (oxi_[a-z0-9_]+)", out))
    assert set(names) <= exported


def test_liboxihip_is_gfx950_only():
    from oxitorch_amd import capi

    out = subprocess.run(["strings", str(capi.LIB_PATH)], capture_output=True, text=True).stdout
    assert "gfx950" in out
    for other in ("gfx90a", "gfx942", "sm_"):
        assert f"amdgcn-amd-amdhsa--{other}" not in out


def test_no_device_is_an_error_not_a_fallback():
    from oxitorch_amd import capi

    if capi.device_count() > 0:
        pytest.skip("a HIP device is visible")
    with pytest.raises(RuntimeError, match="no HIP device"):
        capi.init(0)
    with pytest.raises(RuntimeError, match="no HIP device"):
        capi.DeviceArray((4,))


def test_argument_errors_map_to_value_error():
    import ctypes

    from oxitorch_amd import capi

    # validated before any device use
    with pytest.raises(ValueError, match="unknown reduction kind"):
        capi.call("oxi_reduce", 99, None, None, None, 1, 0, None)
    with pytest.raises(ValueError, match="negative size"):
        capi.call("oxi_rms_norm_fwd", None, None, None, None, -1, 4, 1e-6)
    with pytest.raises(ValueError, match="unknown VJP mode"):
        capi.call("oxi_layer_norm_bwd", None, None, None, None, None, None, None, None, 0, 4, 7)
    # element counts that would overflow the kernels' 64-bit index arithmetic
    with pytest.raises(ValueError, match="exceeds the kernel limits"):
        capi.call("oxi_index_select", None, 1 << 40, 1 << 20, 1 << 20, None, 4, None)
    with pytest.raises(ValueError, match="exceeds the kernel limits"):
        capi.call("oxi_index_select_bwd", None, 1, 1 << 30, 1 << 32, None, 4, None)
    with pytest.raises(ValueError, match="exceeds the kernel limits"):
        capi.call("oxi_softmax_fwd", None, None, 1 << 31, 1 << 30, 1)  # 2^61 elements
    big = capi._i64arr([1 << 31, 1 << 31])  # 2^62 elements
    st = capi._i64arr([0, 0])
    with pytest.raises(ValueError, match="exceeds the kernel limits"):
        capi.call("oxi_unary", 0, None, st, None, st, big, 2)
    with pytest.raises(ValueError, match="exceeds the kernel limits"):
        capi.call("oxi_reduce", 0, None, st, big, 2, 1, None)
    with pytest.raises(ValueError, match="exceeds the kernel limits"):
        capi.call("oxi_scatter_rows", None, 1 << 40, 1 << 30, None, 0, None, None)
    with pytest.raises(ValueError, match="grid too large"):
        capi.call("oxi_masked_select_record_bytes", big, 2, ctypes.byref(ctypes.c_int64()))
    with pytest.raises(ValueError, match="unknown activation"):
        capi.call("oxi_layer_norm_act_bwd", None, None, None, None, None, None, 7, None, None, None, None, 0, 4, 0)
    with pytest.raises(ValueError, match="unknown VJP mode"):
        capi.call("oxi_rms_norm_act_bwd", None, None, None, None, 2, None, None, None, 0, 4, 9)
    # rows that do not vectorize: the caller is told to run the two VJPs
    fake = 1 << 20
    with pytest.raises(NotImplementedError, match="do not vectorize"):
        capi.call("oxi_rms_norm_act_bwd", fake, None, fake, fake, 2, None, None, None, 1, 770, 0)
    with pytest.raises(NotImplementedError, match="do not vectorize"):
        capi.call("oxi_layer_norm_act_bwd", fake, None, None, fake, fake, fake + 4, 1, None, None, None, None, 1, 8, 0)
    # the leading-dim sum's output is written as float4s: an offset dx_sum is
    # refused before any launch (16 rows of 768 in (4, 4) positions)
    for off, ok in ((4, False), (8, False), (16, True)):
        args = (fake, None, fake, fake, 0, None, fake, None, fake + off, 4, 16, 768, 0)
        if ok:
            # past the checks, at initialisation; never on a machine with a
            # device, where the call would launch on the fake addresses
            if capi.device_count() == 0:
                with pytest.raises(RuntimeError, match="no HIP device"):
                    capi.call("oxi_rms_norm_bwd_lead_sum", *args)
        else:
            with pytest.raises(NotImplementedError, match="not 16-byte aligned"):
                capi.call("oxi_rms_norm_bwd_lead_sum", *args)
    with pytest.raises(NotImplementedError, match="not 16-byte aligned"):
        capi.call("oxi_layer_norm_bwd_lead_sum", fake, None, None, fake, fake, fake, 2, None, fake, None, None,
                  fake + 4, 4, 16, 768, 0)


def test_oracle_is_not_imported_by_the_product():
    for p in (ROOT / "oxitorch_amd").rglob("*.py"):
        text = p.read_text()
        assert "import oracle" not in text and "from oracle" not in text, p
    for p in (ROOT / "oxitorch_amd" / "csrc").rglob("*"):
        if p.is_file():
            assert "refcpu" not in p.read_text(errors="ignore"), p


# ---- host core (device="cpu" tensors only stage data) ---------------------------------

@pytest.fixture(scope="module")
def ox():
    import oxitorch_amd

    return oxitorch_amd


def cpu(ox, a):
    return ox.from_numpy(np.ascontiguousarray(a, dtype=np.float32), device="cpu")


def test_views_match_numpy(ox):
    """python/tests/test_smoke.py:124-149 (view part), on host-staged tensors."""
    a = np.random.default_rng(0).standard_normal((4, 6)).astype(np.float32)
    t = cpu(ox, a)
    np.testing.assert_array_equal(t.reshape([24]).numpy(), a.reshape(24))
    np.testing.assert_array_equal(t.reshape([-1, 8]).numpy(), a.reshape(-1, 8))
    np.testing.assert_array_equal(t.transpose().numpy(), a.T)
    np.testing.assert_array_equal(t.permute([1, 0]).numpy(), a.T)
    np.testing.assert_array_equal(t[2].numpy(), a[2])
    np.testing.assert_array_equal(t[-1].numpy(), a[-1])
    np.testing.assert_array_equal(t[1:3].numpy(), a[1:3])
    np.testing.assert_array_equal(t[::2].numpy(), a[::2])
    np.testing.assert_array_equal(t[1:].numpy(), a[1:])
    np.testing.assert_array_equal(t.select(1, 3).numpy(), a[:, 3])
    row = a[0].copy()
    np.testing.assert_array_equal(cpu(ox, row).reshape([1, 6]).broadcast_to([4, 6]).numpy(),
                                  np.broadcast_to(row, (4, 6)))
    assert t.is_contiguous() and not t.transpose().is_contiguous()
    assert t.permute([1, 0]).strides == [1, 6]


def test_shape_errors(ox):
    t = cpu(ox, np.zeros((2, 3)))
    with pytest.raises(ValueError, match="can only infer one dimension"):
        t.reshape([-1, -1])
    with pytest.raises(ValueError, match="cannot reshape 6 elements into shape"):
        t.reshape([4, 2])
    with pytest.raises(ValueError, match="permute expects 2 dims, got 3"):
        t.permute([0, 1, 2])
    with pytest.raises(ValueError, match="repeated dim"):
        t.permute([0, 0])
    with pytest.raises(ValueError, match="transpose\\(\\) expects a 2-D tensor"):
        cpu(ox, np.zeros(3)).transpose()
    with pytest.raises(ValueError, match="dim 5 out of range for 2-D tensor"):
        t.select(5, 0)
    with pytest.raises(RuntimeError, match="index 2 out of range for dim 0 of size 2"):
        t.select(0, 2)
    with pytest.raises(ValueError, match="shape mismatch"):
        t.broadcast_to([4, 3])
    with pytest.raises(NotImplementedError, match="negative slice steps"):
        t.narrow(0, 0, 2, -1)


def test_broadcast_errors_before_device(ox):
    """Broadcasting is validated before any device work (layout.rs:67-88 via error.rs:24-26)."""
    a = cpu(ox, np.zeros((2, 3)))
    b = cpu(ox, np.zeros((4,)))
    with pytest.raises(ValueError, match=r"shape mismatch: \[2, 3\] vs \[4\]"):
        a + b


def test_host_tensor_compute_is_refused(ox):
    a = cpu(ox, np.ones((2, 3)))
    with pytest.raises(NotImplementedError, match="HIP device"):
        a * 2.0
    with pytest.raises(NotImplementedError, match="HIP device"):
        a.sum(0)


def test_index_validation_before_device(ox):
    """Out-of-range ids raise the reference's OutOfBounds text (lib.rs:665-676)."""
    w = cpu(ox, np.zeros((3, 2)))
    with pytest.raises(RuntimeError, match="index 3 out of range for dim 0 of size 3"):
        w.index_select(0, [0, 3])
    with pytest.raises(RuntimeError, match="index -4 out of range for dim 0 of size 3"):
        w.index_select(0, [-4])


def test_cross_entropy_argument_checks(ox):
    """python/tests/test_nn.py:125-128 and numpy's indexing errors."""
    import oxitorch_amd.nn.functional as F

    logits = cpu(ox, np.zeros((2, 3)))
    with pytest.raises(ValueError, match="targets"):
        F.cross_entropy(logits, [0, 1, 2])
    with pytest.raises(IndexError, match="out of bounds for axis 1 with size 3"):
        F.cross_entropy(logits, [0, 3])
    # numpy's fancy indexing of the one-hot refuses float indices
    with pytest.raises(IndexError, match="only integers"):
        F.cross_entropy(logits, [0.0, 2.0])
    with pytest.raises(IndexError, match="must be of integer"):
        F.cross_entropy(logits, np.array([0.0, 2.0]))


def test_boundary_buffer_checks(ox):
    """buffer_to_f32 (bindings lib.rs:31-42)."""
    with pytest.raises(ValueError, match="only contiguous numpy arrays"):
        ox.from_numpy(np.zeros((4, 4), np.float32)[:, ::2], device="cpu")
    with pytest.raises(TypeError):
        ox.from_numpy(np.zeros(3, np.float64), device="cpu")
    t = ox.Tensor([1.0, 2.0, 3.0], device="cpu")
    assert t.shape == [3] and t.dtype == "float32" and t.device == "cpu"


def test_grad_mode_context_managers(ox):
    """python/oxitorch/__init__.py:46-75, crates/oxi-autograd/src/tests.rs:481-503."""
    assert ox.is_grad_enabled()
    with ox.no_grad():
        assert not ox.is_grad_enabled()
        with ox.enable_grad():
            assert ox.is_grad_enabled()
        assert not ox.is_grad_enabled()
    assert ox.is_grad_enabled()
    try:
        with ox.no_grad():
            raise KeyError("x")
    except KeyError:
        pass
    assert ox.is_grad_enabled()


def test_backward_error_paths(ox):
    """graph.rs:379-387: a root that does not require grad."""
    t = cpu(ox, np.ones(3))
    with pytest.raises(ValueError, match="does not require grad"):
        t.backward()


# ---- optimizers: argument checks and schedules (no device work) ----------------------

def test_optimizer_argument_errors():
    from oxitorch_amd import capi

    with pytest.raises(ValueError, match="nesterov momentum requires momentum > 0"):
        capi.call("oxi_sgd_step", None, None, None, None, 4, 0.1, 0.0, 1)
    with pytest.raises(ValueError, match="negative size"):
        capi.call("oxi_sgd_step", None, None, None, None, -1, 0.1, 0.0, 0)
    with pytest.raises(ValueError, match="step count must be >= 1"):
        capi.call("oxi_adamw_step", None, None, None, None, None, 4, 0.1, 0.9, 0.999, 1e-8, 0.0, 1, 0)
    with pytest.raises(ValueError, match="NULL tensor pointer"):
        capi.call("oxi_adamw_step", None, None, None, None, None, 4, 0.1, 0.9, 0.999, 1e-8, 0.0, 1, 1)
    # empty parameters are a no-op before any device use
    capi.call("oxi_adamw_step", None, None, None, None, None, 0, 0.1, 0.9, 0.999, 1e-8, 0.0, 1, 1)
    capi.call("oxi_sgd_step", None, None, None, None, 0, 0.1, 0.9, 1)


def test_native_optimizer_construction(ox):
    """RustSgd / RustAdamW constructors and lr property
    (crates/oxi-bindings/src/lib.rs:838-893)."""
    from oxitorch_amd import _native
    import oxitorch_amd.optim as op

    with pytest.raises(ValueError, match="nesterov momentum requires momentum > 0"):
        _native.RustSgd(0.1, 0.0, True)
    with pytest.raises(ValueError, match="nesterov momentum requires momentum > 0"):
        op.Sgd([], lr=0.1, nesterov=True)
    s = _native.RustSgd()
    assert s.lr == pytest.approx(0.01)
    s.lr = 0.25
    assert s.lr == 0.25
    a = _native.RustAdamW()
    assert a.lr == pytest.approx(1e-3)
    opt = op.AdamW([], lr=0.5)
    assert opt.lr == 0.5 and opt.weight_decay == 1e-2 and opt.betas == (0.9, 0.999)
    assert op.Adam([]).weight_decay == 0.0
    opt.step()  # an empty parameter list steps nothing
    with pytest.raises(TypeError, match="oxitorch.Tensor"):
        _native.RustAdamW().step([1.0])


def test_optimizer_refuses_host_tensors(ox):
    """Parameters staged on the host are not stepped on the CPU."""
    import oxitorch_amd.optim as op

    w = ox.from_numpy(np.ones(3, np.float32), True, device="cpu")
    w.grad = ox.from_numpy(np.ones(3, np.float32), device="cpu")
    with pytest.raises(NotImplementedError, match="on a host"):
        op.Sgd([w], lr=0.1).step()


def test_lr_schedules_refused():
    """The reference's schedule names (python/oxitorch/optim.py:104-226) exist
    and refuse to be made: they are host bookkeeping outside this build."""
    import oxitorch_amd.optim as op

    for name in ("StepLR", "CosineAnnealingLR", "LinearWarmup", "SequentialLR", "LambdaLR"):
        assert name in op.__all__
        with pytest.raises(NotImplementedError, match="outside this build"):
            getattr(op, name)(object(), 1)


def test_data_module_names():
    """Every public name of the reference's utils.data (data.py:31-40, 91)
    imports; the base classes subclass, the per-item pieces refuse."""
    import oxitorch_amd.utils.data as d

    for name in ("DataLoader", "Dataset", "IterableDataset", "RandomSampler", "SequentialSampler", "Subset",
                 "TensorDataset", "default_collate", "Sampler"):
        assert hasattr(d, name), name

    class Squares(d.Dataset):
        def __getitem__(self, i):
            return i * i

        def __len__(self):
            return 4

    assert len(Squares()) == 4 and Squares()[3] == 9
    assert issubclass(d.TensorDataset, d.Dataset) and issubclass(d.IterableDataset, d.Dataset)
    with pytest.raises(NotImplementedError):
        len(d.Dataset())
    with pytest.raises(NotImplementedError):
        iter(d.IterableDataset())
    for cls in (d.Subset, d.Sampler, d.SequentialSampler, d.RandomSampler):
        with pytest.raises(NotImplementedError, match="item by item"):
            cls(Squares())
    with pytest.raises(NotImplementedError, match="item by item"):
        d.default_collate([1, 2])
    with pytest.raises(NotImplementedError, match="Squares"):
        d.DataLoader(Squares(), batch_size=2)


def test_indexing_argument_checks_before_device(ox):
    """Tensor::scatter_dim0 / masked_select argument checks (lib.rs:895-942)
    run on the host with the reference's messages, before any device work."""
    base = cpu(ox, np.zeros((3, 2)))
    with pytest.raises(RuntimeError, match="index 3 out of range for dim 0 of size 3"):
        base.scatter([3], cpu(ox, np.zeros((1, 2))))
    with pytest.raises(ValueError, match=r"shape mismatch: \[1, 3\] vs \[1, 2\]"):
        base.scatter([0], cpu(ox, np.zeros((1, 3))))
    with pytest.raises(ValueError, match="at least a 1-D tensor"):
        ox.from_numpy(np.float32(1.0).reshape(()), device="cpu").scatter([], cpu(ox, np.zeros((0,))))
    with pytest.raises(ValueError, match="shape mismatch"):
        base.masked_select(cpu(ox, np.ones((4,))))
    with pytest.raises(NotImplementedError, match="on a host"):
        base.masked_select(cpu(ox, np.ones((3, 2))))
    from oxitorch_amd import capi

    with pytest.raises(ValueError, match="negative size"):
        capi.call("oxi_scatter_rows", None, -1, 4, None, 0, None, None)
    with pytest.raises(ValueError, match="negative size"):
        capi.call("oxi_masked_select_bwd", None, None, 0, None, -1, None, None, 0)
    nb = capi.c_i64(0)
    capi.call("oxi_masked_select_record_bytes", capi._i64arr([16384, 4096]), 2, capi.ctypes.byref(nb))
    assert nb.value == 8 * (16384 + 1) + 16384 * 4096 // 8  # 4096-element tiles' offsets + one bit per element


# ---- input pipeline host logic (crates/oxi-data/src/{rng,batch}.rs) -------------------

def test_mt19937_permutation_matches_numpy(ox):
    """rng.rs:131-141 (the recorded NumPy stream) and NumPy itself for several
    seeds and sizes, including the loader's 32-bit seed truncation range."""
    from oxitorch_amd import _native

    assert _native._mt19937_permutation(7, 10) == [8, 5, 0, 2, 1, 9, 7, 3, 6, 4]
    for seed in (0, 1, 42, 2**31 + 5, 2**32 - 1):
        for n in (1, 2, 17, 1000, 65537):
            want = np.random.RandomState(seed).permutation(n).tolist()
            assert _native._mt19937_permutation(seed, n) == want, (seed, n)


def test_epoch_plan(ox):
    """batch.rs:430-460: sequential chunks with a remainder; drop_last drops
    only a short tail and keeps a lone short batch; batch size 0 rejected."""
    from oxitorch_amd import _native

    assert _native._epoch_plan(12, 5, False) == [(0, 5), (5, 5), (10, 2)]
    assert _native._epoch_plan(12, 5, True) == [(0, 5), (5, 5)]
    assert _native._epoch_plan(3, 5, True) == [(0, 3)]
    assert _native._epoch_plan(10, 5, True) == [(0, 5), (5, 5)]
    with pytest.raises(ValueError, match="batch_size must be >= 1"):
        _native._epoch_plan(4, 0, False)


def test_loader_argument_checks(ox):
    """bindings data.rs:149-176, before any device work."""
    from oxitorch_amd import _native

    with pytest.raises(ValueError, match="at least one tensor column"):
        _native.DataLoader([])
    with pytest.raises(ValueError, match="dataset is empty"):
        _native.DataLoader([cpu(ox, np.zeros((0, 2)))])
    with pytest.raises(ValueError, match="batch_size must be >= 1"):
        _native.DataLoader([cpu(ox, np.zeros((3, 2)))], batch_size=0)
    with pytest.raises(ValueError, match="column 1 has 2 rows, expected 3"):
        _native.DataLoader([cpu(ox, np.zeros((3, 2))), cpu(ox, np.zeros((2,)))])
    with pytest.raises(NotImplementedError, match="transforms"):
        _native.DataLoader([cpu(ox, np.zeros((3, 2)))], transforms=object())
    from oxitorch_amd.utils.data import DataLoader, TensorDataset

    with pytest.raises(ValueError, match="batch_size must be >= 1"):
        DataLoader(TensorDataset(cpu(ox, np.zeros((3, 2)))), batch_size=0)


def test_out_of_scope_names_raise_not_implemented():
    """The reference's GEMM, convolution, pooling and dropout names
    (nn/functional.py:23-55,104-181,255-268, nn/layers.py:20-92,134-164)
    exist and say they are outside this build when called."""
    import oxitorch_amd.nn as nn
    import oxitorch_amd.nn.functional as F

    for fn in (F.linear, F.bmm, F.conv2d, F.max_pool2d, F.dropout, nn.linear, nn.bmm, nn.conv2d, nn.max_pool2d,
               nn.dropout):
        with pytest.raises(NotImplementedError, match="outside this build's device hot path"):
            fn(None)
    for layer in (nn.Linear, nn.Conv2d, nn.MaxPool2d, nn.Dropout):
        with pytest.raises(NotImplementedError, match="outside this build's device hot path"):
            layer(4, 4)
    assert callable(nn.LeakyReLU)


def test_device_strings(ox):
    """A device is a family and an index (crates/oxi-core/src/lib.rs:139-146):
    "cpu", "hip"/"cuda" or "hip:N"/"cuda:N"; anything else is a ValueError
    before any device use."""
    a = np.zeros(3, np.float32)
    for bad in ("tpu", "hip:", "hip:x", "hip:-1", "cuda:1.5", "hip:0:0"):
        with pytest.raises(ValueError, match="device"):
            ox.from_numpy(a, device=bad)
    assert ox.from_numpy(a, device="cpu").device == "cpu"


def test_hip_device_env_is_checked():
    """OXI_HIP_DEVICE names the device an implicit initialisation binds; a
    value that is not an index is refused (in a child process: the variable is
    read when the library first binds a device)."""
    import os
    import subprocess
    import sys

    code = ("import ctypes, sys\n"
            "from oxitorch_amd import capi\n"
            "d = ctypes.c_int(-7)\n"
            "try:\n"
            "    capi.call('oxi_hip_default_device', ctypes.byref(d))\n"
            "except ValueError as e:\n"
            "    print('ValueError', e)\n"
            "else:\n"
            "    print('device', d.value)\n")
    env = dict(os.environ, PYTHONPATH=str(ROOT))
    for val, want in (("abc", "ValueError"), ("-1", "ValueError"), ("3", "device 3"), ("", "device 0")):
        env["OXI_HIP_DEVICE"] = val
        out = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True, timeout=120)
        assert want in out.stdout, (val, out.stdout, out.stderr)
        if want == "ValueError":
            assert "is not a device index" in out.stdout
