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
    from oxitorch_amd import capi

    # validated before any device use
    with pytest.raises(ValueError, match="unknown reduction kind"):
        capi.call("oxi_reduce", 99, None, None, None, 1, 0, None)
    with pytest.raises(ValueError, match="negative size"):
        capi.call("oxi_rms_norm_fwd", None, None, None, None, -1, 4, 1e-6)
    with pytest.raises(ValueError, match="unknown VJP mode"):
        capi.call("oxi_layer_norm_bwd", None, None, None, None, None, None, None, None, 0, 4, 7)


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
