"""Device selection on one GPU: the reference's Device is a family and an
index (crates/oxi-core/src/lib.rs:139-146) and `device_count()` reports the
devices (bindings lib.rs:781-785). The library runs one device per process:
"hip:N" / "cuda:N" or OXI_HIP_DEVICE=N picks N at the first device use; an
index past the visible devices is a ValueError."""

import os
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parents[1]


def say(*a):
    print("[case]", *a, flush=True)


@pytest.fixture(scope="module")
def ox(hip):
    import oxitorch_amd

    return oxitorch_amd


def test_explicit_device_zero(ox):
    from oxitorch_amd import _native
    say("device hip:0 / cuda:0")
    a = np.arange(6, dtype=np.float32).reshape(2, 3)
    for name in ("hip:0", "cuda:0", "hip", "cuda"):
        t = ox.from_numpy(a, device=name)
        assert t.device == "hip:0", (name, t.device)
        np.testing.assert_array_equal((t * 2.0).numpy(), a * 2)
    assert _native.current_device() == 0
    assert ox.device_count() >= 1


def test_device_index_out_of_range(ox):
    from oxitorch_amd import _native
    say("device index out of range")
    n = _native.device_count()
    a = np.zeros(4, np.float32)
    with pytest.raises(ValueError, match="out of range|one device per process"):
        ox.from_numpy(a, device=f"hip:{n}")
    with pytest.raises(ValueError, match="out of range|one device per process"):
        ox.from_numpy(a, True, device=f"cuda:{n + 3}")
    t = ox.from_numpy(a, device="hip:0")  # the process stays on device 0
    assert t.device == "hip:0"


def _child(env_val, code):
    env = dict(os.environ, PYTHONPATH=str(ROOT))
    env["OXI_HIP_DEVICE"] = env_val
    return subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True, timeout=240)


def test_hip_device_env_binds_the_first_use(ox):
    """OXI_HIP_DEVICE=0 in a fresh process binds device 0 at the first
    device use; OXI_HIP_DEVICE=<count> fails there with the range error."""
    from oxitorch_amd import _native
    say("OXI_HIP_DEVICE in child processes")
    n = _native.device_count()
    code = ("import numpy as np, oxitorch_amd as ox\n"
            "from oxitorch_amd import _native\n"
            "try:\n"
            "    t = ox.from_numpy(np.ones(3, np.float32))\n"
            "    print('ok', t.device, float((t + 1.0).sum().item()), _native.current_device())\n"
            "except Exception as e:\n"
            "    print(type(e).__name__, e)\n")
    out = _child("0", code)
    assert "ok hip:0 6.0 0" in out.stdout, (out.stdout, out.stderr)
    out = _child(str(n), code)
    assert f"device index {n} out of range" in out.stdout, (out.stdout, out.stderr)
