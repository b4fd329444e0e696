"""oxitorch_amd: the MI355X device path for oxitorch's layer-kernel hot path.

Same surface as the reference package `oxitorch` (python/oxitorch/__init__.py):
`Tensor`, `from_numpy`, `zeros`, `full`, `eye`, grad-mode control and the
`nn` namespace, backed by the C++ host core `_native` (device storage,
dispatch, autograd graph) and the gfx950 kernels of liboxihip. Tensors live
on the HIP device by default; compute never falls back to the CPU.
"""

from contextlib import contextmanager

from oxitorch_amd._native import (  # noqa: F401
    Tensor,
    __version__,
    device_count,
    eye,
    from_numpy,
    full,
    get_default_device,
    is_grad_enabled,
    memory_stats,
    set_default_device,
    set_grad_enabled,
    synchronize,
    version,
    zeros,
)
from oxitorch_amd import nn, optim, utils  # noqa: E402

__all__ = [
    "Tensor",
    "__version__",
    "device_count",
    "enable_grad",
    "eye",
    "from_numpy",
    "full",
    "get_default_device",
    "is_grad_enabled",
    "memory_stats",
    "nn",
    "no_grad",
    "optim",
    "utils",
    "set_default_device",
    "set_grad_enabled",
    "synchronize",
    "version",
    "zeros",
]


@contextmanager
def _grad_mode(enabled):
    prev = set_grad_enabled(enabled)
    try:
        yield
    finally:
        set_grad_enabled(prev)


def no_grad():
    """Context manager disabling graph recording (python/oxitorch/__init__.py:46-63)."""
    return _grad_mode(False)


def enable_grad():
    """Context manager force-enabling graph recording (python/oxitorch/__init__.py:66-75)."""
    return _grad_mode(True)
