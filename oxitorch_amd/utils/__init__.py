"""oxitorch_amd.utils: the data pipeline (python/oxitorch/utils/__init__.py)."""

from . import data  # noqa: F401

__all__ = ["data"]
