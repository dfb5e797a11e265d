"""summa_amd — MI355X-native GRPO RL-step engine (gfx950 HIP kernels behind a C ABI).

The compute lives in ``libsumma_amd.so`` (``summa_amd/csrc``); this package is
the host-side mirror of the reference's entry points plus ctypes plumbing.
"""
from ._lib import LIB_PATH, SummaError, lib  # noqa: F401

__all__ = ["LIB_PATH", "SummaError", "lib"]
