"""Loader of the native library (replaces reference ``src/logitfill/packed/kernel_loader.py:14-35``).

The reference JIT-compiles ``kernel.cu`` on first use and silently falls back to
the dense path when that fails.  Here the HIP library is built ahead of time
(``python -m logitfill_amd.build``) and a missing build raises
``NativeLibraryMissing``: no silent fallback.
"""
from __future__ import annotations

from logitfill_amd import _native
from logitfill_amd._native import NativeLibraryMissing  # noqa: F401


def get_kernel():
    """Return the loaded ``liblogitfill_amd.so`` (ctypes handle); raises when it is not built."""
    return _native.load()
