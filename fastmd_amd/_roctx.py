"""roctx ranges around the host-side phases of the MD step (builder, integrator halves, window
launches, logger), the tracing hook of fastmd/_nvtx.py:10-32 (``nvtx_range``, ``nvtx_ranged``).

The ranges go straight to ROCm's ``libroctx64`` (``roctxRangePushA`` / ``roctxRangePop``), which
``rocprofv3 --marker-trace`` records; without a profiler attached they cost one library call. The
library is looked up once; when it is absent the ranges are no-ops. Ranges are host-side markers:
inside a graph capture they mark the capture, not the replays.
"""
from __future__ import annotations

import ctypes
import ctypes.util
import functools
import os
from contextlib import contextmanager
from collections.abc import Iterator

_LIB = None
_LOADED = False


def _library():
    global _LIB, _LOADED
    if not _LOADED:
        _LOADED = True
        names = [os.path.join(os.environ.get("ROCM_PATH", "/opt/rocm"), "lib", "libroctx64.so"),
                 ctypes.util.find_library("roctx64")]
        for name in names:
            if not name:
                continue
            try:
                lib = ctypes.CDLL(name)
            except OSError:
                continue
            lib.roctxRangePushA.argtypes = [ctypes.c_char_p]
            lib.roctxRangePushA.restype = ctypes.c_int
            lib.roctxRangePop.argtypes = []
            lib.roctxRangePop.restype = ctypes.c_int
            _LIB = lib
            break
    return _LIB


@contextmanager
def roctx_range(name: str) -> Iterator[None]:
    """A roctx range named ``name`` around the body (no-op without libroctx64)."""
    lib = _library()
    if lib is None:
        yield
        return
    lib.roctxRangePushA(name.encode())
    try:
        yield
    finally:
        lib.roctxRangePop()


def roctx_ranged(name: str):
    """Decorator: the function's body inside ``roctx_range(name)``."""
    def decorate(fn):
        @functools.wraps(fn)
        def wrapper(*args, **kwargs):
            with roctx_range(name):
                return fn(*args, **kwargs)
        return wrapper
    return decorate


# the reference's names for the same hooks
nvtx_range = roctx_range
nvtx_ranged = roctx_ranged
