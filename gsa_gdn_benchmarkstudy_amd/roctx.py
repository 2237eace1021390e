"""ROCTx markers for rocprofv3: named ranges and the profiler's capture window.

Binds ``librocprofiler-sdk-roctx`` (the marker library rocprofv3 intercepts)
with ctypes.  torch's ``torch.cuda.nvtx`` on ROCm calls the older roctracer
``libroctx64`` bundled with torch, whose ranges rocprofv3's ``--marker-trace``
may not see, so the layer and the harness use this module instead.

When the library is absent every call is a no-op: markers are instrumentation,
never part of the computation.

- ``range_push(name)`` / ``range_pop()``: nested ranges (``--marker-trace``; with
  ``--kernel-rename`` kernels take the innermost range's name).
- ``profiler_resume()`` / ``profiler_pause()``: the capture window that
  ``rocprofv3 --selected-regions`` honours (tid 0 = every thread of the process),
  the counterpart of ``cudaProfilerStart/Stop`` in the reference harness
  (gsa_triton/benchmark.py:331,349).
"""

from __future__ import annotations

import contextlib
import ctypes
import os
from typing import Iterator, Optional

_LIB: Optional[ctypes.CDLL] = None
_TRIED = False


def _candidates():
    names = ("librocprofiler-sdk-roctx.so.1", "librocprofiler-sdk-roctx.so")
    roots = [os.environ.get("ROCM_PATH"), "/opt/rocm"]
    for root in roots:
        if root:
            for n in names:
                yield os.path.join(root, "lib", n)
    yield from names  # the loader's own search path


def _lib() -> Optional[ctypes.CDLL]:
    global _LIB, _TRIED
    if _TRIED:
        return _LIB
    _TRIED = True
    if os.environ.get("GSA_ROCTX", "1") == "0":
        return None
    for path in _candidates():
        try:
            lib = ctypes.CDLL(path)
        except OSError:
            continue
        lib.roctxRangePushA.argtypes = [ctypes.c_char_p]
        lib.roctxRangePushA.restype = ctypes.c_int
        lib.roctxRangePop.argtypes = []
        lib.roctxRangePop.restype = ctypes.c_int
        lib.roctxMarkA.argtypes = [ctypes.c_char_p]
        lib.roctxMarkA.restype = None
        lib.roctxProfilerPause.argtypes = [ctypes.c_uint64]
        lib.roctxProfilerPause.restype = ctypes.c_int
        lib.roctxProfilerResume.argtypes = [ctypes.c_uint64]
        lib.roctxProfilerResume.restype = ctypes.c_int
        _LIB = lib
        break
    return _LIB


def available() -> bool:
    """True when the marker library is loaded (markers reach a profiler, if one runs)."""
    return _lib() is not None


def range_push(name: str) -> int:
    lib = _lib()
    return lib.roctxRangePushA(name.encode()) if lib is not None else 0


def range_pop() -> int:
    lib = _lib()
    return lib.roctxRangePop() if lib is not None else 0


def mark(name: str) -> None:
    lib = _lib()
    if lib is not None:
        lib.roctxMarkA(name.encode())


def profiler_resume() -> int:
    """Open the capture window (``rocprofv3 --selected-regions``)."""
    lib = _lib()
    return lib.roctxProfilerResume(0) if lib is not None else 0


def profiler_pause() -> int:
    """Close the capture window."""
    lib = _lib()
    return lib.roctxProfilerPause(0) if lib is not None else 0


@contextlib.contextmanager
def region(name: str) -> Iterator[None]:
    """``with region("gsa_hip/iter0"): ...`` -- a range that is popped on exit."""
    range_push(name)
    try:
        yield
    finally:
        range_pop()
