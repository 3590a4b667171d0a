"""roctx ranges around the beam path's host-side phases.

``roctx_range(name)`` pushes a roctx range on entry and pops it on exit
(``roctxRangePushA`` / ``roctxRangePop`` of ROCm's rocprofiler-sdk roctx
library, bound with ctypes), so ``rocprofv3 --marker-trace --kernel-trace`` shows each phase
around the kernels it launches.  The reference brackets its attention
metadata build the same way with NVTX
(vllm_gr/v1/attention/backends/beam_attn.py:486, :526).  Without the library,
or with ``VLLM_GR_ROCTX=0``, a range is a no-op.  The ranges are host-side
only: work captured into a HIP graph is replayed without them.
"""

from __future__ import annotations

import contextlib
import ctypes
import os

# rocprofiler-sdk's roctx first: rocprofv3 --marker-trace intercepts that one;
# the older roctracer library is the fallback
_NAMES = ("librocprofiler-sdk-roctx.so.1", "librocprofiler-sdk-roctx.so", "/opt/rocm/lib/librocprofiler-sdk-roctx.so.1",
          "libroctx64.so.4", "libroctx64.so", "/opt/rocm/lib/libroctx64.so")
_lib = None
_loaded = False


def enabled() -> bool:
    return os.environ.get("VLLM_GR_ROCTX", "1") != "0"


def _roctx():
    global _lib, _loaded
    if not _loaded:
        _loaded = True
        for name in _NAMES:
            try:
                lib = ctypes.CDLL(name)
            except OSError:
                continue
            lib.roctxRangePushA.argtypes = [ctypes.c_char_p]
            lib.roctxRangePushA.restype = ctypes.c_int
            lib.roctxRangePop.argtypes = []
            lib.roctxRangePop.restype = ctypes.c_int
            _lib = lib
            break
    return _lib


def available() -> bool:
    """The roctx library was found."""
    return _roctx() is not None


@contextlib.contextmanager
def roctx_range(name: str):
    lib = _roctx() if enabled() else None
    if lib is None:
        yield
        return
    lib.roctxRangePushA(name.encode())
    try:
        yield
    finally:
        lib.roctxRangePop()
