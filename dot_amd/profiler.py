"""Per-kernel durations from the C ABI's event profiler (``dot_profile_*``).

When enabled, every selected kernel launch is bracketed by two HIP events on
the stream it runs on; :func:`collect` waits for them and accumulates
durations by kernel name.  Used by ``bench.py`` for the roofline figures.
"""

import atexit
import ctypes
import os

from . import _ops  # noqa: F401  (loads libdot_amd.so through _C.so)

_lib = ctypes.CDLL(os.path.join(os.path.dirname(os.path.abspath(__file__)), "libdot_amd.so"))
_lib.dot_profile_enable.argtypes = [ctypes.c_int]
_lib.dot_profile_enable.restype = None
_lib.dot_profile_select.argtypes = [ctypes.c_char_p]
_lib.dot_profile_select.restype = None
_lib.dot_profile_collect.argtypes = []
_lib.dot_profile_collect.restype = ctypes.c_int
_lib.dot_profile_query.argtypes = [ctypes.c_char_p, ctypes.POINTER(ctypes.c_int64),
                                   ctypes.POINTER(ctypes.c_double)]
_lib.dot_profile_query.restype = ctypes.c_int
_lib.dot_profile_reset.argtypes = []
_lib.dot_profile_reset.restype = None
_lib.dot_profile_shutdown.argtypes = []
_lib.dot_profile_shutdown.restype = ctypes.c_int
_lib.dot_last_error.restype = ctypes.c_char_p


def enable(on: bool = True, kernels=None) -> None:
    """Turn the profiler on or off; ``kernels`` limits it to those kernel names."""
    _lib.dot_profile_select((",".join(kernels)).encode() if kernels else None)
    _lib.dot_profile_enable(1 if on else 0)


def collect() -> None:
    """Wait for recorded events and fold them into the per-kernel totals."""
    if _lib.dot_profile_collect() != 0:
        raise RuntimeError(_lib.dot_last_error().decode())


def query(kernel: str):
    """(launches, total milliseconds) recorded for ``kernel``."""
    n = ctypes.c_int64()
    ms = ctypes.c_double()
    if _lib.dot_profile_query(kernel.encode(), ctypes.byref(n), ctypes.byref(ms)) != 0:
        raise RuntimeError(_lib.dot_last_error().decode())
    return int(n.value), float(ms.value)


def reset() -> None:
    _lib.dot_profile_reset()


def shutdown() -> None:
    """Disable the profiler and destroy its HIP events (idempotent)."""
    if _lib.dot_profile_shutdown() != 0:
        raise RuntimeError(_lib.dot_last_error().decode())


# Events left to process teardown outlive the HIP runtime; release them while
# it is still up (Python's exit hooks run before the C library's).
atexit.register(_lib.dot_profile_shutdown)
