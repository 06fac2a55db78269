"""TEST INFRASTRUCTURE ONLY — ctypes access to the reference's compiled CPU kernels.

``oracle/_ref/libdotref.so`` is built by ``oracle/Makefile`` from the
reference's own ``src/sinkhorn/kernels_cpu.cpp`` and
``src/bidirectional_softmax/kernels_cpu.cpp`` (single-threaded fp32, Kahan
row/column LSE, ``safe_exp``).  It exists only where ``/root/reference`` was
present at build time; callers must handle :func:`available` being False.

Only ``tests/``, ``tests/golden/make_golden.py`` and ``bench.py``'s
``cpu_baseline`` leg may use this module, and only as a checker or as the timed
CPU baseline — never as a product code path.

Each wrapper reproduces what the reference's torch glue does around the raw
kernel (``src/sinkhorn/torch_cpu.cpp``, ``src/bidirectional_softmax/torch_cpu.cpp``):
fp32 contiguous inputs, freshly allocated fp32 outputs.
"""

from __future__ import annotations

import ctypes
import os
from typing import Optional

import numpy as np

_LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_ref", "libdotref.so")
_lib = None

_F = ctypes.POINTER(ctypes.c_float)
_I = ctypes.POINTER(ctypes.c_int)


def available() -> bool:
    return os.path.exists(_LIB_PATH)


def _load():
    global _lib
    if _lib is None:
        if not available():
            raise FileNotFoundError(
                f"{_LIB_PATH} is not built (run `make -C oracle` where /root/reference exists)"
            )
        lib = ctypes.CDLL(_LIB_PATH)
        lib.ref_sinkhorn_forward.argtypes = [_F, _F, _F, _F] + [ctypes.c_int] * 3 + [
            ctypes.c_float, ctypes.c_int, ctypes.c_int]
        lib.ref_sinkhorn_forward_with_intermediates.argtypes = [_F] * 6 + [ctypes.c_int] * 3 + [
            ctypes.c_float, ctypes.c_int]
        lib.ref_sinkhorn_backward_unrolled.argtypes = [_F] * 9 + [ctypes.c_int] * 3 + [
            ctypes.c_float, ctypes.c_int]
        lib.ref_sinkhorn_backward_implicit.argtypes = [_F] * 7 + [ctypes.c_int] * 3 + [
            ctypes.c_float, ctypes.c_int, ctypes.c_float]
        lib.ref_bidi_forward.argtypes = [_F] * 4 + [_I] + [ctypes.c_int] * 3 + [ctypes.c_float]
        lib.ref_bidi_backward.argtypes = [_F] * 7 + [_I] + [ctypes.c_int] * 3 + [ctypes.c_float]
        for name in ("ref_sinkhorn_forward", "ref_sinkhorn_forward_with_intermediates",
                     "ref_sinkhorn_backward_unrolled", "ref_sinkhorn_backward_implicit",
                     "ref_bidi_forward", "ref_bidi_backward"):
            getattr(lib, name).restype = None
        _lib = lib
    return _lib


def _f32(x: Optional[np.ndarray]) -> Optional[np.ndarray]:
    if x is None:
        return None
    return np.ascontiguousarray(x, dtype=np.float32)


def _p(x: Optional[np.ndarray]):
    if x is None:
        return ctypes.cast(None, _F)
    return x.ctypes.data_as(_F)


def sinkhorn_forward(log_alpha, tau, n_iters, log_a=None, log_b=None, return_log=False):
    """``sinkhorn_forward_cpu`` (src/sinkhorn/kernels_cpu.cpp:60-107); the CPU op path."""
    la = _f32(log_alpha)
    B, n, m = la.shape
    la_, lb_ = _f32(log_a), _f32(log_b)
    out = np.empty_like(la)
    _load().ref_sinkhorn_forward(_p(la), _p(out), _p(la_), _p(lb_), B, n, m,
                                 float(tau), int(n_iters), int(bool(return_log)))
    return out


def sinkhorn_forward_with_intermediates(log_alpha, tau, n_iters, log_a=None, log_b=None):
    """``sinkhorn_forward_with_intermediates_cpu`` (kernels_cpu.cpp:109-167) -> (P, log_X, log_Y)."""
    la = _f32(log_alpha)
    B, n, m = la.shape
    la_, lb_ = _f32(log_a), _f32(log_b)
    P = np.empty_like(la)
    log_X = np.empty((B, n_iters + 1, n, m), np.float32)
    log_Y = np.empty((B, max(n_iters, 1), n, m), np.float32)
    _load().ref_sinkhorn_forward_with_intermediates(_p(la), _p(P), _p(log_X), _p(log_Y), _p(la_),
                                                    _p(lb_), B, n, m, float(tau), int(n_iters))
    return P, log_X, log_Y


def sinkhorn_with_grads_unrolled(log_alpha, grad_P, tau, n_iters, log_a=None, log_b=None):
    """The CPU op ``sinkhorn_with_grads_unrolled`` (torch_cpu.cpp:188-259) -> (P, grad, grad_tau)."""
    la = _f32(log_alpha)
    gP = _f32(grad_P)
    B, n, m = la.shape
    P, log_X, log_Y = sinkhorn_forward_with_intermediates(la, tau, n_iters, log_a, log_b)
    grad = np.empty_like(la)
    grad_tau = np.empty((B,), np.float32)
    _load().ref_sinkhorn_backward_unrolled(_p(la), _p(P), _p(gP), _p(log_X), _p(log_Y),
                                           _p(_f32(log_a)), _p(_f32(log_b)), _p(grad),
                                           _p(grad_tau), B, n, m, float(tau), int(n_iters))
    return P, grad, grad_tau


def sinkhorn_backward_implicit(log_alpha, P, grad_P, tau, max_iters, tol):
    """``sinkhorn_backward_implicit_cpu`` (kernels_cpu.cpp:247-327) -> (grad, grad_tau).

    With ``tol=0`` the per-batch early break (``max_change < tol``) never
    fires, so exactly ``max_iters`` Gauss-Seidel sweeps run — the fixed-count
    semantics of the GPU adjoint (src/sinkhorn/kernels.cu:1715-1718)."""
    la, P_, gP = _f32(log_alpha), _f32(P), _f32(grad_P)
    B, n, m = la.shape
    grad = np.empty_like(la)
    grad_tau = np.empty((B,), np.float32)
    _load().ref_sinkhorn_backward_implicit(_p(la), _p(P_), _p(gP), _p(None), _p(None), _p(grad),
                                           _p(grad_tau), B, n, m, float(tau), int(max_iters),
                                           float(tol))
    return grad, grad_tau


def sinkhorn_with_grads_implicit(log_alpha, grad_P, tau, n_iters, backward_iters,
                                 log_a=None, log_b=None, tol=1e-6):
    """The CPU op ``sinkhorn_with_grads_implicit`` (torch_cpu.cpp:261-328): forward, then the
    adjoint with the CPU's 1e-6 early break (pass ``tol=0`` for the GPU's fixed count)."""
    P = sinkhorn_forward(log_alpha, tau, n_iters, log_a, log_b)
    grad, grad_tau = sinkhorn_backward_implicit(log_alpha, P, grad_P, tau, backward_iters, tol)
    return P, grad, grad_tau


def bidirectional_softmax(sim, tau, lengths):
    """``bidirectional_softmax_forward_cpu`` (bidirectional_softmax/kernels_cpu.cpp:41-133)."""
    s = _f32(sim)
    B, L1, L2 = s.shape
    ln = np.ascontiguousarray(lengths, dtype=np.int32)
    out, r, c = np.empty_like(s), np.empty_like(s), np.empty_like(s)
    _load().ref_bidi_forward(_p(s), _p(out), _p(r), _p(c), ln.ctypes.data_as(_I), B, L1, L2,
                             float(tau))
    return out, r, c


def bidirectional_softmax_backward(sim, out, grad_out, row_sm, col_sm, tau, lengths):
    """``bidirectional_softmax_backward_cpu`` (bidirectional_softmax/kernels_cpu.cpp:139-232)."""
    s, o, g, r, c = (_f32(x) for x in (sim, out, grad_out, row_sm, col_sm))
    B, L1, L2 = s.shape
    ln = np.ascontiguousarray(lengths, dtype=np.int32)
    grad = np.empty_like(s)
    grad_T = np.empty((B,), np.float32)
    _load().ref_bidi_backward(_p(s), _p(o), _p(g), _p(r), _p(c), _p(grad), _p(grad_T),
                              ln.ctypes.data_as(_I), B, L1, L2, float(tau))
    return grad, grad_T
