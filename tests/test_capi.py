"""CPU: the C ABI library loads, exports every declared symbol, and rejects bad
arguments on the host before touching a device.  No compute call is made."""

import ctypes
import os
import re

import pytest

from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "dot_amd.h")
LIB = os.path.join(ROOT, "dot_amd", "libdot_amd.so")

DOT_OK, DOT_ERR_INVALID_ARG, DOT_ERR_WORKSPACE, DOT_ERR_UNSUPPORTED = 0, 1, 2, 3


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = re.findall(r"^\s*(?:const\s+)?[A-Za-z_][A-Za-z0-9_]*\s*\*?\s*(dot_[a-z0-9_]+)\s*\(", text, re.M)
    return sorted(set(names))


@pytest.fixture(scope="module")
def lib():
    assert os.path.exists(LIB), "libdot_amd.so is not built (python -m dot_amd._build)"
    return ctypes.CDLL(LIB)


class FwdArgs(ctypes.Structure):
    _fields_ = [("scores", ctypes.c_void_p), ("log_a", ctypes.c_void_p), ("log_b", ctypes.c_void_p),
                ("B", ctypes.c_int), ("M", ctypes.c_int), ("N", ctypes.c_int),
                ("scores_kind", ctypes.c_int), ("tau", ctypes.c_float), ("max_iter", ctypes.c_int),
                ("tol", ctypes.c_float), ("flags", ctypes.c_int),
                ("plan", ctypes.c_void_p), ("cost", ctypes.c_void_p), ("u_out", ctypes.c_void_p),
                ("v_out", ctypes.c_void_p), ("u_hist", ctypes.c_void_p), ("v_hist", ctypes.c_void_p),
                ("iters_used", ctypes.c_void_p), ("converged", ctypes.c_void_p),
                ("workspace", ctypes.c_void_p), ("workspace_bytes", ctypes.c_size_t),
                ("exchange", ctypes.c_void_p), ("exchange_epoch", ctypes.c_uint32)]


def test_header_declares_the_expected_entry_points():
    names = declared_functions()
    for required in ("dot_sinkhorn_forward", "dot_sinkhorn_backward_implicit",
                     "dot_sinkhorn_backward_unrolled", "dot_bidisoftmax_forward",
                     "dot_bidisoftmax_backward", "dot_last_error"):
        assert required in names


def test_every_declared_symbol_is_exported(lib):
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing


def test_workspace_queries_are_pure_host(lib):
    for fn, args in (("dot_sinkhorn_forward_workspace_bytes", (64, 512, 512, 200, 0)),
                     ("dot_sinkhorn_backward_implicit_workspace_bytes", (64, 512, 512)),
                     ("dot_sinkhorn_backward_unrolled_workspace_bytes", (64, 512, 512)),
                     ("dot_bidisoftmax_forward_workspace_bytes", (32, 1024, 1024)),
                     ("dot_bidisoftmax_backward_workspace_bytes", (32, 1024, 1024))):
        f = getattr(lib, fn)
        f.restype = ctypes.c_size_t
        assert f(*args) > 0
        assert f(*((-1,) + args[1:])) == 0
    f = lib.dot_sinkhorn_backward_unrolled_workspace_bytes
    f.restype = ctypes.c_size_t
    assert f(4, 64, 64) >= 4 * 64 * 64 * 4  # holds the Gamma matrix


def _last_error(lib):
    lib.dot_last_error.restype = ctypes.c_char_p
    return lib.dot_last_error().decode()


def test_forward_rejects_bad_arguments_on_the_host(lib):
    lib.dot_sinkhorn_forward.argtypes = [ctypes.POINTER(FwdArgs), ctypes.c_void_p]
    assert lib.dot_sinkhorn_forward(None, None) == DOT_ERR_INVALID_ARG
    assert "NULL" in _last_error(lib)
    a = FwdArgs(B=2, M=8, N=8, scores_kind=1, tau=0.0, max_iter=10)
    assert lib.dot_sinkhorn_forward(ctypes.byref(a), None) == DOT_ERR_INVALID_ARG
    assert "tau" in _last_error(lib)
    a.tau = 1.0
    a.scores_kind = 7
    assert lib.dot_sinkhorn_forward(ctypes.byref(a), None) == DOT_ERR_INVALID_ARG
    a.scores_kind = 1
    a.N = -3
    assert lib.dot_sinkhorn_forward(ctypes.byref(a), None) == DOT_ERR_INVALID_ARG
    assert ">= 0" in _last_error(lib)
    a.N = 8
    a.max_iter = -1
    assert lib.dot_sinkhorn_forward(ctypes.byref(a), None) == DOT_ERR_INVALID_ARG
    a.max_iter = 10
    dummy = ctypes.c_int(0)
    a.iters_used = a.converged = ctypes.addressof(dummy)
    a.scores = ctypes.addressof(dummy)
    a.workspace, a.workspace_bytes = ctypes.addressof(dummy), 4
    assert lib.dot_sinkhorn_forward(ctypes.byref(a), None) == DOT_ERR_WORKSPACE


def test_version_string(lib):
    lib.dot_version.restype = ctypes.c_char_p
    assert lib.dot_version().decode().startswith("dot_amd")


class MethodArgs(ctypes.Structure):
    _fields_ = [("base", FwdArgs), ("method", ctypes.c_int), ("omega", ctypes.c_float),
                ("anderson_k", ctypes.c_int), ("mixing_beta", ctypes.c_float), ("lr", ctypes.c_float),
                ("beta1", ctypes.c_float), ("beta2", ctypes.c_float), ("eps_adam", ctypes.c_float),
                ("bias_correction", ctypes.c_int), ("reg_start", ctypes.c_float), ("schedule", ctypes.c_int)]


def test_method_forward_rejects_bad_arguments_on_the_host(lib):
    f = lib.dot_sinkhorn_forward_method
    f.argtypes = [ctypes.POINTER(MethodArgs), ctypes.c_void_p]
    q = lib.dot_sinkhorn_forward_method_workspace_bytes
    q.restype = ctypes.c_size_t
    # Anderson keeps anderson_k (state, residual) pairs: the query grows with it
    assert q(2, 64, 64, 50, 2, 8) > q(2, 64, 64, 50, 2, 2) > 0
    assert q(2, 64, 64, 50, 3, 5) > q(2, 64, 64, 50, 1, 5)  # Adam's moments
    # the plain method runs on dot_sinkhorn_forward's workspace after a table of T scales
    fq = lib.dot_sinkhorn_forward_workspace_bytes
    fq.restype = ctypes.c_size_t
    assert q(2, 64, 64, 50, 0, 5) == fq(2, 64, 64, 50, 0) + 256
    assert q(-1, 64, 64, 50, 0, 5) == 0
    assert f(None, None) == DOT_ERR_INVALID_ARG
    dummy = ctypes.c_int(0)
    m = MethodArgs(base=FwdArgs(B=2, M=8, N=8, scores_kind=1, tau=1.0, max_iter=10),
                   method=1, omega=1.5, anderson_k=5, schedule=0)
    m.base.iters_used = m.base.converged = ctypes.addressof(dummy)
    for field, value, code, text in (("method", 4, DOT_ERR_INVALID_ARG, "method"),
                                     ("schedule", 9, DOT_ERR_INVALID_ARG, "schedule"),
                                     ("anderson_k", 0, DOT_ERR_INVALID_ARG, "anderson_k")):
        good = getattr(m, field)
        setattr(m, field, value)
        assert f(ctypes.byref(m), None) == code
        assert text in _last_error(lib)
        setattr(m, field, good)
    # the ring holds min(anderson_k, max_iter) pairs, at most DOT_SK_MAX_ANDERSON = 64
    m.method, m.anderson_k, m.base.max_iter = 2, 65, 65
    assert f(ctypes.byref(m), None) == DOT_ERR_UNSUPPORTED
    assert "anderson_k and max_iter" in _last_error(lib)
    assert q(2, 64, 64, 40, 2, 1000) == q(2, 64, 64, 40, 2, 40)  # a ring of max_iter pairs
    assert "#define DOT_SK_MAX_ANDERSON 64" in open(HEADER).read()
    m.anderson_k = 5
    m.base.flags = 0x2  # history is not kept by the accelerated solvers
    assert f(ctypes.byref(m), None) == DOT_ERR_INVALID_ARG
    m.base.flags = 0
    m.base.tau = -1.0
    assert f(ctypes.byref(m), None) == DOT_ERR_INVALID_ARG
    m.base.tau = 1.0
    m.base.scores = ctypes.addressof(dummy)
    m.base.workspace, m.base.workspace_bytes = ctypes.addressof(dummy), 4
    assert f(ctypes.byref(m), None) == DOT_ERR_WORKSPACE


def test_noalloc_forward_rejects_on_the_host(lib):
    """The allocation-free forward checks the shape against its static scratch
    (DOT_STATIC_SCRATCH_BYTES) before touching a device."""
    f = lib.dot_sinkhorn_forward_noalloc
    f.argtypes = [ctypes.POINTER(FwdArgs), ctypes.c_void_p]
    q = lib.dot_sinkhorn_forward_workspace_bytes
    q.restype = ctypes.c_size_t
    assert f(None, None) == DOT_ERR_INVALID_ARG
    assert q(256, 2048, 2048, 100, 0) > 64 << 20
    a = FwdArgs(B=256, M=2048, N=2048, scores_kind=1, tau=1.0, max_iter=100)
    assert f(ctypes.byref(a), None) == DOT_ERR_UNSUPPORTED
    assert "static scratch holds 67108864" in _last_error(lib)
    assert "#define DOT_STATIC_SCRATCH_BYTES (64u << 20)" in open(HEADER).read()


def test_long_rows_and_large_batches_have_workspace(lib):
    """Rows longer than 4096 columns and batches above 65535 are accepted: the
    workspace queries size their chunk and strip partials."""
    q = lib.dot_sinkhorn_forward_workspace_bytes
    q.restype = ctypes.c_size_t
    # the tiled path adds a [B, nchunks, M] plane of (max, sum) row partials to
    # the double-buffered potentials and the strip partials
    B, M, N = 2, 64, 8192
    assert q(B, M, N, 10, 0) >= B * 4 * M * 8 + 2 * B * (M + N) * 4 + B * N * 4
    assert q(70001, 3, 6, 10, 0) > 2 * 70001 * (3 + 6) * 4
    u = lib.dot_sinkhorn_backward_unrolled_workspace_bytes
    u.restype = ctypes.c_size_t
    assert u(B, M, N) >= B * M * N * 4 + B * 4 * M * 4  # Gamma and the row partials
    # the accelerated methods and the preflight tile rows the same way
    mq = lib.dot_sinkhorn_forward_method_workspace_bytes
    mq.restype = ctypes.c_size_t
    assert mq(B, M, N, 10, 1, 5) >= B * 4 * M * 8 + 3 * B * M * 4  # (max, sum) plane and row terms
    assert mq(B, M, N, 10, 2, 5) > mq(B, M, 4096, 10, 2, 5)
    pq = lib.dot_sinkhorn_spectral_preflight_workspace_bytes
    pq.restype = ctypes.c_size_t
    assert pq(B, M, N) >= B * 4 * M * (8 + 4)  # LSE and row-dot chunk planes
    for name in ("dot_sinkhorn_backward_implicit_workspace_bytes", "dot_bidisoftmax_forward_workspace_bytes",
                 "dot_bidisoftmax_backward_workspace_bytes"):
        f = getattr(lib, name)
        f.restype = ctypes.c_size_t
        assert f(B, M, N) >= B * 4 * M * 4
        assert f(70001, 3, 6) > 0
