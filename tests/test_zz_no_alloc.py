"""GPU: the allocation-free forward ``dot_sinkhorn_forward_noalloc`` (static
device scratch, no workspace argument) against ``dot_sinkhorn_forward`` with a
caller workspace, through the C ABI, on two calls in a row (the second on a
smaller input, so it runs over what the first left in the shared scratch).
Both run the same kernels on the same inputs: results must be bitwise equal."""

import ctypes
import os

import numpy as np
import pytest
import torch

import dot_amd  # noqa: F401  (loads the library and initialises torch's HIP context)
from conftest import ROOT

pytestmark = pytest.mark.gpu
LIB = os.path.join(ROOT, "dot_amd", "libdot_amd.so")
DEV = torch.device("cuda", 0)
STATIC_SCRATCH_BYTES = 64 << 20


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


@pytest.fixture(scope="module")
def lib():
    lib = ctypes.CDLL(LIB)
    for name in ("dot_sinkhorn_forward", "dot_sinkhorn_forward_noalloc"):
        getattr(lib, name).argtypes = [ctypes.POINTER(FwdArgs), ctypes.c_void_p]
        getattr(lib, name).restype = ctypes.c_int
    lib.dot_sinkhorn_forward_workspace_bytes.restype = ctypes.c_size_t
    lib.dot_last_error.restype = ctypes.c_char_p
    return lib


def _run(lib, entry, C, log_a, log_b, tau, T, tol, workspace):
    B, M, N = C.shape
    out = {"plan": torch.empty_like(C), "cost": torch.empty(B, device=DEV),
           "u": torch.empty(B, M, device=DEV), "v": torch.empty(B, N, device=DEV),
           "counts": torch.full((2,), -7, dtype=torch.int32, device=DEV)}
    a = FwdArgs(scores=C.data_ptr(), log_a=log_a.data_ptr() if log_a is not None else None,
                log_b=log_b.data_ptr() if log_b is not None else None, B=B, M=M, N=N,
                scores_kind=-1, tau=tau, max_iter=T, tol=tol, flags=0,
                plan=out["plan"].data_ptr(), cost=out["cost"].data_ptr(), u_out=out["u"].data_ptr(),
                v_out=out["v"].data_ptr(), iters_used=out["counts"].data_ptr(),
                converged=out["counts"].data_ptr() + 4)
    if workspace is not None:
        a.workspace, a.workspace_bytes = workspace.data_ptr(), workspace.numel()
    stream = torch.cuda.current_stream(DEV).cuda_stream
    rc = getattr(lib, entry)(ctypes.byref(a), ctypes.c_void_p(stream))
    assert rc == 0, (entry, rc, lib.dot_last_error().decode())
    torch.cuda.synchronize(DEV)
    return out


# (B, M, N, tau, T, tol, Dirichlet marginals): the register-resident tier with a
# batch-global stop test first, then a smaller streaming-tier shape with fixed
# iterations and marginals, so the second call starts on the first one's scratch.
CALLS = [(16, 512, 512, 0.1, 200, 1e-6, False), (3, 130, 1500, 0.3, 25, 0.0, True)]


def test_noalloc_forward_matches_workspace_forward(lib):
    rng = np.random.default_rng(2024)
    for B, M, N, tau, T, tol, marg in CALLS:
        need = lib.dot_sinkhorn_forward_workspace_bytes(B, M, N, T, 0)
        assert 0 < need <= STATIC_SCRATCH_BYTES
        print(f"[no_alloc] B={B} M={M} N={N} tau={tau} T={T} tol={tol} scratch={need}", flush=True)
        C = torch.from_numpy(rng.random((B, M, N), dtype=np.float32)).to(DEV)
        log_a = log_b = None
        if marg:
            ea, eb = -np.log(rng.random((B, M))), -np.log(rng.random((B, N)))
            log_a = torch.from_numpy(np.log(ea / ea.sum(1, keepdims=True)).astype(np.float32)).to(DEV)
            log_b = torch.from_numpy(np.log(eb / eb.sum(1, keepdims=True)).astype(np.float32)).to(DEV)
        ws = torch.empty(need, dtype=torch.uint8, device=DEV)
        ref = _run(lib, "dot_sinkhorn_forward", C, log_a, log_b, tau, T, tol, ws)
        got = _run(lib, "dot_sinkhorn_forward_noalloc", C, log_a, log_b, tau, T, tol, None)
        used = int(ref["counts"][0])
        assert 1 <= used <= T and int(got["counts"][0]) == used
        if tol > 0:
            assert used < T and int(ref["counts"][1]) == 1
        for k in ref:
            assert torch.equal(got[k], ref[k]), k
        assert torch.isfinite(got["plan"]).all()
        # column sums of the plan equal the column marginal (exact after a column update)
        b = torch.full((B, N), 1.0 / N, device=DEV) if log_b is None else log_b.exp()
        assert torch.allclose(got["plan"].sum(-2), b, rtol=1e-4, atol=1e-9)


def test_noalloc_forward_rejects_shapes_beyond_the_scratch(lib):
    B, M, N, T = 256, 2048, 2048, 100
    assert lib.dot_sinkhorn_forward_workspace_bytes(B, M, N, T, 0) > STATIC_SCRATCH_BYTES
    a = FwdArgs(B=B, M=M, N=N, scores_kind=-1, tau=0.1, max_iter=T)
    assert lib.dot_sinkhorn_forward_noalloc(ctypes.byref(a), None) == 3  # DOT_ERR_UNSUPPORTED
    assert "static scratch" in lib.dot_last_error().decode()
