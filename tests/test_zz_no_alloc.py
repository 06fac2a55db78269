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


def test_scratch_is_reserved_by_the_first_noalloc_call(lib):
    """The static scratch is a code object of its own (noalloc.hip, no
    kernels): the Sinkhorn kernels' use does not place it on the GPU, the first
    dot_sinkhorn_forward_noalloc call on the GPU does.  Runs before every other
    call of the entry point in the process (this file's first test; no other
    test file calls it)."""
    B, M, N, T = 4, 64, 64, 20
    C = torch.rand(B, M, N, device=DEV)
    out = {k: torch.empty(n, device=DEV) for k, n in (("plan", B * M * N), ("cost", B))}
    counts = torch.zeros(2, dtype=torch.int32, device=DEV)
    ws = torch.empty(lib.dot_sinkhorn_forward_workspace_bytes(B, M, N, T, 0), dtype=torch.uint8, device=DEV)
    a = FwdArgs(scores=C.data_ptr(), B=B, M=M, N=N, scores_kind=-1, tau=0.5, max_iter=T, tol=0.0,
                plan=out["plan"].data_ptr(), cost=out["cost"].data_ptr(), iters_used=counts.data_ptr(),
                converged=counts.data_ptr() + 4, workspace=ws.data_ptr(), workspace_bytes=ws.numel())
    stream = ctypes.c_void_p(torch.cuda.current_stream(DEV).cuda_stream)
    assert lib.dot_sinkhorn_forward(ctypes.byref(a), stream) == 0
    torch.cuda.synchronize(DEV)
    free0 = torch.cuda.mem_get_info(DEV)[0]
    assert lib.dot_sinkhorn_forward_noalloc(ctypes.byref(a), stream) == 0
    torch.cuda.synchronize(DEV)
    free1 = torch.cuda.mem_get_info(DEV)[0]
    assert lib.dot_sinkhorn_forward_noalloc(ctypes.byref(a), stream) == 0
    torch.cuda.synchronize(DEV)
    free2 = torch.cuda.mem_get_info(DEV)[0]
    print(f"[no_alloc] device free bytes: {free0} before the first call, {free1} after, {free2} after the second",
          flush=True)
    assert free0 - free1 >= STATIC_SCRATCH_BYTES
    assert free1 == free2


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
