"""GPU parity of the one-pass bidirectional softmax (rows and columns of
513..1024, a batch of at least the GPU's XCD count): against the oracle, the
two-sweep kernels, and itself through the fallback that a late workgroup takes
(which must give the exchange's results bit for bit)."""

import ctypes
import os

import numpy as np
import pytest
import torch

import dot_amd
from conftest import ROOT, rel_err
from oracle import bidirectional_softmax as obs

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)
FWD_TOL, GRAD_TOL = 1e-5, 1e-4


def _t(x):
    return torch.as_tensor(np.ascontiguousarray(x)).to(DEV)


def _fused(sim, G, tau, ln):
    """Forward and backward through the autograd path (statistics, no grad_tau),
    the calls the one-pass kernels serve."""
    x = sim.clone().requires_grad_(True)
    P = dot_amd.bidirectional_softmax(x, tau, ln)
    P.backward(G)
    torch.cuda.synchronize()
    return P.detach(), x.grad


ONEPASS_SHAPES = [
    # (B, L1, L2, tau, lengths or None)
    (8, 1024, 1024, 1.0, None),
    (9, 600, 1000, 0.5, "ragged"),
    (12, 1024, 516, 2.0, "ragged"),
    (16, 777, 1024, 0.8, "ragged"),
    (8, 513, 772, 1.0, None),
    (8, 1024, 768, 1.3, "ragged"),  # 768 columns: constant column bounds with lengths
]


def _lengths(B, L1, L2, kind, rng):
    if kind is None:
        return np.array([[L1, L2]] * B, np.int32)
    ln = np.stack([rng.integers(0, L1 + 1, B), rng.integers(0, L2 + 1, B)], 1).astype(np.int32)
    ln[0] = [L1, L2]
    ln[1] = [0, L2]
    ln[2] = [L1, 0]
    ln[3] = [1, 1]
    return ln


@pytest.mark.parametrize("B,L1,L2,tau,kind", ONEPASS_SHAPES)
def test_onepass_matches_oracle(B, L1, L2, tau, kind):
    print(f"one-pass vs oracle B={B} L1={L1} L2={L2} tau={tau} lengths={kind}", flush=True)
    rng = np.random.default_rng(B * 7 + L1 + L2)
    s = (2.0 * rng.standard_normal((B, L1, L2))).astype(np.float32)
    g = rng.standard_normal((B, L1, L2)).astype(np.float32)
    ln = _lengths(B, L1, L2, kind, rng)
    out_o, r_o, c_o = obs.forward(s, tau, ln)
    gs_o, _ = obs.backward(s, out_o, g, r_o, c_o, tau, ln)
    P, grad = _fused(_t(s), _t(g), tau, _t(ln))
    assert rel_err(P, out_o) < FWD_TOL
    assert rel_err(grad, gs_o) < GRAD_TOL
    for b in range(B):
        l1, l2 = ln[b]
        for T in (P, grad):
            assert (T[b, l1:, :] == 0).all() and (T[b, :, l2:] == 0).all()


def test_onepass_agrees_with_two_sweeps(monkeypatch):
    """The one-pass tier and the two-sweep kernels on the same C2-sized input."""
    B, L1, L2, tau = 32, 1024, 1024, 1.0
    sim = torch.randn(B, L1, L2, generator=torch.Generator().manual_seed(1)).to(DEV)
    G = torch.randn(B, L1, L2, generator=torch.Generator().manual_seed(2)).to(DEV)
    ln = torch.tensor([[L1, L2]] * B, dtype=torch.int32, device=DEV)
    P1, g1 = _fused(sim, G, tau, ln)
    monkeypatch.setenv("DOT_AMD_BIDI_ONEPASS", "0")
    P2, g2 = _fused(sim, G, tau, ln)
    assert rel_err(P1, P2) < 2e-6
    assert rel_err(g1, g2) < 2e-5


@pytest.mark.parametrize("ticks", ["-1", "0"])
@pytest.mark.parametrize("tile", [False, True])
def test_fallback_is_bitwise_the_exchange(monkeypatch, ticks, tile):
    """-1: every workgroup computes the column statistics itself; 0: a wait gives
    up at its first miss, so exchange and fallback mix.  Either way the results
    are bitwise those of the exchange path (same arithmetic, same order).  `tile`:
    no lengths and 1024 x 1024 elements (the kernels with constant extents)."""
    print(f"fallback ticks={ticks} tile={tile}", flush=True)
    rng = np.random.default_rng(5)
    B, L1, L2, tau = (8, 1024, 1024, 0.7) if tile else (10, 1000, 1024, 0.7)
    s = _t((2.0 * rng.standard_normal((B, L1, L2))).astype(np.float32))
    g = _t(rng.standard_normal((B, L1, L2)).astype(np.float32))
    ln = None if tile else _t(_lengths(B, L1, L2, "ragged", rng))
    P1, g1 = _fused(s, g, tau, ln)
    monkeypatch.setenv("DOT_AMD_BIDI_WAIT_TICKS", ticks)
    P2, g2 = _fused(s, g, tau, ln)
    assert torch.equal(P1, P2)
    assert torch.equal(g1, g2)


@pytest.mark.parametrize("L2", [1024, 768])
def test_full_tile_matches_oracle(L2):
    """No lengths and 1024 x 1024 (or 1024 x 768) elements: the kernels whose
    extents are constants, against the oracle."""
    rng = np.random.default_rng(21)
    B, L1, tau = 8, 1024, 0.6
    s = (2.0 * rng.standard_normal((B, L1, L2))).astype(np.float32)
    g = rng.standard_normal((B, L1, L2)).astype(np.float32)
    ln = np.array([[L1, L2]] * B, np.int32)
    out_o, r_o, c_o = obs.forward(s, tau, ln)
    gs_o, _ = obs.backward(s, out_o, g, r_o, c_o, tau, ln)
    P, grad = _fused(_t(s), _t(g), tau, None)
    assert rel_err(P, out_o) < FWD_TOL
    assert rel_err(grad, gs_o) < GRAD_TOL


def test_repeated_calls_are_deterministic():
    """Successive calls advance the exchange epoch of the stream's words; the
    results do not change."""
    rng = np.random.default_rng(11)
    B, L1, L2 = 16, 1024, 1024
    s = _t(rng.standard_normal((B, L1, L2)).astype(np.float32))
    g = _t(rng.standard_normal((B, L1, L2)).astype(np.float32))
    ln = torch.tensor([[L1, L2]] * B, dtype=torch.int32, device=DEV)
    P0, g0 = _fused(s, g, 1.0, ln)
    for _ in range(5):
        P, gr = _fused(s, g, 1.0, ln)
        assert torch.equal(P, P0) and torch.equal(gr, g0)


class BidiFwdArgs(ctypes.Structure):
    _fields_ = [("sim", ctypes.c_void_p), ("lengths", ctypes.c_void_p),
                ("B", ctypes.c_int), ("L1", ctypes.c_int), ("L2", ctypes.c_int), ("tau", ctypes.c_float),
                ("out", ctypes.c_void_p), ("row_sm", ctypes.c_void_p), ("col_sm", ctypes.c_void_p),
                ("row_stats", ctypes.c_void_p), ("col_stats", ctypes.c_void_p),
                ("workspace", ctypes.c_void_p), ("workspace_bytes", ctypes.c_size_t),
                ("exchange", ctypes.c_void_p), ("exchange_epoch", ctypes.c_uint32)]


class BidiBwdArgs(ctypes.Structure):
    _fields_ = [("sim", ctypes.c_void_p), ("lengths", ctypes.c_void_p),
                ("B", ctypes.c_int), ("L1", ctypes.c_int), ("L2", ctypes.c_int), ("tau", ctypes.c_float),
                ("grad_out", ctypes.c_void_p), ("out", ctypes.c_void_p), ("row_sm", ctypes.c_void_p),
                ("col_sm", ctypes.c_void_p), ("row_stats", ctypes.c_void_p), ("col_stats", ctypes.c_void_p),
                ("grad_sim", ctypes.c_void_p), ("grad_tau", ctypes.c_void_p),
                ("workspace", ctypes.c_void_p), ("workspace_bytes", ctypes.c_size_t),
                ("exchange", ctypes.c_void_p), ("exchange_epoch", ctypes.c_uint32)]


def test_capi_workspace_and_caller_exchange_agree():
    """Through the C ABI: exchange words from the workspace (cleared per call)
    and caller-owned words with a growing epoch give the same bits; an epoch of
    0 is rejected."""
    lib = ctypes.CDLL(os.path.join(ROOT, "dot_amd", "libdot_amd.so"))
    for f in ("dot_bidisoftmax_forward_workspace_bytes", "dot_bidisoftmax_backward_workspace_bytes",
              "dot_bidisoftmax_exchange_bytes"):
        getattr(lib, f).restype = ctypes.c_size_t
    B, L1, L2, tau = 8, 1024, 1024, 1.0
    rng = np.random.default_rng(3)
    sim = _t(rng.standard_normal((B, L1, L2)).astype(np.float32))
    G = _t(rng.standard_normal((B, L1, L2)).astype(np.float32))
    ln = torch.tensor([[L1, L2]] * B, dtype=torch.int32, device=DEV)
    ws = torch.empty(max(lib.dot_bidisoftmax_forward_workspace_bytes(B, L1, L2),
                         lib.dot_bidisoftmax_backward_workspace_bytes(B, L1, L2)), dtype=torch.uint8, device=DEV)
    xw = torch.zeros(lib.dot_bidisoftmax_exchange_bytes(), dtype=torch.uint8, device=DEV)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

    def run(exchange, epoch):
        out = torch.empty_like(sim)
        rs = torch.empty(B, 2, L1, device=DEV)
        cs = torch.empty(B, 2, L2, device=DEV)
        gs = torch.empty_like(sim)
        f = BidiFwdArgs(sim.data_ptr(), ln.data_ptr(), B, L1, L2, tau, out.data_ptr(), None, None, rs.data_ptr(),
                        cs.data_ptr(), ws.data_ptr(), ws.numel(), exchange, epoch)
        assert lib.dot_bidisoftmax_forward(ctypes.byref(f), stream) == 0
        b = BidiBwdArgs(sim.data_ptr(), ln.data_ptr(), B, L1, L2, tau, G.data_ptr(), None, None, None,
                        rs.data_ptr(), cs.data_ptr(), gs.data_ptr(), None, ws.data_ptr(), ws.numel(), exchange,
                        epoch + 1)
        assert lib.dot_bidisoftmax_backward(ctypes.byref(b), stream) == 0
        torch.cuda.synchronize()
        return out, gs

    o1, g1 = run(None, 0)
    o2, g2 = run(xw.data_ptr(), 1)
    o3, g3 = run(xw.data_ptr(), 3)
    assert torch.equal(o1, o2) and torch.equal(g1, g2)
    assert torch.equal(o1, o3) and torch.equal(g1, g3)
    out = torch.empty_like(sim)
    f = BidiFwdArgs(sim.data_ptr(), ln.data_ptr(), B, L1, L2, tau, out.data_ptr(), None, None, None, None,
                    ws.data_ptr(), ws.numel(), xw.data_ptr(), 0)
    assert lib.dot_bidisoftmax_forward(ctypes.byref(f), stream) == 1
