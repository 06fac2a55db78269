"""HIP graph capture of the exchange kernels.

The torch ops keep one set of exchange words per (device, stream) and tag the
words with a call epoch fixed when the call is issued.  A captured call would
keep that epoch on every replay and could read the words the previous replay
left, so under capture the ops pass no caller-owned words: the library then
takes the words from the call's workspace and clears them with a kernel that
the graph records.  These tests capture the one-pass bidirectional softmax
(fwd+bwd, C2's shape and a small ragged one), the register-resident and the
persistent Sinkhorn forward + implicit adjoint, replay each graph on changing
inputs with the program's own eager calls and synchronisations between the
replays, and compare every replay with an eager run on the same input and
with the oracle.
"""

import numpy as np
import pytest
import torch

import dot_amd
from dot_amd import _ops
from conftest import rel_err
from oracle import bidirectional_softmax as obs
from oracle import sinkhorn as osk

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)
FWD_TOL, GRAD_TOL = 1e-5, 1e-4


def _bidi_step(sim, G, tau, lengths):
    x = sim.detach().requires_grad_(True)
    P = dot_amd.bidirectional_softmax(x, tau, lengths)
    (gx,) = torch.autograd.grad(P, x, G)
    return P.detach(), gx


@pytest.mark.parametrize("B,L1,L2,tau,ragged", [(32, 1024, 1024, 1.0, False), (9, 700, 600, 0.7, True)])
def test_bidirectional_softmax_graph_replays(B, L1, L2, tau, ragged):
    print(f"[graph] bidi B={B} L1={L1} L2={L2} ragged={ragged}", flush=True)
    rng = np.random.default_rng(B + L1)
    lengths = None
    if ragged:
        ln = np.stack([rng.integers(L1 // 2, L1 + 1, B), rng.integers(L2 // 2, L2 + 1, B)], 1).astype(np.int32)
        ln[0] = (L1, L2)
        lengths = torch.as_tensor(ln).to(DEV)
    inputs = [(torch.as_tensor(rng.standard_normal((B, L1, L2)).astype(np.float32)),
               torch.as_tensor(rng.standard_normal((B, L1, L2)).astype(np.float32))) for _ in range(3)]
    s_sim = inputs[0][0].to(DEV)
    s_G = inputs[0][1].to(DEV)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            _bidi_step(s_sim, s_G, tau, lengths)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        s_P, s_g = _bidi_step(s_sim, s_G, tau, lengths)
    for k, (sim, G) in enumerate(inputs[1:] + inputs[:1]):
        s_sim.copy_(sim.to(DEV))
        s_G.copy_(G.to(DEV))
        graph.replay()
        torch.cuda.synchronize()
        # the program's own eager calls between the replays, on the same stream
        P_e, g_e = _bidi_step(sim.to(DEV), G.to(DEV), tau, lengths)
        torch.cuda.synchronize()
        assert torch.equal(s_P, P_e) and torch.equal(s_g, g_e), k
        if k < 2 or B < 32:  # the float64 oracle at C2 size takes seconds: two replays
            ln_np = lengths.cpu().numpy() if lengths is not None else np.tile([[L1, L2]], (B, 1)).astype(np.int32)
            out, r, c = obs.forward(sim.numpy(), tau, ln_np)
            gs, _ = obs.backward(sim.numpy(), out, G.numpy(), r, c, tau, ln_np)
            assert rel_err(s_P, out) < FWD_TOL, k
            assert rel_err(s_g, gs) < GRAD_TOL, k


def _sk_step(C, G, tau, T, BT, tol):
    """Fused Sinkhorn forward (cost kind) and implicit adjoint, device outputs only."""
    P, cost, counts, _, _ = _ops.fused.sinkhorn_forward(C, -1, tau, T, tol, None, None, True, False)
    grad, gtau, status = _ops.fused.sinkhorn_backward(C, -1, P, G, None, tau, 0, BT, None, None)
    return P, cost, counts, grad, gtau


@pytest.mark.parametrize("tier,B,M,N,tau,T,tol", [
    ("resident", 8, 256, 256, 0.2, 60, 1e-6),
    ("persistent", 2, 300, 2048, 0.3, 30, 0.0),
])
def test_sinkhorn_graph_replays(tier, B, M, N, tau, T, tol):
    print(f"[graph] sinkhorn {tier} B={B} M={M} N={N}", flush=True)
    rng = np.random.default_rng(M + N)
    inputs = [(torch.as_tensor(rng.random((B, M, N)).astype(np.float32)),
               torch.as_tensor(rng.standard_normal((B, M, N)).astype(np.float32))) for _ in range(3)]
    s_C = inputs[0][0].to(DEV)
    s_G = inputs[0][1].to(DEV)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            _sk_step(s_C, s_G, tau, T, T, tol)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = _sk_step(s_C, s_G, tau, T, T, tol)
    for k, (C, G) in enumerate(inputs[1:] + inputs[:1]):
        s_C.copy_(C.to(DEV))
        s_G.copy_(G.to(DEV))
        graph.replay()
        torch.cuda.synchronize()
        eager = _sk_step(C.to(DEV), G.to(DEV), tau, T, T, tol)
        torch.cuda.synchronize()
        for a, e in zip(outs, eager):
            assert torch.equal(a, e), k
        used = int(outs[2][0])
        Po, go, _ = osk.with_grads_implicit(-C.numpy(), G.numpy(), tau, used, T)
        assert rel_err(outs[0], Po) < FWD_TOL, k
        assert rel_err(outs[3], -go) < GRAD_TOL, k
