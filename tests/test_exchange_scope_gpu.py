"""Exchange-store scope of the one-launch kernels.

On gfx950 the register-resident and persistent Sinkhorn kernels and the
one-pass bidirectional softmax let an exchange word stop in the writer's XCD
L2 when every reader runs on that XCD (workgroup-scope stores read by
agent-scope loads, checked per launch by the XCC ids the workgroups
announce).  DOT_AMD_AGENT_SCOPE=1 keeps every exchange store at agent scope.
The scope changes only where a word is visible from, never the arithmetic or
its order, so both settings must give the same bits.
"""

import numpy as np
import pytest
import torch

import dot_amd

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)


def _both_scopes(monkeypatch, fn):
    out = {}
    for mode in ("default", "agent"):
        if mode == "agent":
            monkeypatch.setenv("DOT_AMD_AGENT_SCOPE", "1")
        out[mode] = fn()
        torch.cuda.synchronize()
        monkeypatch.delenv("DOT_AMD_AGENT_SCOPE", raising=False)
    return out["default"], out["agent"]


@pytest.mark.parametrize("tier,B,M,N,tau,T,tol,mode", [
    ("resident", 8, 512, 512, 0.1, 100, 1e-6, "implicit"),
    ("persistent", 2, 300, 2048, 0.3, 30, 0.0, "implicit"),
    ("persistent", 2, 300, 2048, 0.3, 12, 0.0, "unrolled"),
])
def test_sinkhorn_bits_do_not_depend_on_the_store_scope(tier, B, M, N, tau, T, tol, mode, monkeypatch):
    print(f"[scope] sinkhorn {tier} {mode} B={B} M={M} N={N}", flush=True)
    rng = np.random.default_rng(B + M + N)
    C = torch.as_tensor(rng.random((B, M, N)).astype(np.float32)).to(DEV)
    if tier == "persistent":
        monkeypatch.setenv("DOT_AMD_RESIDENT", "0")

    def run():
        leaf = C.clone().requires_grad_(True)
        res = dot_amd.sinkhorn(leaf, reg=tau, n_iters=T, tol=tol, backward_mode=mode)
        res.cost.sum().backward()
        return res.transport_plan.detach(), res.cost.detach(), leaf.grad, res.n_iters_used

    d, a = _both_scopes(monkeypatch, run)
    assert d[3] == a[3]
    for x, y in zip(d[:3], a[:3]):
        assert torch.equal(x, y)


@pytest.mark.parametrize("B,L1,L2,ragged", [(16, 1024, 1024, False), (9, 700, 600, True)])
def test_onepass_softmax_bits_do_not_depend_on_the_store_scope(B, L1, L2, ragged, monkeypatch):
    print(f"[scope] bidi B={B} L1={L1} L2={L2} ragged={ragged}", flush=True)
    rng = np.random.default_rng(B + L1 + L2)
    sim = torch.as_tensor(rng.standard_normal((B, L1, L2)).astype(np.float32)).to(DEV)
    G = torch.as_tensor(rng.standard_normal((B, L1, L2)).astype(np.float32)).to(DEV)
    lengths = None
    if ragged:
        ln = np.stack([rng.integers(L1 // 2, L1 + 1, B), rng.integers(L2 // 2, L2 + 1, B)], 1).astype(np.int32)
        lengths = torch.as_tensor(ln).to(DEV)

    def run():
        x = sim.clone().requires_grad_(True)
        P = dot_amd.bidirectional_softmax(x, 0.8, lengths)
        P.backward(G)
        return P.detach(), x.grad

    d, a = _both_scopes(monkeypatch, run)
    for x, y in zip(d, a):
        assert torch.equal(x, y)
