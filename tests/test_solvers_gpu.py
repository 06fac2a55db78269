"""GPU: the reference's PyTorch-level solvers on HIP tensors — ``dual=False``
momentum, Anderson, Adam and scheduled plain Sinkhorn, and Newton and Muon
(which have no fused device path in the reference either).  Their iterations
are ATen calls on the device; Muon's inner plain runs and every solver's
backward are this package's HIP operators (``torch.ops.dot.sinkhorn``,
``sinkhorn_with_grads_implicit``).

Each case is compared with the same call on CPU tensors (whose operators are
pinned to the reference's golden vectors): plans 1e-5 norm-wise, gradients
1e-4, iteration counts within one.
"""

from unittest import mock

import numpy as np
import pytest
import torch

import dot_amd
from dot_amd import _ops, solvers
from conftest import rel_err
from oracle import solvers as osv

pytestmark = pytest.mark.gpu
DEV = "cuda"
FWD_TOL, GRAD_TOL = 1e-5, 1e-4


def _grid(n, weight=3.0):
    g = torch.linspace(-1.0, 1.0, n)
    c = (g[:, None] - g[None, :]).abs().pow(2) * torch.linspace(1.0, weight, n).unsqueeze(0)
    return c.unsqueeze(0)


CASES = [
    ("momentum", dict(method="momentum", omega=1.4, dual=False), 0.05, 120),
    ("momentum_auto_omega", dict(method="momentum", dual=False), 0.05, 120),
    ("anderson", dict(method="anderson", anderson_k=5, dual=False), 0.1, 60),
    ("adam", dict(method="adam", lr=0.5, dual=False), 0.1, 80),
    ("rmsprop", dict(method="adam", lr=0.25, beta1=0.0, bias_correction=False, dual=False), 0.02, 20),
    ("scheduled", dict(schedule="cosine", reg_start=0.5, dual=False), 0.05, 60),
    ("newton", dict(method="newton"), 0.1, 8),
    ("auto", dict(method="auto"), 0.1, 8),
    ("muon", dict(method="muon", lr=0.05), 0.1, 3),
]


@pytest.mark.parametrize("name,kw,tau,iters", CASES, ids=[c[0] for c in CASES])
def test_solver_on_device_matches_cpu(name, kw, tau, iters):
    torch.manual_seed(7)
    C = torch.rand(2, 12, 10) if name not in ("rmsprop",) else _grid(16).expand(2, -1, -1).contiguous()
    W = torch.rand_like(C)
    print(f"[solvers_gpu] {name} shape={tuple(C.shape)} tau={tau} iters={iters}", flush=True)
    out = {}
    for dev in ("cpu", DEV):
        c = C.detach().to(dev).clone().requires_grad_(True)
        r = dot_amd.sinkhorn(c, reg=tau, n_iters=iters, **kw)
        ((r.transport_plan * W.to(dev)).sum() + r.cost.sum()).backward()
        out[dev] = (r.transport_plan.detach().cpu(), r.cost.detach().cpu(), r.n_iters_used, c.grad.cpu())
    P, cost, used, grad = out[DEV]
    Pc, costc, usedc, gradc = out["cpu"]
    # the solvers' fixed stop tests (1e-6; 1e-8 for Newton) sit at the float32
    # rounding floor of potentials of size ~10, so where the largest change
    # first drops below them is rounding, not algorithm (the momentum case
    # stops at 37 on the CPU and 41 on the GPU; float32 vs float64 on the CPU
    # alone gives 34 vs 35 for Anderson); the fixed-count trajectories are
    # compared in test_solver_trajectory_on_device_matches_cpu
    assert 1 <= used <= iters + (5 if name == "muon" else 0)
    assert rel_err(P, Pc) < FWD_TOL
    assert rel_err(cost, costc) < FWD_TOL
    assert torch.isfinite(P).all()
    # the reference's backward is the plain implicit adjoint at n_iters_used
    # (sinkhorn.py:361-380), so the device gradient is checked against the CPU
    # operator at the device's own count: P + adjoint applied to (W + C)
    _, g_la, _ = _ops.sinkhorn_with_grads_implicit(-C, (W + C).contiguous(), tau, used, iters, None, None)
    assert rel_err(grad, P - g_la) < GRAD_TOL
    if used == usedc:
        assert rel_err(grad, gradc) < GRAD_TOL


def test_newton_marginals_on_device():
    torch.manual_seed(3)
    C = torch.rand(3, 9, 7, device=DEV)
    a = torch.rand(9, device=DEV) + 0.2
    a = a / a.sum()
    b = torch.rand(3, 7, device=DEV) + 0.2
    b = b / b.sum(-1, keepdim=True)
    r = dot_amd.sinkhorn(C, reg=0.1, n_iters=10, a=a, b=b, method="newton")
    assert r.transport_plan.is_cuda
    assert torch.allclose(r.transport_plan.sum(-1), a.expand(3, -1), atol=1e-5)
    assert torch.allclose(r.transport_plan.sum(-2), b, atol=1e-5)


def test_reg_tensor_gradient_on_device():
    torch.manual_seed(4)
    C = torch.rand(2, 8, 8)
    grads = []
    for dev in ("cpu", DEV):
        reg = torch.tensor(0.2, device=dev, requires_grad=True)
        r = dot_amd.sinkhorn(C.to(dev), reg=reg, n_iters=40, method="anderson", dual=False)
        r.cost.sum().backward()
        assert reg.grad.device.type == torch.device(dev).type
        grads.append(float(reg.grad))
    assert grads[1] == pytest.approx(grads[0], rel=GRAD_TOL, abs=1e-7)


TRAJECTORIES = [
    ("momentum", solvers.momentum_forward, dict(omega=1.4, tol=0.0), 0.05, 40),
    ("anderson", solvers.anderson_forward, dict(anderson_k=5, mixing_beta=1.0, tol=0.0), 0.1, 25),
    ("adam", solvers.adam_forward, dict(lr=0.5, beta1=0.9, beta2=0.999, eps_adam=1e-8, bias_correction=True,
                                         tol=0.0), 0.1, 40),
    ("scheduled", solvers.scheduled_forward, dict(reg_start=0.5, schedule="exponential", tol=0.0), 0.05, 40),
    ("newton", solvers.newton_forward, dict(tol=0.0), 0.1, 4),
]


@pytest.mark.parametrize("name,fn,opts,tau,iters", TRAJECTORIES, ids=[t[0] for t in TRAJECTORIES])
def test_solver_trajectory_on_device_matches_cpu(name, fn, opts, tau, iters):
    """A fixed number of iterations (tol = 0) on both devices."""
    torch.manual_seed(11)
    la = -torch.rand(3, 11, 13)
    print(f"[solvers_gpu] trajectory {name} iters={iters}", flush=True)
    P, used = fn(la.to(DEV), tau, iters, None, None, **opts)
    Pc, usedc = fn(la, tau, iters, None, None, **opts)
    assert used == usedc == iters
    assert P.is_cuda and rel_err(P.cpu(), Pc) < FWD_TOL


# ---------------------------------------------------------------------------
# Newton and Muon on the device against oracle/solvers.py directly
# ---------------------------------------------------------------------------
ORACLE_CASES = [  # (B, n, m, tau, schedule, reg_start, marginals)
    (1, 12, 12, 0.1, None, None, False),
    (3, 9, 14, 0.05, None, None, True),
    (2, 10, 7, 0.02, "cosine", 0.2, True),
]


def _oracle_inputs(case, seed):
    """log_alpha and log marginals exactly representable in float32, so the
    float32 device run and the float64 oracle start from the same numbers."""
    B, n, m, tau, sched, start, marg = case
    rng = np.random.default_rng(seed)
    la = (-rng.random((B, n, m))).astype(np.float32).astype(np.float64)
    lga = lgb = None
    if marg:
        a, b = rng.random((B, n)) + 0.5, rng.random((B, m)) + 0.5
        lga = np.log(a / a.sum(1, keepdims=True)).astype(np.float32).astype(np.float64)
        lgb = np.log(b / b.sum(1, keepdims=True)).astype(np.float32).astype(np.float64)
    return la, lga, lgb, tau, sched, start


def _dev(x, dtype):
    return None if x is None else torch.from_numpy(np.ascontiguousarray(x)).to(DEV, dtype)


@pytest.mark.parametrize("case", ORACLE_CASES)
def test_newton_on_device_matches_oracle(case):
    """sinkhorn.py:1156-1256 on HIP tensors: in float64 the device trajectory
    (the per-element dense solves, the six halvings, the rebalancing) equals
    the oracle's to 1e-9 at every count; in float32, the product dtype, the
    converged plan agrees to the 1e-5 plan tolerance."""
    la, lga, lgb, tau, sched, start = _oracle_inputs(case, 14)
    print(f"[solvers_gpu] newton vs oracle case={case}", flush=True)
    for T in (1, 3, 12):
        P, used = solvers.newton_forward(_dev(la, torch.float64), tau, T, _dev(lga, torch.float64),
                                         _dev(lgb, torch.float64), start, sched)
        Po, uo = osv.newton(la, tau, T, lga, lgb, start, sched)
        assert P.is_cuda and used == uo and rel_err(P.cpu(), Po) < 1e-9, T
    P, used = solvers.newton_forward(_dev(la, torch.float32), tau, 30, _dev(lga, torch.float32),
                                     _dev(lgb, torch.float32), start, sched)
    Po, uo = osv.newton(la, tau, 30, lga, lgb, start, sched)
    assert P.dtype == torch.float32 and rel_err(P.cpu(), Po) < FWD_TOL


def _plain64(log_alpha, tau, iters, log_a, log_b):
    """The plain operator in float64 torch on the input's device (the product
    operator computes in float32), to compare Muon's own arithmetic exactly."""
    K = log_alpha / tau
    u = log_alpha.new_zeros(log_alpha.shape[:2])
    v = log_alpha.new_zeros((log_alpha.shape[0], log_alpha.shape[2]))
    for _ in range(iters):
        u, v = solvers.fixed_point_map(u, v, K, log_a, log_b)
    return (K + u.unsqueeze(-1) + v.unsqueeze(-2)).exp()


@pytest.mark.parametrize("case", ORACLE_CASES)
def test_muon_on_device_matches_oracle(case):
    """sinkhorn.py:1119-1153 on HIP tensors.  Muon divides by the plan's
    entries, so its trajectory amplifies rounding: with a float64 inner
    operator the device run equals the oracle to 1e-9 over 3 steps; with the
    product's float32 HIP operator one step agrees to 1e-4."""
    la, lga, lgb, tau, sched, start = _oracle_inputs(case, 15)
    print(f"[solvers_gpu] muon vs oracle case={case}", flush=True)
    with mock.patch.object(solvers._ops, "sinkhorn", _plain64):
        for lr, T in ((0.05, 3), (0.5, 3), (0.05, 1)):
            P, used = solvers.muon_forward(_dev(la, torch.float64), tau, T, _dev(lga, torch.float64),
                                           _dev(lgb, torch.float64), lr, start, sched)
            Po, uo = osv.muon(la, tau, T, lr, lga, lgb, start, sched)
            assert P.is_cuda and used == uo and rel_err(P.cpu(), Po) < 1e-9, (lr, T)
    P, used = solvers.muon_forward(_dev(la, torch.float32), tau, 1, _dev(lga, torch.float32),
                                   _dev(lgb, torch.float32), 0.05, start, sched)
    Po, uo = osv.muon(la, tau, 1, 0.05, lga, lgb, start, sched)
    assert used == uo and rel_err(P.cpu(), Po) < 1e-4
