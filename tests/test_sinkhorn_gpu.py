"""GPU parity of the Sinkhorn path: HIP kernels against the oracle and the golden fixtures.

Tolerances (norm-wise relative, max|a - e| / max|e|): plan and cost 1e-5,
gradients 1e-4.  grad_tau, a sum with heavy
cancellation, is judged against the magnitude of its terms (conftest.sum_err).
Comparisons of early-stopped runs use the oracle at the HIP run's own
n_iters_used with tol = 0: fp32 and float64 can cross the tolerance one
iteration apart.
"""

import ctypes
import os

import numpy as np
import pytest
import torch

import dot_amd
from dot_amd import _ops
from conftest import ROOT, load_golden, rel_err, sum_err
from oracle import sinkhorn as osk

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)
FWD_TOL, GRAD_TOL = 1e-5, 1e-4


def _t(x):
    return torch.as_tensor(np.ascontiguousarray(x)).to(DEV)


def _dirichlet(rng, B, n):
    e = -np.log(rng.random((B, n)))
    return (e / e.sum(1, keepdims=True)).astype(np.float32)


def test_native_library_is_loaded():
    maps = open("/proc/self/maps").read()
    assert "libdot_amd.so" in maps and "_C.so" in maps
    assert _ops._extension_loaded


# ---------------------------------------------------------------------------
# Golden fixtures of the reference through the drop-in torch.ops.dot operators
# ---------------------------------------------------------------------------
def test_ops_forward_golden_6x9():
    g = load_golden("sk_fwd_6x9")
    la, lga, lgb = _t(g["log_alpha"]), _t(g["log_a"]), _t(g["log_b"])
    tau, T = float(g["tau"]), int(g["n_iters"])
    P, used, conv = _ops.sinkhorn_dual_forward(la, tau, T, 0.0, lga, lgb)
    assert used.device.type == "cpu" and int(used) == T and int(conv) == 0
    assert rel_err(P, g["P"]) < FWD_TOL
    logP, _, _ = _ops.sinkhorn_dual_forward(la, tau, T, 0.0, lga, lgb, True)
    assert (logP.cpu().numpy() - g["logP"]).__abs__().max() < 1e-4
    assert rel_err(_ops.sinkhorn(la, tau, T, lga, lgb), g["P"]) < FWD_TOL
    assert (_ops.sinkhorn_log(la, tau, T, lga, lgb).cpu().numpy() - g["logP"]).__abs__().max() < 1e-4


def test_ops_c1_golden_forward_and_implicit():
    g = load_golden("sk_c1")
    C = g["cost"]
    P, grad, gtau = _ops.sinkhorn_with_grads_implicit(_t(-C), _t(C), float(g["tau"]),
                                                      int(g["n_iters"]), int(g["backward_iters"]))
    assert rel_err(P, g["P"]) < FWD_TOL
    assert rel_err(grad, g["grad_fixed"]) < GRAD_TOL
    assert sum_err(gtau, g["grad_tau_fixed"], grad.cpu().numpy() * -C / float(g["tau"])) < GRAD_TOL


def test_ops_small_reg_golden():
    g = load_golden("sk_fwd_smallreg")
    P = _ops.sinkhorn(_t(-g["cost"]), float(g["tau"]), int(g["n_iters"]))
    assert rel_err(P, g["P"]) < FWD_TOL


def test_ops_grads_golden_rectangular_nonuniform():
    g = load_golden("sk_grads_8x16")
    la, G, lga, lgb = _t(g["log_alpha"]), _t(g["grad_P"]), _t(g["log_a"]), _t(g["log_b"])
    tau, T, BT = float(g["tau"]), int(g["n_iters"]), int(g["backward_iters"])
    terms = lambda gr: gr.cpu().numpy() * g["log_alpha"] / tau  # noqa: E731
    P, gi, gti = _ops.sinkhorn_with_grads_implicit(la, G, tau, T, BT, lga, lgb)
    assert rel_err(P, g["P"]) < FWD_TOL
    assert rel_err(gi, g["grad_implicit"]) < GRAD_TOL
    assert sum_err(gti, g["grad_tau_implicit"], terms(gi)) < GRAD_TOL
    Pu, gu, gtu = _ops.sinkhorn_with_grads_unrolled(la, G, tau, T, lga, lgb)
    assert rel_err(Pu, g["P_unrolled"]) < FWD_TOL
    assert rel_err(gu, g["grad_unrolled"]) < GRAD_TOL
    assert sum_err(gtu, g["grad_tau_unrolled"], terms(gu)) < GRAD_TOL


def test_ops_unrolled_golden_48x64():
    g = load_golden("sk_unrolled_48x64")
    C = g["cost"]
    P, gu, gtu = _ops.sinkhorn_with_grads_unrolled(_t(-C), _t(C), float(g["tau"]), int(g["n_iters"]))
    assert rel_err(P, g["P"]) < FWD_TOL
    assert rel_err(gu, g["grad_unrolled"]) < GRAD_TOL
    assert sum_err(gtu, g["grad_tau_unrolled"], gu.cpu().numpy() * -C / float(g["tau"])) < GRAD_TOL


# ---------------------------------------------------------------------------
# Oracle parity across shapes and kernel variants
# ---------------------------------------------------------------------------
SHAPES = [
    # (B, M, N, tau, T, nonuniform)   N % 4 != 0 takes the scalar-load kernels
    (1, 1, 1, 1.0, 5, False),
    (3, 5, 7, 0.5, 30, True),
    (2, 64, 64, 1.0, 50, False),
    (2, 37, 250, 0.1, 40, True),
    (4, 200, 96, 0.2, 60, True),
    (1, 300, 1024, 0.05, 80, False),
    (2, 64, 2048, 0.1, 30, True),
    (1, 96, 4096, 0.1, 20, False),
    (1, 257, 4095, 0.3, 15, True),
    (5, 1000, 3, 1.0, 25, True),
]


@pytest.mark.parametrize("B,M,N,tau,T,nonuni", SHAPES)
def test_forward_and_implicit_match_oracle(B, M, N, tau, T, nonuni):
    rng = np.random.default_rng(B * 1000 + M + N)
    C = rng.random((B, M, N)).astype(np.float32)
    G = rng.standard_normal((B, M, N)).astype(np.float32)
    lga = lgb = None
    if nonuni:
        lga, lgb = np.log(_dirichlet(rng, B, M)), np.log(_dirichlet(rng, B, N))
    P, gi, gti = _ops.sinkhorn_with_grads_implicit(
        _t(-C), _t(G), tau, T, T, None if lga is None else _t(lga), None if lgb is None else _t(lgb))
    Po, go, gto = osk.with_grads_implicit(-C, G, tau, T, T, lga, lgb)
    assert rel_err(P, Po) < FWD_TOL
    assert rel_err(gi, go) < GRAD_TOL
    assert sum_err(gti, gto, go * -C / tau) < GRAD_TOL


@pytest.mark.parametrize("B,M,N,tau,T,nonuni", SHAPES[:8])
def test_unrolled_matches_oracle(B, M, N, tau, T, nonuni):
    rng = np.random.default_rng(B * 7 + M + N)
    C = rng.random((B, M, N)).astype(np.float32)
    G = rng.standard_normal((B, M, N)).astype(np.float32)
    lga = lgb = None
    if nonuni:
        lga, lgb = np.log(_dirichlet(rng, B, M)), np.log(_dirichlet(rng, B, N))
    T = min(T, 20)
    P, gu, gtu = _ops.sinkhorn_with_grads_unrolled(
        _t(-C), _t(G), tau, T, None if lga is None else _t(lga), None if lgb is None else _t(lgb))
    Po, go, gto = osk.with_grads_unrolled(-C, G, tau, T, lga, lgb)
    assert rel_err(P, Po) < FWD_TOL
    assert rel_err(gu, go) < GRAD_TOL
    assert sum_err(gtu, gto, go * -C / tau) < GRAD_TOL


@pytest.mark.parametrize("B,M,N,tau,T,nonuni", [(2, 300, 4096, 0.3, 12, True), (3, 64, 4096, 0.1, 25, False)])
def test_unrolled_rows_of_4096_persistent(B, M, N, tau, T, nonuni, monkeypatch):
    """Rows of 4096 floats: the persistent unrolled kernel streams each row in
    two halves (C5's shape).  Against the float64 oracle, and against the
    per-step sweeps (DOT_AMD_PERSISTENT=0) of the same arithmetic."""
    print(f"[sk_gpu] unrolled halves B={B} M={M} N={N} T={T}", flush=True)
    rng = np.random.default_rng(B * 31 + M)
    C = rng.random((B, M, N)).astype(np.float32)
    G = rng.standard_normal((B, M, N)).astype(np.float32)
    lga = lgb = None
    if nonuni:
        lga, lgb = np.log(_dirichlet(rng, B, M)), np.log(_dirichlet(rng, B, N))
    t = lambda x: None if x is None else _t(x)
    P, gu, gtu = _ops.sinkhorn_with_grads_unrolled(_t(-C), _t(G), tau, T, t(lga), t(lgb))
    Po, go, gto = osk.with_grads_unrolled(-C, G, tau, T, lga, lgb)
    assert rel_err(P, Po) < FWD_TOL
    assert rel_err(gu, go) < GRAD_TOL
    assert sum_err(gtu, gto, go * -C / tau) < GRAD_TOL
    monkeypatch.setenv("DOT_AMD_PERSISTENT", "0")
    P2, gu2, gtu2 = _ops.sinkhorn_with_grads_unrolled(_t(-C), _t(G), tau, T, t(lga), t(lgb))
    assert rel_err(gu, gu2.cpu().numpy()) < 1e-5
    assert torch.allclose(gtu, gtu2, rtol=1e-4, atol=1e-6)


@pytest.mark.parametrize("seed,shape,tau", [(0, (1, 256, 256), 0.1), (1, (4, 96, 128), 0.05),
                                            (2, (3, 40, 60), 0.5), (3, (2, 512, 300), 0.02)])
def test_early_stop_matches_oracle(seed, shape, tau):
    C = torch.rand(*shape, generator=torch.Generator().manual_seed(seed)).numpy()
    P, used, conv = _ops.sinkhorn_dual_forward(_t(-C), tau, 300, 1e-6)
    used, conv = int(used), int(conv)
    o = osk.dual_forward(-C, tau, 300, tol=1e-6)
    assert abs(used - o.n_iters_used) <= 1, (used, o.n_iters_used)
    if used < 300:
        assert conv == 1
    matched = osk.dual_forward(-C, tau, used)
    assert rel_err(P, matched.P) < FWD_TOL


@pytest.mark.parametrize("B,M,N", [(3, 64, 96), (2, 200, 1500), (5, 33, 17)])
def test_early_stop_count_convention_rank_one(B, M, N, monkeypatch):
    """A rank-one kernel is exact after iteration 1, so the u-change test fires
    at iteration 2 (used_iters = iter + 1 at the break, torch_cuda.cpp:223-236)
    on every tier: register-resident, persistent and per-iteration sweeps."""
    rng = np.random.default_rng(B * M + N)
    la = (rng.standard_normal((B, M, 1)) + rng.standard_normal((B, 1, N))).astype(np.float32)
    lga = np.log(_dirichlet(rng, B, M))
    lgb = np.log(_dirichlet(rng, B, N))
    Po = osk.dual_forward(la, 0.7, 2, log_a=lga, log_b=lgb).P
    runs = {"default": _ops.sinkhorn_dual_forward(_t(la), 0.7, 50, 1e-3, _t(lga), _t(lgb))}
    runs.update(_three_paths(monkeypatch, lambda: _ops.sinkhorn_dual_forward(
        _t(la), 0.7, 50, 1e-3, _t(lga), _t(lgb))))
    for name, (P, used, conv) in runs.items():
        assert int(used) == 2 and int(conv) == 1, (name, int(used))
        assert rel_err(P, Po) < FWD_TOL, name


def test_zero_iterations_and_degenerate_shapes():
    C = np.random.default_rng(0).random((2, 5, 6)).astype(np.float32)
    P, used, conv = _ops.sinkhorn_dual_forward(_t(-C), 0.5, 0, 1e-6)
    assert int(used) == 0 and int(conv) == 0
    assert rel_err(P, osk.dual_forward(-C, 0.5, 0).P) < FWD_TOL
    P, used, conv = _ops.sinkhorn_dual_forward(torch.zeros(0, 4, 4, device=DEV), 1.0, 10, 1e-6)
    assert P.shape == (0, 4, 4)
    _, g, gt = _ops.sinkhorn_with_grads_implicit(_t(-C), _t(C), 0.5, 0, 0)
    o = osk.dual_forward(-C, 0.5, 0)
    go, _, _ = osk.implicit_backward(-C, o.P, C, 0.5, 0)
    assert rel_err(g, go) < GRAD_TOL


def test_op_argument_errors():
    x = torch.rand(2, 4, 4, device=DEV)
    with pytest.raises(RuntimeError, match="tau must be > 0"):
        _ops.sinkhorn(x, 0.0, 5)
    with pytest.raises(RuntimeError, match="3D"):
        _ops.sinkhorn(x[0], 1.0, 5)
    with pytest.raises(RuntimeError, match="log_a must have shape"):
        _ops.sinkhorn(x, 1.0, 5, torch.zeros(2, 5, device=DEV))
    with pytest.raises(RuntimeError, match="grad_P must match"):
        _ops.sinkhorn_with_grads_implicit(x, torch.zeros(2, 4, 5, device=DEV), 1.0, 5, 5)
    with pytest.raises(RuntimeError, match="anderson_k"):
        _ops.sinkhorn_dual_forward(x, 1.0, 5, 0.0, None, None, False, 2, 1.5, 0)
    with pytest.raises(RuntimeError, match="method"):
        _ops.sinkhorn_dual_forward(x, 1.0, 5, 0.0, None, None, False, 7)


# ---------------------------------------------------------------------------
# Public API (fused autograd path)
# ---------------------------------------------------------------------------
def _oracle_cost_grads(C, tau, T, BT, a=None, b=None, W=None, mode="implicit"):
    """dL/dC for L = cost.sum() (+ sum(P * W)) as the reference composes it."""
    lga = None if a is None else np.log(a)
    lgb = None if b is None else np.log(b)
    G = C.copy() if W is None else C + W
    if mode == "implicit":
        f = osk.dual_forward(-C, tau, T, 0.0, lga, lgb)
        gla, gt, _ = osk.implicit_backward(-C, f.P, G, tau, BT)
    else:
        f = osk.dual_forward(-C, tau, T, 0.0, lga, lgb, keep_history=True)
        gla, gt = osk.unrolled_backward(-C, f.P, G, f.K, f.u_hist, f.v_hist, tau)
    return f.P, (f.P * C).sum((1, 2)), f.P - gla, gt, gla


@pytest.mark.parametrize("mode", ["implicit", "unrolled"])
def test_api_plan_cost_and_cost_gradient(mode):
    rng = np.random.default_rng(11)
    C = rng.random((3, 48, 80)).astype(np.float32)
    a, b = _dirichlet(rng, 3, 48), _dirichlet(rng, 3, 80)
    leaf = _t(C).requires_grad_(True)
    res = dot_amd.sinkhorn(leaf, reg=0.3, n_iters=40, backward_mode=mode, a=_t(a), b=_t(b), tol=0)
    res.cost.sum().backward()
    P, cost, dC, _, _ = _oracle_cost_grads(C, 0.3, 40, 40, a, b, mode=mode)
    assert res.n_iters_used == 40 and res.converged is True
    assert rel_err(res.transport_plan, P) < FWD_TOL
    assert rel_err(res.cost, cost) < FWD_TOL
    assert rel_err(leaf.grad, dC) < GRAD_TOL


def test_api_gradient_through_plan_and_cost():
    rng = np.random.default_rng(12)
    C = rng.random((2, 30, 20)).astype(np.float32)
    W = rng.standard_normal((2, 30, 20)).astype(np.float32)
    leaf = _t(C).requires_grad_(True)
    res = dot_amd.sinkhorn(leaf, reg=0.5, n_iters=60, tol=0)
    (res.cost.sum() + (res.transport_plan * _t(W)).sum()).backward()
    _, _, dC, _, _ = _oracle_cost_grads(C, 0.5, 60, 60, W=W)
    assert rel_err(leaf.grad, dC) < GRAD_TOL


def test_api_reg_tensor_gradient():
    rng = np.random.default_rng(13)
    C = rng.random((2, 16, 24)).astype(np.float32)
    reg = torch.tensor(0.4, device=DEV, requires_grad=True)
    leaf = _t(C).requires_grad_(True)
    res = dot_amd.sinkhorn(leaf, reg=reg, n_iters=50, tol=0)
    res.cost.sum().backward()
    _, _, _, gt, gla = _oracle_cost_grads(C, 0.4, 50, 50)
    assert reg.grad is not None
    assert sum_err(reg.grad.reshape(1), np.array([gt.sum()]), (gla * -C / 0.4).reshape(1, -1)) < GRAD_TOL


def test_api_early_stop_and_result_fields():
    C = torch.rand(2, 128, 128, generator=torch.Generator().manual_seed(5))
    leaf = C.to(DEV).requires_grad_(True)
    res = dot_amd.sinkhorn(leaf, reg=0.1, n_iters=200)  # default tol 1e-6
    assert isinstance(res, dot_amd.SinkhornResult)
    assert isinstance(res.n_iters_used, int) and res.n_iters_used < 200 and res.converged is True
    res.cost.sum().backward()
    P, _, dC, _, _ = _oracle_cost_grads(C.numpy(), 0.1, res.n_iters_used, 200)
    assert rel_err(res.transport_plan, P) < FWD_TOL
    assert rel_err(leaf.grad, dC) < GRAD_TOL


def test_api_unbatched_alias_and_modules():
    C = torch.rand(24, 40, generator=torch.Generator().manual_seed(6))
    r1 = dot_amd.sinkhorn(C.to(DEV), reg=0.5, max_iter=30, tol=0)
    r2 = dot_amd.Sinkhorn(reg=0.5, max_iter=30)(C.to(DEV))
    P = osk.dual_forward(-C.numpy()[None], 0.5, 30).P[0]
    assert r1.transport_plan.shape == (24, 40) and r1.cost.shape == ()
    assert rel_err(r1.transport_plan, P) < FWD_TOL
    assert r2.transport_plan.shape == (24, 40)
    la = torch.randn(2, 8, 8, generator=torch.Generator().manual_seed(7))
    Q = dot_amd.SinkhornFromScores(tau=0.7, n_iters=25)(la.to(DEV))
    assert Q.shape == (2, 8, 8)
    Q0 = dot_amd.sinkhorn_from_scores(la.to(DEV), tau=0.7, n_iters=25, tol=0)
    assert rel_err(Q0, osk.dual_forward(la.numpy(), 0.7, 25).P) < FWD_TOL
    logQ = dot_amd.sinkhorn_from_scores(la.to(DEV), tau=0.7, n_iters=25, tol=0, return_log=True)
    assert (logQ.cpu().numpy() - osk.dual_forward(la.numpy(), 0.7, 25, return_log=True).P).__abs__().max() < 1e-4


def test_from_scores_gradient():
    rng = np.random.default_rng(14)
    la = rng.standard_normal((2, 10, 12)).astype(np.float32)
    W = rng.standard_normal((2, 10, 12)).astype(np.float32)
    x = _t(la).requires_grad_(True)
    P = dot_amd.sinkhorn_from_scores(x, tau=0.8, n_iters=40, tol=0)
    (P * _t(W)).sum().backward()
    f = osk.dual_forward(la, 0.8, 40)
    g, _, _ = osk.implicit_backward(la, f.P, W, 0.8, 40)
    assert rel_err(x.grad, g) < GRAD_TOL


def test_dual_false_is_the_fixed_count_path():
    C = torch.rand(1, 96, 128, generator=torch.Generator().manual_seed(0)).to(DEV)
    dual = dot_amd.sinkhorn(C, reg=0.1, n_iters=50, tol=0, dual=True)
    full = dot_amd.sinkhorn(C, reg=0.1, n_iters=50, tol=0, dual=False)
    assert dual.n_iters_used == 50 and full.n_iters_used == 50
    assert torch.allclose(dual.transport_plan, full.transport_plan, atol=1e-5)
    # dual=False ignores tol (the reference's full-matrix op) and reports converged=False
    f2 = dot_amd.sinkhorn(C, reg=0.1, n_iters=50, dual=False)
    assert f2.n_iters_used == 50 and f2.converged is False


def test_api_errors():
    C = torch.rand(2, 6, 6, device=DEV)
    with pytest.raises(ValueError, match="anderson_k <= 64"):  # a ring longer than the kernels hold
        dot_amd.sinkhorn(C, method="anderson", anderson_k=100, n_iters=200, reg=0.02)
    with pytest.raises(ValueError, match="strictly positive"):
        dot_amd.sinkhorn(C, a=torch.zeros(6, device=DEV))
    with pytest.raises(ValueError, match="sum to 1"):
        dot_amd.sinkhorn(C, a=torch.full((6,), 0.5, device=DEV))
    with pytest.raises(ValueError, match="n_iters must be an int"):
        dot_amd.sinkhorn(C, n_iters="many")
    with pytest.raises(ValueError, match="only supports n, m <= 100"):
        dot_amd.sinkhorn(torch.rand(1, 101, 4, device=DEV), reg=0.02, method="newton")
    with pytest.raises(ValueError, match="only supports implicit"):
        dot_amd.sinkhorn(C, reg=0.02, method="adam", lr=0.5, dual=False, backward_mode="unrolled")
    with pytest.raises(ValueError):
        dot_amd.sinkhorn(C, backward_mode="sideways")


# ---------------------------------------------------------------------------
# The reference's own GPU tests (tests/test_sinkhorn.py), re-expressed
# ---------------------------------------------------------------------------
def _uniform(B, n):
    return torch.full((B, n), 1.0 / n, device=DEV)


def _assert_marginals(plan, a, b, atol=1e-3):
    assert torch.allclose(plan.sum(-1), a, atol=atol)
    assert torch.allclose(plan.sum(-2), b, atol=atol)


def _reference_from_scores(log_alpha, tau, n_iters):
    x = log_alpha / tau
    B, n, m = x.shape
    log_a = torch.full((B, n, 1), -np.log(n), device=x.device, dtype=x.dtype)
    log_b = torch.full((B, 1, m), -np.log(m), device=x.device, dtype=x.dtype)
    for _ in range(n_iters):
        x = x - torch.logsumexp(x, dim=-1, keepdim=True) + log_a
        x = x - torch.logsumexp(x, dim=-2, keepdim=True) + log_b
    return x.exp()


@pytest.mark.parametrize("n,m", [(10, 10), (8, 16)])
def test_reference_uniform_marginals(n, m):  # test_sinkhorn.py:144-183
    cost = torch.rand(2, n, m, device=DEV)
    res = dot_amd.sinkhorn(cost, reg=1.0)
    _assert_marginals(res.transport_plan, _uniform(2, n), _uniform(2, m))


def test_reference_nonuniform_marginals():  # :212-223
    cost = torch.rand(1, 8, 16, device=DEV)
    a = torch.tensor([[0.20, 0.10, 0.15, 0.15, 0.10, 0.10, 0.10, 0.10]], device=DEV)
    res = dot_amd.sinkhorn(cost, reg=1.0, n_iters=100, a=a, b=_uniform(1, 16))
    _assert_marginals(res.transport_plan, a, _uniform(1, 16))


def test_reference_backward_and_modes():  # :254-313
    cost = torch.rand(2, 8, 16, device=DEV)
    a = torch.softmax(torch.randn(2, 8, device=DEV), -1)
    b = torch.softmax(torch.randn(2, 16, device=DEV), -1)
    cu = cost.clone().requires_grad_(True)
    ru = dot_amd.sinkhorn(cu, reg=1.0, backward_mode="unrolled", a=a, b=b)
    ru.cost.sum().backward()
    ci = cost.clone().requires_grad_(True)
    ri = dot_amd.sinkhorn(ci, reg=1.0, backward_mode="implicit", a=a, b=b)
    ri.cost.sum().backward()
    assert cu.grad is not None and ci.grad is not None and cu.grad.shape == cost.shape
    assert torch.allclose(ru.transport_plan, ri.transport_plan, atol=1e-4)


def test_reference_differentiable_reg_finite_difference():  # :399-416
    cost = torch.eye(5, device=DEV).unsqueeze(0)
    eps = torch.tensor(0.2, requires_grad=True, device=DEV)
    res = dot_amd.sinkhorn(cost, reg=eps, n_iters=80)
    res.cost.sum().backward()
    analytic = eps.grad.item()
    d = 1e-3
    plus = dot_amd.sinkhorn(cost, reg=float(eps.detach() + d), n_iters=80).cost.sum().item()
    minus = dot_amd.sinkhorn(cost, reg=float(eps.detach() - d), n_iters=80).cost.sum().item()
    assert analytic > 0
    assert abs(analytic - (plus - minus) / (2 * d)) < 5e-2


def test_reference_large_rectangular_matches_torch():  # :763-773
    torch.manual_seed(0)
    cost = torch.rand(1, 320, 640, device=DEV)
    res = dot_amd.sinkhorn(cost, reg=0.1, n_iters=50)
    ref = _reference_from_scores(-cost.double(), 0.1, 50)
    assert torch.allclose(res.transport_plan.double(), ref, atol=2e-3)


def test_reference_very_large_square_marginals():  # :776-788
    torch.manual_seed(0)
    n = 1300
    cost = torch.rand(1, n, n, device=DEV)
    res = dot_amd.sinkhorn(cost, reg=0.1, n_iters=50)
    assert torch.isfinite(res.transport_plan).all()
    _assert_marginals(res.transport_plan, _uniform(1, n), _uniform(1, n), atol=2e-3)


def test_reference_unrolled_dual_matches_full():  # :806-823
    torch.manual_seed(0)
    dc = torch.rand(1, 48, 64, device=DEV, requires_grad=True)
    fc = dc.detach().clone().requires_grad_(True)
    d = dot_amd.sinkhorn(dc, reg=0.1, n_iters=30, tol=0, dual=True, backward_mode="unrolled")
    f = dot_amd.sinkhorn(fc, reg=0.1, n_iters=30, tol=0, dual=False, backward_mode="unrolled")
    d.cost.sum().backward()
    f.cost.sum().backward()
    assert d.n_iters_used == 30 and f.n_iters_used == 30
    assert torch.allclose(d.transport_plan, f.transport_plan, atol=1e-5)
    assert torch.allclose(dc.grad, fc.grad, atol=1e-4)


def test_reference_convergence_reduces_iterations():  # :826-839
    torch.manual_seed(0)
    cost = torch.rand(1, 256, 256, device=DEV)
    early = dot_amd.sinkhorn(cost, reg=0.1, n_iters=50)
    fixed = dot_amd.sinkhorn(cost, reg=0.1, n_iters=50, tol=0)
    assert early.n_iters_used is not None and early.n_iters_used < 50
    assert fixed.n_iters_used == 50
    assert torch.allclose(early.transport_plan, fixed.transport_plan, atol=2e-3)


# ---------------------------------------------------------------------------
# BASELINE.json configurations at full size
# ---------------------------------------------------------------------------
def _c3_cost():
    g = torch.Generator().manual_seed(3)
    x, y = torch.randn(64, 512, 64, generator=g), torch.randn(64, 512, 64, generator=g)
    C = torch.cdist(x.to(DEV), y.to(DEV)).square()
    return (C / C.amax(dim=(-2, -1), keepdim=True)).contiguous()


def test_config_c1_full_against_golden():
    g = load_golden("sk_c1")
    leaf = _t(g["cost"]).requires_grad_(True)
    res = dot_amd.sinkhorn(leaf, reg=1.0, n_iters=100, tol=0)
    res.cost.sum().backward()
    assert rel_err(res.transport_plan, g["P"]) < FWD_TOL
    assert rel_err(leaf.grad, g["P"] - g["grad_fixed"]) < GRAD_TOL


def test_config_c3_full_size():
    C = _c3_cost()
    leaf = C.clone().requires_grad_(True)
    res = dot_amd.sinkhorn(leaf, reg=0.1, n_iters=200)
    res.cost.sum().backward()
    T = res.n_iters_used
    P = res.transport_plan.detach()
    # size-independent properties on the whole batch
    assert torch.allclose(P.sum(-2), torch.full_like(P.sum(-2), 1 / 512), rtol=1e-4, atol=0)
    assert torch.allclose(res.cost.detach(), (P * C).sum((-2, -1)), rtol=1e-5)
    # dL/dlog_alpha = P - dC; after the final mu update its column sums vanish exactly
    # (in exact arithmetic): sum_i P (G - lambda - mu) = c - P^T lambda - mu * colsum(P) = 0
    grad_la = P - leaf.grad
    scale = grad_la.abs().sum(-2).amax()
    assert (grad_la.sum(-2).abs().amax() / scale) < 1e-3
    # parity with the oracle on two batch elements at the run's own iteration count
    Cn = C.cpu().numpy()
    for b in (0, 63):
        Pb, costb, dCb, _, _ = _oracle_cost_grads(Cn[b:b + 1], 0.1, T, 200)
        assert rel_err(P[b:b + 1], Pb) < FWD_TOL
        assert rel_err(res.cost[b:b + 1], costb) < FWD_TOL
        assert rel_err(leaf.grad[b:b + 1], dCb) < GRAD_TOL
    # bitwise reproducible
    leaf2 = C.clone().requires_grad_(True)
    res2 = dot_amd.sinkhorn(leaf2, reg=0.1, n_iters=200)
    res2.cost.sum().backward()
    assert torch.equal(res2.transport_plan, res.transport_plan) and torch.equal(leaf2.grad, leaf.grad)


def _column_sum_invariant(P, grad_C, tol=1e-3):
    """dL/dlog_alpha = P - dL/dC for L = cost.sum(); after the adjoint's final
    mu update its column sums vanish in exact arithmetic:
    sum_i P (G - lambda - mu) = c - P^T lambda - mu * colsum(P) = 0."""
    grad_la = P - grad_C
    scale = grad_la.abs().sum(-2).amax()
    return float(grad_la.sum(-2).abs().amax() / scale) < tol


def _tier_grad_parity(C1, a1, b1, tau, T, monkeypatch):
    """One batch element at its real shape, reg and marginals: plan, cost and
    cost gradient after exactly T forward iterations and T adjoint sweeps on the
    persistent tier and on the per-iteration sweeps, against the float64 oracle."""
    Po, costo, dCo, _, _ = _oracle_cost_grads(C1, tau, T, T, a1, b1)
    lt = lambda x: None if x is None else _t(x)

    def run():
        leaf = _t(C1).requires_grad_(True)
        res = dot_amd.sinkhorn(leaf, reg=tau, n_iters=T, tol=0, a=lt(a1), b=lt(b1))
        res.cost.sum().backward()
        assert res.n_iters_used == T
        return res.transport_plan.detach(), res.cost.detach(), leaf.grad

    for name, (P, cost, g) in _three_paths(monkeypatch, run).items():
        assert rel_err(P, Po) < FWD_TOL, name
        assert rel_err(cost, costo) < FWD_TOL, name
        assert rel_err(g, dCo) < GRAD_TOL, (name, rel_err(g, dCo))
        assert _column_sum_invariant(P, g), name


def test_config_c4_full_size(monkeypatch):
    g = torch.Generator().manual_seed(4)
    C = torch.rand(16, 1024, 2048, generator=g)
    ea, eb = -torch.log(torch.rand(16, 1024, generator=g)), -torch.log(torch.rand(16, 2048, generator=g))
    a, b = ea / ea.sum(-1, keepdim=True), eb / eb.sum(-1, keepdim=True)
    leaf = C.to(DEV).requires_grad_(True)
    res = dot_amd.sinkhorn(leaf, reg=0.05, n_iters=500, a=a.to(DEV), b=b.to(DEV))
    res.cost.sum().backward()
    P = res.transport_plan.detach()
    assert torch.isfinite(P).all() and torch.isfinite(leaf.grad).all()
    assert torch.allclose(P.sum(-2), b.to(DEV), rtol=1e-4, atol=1e-9)
    if res.converged:
        assert torch.allclose(P.sum(-1), a.to(DEV), rtol=1e-3, atol=1e-8)
    # the 500-sweep adjoint at reg 0.05 on the whole batch: exact column-sum invariant
    assert _column_sum_invariant(P, leaf.grad)
    # parity at the real shape, reg and Dirichlet marginals, 100 + 100 sweeps, both tiers
    _tier_grad_parity(C[:1].numpy(), a[:1].numpy(), b[:1].numpy(), 0.05, 100, monkeypatch)


def test_config_c5_full_size(monkeypatch):
    g = torch.Generator().manual_seed(5)
    x, y = torch.randn(4, 4096, 128, generator=g), torch.randn(4, 4096, 128, generator=g)
    C = torch.cdist(x.to(DEV), y.to(DEV))
    C = (C / C.amax(dim=(-2, -1), keepdim=True)).contiguous()
    leaf = C.clone().requires_grad_(True)
    res = dot_amd.sinkhorn(leaf, reg=0.02, n_iters=1000)
    res.cost.sum().backward()
    P = res.transport_plan.detach()
    assert torch.isfinite(P).all() and torch.isfinite(leaf.grad).all()
    assert torch.allclose(P.sum(-2), torch.full_like(P.sum(-2), 1 / 4096), rtol=1e-4, atol=0)
    assert torch.allclose(P.sum((-2, -1)), torch.ones(4, device=DEV), rtol=1e-4)
    # the 1000-sweep adjoint at reg 0.02 on the whole batch: exact column-sum invariant
    assert _column_sum_invariant(P, leaf.grad)
    # parity at the real shape and reg, 30 + 30 sweeps, one element, both tiers
    _tier_grad_parity(C[:1].cpu().numpy(), None, None, 0.02, 30, monkeypatch)


@pytest.mark.parametrize("B,M,N,tau,T", [(8, 64, 64, 1.0, 100), (4, 512, 512, 0.1, 150),
                                         (3, 130, 70, 0.5, 40), (2, 1000, 1024, 0.2, 30),
                                         (1, 2048, 256, 0.3, 20)])
def test_resident_and_streaming_adjoints_agree_with_oracle(B, M, N, tau, T, monkeypatch):
    """The register-resident adjoint (one cooperative launch) and the streaming
    sweeps (one launch pair per sweep) against the oracle on the same inputs."""
    rng = np.random.default_rng(M + N)
    C = rng.random((B, M, N)).astype(np.float32)
    G = rng.standard_normal((B, M, N)).astype(np.float32)
    Po, go, gto = osk.with_grads_implicit(-C, G, tau, T, T)
    out = {}
    for mode in ("1", "0"):
        monkeypatch.setenv("DOT_AMD_RESIDENT", mode)
        P, g, gt = _ops.sinkhorn_with_grads_implicit(_t(-C), _t(G), tau, T, T)
        assert rel_err(P, Po) < FWD_TOL
        assert rel_err(g, go) < GRAD_TOL, mode
        assert sum_err(gt, gto, go * -C / tau) < GRAD_TOL
        out[mode] = g
    assert rel_err(out["1"], out["0"].cpu().numpy()) < 1e-5


def _both_paths(monkeypatch, fn):
    """fn() with the register-resident kernels allowed ("1") and disabled ("0")."""
    out = {}
    for mode in ("1", "0"):
        monkeypatch.setenv("DOT_AMD_RESIDENT", mode)
        out[mode] = fn()
    monkeypatch.delenv("DOT_AMD_RESIDENT")
    return out


@pytest.mark.parametrize("B,M,N,tau,T,tol,nonuni", [
    (8, 64, 64, 1.0, 50, 0.0, False),
    (16, 512, 512, 0.1, 200, 1e-6, False),
    (4, 96, 128, 0.05, 300, 1e-6, True),
    (3, 130, 70, 0.5, 40, 0.0, True),
    (2, 1000, 1024, 0.2, 20, 0.0, False),
    (5, 300, 257, 0.3, 60, 1e-5, True),
    (1, 7, 3, 0.7, 25, 1e-6, True),
])
def test_resident_and_streaming_forwards_agree_with_oracle(B, M, N, tau, T, tol, nonuni, monkeypatch):
    """The register-resident forward (one cooperative launch, lagged on-device
    stop test) and the streaming sweeps against the oracle, each at its own
    iteration count.  The two fp32 paths stop within one iteration of each
    other; the float64 oracle may stop earlier, where the fp32 change of u sits
    at its rounding floor near tol (|u| ~ 10 has an ulp of 1e-6)."""
    rng = np.random.default_rng(B * M + N)
    C = rng.random((B, M, N)).astype(np.float32)
    lga = np.log(_dirichlet(rng, B, M)) if nonuni else None
    lgb = np.log(_dirichlet(rng, B, N)) if nonuni else None
    args = (_t(-C), tau, T, tol, None if lga is None else _t(lga), None if lgb is None else _t(lgb))
    res = _both_paths(monkeypatch, lambda: _ops.sinkhorn_dual_forward(*args))
    counts = {mode: int(r[1]) for mode, r in res.items()}
    assert abs(counts["1"] - counts["0"]) <= 1, counts
    for mode, (P, used, conv) in res.items():
        used = int(used)
        assert int(conv) == (1 if tol > 0 and used < T else 0) or (tol > 0 and used == T), (mode, used)
        Po = osk.dual_forward(-C, tau, used, log_a=lga, log_b=lgb).P
        assert rel_err(P, Po) < FWD_TOL, mode
    if counts["1"] == counts["0"]:
        assert rel_err(res["1"][0], res["0"][0].cpu().numpy()) < 1e-5


_TIERS = (("resident", {}), ("persistent", {"DOT_AMD_RESIDENT": "0"}),
          ("sweeps", {"DOT_AMD_RESIDENT": "0", "DOT_AMD_PERSISTENT": "0"}))


def test_c3_stop_count_is_the_same_on_every_tier(monkeypatch):
    """n_iters_used is a function of the input, not of the tier the batch size
    selects: C3's input (seed 3, its first 16 elements, reg 0.1, tol 1e-6) on
    the register-resident tier, the persistent tier and the per-iteration
    sweeps stops within one iteration of both the float64 and the float32
    oracle (torch_cuda.cpp:199-238), and so does a batch of 300 (above the
    CUs, so the sweeps by shape) made of those 16 elements repeated, whose
    batch-global stop test sees the same maxima."""
    C = _c3_cost()[:16].contiguous()
    Cn = C.cpu().numpy()
    o64 = osk.dual_forward(-Cn, 0.1, 200, tol=1e-6).n_iters_used
    o32 = osk.dual_forward(-Cn, 0.1, 200, tol=1e-6, dtype=np.float32).n_iters_used
    print(f"[c3 stop] oracle float64 {o64} float32 {o32}", flush=True)
    counts = {}
    for name, env in _TIERS:
        for k, v in env.items():
            monkeypatch.setenv(k, v)
        res = dot_amd.sinkhorn(C, reg=0.1, n_iters=200, tol=1e-6)
        counts[name] = res.n_iters_used
        assert res.converged, name
        Po = osk.dual_forward(-Cn[:2], 0.1, res.n_iters_used).P
        assert rel_err(res.transport_plan[:2], Po) < FWD_TOL, name
        for k in env:
            monkeypatch.delenv(k)
    reps = C.repeat(19, 1, 1)[:300].contiguous()
    res = dot_amd.sinkhorn(reps, reg=0.1, n_iters=200, tol=1e-6)
    counts["B=300"] = res.n_iters_used
    Po = osk.dual_forward(-Cn[:2], 0.1, res.n_iters_used).P
    assert rel_err(res.transport_plan[16:18], Po) < FWD_TOL
    print(f"[c3 stop] counts {counts}", flush=True)
    for name, used in counts.items():
        assert abs(used - o64) <= 1 and abs(used - o32) <= 1, (name, counts, o64, o32)


def test_resident_forward_outputs_cost_log_and_history(monkeypatch):
    """Cost-kind scores with the transport cost, log-plan output and the
    per-iteration history of the unrolled mode, resident against streaming."""
    rng = np.random.default_rng(11)
    B, M, N, tau, T = 6, 200, 136, 0.25, 30
    C = _t(rng.random((B, M, N)).astype(np.float32))
    lga = _t(np.log(_dirichlet(rng, B, M)))
    fused = lambda: _ops.fused.sinkhorn_forward(C, -1, tau, T, 0.0, lga, None, True, True)
    res = _both_paths(monkeypatch, fused)
    torch.cuda.synchronize()  # the counts are pinned host words written by the kernels
    for i, name in enumerate(("plan", "cost", "counts", "u_hist", "v_hist")):
        a, b = res["1"][i], res["0"][i]
        if name == "counts":
            assert a.tolist() == b.tolist() == [T, 0]
        elif name.endswith("_hist"):
            # log-domain: the potentials of two fp32 paths that round differently
            # (the resident row update shifts by the last iteration's LSE, the
            # sweeps by the row maximum) agree to an absolute 1e-5, as each does
            # with the float64 oracle below
            assert (a - b).abs().max().item() < FWD_TOL, name
        else:
            assert rel_err(a, b.cpu().numpy()) < 1e-5, name
    o = osk.dual_forward(-C.cpu().numpy(), tau, T, log_a=lga.cpu().numpy(), keep_history=True)
    assert rel_err(res["1"][0], o.P) < FWD_TOL
    assert rel_err(res["1"][1], osk.transport_cost(o.P, C.cpu().numpy())) < FWD_TOL
    # dual potentials are log-domain: an absolute error e is a relative error e of P
    for i, hist in ((3, o.u_hist), (4, o.v_hist)):
        for mode in ("1", "0"):
            assert np.abs(res[mode][i].cpu().numpy() - hist).max() < FWD_TOL, (i, mode)
    logP = _both_paths(monkeypatch, lambda: _ops.sinkhorn_dual_forward(-C, tau, T, 0.0, lga, None, True))
    assert (logP["1"][0] - logP["0"][0]).abs().max().item() < 1e-4


def test_resident_forward_exact_column_fallback(monkeypatch):
    """A column far costlier than the rest underflows the shared-exponential
    column sum at small reg; both paths take the exact max-shifted LSE for it."""
    rng = np.random.default_rng(5)
    B, M, N, tau, T = 4, 160, 96, 0.01, 15
    C = (0.1 * rng.random((B, M, N))).astype(np.float32)
    C[:, :, 7] = 0.7   # exp(K - row max) <= exp(-60): the column sum is exactly 0 in fp32
    C[1, :, 50] = 0.8
    res = _both_paths(monkeypatch, lambda: _ops.sinkhorn_dual_forward(_t(-C), tau, T, 0.0))
    Po = osk.dual_forward(-C, tau, T).P
    for mode, (P, used, _) in res.items():
        assert int(used) == T
        assert torch.isfinite(P).all(), mode
        assert rel_err(P, Po) < FWD_TOL, mode


@pytest.mark.parametrize("B,M,N,tau,T,tol,b_range", [
    (4, 256, 384, 0.05, 60, 0.0, 30.0),
    (4, 256, 384, 0.05, 60, 0.0, 60.0),
    (3, 130, 70, 0.02, 40, 0.0, 60.0),
    (2, 1000, 1024, 0.2, 20, 1e-5, 45.0),
])
def test_resident_forward_wide_column_marginals(B, M, N, tau, T, tol, b_range, monkeypatch):
    """Column marginals b_j ~ exp(-b_range q_j) spread the dual potentials v
    over tens of nats from the first iteration on (and push some column sums
    under the exact-LSE floor); the resident forward against the oracle and
    against the streaming sweeps."""
    print(f"[sk_gpu] wide column marginals B={B} M={M} N={N} tau={tau} b_range={b_range}", flush=True)
    rng = np.random.default_rng(M + N + int(1000 * tau))
    C = rng.random((B, M, N)).astype(np.float32)
    lb = -b_range * rng.random((B, N))
    lgb = (lb - np.log(np.exp(lb).sum(1, keepdims=True))).astype(np.float32)
    args = (_t(-C), tau, T, tol, None, _t(lgb))
    res = _both_paths(monkeypatch, lambda: _ops.sinkhorn_dual_forward(*args))
    for mode, (P, used, _) in res.items():
        Po = osk.dual_forward(-C, tau, int(used), log_b=lgb).P
        assert rel_err(P, Po) < FWD_TOL, mode
    if int(res["1"][1]) == int(res["0"][1]):
        assert rel_err(res["1"][0], res["0"][0].cpu().numpy()) < 1e-5
    else:  # fp32 rounding at the stop threshold: one iteration apart at most
        assert abs(int(res["1"][1]) - int(res["0"][1])) <= 1


class SkFwdArgs(ctypes.Structure):
    _fields_ = [("scores", ctypes.c_void_p), ("log_a", ctypes.c_void_p), ("log_b", ctypes.c_void_p),
                ("B", ctypes.c_int), ("M", ctypes.c_int), ("N", ctypes.c_int),
                ("scores_kind", ctypes.c_int), ("tau", ctypes.c_float), ("max_iter", ctypes.c_int),
                ("tol", ctypes.c_float), ("flags", ctypes.c_int),
                ("plan", ctypes.c_void_p), ("cost", ctypes.c_void_p), ("u_out", ctypes.c_void_p),
                ("v_out", ctypes.c_void_p), ("u_hist", ctypes.c_void_p), ("v_hist", ctypes.c_void_p),
                ("iters_used", ctypes.c_void_p), ("converged", ctypes.c_void_p),
                ("workspace", ctypes.c_void_p), ("workspace_bytes", ctypes.c_size_t),
                ("exchange", ctypes.c_void_p), ("exchange_epoch", ctypes.c_uint32)]


class SkBwdArgs(ctypes.Structure):
    _fields_ = [("scores", ctypes.c_void_p), ("scores_kind", ctypes.c_int), ("plan", ctypes.c_void_p),
                ("grad_plan", ctypes.c_void_p), ("grad_cost", ctypes.c_void_p),
                ("B", ctypes.c_int), ("M", ctypes.c_int), ("N", ctypes.c_int), ("tau", ctypes.c_float),
                ("iters", ctypes.c_int), ("u_hist", ctypes.c_void_p), ("v_hist", ctypes.c_void_p),
                ("grad_scores", ctypes.c_void_p), ("grad_tau", ctypes.c_void_p),
                ("workspace", ctypes.c_void_p), ("workspace_bytes", ctypes.c_size_t),
                ("status", ctypes.c_void_p), ("exchange", ctypes.c_void_p), ("exchange_epoch", ctypes.c_uint32),
                ("sweeps_used", ctypes.c_void_p), ("flags", ctypes.c_int)]


@pytest.mark.parametrize("B,M,N,tau,T,tol", [(16, 512, 512, 0.1, 200, 1e-6), (6, 200, 136, 0.25, 30, 0.0),
                                            (8, 64, 64, 1.0, 40, 1e-6)])
def test_capi_exchange_words_match_the_workspace_path(B, M, N, tau, T, tol):
    """Through the C ABI: the register-resident forward and adjoint with
    caller-owned exchange words (epoch-tagged, never cleared by the library)
    give the bits of the workspace path (slots cleared per call), call after
    call; an epoch of 0 or above DOT_SINKHORN_MAX_EPOCH is rejected."""
    print(f"[sk_gpu] C ABI exchange words B={B} M={M} N={N} tol={tol}", flush=True)
    lib = ctypes.CDLL(os.path.join(ROOT, "dot_amd", "libdot_amd.so"))
    for f in ("dot_sinkhorn_exchange_bytes", "dot_sinkhorn_forward_workspace_bytes",
              "dot_sinkhorn_backward_implicit_workspace_bytes"):
        getattr(lib, f).restype = ctypes.c_size_t
    lib.dot_sinkhorn_forward.argtypes = [ctypes.POINTER(SkFwdArgs), ctypes.c_void_p]
    lib.dot_sinkhorn_backward_implicit.argtypes = [ctypes.POINTER(SkBwdArgs), ctypes.c_void_p]
    rng = np.random.default_rng(B + M + N)
    C = _t(rng.random((B, M, N)).astype(np.float32))
    G = _t(rng.standard_normal((B, M, N)).astype(np.float32))
    gc = _t(rng.random(B).astype(np.float32))
    ws = torch.empty(max(lib.dot_sinkhorn_forward_workspace_bytes(B, M, N, T, 0),
                         lib.dot_sinkhorn_backward_implicit_workspace_bytes(B, M, N)), dtype=torch.uint8, device=DEV)
    xw = torch.zeros(lib.dot_sinkhorn_exchange_bytes(), dtype=torch.uint8, device=DEV)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

    def run(exchange, epoch):
        P = torch.empty_like(C)
        cost = torch.empty(B, device=DEV)
        counts = torch.zeros(2, dtype=torch.int32, device=DEV)
        f = SkFwdArgs(C.data_ptr(), None, None, B, M, N, -1, tau, T, tol, 0, P.data_ptr(), cost.data_ptr(),
                      None, None, None, None, counts.data_ptr(), counts.data_ptr() + 4, ws.data_ptr(), ws.numel(),
                      exchange, epoch)
        assert lib.dot_sinkhorn_forward(ctypes.byref(f), stream) == 0
        grad = torch.empty_like(C)
        gtau = torch.empty(B, device=DEV)
        status = torch.full((1,), 7, dtype=torch.int32, device=DEV)
        b = SkBwdArgs(C.data_ptr(), -1, P.data_ptr(), G.data_ptr(), gc.data_ptr(), B, M, N, tau, T, None, None,
                      grad.data_ptr(), gtau.data_ptr(), ws.data_ptr(), ws.numel(), status.data_ptr(), exchange,
                      epoch + 1 if exchange else 0)
        assert lib.dot_sinkhorn_backward_implicit(ctypes.byref(b), stream) == 0
        torch.cuda.synchronize()
        return P, cost, counts, grad, gtau, status

    ref = run(None, 0)
    assert int(ref[5]) == 0
    # growing epochs; the last pair of the sequence (DOT_SINKHORN_MAX_EPOCH = 65534);
    # then the words cleared again and the sequence restarted at 1
    for epoch in (1, 3, 5, 65533, "clear", 1):
        if epoch == "clear":
            xw.zero_()
            continue
        out = run(xw.data_ptr(), epoch)
        for a, e in zip(out, ref):
            assert torch.equal(a, e), epoch
    P = torch.empty_like(C)
    counts = torch.zeros(2, dtype=torch.int32, device=DEV)
    for bad in (0, 65535):
        f = SkFwdArgs(C.data_ptr(), None, None, B, M, N, -1, tau, T, tol, 0, P.data_ptr(), None, None, None, None,
                      None, counts.data_ptr(), counts.data_ptr() + 4, ws.data_ptr(), ws.numel(), xw.data_ptr(), bad)
        assert lib.dot_sinkhorn_forward(ctypes.byref(f), stream) == 1


@pytest.mark.parametrize("B,M,N,tau,T,tol,b_range", [
    (2, 300, 4096, 0.1, 40, 0.0, None),
    (4, 512, 3072, 0.05, 60, 1e-6, None),
    (1, 1000, 4096, 0.02, 30, 0.0, None),
    (3, 256, 2560, 0.05, 40, 0.0, 60.0),   # v spreads past the range after iteration 1: log domain from there
])
def test_persistent_forward_scaled_kernel_matches_log_domain(B, M, N, tau, T, tol, b_range):
    """The persistent forward with rows of 64 floats per lane (N > 2048)
    streams a scaled copy of the kernel when the workspace holds it
    (dot_sinkhorn_forward_workspace_bytes) and the scores in the log domain
    when it does not: both against the oracle and each other."""
    print(f"[sk_gpu] persistent scaled kernel B={B} M={M} N={N} tau={tau} b_range={b_range}", flush=True)
    lib = ctypes.CDLL(os.path.join(ROOT, "dot_amd", "libdot_amd.so"))
    lib.dot_sinkhorn_forward_workspace_bytes.restype = ctypes.c_size_t
    lib.dot_sinkhorn_forward.argtypes = [ctypes.POINTER(SkFwdArgs), ctypes.c_void_p]
    rng = np.random.default_rng(B * M + N)
    C = rng.random((B, M, N)).astype(np.float32)
    lgb = None
    if b_range is not None:
        lb = -b_range * rng.random((B, N))
        lgb = (lb - np.log(np.exp(lb).sum(1, keepdims=True))).astype(np.float32)
    Cd = _t(C)
    lgbd = None if lgb is None else _t(lgb)
    full = lib.dot_sinkhorn_forward_workspace_bytes(B, M, N, T, 0)
    ek = (B * M * N * 4 + 255) // 256 * 256
    assert full > ek  # this shape takes the persistent tier on this device
    ws = torch.empty(full, dtype=torch.uint8, device=DEV)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    out = {}
    for name, nbytes in (("scaled", full), ("log", full - ek)):
        P = torch.empty_like(Cd)
        cost = torch.empty(B, device=DEV)
        counts = torch.zeros(2, dtype=torch.int32, device=DEV)
        f = SkFwdArgs(Cd.data_ptr(), None, None if lgbd is None else lgbd.data_ptr(), B, M, N, -1, tau, T, tol, 0,
                      P.data_ptr(), cost.data_ptr(), None, None, None, None, counts.data_ptr(), counts.data_ptr() + 4,
                      ws.data_ptr(), nbytes, None, 0)
        assert lib.dot_sinkhorn_forward(ctypes.byref(f), stream) == 0
        torch.cuda.synchronize()
        out[name] = (P, cost, [int(x) for x in counts.tolist()])
    for name, (P, cost, (used, _)) in out.items():
        o = osk.dual_forward(-C, tau, used, log_b=lgb)
        assert rel_err(P, o.P) < FWD_TOL, name
        assert rel_err(cost, osk.transport_cost(o.P, C)) < FWD_TOL, name
    if out["scaled"][2] == out["log"][2]:
        assert rel_err(out["scaled"][0], out["log"][0].cpu().numpy()) < 2e-6
    else:  # fp32 rounding at the stop threshold: one iteration apart at most
        assert abs(out["scaled"][2][0] - out["log"][2][0]) <= 1


def test_config_c5_forward_scaled_matches_log_domain_full_count():
    """C5 at its full count (4 x 4096^2, reg 0.02, 1000 iterations, tol 1e-6):
    the default persistent forward streams the scaled kernel (scaling domain
    while the range of v allows); the same call with a workspace that has no
    room for it runs the log domain, which the oracle pins at short counts
    (test_persistent_forward_scaled_kernel_matches_log_domain,
    test_config_c5_full_size).  The two 1000-iteration plans and costs agree
    within 1e-5."""
    lib = ctypes.CDLL(os.path.join(ROOT, "dot_amd", "libdot_amd.so"))
    lib.dot_sinkhorn_forward_workspace_bytes.restype = ctypes.c_size_t
    lib.dot_sinkhorn_forward.argtypes = [ctypes.POINTER(SkFwdArgs), ctypes.c_void_p]
    g = torch.Generator().manual_seed(5)
    x, y = torch.randn(4, 4096, 128, generator=g), torch.randn(4, 4096, 128, generator=g)
    C = torch.cdist(x.to(DEV), y.to(DEV))
    C = (C / C.amax(dim=(-2, -1), keepdim=True)).contiguous()
    B, M, N, T = 4, 4096, 4096, 1000
    full = lib.dot_sinkhorn_forward_workspace_bytes(B, M, N, T, 0)
    ek = (B * M * N * 4 + 255) // 256 * 256
    assert full > ek
    ws = torch.empty(full, dtype=torch.uint8, device=DEV)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    out = {}
    for name, nbytes in (("scaled", full), ("log", full - ek)):
        P = torch.empty_like(C)
        cost = torch.empty(B, device=DEV)
        counts = torch.zeros(2, dtype=torch.int32, device=DEV)
        f = SkFwdArgs(C.data_ptr(), None, None, B, M, N, -1, 0.02, T, 1e-6, 0, P.data_ptr(), cost.data_ptr(),
                      None, None, None, None, counts.data_ptr(), counts.data_ptr() + 4, ws.data_ptr(), nbytes,
                      None, 0)
        assert lib.dot_sinkhorn_forward(ctypes.byref(f), stream) == 0
        torch.cuda.synchronize()
        out[name] = (P, cost, [int(v) for v in counts.tolist()])
    print(f"[sk_gpu] C5 full count: counts {out['scaled'][2]} {out['log'][2]}", flush=True)
    assert out["scaled"][2] == out["log"][2] == [T, 0]
    (Ps, cs, _), (Pl, cl, _) = out["scaled"], out["log"]
    assert rel_err(Ps, Pl.cpu().numpy()) < FWD_TOL
    assert rel_err(cs, cl.cpu().numpy()) < FWD_TOL
    for P in (Ps, Pl):
        assert torch.allclose(P.sum(-2), torch.full_like(P.sum(-2), 1 / 4096), rtol=1e-4, atol=0)


def test_resident_launches_on_two_streams():
    """Resident forwards and adjoints enqueued on two streams with no host wait
    in between, each batch filling the device: the library orders its exchange
    kernels across streams (plain launches), and both streams get the bits of
    a run on one stream."""
    rng = np.random.default_rng(17)
    B, M, N, tau, T = 64, 512, 512, 0.1, 20
    C = [_t(rng.random((B, M, N)).astype(np.float32)) for _ in range(2)]
    G = [_t(rng.standard_normal((B, M, N)).astype(np.float32)) for _ in range(2)]
    run = lambda k: _ops.sinkhorn_with_grads_implicit(-C[k], G[k], tau, T, T)  # noqa: E731
    ref = [run(0), run(1)]
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    out = [None, None]
    for rep in range(3):
        for k in (0, 1):
            with torch.cuda.stream(streams[k]):
                out[k] = run(k)
        torch.cuda.synchronize()
        for k in (0, 1):
            for a, b in zip(out[k], ref[k]):
                assert torch.equal(a, b), (rep, k)


def _three_paths(monkeypatch, fn):
    """fn() on the persistent streaming kernels ("persistent", the register-
    resident tier switched off) and on the per-iteration sweeps ("sweeps")."""
    out = {}
    for name, env in (("persistent", {"DOT_AMD_RESIDENT": "0"}),
                      ("sweeps", {"DOT_AMD_RESIDENT": "0", "DOT_AMD_PERSISTENT": "0"})):
        for k, v in env.items():
            monkeypatch.setenv(k, v)
        out[name] = fn()
        for k in env:
            monkeypatch.delenv(k)
    return out


@pytest.mark.parametrize("B,M,N,tau,T,tol,nonuni", [
    (2, 300, 2048, 0.3, 30, 0.0, False),
    (3, 130, 4096, 0.5, 12, 0.0, True),
    (4, 257, 1000, 0.2, 300, 1e-5, True),
    (5, 64, 64, 1.0, 50, 0.0, False),
    (1, 7, 3, 0.7, 25, 1e-6, True),
])
def test_persistent_and_sweeps_agree_with_oracle(B, M, N, tau, T, tol, nonuni, monkeypatch):
    """Forward and implicit adjoint of the persistent streaming tier (one
    cooperative launch, reduce-scatter/all-gather exchange) and of the
    per-iteration sweeps, each against the oracle at its own iteration count."""
    rng = np.random.default_rng(7 * B + M + N)
    C = rng.random((B, M, N)).astype(np.float32)
    G = rng.standard_normal((B, M, N)).astype(np.float32)
    lga = np.log(_dirichlet(rng, B, M)) if nonuni else None
    lgb = np.log(_dirichlet(rng, B, N)) if nonuni else None
    lt = lambda x: None if x is None else _t(x)
    fwd = _three_paths(monkeypatch, lambda: _ops.sinkhorn_dual_forward(_t(-C), tau, T, tol, lt(lga), lt(lgb)))
    counts = {k: int(v[1]) for k, v in fwd.items()}
    assert abs(counts["persistent"] - counts["sweeps"]) <= 1, counts
    for name, (P, used, conv) in fwd.items():
        Po = osk.dual_forward(-C, tau, int(used), log_a=lga, log_b=lgb).P
        assert rel_err(P, Po) < FWD_TOL, name
    bwd = _three_paths(monkeypatch, lambda: _ops.sinkhorn_with_grads_implicit(
        _t(-C), _t(G), tau, min(T, 40), min(T, 40), lt(lga), lt(lgb)))
    Po, go, gto = osk.with_grads_implicit(-C, G, tau, min(T, 40), min(T, 40), lga, lgb)
    for name, (P, g, gt) in bwd.items():
        assert rel_err(P, Po) < FWD_TOL, name
        assert rel_err(g, go) < GRAD_TOL, name
        assert sum_err(gt, gto, go * -C / tau) < GRAD_TOL, name


def test_persistent_exact_column_fallback(monkeypatch):
    """The underflowing-column case of test_resident_forward_exact_column_fallback
    on the persistent tier, with a row longer than the resident limit."""
    rng = np.random.default_rng(9)
    B, M, N, tau, T = 2, 96, 1536, 0.01, 10
    C = (0.1 * rng.random((B, M, N))).astype(np.float32)
    C[:, :, 7] = 0.7
    C[1, :, 1500] = 0.8
    fwd = _three_paths(monkeypatch, lambda: _ops.sinkhorn_dual_forward(_t(-C), tau, T, 0.0))
    Po = osk.dual_forward(-C, tau, T).P
    for name, (P, used, _) in fwd.items():
        assert int(used) == T
        assert torch.isfinite(P).all(), name
        assert rel_err(P, Po) < FWD_TOL, name


def test_counts_are_read_lazily_and_match():
    """n_iters_used / converged are copied to the host behind the forward and
    read on first access, after the backward has been queued."""
    import importlib

    sk = importlib.import_module("dot_amd.sinkhorn")
    torch.manual_seed(5)
    C = torch.rand(4, 64, 48, device=DEV, requires_grad=True)
    r = dot_amd.sinkhorn(C, reg=0.1, n_iters=300, tol=1e-5)
    assert r.__dict__.get("_resolve") is not None  # nothing read yet
    r.cost.sum().backward()
    used = r.n_iters_used
    assert isinstance(used, int) and 1 <= used <= 300 and isinstance(r.converged, bool)
    if used < 300:
        assert r.converged
    r2 = dot_amd.sinkhorn(C.detach(), reg=0.1, n_iters=300, tol=1e-5)
    assert r2.n_iters_used == used and r2.converged == r.converged
    assert dot_amd.sinkhorn(C.detach(), reg=0.1, n_iters=7, tol=0.0).n_iters_used == 7
    for _ in range(100):
        dot_amd.sinkhorn_from_scores(-C.detach(), 0.1, 5)
    assert len(sk._unchecked) <= sk._MAX_UNCHECKED + 1
    torch.cuda.synchronize()
    sk._check_finished_forwards()
    assert len(sk._unchecked) == 0


def test_reference_explicit_uniform_rectangular_cpu_and_composed_gradient():
    """The reference's test_explicit_uniform_matches_default,
    test_rectangular_cuda_matches_cpu, test_composed_gradient_through_points_and_reg
    and test_sinkhorn_cuda_dual_matches_full_matrix_fixed_iterations
    (test_sinkhorn.py:186-199, 359-371, 419-432, 792-804) on HIP tensors."""
    torch.manual_seed(0)
    B, n, m = 2, 8, 16
    cost = torch.rand(B, n, m, device=DEV)
    a = torch.full((B, n), 1.0 / n, device=DEV)
    b = torch.full((B, m), 1.0 / m, device=DEV)
    default = dot_amd.sinkhorn(cost, reg=1.0, n_iters=50)
    explicit = dot_amd.sinkhorn(cost, reg=1.0, n_iters=50, a=a, b=b)
    assert torch.allclose(default.transport_plan, explicit.transport_plan, atol=1e-4)
    assert torch.allclose(default.cost, explicit.cost, atol=1e-4)

    cost_cpu = torch.rand(B, n, m)
    a_cpu = torch.softmax(torch.randn(B, n), dim=-1)
    b_cpu = torch.softmax(torch.randn(B, m), dim=-1)
    r_cpu = dot_amd.sinkhorn(cost_cpu, reg=1.0, a=a_cpu, b=b_cpu)
    r_dev = dot_amd.sinkhorn(cost_cpu.to(DEV), reg=1.0, a=a_cpu.to(DEV), b=b_cpu.to(DEV))
    assert torch.allclose(r_cpu.transport_plan, r_dev.transport_plan.cpu(), atol=1e-3)

    source = torch.randn(5, 3, device=DEV, requires_grad=True)
    target = torch.randn(5, 3, device=DEV)
    eps = torch.tensor(0.1, device=DEV, requires_grad=True)
    r = dot_amd.sinkhorn(torch.cdist(source, target).unsqueeze(0), reg=eps, n_iters=50)
    r.cost.sum().backward()
    assert source.grad is not None and torch.isfinite(source.grad).all()
    assert eps.grad is not None and torch.isfinite(eps.grad).all()
    # the same composition on the CPU gives the same gradients
    s_cpu = source.detach().cpu().requires_grad_(True)
    e_cpu = torch.tensor(0.1, requires_grad=True)
    rc = dot_amd.sinkhorn(torch.cdist(s_cpu, target.cpu()).unsqueeze(0), reg=e_cpu, n_iters=50)
    rc.cost.sum().backward()
    assert rel_err(source.grad.cpu(), s_cpu.grad) < 1e-4
    assert float(eps.grad) == pytest.approx(float(e_cpu.grad), rel=1e-4, abs=1e-6)

    cost = torch.rand(1, 96, 128, device=DEV)
    dual = dot_amd.sinkhorn(cost, reg=0.1, n_iters=50, tol=0, dual=True)
    full = dot_amd.sinkhorn(cost, reg=0.1, n_iters=50, tol=0, dual=False)
    assert dual.n_iters_used == 50 and full.n_iters_used == 50
    assert torch.allclose(dual.transport_plan, full.transport_plan, atol=1e-5)


def test_counts_on_a_side_stream():
    """A forward queued on a non-default stream: its counts are copied and
    awaited on that stream, so reading them after leaving the stream context
    gives the same values as a run on the default stream."""
    torch.manual_seed(6)
    C = torch.rand(3, 40, 56, device=DEV)
    ref = dot_amd.sinkhorn(C, reg=0.05, n_iters=400, tol=1e-5)
    used_ref, conv_ref = ref.n_iters_used, ref.converged
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        r = dot_amd.sinkhorn(C, reg=0.05, n_iters=400, tol=1e-5)
    assert r.n_iters_used == used_ref and r.converged == conv_ref
    torch.cuda.current_stream().wait_stream(side)
    assert torch.equal(r.transport_plan, ref.transport_plan)


def _drain_errors():
    """Empty the queue of unread device statuses, collecting the errors raised."""
    from dot_amd.sinkhorn import check_device_errors

    errors = []
    while True:
        try:
            check_device_errors()
            return errors
        except RuntimeError as e:
            errors.append(str(e))


@pytest.mark.parametrize("shape,env", [((4, 512, 512), {}),
                                       ((2, 300, 2048), {"DOT_AMD_RESIDENT": "0"})],
                         ids=["resident", "persistent"])
def test_exchange_timeout_is_raised(shape, env, monkeypatch):
    """DOT_AMD_SPIN_LIMIT=-1 makes every bounded wait of the cooperative kernels
    give up at once (the kernels then finish with NaN outputs): the forward's
    count read, the schema ops and the lazily checked backward status raise,
    and the next normal call is unaffected."""
    for k, v in env.items():
        monkeypatch.setenv(k, v)
    _drain_errors()
    rng = np.random.default_rng(sum(shape))
    C = _t(rng.random(shape).astype(np.float32))
    print(f"[timeout] shape={shape} env={env}", flush=True)
    # forward timed out: reading the count raises
    monkeypatch.setenv("DOT_AMD_SPIN_LIMIT", "-1")
    res = dot_amd.sinkhorn(C, reg=0.1, n_iters=20, tol=1e-6)
    with pytest.raises(RuntimeError, match="forward: a cross-workgroup exchange timed out"):
        res.n_iters_used
    assert torch.isnan(res.transport_plan).all()
    # the reference-schema op checks both statuses itself
    with pytest.raises(RuntimeError, match="timed out"):
        _ops.sinkhorn_with_grads_implicit(-C, torch.ones_like(C), 0.1, 10, 10)
    monkeypatch.delenv("DOT_AMD_SPIN_LIMIT")
    _drain_errors()
    # backward timed out after a normal forward: raised by the next check
    leaf = C.clone().requires_grad_(True)
    res = dot_amd.sinkhorn(leaf, reg=0.1, n_iters=20, tol=0)
    assert res.n_iters_used == 20
    monkeypatch.setenv("DOT_AMD_SPIN_LIMIT", "-1")
    res.cost.sum().backward()
    monkeypatch.delenv("DOT_AMD_SPIN_LIMIT")
    errors = _drain_errors()
    assert any("backward: a cross-workgroup exchange timed out" in e for e in errors), errors
    assert torch.isnan(leaf.grad).all()
    # the library state is clean afterwards
    leaf = C.clone().requires_grad_(True)
    res = dot_amd.sinkhorn(leaf, reg=0.1, n_iters=20, tol=0)
    res.cost.sum().backward()
    assert res.n_iters_used == 20 and torch.isfinite(leaf.grad).all()
    assert _drain_errors() == []


# ---------------------------------------------------------------------------
# Rows longer than 4096 columns (strips x chunks tiles) and batches above 65535
# ---------------------------------------------------------------------------
WIDE = [
    # (B, M, N, tau, T, tol, nonuniform); N % 4 != 0 takes the scalar-load tiles
    (1, 64, 4097, 0.3, 20, 0.0, False),
    (2, 40, 6000, 0.1, 30, 1e-6, True),
    (1, 33, 8192, 0.5, 15, 0.0, True),
    (2, 17, 5001, 1.0, 10, 0.0, False),
]


@pytest.mark.parametrize("B,M,N,tau,T,tol,nonuni", WIDE)
def test_wide_rows_match_oracle(B, M, N, tau, T, tol, nonuni):
    """Forward (with and without the stop test), implicit and unrolled adjoints,
    and the public API's cost gradient, for rows longer than a wave holds in
    registers (the reference chunks any row length: kernels.cuh:36-44,
    kernels.cu:547-627)."""
    rng = np.random.default_rng(B * 31 + M + N)
    C = rng.random((B, M, N)).astype(np.float32)
    G = rng.standard_normal((B, M, N)).astype(np.float32)
    lga = lgb = None
    if nonuni:
        lga, lgb = np.log(_dirichlet(rng, B, M)), np.log(_dirichlet(rng, B, N))
    lt = lambda x: None if x is None else _t(x)
    print(f"[wide] B={B} M={M} N={N} tau={tau} T={T} tol={tol}", flush=True)
    P, used, conv = _ops.sinkhorn_dual_forward(_t(-C), tau, T, tol, lt(lga), lt(lgb))
    used = int(used)
    if tol > 0:
        o = osk.dual_forward(-C, tau, T, tol=tol, log_a=lga, log_b=lgb)
        assert abs(used - o.n_iters_used) <= 1, (used, o.n_iters_used)
    else:
        assert used == T and int(conv) == 0
    assert rel_err(P, osk.dual_forward(-C, tau, used, log_a=lga, log_b=lgb).P) < FWD_TOL
    P, gi, gti = _ops.sinkhorn_with_grads_implicit(_t(-C), _t(G), tau, T, T, lt(lga), lt(lgb))
    Po, go, gto = osk.with_grads_implicit(-C, G, tau, T, T, lga, lgb)
    assert rel_err(P, Po) < FWD_TOL
    assert rel_err(gi, go) < GRAD_TOL
    assert sum_err(gti, gto, go * -C / tau) < GRAD_TOL
    Tu = min(T, 12)
    P, gu, gtu = _ops.sinkhorn_with_grads_unrolled(_t(-C), _t(G), tau, Tu, lt(lga), lt(lgb))
    Po, go, gto = osk.with_grads_unrolled(-C, G, tau, Tu, lga, lgb)
    assert rel_err(P, Po) < FWD_TOL
    assert rel_err(gu, go) < GRAD_TOL
    assert sum_err(gtu, gto, go * -C / tau) < GRAD_TOL
    # public API: plan, cost and cost gradient, return_log
    leaf = _t(C).requires_grad_(True)
    a = None if lga is None else _t(np.exp(lga))
    b = None if lgb is None else _t(np.exp(lgb))
    res = dot_amd.sinkhorn(leaf, reg=tau, n_iters=T, tol=0, a=a, b=b)
    res.cost.sum().backward()
    Pc, costc, dC, _, _ = _oracle_cost_grads(C, tau, T, T, None if a is None else np.exp(lga),
                                             None if b is None else np.exp(lgb))
    assert rel_err(res.transport_plan, Pc) < FWD_TOL
    assert rel_err(res.cost, costc) < FWD_TOL
    assert rel_err(leaf.grad, dC) < GRAD_TOL
    logP = _ops.sinkhorn_log(_t(-C), tau, T, lt(lga), lt(lgb))
    assert rel_err(logP.exp(), Pc) < FWD_TOL


def test_wide_rows_exact_column_fallback():
    """Columns whose sum underflows take the exact column log-sum-exp on the
    tiled path too."""
    rng = np.random.default_rng(91)
    B, M, N, tau, T = 1, 24, 4500, 0.01, 8
    C = (0.1 * rng.random((B, M, N))).astype(np.float32)
    C[:, :, 7] = 0.7
    C[:, :, 4400] = 0.8
    P, used, _ = _ops.sinkhorn_dual_forward(_t(-C), tau, T, 0.0)
    assert int(used) == T and torch.isfinite(P).all()
    assert rel_err(P, osk.dual_forward(-C, tau, T).P) < FWD_TOL


def test_batch_above_65535():
    """Grids put batch elements on y and z (at most 65535 per dimension):
    forward, both adjoints and the cost gradient at B = 70001 against the
    oracle, on small matrices of the streaming tier."""
    rng = np.random.default_rng(70001)
    B, M, N, tau, T = 70001, 3, 6, 0.5, 12
    C = rng.random((B, M, N)).astype(np.float32)
    G = rng.standard_normal((B, M, N)).astype(np.float32)
    print(f"[batch] B={B} M={M} N={N}", flush=True)
    P, used, conv = _ops.sinkhorn_dual_forward(_t(-C), tau, 200, 1e-6)
    o = osk.dual_forward(-C, tau, 200, tol=1e-6)
    assert abs(int(used) - o.n_iters_used) <= 1
    assert rel_err(P, osk.dual_forward(-C, tau, int(used)).P) < FWD_TOL
    P, gi, gti = _ops.sinkhorn_with_grads_implicit(_t(-C), _t(G), tau, T, T)
    Po, go, gto = osk.with_grads_implicit(-C, G, tau, T, T)
    assert rel_err(P, Po) < FWD_TOL and rel_err(gi, go) < GRAD_TOL
    assert sum_err(gti, gto, go * -C / tau) < GRAD_TOL
    P, gu, gtu = _ops.sinkhorn_with_grads_unrolled(_t(-C), _t(G), tau, T)
    Po, go, gto = osk.with_grads_unrolled(-C, G, tau, T)
    assert rel_err(P, Po) < FWD_TOL and rel_err(gu, go) < GRAD_TOL
    # the last batch element is computed (not dropped by the z slab's tail)
    assert rel_err(gu[-1:], go[-1:]) < GRAD_TOL
    leaf = _t(C).requires_grad_(True)
    res = dot_amd.sinkhorn(leaf, reg=tau, n_iters=T, tol=0)
    res.cost.sum().backward()
    Pc, costc, dC, _, _ = _oracle_cost_grads(C, tau, T, T)
    assert rel_err(res.cost, costc) < FWD_TOL and rel_err(leaf.grad, dC) < GRAD_TOL


@pytest.mark.parametrize("B,M,N,tau,T,nonuni", [
    (2, 300, 2048, 0.3, 12, True),
    (3, 64, 96, 0.5, 20, False),
    (1, 7, 3, 0.7, 6, True),
    (4, 257, 1000, 0.2, 0, False),
])
def test_unrolled_persistent_and_sweeps_agree_with_oracle(B, M, N, tau, T, nonuni, monkeypatch):
    """The unrolled backward as one cooperative launch (Gamma streamed each
    step, column sums through the tagged exchange) and as per-step sweeps,
    each against the oracle's restatement of kernels.cu:1622-1680; plus the
    public API's cost gradient in unrolled mode on both tiers."""
    rng = np.random.default_rng(3 * B + M + N + T)
    C = rng.random((B, M, N)).astype(np.float32)
    G = rng.standard_normal((B, M, N)).astype(np.float32)
    lga = np.log(_dirichlet(rng, B, M)) if nonuni else None
    lgb = np.log(_dirichlet(rng, B, N)) if nonuni else None
    lt = lambda x: None if x is None else _t(x)
    print(f"[unrolled tiers] B={B} M={M} N={N} T={T}", flush=True)
    runs = _three_paths(monkeypatch, lambda: _ops.sinkhorn_with_grads_unrolled(
        _t(-C), _t(G), tau, T, lt(lga), lt(lgb)))
    Po, go, gto = osk.with_grads_unrolled(-C, G, tau, T, lga, lgb)
    for name, (P, g, gt) in runs.items():
        assert rel_err(P, Po) < FWD_TOL, name
        assert rel_err(g, go) < GRAD_TOL, (name, rel_err(g, go))
        assert sum_err(gt, gto, go * -C / tau) < GRAD_TOL, name
    a = None if lga is None else np.exp(lga)
    b = None if lgb is None else np.exp(lgb)
    _, _, dC, _, _ = _oracle_cost_grads(C, tau, T, T, a, b, mode="unrolled")

    def api():
        leaf = _t(C).requires_grad_(True)
        res = dot_amd.sinkhorn(leaf, reg=tau, n_iters=T, tol=0, a=lt(a), b=lt(b), backward_mode="unrolled")
        res.cost.sum().backward()
        return leaf.grad

    for name, g in _three_paths(monkeypatch, api).items():
        assert rel_err(g, dC) < GRAD_TOL, (name, rel_err(g, dC))
