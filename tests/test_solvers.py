"""CPU: the reference's PyTorch-level solvers (dot/sinkhorn.py:743-1256) —
momentum, Anderson, Adam, scheduled plain Sinkhorn, Newton, Muon and the
over-relaxation estimate — as ``dot_amd.solvers`` and through
``dot_amd.sinkhorn`` on CPU tensors (and ``dual=False``).

Three layers:

* the numpy oracle (``oracle.solvers``) pinned by reductions to the plain
  iteration, closed forms and fixed points (its header lists them);
* ``dot_amd.solvers`` in float64 against the oracle (1e-10 norm-wise; Muon,
  whose inner plain runs are the float32 operator, 1e-5);
* the reference's own solver tests (test_sinkhorn.py:434-760), restated on the
  public API.
"""

import math
from unittest import mock

import numpy as np
import pytest
import torch

import dot_amd
from dot_amd import _ops, solvers
from conftest import rel_err
from oracle import sinkhorn as osk
from oracle import solvers as osv

EXACT = 1e-10


def _problem(B, n, m, seed, scale=1.0):
    """log_alpha exactly representable in float32, and float32-representable
    log marginals (so the float32-input oracle paths see the same numbers)."""
    rng = np.random.default_rng(seed)
    la = (-scale * rng.random((B, n, m))).astype(np.float32).astype(np.float64)
    a = rng.random((B, n)) + 0.5
    b = rng.random((B, m)) + 0.5
    lga = np.log(a / a.sum(1, keepdims=True)).astype(np.float32).astype(np.float64)
    lgb = np.log(b / b.sum(1, keepdims=True)).astype(np.float32).astype(np.float64)
    return la, lga, lgb


def _t(x):
    return None if x is None else torch.from_numpy(np.ascontiguousarray(x))


# ---------------------------------------------------------------------------
# Oracle pins
# ---------------------------------------------------------------------------
def test_oracle_plain_plan_is_the_golden_pinned_forward():
    la, lga, lgb = _problem(2, 7, 5, 0)
    for tau, T in ((0.5, 1), (0.5, 17), (0.25, 40)):
        ref = osk.dual_forward(la, tau, T, log_a=lga, log_b=lgb).P
        assert rel_err(osv.plain_plan(la, tau, T, lga, lgb), ref) < 1e-12


def test_oracle_momentum_omega_one_is_plain_and_omega_zero_never_moves():
    la, lga, lgb = _problem(2, 6, 8, 1)
    for T in (1, 3, 25):
        P, used = osv.momentum(la, 0.5, T, 1.0, lga, lgb, tol=0.0)
        assert used == T
        assert rel_err(P, osv.plain_plan(la, 0.5, T, lga, lgb)) < 1e-12
    P, used = osv.momentum(la, 0.5, 9, 0.0, lga, lgb)
    assert used == 1  # no change at all: stops after the first iteration
    assert np.array_equal(P, np.exp(la / 0.5))


def test_oracle_anderson_history_of_one_is_plain():
    la, lga, lgb = _problem(2, 9, 4, 2)
    for k in (0, 1):
        P, used = osv.anderson(la, 0.5, 12, k, 1.0, lga, lgb, tol=0.0)
        assert used == 12
        assert rel_err(P, osv.plain_plan(la, 0.5, 12, lga, lgb)) < 1e-12


def test_oracle_anderson_weights_solve_the_constrained_least_squares():
    """min |F w| subject to sum(w) = 1: w = e_h + Z y with Z = [e_i - e_h]."""
    rng = np.random.default_rng(3)
    for h in (2, 3, 5):
        F = rng.standard_normal((40, h))
        w = osv.anderson_weights(F)
        Z = np.eye(h)[:, :h - 1] - np.eye(h)[:, [h - 1]]
        y = np.linalg.lstsq(F @ Z, -F[:, h - 1], rcond=None)[0]
        closed = np.eye(h)[:, h - 1] + Z @ y
        assert abs(w.sum() - 1.0) < 1e-12
        assert np.abs(w - closed).max() < 1e-6


def test_oracle_anderson_reaches_the_plain_fixed_point():
    la, lga, lgb = _problem(1, 10, 10, 4)
    fixed = osv.plain_plan(la, 0.1, 3000, lga, lgb)
    for k in (2, 5, 8):
        P, used = osv.anderson(la, 0.1, 400, k, 1.0, lga, lgb)
        assert used < 100 and rel_err(P, fixed) < 1e-5
        # the 1e-8 ridge dominates once the residuals are ~1e-4 (equal weights),
        # so the residual itself stalls near 1e-8; the plan still converges
        P, used = osv.anderson(la, 0.1, 400, k, 1.0, lga, lgb, tol=0.0)
        assert rel_err(P, fixed) < 1e-9


def test_oracle_adam_reduces_to_the_plain_update():
    la, lga, lgb = _problem(2, 6, 7, 5)
    E = 1e9
    P, _ = osv.adam(la, 0.5, 15, E, 0.0, 0.0, E, False, lga, lgb, tol=0.0)
    assert rel_err(P, osv.plain_plan(la, 0.5, 15, lga, lgb)) < 1e-7
    # first bias-corrected step: lr g / (|g| + eps) whatever beta1, beta2
    for b1, b2 in ((0.9, 0.999), (0.3, 0.5)):
        P, used = osv.adam(la, 0.5, 1, E, b1, b2, E, True, lga, lgb, tol=0.0)
        assert used == 1
        assert rel_err(P, osv.plain_plan(la, 0.5, 1, lga, lgb)) < 1e-7
    # without correction the first step is damped by (1 - b1) / sqrt(1 - b2)
    P1, _ = osv.adam(la, 0.5, 1, 1.0, 0.5, 0.75, 0.0, False, lga, lgb, tol=0.0)
    K = la[0] / 0.5
    g = lga[0] - osv._lse(K, axis=1)
    u = 0.5 * g / (0.5 * np.abs(g))
    gv = lgb[0] - osv._lse(K + u[:, None], axis=0)
    v = 0.5 * gv / (0.5 * np.abs(gv))
    assert np.abs(P1[0] - np.exp(K + u[:, None] + v[None, :])).max() < 1e-12


@pytest.mark.parametrize("schedule", ["linear", "cosine", "exponential"])
def test_oracle_scheduled_tau_closed_forms(schedule):
    s, t, T = 0.8, 0.05, 9
    assert osv.scheduled_tau(0, T, t, s, schedule) == pytest.approx(s, rel=1e-15)
    assert osv.scheduled_tau(T - 1, T, t, s, schedule) == pytest.approx(t, rel=1e-15)
    mid = {"linear": (s + t) / 2, "cosine": (s + t) / 2, "exponential": math.sqrt(s * t)}[schedule]
    assert osv.scheduled_tau(4, T, t, s, schedule) == pytest.approx(mid, rel=1e-14)
    # cosine: a quarter of the way is s - (s - t)(1 - cos(pi/4)) / 2
    if schedule == "cosine":
        q = t + 0.5 * (s - t) * (1 + math.cos(math.pi / 4))
        assert osv.scheduled_tau(2, T, t, s, schedule) == pytest.approx(q, rel=1e-14)
    assert osv.scheduled_tau(3, 1, t, s, schedule) == t
    assert osv.scheduled_tau(3, T, t, None, schedule) == osv.scheduled_tau(3, T, t, 10 * t, schedule)


def test_oracle_scheduled_start_equal_target_is_plain_and_stop_rule():
    la, lga, lgb = _problem(2, 5, 6, 6)
    P, used = osv.scheduled(la, 0.5, 11, 0.5, "cosine", lga, lgb, tol=0.0)
    assert used == 11 and rel_err(P, osv.plain_plan(la, 0.5, 11, lga, lgb)) < 1e-12
    # the stop test counts from iteration max(n // 2, 1): with a huge tol the
    # run ends exactly there
    for n, expect in ((1, 1), (2, 2), (3, 2), (10, 6), (11, 6)):
        assert osv.scheduled(la, 0.5, n, 0.5, "linear", lga, lgb, tol=1e9)[1] == expect


def test_oracle_newton_system_is_the_residual_jacobian():
    la, lga, lgb = _problem(1, 5, 4, 7)
    K = la[0] / 0.3
    rng = np.random.default_rng(0)
    u, v = rng.standard_normal(5) * 0.1, rng.standard_normal(4) * 0.1
    a, b = np.exp(lga[0]), np.exp(lgb[0])

    def resid(x):
        P = np.exp(K + x[:5, None] + x[None, 5:])
        return np.concatenate([P.sum(1) - a, P.sum(0) - b])

    x0 = np.concatenate([u, v])
    J = np.zeros((9, 9))
    for k in range(9):
        e = np.zeros(9)
        e[k] = 1e-6
        J[:, k] = (resid(x0 + e) - resid(x0 - e)) / 2e-6
    H = osv.newton_system(np.exp(K + u[:, None] + v[None, :]), a, b)
    assert np.abs(H[1:, 1:] - J[1:, 1:]).max() < 1e-8
    assert H[0, 0] == 1.0 and not H[0, 1:].any() and not H[1:, 0].any()


def test_oracle_newton_converges_to_the_plain_fixed_point():
    la, lga, lgb = _problem(2, 9, 7, 8)
    # float64-normalised marginals (the float32-rounded ones differ in mass by ~1e-8)
    lga = lga - np.log(np.exp(lga).sum(1, keepdims=True))
    lgb = lgb - np.log(np.exp(lgb).sum(1, keepdims=True))
    P, used = osv.newton(la, 0.1, 30, lga, lgb)
    assert used < 30
    assert np.abs(P.sum(-1) - np.exp(lga)).max() < 1e-10
    assert np.abs(P.sum(-2) - np.exp(lgb)).max() < 1e-10
    assert rel_err(P, osv.plain_plan(la, 0.1, 3000, lga, lgb)) < 1e-9


def test_oracle_muon_fixed_point_and_tangent():
    la, lga, lgb = _problem(1, 8, 8, 9)
    G = np.random.default_rng(1).standard_normal((3, 8, 6))
    Tg = osv.birkhoff_tangent(G)
    assert np.abs(Tg.sum(-1)).max() < 1e-12 and np.abs(Tg.sum(-2)).max() < 1e-12
    assert np.abs(osv.birkhoff_tangent(Tg) - Tg).max() < 1e-12  # a projection
    # if the plan already is the target, no step is taken
    T = osv.plain_plan(la, 0.2, 200, lga, lgb)
    P, used = osv.muon(la, 0.2, 3, 0.5, lga, lgb, plain=lambda x, t, it, A, B_: T)
    assert used == 6 and rel_err(P, T) < 1e-9
    # it approaches the plain plan (test_sinkhorn.py:728-736's bound)
    P, used = osv.muon(la, 0.2, 120, 0.05, lga, lgb)
    assert np.abs(P - osv.plain_plan(la, 0.2, 2000, lga, lgb)).max() < 1e-4


def test_oracle_estimate_omega_rank_one_and_asymptotic_rate():
    r, c = np.random.default_rng(2).random(6), np.random.default_rng(3).random(5)
    la = (r[:, None] + c[None, :])[None]
    assert osv.estimate_omega(la, 0.3) == pytest.approx(1.0, abs=1e-12)
    # the pilot ratio tends to sigma_2^2 of diag(a)^-1/2 P diag(b)^-1/2
    la = -np.random.default_rng(1).random((1, 12, 12))
    for tau in (0.1, 0.05):
        _, ratio = osv.estimate_omega(la, tau, pilot_iters=40, return_ratio=True)
        P = osv.plain_plan(la, tau, 4000, *osv._marginals(1, 12, 12, None, None))[0]
        M = P / np.sqrt(P.sum(1))[:, None] / np.sqrt(P.sum(0))[None, :]
        s2 = np.linalg.svd(M, compute_uv=False)[1] ** 2
        assert ratio == pytest.approx(s2, rel=0.02)
        omega = osv.estimate_omega(la, tau, pilot_iters=40)
        assert omega == pytest.approx(2.0 / (1.0 + math.sqrt(1.0 - ratio ** 2)), rel=1e-12)


# ---------------------------------------------------------------------------
# dot_amd.solvers (float64 CPU tensors) against the oracle
# ---------------------------------------------------------------------------
CASES = [  # (B, n, m, tau, schedule, reg_start, marginals)
    (1, 12, 12, 0.1, None, None, False),
    (3, 9, 14, 0.05, None, None, True),
    (2, 10, 7, 0.02, "cosine", 0.2, True),
    (2, 8, 8, 0.05, "exponential", None, False),
]


def _inputs(case, seed):
    B, n, m, tau, sched, start, marg = case
    la, lga, lgb = _problem(B, n, m, seed)
    if not marg:
        lga = lgb = None
    return la, lga, lgb, tau, sched, start


@pytest.mark.parametrize("case", CASES)
def test_momentum_matches_oracle(case):
    la, lga, lgb, tau, sched, start = _inputs(case, 10)
    for omega, T in ((1.5, 60), (1.2, 7)):
        P, used = solvers.momentum_forward(_t(la), tau, T, _t(lga), _t(lgb), omega, start, sched)
        Po, uo = osv.momentum(la, tau, T, omega, lga, lgb, start, sched)
        assert used == uo and rel_err(P, Po) < EXACT


@pytest.mark.parametrize("case", CASES)
def test_anderson_matches_oracle(case):
    la, lga, lgb, tau, sched, start = _inputs(case, 11)
    # under a schedule the mixed states come from different taus and the Gram
    # solve amplifies rounding (1e-16 -> 1e-6 by iteration 40 between two
    # correct float64 implementations), so those runs are compared early
    for k, beta, T in ((5, 1.0, 15 if sched else 80), (3, 0.5, 9), (1, 1.0, 5)):
        P, used = solvers.anderson_forward(_t(la), tau, T, _t(lga), _t(lgb), k, beta, start, sched)
        Po, uo = osv.anderson(la, tau, T, k, beta, lga, lgb, start, sched)
        assert used == uo and rel_err(P, Po) < 1e-8


@pytest.mark.parametrize("case", CASES)
def test_adam_matches_oracle(case):
    la, lga, lgb, tau, sched, start = _inputs(case, 12)
    for args in ((0.5, 0.9, 0.999, 1e-8, True), (0.25, 0.0, 0.999, 1e-8, False), (1.0, 0.5, 0.9, 1e-6, True)):
        P, used = solvers.adam_forward(_t(la), tau, 40, _t(lga), _t(lgb), *args, start, sched)
        Po, uo = osv.adam(la, tau, 40, *args, lga, lgb, start, sched)
        assert used == uo and rel_err(P, Po) < EXACT


@pytest.mark.parametrize("case", CASES)
def test_scheduled_matches_oracle(case):
    la, lga, lgb, tau, sched, start = _inputs(case, 13)
    sched = sched or "linear"
    start = start if start is not None else 10.0 * tau
    for T in (1, 2, 30, 200):
        P, used = solvers.scheduled_forward(_t(la), tau, T, _t(lga), _t(lgb), start, sched)
        Po, uo = osv.scheduled(la, tau, T, start, sched, lga, lgb)
        assert used == uo and rel_err(P, Po) < EXACT


@pytest.mark.parametrize("case", CASES)
def test_newton_matches_oracle(case):
    la, lga, lgb, tau, sched, start = _inputs(case, 14)
    for T in (1, 3, 12):
        P, used = solvers.newton_forward(_t(la), tau, T, _t(lga), _t(lgb), start, sched)
        Po, uo = osv.newton(la, tau, T, lga, lgb, start, sched)
        assert used == uo and rel_err(P, Po) < 1e-9


def _plain64(log_alpha, tau, iters, log_a, log_b):
    """The plain operator in float64 torch (the reference's ``_ops.sinkhorn``
    computes in float32), for comparing Muon's own arithmetic exactly."""
    K = log_alpha / tau
    u = log_alpha.new_zeros(log_alpha.shape[:2])
    v = log_alpha.new_zeros((log_alpha.shape[0], log_alpha.shape[2]))
    for _ in range(iters):
        u, v = solvers.fixed_point_map(u, v, K, log_a, log_b)
    return (K + u.unsqueeze(-1) + v.unsqueeze(-2)).exp()


@pytest.mark.parametrize("case", CASES)
def test_muon_matches_oracle(case):
    """Muon divides by the plan's entries (down to 1e-24 here), so its
    trajectory amplifies rounding: with a float64 inner operator the two
    implementations agree to 1e-9 over 3 steps; with the product's float32
    operator (the reference's) one step agrees to the float32 spread."""
    la, lga, lgb, tau, sched, start = _inputs(case, 15)
    with mock.patch.object(solvers._ops, "sinkhorn", _plain64):
        for lr, T in ((0.05, 3), (0.5, 3), (0.05, 1)):
            P, used = solvers.muon_forward(_t(la), tau, T, _t(lga), _t(lgb), lr, start, sched)
            Po, uo = osv.muon(la, tau, T, lr, lga, lgb, start, sched)
            assert used == uo and rel_err(P, Po) < 1e-9
    P, used = solvers.muon_forward(_t(la), tau, 1, _t(lga), _t(lgb), 0.05, start, sched)
    Po, uo = osv.muon(la, tau, 1, 0.05, lga, lgb, start, sched)
    assert used == uo and rel_err(P, Po) < 1e-4


def test_estimate_omega_matches_oracle():
    for seed, (B, n, m), tau in ((0, (1, 12, 12), 0.1), (1, (3, 9, 5), 0.05), (2, (2, 6, 6), 1.0)):
        la, lga, lgb = _problem(B, n, m, seed)
        got = solvers.estimate_omega(_t(la), tau, _t(lga), _t(lgb))
        assert got == pytest.approx(osv.estimate_omega(la, tau, lga, lgb), rel=1e-12)


def test_scheduled_tau_matches_oracle():
    for sched in ("linear", "cosine", "exponential", None):
        for step in range(7):
            assert solvers.scheduled_tau(step, 7, 0.03, 0.4, sched) == osv.scheduled_tau(step, 7, 0.03, 0.4, sched)


# ---------------------------------------------------------------------------
# Dispatch, results and gradients through dot_amd.sinkhorn (CPU tensors)
# ---------------------------------------------------------------------------
def test_api_routes_methods_to_the_solvers():
    C = torch.rand(2, 8, 6, dtype=torch.float64)
    cases = [
        (dict(method="momentum", omega=1.5), solvers.momentum_forward, dict(omega=1.5)),
        (dict(method="anderson", anderson_k=4, mixing_beta=0.7), solvers.anderson_forward,
         dict(anderson_k=4, mixing_beta=0.7)),
        (dict(method="adam", lr=0.5), solvers.adam_forward,
         dict(lr=0.5, beta1=0.9, beta2=0.999, eps_adam=1e-8, bias_correction=True)),
        (dict(method="newton"), solvers.newton_forward, {}),
        (dict(method="auto"), solvers.newton_forward, {}),
        (dict(method="muon", lr=0.1), solvers.muon_forward, dict(lr=0.1)),
        (dict(schedule="cosine"), solvers.scheduled_forward, dict(reg_start=1.0, schedule="cosine")),
        (dict(schedule="linear", reg_start=0.5), solvers.scheduled_forward, dict(reg_start=0.5, schedule="linear")),
    ]
    for kw, fn, opts in cases:
        r = dot_amd.sinkhorn(C, reg=0.1, n_iters=25, **kw)
        P, used = fn(-C, 0.1, 25, None, None, **opts)
        assert torch.equal(r.transport_plan, P), kw
        assert r.n_iters_used == used
        assert r.converged == (used < 25)
        assert torch.allclose(r.cost, (P * C).sum((-2, -1)), rtol=1e-12, atol=0)
    # momentum without omega estimates it from a pilot run
    omega = solvers.estimate_omega(-C, 0.1, None, None)
    r = dot_amd.sinkhorn(C, reg=0.1, n_iters=25, method="momentum")
    assert torch.equal(r.transport_plan, solvers.momentum_forward(-C, 0.1, 25, None, None, omega)[0])
    # tol == 0 reports converged, as the reference does
    assert dot_amd.sinkhorn(C, reg=0.1, n_iters=3, method="adam", tol=0.0).converged is True
    # unbatched input
    r = dot_amd.sinkhorn(C[0], reg=0.1, n_iters=25, method="anderson")
    assert r.transport_plan.shape == (8, 6) and r.cost.dim() == 0


def test_api_solver_errors():
    C = torch.rand(1, 6, 6)
    for method in ("momentum", "anderson", "adam", "newton", "muon"):
        with pytest.raises(ValueError, match="only supports implicit backward"):
            dot_amd.sinkhorn(C, method=method, backward_mode="unrolled")
    with pytest.raises(ValueError, match="only supports n, m <= 100"):
        dot_amd.sinkhorn(torch.rand(1, 3, 101), method="newton")
    with pytest.raises(ValueError, match="schedule must be"):
        dot_amd.sinkhorn(C, method="momentum", omega=1.2, schedule="quadratic")
    # the reference reads float(reg.item()) first (sinkhorn.py:1352)
    with pytest.raises(RuntimeError, match="cannot be converted to Scalar"):
        dot_amd.sinkhorn(C, reg=torch.ones(2), method="anderson")
    with pytest.raises(ValueError, match="reg/tau tensor must be scalar"):
        solvers.ImplicitSolverFunction.apply(-C, torch.ones(2), 3, 3, None, None, solvers.momentum_forward,
                                             dict(omega=1.0))


@pytest.mark.parametrize("kw", [dict(method="momentum", omega=1.3), dict(method="anderson"),
                                dict(method="adam", lr=0.5), dict(method="newton"),
                                dict(method="muon", lr=0.3), dict(schedule="exponential", reg_start=0.5)])
def test_api_solver_gradients_are_the_implicit_adjoint_at_n_iters_used(kw):
    """The reference's backward: sinkhorn_with_grads_implicit at n_iters_used
    for the plan's gradient, plus the cost's direct term P."""
    torch.manual_seed(0)
    C = torch.rand(2, 7, 5)
    W = torch.rand(2, 7, 5)
    reg = torch.tensor(0.2, requires_grad=True)
    Cg = C.clone().requires_grad_(True)
    r = dot_amd.sinkhorn(Cg, reg=reg, n_iters=40, backward_iters=30, **kw)
    ((r.transport_plan * W).sum() + r.cost.sum()).backward()
    P = r.transport_plan.detach()
    _, g_la, g_tau = _ops.sinkhorn_with_grads_implicit(-C, (W + C).contiguous(), 0.2, r.n_iters_used, 30,
                                                       None, None)
    assert rel_err(Cg.grad, P - g_la) < 1e-6
    assert reg.grad.dtype == reg.dtype
    assert float(reg.grad) == pytest.approx(float(g_tau.sum()), rel=1e-6, abs=1e-9)


def test_api_marginals_and_dual_false_on_cpu():
    torch.manual_seed(1)
    C = torch.rand(2, 9, 6, dtype=torch.float64)
    a = torch.rand(9, dtype=torch.float64) + 0.2
    a = a / a.sum()
    b = torch.rand(2, 6, dtype=torch.float64) + 0.2
    b = b / b.sum(-1, keepdim=True)
    r = dot_amd.sinkhorn(C, reg=0.1, n_iters=30, a=a, b=b, method="newton")
    assert torch.allclose(r.transport_plan.sum(-1), a.expand(2, -1), atol=1e-10)
    assert torch.allclose(r.transport_plan.sum(-2), b, atol=1e-10)
    r2 = dot_amd.sinkhorn(C, reg=0.1, n_iters=30, a=a, b=b, method="newton", dual=False)
    assert torch.equal(r.transport_plan, r2.transport_plan)


# ---------------------------------------------------------------------------
# The reference's solver tests (test_sinkhorn.py:434-760), CPU tensors
# ---------------------------------------------------------------------------
def _vanilla_convergence_iters(log_alpha, tau, max_iters=100, tol=1e-6):
    """Iterations of plain Sinkhorn until the largest potential change is below
    tol (the reference test helper, test_sinkhorn.py:44-75)."""
    log_alpha = log_alpha if log_alpha.dim() == 3 else log_alpha.unsqueeze(0)
    B, n, m = log_alpha.shape
    K = log_alpha / tau
    la = torch.full((B, n), -math.log(n), dtype=log_alpha.dtype)
    lb = torch.full((B, m), -math.log(m), dtype=log_alpha.dtype)
    u, v = torch.zeros(B, n, dtype=K.dtype), torch.zeros(B, m, dtype=K.dtype)
    for it in range(max_iters):
        un, vn = solvers.fixed_point_map(u, v, K, la, lb)
        if max(float((un - u).abs().max()), float((vn - v).abs().max())) < tol:
            return it + 1
        u, v = un, vn
    return max_iters


def _grid(n, lo=-1.0, hi=1.0, weight=None, eye=0.0):
    g = torch.linspace(lo, hi, n)
    c = (g[:, None] - g[None, :]).abs().pow(2)
    if weight is not None:
        c = c * torch.linspace(1.0, weight, n).unsqueeze(0)
    return (c + eye * torch.eye(n)).unsqueeze(0)


def test_ref_momentum_matches_vanilla_and_auto_omega():
    torch.manual_seed(0)
    cost = torch.rand(1, 12, 12)
    van = dot_amd.sinkhorn(cost, reg=1.0, n_iters=80)
    mom = dot_amd.sinkhorn(cost, reg=1.0, n_iters=80, method="momentum", omega=1.5)
    assert torch.allclose(van.transport_plan, mom.transport_plan, atol=1e-4)
    r = dot_amd.sinkhorn(cost, reg=0.1, n_iters=80, method="momentum")
    assert r.transport_plan.shape == (1, 12, 12) and r.n_iters_used is not None


def test_ref_momentum_and_anderson_use_fewer_iterations_than_vanilla():
    cost = _grid(32)
    van_iters = _vanilla_convergence_iters(-cost, tau=0.02, max_iters=120)
    mom = dot_amd.sinkhorn(cost, reg=0.02, n_iters=120, method="momentum", omega=1.4)
    aa = dot_amd.sinkhorn(cost, reg=0.02, n_iters=120, method="anderson", anderson_k=5)
    assert mom.n_iters_used < van_iters
    assert aa.n_iters_used < van_iters


def test_ref_anderson_matches_vanilla_with_gradients_and_fallback():
    torch.manual_seed(0)
    cost = torch.rand(1, 12, 12)
    van = dot_amd.sinkhorn(cost, reg=0.1, n_iters=120)
    aa = dot_amd.sinkhorn(cost, reg=0.1, n_iters=120, method="anderson", anderson_k=5)
    assert torch.allclose(van.transport_plan, aa.transport_plan, atol=1e-4)

    cost = torch.rand(1, 10, 10)
    cv = cost.clone().requires_grad_(True)
    van = dot_amd.sinkhorn(cv, reg=0.1, n_iters=120)
    van.cost.sum().backward()
    ca = cost.clone().requires_grad_(True)
    aa = dot_amd.sinkhorn(ca, reg=0.1, n_iters=120, method="anderson", anderson_k=5)
    aa.cost.sum().backward()
    assert torch.allclose(van.transport_plan, aa.transport_plan, atol=1e-4)
    assert torch.allclose(cv.grad, ca.grad, atol=1e-4)

    van = dot_amd.sinkhorn(cost, reg=0.1, n_iters=80)
    with mock.patch("torch.linalg.solve", side_effect=RuntimeError("singular")):
        aa = dot_amd.sinkhorn(cost, reg=0.1, n_iters=80, method="anderson", anderson_k=5)
    assert torch.allclose(van.transport_plan, aa.transport_plan, atol=1e-4)


def test_ref_adam_tests():
    torch.manual_seed(0)
    cost = torch.rand(1, 12, 12)
    van = dot_amd.sinkhorn(cost, reg=0.1, n_iters=200)
    adam = dot_amd.sinkhorn(cost, reg=0.1, n_iters=200, method="adam", lr=0.5)
    assert torch.allclose(van.transport_plan, adam.transport_plan, atol=5e-4)

    r = dot_amd.sinkhorn(_grid(24, -2.0, 2.0, weight=3.0), reg=0.02, n_iters=40, method="adam", lr=0.5)
    assert torch.isfinite(r.transport_plan).all() and r.n_iters_used is not None

    cost = _grid(32, -3.0, 3.0, weight=5.0)
    ref = dot_amd.sinkhorn(cost, reg=0.02, n_iters=800)
    van = dot_amd.sinkhorn(cost, reg=0.02, n_iters=20)
    default = dot_amd.sinkhorn(cost, reg=0.02, n_iters=20, method="adam", lr=0.5)
    rms = dot_amd.sinkhorn(cost, reg=0.02, n_iters=20, method="adam", lr=0.25, beta1=0.0, beta2=0.999,
                           bias_correction=False)
    err = lambda r: (r.transport_plan - ref.transport_plan).abs().mean()  # noqa: E731
    assert err(rms) < err(van)
    assert err(rms) < err(default)

    c = torch.rand(1, 10, 10, requires_grad=True)
    dot_amd.sinkhorn(c, reg=0.1, n_iters=80, method="adam", lr=0.5).cost.sum().backward()
    assert c.grad is not None


def test_ref_scheduled_tests():
    torch.manual_seed(0)
    cost = torch.rand(1, 12, 12)
    van = dot_amd.sinkhorn(cost, reg=0.1, n_iters=200)
    sch = dot_amd.sinkhorn(cost, reg=0.1, n_iters=200, schedule="cosine", reg_start=0.1)
    assert torch.allclose(van.transport_plan, sch.transport_plan, atol=1e-4)

    torch.manual_seed(4)
    base = torch.rand(24, 24)
    cost = ((base + base.t()) / 2).unsqueeze(0)
    ref = dot_amd.sinkhorn(cost, reg=0.001, n_iters=600)
    van = dot_amd.sinkhorn(cost, reg=0.001, n_iters=10)
    sch = dot_amd.sinkhorn(cost, reg=0.001, n_iters=10, schedule="linear", reg_start=0.1)
    assert (sch.transport_plan - ref.transport_plan).abs().mean() < (van.transport_plan - ref.transport_plan).abs().mean()

    c = torch.rand(1, 10, 10, requires_grad=True)
    dot_amd.sinkhorn(c, reg=0.01, n_iters=80, schedule="cosine", reg_start=0.1).cost.sum().backward()
    assert c.grad is not None

    cost = torch.rand(1, 12, 12)
    aa = dot_amd.sinkhorn(cost, reg=0.1, n_iters=120, method="anderson", anderson_k=5)
    sa = dot_amd.sinkhorn(cost, reg=0.1, n_iters=120, method="anderson", anderson_k=5, schedule="cosine",
                          reg_start=0.1)
    assert torch.allclose(aa.transport_plan, sa.transport_plan, atol=1e-4)
    c = torch.rand(1, 12, 12, requires_grad=True)
    dot_amd.sinkhorn(c, reg=0.01, n_iters=80, method="anderson", schedule="cosine", reg_start=0.1).cost.sum().backward()
    assert c.grad is not None


@pytest.mark.parametrize("n", [5, 10, 20])
def test_ref_newton_matches_vanilla_on_small_problems(n):
    torch.manual_seed(n)
    cost = torch.rand(1, n, n)
    van = dot_amd.sinkhorn(cost, reg=0.1, n_iters=200)
    newton = dot_amd.sinkhorn(cost, reg=0.1, n_iters=5, method="newton")
    assert torch.allclose(van.transport_plan, newton.transport_plan, atol=1e-5)


def test_ref_newton_tests():
    torch.manual_seed(0)
    r = dot_amd.sinkhorn(torch.rand(1, 20, 20), reg=0.1, n_iters=5, method="newton")
    assert r.n_iters_used is not None and r.n_iters_used <= 5

    torch.manual_seed(0)
    cost = torch.rand(1, 12, 9)
    a = torch.rand(12)
    a = a / a.sum()
    b = torch.rand(9)
    b = b / b.sum()
    r = dot_amd.sinkhorn(cost, reg=0.1, n_iters=5, method="newton", a=a, b=b)
    assert torch.allclose(r.transport_plan.sum(dim=-1).squeeze(0), a, atol=1e-5)
    assert torch.allclose(r.transport_plan.sum(dim=-2).squeeze(0), b, atol=1e-5)

    c = torch.rand(1, 10, 10, requires_grad=True)
    dot_amd.sinkhorn(c, reg=0.1, n_iters=5, method="newton").cost.sum().backward()
    assert c.grad is not None

    torch.manual_seed(0)
    cost = torch.rand(1, 11, 11)
    auto = dot_amd.sinkhorn(cost, reg=0.1, n_iters=5, method="auto")
    newton = dot_amd.sinkhorn(cost, reg=0.1, n_iters=5, method="newton")
    assert torch.allclose(auto.transport_plan, newton.transport_plan, atol=1e-6)


def test_ref_muon_tests():
    torch.manual_seed(0)
    cost = torch.rand(1, 12, 12)
    van = dot_amd.sinkhorn(cost, reg=0.1, n_iters=120)
    muon = dot_amd.sinkhorn(cost, reg=0.1, n_iters=120, method="muon", lr=0.05)
    assert torch.allclose(van.transport_plan, muon.transport_plan, atol=1e-4)

    cost = _grid(24, eye=1e-4)
    ref = dot_amd.sinkhorn(cost, reg=0.005, n_iters=400)
    muon = dot_amd.sinkhorn(cost, reg=0.005, n_iters=40, method="muon", lr=0.05)
    assert torch.isfinite(muon.transport_plan).all() and muon.n_iters_used is not None
    assert (muon.transport_plan - ref.transport_plan).abs().mean() < 5e-3

    c = torch.rand(1, 10, 10, requires_grad=True)
    dot_amd.sinkhorn(c, reg=0.1, n_iters=80, method="muon", lr=0.5).cost.sum().backward()
    assert c.grad is not None
