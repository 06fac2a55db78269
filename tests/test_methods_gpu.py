"""GPU parity of the accelerated and scheduled dual Sinkhorn (dot_sinkhorn_forward_method).

The oracle is oracle.sinkhorn.dual_forward_method (float64).  Tolerances are
norm-wise relative (max|a - e| / max|e|): plans 1e-5 for the iterations with
no data-dependent branch or a branch decided by a wide margin (schedules,
momentum with omega in (0, 2), where the candidate's gap is |1 - omega| times
the current one), gradients 1e-4.  Adam's and Anderson's acceptance tests
and Anderson's small least-squares solves can amplify fp32 rounding, so their
per-iteration parity is judged against the spread of an fp32 run of the same
oracle (the rounding the algorithm itself has in fp32), floored at 1e-5.
The reference's own method tests (test_sinkhorn.py:427-666) are run on HIP
tensors at the end.
"""

import numpy as np
import pytest
import torch

import dot_amd
from dot_amd import solvers
from dot_amd import _ops
from conftest import rel_err, sum_err
from oracle import sinkhorn as osk

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)
FWD_TOL, GRAD_TOL = 1e-5, 1e-4
VAN, MOM, AND, ADAM = 0, 1, 2, 3
LIN, EXP, COS = 1, 2, 3


def _t(x):
    return None if x is None else torch.as_tensor(np.ascontiguousarray(x)).to(DEV)


def _dirichlet(rng, B, n):
    e = -np.log(rng.random((B, n)))
    return (e / e.sum(1, keepdims=True)).astype(np.float32)


def _case(seed, B, M, N, marginals=False):
    rng = np.random.default_rng(seed)
    la = (-rng.random((B, M, N))).astype(np.float32)  # log_alpha = -C, C in [0, 1)
    if not marginals:
        return la, None, None
    return la, np.log(_dirichlet(rng, B, M)), np.log(_dirichlet(rng, B, N))


def _gpu(la, tau, T, tol=0.0, log_a=None, log_b=None, method=VAN, omega=1.5, anderson_k=5, mixing_beta=1.0,
         lr=1.0, beta1=0.9, beta2=0.999, eps_adam=1e-8, bias_correction=True, reg_start=-1.0, schedule=0,
         return_log=False):
    P, used, conv = _ops.sinkhorn_dual_forward(_t(la), tau, T, tol, _t(log_a), _t(log_b), return_log, method,
                                               omega, anderson_k, mixing_beta, lr, beta1, beta2, eps_adam,
                                               bias_correction, reg_start, schedule)
    return P, int(used), int(conv)


def _oracle(la, tau, T, tol=0.0, log_a=None, log_b=None, method=VAN, dtype=np.float64, **kw):
    return osk.dual_forward_method(la, tau, T, tol, log_a, log_b, method=method, dtype=dtype, **kw)


SHAPES = [(2, 40, 56), (1, 37, 29), (3, 64, 256), (2, 300, 132)]


def test_native_library_is_loaded():
    maps = open("/proc/self/maps").read()
    assert "libdot_amd.so" in maps and "_C.so" in maps


# ---------------------------------------------------------------------------
# Schedules (vanilla loop): per-iteration parity
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("schedule", [LIN, EXP, COS])
@pytest.mark.parametrize("shape", SHAPES)
def test_schedule_matches_oracle(schedule, shape):
    B, M, N = shape
    la, lga, lgb = _case(11 + M, B, M, N, marginals=(M == 40))
    for T, reg_start in ((1, -1.0), (7, 0.5), (25, -1.0)):
        print(f"schedule={schedule} shape={shape} T={T} reg_start={reg_start}", flush=True)
        P, used, conv = _gpu(la, 0.1, T, 0.0, lga, lgb, schedule=schedule, reg_start=reg_start)
        ref = _oracle(la, 0.1, T, 0.0, lga, lgb, schedule=schedule, reg_start=reg_start)
        assert used == T and conv == 0
        assert rel_err(P, ref.P) < FWD_TOL, (T, reg_start)


TIERS = {"resident": {}, "persistent": {"DOT_AMD_RESIDENT": "0"},
         "sweeps": {"DOT_AMD_RESIDENT": "0", "DOT_AMD_PERSISTENT": "0"}}


@pytest.mark.parametrize("tier", sorted(TIERS))
@pytest.mark.parametrize("shape", [(2, 40, 56), (1, 37, 29), (3, 64, 256), (1, 130, 1030)])
def test_scheduled_plain_iteration_on_every_tier(tier, shape, monkeypatch):
    # the plain method runs on the vanilla forward's tiers with a per-iteration K scale
    for k, v in TIERS[tier].items():
        monkeypatch.setenv(k, v)
    B, M, N = shape
    la, lga, lgb = _case(17 + N, B, M, N, marginals=True)
    for schedule, T in ((LIN, 1), (COS, 9), (EXP, 25)):
        print(f"tier={tier} shape={shape} schedule={schedule} T={T}", flush=True)
        P, used, conv = _gpu(la, 0.1, T, 0.0, lga, lgb, schedule=schedule, reg_start=0.4)
        ref = _oracle(la, 0.1, T, 0.0, lga, lgb, schedule=schedule, reg_start=0.4)
        assert used == T and conv == 0
        assert rel_err(P, ref.P) < FWD_TOL, (schedule, T)
    # the device stop test under a schedule
    P, used, conv = _gpu(la, 0.1, 150, 1e-3, lga, lgb, schedule=COS, reg_start=0.15)
    ref = _oracle(la, 0.1, 150, 1e-3, lga, lgb, schedule=COS, reg_start=0.15)
    assert conv == int(ref.converged) and used == ref.n_iters_used
    assert rel_err(P, ref.P) < FWD_TOL


def test_scheduled_plain_iteration_on_long_rows():
    """The plain method with a schedule on rows longer than 4096 columns (the
    forward's strips x chunks tiles with a per-iteration K scale)."""
    B, M, N = 1, 24, 4500
    la, lga, lgb = _case(4500, B, M, N, marginals=True)
    for schedule, T in ((LIN, 3), (EXP, 12)):
        P, used, conv = _gpu(la, 0.1, T, 0.0, lga, lgb, schedule=schedule, reg_start=0.4)
        ref = _oracle(la, 0.1, T, 0.0, lga, lgb, schedule=schedule, reg_start=0.4)
        assert used == T and conv == 0
        assert rel_err(P, ref.P) < FWD_TOL, (schedule, T)


LONG_ROW_METHODS = [(MOM, {"omega": 1.3}), (ADAM, {"lr": 0.5}), (AND, {"anderson_k": 4})]


@pytest.mark.parametrize("method,kw", LONG_ROW_METHODS)
@pytest.mark.parametrize("shape", [(2, 20, 4500), (1, 9, 4097), (1, 70, 8192)])
def test_methods_on_long_rows(method, kw, shape):
    """Momentum, Adam and Anderson on rows longer than 4096 columns: the sweep
    as a rows pass, a per-row finish and a columns pass over strips x chunks
    tiles (N % 4 != 0 takes scalar loads).  Judged against the fp32 spread of
    the oracle, as the short-row tests of these methods."""
    B, M, N = shape
    la, lga, lgb = _case(83 + N, B, M, N, marginals=(B == 2))
    for T in (1, 4, 15):
        print(f"long rows method={method} shape={shape} T={T}", flush=True)
        P, used, conv = _gpu(la, 0.1, T, 0.0, lga, lgb, method=method, **kw)
        ref, tol = _fp32_spread(la, 0.1, T, lga, lgb, method=method, **kw)
        assert used == T and conv == 0
        assert rel_err(P, ref.P) < tol, (T, tol)


@pytest.mark.parametrize("method,kw", LONG_ROW_METHODS)
def test_methods_on_long_rows_stop_test_and_cost(method, kw):
    # the device stop test, and the cost through the public API (per-tile cost partials)
    la, _, _ = _case(89, 2, 16, 5000)
    P, used, conv = _gpu(la, 0.2, 120, 1e-4, method=method, **kw)
    ref = _oracle(la, 0.2, 120, 1e-4, method=method, **kw)
    assert ref.converged and conv == 1
    assert abs(used - ref.n_iters_used) <= 1, (used, ref.n_iters_used)
    # reg 0.03: the API keeps Adam (non-default lr) and Anderson below 0.05 (sinkhorn.py:1362-1390)
    name = {MOM: "momentum", ADAM: "adam", AND: "anderson"}[method]
    C = -la
    res = dot_amd.sinkhorn(_t(C), reg=0.03, n_iters=12, tol=0.0, method=name, **kw)
    at, tol_p = _fp32_spread(la, 0.03, 12, None, None, method=method, **kw)
    assert rel_err(res.transport_plan, at.P) < tol_p
    assert rel_err(res.cost, (at.P * C).sum((1, 2))) < tol_p


def test_schedule_with_start_equal_to_target_is_the_plain_iteration():
    la, _, _ = _case(3, 2, 48, 40)
    P_plain, _, _ = _gpu(la, 0.1, 30)
    for schedule in (LIN, EXP, COS):
        P, _, _ = _gpu(la, 0.1, 30, reg_start=0.1, schedule=schedule)
        assert rel_err(P, P_plain) < FWD_TOL


def test_schedule_return_log():
    la, lga, lgb = _case(5, 2, 33, 47, marginals=True)
    logP, _, _ = _gpu(la, 0.05, 12, 0.0, lga, lgb, schedule=COS, return_log=True)
    ref = _oracle(la, 0.05, 12, 0.0, lga, lgb, schedule=COS, return_log=True)
    assert np.abs(logP.cpu().numpy() - ref.P).max() < 1e-4


# ---------------------------------------------------------------------------
# Momentum
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("omega", [1.5, 1.2, 0.8])
@pytest.mark.parametrize("shape", SHAPES)
def test_momentum_matches_oracle(omega, shape):
    B, M, N = shape
    la, lga, lgb = _case(23 + N, B, M, N, marginals=(N == 256))
    for T in (1, 5, 30):
        print(f"momentum omega={omega} shape={shape} T={T}", flush=True)
        P, used, conv = _gpu(la, 0.1, T, 0.0, lga, lgb, method=MOM, omega=omega)
        ref = _oracle(la, 0.1, T, 0.0, lga, lgb, method=MOM, omega=omega)
        assert used == T and conv == 0
        assert rel_err(P, ref.P) < FWD_TOL, T


def test_momentum_omega_one_is_the_plain_iteration():
    la, lga, lgb = _case(7, 3, 50, 70, marginals=True)
    P, _, _ = _gpu(la, 0.05, 40, 0.0, lga, lgb, method=MOM, omega=1.0)
    ref = osk.dual_forward(la, 0.05, 40, 0.0, lga, lgb)
    assert rel_err(P, ref.P) < FWD_TOL


# ---------------------------------------------------------------------------
# Adam
# ---------------------------------------------------------------------------
def _fp32_spread(la, tau, T, lga, lgb, **kw):
    r64 = _oracle(la, tau, T, 0.0, lga, lgb, **kw)
    r32 = _oracle(la, tau, T, 0.0, lga, lgb, dtype=np.float32, **kw)
    return r64, max(FWD_TOL, 20.0 * rel_err(r32.P, r64.P))


@pytest.mark.parametrize("bias_correction", [True, False])
@pytest.mark.parametrize("shape", SHAPES[:3])
def test_adam_matches_oracle(bias_correction, shape):
    B, M, N = shape
    la, lga, lgb = _case(31 + M, B, M, N, marginals=(M == 64))
    kw = dict(method=ADAM, lr=0.5, beta1=0.9 if bias_correction else 0.0, beta2=0.999,
              bias_correction=bias_correction)
    for T in (1, 3, 20):
        print(f"adam bc={bias_correction} shape={shape} T={T}", flush=True)
        P, used, _ = _gpu(la, 0.1, T, 0.0, lga, lgb, **{**kw, "eps_adam": 1e-8})
        ref, tol = _fp32_spread(la, 0.1, T, lga, lgb, eps_adam=1e-8, **kw)
        assert used == T
        assert rel_err(P, ref.P) < tol, (T, tol)


# ---------------------------------------------------------------------------
# Anderson
# ---------------------------------------------------------------------------
def test_anderson_history_of_one_is_the_plain_iteration():
    la, lga, lgb = _case(41, 2, 45, 60, marginals=True)
    for T in (1, 6, 30):
        P, used, _ = _gpu(la, 0.1, T, 0.0, lga, lgb, method=AND, anderson_k=1)
        ref = osk.dual_forward(la, 0.1, T, 0.0, lga, lgb)
        assert used == T
        assert rel_err(P, ref.P) < FWD_TOL, T


@pytest.mark.parametrize("k", [2, 5, 16])
def test_anderson_early_iterations_match_oracle(k):
    la, _, _ = _case(43, 1, 36, 52)
    for T in (2, 3, 4):
        print(f"anderson k={k} T={T}", flush=True)
        P, _, _ = _gpu(la, 0.2, T, method=AND, anderson_k=k)
        ref, tol = _fp32_spread(la, 0.2, T, None, None, method=AND, anderson_k=k)
        assert rel_err(P, ref.P) < tol, (T, tol)


@pytest.mark.parametrize("B", [1, 3])
def test_anderson_reaches_the_vanilla_fixed_point(B):
    la, _, _ = _case(47, B, 24, 24)
    P, used, conv = _gpu(la, 0.1, 200, 1e-5, method=AND, anderson_k=5)
    ref = osk.dual_forward(la, 0.1, 2000, 1e-9)
    assert conv == 1 and used < 200
    assert rel_err(P, ref.P) < 1e-4


@pytest.mark.parametrize("k,T", [(20, 24), (40, 43), (100, 30)])
def test_anderson_long_histories(k, T):
    """Histories above 16 pairs (the reference takes any anderson_k >= 1,
    torch_cuda.cpp:290, :395-446): rings of 20 and 40 pairs that wrap, and
    anderson_k = 100 over 30 iterations (a ring of 30 pairs never wraps)."""
    la, _, _ = _case(61 + k, 1, 28, 33)
    print(f"anderson k={k} T={T}", flush=True)
    P, used, _ = _gpu(la, 0.5, T, method=AND, anderson_k=k)
    ref, tol = _fp32_spread(la, 0.5, T, None, None, method=AND, anderson_k=k)
    assert used == T and rel_err(P, ref.P) < tol, (k, T, tol)
    # through the public API, with the implicit backward
    C = torch.from_numpy(-la).to(DEV).requires_grad_(True)
    res = dot_amd.sinkhorn(C, reg=0.5, n_iters=T, tol=0, method="anderson", anderson_k=k)
    res.cost.sum().backward()
    assert rel_err(res.transport_plan, ref.P) < tol and torch.isfinite(C.grad).all()


def test_anderson_ring_beyond_its_length():
    # more iterations than the history holds: the ring wraps, oldest pairs drop
    la, _, _ = _case(53, 1, 30, 30)
    for k in (2, 3):
        P, _, _ = _gpu(la, 0.5, 9, method=AND, anderson_k=k)
        ref, tol = _fp32_spread(la, 0.5, 9, None, None, method=AND, anderson_k=k)
        assert rel_err(P, ref.P) < tol, (k, tol)


# ---------------------------------------------------------------------------
# Stop test, determinism, edge cases
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("method,kw,tol", [(VAN, {"schedule": COS, "reg_start": 0.15}, 1e-3),
                                           (MOM, {"omega": 1.4}, 1e-4), (ADAM, {"lr": 0.5}, 1e-4),
                                           (AND, {"anderson_k": 5}, 1e-4)])
def test_device_stop_test(method, kw, tol):
    la, _, _ = _case(59, 2, 40, 40)
    T = 150
    P, used, conv = _gpu(la, 0.1, T, tol, method=method, **kw)
    ref = _oracle(la, 0.1, T, tol, method=method, **kw)
    assert ref.converged and conv == 1
    if "schedule" in kw:
        # a schedule depends on the iteration budget: only the same stop compares
        assert used == ref.n_iters_used
        _, tol_p = _fp32_spread(la, 0.1, T, None, None, method=method, **kw)
        assert rel_err(P, ref.P) < tol_p
        return
    # fp32 and float64 can cross the tolerance one iteration apart
    assert abs(used - ref.n_iters_used) <= 1, (used, ref.n_iters_used)
    at, tol_p = _fp32_spread(la, 0.1, used, None, None, method=method, **kw)
    assert rel_err(P, at.P) < tol_p


def test_stop_test_past_the_host_check_interval():
    # convergence after more than 16 iterations: the host reads the stop flag
    # every 16 iterations and the count stays the device's
    la, _, _ = _case(61, 1, 32, 32)
    P, used, conv = _gpu(la, 0.02, 400, 1e-5, method=MOM, omega=1.1)
    ref = _oracle(la, 0.02, 400, 1e-5, method=MOM, omega=1.1)
    assert conv == 1 and 16 < used < 400
    assert abs(used - ref.n_iters_used) <= 1


@pytest.mark.parametrize("method", [MOM, AND, ADAM])
def test_methods_are_deterministic(method):
    la, _, _ = _case(67, 3, 70, 90)
    P1, u1, _ = _gpu(la, 0.1, 25, 1e-7, method=method, lr=0.5)
    P2, u2, _ = _gpu(la, 0.1, 25, 1e-7, method=method, lr=0.5)
    assert u1 == u2
    assert torch.equal(P1, P2)


def test_empty_shapes_and_zero_iterations():
    for shape in ((0, 4, 4), (2, 0, 5), (2, 5, 0)):
        P, used, conv = _gpu(np.zeros(shape, np.float32), 0.1, 10, 1e-6, method=MOM)
        assert P.shape == shape and used == 1 and conv == 1
    la, _, _ = _case(71, 2, 6, 7)
    P, used, conv = _gpu(la, 0.1, 0, method=ADAM)
    assert used == 0 and conv == 0
    ref = _oracle(la, 0.1, 0, method=ADAM)
    assert rel_err(P, ref.P) < FWD_TOL


def test_argument_errors():
    la = torch.rand(1, 4, 4, device=DEV)
    with pytest.raises(RuntimeError, match="anderson_k"):
        _ops.sinkhorn_dual_forward(la, 0.1, 5, 0.0, None, None, False, 2, 1.5, 0)
    with pytest.raises(RuntimeError, match="anderson_k and max_iter"):
        _ops.sinkhorn_dual_forward(la, 0.1, 65, 0.0, None, None, False, 2, 1.5, 65)
    with pytest.raises(RuntimeError, match="method"):
        _ops.sinkhorn_dual_forward(la, 0.1, 5, 0.0, None, None, False, 9)
    with pytest.raises(RuntimeError, match="schedule"):
        _ops.sinkhorn_dual_forward(la, 0.1, 5, 0.0, None, None, False, 0, 1.5, 5, 1.0, 1.0, 0.9, 0.999,
                                   1e-8, True, -1.0, 7)


# ---------------------------------------------------------------------------
# Python API: dispatch, cost and gradients
# ---------------------------------------------------------------------------
def test_api_momentum_cost_and_gradients_follow_the_reference():
    # cost = sum(P_method * C); its gradient: the direct term P_method plus the
    # implicit adjoint of the vanilla plan at n_iters_used (sinkhorn.py:155-240)
    rng = np.random.default_rng(73)
    C = rng.random((2, 30, 44)).astype(np.float32)
    tau, T, bw = 0.1, 40, 25
    cost = _t(C).requires_grad_(True)
    reg = torch.tensor(tau, device=DEV, requires_grad=True)
    res = dot_amd.sinkhorn(cost, reg=reg, n_iters=T, backward_iters=bw, method="momentum", omega=1.3, tol=0.0)
    assert res.n_iters_used == T and res.converged
    res.cost.sum().backward()
    ref = _oracle(-C, tau, T, method=MOM, omega=1.3)
    assert rel_err(res.transport_plan, ref.P) < FWD_TOL
    assert rel_err(res.cost, (ref.P * C).sum((1, 2))) < FWD_TOL
    _, g_la, g_tau = osk.with_grads_implicit(-C, C, tau, T, bw)
    expected = ref.P - g_la
    assert rel_err(cost.grad, expected) < GRAD_TOL
    assert sum_err(reg.grad.reshape(1), np.array([g_tau.sum()]), (g_la * C / tau).reshape(1, -1)) < GRAD_TOL


def test_api_dispatch_rules():
    cost = torch.rand(1, 12, 12, device=DEV)
    # momentum without omega and default Adam resolve to the vanilla solver on the GPU
    r = dot_amd.sinkhorn(cost, reg=0.1, n_iters=50, method="momentum")
    v = dot_amd.sinkhorn(cost, reg=0.1, n_iters=50)
    assert torch.equal(r.transport_plan, v.transport_plan)
    r = dot_amd.sinkhorn(cost, reg=0.1, n_iters=50, method="adam")
    assert torch.equal(r.transport_plan, v.transport_plan)
    # Anderson at tau <= 0.01 runs the exponential schedule from 10 tau
    r = dot_amd.sinkhorn(cost, reg=0.01, n_iters=30, method="anderson", tol=0.0)
    s = dot_amd.sinkhorn(cost, reg=0.01, n_iters=30, method="anderson", schedule="exponential", reg_start=0.1,
                         tol=0.0)
    assert rel_err(r.transport_plan, s.transport_plan.cpu()) < FWD_TOL
    with pytest.raises(ValueError, match="only supports implicit"):
        dot_amd.sinkhorn(cost, reg=0.1, n_iters=5, method="momentum", omega=1.5, backward_mode="unrolled")
    with pytest.raises(ValueError, match="schedule is only supported"):
        dot_amd.sinkhorn(cost, reg=0.1, n_iters=5, schedule="linear", backward_mode="unrolled")
    # dual=False runs the reference's PyTorch momentum solver (sinkhorn.py:1531-1556)
    r = dot_amd.sinkhorn(cost, reg=0.1, n_iters=5, method="momentum", omega=1.5, dual=False)
    P, used = solvers.momentum_forward(-cost, 0.1, 5, None, None, 1.5)
    assert torch.equal(r.transport_plan, P) and r.n_iters_used == used


# ---------------------------------------------------------------------------
# The reference's method tests (test_sinkhorn.py:427-666) on HIP tensors
# ---------------------------------------------------------------------------
def _grid_cost(n, lo=-1.0, hi=1.0, weight=None):
    grid = torch.linspace(lo, hi, n)
    c = (grid[:, None] - grid[None, :]).abs().pow(2)
    if weight is not None:
        c = c * torch.linspace(1.0, weight, n).unsqueeze(0)
    return c.unsqueeze(0).to(DEV)


def _vanilla_convergence_iters(cost, tau, max_iters, tol=1e-6):
    ref = osk.dual_forward(-cost.cpu().numpy(), tau, max_iters, tol)
    return ref.n_iters_used if ref.converged else max_iters


def test_ref_momentum_matches_vanilla():
    cost = torch.rand(1, 12, 12, device=DEV)
    vanilla = dot_amd.sinkhorn(cost, reg=1.0, n_iters=80)
    momentum = dot_amd.sinkhorn(cost, reg=1.0, n_iters=80, method="momentum", omega=1.5)
    assert torch.allclose(vanilla.transport_plan, momentum.transport_plan, atol=1e-4)


def test_ref_momentum_uses_fewer_iterations_than_vanilla():
    cost = _grid_cost(32)
    vanilla_iters = _vanilla_convergence_iters(cost, 0.02, 120)
    momentum = dot_amd.sinkhorn(cost, reg=0.02, n_iters=120, method="momentum", omega=1.4)
    assert momentum.n_iters_used is not None and momentum.n_iters_used < vanilla_iters


def test_ref_anderson_matches_vanilla():
    cost = torch.rand(1, 12, 12, device=DEV)
    vanilla = dot_amd.sinkhorn(cost, reg=0.1, n_iters=120)
    anderson = dot_amd.sinkhorn(cost, reg=0.1, n_iters=120, method="anderson", anderson_k=5)
    assert torch.allclose(vanilla.transport_plan, anderson.transport_plan, atol=1e-4)


def test_ref_anderson_uses_fewer_iterations_than_vanilla():
    # at tau = 0.02 the GPU path keeps Anderson (0.01 < tau < 0.05, sinkhorn.py:1374-1380)
    cost = _grid_cost(32)
    vanilla_iters = _vanilla_convergence_iters(cost, 0.02, 120)
    anderson = dot_amd.sinkhorn(cost, reg=0.02, n_iters=120, method="anderson", anderson_k=5)
    assert anderson.n_iters_used is not None and anderson.n_iters_used < vanilla_iters


def test_ref_anderson_backward_matches_vanilla():
    cost = torch.rand(1, 10, 10, device=DEV)
    cost_vanilla = cost.clone().requires_grad_(True)
    vanilla = dot_amd.sinkhorn(cost_vanilla, reg=0.1, n_iters=120)
    vanilla.cost.sum().backward()
    cost_anderson = cost.clone().requires_grad_(True)
    anderson = dot_amd.sinkhorn(cost_anderson, reg=0.1, n_iters=120, method="anderson", anderson_k=5)
    anderson.cost.sum().backward()
    assert torch.allclose(vanilla.transport_plan, anderson.transport_plan, atol=1e-4)
    assert torch.allclose(cost_vanilla.grad, cost_anderson.grad, atol=1e-4)


def test_ref_adam_matches_vanilla_on_well_conditioned_problem():
    torch.manual_seed(0)
    cost = torch.rand(1, 12, 12).to(DEV)
    vanilla = dot_amd.sinkhorn(cost, reg=0.1, n_iters=200)
    adam = dot_amd.sinkhorn(cost, reg=0.1, n_iters=200, method="adam", lr=0.5)
    assert torch.allclose(vanilla.transport_plan, adam.transport_plan, atol=5e-4)


def test_ref_adam_handles_nonuniform_costs():
    cost = _grid_cost(24, -2.0, 2.0, weight=3.0)
    result = dot_amd.sinkhorn(cost, reg=0.02, n_iters=40, method="adam", lr=0.5)
    assert torch.isfinite(result.transport_plan).all()
    assert result.n_iters_used is not None


def test_ref_adam_rmsprop_regime_can_beat_vanilla():
    # The reference's test (test_sinkhorn.py:544-566) runs its CPU PyTorch
    # solver.  On its CUDA path, restated by the oracle, this regime's first
    # RMSprop step (lr / sqrt(1 - beta2) = 7.9 units) never passes the
    # candidate test, so the run is the plain iteration and both errors agree
    # (oracle: 2.6173e-6 each); the strict inequality would be decided by
    # rounding.  Checked here: no worse than vanilla, and equal to the
    # oracle's error.
    cost = _grid_cost(32, -3.0, 3.0, weight=5.0)
    tau = 0.02
    ref = dot_amd.sinkhorn(cost, reg=tau, n_iters=800)
    vanilla = dot_amd.sinkhorn(cost, reg=tau, n_iters=20)
    rms = dot_amd.sinkhorn(cost, reg=tau, n_iters=20, method="adam", lr=0.25, beta1=0.0, beta2=0.999,
                           bias_correction=False)
    rms_err = float((rms.transport_plan - ref.transport_plan).abs().mean())
    van_err = float((vanilla.transport_plan - ref.transport_plan).abs().mean())
    assert rms_err <= van_err * (1 + 1e-4)
    la = -cost.cpu().numpy()
    o_ref = osk.dual_forward(la, tau, 800, 1e-6)
    o_rms = osk.dual_forward_method(la, tau, 20, 1e-6, method=ADAM, lr=0.25, beta1=0.0, beta2=0.999,
                                    bias_correction=False)
    assert abs(rms_err - float(np.abs(o_rms.P - o_ref.P).mean())) < 1e-3 * rms_err


def test_ref_adam_bias_correction_can_hurt_deterministic_residuals():
    cost = _grid_cost(32, -3.0, 3.0, weight=5.0)
    tau = 0.02
    ref = dot_amd.sinkhorn(cost, reg=tau, n_iters=800)
    default = dot_amd.sinkhorn(cost, reg=tau, n_iters=20, method="adam", lr=0.5)
    rms = dot_amd.sinkhorn(cost, reg=tau, n_iters=20, method="adam", lr=0.25, beta1=0.0, beta2=0.999,
                           bias_correction=False)
    assert (rms.transport_plan - ref.transport_plan).abs().mean() < \
        (default.transport_plan - ref.transport_plan).abs().mean()


def test_ref_adam_backward_works():
    cost = torch.rand(1, 10, 10, device=DEV, requires_grad=True)
    result = dot_amd.sinkhorn(cost, reg=0.1, n_iters=80, method="adam", lr=0.5)
    result.cost.sum().backward()
    assert cost.grad is not None and torch.isfinite(cost.grad).all()


def test_ref_scheduled_vanilla_matches_unscheduled_when_reg_start_equals_target():
    cost = torch.rand(1, 12, 12, device=DEV)
    vanilla = dot_amd.sinkhorn(cost, reg=0.1, n_iters=200)
    scheduled = dot_amd.sinkhorn(cost, reg=0.1, n_iters=200, schedule="cosine", reg_start=0.1)
    assert torch.allclose(vanilla.transport_plan, scheduled.transport_plan, atol=1e-4)


def test_ref_scheduled_vanilla_handles_small_epsilon_better_than_vanilla():
    torch.manual_seed(4)
    base = torch.rand(24, 24)
    cost = ((base + base.t()) / 2).unsqueeze(0).to(DEV)
    tau = 0.001
    ref = dot_amd.sinkhorn(cost, reg=tau, n_iters=600)
    vanilla = dot_amd.sinkhorn(cost, reg=tau, n_iters=10)
    scheduled = dot_amd.sinkhorn(cost, reg=tau, n_iters=10, schedule="linear", reg_start=0.1)
    assert (scheduled.transport_plan - ref.transport_plan).abs().mean() < \
        (vanilla.transport_plan - ref.transport_plan).abs().mean()


def test_ref_scheduled_vanilla_backward_works():
    cost = torch.rand(1, 10, 10, device=DEV, requires_grad=True)
    result = dot_amd.sinkhorn(cost, reg=0.01, n_iters=80, schedule="cosine", reg_start=0.1)
    result.cost.sum().backward()
    assert cost.grad is not None and torch.isfinite(cost.grad).all()


def test_ref_scheduled_anderson_matches_unscheduled_when_reg_start_equals_target():
    cost = torch.rand(1, 12, 12, device=DEV)
    anderson = dot_amd.sinkhorn(cost, reg=0.1, n_iters=120, method="anderson", anderson_k=5)
    scheduled = dot_amd.sinkhorn(cost, reg=0.1, n_iters=120, method="anderson", anderson_k=5,
                                 schedule="cosine", reg_start=0.1)
    assert torch.allclose(anderson.transport_plan, scheduled.transport_plan, atol=1e-4)


def test_ref_scheduled_anderson_works():
    cost = torch.rand(1, 12, 12, device=DEV, requires_grad=True)
    result = dot_amd.sinkhorn(cost, reg=0.01, n_iters=80, method="anderson", schedule="cosine", reg_start=0.1)
    result.cost.sum().backward()
    assert cost.grad is not None and torch.isfinite(cost.grad).all()
