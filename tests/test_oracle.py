"""CPU: the oracle against the reference's golden vectors and independent checks.

The golden fixtures (tests/golden/*.npz) hold outputs of the reference's own
compiled CPU kernels (src/sinkhorn/kernels_cpu.cpp,
src/bidirectional_softmax/kernels_cpu.cpp).  The independent checks fix what a
restatement could plausibly get wrong (a sign, an index, a dropped term): a
rank-one kernel converges in one iteration to a b^T, columns match b exactly
after every iteration, shifts of rows/columns leave the plan unchanged, the
implicit gradient at convergence equals float64 autograd through the fixed
point, grad_tau equals a finite difference in tau, and the bidirectional
softmax equals its closed form with torch.softmax and its autograd gradient.
"""

import numpy as np
import pytest
import torch

from conftest import load_golden, rel_err, sum_err
from oracle import bidirectional_softmax as obs
from oracle import ref
from oracle import sinkhorn as osk

FWD_TOL = 1e-5    # plan / cost, norm-wise relative
GRAD_TOL = 1e-4   # gradients


# ---------------------------------------------------------------------------
# Golden vectors of the reference's CPU kernels
# ---------------------------------------------------------------------------
def test_forward_matches_reference_golden_6x9():
    g = load_golden("sk_fwd_6x9")
    f = osk.dual_forward(g["log_alpha"], float(g["tau"]), int(g["n_iters"]), 0.0, g["log_a"], g["log_b"])
    assert rel_err(f.P, g["P"]) < FWD_TOL
    f_log = osk.dual_forward(g["log_alpha"], float(g["tau"]), int(g["n_iters"]), 0.0, g["log_a"],
                             g["log_b"], return_log=True)
    assert np.abs(f_log.P - g["logP"]).max() < 1e-4


def test_forward_matches_reference_golden_c1():
    g = load_golden("sk_c1")
    f = osk.dual_forward(-g["cost"], float(g["tau"]), int(g["n_iters"]))
    assert rel_err(f.P, g["P"]) < FWD_TOL


def test_forward_matches_reference_golden_small_reg():
    g = load_golden("sk_fwd_smallreg")
    f = osk.dual_forward(-g["cost"], float(g["tau"]), int(g["n_iters"]))
    assert rel_err(f.P, g["P"]) < FWD_TOL


def test_implicit_backward_matches_reference_golden():
    g = load_golden("sk_c1")
    la, C = -g["cost"], g["cost"]
    f = osk.dual_forward(la, float(g["tau"]), int(g["n_iters"]))
    grad, gtau, sweeps = osk.implicit_backward(la, f.P, C, float(g["tau"]), int(g["backward_iters"]))
    assert (sweeps == int(g["backward_iters"])).all()
    assert rel_err(grad, g["grad_fixed"]) < GRAD_TOL
    assert rel_err(gtau, g["grad_tau_fixed"]) < GRAD_TOL
    # CPU semantics: per-batch early break at max change < 1e-6 (kernels_cpu.cpp:309-311)
    grad_c, gtau_c, sweeps_c = osk.implicit_backward(la, f.P, C, float(g["tau"]),
                                                     int(g["backward_iters"]), tol=1e-6)
    assert (sweeps_c < int(g["backward_iters"])).all()
    assert rel_err(grad_c, g["grad_cpu"]) < GRAD_TOL
    assert rel_err(gtau_c, g["grad_tau_cpu"]) < GRAD_TOL


def test_grads_match_reference_golden_rectangular_nonuniform():
    g = load_golden("sk_grads_8x16")
    la, G, tau, T, BT = g["log_alpha"], g["grad_P"], float(g["tau"]), int(g["n_iters"]), int(g["backward_iters"])
    P, gi, gti = osk.with_grads_implicit(la, G, tau, T, BT, g["log_a"], g["log_b"])
    assert rel_err(P, g["P"]) < FWD_TOL
    assert rel_err(gi, g["grad_implicit"]) < GRAD_TOL
    assert rel_err(gti, g["grad_tau_implicit"]) < GRAD_TOL
    gic, gtic, _ = osk.implicit_backward(la, P, G, tau, BT, tol=1e-6)
    assert rel_err(gic, g["grad_implicit_cpu"]) < GRAD_TOL
    assert rel_err(gtic, g["grad_tau_implicit_cpu"]) < GRAD_TOL
    Pu, gu, gtu = osk.with_grads_unrolled(la, G, tau, T, g["log_a"], g["log_b"])
    assert rel_err(Pu, g["P_unrolled"]) < FWD_TOL
    assert rel_err(gu, g["grad_unrolled"]) < GRAD_TOL
    assert rel_err(gtu, g["grad_tau_unrolled"]) < GRAD_TOL


def test_unrolled_matches_reference_golden_48x64():
    g = load_golden("sk_unrolled_48x64")
    C = g["cost"]
    P, gu, gtu = osk.with_grads_unrolled(-C, C, float(g["tau"]), int(g["n_iters"]))
    assert rel_err(P, g["P"]) < FWD_TOL
    assert rel_err(gu, g["grad_unrolled"]) < GRAD_TOL
    assert rel_err(gtu, g["grad_tau_unrolled"]) < GRAD_TOL


@pytest.mark.parametrize("name", ["bidi_varlen", "bidi_full", "bidi_64x80"])
def test_bidi_matches_reference_golden(name):
    g = load_golden(name)
    tau = float(g["tau"])
    out, r, c = obs.forward(g["sim"], tau, g["lengths"])
    assert rel_err(out, g["out"]) < FWD_TOL
    assert rel_err(r, g["row_sm"]) < FWD_TOL
    assert rel_err(c, g["col_sm"]) < FWD_TOL
    gs, gt = obs.backward(g["sim"], g["out"], g["grad_out"], g["row_sm"], g["col_sm"], tau, g["lengths"])
    assert rel_err(gs, g["grad_sim"]) < GRAD_TOL
    assert rel_err(gt, g["grad_tau"]) < GRAD_TOL


def test_bidi_matches_reference_golden_temperatures():
    g = load_golden("bidi_diag")
    for name, tau in (("sharp", 0.1), ("soft", 10.0)):
        out, r, c = obs.forward(g["sim"], tau, g["lengths"])
        assert rel_err(out, g[f"out_{name}"]) < FWD_TOL
        gs, gt = obs.backward(g["sim"], out, g["grad_out"], r, c, tau, g["lengths"])
        # With a diagonal sim and a ones upstream gradient the exact gradient is 0 at
        # both temperatures; both sides hold ~1e-9 of rounding noise, so only an
        # absolute bound is meaningful here.
        assert np.abs(gs).max() < 1e-6 and np.abs(g[f"grad_sim_{name}"]).max() < 1e-6
    sharp, soft = g["out_sharp"][0], g["out_soft"][0]
    assert np.trace(sharp) > np.trace(soft)


# ---------------------------------------------------------------------------
# Independent pins of the Sinkhorn restatement
# ---------------------------------------------------------------------------
def _dirichlet(rng, B, n):
    e = -np.log(rng.random((B, n)))
    return (e / e.sum(1, keepdims=True)).astype(np.float32)


def test_rank_one_kernel_converges_in_one_iteration():
    # log_alpha_ij = f_i + g_j: the row then column update gives exactly a b^T.
    rng = np.random.default_rng(1)
    f, g = rng.standard_normal((2, 7, 1)), rng.standard_normal((2, 1, 11))
    la = (f + g).astype(np.float32)
    a, b = _dirichlet(rng, 2, 7), _dirichlet(rng, 2, 11)
    out = osk.dual_forward(la, 0.5, 1, 0.0, np.log(a), np.log(b))
    assert np.abs(out.P - a[:, :, None] * b[:, None, :]).max() < 1e-6


def test_columns_match_b_after_every_iteration_and_rows_converge():
    rng = np.random.default_rng(2)
    la = -rng.random((2, 9, 13)).astype(np.float32)
    a, b = _dirichlet(rng, 2, 9), _dirichlet(rng, 2, 13)
    for T in (1, 3, 10):
        P = osk.dual_forward(la, 0.3, T, 0.0, np.log(a), np.log(b)).P
        assert np.abs(P.sum(1) - b).max() < 1e-7  # column update is the last step
    P = osk.dual_forward(la, 0.3, 400, 0.0, np.log(a), np.log(b)).P
    assert np.abs(P.sum(2) - a).max() < 1e-7


def test_plan_is_invariant_to_row_and_column_shifts():
    rng = np.random.default_rng(3)
    la = -rng.random((1, 6, 8)).astype(np.float32)
    shifted = (la + rng.standard_normal((1, 6, 1)) + rng.standard_normal((1, 1, 8))).astype(np.float32)
    P1 = osk.dual_forward(la, 0.7, 30).P
    P2 = osk.dual_forward(shifted, 0.7, 30).P
    assert rel_err(P2, P1) < 1e-5


def _torch_converged_loss(la, tau, G, iters=3000):
    """float64 autograd through a converged dual Sinkhorn: the exact gradient of the fixed point."""
    x = torch.tensor(la, dtype=torch.float64, requires_grad=True)
    K = x / tau
    B, n, m = K.shape
    log_a = torch.full((B, n), -np.log(n), dtype=torch.float64)
    log_b = torch.full((B, m), -np.log(m), dtype=torch.float64)
    v = torch.zeros(B, m, dtype=torch.float64)
    for _ in range(iters):
        u = log_a - torch.logsumexp(K + v[:, None, :], dim=2)
        v = log_b - torch.logsumexp(K + u[:, :, None], dim=1)
    P = torch.exp(K + u[:, :, None] + v[:, None, :])
    loss = (P * torch.tensor(G, dtype=torch.float64)).sum()
    loss.backward()
    return x.grad.numpy()


def test_implicit_gradient_at_convergence_equals_autograd():
    rng = np.random.default_rng(4)
    la = -rng.random((2, 5, 7)).astype(np.float32)
    G = rng.standard_normal((2, 5, 7)).astype(np.float32)
    tau = 0.5  # exact in fp32, so the oracle's fp32 1/tau equals the float64 one
    fwd = osk.dual_forward(la, tau, 3000)
    grad, _, _ = osk.implicit_backward(la, fwd.P, G, tau, 3000)
    exact = _torch_converged_loss(la, tau, G)
    # 1e-6 rather than 1e-12: the oracle rounds -log(n) to fp32 as the reference does
    assert rel_err(grad, exact) < 1e-6


def test_grad_tau_matches_finite_difference():
    rng = np.random.default_rng(5)
    la = -rng.random((1, 6, 6)).astype(np.float32)
    G = rng.standard_normal((1, 6, 6))
    tau, h = 0.6, 1e-6

    def loss(t):
        # float64 all the way: la / t in float64 to make the difference smooth in t
        K = la.astype(np.float64) / t
        u = np.zeros((1, 6))
        v = np.zeros((1, 6))
        lg = -np.log(6.0)
        for _ in range(3000):
            u = lg - osk._lse(K + v[:, None, :], 2)
            v = lg - osk._lse(K + u[:, :, None], 1)
        return float((np.exp(K + u[:, :, None] + v[:, None, :]) * G).sum())

    fd = (loss(tau + h) - loss(tau - h)) / (2 * h)
    fwd = osk.dual_forward(la, tau, 3000)
    _, gtau, _ = osk.implicit_backward(la, fwd.P, G, tau, 3000)
    assert abs(gtau[0] - fd) < 1e-5 * max(1.0, abs(fd))


def test_unrolled_formula_is_not_the_exact_jacobian():
    # The reference's unrolled backward drops the log-marginal terms (kernels_cpu.cpp:206-232);
    # with non-uniform marginals and few iterations it differs from autograd, which is why
    # only the golden vectors can pin it.
    rng = np.random.default_rng(6)
    la = -rng.random((1, 4, 5)).astype(np.float32)
    a, b = _dirichlet(rng, 1, 4), _dirichlet(rng, 1, 5)
    G = rng.standard_normal((1, 4, 5)).astype(np.float32)
    _, g_unr, _ = osk.with_grads_unrolled(la, G, 1.0, 3, np.log(a), np.log(b))
    x = torch.tensor(la, dtype=torch.float64, requires_grad=True)
    K = x / 1.0
    la_t, lb_t = torch.tensor(np.log(a), dtype=torch.float64), torch.tensor(np.log(b), dtype=torch.float64)
    v = torch.zeros(1, 5, dtype=torch.float64)
    for _ in range(3):
        u = la_t - torch.logsumexp(K + v[:, None, :], dim=2)
        v = lb_t - torch.logsumexp(K + u[:, :, None], dim=1)
    (torch.exp(K + u[:, :, None] + v[:, None, :]) * torch.tensor(G, dtype=torch.float64)).sum().backward()
    assert rel_err(g_unr, x.grad.numpy()) > 1e-2


def test_early_stop_property_of_reference_tests():
    # test_sinkhorn.py:827-839: 256x256 rand cost, reg 0.1, n_iters 50 stops early, plan within 2e-3.
    C = torch.rand(1, 256, 256, generator=torch.Generator().manual_seed(0)).numpy()
    early = osk.dual_forward(-C, 0.1, 50, tol=1e-6)
    fixed = osk.dual_forward(-C, 0.1, 50, tol=0.0)
    assert early.converged and early.n_iters_used < 50
    assert fixed.n_iters_used == 50 and not fixed.converged
    assert np.abs(early.P - fixed.P).max() < 2e-3
    # The stop fires at the first iteration whose batch-global u change is below tol
    assert early.deltas[early.n_iters_used - 1] < 1e-6
    assert (early.deltas[: early.n_iters_used - 1] >= 1e-6).all()


def test_early_stop_count_convention_rank_one():
    # K_ij = x_i + y_j is exact after one iteration (u_2 = u_1 up to the float32
    # rounding of the inputs, ~1e-7 here), so the
    # u-change test fires at iteration 2: used_iters = iter + 1 at the break
    # (torch_cuda.cpp:223-236).  A count off by one in either direction fails.
    rng = np.random.default_rng(11)
    for B, n, m in ((1, 5, 7), (3, 16, 9), (2, 33, 64)):
        x = rng.standard_normal((B, n, 1))
        y = rng.standard_normal((B, 1, m))
        la = (x + y).astype(np.float32)
        a = rng.random((B, n)) + 0.1
        b = rng.random((B, m)) + 0.1
        lga = np.log(a / a.sum(-1, keepdims=True)).astype(np.float32)
        lgb = np.log(b / b.sum(-1, keepdims=True)).astype(np.float32)
        f = osk.dual_forward(la, 0.7, 50, tol=1e-5, log_a=lga, log_b=lgb)
        assert f.converged and f.n_iters_used == 2, f.deltas
        assert f.deltas[0] > 1e-3


def test_u_and_v_stop_criteria_coincide():
    # The column update v = log b - LSE_i(K + u) is 1-Lipschitz in the max
    # norm, so max|dv_t| <= max|du_t| at every t: a u-and-v criterion stops at
    # the same iteration as the reference's u-only one on every input.
    rng = np.random.default_rng(12)
    for trial in range(12):
        B, n, m = 2, int(rng.integers(3, 40)), int(rng.integers(3, 40))
        la = -rng.random((B, n, m)).astype(np.float32) * float(rng.choice([0.5, 2.0, 8.0]))
        lga = lgb = None
        if trial % 2:
            ea = -np.log(rng.random((B, n)))
            eb = -np.log(rng.random((B, m)))
            lga = np.log(ea / ea.sum(-1, keepdims=True)).astype(np.float32)
            lgb = np.log(eb / eb.sum(-1, keepdims=True)).astype(np.float32)
        f = osk.dual_forward(la, float(rng.choice([0.05, 0.2, 1.0])), 60, log_a=lga, log_b=lgb,
                             keep_history=True)
        du = np.abs(np.diff(f.u_hist, axis=0, prepend=0.0)).max(axis=(1, 2))
        dv = np.abs(np.diff(f.v_hist, axis=0)).max(axis=(1, 2))
        assert (dv <= du[1:] * (1 + 1e-9) + 1e-12).all()


def test_early_stop_criterion_is_batch_global():
    # One slow batch element keeps the whole batch iterating (torch_cuda.cpp:226-233).
    rng = np.random.default_rng(7)
    fast = -0.01 * rng.random((1, 16, 16)).astype(np.float32)
    slow = -rng.random((1, 16, 16)).astype(np.float32)
    alone = osk.dual_forward(fast, 0.05, 500, tol=1e-6).n_iters_used
    both = osk.dual_forward(np.concatenate([fast, slow]), 0.05, 500, tol=1e-6).n_iters_used
    assert both > alone


# ---------------------------------------------------------------------------
# Independent pins of the bidirectional softmax restatement
# ---------------------------------------------------------------------------
def _torch_bidi(sim, tau, lengths):
    s = torch.tensor(sim, dtype=torch.float64, requires_grad=True)
    inv_t = float(np.float32(1.0) / np.float32(tau))
    y = s * inv_t
    B, L1, L2 = s.shape
    ln = torch.tensor(lengths, dtype=torch.long)
    rows = torch.arange(L1)[None, :, None] < ln[:, 0][:, None, None]
    cols = torch.arange(L2)[None, None, :] < ln[:, 1][:, None, None]
    mask = rows & cols
    ym = y.masked_fill(~mask, float("-inf"))
    r = torch.nan_to_num(torch.softmax(ym, dim=2), nan=0.0)
    c = torch.nan_to_num(torch.softmax(ym, dim=1), nan=0.0)
    out = torch.where(mask, torch.sqrt(1e-9 + r * c), torch.zeros_like(r))
    return s, out


def test_bidi_closed_form_and_autograd():
    rng = np.random.default_rng(8)
    sim = rng.standard_normal((3, 9, 14)).astype(np.float32)
    lengths = np.array([[9, 14], [5, 11], [1, 1]], np.int32)
    G = rng.standard_normal(sim.shape)
    tau = 0.7
    s, out_t = _torch_bidi(sim, tau, lengths)
    out, r, c = obs.forward(sim, tau, lengths)
    # the oracle rounds sim * (1/tau) to fp32 as the reference does; float64 otherwise
    assert rel_err(out, out_t.detach().numpy()) < 1e-6
    out_t.backward(torch.tensor(G))
    gs, _ = obs.backward(sim, out, G, r, c, tau, lengths)
    assert rel_err(gs, s.grad.numpy()) < 1e-6


# ---------------------------------------------------------------------------
# Oracle vs the compiled reference on more shapes (only where oracle/_ref is built)
# ---------------------------------------------------------------------------
needs_ref = pytest.mark.skipif(not ref.available(), reason="oracle/_ref not built (no /root/reference)")


@needs_ref
@pytest.mark.parametrize("shape,tau,T", [((3, 17, 5), 0.3, 40), ((2, 33, 64), 0.05, 150),
                                         ((1, 128, 100), 1.0, 10)])
def test_oracle_vs_compiled_reference(shape, tau, T):
    rng = np.random.default_rng(sum(shape))
    la = -rng.random(shape).astype(np.float32)
    G = rng.standard_normal(shape).astype(np.float32)
    a, b = _dirichlet(rng, shape[0], shape[1]), _dirichlet(rng, shape[0], shape[2])
    P_ref, g_ref, gt_ref = ref.sinkhorn_with_grads_implicit(la, G, tau, T, T, np.log(a), np.log(b), tol=0.0)
    P, g, gt = osk.with_grads_implicit(la, G, tau, T, T, np.log(a), np.log(b))
    assert rel_err(P, P_ref) < FWD_TOL
    assert rel_err(g, g_ref) < GRAD_TOL
    assert sum_err(gt, gt_ref, g * la / tau) < GRAD_TOL
    Pu_ref, gu_ref, gtu_ref = ref.sinkhorn_with_grads_unrolled(la, G, tau, min(T, 25), np.log(a), np.log(b))
    Pu, gu, gtu = osk.with_grads_unrolled(la, G, tau, min(T, 25), np.log(a), np.log(b))
    assert rel_err(gu, gu_ref) < GRAD_TOL
    assert sum_err(gtu, gtu_ref, gu * la / tau) < GRAD_TOL


def _centred_svd_top(log_alpha, tau):
    """Largest singular value of C_M P C_N (C the centring projector) per batch
    element, by numpy's SVD in float64."""
    K = log_alpha / tau
    P = np.exp(K - np.log(np.exp(K - K.max(-1, keepdims=True)).sum(-1, keepdims=True)) - K.max(-1, keepdims=True))
    out = []
    for Pb in P:
        M, N = Pb.shape
        CM = np.eye(M) - 1.0 / M
        CN = np.eye(N) - 1.0 / N
        out.append(np.linalg.svd(CM @ Pb @ CN, compute_uv=False)[0])
    return np.array(out)


def test_spectral_preflight_converges_to_centred_singular_value():
    """The deflated power iteration's limit is sigma_max(C_M P C_N): a missing
    centring step would converge to sigma_max(P) >= 1 instead."""
    rng = np.random.default_rng(11)
    X = 0.5 * rng.standard_normal((3, 20, 15))
    for tau in (0.4, 1.5):
        est = osk.spectral_preflight_tau(X, tau, 400)
        ref_sv = _centred_svd_top(X, tau)
        assert np.all(ref_sv < 0.999)
        np.testing.assert_allclose(est, ref_sv, rtol=1e-6)


def test_spectral_preflight_rank_one_plan_gives_the_floor():
    """Rows of log_alpha that are constant give P = 1 1^T / N, whose centred
    image vanishes: the estimate is the 1e-12 floor under the root."""
    X = np.repeat(np.linspace(-1, 1, 9)[:, None], 7, axis=1)[None].repeat(2, 0)
    est = osk.spectral_preflight_tau(X, 0.3, 5)
    np.testing.assert_allclose(est, 1e-6, rtol=1e-9)


# --- accelerated methods and regularisation schedules (torch_cuda.cpp:323-557) ---
def _small_problem(seed=0, B=2, n=12, m=10):
    rng = np.random.default_rng(seed)
    return -rng.random((B, n, m)).astype(np.float32)


def test_momentum_with_unit_omega_is_vanilla_step_for_step():
    la = _small_problem(1)
    ref_ = osk.dual_forward_method(la, 0.1, 37, 0.0)
    mom = osk.dual_forward_method(la, 0.1, 37, 0.0, method=osk.METHOD_MOMENTUM, omega=1.0)
    np.testing.assert_array_equal(mom.u, ref_.u)
    np.testing.assert_array_equal(mom.v, ref_.v)
    # and the method-free path is the vanilla oracle itself
    van = osk.dual_forward(la, 0.1, 37, 0.0)
    np.testing.assert_allclose(ref_.u, van.u, rtol=0, atol=0)


def test_anderson_with_history_of_one_is_vanilla_step_for_step():
    la = _small_problem(2)
    van = osk.dual_forward(la, 0.2, 25, 0.0)
    aa = osk.dual_forward_method(la, 0.2, 25, 0.0, method=osk.METHOD_ANDERSON, anderson_k=1)
    np.testing.assert_allclose(aa.u, van.u, rtol=0, atol=1e-12)
    np.testing.assert_allclose(aa.v, van.v, rtol=0, atol=1e-12)


@pytest.mark.parametrize("schedule", [osk.SCHEDULE_COSINE, osk.SCHEDULE_EXPONENTIAL])
def test_schedule_starting_at_the_target_is_unscheduled(schedule):
    la = _small_problem(3)
    van = osk.dual_forward(la, 0.1, 30, 0.0)
    sch = osk.dual_forward_method(la, 0.1, 30, 0.0, schedule=schedule, reg_start=0.1)
    np.testing.assert_array_equal(sch.u, van.u)


def test_schedule_endpoints_and_shape():
    for sched in (osk.SCHEDULE_LINEAR, osk.SCHEDULE_COSINE, osk.SCHEDULE_EXPONENTIAL):
        taus = [float(osk.scheduled_tau(t, 11, 0.01, 0.5, sched)) for t in range(11)]
        assert abs(taus[0] - 0.5) < 1e-6 and abs(taus[-1] - 0.01) < 1e-7, (sched, taus)
        assert all(a >= b for a, b in zip(taus, taus[1:])), sched
    # default start 10 tau; exponential midpoint is the geometric mean
    assert abs(float(osk.scheduled_tau(0, 5, 0.02, -1.0, osk.SCHEDULE_LINEAR)) - 0.2) < 1e-7
    mid = float(osk.scheduled_tau(5, 11, 0.01, 1.0, osk.SCHEDULE_EXPONENTIAL))
    assert abs(mid - 0.1) < 1e-7


@pytest.mark.parametrize("method,kw", [
    (osk.METHOD_MOMENTUM, dict(omega=1.5)),
    (osk.METHOD_ADAM, dict(lr=0.5)),
    (osk.METHOD_ANDERSON, dict(anderson_k=5)),
])
def test_methods_reach_the_vanilla_fixed_point(method, kw):
    la = _small_problem(4, B=2, n=12, m=12)
    van = osk.dual_forward(la, 0.1, 400, 0.0)
    r = osk.dual_forward_method(la, 0.1, 400, 0.0, method=method, **kw)
    np.testing.assert_allclose(r.P, van.P, rtol=0, atol=1e-7)


def test_anderson_ring_longer_than_the_run_never_wraps():
    # A ring of anderson_k pairs over T < anderson_k iterations holds every
    # push (torch_cuda.cpp:395-420), so it equals a ring of T pairs: the build
    # holds min(anderson_k, max_iter) pairs and accepts any anderson_k.
    la = -np.random.default_rng(5).random((2, 9, 11)).astype(np.float32)
    a = osk.dual_forward_method(la, 0.3, 12, method=osk.METHOD_ANDERSON, anderson_k=100)
    b = osk.dual_forward_method(la, 0.3, 12, method=osk.METHOD_ANDERSON, anderson_k=12)
    c = osk.dual_forward_method(la, 0.3, 12, method=osk.METHOD_ANDERSON, anderson_k=11)
    assert np.array_equal(a.P, b.P)
    assert not np.array_equal(a.P, c.P)  # a ring one pair shorter does wrap
