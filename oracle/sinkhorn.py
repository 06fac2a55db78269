"""TEST INFRASTRUCTURE ONLY — numpy restatement of the reference's Sinkhorn hot path.

This is the checker the HIP kernels are compared against.  Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import
it, and never as a product code path: the ``dot_amd`` package does not import
anything under ``oracle/``.

Every function follows the reference's GPU semantics unless it says otherwise,
and computes in float64 by default (``dtype=np.float32`` gives an fp32 run of
the same algorithm, used to measure the rounding spread of fp32 itself).

Pinning (which independent checks fix each function) is stated per function
and exercised by ``tests/test_oracle.py``:

* ``dual_forward`` — golden vectors of the reference's compiled
  ``sinkhorn_forward_cpu`` at matched iteration counts; closed forms (rank-one
  kernels converge in one iteration to ``a b^T``); exact column marginals
  after every iteration; row/column shift invariance.  The batch-global
  ``max|u_t - u_{t-1}| < tol`` stopping rule (GPU only, torch_cuda.cpp:199-238)
  is restated from the source.  Pins: the reference tests' behavioural
  property (early stop before ``n_iters`` with the plan within 2e-3 of the
  fixed-count plan, test_sinkhorn.py:827-839); the count convention, by a
  rank-one kernel, which is exact after iteration 1, so the test must fire at
  iteration 2 (``n_iters_used == 2``: a count off by one fails); the
  batch-global reduction, by an input where a per-element test stops earlier.
  A criterion over u *and* v cannot be told apart from the u-only one: the
  column update is 1-Lipschitz in the max norm, so ``max|v_t - v_{t-1}| <=
  max|u_t - u_{t-1}|`` at every iteration (checked on random inputs).  The
  iteration at which a general input crosses tol is property-pinned only
  (float32 and float64 can cross one iteration apart).
* ``implicit_backward`` — golden vectors of the reference's compiled
  ``sinkhorn_backward_implicit_cpu`` with ``tol=0`` (which runs exactly the
  GPU's fixed sweep count); at convergence, a dense float64 solve of the
  adjoint system / float64 autograd through a converged Sinkhorn; finite
  differences of ``cost`` in ``reg``.
* ``unrolled_backward`` — golden vectors of the reference's compiled
  ``sinkhorn_backward_unrolled_cpu`` (autograd cannot pin it: the reference's
  formula is not the exact Jacobian; see ``unrolled_backward``).
* ``dual_forward_method`` (momentum, Adam, Anderson, regularisation
  schedules) — restated from torch_cuda.cpp:323-557 and :61-84.  Pinned by
  reductions to the vanilla forward (momentum with omega = 1, an Anderson
  history of one, a schedule whose start equals the target, each equal to
  ``dual_forward`` step for step) and by the fixed point: every method that
  converges reaches the vanilla plan.  The per-iteration values of the
  accelerated methods between those pins are restated, not independently
  pinned (the reference ships no fixture for them).
* ``spectral_preflight_tau`` — the deflated power iteration converges to the
  largest singular value of C_M P C_N (C the centring projector), checked
  against ``numpy.linalg.svd`` at a large iteration count; a row-constant
  ``log_alpha`` (P = 1 1^T / N, rank one) gives the 1e-12 floor.  The start
  vector is restated from the source and not independently pinned: no golden
  vector of the reference exists for the preflight (its compiled CPU library
  has none), so the value after 5 or 8 iterations, which still depends on
  the start vector, is parity unpinned beyond the restated algorithm.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import numpy as np

SAFE_EXP_LO = -88.0
SAFE_EXP_HI = 88.0
SUM_FLOOR = 1.0e-12


def safe_exp(x: np.ndarray) -> np.ndarray:
    """``safe_exp`` of src/sinkhorn/kernels.cu:21-25 (and kernels_cpu.cpp:18-22):
    0 below -88, exp(88) above 88."""
    with np.errstate(over="ignore", under="ignore"):
        y = np.exp(np.minimum(x, SAFE_EXP_HI))
    return np.where(x < SAFE_EXP_LO, np.zeros_like(y), y)


def default_log_marginal(batch: int, size: int, dtype) -> np.ndarray:
    """``-log(size)`` per entry (torch_cuda.cpp:33-43; computed in fp32 there)."""
    return np.full((batch, size), -np.log(np.float32(size)), dtype=np.float32).astype(dtype)


def _lse(x: np.ndarray, axis: int) -> np.ndarray:
    """Max-shifted log-sum-exp with the reference's guards
    (kernels.cu:523-538 rows, :649-664 columns): ``max + log(max(sum safe_exp(x - max), 1e-12))``."""
    mx = x.max(axis=axis, keepdims=True)
    s = safe_exp(x - mx).sum(axis=axis, keepdims=True)
    return np.squeeze(mx + np.log(np.maximum(s, SUM_FLOOR)), axis=axis)


@dataclass
class ForwardResult:
    P: np.ndarray                      # [B, n, m] plan (or log plan when return_log)
    n_iters_used: int
    converged: bool
    u: np.ndarray                      # [B, n] final row potential
    v: np.ndarray                      # [B, m] final column potential
    K: np.ndarray                      # [B, n, m] log kernel = log_alpha / tau
    u_hist: Optional[np.ndarray] = None  # [T, B, n] when history was requested
    v_hist: Optional[np.ndarray] = None  # [T, B, m]
    deltas: Optional[np.ndarray] = None  # [T] batch-global max|u_t - u_{t-1}|


def dual_forward(log_alpha, tau: float, n_iters: int, tol: float = 0.0,
                 log_a=None, log_b=None, return_log: bool = False,
                 keep_history: bool = False, dtype=np.float64) -> ForwardResult:
    """Dual log-domain Sinkhorn, the reference's default GPU forward.

    Follows ``sinkhorn_dual_vanilla_cuda`` (src/sinkhorn/torch_cuda.cpp:147-264):
    K = log_alpha * (1/tau) (kernels.cu:1104-1137); u = v = 0; each iteration
    updates all rows (u_i = log a_i - LSE_j(K_ij + v_j), kernels.cu:503-545),
    then all columns from the new u (v_j = log b_j - LSE_i(K_ij + u_i),
    kernels.cu:629-671); when tol > 0 it stops after the first iteration whose
    batch-global ``max|u - u_prev|`` (u only, kernels.cu:825-842) is below tol.
    The plan is ``safe_exp(K + u_i + v_j)`` (kernels.cu:755-775).
    """
    la = np.asarray(log_alpha, dtype=np.float32)
    B, n, m = la.shape
    inv_tau = np.float32(1.0) / np.float32(tau)
    K = (la * inv_tau).astype(dtype)
    lga = default_log_marginal(B, n, dtype) if log_a is None else np.asarray(log_a, np.float32).astype(dtype)
    lgb = default_log_marginal(B, m, dtype) if log_b is None else np.asarray(log_b, np.float32).astype(dtype)
    u = np.zeros((B, n), dtype)
    v = np.zeros((B, m), dtype)
    u_hist, v_hist, deltas = [], [], []
    used, converged = 0, False
    for it in range(n_iters):
        u_prev = u
        u = lga - _lse(K + v[:, None, :], axis=2)
        v = lgb - _lse(K + u[:, :, None], axis=1)
        used = it + 1
        if keep_history:
            u_hist.append(u.copy())
            v_hist.append(v.copy())
        d = float(np.abs(u - u_prev).max()) if u.size else 0.0
        deltas.append(d)
        if tol > 0.0 and d < tol:
            converged = True
            break
    logP = K + u[:, :, None] + v[:, None, :]
    P = logP if return_log else safe_exp(logP)
    return ForwardResult(
        P=P, n_iters_used=used, converged=converged, u=u, v=v, K=K,
        u_hist=np.stack(u_hist) if keep_history and u_hist else None,
        v_hist=np.stack(v_hist) if keep_history and v_hist else None,
        deltas=np.asarray(deltas),
    )


def transport_cost(P, cost) -> np.ndarray:
    """``(P * C).sum((-2, -1))`` of dot/sinkhorn.py:1703."""
    return (np.asarray(P) * np.asarray(cost)).sum(axis=(-2, -1))


def implicit_backward(log_alpha, P, grad_P, tau: float, iters: int,
                      tol: Optional[float] = None, dtype=np.float64):
    """Implicit-function adjoint (Gauss-Seidel on lambda then mu, from zero).

    GPU semantics (``tol=None``): exactly ``iters`` sweeps, no early exit
    (src/sinkhorn/kernels.cu:1682-1726 with the lambda/mu kernels :965-1047).
    CPU semantics (``tol`` given): per batch element, stop after the first
    sweep whose max change over lambda and mu is below tol
    (kernels_cpu.cpp:276-312; the CPU op passes 1e-6, torch_cpu.cpp:324).

    lambda_i = (sum_k P_ik G_ik - sum_k P_ik mu_k) / max(sum_k P_ik, 1e-12)
    mu_k     = (sum_i P_ik G_ik - sum_i P_ik lambda_i) / max(sum_i P_ik, 1e-12)
    grad     = P (G - lambda_i - mu_k) / tau        (kernels.cu:1049-1071)
    grad_tau = -sum(grad * log_alpha) / tau          (kernels.cu:1073-1098)

    Returns ``(grad_log_alpha [B,n,m], grad_tau [B], sweeps_run [B])``.
    """
    la = np.asarray(log_alpha, np.float32).astype(dtype)
    P = np.asarray(P).astype(dtype)
    G = np.asarray(grad_P).astype(dtype)
    B, n, m = P.shape
    r = (P * G).sum(axis=2)
    rs = np.maximum(P.sum(axis=2), SUM_FLOOR)
    c = (P * G).sum(axis=1)
    cs = np.maximum(P.sum(axis=1), SUM_FLOOR)
    lam = np.zeros((B, n), dtype)
    mu = np.zeros((B, m), dtype)
    sweeps = np.zeros(B, dtype=np.int64)
    active = np.ones(B, dtype=bool)
    for _ in range(iters):
        if not active.any():
            break
        # P mu and P^T lambda as batched matrix-vector products (BLAS)
        lam_new = (r - np.matmul(P, mu[:, :, None])[:, :, 0]) / rs
        mu_new = (c - np.matmul(lam_new[:, None, :], P)[:, 0, :]) / cs
        change = np.maximum(np.abs(lam_new - lam).max(axis=1, initial=0.0),
                            np.abs(mu_new - mu).max(axis=1, initial=0.0))
        lam = np.where(active[:, None], lam_new, lam)
        mu = np.where(active[:, None], mu_new, mu)
        sweeps += active
        if tol is not None:
            active &= ~(change < tol)
    grad = P * (G - lam[:, :, None] - mu[:, None, :]) / dtype(tau)
    grad_tau = -(grad * la).sum(axis=(1, 2)) / dtype(tau)
    return grad, grad_tau, sweeps


def unrolled_backward(log_alpha, P, grad_P, K, u_hist, v_hist, tau: float, dtype=np.float64):
    """Reverse pass through T iterations, as the reference computes it.

    Follows ``sinkhorn_backward_unrolled_dual_cuda`` (src/sinkhorn/kernels.cu:1622-1680)
    and its CPU twin ``sinkhorn_backward_unrolled_cpu`` (kernels_cpu.cpp:169-245):
    Gamma = grad_P * P; for t = T-1 .. 0, with X = K + u_t + v_t and
    Y = K + u_t + v_{t-1} (v_{-1} = 0):
        Gamma_Y = Gamma   - safe_exp(X) * colsum(Gamma)      (kernels.cu:856-889)
        Gamma   = Gamma_Y - safe_exp(Y) * rowsum(Gamma_Y)    (kernels.cu:891-924)
    grad = Gamma / tau; grad_tau = -sum(Gamma * log_alpha) / tau^2.

    This is NOT the exact Jacobian of the forward: the true softmax factors
    would be exp(X - log b) and exp(Y - log a).  The reference's formula is
    reproduced literally because parity is with the reference.
    """
    la = np.asarray(log_alpha, np.float32).astype(dtype)
    K = np.asarray(K).astype(dtype)
    G = (np.asarray(grad_P).astype(dtype) * np.asarray(P).astype(dtype))
    T = 0 if u_hist is None else len(u_hist)
    for t in range(T - 1, -1, -1):
        u_t = u_hist[t].astype(dtype)
        v_t = v_hist[t].astype(dtype)
        v_p = v_hist[t - 1].astype(dtype) if t > 0 else np.zeros_like(v_t)
        q = safe_exp(K + u_t[:, :, None] + v_t[:, None, :])
        G = G - q * G.sum(axis=1, keepdims=True)
        p = safe_exp(K + u_t[:, :, None] + v_p[:, None, :])
        G = G - p * G.sum(axis=2, keepdims=True)
    grad = G / dtype(tau)
    grad_tau = -(G * la).sum(axis=(1, 2)) / (dtype(tau) * dtype(tau))
    return grad, grad_tau


def with_grads_implicit(log_alpha, grad_P, tau, n_iters, backward_iters,
                        log_a=None, log_b=None, dtype=np.float64):
    """The GPU op ``sinkhorn_with_grads_implicit`` (torch_cuda.cpp:803-871):
    forward with tol=0 for ``n_iters``, then exactly ``backward_iters`` adjoint sweeps."""
    fwd = dual_forward(log_alpha, tau, n_iters, 0.0, log_a, log_b, dtype=dtype)
    grad, grad_tau, _ = implicit_backward(log_alpha, fwd.P, grad_P, tau, backward_iters, None, dtype)
    return fwd.P, grad, grad_tau


def with_grads_unrolled(log_alpha, grad_P, tau, n_iters, log_a=None, log_b=None, dtype=np.float64):
    """The GPU op ``sinkhorn_with_grads_unrolled`` (torch_cuda.cpp:717-801)."""
    fwd = dual_forward(log_alpha, tau, n_iters, 0.0, log_a, log_b, keep_history=True, dtype=dtype)
    grad, grad_tau = unrolled_backward(log_alpha, fwd.P, grad_P, fwd.K, fwd.u_hist, fwd.v_hist,
                                       tau, dtype)
    return fwd.P, grad, grad_tau


def spectral_preflight_tau(log_alpha, tau: float, n_power: int, dtype=np.float64) -> np.ndarray:
    """Contraction estimate per batch element (reference dot/sinkhorn.py:878-897,
    the same math as the GPU kernel src/sinkhorn/kernels.cu:141-241):
    P = softmax_row(log_alpha / tau); v0_j = sin((j+1) 12.9898 + (b+1) 78.233)
    (arguments rounded in float32 as the kernel forms them), centred and
    normalised; n_power times u = centre(P v), v = centre_normalise(P^T u);
    finally ||centre(P v)||, floored at 1e-12 under the root and clamped to
    [0, 0.999999] (kernels.cu:238-240)."""
    X = np.asarray(log_alpha, dtype=dtype)
    B, M, N = X.shape
    K = X * (dtype(1.0) / dtype(tau)) if dtype is np.float32 else X / tau
    lse = np.max(K, axis=2, keepdims=True)
    s = np.sum(safe_exp(K - lse), axis=2, keepdims=True)
    P = safe_exp(K - (lse + np.log(np.maximum(s, 1e-12))))
    j = np.arange(1, N + 1, dtype=np.float32)[None, :] * np.float32(12.9898)
    bb = np.arange(1, B + 1, dtype=np.float32)[:, None] * np.float32(78.233)
    v = np.sin((j + bb).astype(np.float32)).astype(dtype)

    def centre(x):
        return x - x.mean(axis=-1, keepdims=True)

    def normalise(x):
        return x / np.sqrt(np.maximum((x * x).sum(axis=-1, keepdims=True), 1e-12))

    v = normalise(centre(v))
    for _ in range(n_power):
        u = centre(np.einsum("bij,bj->bi", P, v))
        v = normalise(centre(np.einsum("bij,bi->bj", P, u)))
    u = centre(np.einsum("bij,bj->bi", P, v))
    est = np.sqrt(np.maximum((u * u).sum(axis=-1), 1e-12))
    return np.clip(est, 0.0, 0.999999)


SCHEDULE_NONE, SCHEDULE_LINEAR, SCHEDULE_EXPONENTIAL, SCHEDULE_COSINE = 0, 1, 2, 3
METHOD_VANILLA, METHOD_MOMENTUM, METHOD_ANDERSON, METHOD_ADAM = 0, 1, 2, 3


def scheduled_tau(step: int, total: int, tau: float, reg_start: float, schedule: int) -> np.float32:
    """Regularisation at iteration ``step`` (torch_cuda.cpp:61-84), in float32
    like the reference's host code: start = reg_start if > 0 else 10 tau;
    frac = step / (total - 1); linear, cosine or exponential from start to tau."""
    f = np.float32
    tau = f(tau)
    if schedule == SCHEDULE_NONE or total <= 1:
        return tau
    start = f(reg_start) if reg_start > 0.0 else f(10.0) * tau
    frac = f(step) / f(total - 1)
    if schedule == SCHEDULE_LINEAR:
        return start * (f(1.0) - frac) + tau * frac
    if schedule == SCHEDULE_COSINE:
        return tau + f(0.5) * (start - tau) * (f(1.0) + f(np.cos(f(np.pi) * frac)))
    if schedule == SCHEDULE_EXPONENTIAL:
        return tau * f(np.power(start / tau, f(1.0) - frac))
    return tau


def dual_forward_method(log_alpha, tau: float, n_iters: int, tol: float = 0.0, log_a=None, log_b=None,
                        method: int = METHOD_VANILLA, omega: float = 1.5, anderson_k: int = 5,
                        mixing_beta: float = 1.0, lr: float = 1.0, beta1: float = 0.9, beta2: float = 0.999,
                        eps_adam: float = 1e-8, bias_correction: bool = True, reg_start: float = -1.0,
                        schedule: int = SCHEDULE_NONE, return_log: bool = False, dtype=np.float64):
    """Accelerated / scheduled dual Sinkhorn of the reference's GPU path.

    method 0 with a schedule is ``sinkhorn_dual_vanilla_cuda`` (torch_cuda.cpp:
    147-264: K rebuilt from log_alpha at each iteration's tau, the u-only stop
    test).  Methods 1-3 are ``torch_cuda.cpp:323-557``:

    * momentum: u' = (1 - omega) u + omega u*, kept when the batch-global
      max|u' - u*| < max|u - u*| (u* the plain row update); the same for v
      after the column update from the kept u;
    * Adam: g = u* - u, first/second moments, optional bias correction
      (beta^(t+1) in float32), u' = u + lr m^ / (sqrt(v^) + eps), kept by the
      same test;
    * Anderson: state x = (u, v), x_new = one plain row+column update of x,
      residual f = x_new - x, the last k (x, f) pairs; with at least two,
      alpha solves (F^T F + 1e-8 I) alpha = 1 per batch element, normalised
      by its sum (all elements fall back to x_new when any |sum| < 1e-12 or a
      solve fails), x = (X + mixing_beta F) alpha.

    Stop test (tol > 0): methods 1 and 3 use max over u and v of the change;
    Anderson max|x_new - x|; vanilla max|u - u_prev|.  The plan is
    exp(K + u + v) with K at the target tau (safe_exp for the vanilla loop).
    Anderson's map is per batch element: the reference's CUDA map reads v
    through a strided view as if dense (torch_cuda.cpp:116-117 with
    kernels.cu:518), which mixes batch elements when B > 1; the two agree at
    B = 1.  Returns ForwardResult.
    """
    f32 = np.float32
    # the reference passes every hyperparameter as float (static_cast<float>,
    # torch_cuda.cpp:470-530): 1 - beta2 for beta2 = 0.999 differs from its
    # double by 1.3e-5 relative, which the moments carry into every step
    omega, mixing_beta, lr, beta1, beta2, eps_adam = (
        float(f32(x)) for x in (omega, mixing_beta, lr, beta1, beta2, eps_adam))
    la = np.asarray(log_alpha, dtype=np.float32)
    B, n, m = la.shape
    lga = default_log_marginal(B, n, dtype) if log_a is None else np.asarray(log_a, np.float32).astype(dtype)
    lgb = default_log_marginal(B, m, dtype) if log_b is None else np.asarray(log_b, np.float32).astype(dtype)

    def kernel_at(t):
        return (la * (f32(1.0) / f32(t))).astype(dtype)

    K = kernel_at(scheduled_tau(0, n_iters, tau, reg_start, schedule))
    u = np.zeros((B, n), dtype)
    v = np.zeros((B, m), dtype)
    row = lambda K, v: lga - _lse(K + v[:, None, :], axis=2)
    col = lambda K, u: lgb - _lse(K + u[:, :, None], axis=1)
    gmax = lambda x: float(np.abs(x).max()) if x.size else 0.0
    used, converged = 0, False
    if method == METHOD_ADAM:
        mu_u, vu_u = np.zeros_like(u), np.zeros_like(u)
        mu_v, vu_v = np.zeros_like(v), np.zeros_like(v)
    if method == METHOD_ANDERSON:
        state = np.zeros((B, n + m), dtype)
        hist_x, hist_f = [], []
    for it in range(n_iters):
        if schedule != SCHEDULE_NONE:
            K = kernel_at(scheduled_tau(it, n_iters, tau, reg_start, schedule))
        if method == METHOD_ANDERSON:
            un = row(K, state[:, n:])
            vn = col(K, un)
            x_new = np.concatenate([un, vn], axis=1)
            resid = x_new - state
            delta = gmax(resid) if tol > 0.0 else 0.0
            hist_x.append(state.copy())
            hist_f.append(resid)
            if len(hist_x) > anderson_k:
                hist_x.pop(0)
                hist_f.pop(0)
            if len(hist_x) >= 2:
                X = np.stack(hist_x, axis=2)
                F = np.stack(hist_f, axis=2)
                h = X.shape[2]
                gram = np.einsum("blp,blq->bpq", F, F) + np.asarray(1e-8, dtype) * np.eye(h, dtype=dtype)[None]
                try:
                    alpha = np.linalg.solve(gram, np.ones((B, h, 1), dtype))[..., 0]
                    denom = alpha.sum(1, keepdims=True)
                    if np.abs(denom).min() >= 1e-12:
                        alpha = alpha / denom
                        state = np.einsum("blh,bh->bl", X + mixing_beta * F, alpha)
                    else:
                        state = x_new
                except np.linalg.LinAlgError:
                    state = x_new
            else:
                state = x_new
            used = it + 1
            if tol > 0.0 and delta < tol:
                converged = True
                break
            continue
        u_prev = u
        ut = row(K, v)
        if method == METHOD_MOMENTUM:
            un = float(f32(1.0) - f32(omega)) * u + omega * ut
            if gmax(un - ut) < gmax(u - ut):
                ut = un
        elif method == METHOD_ADAM:
            g = ut - u
            mu_u = beta1 * mu_u + float(f32(1.0) - f32(beta1)) * g
            vu_u = beta2 * vu_u + float(f32(1.0) - f32(beta2)) * g * g
            c1 = float(f32(1.0) - np.power(f32(beta1), f32(it + 1))) if bias_correction else 1.0
            c2 = float(f32(1.0) - np.power(f32(beta2), f32(it + 1))) if bias_correction else 1.0
            un = u + lr * (mu_u / c1) / (np.sqrt(vu_u / c2) + eps_adam)
            if gmax(un - ut) < gmax(u - ut):
                ut = un
        vt = col(K, ut)
        if method == METHOD_MOMENTUM:
            vn = float(f32(1.0) - f32(omega)) * v + omega * vt
            if gmax(vn - vt) < gmax(v - vt):
                vt = vn
        elif method == METHOD_ADAM:
            g = vt - v
            mu_v = beta1 * mu_v + float(f32(1.0) - f32(beta1)) * g
            vu_v = beta2 * vu_v + float(f32(1.0) - f32(beta2)) * g * g
            c1 = float(f32(1.0) - np.power(f32(beta1), f32(it + 1))) if bias_correction else 1.0
            c2 = float(f32(1.0) - np.power(f32(beta2), f32(it + 1))) if bias_correction else 1.0
            vn = v + lr * (mu_v / c1) / (np.sqrt(vu_v / c2) + eps_adam)
            if gmax(vn - vt) < gmax(v - vt):
                vt = vn
        if method == METHOD_VANILLA:
            delta = gmax(ut - u_prev)
        else:
            delta = max(gmax(ut - u), gmax(vt - v)) if tol > 0.0 else 0.0
        u, v = ut, vt
        used = it + 1
        if tol > 0.0 and delta < tol:
            converged = True
            break
    if method == METHOD_ANDERSON:
        u, v = state[:, :n], state[:, n:]
    if schedule != SCHEDULE_NONE:
        K = kernel_at(tau)
    logP = K + u[:, :, None] + v[:, None, :]
    # the vanilla loop materialises with safe_exp (kernels.cu:755-772), the
    # methods with torch's exp (torch_cuda.cpp:550-551)
    with np.errstate(over="ignore", under="ignore"):
        P = logP if return_log else (safe_exp(logP) if method == METHOD_VANILLA else np.exp(logP))
    return ForwardResult(P=P, n_iters_used=used, converged=converged, u=u, v=v, K=K)
