"""The reference's PyTorch-level Sinkhorn solvers (dot/sinkhorn.py:743-1256).

These run where the reference's dual device path does not: CPU tensors,
``dual=False``, and the methods that path never had (Newton, Muon).  As in the
reference they are iterations over whole tensors with a few ATen calls each
(log-sum-exp, small dense solves) and a host-side stop test per iteration;
they are the reference's slow paths, kept for completeness of the API, not the
fused device path.

Each ``*_forward`` returns ``(P, n_iters_used)``.  ``ImplicitSolverFunction``
gives all of them the reference's backward (its per-method autograd functions,
sinkhorn.py:312-740): the implicit adjoint of the plain iteration recomputed at
``n_iters_used`` iterations (``sinkhorn_with_grads_implicit``); the marginals
receive no gradient.  The solvers' internal stop tests use the reference's
fixed tolerances (1e-6; 1e-8 for Newton), not the caller's ``tol``: the
reference does not pass it on.
"""

from __future__ import annotations

import math
from typing import Callable, Optional

import torch

from . import _ops


def default_log_marginals(log_alpha, log_a, log_b):
    """-log(n) and -log(m) where a marginal is not given (sinkhorn.py:743-753)."""
    B, n, m = log_alpha.shape
    if log_a is None:
        log_a = log_alpha.new_full((B, n), -math.log(float(n)))
    if log_b is None:
        log_b = log_alpha.new_full((B, m), -math.log(float(m)))
    return log_a, log_b


def scheduled_tau(step: int, total: int, target: float, reg_start: Optional[float],
                  schedule: Optional[str]) -> float:
    """Iteration ``step``'s tau under an annealing schedule (sinkhorn.py:805-833),
    in double precision: start = reg_start or 10 * target, frac = step / (total - 1);
    linear interpolation, half a cosine, or geometric interpolation."""
    if schedule is None or total <= 1:
        return target
    start = reg_start if reg_start is not None else 10.0 * target
    frac = step / float(total - 1)
    if schedule == "linear":
        return start * (1.0 - frac) + target * frac
    if schedule == "cosine":
        return target + 0.5 * (start - target) * (1.0 + math.cos(math.pi * frac))
    if schedule == "exponential":
        return target * (start / target) ** (1.0 - frac)
    raise ValueError("schedule must be 'linear', 'exponential', or 'cosine'")


def _zero_potentials(log_alpha):
    B, n, m = log_alpha.shape
    return log_alpha.new_zeros((B, n)), log_alpha.new_zeros((B, m))


def _row_target(kernel, v, log_a):
    """u* = log a - LSE_j(K + v): the plain row update."""
    return log_a - torch.logsumexp(kernel + v.unsqueeze(-2), dim=-1)


def _col_target(kernel, u, log_b):
    """v* = log b - LSE_i(K + u): the plain column update."""
    return log_b - torch.logsumexp(kernel + u.unsqueeze(-1), dim=-2)


def fixed_point_map(u, v, kernel, log_a, log_b):
    """One plain row-then-column update of the dual state (sinkhorn.py:756-768)."""
    un = _row_target(kernel, v, log_a)
    return un, _col_target(kernel, un, log_b)


def _plan(kernel, u, v):
    return (kernel + u.unsqueeze(-1) + v.unsqueeze(-2)).exp()


def _largest_change(u_new, u, v_new, v) -> float:
    """max(max|u_new - u|, max|v_new - v|) as a Python float (one host sync)."""
    parts = [(x - y).abs().amax() for x, y in ((u_new, u), (v_new, v)) if x.numel()]
    return float(torch.stack(parts).max().item()) if parts else 0.0


def estimate_omega(log_alpha, tau: float, log_a, log_b, pilot_iters: int = 10) -> float:
    """Over-relaxation factor from a short plain run (sinkhorn.py:777-802): the
    ratio r of successive largest changes (clamped to [0, 0.999]) gives
    omega = 2 / (1 + sqrt(max(1 - r^2, 1e-6))), clamped to [1, 1.95]."""
    log_a, log_b = default_log_marginals(log_alpha, log_a, log_b)
    kernel = log_alpha / tau
    u, v = _zero_potentials(log_alpha)
    prev, ratio = None, 0.0
    for _ in range(max(pilot_iters, 2)):
        un, vn = fixed_point_map(u, v, kernel, log_a, log_b)
        d = _largest_change(un, u, vn, v)
        if prev is not None and prev > 0.0:
            ratio = min(max(d / prev, 0.0), 0.999)
        prev = max(d, 1e-12)
        u, v = un, vn
    omega = 2.0 / (1.0 + math.sqrt(max(1.0 - ratio * ratio, 1e-6)))
    return float(min(max(omega, 1.0), 1.95))


def momentum_forward(log_alpha, tau, n_iters, log_a, log_b, omega, reg_start=None, schedule=None,
                     tol=1e-6):
    """Over-relaxed updates u <- (1 - w) u + w u*, then v likewise from the new u
    (sinkhorn.py:908-939); stop once the largest change is below tol."""
    log_a, log_b = default_log_marginals(log_alpha, log_a, log_b)
    u, v = _zero_potentials(log_alpha)
    used = 0
    for it in range(n_iters):
        used = it + 1
        kernel = log_alpha / scheduled_tau(it, n_iters, tau, reg_start, schedule)
        un = (1.0 - omega) * u + omega * _row_target(kernel, v, log_a)
        vn = (1.0 - omega) * v + omega * _col_target(kernel, un, log_b)
        d = _largest_change(un, u, vn, v)
        u, v = un, vn
        if d < tol:
            break
    return _plan(log_alpha / tau, u, v), used


def anderson_forward(log_alpha, tau, n_iters, log_a, log_b, anderson_k, mixing_beta, reg_start=None,
                     schedule=None, tol=1e-6):
    """Anderson mixing of the dual state x = [u, v] (sinkhorn.py:942-995).

    With the last anderson_k pairs (x_i, f_i = G(x_i) - x_i), G the plain map,
    and at least two of them, the weights solve (F^T F + 1e-8 I) w = 1 and are
    divided by their sum (floored at 1e-12); the new state is
    sum_i w_i (x_i + beta f_i).  A failed solve keeps G(x).  Stop once the
    largest residual 2-norm over the batch is below tol."""
    log_a, log_b = default_log_marginals(log_alpha, log_a, log_b)
    B, n, m = log_alpha.shape
    state = log_alpha.new_zeros((B, n + m))
    hist_x, hist_f = [], []
    used = 0
    for it in range(n_iters):
        used = it + 1
        kernel = log_alpha / scheduled_tau(it, n_iters, tau, reg_start, schedule)
        un, vn = fixed_point_map(state[:, :n], state[:, n:], kernel, log_a, log_b)
        mapped = torch.cat([un, vn], dim=-1)
        resid = mapped - state
        res_norm = float(resid.norm(dim=-1).max().item()) if resid.numel() else 0.0
        hist_x.append(state)
        hist_f.append(resid)
        while len(hist_x) > anderson_k:
            hist_x.pop(0)
            hist_f.pop(0)
        h = len(hist_x)
        if h >= 2:
            X = torch.stack(hist_x, dim=-1)
            F = torch.stack(hist_f, dim=-1)
            gram = F.transpose(-2, -1) @ F + 1e-8 * torch.eye(h, dtype=F.dtype, device=F.device)
            try:
                w = torch.linalg.solve(gram, F.new_ones((B, h, 1)))
                w = w / w.sum(dim=1, keepdim=True).clamp_min(1e-12)
                state = ((X + mixing_beta * F) * w.squeeze(-1).unsqueeze(1)).sum(dim=-1)
            except RuntimeError:
                state = mapped
        else:
            state = mapped
        if res_norm < tol:
            break
    return _plan(log_alpha / tau, state[:, :n], state[:, n:]), used


def adam_forward(log_alpha, tau, n_iters, log_a, log_b, lr, beta1, beta2, eps_adam, bias_correction,
                 reg_start=None, schedule=None, tol=1e-6):
    """Adam steps along g = x* - x, u first and v from the new u
    (sinkhorn.py:998-1056): m <- b1 m + (1 - b1) g, s <- b2 s + (1 - b2) g^2,
    x <- x + lr m^ / (sqrt(s^) + eps) with m^, s^ bias-corrected by step t = it + 1
    when asked; stop once the largest change is below tol."""
    log_a, log_b = default_log_marginals(log_alpha, log_a, log_b)
    u, v = _zero_potentials(log_alpha)
    moments = {"u": (torch.zeros_like(u), torch.zeros_like(u)),
               "v": (torch.zeros_like(v), torch.zeros_like(v))}

    def adam_step(name, x, target, step):
        g = target - x
        m1, m2 = moments[name]
        m1 = beta1 * m1 + (1.0 - beta1) * g
        m2 = beta2 * m2 + (1.0 - beta2) * (g * g)
        moments[name] = (m1, m2)
        if bias_correction:
            m1 = m1 / (1.0 - beta1 ** step)
            m2 = m2 / (1.0 - beta2 ** step)
        return x + lr * m1 / (torch.sqrt(m2) + eps_adam)

    used = 0
    for it in range(n_iters):
        used = it + 1
        kernel = log_alpha / scheduled_tau(it, n_iters, tau, reg_start, schedule)
        un = adam_step("u", u, _row_target(kernel, v, log_a), it + 1)
        vn = adam_step("v", v, _col_target(kernel, un, log_b), it + 1)
        d = _largest_change(un, u, vn, v)
        u, v = un, vn
        if d < tol:
            break
    return _plan(log_alpha / tau, u, v), used


def scheduled_forward(log_alpha, tau, n_iters, log_a, log_b, reg_start, schedule, tol=1e-6):
    """The plain iteration with K = log_alpha / tau_t (sinkhorn.py:1059-1085);
    the stop test (largest change below tol) counts only from iteration
    max(n_iters // 2, 1) on."""
    log_a, log_b = default_log_marginals(log_alpha, log_a, log_b)
    u, v = _zero_potentials(log_alpha)
    used = 0
    for it in range(n_iters):
        used = it + 1
        kernel = log_alpha / scheduled_tau(it, n_iters, tau, reg_start, schedule)
        un, vn = fixed_point_map(u, v, kernel, log_a, log_b)
        d = _largest_change(un, u, vn, v)
        u, v = un, vn
        if it >= max(n_iters // 2, 1) and d < tol:
            break
    return _plan(log_alpha / tau, u, v), used


def birkhoff_tangent(g):
    """g minus its row and column means plus its overall mean (sinkhorn.py:1088-1092)."""
    return g - g.mean(dim=-1, keepdim=True) - g.mean(dim=-2, keepdim=True) + g.mean(dim=(-2, -1), keepdim=True)


def rebalance(plan, log_a, log_b, rounds: int):
    """``rounds`` row-then-column normalisations of log(max(P, 1e-30)) onto the
    marginals (sinkhorn.py:1095-1116)."""
    lp = plan.clamp_min(1e-30).log()
    for _ in range(rounds):
        lp = lp - torch.logsumexp(lp, dim=-1, keepdim=True) + log_a.unsqueeze(-1)
        lp = lp - torch.logsumexp(lp, dim=-2, keepdim=True) + log_b.unsqueeze(-2)
    return lp.exp()


def muon_forward(log_alpha, tau, n_iters, log_a, log_b, lr, reg_start=None, schedule=None, tol=1e-6):
    """Multiplicative steps on the plan toward a long plain run (sinkhorn.py:1119-1153).

    From 5 plain iterations, each step computes T, the plain plan after
    max(n_iters, 200) iterations at the step's tau, takes the Birkhoff-tangent
    part of g = P (log T - log P) (logs floored at 1e-30), sets
    P <- rebalance(P exp(clamp(lr g_t / P, +-20)), 1); stop once the largest
    change of P is below tol.  A scheduled run is rebalanced once more.  The
    count includes the 5 warm-start iterations."""
    log_a, log_b = default_log_marginals(log_alpha, log_a, log_b)
    warm, target_iters = 5, max(n_iters, 200)
    plan = _ops.sinkhorn(log_alpha, scheduled_tau(0, n_iters, tau, reg_start, schedule), warm, log_a, log_b)
    used = 0
    for it in range(n_iters):
        used = it + 1
        target = _ops.sinkhorn(log_alpha, scheduled_tau(it, n_iters, tau, reg_start, schedule), target_iters,
                               log_a, log_b)
        grad = plan * (target.clamp_min(1e-30).log() - plan.clamp_min(1e-30).log())
        step = (lr * birkhoff_tangent(grad) / plan.clamp_min(1e-30)).clamp(min=-20.0, max=20.0)
        nxt = rebalance(plan * torch.exp(step), log_a, log_b, 1)
        d = float((nxt - plan).abs().max().item()) if plan.numel() else 0.0
        plan = nxt
        if d < tol:
            break
    if schedule is not None:
        plan = rebalance(plan, log_a, log_b, 1)
    return plan, warm + used


def _newton_element(P_e, row_sum, col_sum, resid, rnorm, u_e, v_e, kernel_e, a_e, b_e, la_e, lb_e):
    """One batch element's damped Newton step (sinkhorn.py:1189-1250); returns the
    next (u, v), or None when the plain update is to be taken instead."""
    n, m = u_e.numel(), v_e.numel()
    H = P_e.new_zeros((n + m, n + m))
    H[:n, :n] = torch.diag(row_sum)
    H[n:, n:] = torch.diag(col_sum)
    H[:n, n:] = P_e
    H[n:, :n] = P_e.transpose(0, 1)
    rhs = -resid
    # the dual has one free shift (u + c, v - c): pin the first unknown
    H[0, :] = 0
    H[:, 0] = 0
    H[0, 0] = 1
    rhs[0] = 0
    try:
        d = torch.linalg.solve(H, rhs)
    except RuntimeError:
        return None
    for k in range(6):
        s = 0.5 ** k
        cu, cv = u_e + s * d[:n], v_e + s * d[n:]
        lp = kernel_e + cu.unsqueeze(-1) + cv.unsqueeze(-2)
        if not bool(torch.isfinite(lp).all()) or float(lp.max().item()) > 80.0:
            continue
        cp = lp.exp()
        cnorm = max(float((cp.sum(dim=-1) - a_e).abs().max().item()),
                    float((cp.sum(dim=-2) - b_e).abs().max().item()))
        if cnorm < rnorm:
            nu, nv = fixed_point_map(cu.unsqueeze(0), cv.unsqueeze(0), kernel_e.unsqueeze(0), la_e, lb_e)
            return nu[0], nv[0]
    return None


def newton_forward(log_alpha, tau, n_iters, log_a, log_b, reg_start=None, schedule=None, tol=1e-8):
    """Damped Newton on the marginal residuals (sinkhorn.py:1156-1256), n, m <= 100.

    Each iteration stops if every element's max residual |P1 - a|, |P^T 1 - b|
    is below tol; otherwise per batch element it solves
    [diag(P1) P; P^T diag(P^T 1)] d = -(P1 - a, P^T 1 - b) with the first unknown
    pinned to 0, halves the step (1 .. 1/32) until the residual shrinks (log P
    finite and at most 80), and follows the accepted point with one plain
    update; with no accepted step, or a failed solve, it takes the plain update.
    The plan at the target tau gets 10 rebalancing rounds."""
    log_a, log_b = default_log_marginals(log_alpha, log_a, log_b)
    B, n, m = log_alpha.shape
    if n > 100 or m > 100:
        raise ValueError("method='newton' only supports n, m <= 100")
    a, b = log_a.exp(), log_b.exp()
    u, v = _zero_potentials(log_alpha)
    used = 0
    for it in range(n_iters):
        used = it + 1
        kernel = log_alpha / scheduled_tau(it, n_iters, tau, reg_start, schedule)
        P = _plan(kernel, u, v)
        rs, cs = P.sum(dim=-1), P.sum(dim=-2)
        resid = torch.cat([rs - a, cs - b], dim=-1)
        rnorm = resid.abs().amax(dim=-1)
        if float(rnorm.max().item()) < tol:
            break
        u_next, v_next = u.clone(), v.clone()
        for e in range(B):
            sl = slice(e, e + 1)
            step = _newton_element(P[e], rs[e], cs[e], resid[e], float(rnorm[e].item()), u[e], v[e], kernel[e],
                                   a[e], b[e], log_a[sl], log_b[sl])
            if step is None:
                nu, nv = fixed_point_map(u[sl], v[sl], kernel[sl], log_a[sl], log_b[sl])
                step = (nu[0], nv[0])
            u_next[e], v_next[e] = step
        u, v = u_next, v_next
    return rebalance(_plan(log_alpha / tau, u, v), log_a, log_b, 10), used


class ImplicitSolverFunction(torch.autograd.Function):
    """A solver's plan with the reference's implicit backward (sinkhorn.py:312-740):
    the adjoint of the plain iteration at the solver's n_iters_used iterations,
    ``backward_iters`` sweeps.  Returns (P, n_iters_used as a 0-d int64 tensor)."""

    @staticmethod
    def forward(ctx, log_alpha, tau, n_iters, backward_iters, log_a, log_b, runner: Callable, options: dict):
        tau_is_tensor = torch.is_tensor(tau)
        if tau_is_tensor and tau.numel() != 1:
            raise ValueError("reg/tau tensor must be scalar")
        tau_value = float(tau.detach().item()) if tau_is_tensor else float(tau)
        P, used = runner(log_alpha, tau_value, n_iters, log_a, log_b, **options)
        ctx.save_for_backward(log_alpha,
                              log_a if log_a is not None else torch.Tensor(),
                              log_b if log_b is not None else torch.Tensor())
        ctx.has_log_a, ctx.has_log_b = log_a is not None, log_b is not None
        ctx.tau, ctx.used, ctx.backward_iters = tau_value, int(used), backward_iters
        ctx.tau_like = (tau.device, tau.dtype) if tau_is_tensor else None
        used_t = torch.tensor(int(used), dtype=torch.int64)
        ctx.mark_non_differentiable(used_t)
        return P, used_t

    @staticmethod
    def backward(ctx, grad_P, _grad_used):
        log_alpha, log_a, log_b = ctx.saved_tensors
        _, grad, grad_tau = _ops.sinkhorn_with_grads_implicit(
            log_alpha, grad_P.contiguous(), ctx.tau, ctx.used, ctx.backward_iters,
            log_a if ctx.has_log_a else None, log_b if ctx.has_log_b else None)
        tau_grad = None
        if ctx.tau_like is not None:
            tau_grad = grad_tau.sum().to(device=ctx.tau_like[0], dtype=ctx.tau_like[1])
        return grad, tau_grad, None, None, None, None, None, None
