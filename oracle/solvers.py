"""TEST INFRASTRUCTURE ONLY — numpy restatement of the reference's PyTorch-level
Sinkhorn solvers (dot/sinkhorn.py:743-1256).

These are the checker for ``dot_amd.solvers``; only ``tests/`` may import this
module.  Everything runs in float64 numpy, one batch element at a time, with
an unguarded max-shifted log-sum-exp (the reference's solvers use
``torch.logsumexp``, which has no floors).  Each solver returns
``(P, n_iters_used)`` like the reference's ``_run_*_forward``.

Pinning (tests/test_solvers.py):

* ``momentum`` — with omega = 1 it is the plain iteration step for step
  (``oracle.sinkhorn.dual_forward``, float64); with omega = 0 the potentials
  never move (P = exp(K) exactly).
* ``anderson`` — a history of one is the plain iteration step for step; with
  a history >= 2 the Anderson weights are checked against the closed form of
  the constrained least-squares problem (min |F w| s.t. sum w = 1, through
  ``numpy.linalg.lstsq`` on the null-space parametrisation) for a well-
  conditioned F; at convergence every history leads to the plain fixed point.
* ``adam`` — with beta1 = beta2 = 0, eps = lr = E large and no bias
  correction the step is g E / (|g| + E), the plain update to O(g^2 / E);
  with bias correction the first step equals lr g / (|g| + eps) for every
  beta1, beta2 (both corrected moments equal g and g^2).
* ``scheduled`` — with reg_start = tau it is the plain iteration (with the
  second-half stop rule, restated); ``scheduled_tau`` hits reg_start at step 0
  and tau at the last step for every schedule, and its midpoints are the
  closed forms (arithmetic, cosine, geometric means).
* ``newton`` — the plan it returns satisfies both marginals to 1e-10 and
  equals the converged plain plan; the Hessian blocks are checked against
  central finite differences of the marginal residual.
* ``muon`` — a plan equal to the target is a fixed point (zero step); the
  Birkhoff projection leaves zero row and column sums and is idempotent; the
  plan approaches the plain plan (within the reference test's 1e-4).
* ``estimate_omega`` — a rank-one kernel (plain Sinkhorn exact after one
  iteration, ratio 0) gives omega = 1; on a slowly converging problem the
  pilot ratio approaches the asymptotic rate sigma_2^2 of the converged
  scaled plan (Knight, SIAM J. Matrix Anal. Appl. 30(1), 2008).
"""

from __future__ import annotations

import math
from typing import Optional

import numpy as np


def _lse(x: np.ndarray, axis: int) -> np.ndarray:
    mx = np.max(x, axis=axis, keepdims=True)
    mx = np.where(np.isfinite(mx), mx, 0.0)
    return np.squeeze(mx + np.log(np.sum(np.exp(x - mx), axis=axis, keepdims=True)), axis=axis)


def _marginals(B, n, m, log_a, log_b):
    la = np.full((B, n), -math.log(float(n))) if log_a is None else np.asarray(log_a, np.float64)
    lb = np.full((B, m), -math.log(float(m))) if log_b is None else np.asarray(log_b, np.float64)
    return la, lb


def scheduled_tau(step, total, tau, reg_start, schedule):
    """Iteration ``step``'s tau (sinkhorn.py:805-833), double precision."""
    if schedule is None or total <= 1:
        return tau
    s = 10.0 * tau if reg_start is None else reg_start
    f = step / float(total - 1)
    if schedule == "linear":
        return s * (1.0 - f) + tau * f
    if schedule == "cosine":
        return tau + 0.5 * (s - tau) * (1.0 + math.cos(math.pi * f))
    if schedule == "exponential":
        return tau * (s / tau) ** (1.0 - f)
    raise ValueError(schedule)


def plain_step(K, u, v, la, lb):
    """u* from v, then v* from the new u (sinkhorn.py:756-768), one element."""
    un = la - _lse(K + v[None, :], axis=1)
    vn = lb - _lse(K + un[:, None], axis=0)
    return un, vn


def _run(log_alpha, tau, n_iters, log_a, log_b, reg_start, schedule, step_fn, stop_fn):
    """Shared skeleton: batch-global stop decided by ``stop_fn(it, deltas)``."""
    la_all = np.asarray(log_alpha, np.float64)
    B, n, m = la_all.shape
    LA, LB = _marginals(B, n, m, log_a, log_b)
    U, V = np.zeros((B, n)), np.zeros((B, m))
    state = [None] * B
    used = 0
    for it in range(n_iters):
        used = it + 1
        t = scheduled_tau(it, n_iters, tau, reg_start, schedule)
        worst = 0.0
        for e in range(B):
            K = la_all[e] / t
            un, vn, state[e], d = step_fn(K, U[e], V[e], LA[e], LB[e], state[e], it)
            U[e], V[e] = un, vn
            worst = max(worst, d)
        if stop_fn(it, worst):
            break
    K = la_all / tau
    return np.exp(K + U[:, :, None] + V[:, None, :]), used


def momentum(log_alpha, tau, n_iters, omega, log_a=None, log_b=None, reg_start=None, schedule=None, tol=1e-6):
    """sinkhorn.py:908-939."""
    def step(K, u, v, la, lb, st, it):
        un = (1 - omega) * u + omega * (la - _lse(K + v[None, :], axis=1))
        vn = (1 - omega) * v + omega * (lb - _lse(K + un[:, None], axis=0))
        return un, vn, st, max(np.abs(un - u).max(initial=0.0), np.abs(vn - v).max(initial=0.0))
    return _run(log_alpha, tau, n_iters, log_a, log_b, reg_start, schedule, step, lambda it, d: d < tol)


def adam(log_alpha, tau, n_iters, lr, beta1, beta2, eps_adam, bias_correction, log_a=None, log_b=None,
         reg_start=None, schedule=None, tol=1e-6):
    """sinkhorn.py:998-1056."""
    def move(x, g, mom, t):
        m1 = beta1 * mom[0] + (1 - beta1) * g
        m2 = beta2 * mom[1] + (1 - beta2) * g * g
        h1, h2 = (m1 / (1 - beta1 ** t), m2 / (1 - beta2 ** t)) if bias_correction else (m1, m2)
        return x + lr * h1 / (np.sqrt(h2) + eps_adam), (m1, m2)

    def step(K, u, v, la, lb, st, it):
        if st is None:
            st = ((np.zeros_like(u), np.zeros_like(u)), (np.zeros_like(v), np.zeros_like(v)))
        un, mu = move(u, la - _lse(K + v[None, :], axis=1) - u, st[0], it + 1)
        vn, mv = move(v, lb - _lse(K + un[:, None], axis=0) - v, st[1], it + 1)
        return un, vn, (mu, mv), max(np.abs(un - u).max(initial=0.0), np.abs(vn - v).max(initial=0.0))
    return _run(log_alpha, tau, n_iters, log_a, log_b, reg_start, schedule, step, lambda it, d: d < tol)


def scheduled(log_alpha, tau, n_iters, reg_start, schedule, log_a=None, log_b=None, tol=1e-6):
    """sinkhorn.py:1059-1085: stop test only from iteration max(n_iters // 2, 1)."""
    def step(K, u, v, la, lb, st, it):
        un, vn = plain_step(K, u, v, la, lb)
        return un, vn, st, max(np.abs(un - u).max(initial=0.0), np.abs(vn - v).max(initial=0.0))
    half = max(n_iters // 2, 1)
    return _run(log_alpha, tau, n_iters, log_a, log_b, reg_start, schedule, step,
                lambda it, d: it >= half and d < tol)


def anderson_weights(F: np.ndarray) -> Optional[np.ndarray]:
    """(F^T F + 1e-8 I) w = 1, then w / max(sum w, 1e-12) (sinkhorn.py:975-982)."""
    h = F.shape[1]
    try:
        w = np.linalg.solve(F.T @ F + 1e-8 * np.eye(h), np.ones(h))
    except np.linalg.LinAlgError:
        return None
    return w / max(w.sum(), 1e-12)


def anderson(log_alpha, tau, n_iters, anderson_k, mixing_beta, log_a=None, log_b=None, reg_start=None,
             schedule=None, tol=1e-6):
    """sinkhorn.py:942-995: the state x = [u, v]; the batch-global stop on the
    residual 2-norm is taken before the mixing of the same iteration."""
    la_all = np.asarray(log_alpha, np.float64)
    B, n, m = la_all.shape
    LA, LB = _marginals(B, n, m, log_a, log_b)
    X = np.zeros((B, n + m))
    hist = [[] for _ in range(B)]
    used = 0
    for it in range(n_iters):
        used = it + 1
        t = scheduled_tau(it, n_iters, tau, reg_start, schedule)
        worst = 0.0
        for e in range(B):
            un, vn = plain_step(la_all[e] / t, X[e, :n], X[e, n:], LA[e], LB[e])
            g = np.concatenate([un, vn])
            f = g - X[e]
            worst = max(worst, float(np.sqrt((f * f).sum())))
            hist[e].append((X[e].copy(), f))
            hist[e] = hist[e][-anderson_k:] if anderson_k > 0 else []
            w = anderson_weights(np.stack([p[1] for p in hist[e]], axis=1)) if len(hist[e]) >= 2 else None
            if w is None:
                X[e] = g
            else:
                X[e] = sum(wi * (x + mixing_beta * fi) for wi, (x, fi) in zip(w, hist[e]))
        if worst < tol:
            break
    K = la_all / tau
    return np.exp(K + X[:, :n, None] + X[:, None, n:]), used


def newton_system(P, a, b):
    """Jacobian of r(u, v) = (P1 - a, P^T 1 - b) for P = exp(K + u + v^T):
    [[diag(P1), P], [P^T, diag(P^T 1)]], with the first unknown pinned
    (row and column 0 zeroed, diagonal 1) — sinkhorn.py:1189-1199."""
    n, m = P.shape
    H = np.zeros((n + m, n + m))
    H[:n, :n] = np.diag(P.sum(1))
    H[n:, n:] = np.diag(P.sum(0))
    H[:n, n:] = P
    H[n:, :n] = P.T
    H[0, :] = 0.0
    H[:, 0] = 0.0
    H[0, 0] = 1.0
    return H


def newton(log_alpha, tau, n_iters, log_a=None, log_b=None, reg_start=None, schedule=None, tol=1e-8):
    """sinkhorn.py:1156-1256."""
    la_all = np.asarray(log_alpha, np.float64)
    B, n, m = la_all.shape
    if n > 100 or m > 100:
        raise ValueError("method='newton' only supports n, m <= 100")
    LA, LB = _marginals(B, n, m, log_a, log_b)
    A, Bm = np.exp(LA), np.exp(LB)
    U, V = np.zeros((B, n)), np.zeros((B, m))
    used = 0
    for it in range(n_iters):
        used = it + 1
        t = scheduled_tau(it, n_iters, tau, reg_start, schedule)
        Ks = la_all / t
        res = []
        for e in range(B):
            P = np.exp(Ks[e] + U[e][:, None] + V[e][None, :])
            r = np.concatenate([P.sum(1) - A[e], P.sum(0) - Bm[e]])
            res.append((P, r, np.abs(r).max(initial=0.0)))
        if max(x[2] for x in res) < tol:
            break
        nU, nV = U.copy(), V.copy()
        for e, (P, r, rn) in enumerate(res):
            nxt = None
            rhs = -r.copy()
            rhs[0] = 0.0
            try:
                d = np.linalg.solve(newton_system(P, A[e], Bm[e]), rhs)
            except np.linalg.LinAlgError:
                d = None
            if d is not None:
                for k in range(6):
                    cu, cv = U[e] + 0.5 ** k * d[:n], V[e] + 0.5 ** k * d[n:]
                    lp = Ks[e] + cu[:, None] + cv[None, :]
                    if not np.all(np.isfinite(lp)) or lp.max() > 80.0:
                        continue
                    cp = np.exp(lp)
                    cn = max(np.abs(cp.sum(1) - A[e]).max(), np.abs(cp.sum(0) - Bm[e]).max())
                    if cn < rn:
                        nxt = plain_step(Ks[e], cu, cv, LA[e], LB[e])
                        break
            if nxt is None:
                nxt = plain_step(Ks[e], U[e], V[e], LA[e], LB[e])
            nU[e], nV[e] = nxt
        U, V = nU, nV
    P = np.exp(la_all / tau + U[:, :, None] + V[:, None, :])
    return rebalance(P, LA, LB, 10), used


def birkhoff_tangent(G):
    """G - row means - column means + grand mean (sinkhorn.py:1088-1092)."""
    return G - G.mean(-1, keepdims=True) - G.mean(-2, keepdims=True) + G.mean((-2, -1), keepdims=True)


def rebalance(P, LA, LB, rounds):
    """sinkhorn.py:1095-1116."""
    L = np.log(np.maximum(P, 1e-30))
    for _ in range(rounds):
        L = L - _lse(L, axis=-1)[..., None] + LA[..., None]
        L = L - _lse(L, axis=-2)[..., None, :] + LB[..., None, :]
    return np.exp(L)


def plain_plan(log_alpha, tau, iters, LA, LB):
    """The reference's plain operator ``_ops.sinkhorn`` (kernels_cpu.cpp: row then
    column normalisation of log P, ``iters`` times) in float64, dual form."""
    la_all = np.asarray(log_alpha, np.float64)
    out = np.empty_like(la_all)
    for e in range(la_all.shape[0]):
        K = la_all[e] / tau
        u, v = np.zeros(K.shape[0]), np.zeros(K.shape[1])
        for _ in range(iters):
            u, v = plain_step(K, u, v, LA[e], LB[e])
        out[e] = np.exp(K + u[:, None] + v[None, :])
    return out


def muon(log_alpha, tau, n_iters, lr, log_a=None, log_b=None, reg_start=None, schedule=None, tol=1e-6,
         plain=plain_plan):
    """sinkhorn.py:1119-1153; ``plain(log_alpha, tau, iters, LA, LB)`` is the
    plain operator (float64 by default)."""
    la_all = np.asarray(log_alpha, np.float64)
    B, n, m = la_all.shape
    LA, LB = _marginals(B, n, m, log_a, log_b)
    P = plain(la_all, scheduled_tau(0, n_iters, tau, reg_start, schedule), 5, LA, LB)
    used = 0
    for it in range(n_iters):
        used = it + 1
        T = plain(la_all, scheduled_tau(it, n_iters, tau, reg_start, schedule), max(n_iters, 200), LA, LB)
        G = P * (np.log(np.maximum(T, 1e-30)) - np.log(np.maximum(P, 1e-30)))
        S = np.clip(lr * birkhoff_tangent(G) / np.maximum(P, 1e-30), -20.0, 20.0)
        Pn = rebalance(P * np.exp(S), LA, LB, 1)
        d = np.abs(Pn - P).max(initial=0.0)
        P = Pn
        if d < tol:
            break
    if schedule is not None:
        P = rebalance(P, LA, LB, 1)
    return P, 5 + used


def estimate_omega(log_alpha, tau, log_a=None, log_b=None, pilot_iters=10, return_ratio=False):
    """sinkhorn.py:777-802."""
    la_all = np.asarray(log_alpha, np.float64)
    B, n, m = la_all.shape
    LA, LB = _marginals(B, n, m, log_a, log_b)
    K = la_all / tau
    U, V = np.zeros((B, n)), np.zeros((B, m))
    prev, ratio = None, 0.0
    for _ in range(max(pilot_iters, 2)):
        d = 0.0
        for e in range(B):
            un, vn = plain_step(K[e], U[e], V[e], LA[e], LB[e])
            d = max(d, np.abs(un - U[e]).max(initial=0.0), np.abs(vn - V[e]).max(initial=0.0))
            U[e], V[e] = un, vn
        if prev is not None and prev > 0.0:
            ratio = min(max(d / prev, 0.0), 0.999)
        prev = max(d, 1e-12)
    omega = min(max(2.0 / (1.0 + math.sqrt(max(1.0 - ratio ** 2, 1e-6))), 1.0), 1.95)
    return (omega, ratio) if return_ratio else omega
