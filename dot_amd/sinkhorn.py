"""Sinkhorn optimal transport and soft permutations — the reference's Python API.

Mirrors dot/sinkhorn.py of the reference: ``sinkhorn`` (:1284-1714),
``sinkhorn_from_scores`` (:1717-1860), ``spectral_preflight`` (:860-905),
``SinkhornResult`` (:22-34), ``Sinkhorn`` (:1863-1906) and
``SinkhornFromScores`` (:1909-1954), with the same argument names, defaults,
validation errors and result fields.  ``max_iter`` is accepted as an alias of
``n_iters`` (the reference README's spelling, README.md:43).

On HIP tensors the forward and backward run as fused dot_amd operators:

* the forward iterates on the device, decides the stopping test on the
  device, and writes the plan and the transport cost ``sum(P * C)`` in one
  pass, with no host wait: ``n_iters_used`` and ``converged`` are copied to
  the host behind it and read when the result's fields are first accessed;
* the backward takes the plan saved by the forward (the reference recomputes
  the whole forward, torch_cuda.cpp:842-853, which yields the same plan) and
  runs the implicit adjoint (exactly ``backward_iters`` sweeps) or the
  unrolled reverse pass over the ``n_iters_used`` recorded potentials, with the
  cost's direct gradient ``grad_cost * P`` folded in.

On HIP tensors with ``dual=True`` and the implicit backward, the momentum,
Anderson and Adam solvers and the linear / exponential / cosine
regularisation schedules run as the ``dot_sinkhorn_forward_method`` operator,
as on the reference's CUDA path (sinkhorn.py:1393-1530); their backward is the
reference's: the implicit adjoint of the vanilla plan recomputed at
``n_iters_used`` iterations.

On CPU tensors the reference's CPU path is followed through the
``torch.ops.dot`` CPU operators.  The reference's PyTorch-level solvers (its
CPU and ``dual=False`` paths for momentum, Anderson, Adam and the schedules,
and Newton and Muon everywhere) run as in the reference, from
``dot_amd.solvers``, with the implicit backward at ``n_iters_used``.
"""

from __future__ import annotations

import atexit
import collections
import math
from dataclasses import dataclass
from typing import List, Literal, Optional

import torch
import torch.nn as nn

from . import _ops, solvers

SCORES_LOG_ALPHA = 1
SCORES_COST = -1
_MODE_IMPLICIT = 0
_MODE_UNROLLED = 1

DEFAULT_SPECTRAL_PREFLIGHT_ALPHA = 1.0
SPECTRAL_PREFLIGHT_MIN_ITERS = 3
SPECTRAL_PREFLIGHT_MAX_ITERS = 1000


@dataclass
class SinkhornResult:
    """Result from Sinkhorn computation.

    Attributes:
        transport_plan: Transport plan P of shape (B, n, m)
        cost: Transport cost sum(P * C) of shape (B,)
        converged: Whether the stopping test fired (True when tol == 0)
        n_iters_used: Forward iterations executed

    On HIP tensors ``converged`` and ``n_iters_used`` come from the device:
    the forward queues their copy to host memory without waiting, and the
    first read of either field waits for that copy (for the forward only, not
    for work queued after it, such as a backward).  A caller that reads them
    only after queuing its backward keeps the device busy throughout; the
    values are the same plain ``bool`` and ``int`` either way.
    """

    transport_plan: torch.Tensor
    cost: Optional[torch.Tensor] = None
    converged: bool = True
    n_iters_used: Optional[int] = None

    def __getattribute__(self, name):
        if name == "converged" or name == "n_iters_used":
            d = object.__getattribute__(self, "__dict__")
            resolve = d.get("_resolve")
            if resolve is not None:
                d["n_iters_used"], d["converged"] = resolve()
                d["_resolve"] = None
        return object.__getattribute__(self, name)

    def __setattr__(self, name, value):
        if name == "converged" or name == "n_iters_used":
            getattr(self, name)  # settle a deferred pair before one half is replaced
        object.__setattr__(self, name, value)

    def __getstate__(self):
        getattr(self, "n_iters_used")
        state = dict(self.__dict__)
        state.pop("_resolve", None)
        state.pop("_adjoint", None)
        return state

    @property
    def adjoint_sweeps(self) -> Optional[List[int]]:
        """Adjoint sweeps each batch element ran in this result's implicit
        backward on HIP tensors (waits for that backward; raises if one of its
        exchanges timed out), or None before a backward ran or on other paths.

        An extension of this build: the register-resident and persistent
        adjoints end an element's sweeps once they have converged (at most
        ``backward_iters``; exactly that many with DOT_AMD_EXACT_SWEEPS=1)."""
        report = self.__dict__.get("_adjoint")
        if report is None or report.status is None:
            return None
        return report.status.sweeps()

    @classmethod
    def _deferred(cls, transport_plan, cost, resolve, report=None):
        """A result whose (n_iters_used, converged) come from ``resolve()`` on first read.

        Until then the two fields are absent from the instance ``__dict__`` (so
        ``vars(result)`` never shows placeholder values); every attribute read,
        ``dataclasses.asdict``, ``repr``, ``==`` and pickling resolve them first.
        ``report`` (a _CallRecord) receives the backward's status words."""
        r = cls(transport_plan=transport_plan, cost=cost)
        d = r.__dict__
        del d["n_iters_used"], d["converged"]
        d["_resolve"] = resolve
        if report is not None:
            d["_adjoint"] = report
        return r


_TIMEOUT_MESSAGE = "dot_sinkhorn_forward: a cross-workgroup exchange timed out (outputs are NaN)"
_BWD_TIMEOUT_MESSAGE = "dot_sinkhorn_backward: a cross-workgroup exchange timed out (gradients are NaN)"


class _DeviceCounts:
    """A device forward's int32 ``[iters_used, converged]``, copied to pinned
    host memory behind the forward on its stream; ``get()`` waits for that copy
    only.  Words already in pinned host memory (written there by the call's
    last kernel) need no copy: ``get()`` waits for the call itself.  A negative
    count means a cross-workgroup exchange of the forward timed out (the
    kernels bound every wait); ``get()`` raises for it."""

    __slots__ = ("_host", "_event", "_value")

    def __init__(self, words: torch.Tensor, device: Optional[torch.device] = None):
        if words.is_cuda:
            stream = torch.cuda.current_stream(words.device)  # the stream the kernels ran on
            self._host = torch.empty(words.numel(), dtype=torch.int32, pin_memory=True)
            with torch.cuda.stream(stream):
                self._host.copy_(words, non_blocking=True)
        else:
            stream = torch.cuda.current_stream(device)
            self._host = words
        self._event = torch.cuda.Event()
        self._event.record(stream)
        self._value = None

    def ready(self) -> bool:
        return self._value is not None or self._event.query()

    def _decode(self, words):
        used, conv = words
        if used < 0:
            raise RuntimeError(_TIMEOUT_MESSAGE)
        return used, bool(conv)

    def get(self):
        if self._value is None:
            self._event.synchronize()
            self._value = self._decode([int(x) for x in self._host.tolist()])
        return self._value


class _DeviceStatus(_DeviceCounts):
    """A device backward's int32 status word (1 when a cross-workgroup exchange
    of the adjoint timed out), followed for the implicit adjoint by the sweeps
    each batch element ran; ``get()`` raises for a timeout."""

    __slots__ = ()

    def _decode(self, words):
        if words[0] != 0:
            raise RuntimeError(_BWD_TIMEOUT_MESSAGE)
        return True

    def sweeps(self) -> Optional[List[int]]:
        self.get()
        words = [int(x) for x in self._host.tolist()]
        return words[1:] if len(words) > 1 else None


class _CallRecord:
    """A device call's trackers: the forward's _DeviceCounts and, once the
    result's backward has run, its _DeviceStatus."""

    __slots__ = ("counts", "status")

    def __init__(self):
        self.counts = None
        self.status = None


# Device calls whose status nobody has read yet: each new device forward or
# backward checks the finished ones, so a timed-out exchange raises by the
# next call at the latest.
_unchecked = collections.deque()
_MAX_UNCHECKED = 64


def _release_unchecked():
    """Wait for the pending status copies and drop their pinned buffers and
    events while the HIP runtime is up (registered with atexit: objects left to
    interpreter teardown are released after it)."""
    while _unchecked:
        dc = _unchecked.popleft()
        try:
            dc._event.synchronize()
        except Exception:  # a failed device leaves nothing to wait for
            pass


atexit.register(_release_unchecked)


def _check_finished_forwards():
    while _unchecked and (_unchecked[0].ready() or len(_unchecked) > _MAX_UNCHECKED):
        _unchecked.popleft().get()


def check_device_errors() -> None:
    """Wait for every HIP Sinkhorn forward and backward issued so far and
    raise RuntimeError if a cross-workgroup exchange of one of them timed out
    (its outputs are then NaN).  Later calls check finished ones by themselves."""
    while _unchecked:
        _unchecked.popleft().get()


def _track(counts: torch.Tensor, device: Optional[torch.device] = None) -> _DeviceCounts:
    _check_finished_forwards()
    dc = _DeviceCounts(counts, device)
    _unchecked.append(dc)
    return dc


def _track_status(status: torch.Tensor, device: torch.device, report=None) -> None:
    _check_finished_forwards()
    ds = _DeviceStatus(status, device)
    _unchecked.append(ds)
    if report is not None:
        report.status = ds


def _tau_value(tau) -> float:
    return float(tau.detach().item()) if torch.is_tensor(tau) else float(tau)


def _check_tau_tensor(tau):
    if torch.is_tensor(tau) and tau.numel() != 1:
        raise ValueError("reg/tau tensor must be scalar")


# ---------------------------------------------------------------------------
# HIP: fused autograd function
# ---------------------------------------------------------------------------
class _SinkhornFusedFunction(torch.autograd.Function):
    """Fused forward (plan + cost + device-side stop) and fused backward on HIP tensors.

    Outputs ``(P, cost)``.  ``record`` (a _CallRecord) receives the tracker of
    the int32 ``[iters_used, converged]`` that the forward's last kernel writes
    to pinned host memory, and the backward's status tracker.  ``scores_kind``
    says whether ``scores`` is a cost matrix C (log_alpha = -C) or log_alpha
    itself.
    """

    @staticmethod
    def forward(ctx, scores, tau, scores_kind, n_iters, backward_iters, log_a, log_b, tol, mode,
                want_cost, record):
        _check_tau_tensor(tau)
        tau_value = _tau_value(tau)
        ctx.record = record
        needs_grad = ctx.needs_input_grad[0] or (torch.is_tensor(tau) and ctx.needs_input_grad[1])
        keep_history = bool(needs_grad and mode == _MODE_UNROLLED)
        P, cost, counts, u_hist, v_hist = _ops.fused.sinkhorn_forward(
            scores, scores_kind, tau_value, n_iters, tol, log_a, log_b, want_cost, keep_history
        )
        record.counts = _track(counts, scores.device)
        if not want_cost:
            ctx.mark_non_differentiable(cost)
        # An unused plan or cost reaches backward as None, not as a zero-filled
        # [B, M, N] tensor the adjoint would have to read.
        ctx.set_materialize_grads(False)
        ctx.save_for_backward(scores, P, u_hist, v_hist)
        ctx.tau = tau_value
        ctx.tau_is_tensor = torch.is_tensor(tau)
        ctx.scores_kind = scores_kind
        ctx.backward_iters = backward_iters
        ctx.mode = mode
        ctx.scores_dtype = scores.dtype
        return P, cost

    @staticmethod
    def backward(ctx, grad_P, grad_cost):
        scores, P, u_hist, v_hist = ctx.saved_tensors
        if grad_cost is not None and grad_cost.numel() == 0:
            grad_cost = None
        if grad_P is None and grad_cost is None:
            return (torch.zeros_like(scores),) + (None,) * 10
        if ctx.mode == _MODE_UNROLLED:
            iters = ctx.record.counts.get()[0]  # waits for the forward only
            uh, vh = u_hist, v_hist
        else:
            iters = ctx.backward_iters
            uh = vh = None
        gc_scalar = False
        if grad_cost is not None:
            if grad_cost.dim() == 1 and grad_cost.numel() > 1 and grad_cost.stride(0) == 0:
                # an expanded scalar (the gradient of cost.sum()): its one value
                grad_cost, gc_scalar = grad_cost[:1], True
            else:
                grad_cost = grad_cost.contiguous()
        grad_scores, grad_tau, status = _ops.fused.sinkhorn_backward(
            scores,
            ctx.scores_kind,
            P,
            grad_P.contiguous() if grad_P is not None else None,
            grad_cost,
            ctx.tau,
            ctx.mode,
            iters,
            uh,
            vh,
            gc_scalar,
        )
        _track_status(status, scores.device, ctx.record)
        tau_grad = None
        if ctx.tau_is_tensor and ctx.needs_input_grad[1]:
            tau_grad = grad_tau.sum()
        return (grad_scores.to(ctx.scores_dtype), tau_grad) + (None,) * 9


def _run_fused(scores, reg, scores_kind, n_iters, backward_iters, log_a, log_b, tol, mode, want_cost,
               record=None):
    tau_arg = reg
    if torch.is_tensor(reg):
        tau_arg = reg.reshape(()).to(device=scores.device)
    if record is None:
        record = _CallRecord()
    P, cost = _SinkhornFusedFunction.apply(
        scores, tau_arg, scores_kind, int(n_iters), int(backward_iters), log_a, log_b, float(tol),
        mode, want_cost, record
    )
    return P, cost, record.counts


_METHOD_CODES = {"vanilla": 0, "momentum": 1, "anderson": 2, "adam": 3}
# Longest Anderson ring the device kernels hold (DOT_SK_MAX_ANDERSON in
# include/dot_amd.h); the ring keeps min(anderson_k, n_iters) pairs.
MAX_ANDERSON_RING = 64


def _check_anderson_ring(anderson_k: int, n_iters: int) -> None:
    """Rejects, before any kernel, an Anderson ring the device path cannot hold.

    The reference's CUDA dual path (torch_cuda.cpp:290, 369-424) takes any
    anderson_k; this build's kernels keep at most MAX_ANDERSON_RING pairs."""
    if min(int(anderson_k), int(n_iters)) > MAX_ANDERSON_RING:
        raise ValueError(
            f"method='anderson' on a GPU tensor keeps min(anderson_k, n_iters) = "
            f"{min(int(anderson_k), int(n_iters))} pairs, above the {MAX_ANDERSON_RING} this build's kernels "
            f"hold; use anderson_k <= {MAX_ANDERSON_RING}")
_SCHEDULE_CODES = {None: 0, "linear": 1, "exponential": 2, "cosine": 3}


class _SinkhornMethodFunction(torch.autograd.Function):
    """Momentum / Anderson / Adam / scheduled dual Sinkhorn on HIP tensors.

    The reference's _SinkhornCudaDualImplicitFunction (sinkhorn.py:155-240)
    with the transport cost sum(P * C) of sinkhorn.py:1702 fused into the
    forward.  Outputs ``(P, cost, counts)`` like _SinkhornFusedFunction.
    Backward, as the reference's: the implicit adjoint (``backward_iters``
    sweeps) of the vanilla plan recomputed at ``n_iters_used`` iterations
    (its sinkhorn_with_grads_implicit), with the cost's upstream gradient
    folded into the plan's, G = grad_P + grad_cost * C, and the cost's direct
    term grad_cost * P taken from this forward's plan.
    """

    @staticmethod
    def forward(ctx, scores, tau, scores_kind, n_iters, backward_iters, log_a, log_b, tol, params,
                want_cost, report):
        _check_tau_tensor(tau)
        tau_value = _tau_value(tau)
        ctx.report = report
        P, cost, counts = _ops.fused.sinkhorn_forward_method(
            scores, scores_kind, tau_value, n_iters, tol, log_a, log_b, *params, want_cost)
        ctx.mark_non_differentiable(counts)
        if not want_cost:
            ctx.mark_non_differentiable(cost)
        ctx.set_materialize_grads(False)
        ctx.save_for_backward(scores, P, counts,
                              log_a if log_a is not None else torch.Tensor(),
                              log_b if log_b is not None else torch.Tensor())
        ctx.has_log_a, ctx.has_log_b = log_a is not None, log_b is not None
        ctx.tau = tau_value
        ctx.tau_is_tensor = torch.is_tensor(tau)
        ctx.scores_kind = scores_kind
        ctx.backward_iters = backward_iters
        ctx.scores_dtype = scores.dtype
        return P, cost, counts

    @staticmethod
    def backward(ctx, grad_P, grad_cost, _grad_counts):
        scores, P, counts, log_a, log_b = ctx.saved_tensors
        log_a = log_a if ctx.has_log_a else None
        log_b = log_b if ctx.has_log_b else None
        none = (None,) * 10
        if grad_cost is not None and grad_cost.numel() == 0:
            grad_cost = None
        if grad_P is None and grad_cost is None:
            return (torch.zeros_like(scores),) + none
        used = int(counts[0].item())
        P_vanilla = _ops.fused.sinkhorn_forward(scores, ctx.scores_kind, ctx.tau, used, 0.0, log_a, log_b,
                                                False, False)[0]
        grad_scores, grad_tau, status = _ops.fused.sinkhorn_backward(
            scores, ctx.scores_kind, P_vanilla,
            grad_P.contiguous() if grad_P is not None else None,
            grad_cost.contiguous() if grad_cost is not None else None,
            ctx.tau, _MODE_IMPLICIT, ctx.backward_iters, None, None)
        _track_status(status, scores.device, ctx.report)
        if grad_cost is not None:
            # the fused backward's direct cost term used P_vanilla; the cost was
            # computed from this forward's plan (d sum(P C)/dC = P, C = -log_alpha)
            grad_scores = grad_scores.add_(grad_cost.view(-1, 1, 1) * (P - P_vanilla),
                                           alpha=float(-ctx.scores_kind))
        tau_grad = None
        if ctx.tau_is_tensor and ctx.needs_input_grad[1]:
            tau_grad = grad_tau.sum()
        return (grad_scores.to(ctx.scores_dtype), tau_grad) + none[1:]


def _run_method(scores, reg, scores_kind, n_iters, backward_iters, log_a, log_b, tol, params, want_cost,
                report=None):
    tau_arg = reg
    if torch.is_tensor(reg):
        tau_arg = reg.reshape(()).to(device=scores.device)
    P, cost, counts = _SinkhornMethodFunction.apply(
        scores, tau_arg, scores_kind, int(n_iters), int(backward_iters), log_a, log_b, float(tol), params,
        want_cost, report)
    return P, cost, _track(counts)


# ---------------------------------------------------------------------------
# CPU: the reference's autograd functions over the CPU operators
# ---------------------------------------------------------------------------
class _SinkhornUnrolledFunction(torch.autograd.Function):
    """CPU autograd with the unrolled backward (reference sinkhorn.py:46-96)."""

    @staticmethod
    def forward(ctx, log_alpha, tau, n_iters, log_a, log_b):
        _check_tau_tensor(tau)
        tau_value = _tau_value(tau)
        P = _ops.sinkhorn(log_alpha, tau_value, n_iters, log_a, log_b)
        ctx.save_for_backward(log_alpha,
                              log_a if log_a is not None else torch.Tensor(),
                              log_b if log_b is not None else torch.Tensor())
        ctx.tau, ctx.n_iters = tau_value, n_iters
        ctx.tau_is_tensor = torch.is_tensor(tau)
        ctx.has_log_a, ctx.has_log_b = log_a is not None, log_b is not None
        return P

    @staticmethod
    def backward(ctx, grad_P):
        log_alpha, log_a, log_b = ctx.saved_tensors
        _, grad_log_alpha, grad_tau = _ops.sinkhorn_with_grads_unrolled(
            log_alpha, grad_P.contiguous(), ctx.tau, ctx.n_iters,
            log_a if ctx.has_log_a else None, log_b if ctx.has_log_b else None)
        tau_grad = grad_tau.sum() if ctx.tau_is_tensor else None
        return grad_log_alpha, tau_grad, None, None, None


class _SinkhornImplicitFunction(torch.autograd.Function):
    """CPU autograd with the implicit backward (reference sinkhorn.py:99-152)."""

    @staticmethod
    def forward(ctx, log_alpha, tau, n_iters, backward_iters, log_a, log_b):
        _check_tau_tensor(tau)
        tau_value = _tau_value(tau)
        P = _ops.sinkhorn(log_alpha, tau_value, n_iters, log_a, log_b)
        ctx.save_for_backward(log_alpha,
                              log_a if log_a is not None else torch.Tensor(),
                              log_b if log_b is not None else torch.Tensor())
        ctx.tau, ctx.n_iters, ctx.backward_iters = tau_value, n_iters, backward_iters
        ctx.tau_is_tensor = torch.is_tensor(tau)
        ctx.has_log_a, ctx.has_log_b = log_a is not None, log_b is not None
        return P

    @staticmethod
    def backward(ctx, grad_P):
        log_alpha, log_a, log_b = ctx.saved_tensors
        _, grad_log_alpha, grad_tau = _ops.sinkhorn_with_grads_implicit(
            log_alpha, grad_P.contiguous(), ctx.tau, ctx.n_iters, ctx.backward_iters,
            log_a if ctx.has_log_a else None, log_b if ctx.has_log_b else None)
        tau_grad = grad_tau.sum() if ctx.tau_is_tensor else None
        return grad_log_alpha, tau_grad, None, None, None, None


# ---------------------------------------------------------------------------
# Argument handling
# ---------------------------------------------------------------------------
def _prepare_marginal(marginal, batch, size, name, device, dtype):
    """Validation of the reference's _prepare_marginal (sinkhorn.py:1259-1281)."""
    if marginal is None:
        return None
    if marginal.dim() == 1:
        marginal = marginal.unsqueeze(0).expand(batch, -1)
    if marginal.shape != (batch, size):
        raise ValueError(f"{name} must have shape ({batch}, {size}) or ({size},)")
    if torch.any(marginal <= 0):
        raise ValueError(f"{name} must be strictly positive")
    marginal = marginal.to(device=device, dtype=dtype)
    sums = marginal.sum(dim=-1)
    if not torch.allclose(sums, torch.ones_like(sums), atol=1e-4, rtol=1e-4):
        raise ValueError(f"{name} must sum to 1 along the last dimension")
    return marginal


def _resolve_iters(n_iters, max_iter):
    if max_iter is not None:
        if n_iters is not None and n_iters != 20 and n_iters != max_iter:
            raise ValueError("pass n_iters or its alias max_iter, not both")
        return max_iter
    return 20 if n_iters is None else n_iters


def _effective_method(method, schedule, reg_start, omega, tau_value, lr, beta1, beta2, eps_adam,
                      bias_correction, backward_mode, on_gpu, dual, size):
    """The reference's method/schedule resolution (sinkhorn.py:1362-1390)."""
    if method == "auto":
        method = "newton" if size[0] <= 100 and size[1] <= 100 else "vanilla"
    effective = method
    eff_schedule = schedule
    eff_reg_start = reg_start
    if dual and on_gpu and backward_mode == "implicit":
        if effective == "momentum" and omega is None:
            effective = "vanilla"
        elif effective == "anderson" and eff_schedule is None:
            if tau_value >= 0.05:
                effective = "vanilla"
            elif tau_value <= 0.01:
                eff_schedule = "exponential"
                if eff_reg_start is None:
                    eff_reg_start = 10.0 * tau_value
        elif effective == "adam" and eff_schedule is None:
            is_default_adam = (lr == 1.0 and beta1 == 0.9 and beta2 == 0.999 and eps_adam == 1e-8
                               and bias_correction)
            if tau_value >= 0.05 or is_default_adam:
                effective = "vanilla"
    return method, effective, eff_schedule, eff_reg_start


_METHODS = ("vanilla", "momentum", "anderson", "adam", "newton", "muon", "auto")


def _solver(method, log_alpha, tau_value, log_a, log_b, omega, anderson_k, mixing_beta, lr, beta1, beta2,
            eps_adam, bias_correction, reg_start, schedule):
    """The reference's PyTorch solver for ``method`` (sinkhorn.py:1531-1693) and
    its options: momentum estimates omega when none is given; plain Sinkhorn
    with a schedule starts from reg_start or 10 * reg."""
    if method == "momentum":
        if omega is None:
            omega = solvers.estimate_omega(log_alpha.detach(), tau_value,
                                           log_a.detach() if log_a is not None else None,
                                           log_b.detach() if log_b is not None else None)
        return solvers.momentum_forward, dict(omega=float(omega), reg_start=reg_start, schedule=schedule)
    if method == "anderson":
        return solvers.anderson_forward, dict(anderson_k=anderson_k, mixing_beta=mixing_beta,
                                              reg_start=reg_start, schedule=schedule)
    if method == "adam":
        return solvers.adam_forward, dict(lr=lr, beta1=beta1, beta2=beta2, eps_adam=eps_adam,
                                          bias_correction=bias_correction, reg_start=reg_start, schedule=schedule)
    if method == "muon":
        return solvers.muon_forward, dict(lr=lr, reg_start=reg_start, schedule=schedule)
    if method == "newton":
        return solvers.newton_forward, dict(reg_start=reg_start, schedule=schedule)
    start = float(reg_start) if reg_start is not None else 10.0 * tau_value
    return solvers.scheduled_forward, dict(reg_start=start, schedule=schedule)


def sinkhorn(
    cost_matrix: torch.Tensor,
    reg: float | torch.Tensor = 1.0,
    n_iters: int | Literal["auto"] = 20,
    backward_mode: Literal["unrolled", "implicit"] = "implicit",
    backward_iters: Optional[int] = None,
    a: Optional[torch.Tensor] = None,
    b: Optional[torch.Tensor] = None,
    method: Literal["vanilla", "momentum", "anderson", "adam", "newton", "muon", "auto"] = "vanilla",
    omega: Optional[float] = None,
    anderson_k: int = 5,
    mixing_beta: float = 1.0,
    lr: float = 1.0,
    beta1: float = 0.9,
    beta2: float = 0.999,
    eps_adam: float = 1e-8,
    bias_correction: bool = True,
    reg_start: Optional[float] = None,
    schedule: Optional[Literal["linear", "exponential", "cosine"]] = None,
    tol: float = 1e-6,
    dual: bool = True,
    max_iter: Optional[int] = None,
) -> SinkhornResult:
    """Entropy-regularised optimal transport with the Sinkhorn algorithm.

    Args:
        cost_matrix: Cost matrix of shape (B, n, m) or (n, m)
        reg: Regularization strength / temperature (float or scalar tensor)
        n_iters: Maximum Sinkhorn iterations, or 'auto' for the spectral preflight
        backward_mode: 'implicit' (adjoint, default) or 'unrolled'
        backward_iters: Adjoint sweeps of the implicit backward (default: n_iters)
        a, b: Optional source/target marginals, shape (B, n)/(n,) and (B, m)/(m,)
        method: Solver: 'vanilla', 'momentum' (omega; estimated from a pilot
            run off the device path when None), 'anderson' (anderson_k,
            mixing_beta), 'adam' (lr, beta1, beta2, eps_adam,
            bias_correction), 'newton' (n, m <= 100), 'muon' (lr); 'auto'
            picks 'newton' up to 100x100.  Every method but 'vanilla' needs
            the implicit backward.  On HIP tensors with dual=True, momentum,
            anderson and adam run fused on the device (with the reference's
            fall-backs to vanilla, sinkhorn.py:1373-1390)
        schedule: 'linear', 'exponential' or 'cosine' annealing of reg from
            reg_start (default 10 * reg) over the iterations
        tol: Stop after the first iteration with max|u_t - u_{t-1}| < tol over
            the whole batch (HIP tensors); 0 forces all iterations
        dual: Prefer the dual-state device path (HIP tensors)
        max_iter: Alias of n_iters

    Returns:
        SinkhornResult(transport_plan, cost, converged, n_iters_used)
    """
    n_iters = _resolve_iters(n_iters, max_iter)
    if method not in _METHODS:
        raise ValueError(f"Unsupported method: {method}")
    if backward_mode not in ("implicit", "unrolled"):
        raise ValueError("backward_mode must be 'unrolled' or 'implicit'")

    unbatched = cost_matrix.dim() == 2
    if unbatched:
        cost_matrix = cost_matrix.unsqueeze(0)
    if cost_matrix.dim() != 3:
        raise ValueError("cost_matrix must have shape (B, n, m) or (n, m)")

    a = _prepare_marginal(a, cost_matrix.size(0), cost_matrix.size(-2), "a", cost_matrix.device,
                          cost_matrix.dtype)
    b = _prepare_marginal(b, cost_matrix.size(0), cost_matrix.size(-1), "b", cost_matrix.device,
                          cost_matrix.dtype)
    log_a = torch.log(a) if a is not None else None
    log_b = torch.log(b) if b is not None else None

    tau_value = _tau_value(reg)
    if isinstance(n_iters, str):
        if n_iters != "auto":
            raise ValueError("n_iters must be an int or 'auto'")
        predicted = spectral_preflight(-cost_matrix.detach(), tau_value, tol=tol)
        n_iters = int(predicted.max().item()) if torch.is_tensor(predicted) else int(predicted)
    if backward_iters is None:
        backward_iters = n_iters

    on_gpu = cost_matrix.is_cuda
    method, effective, eff_schedule, eff_reg_start = _effective_method(
        method, schedule, reg_start, omega, tau_value, lr, beta1, beta2, eps_adam, bias_correction,
        backward_mode, on_gpu, dual, (cost_matrix.size(-2), cost_matrix.size(-1)))
    plain = effective == "vanilla" and eff_schedule is None
    # the reference's use_cuda_dual (sinkhorn.py:1393-1400)
    cuda_dual = on_gpu and dual and (
        (backward_mode == "implicit" and effective in _METHOD_CODES)
        or (backward_mode == "unrolled" and plain))
    if not cuda_dual and not plain:
        # the reference's PyTorch solver branches (sinkhorn.py:1531-1693)
        if method != "vanilla" and backward_mode != "implicit":
            raise ValueError(f"method='{method}' only supports implicit backward")
        if method == "vanilla" and backward_mode == "unrolled" and schedule is not None:
            raise ValueError("schedule is only supported with implicit backward")
        log_alpha = -cost_matrix
        runner, options = _solver(method, log_alpha, tau_value, log_a, log_b, omega, anderson_k, mixing_beta,
                                  lr, beta1, beta2, eps_adam, bias_correction, reg_start, schedule)
        P, used_t = solvers.ImplicitSolverFunction.apply(log_alpha, reg, n_iters, backward_iters, log_a, log_b,
                                                         runner, options)
        used = int(used_t)
        converged = True if tol == 0 else used < n_iters
        cost = (P * cost_matrix).sum(dim=(-2, -1))
        if unbatched:
            P, cost = P.squeeze(0), cost.squeeze(0)
        return SinkhornResult(transport_plan=P, cost=cost, converged=converged, n_iters_used=used)

    mode = _MODE_UNROLLED if backward_mode == "unrolled" else _MODE_IMPLICIT
    report = _CallRecord() if on_gpu else None
    if cuda_dual and not plain:
        if effective == "anderson":
            _check_anderson_ring(anderson_k, n_iters)
        params = (_METHOD_CODES[effective], float(omega) if omega is not None else 1.4, int(anderson_k),
                  float(mixing_beta), float(lr), float(beta1), float(beta2), float(eps_adam),
                  bool(bias_correction), -1.0 if eff_reg_start is None else float(eff_reg_start),
                  _SCHEDULE_CODES[eff_schedule])
        P, cost, counts = _run_method(cost_matrix, reg, SCORES_COST, n_iters, backward_iters, log_a, log_b,
                                      tol, params, True, report)
        rule = _dual_converged(tol)
    elif on_gpu:
        # dual=False is the reference's full-matrix path: it ignores tol and
        # always runs n_iters (sinkhorn.py:1693 with torch_cuda.cpp:599-656).
        run_tol = tol if dual else 0.0
        P, cost, counts = _run_fused(cost_matrix, reg, SCORES_COST, n_iters, backward_iters,
                                     log_a, log_b, run_tol, mode, True, report)
        rule = _dual_converged(tol) if dual else _count_converged(tol, n_iters)
    else:
        log_alpha = -cost_matrix
        if mode == _MODE_UNROLLED:
            P = _SinkhornUnrolledFunction.apply(log_alpha, reg, n_iters, log_a, log_b)
        else:
            P = _SinkhornImplicitFunction.apply(log_alpha, reg, n_iters, backward_iters, log_a, log_b)
        used = n_iters
        converged = True if tol == 0 else used < n_iters
        cost = (P * cost_matrix).sum(dim=(-2, -1))

    if on_gpu and cost.dtype != cost_matrix.dtype:
        cost = cost.to(torch.result_type(P, cost_matrix))
    if unbatched:
        P = P.squeeze(0)
        cost = cost.squeeze(0)
    if on_gpu:
        def resolve():
            used, conv = counts.get()
            return used, rule(used, conv)
        return SinkhornResult._deferred(P, cost, resolve, report)
    return SinkhornResult(transport_plan=P, cost=cost, converged=converged, n_iters_used=used)


def _dual_converged(tol):
    """The dual path's flag (sinkhorn.py:1530): the device's stop flag when tol > 0."""
    return lambda used, conv: conv if tol > 0 else True


def _count_converged(tol, n_iters):
    """The other paths' rule (sinkhorn.py:1698-1699): stopped before n_iters."""
    return lambda used, conv: True if tol == 0 else used < n_iters


def sinkhorn_from_scores(
    log_alpha: torch.Tensor,
    tau: float | torch.Tensor = 1.0,
    n_iters: int | Literal["auto"] = 20,
    backward_mode: Literal["unrolled", "implicit"] = "implicit",
    backward_iters: Optional[int] = None,
    return_log: bool = False,
    a: Optional[torch.Tensor] = None,
    b: Optional[torch.Tensor] = None,
    tol: float = 1e-6,
    dual: bool = True,
    max_iter: Optional[int] = None,
) -> torch.Tensor:
    """Normalised transport plan (or its log) directly from log-space scores.

    Same contract as the reference's sinkhorn_from_scores (sinkhorn.py:1717-1860).
    """
    n_iters = _resolve_iters(n_iters, max_iter)
    unbatched = log_alpha.dim() == 2
    if unbatched:
        log_alpha = log_alpha.unsqueeze(0)
    a = _prepare_marginal(a, log_alpha.size(0), log_alpha.size(-2), "a", log_alpha.device,
                          log_alpha.dtype)
    b = _prepare_marginal(b, log_alpha.size(0), log_alpha.size(-1), "b", log_alpha.device,
                          log_alpha.dtype)
    log_a = torch.log(a) if a is not None else None
    log_b = torch.log(b) if b is not None else None
    tau_value = _tau_value(tau)
    if isinstance(n_iters, str):
        if n_iters != "auto":
            raise ValueError("n_iters must be an int or 'auto'")
        predicted = spectral_preflight(log_alpha.detach(), tau_value, tol=tol)
        n_iters = int(predicted.max().item()) if torch.is_tensor(predicted) else int(predicted)
    if backward_iters is None:
        backward_iters = n_iters

    if log_alpha.is_cuda and dual and backward_mode in ("implicit", "unrolled"):
        if return_log:
            result, _, _ = _ops.sinkhorn_dual_forward(log_alpha, tau_value, n_iters, tol, log_a, log_b,
                                                      True)
        else:
            mode = _MODE_UNROLLED if backward_mode == "unrolled" else _MODE_IMPLICIT
            result, _, _ = _run_fused(log_alpha, tau, SCORES_LOG_ALPHA, n_iters, backward_iters,
                                         log_a, log_b, tol, mode, False)
    elif return_log:
        result = _ops.sinkhorn_log(log_alpha, tau_value, n_iters, log_a, log_b)
    elif backward_mode == "unrolled":
        result = _SinkhornUnrolledFunction.apply(log_alpha, tau, n_iters, log_a, log_b)
    else:
        result = _SinkhornImplicitFunction.apply(log_alpha, tau, n_iters, backward_iters, log_a, log_b)
    if unbatched:
        result = result.squeeze(0)
    return result


def spectral_preflight(
    log_alpha: torch.Tensor,
    tau: float | torch.Tensor,
    tol: float = 1e-6,
    n_power: int = 5,
    alpha: Optional[float] = None,
) -> int | torch.Tensor:
    """Predicted iteration counts from a spectral contraction estimate (reference
    sinkhorn.py:860-905): ceil(alpha * log(1/tol) / -log(tau_hat)), clamped to [3, 1000]."""
    if tol <= 0:
        raise ValueError("spectral_preflight requires tol > 0")
    tau_value = _tau_value(tau)
    if tau_value <= 0:
        raise ValueError("tau/reg must be positive")
    alpha_value = DEFAULT_SPECTRAL_PREFLIGHT_ALPHA if alpha is None else float(alpha)
    unbatched = log_alpha.dim() == 2
    if unbatched:
        log_alpha = log_alpha.unsqueeze(0)
    tau_est = _ops.sinkhorn_spectral_preflight(log_alpha, tau_value, n_power)
    tau_hat = tau_est.clamp(min=1e-6, max=0.999999)
    pred = torch.ceil(alpha_value * math.log(1.0 / tol) / (-torch.log(tau_hat))).to(torch.int64)
    pred = pred.clamp(min=SPECTRAL_PREFLIGHT_MIN_ITERS, max=SPECTRAL_PREFLIGHT_MAX_ITERS)
    if unbatched:
        return int(pred.item())
    return pred


class Sinkhorn(nn.Module):
    """Module wrapper of :func:`sinkhorn` (reference sinkhorn.py:1863-1906).

    Accepts ``max_iter`` as an alias of ``n_iters``.
    """

    def __init__(self, reg: float = 1.0, n_iters: Optional[int] = None,
                 backward_mode: Literal["unrolled", "implicit"] = "implicit",
                 backward_iters: Optional[int] = None, max_iter: Optional[int] = None):
        super().__init__()
        self.reg = reg
        self.n_iters = _resolve_iters(n_iters, max_iter)
        self.backward_mode = backward_mode
        self.backward_iters = backward_iters

    def forward(self, cost_matrix: torch.Tensor) -> SinkhornResult:
        return sinkhorn(cost_matrix, reg=self.reg, n_iters=self.n_iters,
                        backward_mode=self.backward_mode, backward_iters=self.backward_iters)


class SinkhornFromScores(nn.Module):
    """Module wrapper of :func:`sinkhorn_from_scores` (reference sinkhorn.py:1909-1954)."""

    def __init__(self, tau: float = 1.0, n_iters: Optional[int] = None,
                 backward_mode: Literal["unrolled", "implicit"] = "implicit",
                 backward_iters: Optional[int] = None, max_iter: Optional[int] = None):
        super().__init__()
        self.tau = tau
        self.n_iters = _resolve_iters(n_iters, max_iter)
        self.backward_mode = backward_mode
        self.backward_iters = backward_iters

    def forward(self, log_alpha: torch.Tensor) -> torch.Tensor:
        return sinkhorn_from_scores(log_alpha, tau=self.tau, n_iters=self.n_iters,
                                    backward_mode=self.backward_mode,
                                    backward_iters=self.backward_iters)
