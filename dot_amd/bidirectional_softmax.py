"""Bidirectional softmax for soft sequence matching — the reference's Python API.

    out[i, j] = sqrt(1e-9 + softmax(sim/T, row)[i, j] * softmax(sim/T, col)[i, j])

inside the valid region (i < L1_b, j < L2_b) and exactly 0 outside it.

Mirrors dot/bidirectional_softmax.py of the reference
(``bidirectional_softmax`` :60-106, ``bidirectional_softmax_with_lengths``
:109-126, ``BidirectionalSoftmax`` :129-162, ``_make_lengths`` :52-57).  As in
the reference, no gradient flows to ``tau`` (the autograd function returns
None for it, :49).

On HIP tensors the autograd function saves only ``sim`` and the per-row and
per-column (max, sum) statistics instead of the three full [B, L1, L2]
tensors the reference keeps (out, row_sm, col_sm); the backward recomputes
the softmaxes from them.  The operator-level API (``_ops.bidirectional_softmax``
returning [P, row_sm, col_sm]) is unchanged.
"""

from typing import Optional

import torch
import torch.nn as nn

from . import _ops


class _BidirectionalSoftmaxFusedFunction(torch.autograd.Function):
    """HIP: statistics-based forward/backward."""

    @staticmethod
    def forward(ctx, sim_matrix, tau, lengths):
        # lengths None: every element full (no lengths tensor to build per call)
        out, row_stats, col_stats = _ops.fused.bidirectional_softmax_forward(sim_matrix, float(tau),
                                                                             lengths)
        ctx.save_for_backward(sim_matrix, row_stats, col_stats, lengths)
        ctx.tau = float(tau)
        ctx.sim_dtype = sim_matrix.dtype
        return out

    @staticmethod
    def backward(ctx, grad_output):
        sim_matrix, row_stats, col_stats, lengths = ctx.saved_tensors
        grad_sim, _grad_tau = _ops.fused.bidirectional_softmax_backward(
            sim_matrix, grad_output.contiguous(), row_stats, col_stats, ctx.tau, lengths)
        return grad_sim.to(ctx.sim_dtype), None, None


class _BidirectionalSoftmaxFunction(torch.autograd.Function):
    """CPU: the reference's buffer-based autograd function (bidirectional_softmax.py:19-49)."""

    @staticmethod
    def forward(ctx, sim_matrix, tau, lengths):
        output, row_softmax, col_softmax = _ops.bidirectional_softmax(sim_matrix, tau, lengths)
        ctx.save_for_backward(sim_matrix, output, row_softmax, col_softmax, lengths)
        ctx.tau = tau
        return output

    @staticmethod
    def backward(ctx, grad_output):
        sim_matrix, output, row_softmax, col_softmax, lengths = ctx.saved_tensors
        grad_sim, _grad_tau = _ops.bidirectional_softmax_backward(
            sim_matrix, output, grad_output.contiguous(), row_softmax, col_softmax, ctx.tau, lengths)
        return grad_sim, None, None


def _make_lengths(B: int, L1: int, L2: int, device: torch.device) -> torch.Tensor:
    """Default lengths: int32 [B, 2] of (L1, L2)."""
    lengths = torch.empty(B, 2, dtype=torch.int32, device=device)
    lengths[:, 0] = L1
    lengths[:, 1] = L2
    return lengths


def bidirectional_softmax(
    sim_matrix: torch.Tensor,
    tau: float = 1.0,
    lengths: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Geometric mean of row and column softmax of ``sim_matrix / tau``.

    Args:
        sim_matrix: Similarity scores of shape (B, L1, L2) or (L1, L2)
        tau: Temperature (> 0); lower is sharper
        lengths: Optional int32 [B, 2] tensor of valid (L1, L2) per batch element

    Returns:
        Soft matching matrix of the input's shape, values in [0, 1]
    """
    unbatched = sim_matrix.dim() == 2
    if unbatched:
        sim_matrix = sim_matrix.unsqueeze(0)
    B, L1, L2 = sim_matrix.size(0), sim_matrix.size(1), sim_matrix.size(2)
    if sim_matrix.is_cuda:
        result = _BidirectionalSoftmaxFusedFunction.apply(sim_matrix, tau, lengths)
    else:
        if lengths is None:
            lengths = _make_lengths(B, L1, L2, sim_matrix.device)
        result = _BidirectionalSoftmaxFunction.apply(sim_matrix, tau, lengths)
    if unbatched:
        result = result.squeeze(0)
    return result


def bidirectional_softmax_with_lengths(
    sim_matrix: torch.Tensor,
    lengths: torch.Tensor,
    tau: float = 1.0,
) -> torch.Tensor:
    """:func:`bidirectional_softmax` with ``lengths`` required."""
    return bidirectional_softmax(sim_matrix, tau=tau, lengths=lengths)


class BidirectionalSoftmax(nn.Module):
    """Module wrapper of :func:`bidirectional_softmax`."""

    def __init__(self, tau: float = 1.0):
        super().__init__()
        self.tau = tau

    def forward(self, sim_matrix: torch.Tensor, lengths: Optional[torch.Tensor] = None) -> torch.Tensor:
        return bidirectional_softmax(sim_matrix, tau=self.tau, lengths=lengths)
