"""dot_amd — differentiable optimal transport on AMD MI355X (gfx950).

A from-scratch MI355X implementation of DOT's batched Sinkhorn and
bidirectional-softmax operators with the reference's Python API:

    result = dot_amd.sinkhorn(cost, reg=1.0, n_iters=100)   # also max_iter=
    result.transport_plan   # (B, M, N)
    result.cost             # (B,)
    P = dot_amd.bidirectional_softmax(sim, tau=1.0)

The operators are registered as ``torch.ops.dot.*`` (the reference's schemas)
and run hand-written HIP kernels behind the C ABI in ``include/dot_amd.h``.
``import dot`` gives the same API under the reference's package name.
"""

# Load the operator library first (raises ImportError when it is not built).
from . import _ops

from .sinkhorn import (
    sinkhorn,
    sinkhorn_from_scores,
    spectral_preflight,
    SinkhornResult,
    Sinkhorn,
    SinkhornFromScores,
)
from .bidirectional_softmax import (
    bidirectional_softmax,
    bidirectional_softmax_with_lengths,
    BidirectionalSoftmax,
)

__version__ = "0.1.0"

__all__ = [
    "sinkhorn",
    "sinkhorn_from_scores",
    "spectral_preflight",
    "SinkhornResult",
    "Sinkhorn",
    "SinkhornFromScores",
    "bidirectional_softmax",
    "bidirectional_softmax_with_lengths",
    "BidirectionalSoftmax",
]
