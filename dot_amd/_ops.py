"""Low-level operator access for dot_amd.

Loads ``dot_amd/_C.so`` (which links ``libdot_amd.so``, the HIP kernels behind
the C ABI in ``include/dot_amd.h``) and binds the same eight
``torch.ops.dot.*`` handles as the reference's loader (dot/_ops.py:70-82).
``torch.ops.dot_amd.*`` holds the fused operators used by the autograd
functions in ``dot_amd.sinkhorn`` and ``dot_amd.bidirectional_softmax``.

Import fails loudly when the library is not built: there is no fallback.

Usage::

    from dot_amd import _ops
    P = _ops.sinkhorn(log_alpha, 1.0, 20)
    P, used, converged = _ops.sinkhorn_dual_forward(log_alpha, 1.0, 100, 1e-6)
"""

import os

import torch

_LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_C.so")
_extension_loaded = False


def _load_extension():
    """Load the operator library once per process."""
    global _extension_loaded
    if _extension_loaded:
        return
    if not os.path.exists(_LIB_PATH):
        raise ImportError(
            f"dot_amd native library not found at {_LIB_PATH}; build it with "
            "`python -m dot_amd._build` (hipcc, --offload-arch=gfx950)"
        )
    torch.ops.load_library(_LIB_PATH)
    _extension_loaded = True


def _ensure_loaded():
    if not _extension_loaded:
        _load_extension()


_load_extension()

# The full namespaces
dot = torch.ops.dot
fused = torch.ops.dot_amd

# Reference-compatible handles (dot/_ops.py:73-82)
sinkhorn = torch.ops.dot.sinkhorn
sinkhorn_log = torch.ops.dot.sinkhorn_log
sinkhorn_dual_forward = torch.ops.dot.sinkhorn_dual_forward
sinkhorn_spectral_preflight = torch.ops.dot.sinkhorn_spectral_preflight
sinkhorn_with_grads_unrolled = torch.ops.dot.sinkhorn_with_grads_unrolled
sinkhorn_with_grads_implicit = torch.ops.dot.sinkhorn_with_grads_implicit
bidirectional_softmax = torch.ops.dot.bidirectional_softmax
bidirectional_softmax_backward = torch.ops.dot.bidirectional_softmax_backward
