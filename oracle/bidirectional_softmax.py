"""TEST INFRASTRUCTURE ONLY — numpy restatement of the reference's bidirectional softmax.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import this module; the product never does.

Pinned by golden vectors of the reference's compiled CPU kernels
(``src/bidirectional_softmax/kernels_cpu.cpp``) and, independently, by the
closed form ``sqrt(1e-9 + softmax_row * softmax_col)`` written with
``torch.softmax`` and its float64 autograd gradient (tests/test_oracle.py).
"""

from __future__ import annotations

import numpy as np

EPS = 1.0e-9


def _valid_mask(B, L1, L2, lengths):
    ln = np.asarray(lengths, dtype=np.int64).reshape(B, 2)
    rows = np.arange(L1)[None, :, None] < ln[:, 0][:, None, None]
    cols = np.arange(L2)[None, None, :] < ln[:, 1][:, None, None]
    return rows & cols


def _masked_softmax(y, mask, axis):
    neg = np.where(mask, y, -np.inf)
    mx = neg.max(axis=axis, keepdims=True)
    mx = np.where(np.isfinite(mx), mx, 0.0)
    with np.errstate(under="ignore"):
        e = np.where(mask, np.exp(np.where(mask, y - mx, 0.0)), 0.0)
    s = e.sum(axis=axis, keepdims=True)
    return np.where(s > 0, e / np.where(s > 0, s, 1.0), 0.0)


def forward(sim, tau: float, lengths, dtype=np.float64):
    """Forward of ``bidirectional_softmax`` (kernels_cpu.cpp:41-133; GPU kernels.cu:90-242).

    Within the valid region (i < L1, j < L2): row softmax r and column softmax
    c of ``sim * (1/tau)``; ``out = sqrt(1e-9 + r * c)``.  Outside it, out, r
    and c are exactly 0.  Returns ``(out, row_sm, col_sm)``.
    """
    s = np.asarray(sim, np.float32)
    B, L1, L2 = s.shape
    inv_T = np.float32(1.0) / np.float32(tau)
    y = (s * inv_T).astype(dtype)
    mask = _valid_mask(B, L1, L2, lengths)
    r = _masked_softmax(y, mask, axis=2)
    c = _masked_softmax(y, mask, axis=1)
    out = np.where(mask, np.sqrt(EPS + r * c), 0.0)
    return out, r, c


def backward(sim, out, grad_out, row_sm, col_sm, tau: float, lengths, dtype=np.float64):
    """Backward of ``bidirectional_softmax`` (kernels_cpu.cpp:139-232; GPU kernels.cu:249-411).

    d = g * 0.5 / out where valid and out > 1e-9 (else 0); d_r = d * c; d_c = d * r;
    grad = (d_r - sum_j d_r r) r / tau + (d_c - sum_i d_c c) c / tau;
    grad_tau = -sum(grad * sim) / tau over the valid region.
    Returns ``(grad_sim, grad_tau)``.
    """
    s = np.asarray(sim, np.float32).astype(dtype)
    o = np.asarray(out).astype(dtype)
    g = np.asarray(grad_out).astype(dtype)
    r = np.asarray(row_sm).astype(dtype)
    c = np.asarray(col_sm).astype(dtype)
    B, L1, L2 = s.shape
    mask = _valid_mask(B, L1, L2, lengths)
    inv_T = dtype(np.float32(1.0) / np.float32(tau))
    ok = mask & (o > EPS)
    d = np.where(ok, g * 0.5 / np.where(ok, o, 1.0), 0.0)
    d_r = np.where(mask, d * c, 0.0)
    d_c = np.where(mask, d * r, 0.0)
    dot_r = (d_r * r).sum(axis=2, keepdims=True)
    dot_c = (d_c * c).sum(axis=1, keepdims=True)
    grad = np.where(mask, (d_r - dot_r) * r * inv_T + (d_c - dot_c) * c * inv_T, 0.0)
    grad_tau = -(np.where(mask, grad * s, 0.0)).sum(axis=(1, 2)) * inv_T
    return grad, grad_tau


def default_lengths(B, L1, L2):
    """``_make_lengths`` of dot/bidirectional_softmax.py:52-57: int32 [B, 2] of (L1, L2)."""
    ln = np.empty((B, 2), np.int32)
    ln[:, 0] = L1
    ln[:, 1] = L2
    return ln
