"""Writes the golden fixtures under tests/golden/ from the reference's own CPU kernels.

Run here (where /root/reference exists) after ``make -C oracle``:

    python tests/golden/make_golden.py

Every fixture is data only: seeded fp32 inputs plus the outputs of the
reference's compiled ``src/sinkhorn/kernels_cpu.cpp`` and
``src/bidirectional_softmax/kernels_cpu.cpp`` (through oracle/ref.py), saved
as ``.npz``.  The GPU box has no /root/reference; tests there read these files.
"""

from __future__ import annotations

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import ref  # noqa: E402


def _dirichlet(rng, batch, size):
    e = -np.log(rng.random((batch, size)))
    return (e / e.sum(axis=1, keepdims=True)).astype(np.float32)


def _save(name, **arrays):
    path = os.path.join(HERE, name + ".npz")
    np.savez_compressed(path, **arrays)
    print(f"wrote {path} ({os.path.getsize(path)} bytes)")


def sinkhorn_cases():
    rng = np.random.default_rng(1234)

    # Mirrors test_reference_match_cpu (test_sinkhorn.py:226-237): B=2, 6x9, reg 0.7, 75 iters, random a, b.
    C = rng.random((2, 6, 9)).astype(np.float32)
    a, b = _dirichlet(rng, 2, 6), _dirichlet(rng, 2, 9)
    la, lga, lgb = -C, np.log(a), np.log(b)
    P = ref.sinkhorn_forward(la, 0.7, 75, lga, lgb)
    logP = ref.sinkhorn_forward(la, 0.7, 75, lga, lgb, return_log=True)
    _save("sk_fwd_6x9", log_alpha=la, log_a=lga, log_b=lgb, tau=np.float32(0.7), n_iters=75,
          P=P, logP=logP)

    # Config C1: cost = rand(8,64,64) from torch seed 0, reg 1.0, 100 iterations, uniform marginals,
    # loss = cost.sum() so grad_P = C; adjoint at the GPU's fixed count (tol=0) and the CPU's 1e-6 break.
    g = torch.Generator().manual_seed(0)
    C1 = torch.rand(8, 64, 64, generator=g).numpy()
    la1 = -C1
    P1 = ref.sinkhorn_forward(la1, 1.0, 100)
    grad_fixed, gtau_fixed = ref.sinkhorn_backward_implicit(la1, P1, C1, 1.0, 100, 0.0)
    grad_cpu, gtau_cpu = ref.sinkhorn_backward_implicit(la1, P1, C1, 1.0, 100, 1e-6)
    _save("sk_c1", cost=C1, tau=np.float32(1.0), n_iters=100, backward_iters=100, P=P1,
          grad_fixed=grad_fixed, grad_tau_fixed=gtau_fixed, grad_cpu=grad_cpu, grad_tau_cpu=gtau_cpu)

    # Small regularisation, long run.
    C = rng.random((1, 32, 48)).astype(np.float32)
    P = ref.sinkhorn_forward(-C, 0.05, 200)
    _save("sk_fwd_smallreg", cost=C, tau=np.float32(0.05), n_iters=200, P=P)

    # Rectangular, non-uniform marginals, random upstream gradient: implicit (fixed and CPU break)
    # and unrolled backward.
    C = rng.random((2, 8, 16)).astype(np.float32)
    a, b = _dirichlet(rng, 2, 8), _dirichlet(rng, 2, 16)
    la, lga, lgb = -C, np.log(a), np.log(b)
    G = rng.standard_normal((2, 8, 16)).astype(np.float32)
    P, gi, gti = ref.sinkhorn_with_grads_implicit(la, G, 1.0, 20, 20, lga, lgb, tol=0.0)
    _, gic, gtic = ref.sinkhorn_with_grads_implicit(la, G, 1.0, 20, 20, lga, lgb, tol=1e-6)
    Pu, gu, gtu = ref.sinkhorn_with_grads_unrolled(la, G, 1.0, 20, lga, lgb)
    _save("sk_grads_8x16", log_alpha=la, log_a=lga, log_b=lgb, grad_P=G, tau=np.float32(1.0),
          n_iters=20, backward_iters=20, P=P, grad_implicit=gi, grad_tau_implicit=gti,
          grad_implicit_cpu=gic, grad_tau_implicit_cpu=gtic, P_unrolled=Pu, grad_unrolled=gu,
          grad_tau_unrolled=gtu)

    # Mirrors test_sinkhorn_cuda_dual_unrolled_matches_full_matrix_fixed_iterations
    # (test_sinkhorn.py:806-823): 48x64, reg 0.1, 30 iterations, loss = cost.sum().
    C = rng.random((1, 48, 64)).astype(np.float32)
    P, gu, gtu = ref.sinkhorn_with_grads_unrolled(-C, C, 0.1, 30)
    _save("sk_unrolled_48x64", cost=C, tau=np.float32(0.1), n_iters=30, P=P, grad_unrolled=gu,
          grad_tau_unrolled=gtu)


def bidi_cases():
    rng = np.random.default_rng(4321)

    # Variable lengths as in test_bidirectional_softmax_variable_lengths_* (:85-128).
    s = rng.standard_normal((2, 10, 15)).astype(np.float32)
    ln = np.array([[8, 12], [6, 10]], np.int32)
    g = rng.standard_normal(s.shape).astype(np.float32)
    out, r, c = ref.bidirectional_softmax(s, 1.0, ln)
    gs, gt = ref.bidirectional_softmax_backward(s, out, g, r, c, 1.0, ln)
    _save("bidi_varlen", sim=s, lengths=ln, tau=np.float32(1.0), grad_out=g, out=out, row_sm=r,
          col_sm=c, grad_sim=gs, grad_tau=gt)

    # Full lengths, tau 0.5, non-square.
    s = rng.standard_normal((2, 8, 10)).astype(np.float32)
    ln = np.array([[8, 10], [8, 10]], np.int32)
    g = rng.standard_normal(s.shape).astype(np.float32)
    out, r, c = ref.bidirectional_softmax(s, 0.5, ln)
    gs, gt = ref.bidirectional_softmax_backward(s, out, g, r, c, 0.5, ln)
    _save("bidi_full", sim=s, lengths=ln, tau=np.float32(0.5), grad_out=g, out=out, row_sm=r,
          col_sm=c, grad_sim=gs, grad_tau=gt)

    # Strong diagonal at a sharp and a soft temperature (test_temperature_effect_*, :158-196).
    s = np.zeros((1, 5, 5), np.float32)
    s[0, np.arange(5), np.arange(5)] = 10.0
    ln = np.array([[5, 5]], np.int32)
    g = np.ones_like(s)
    outs = {}
    for name, tau in (("sharp", 0.1), ("soft", 10.0)):
        out, r, c = ref.bidirectional_softmax(s, tau, ln)
        gs, gt = ref.bidirectional_softmax_backward(s, out, g, r, c, tau, ln)
        outs.update({f"out_{name}": out, f"grad_sim_{name}": gs, f"grad_tau_{name}": gt})
    _save("bidi_diag", sim=s, lengths=ln, grad_out=g, **outs)

    # Config C2 shape family at a reduced size (B=2, 64x80), tau 1.0, sim ~ N(0,1), grad ~ N(0,1).
    s = rng.standard_normal((2, 64, 80)).astype(np.float32)
    ln = np.array([[64, 80], [50, 33]], np.int32)
    g = rng.standard_normal(s.shape).astype(np.float32)
    out, r, c = ref.bidirectional_softmax(s, 1.0, ln)
    gs, gt = ref.bidirectional_softmax_backward(s, out, g, r, c, 1.0, ln)
    _save("bidi_64x80", sim=s, lengths=ln, tau=np.float32(1.0), grad_out=g, out=out, row_sm=r,
          col_sm=c, grad_sim=gs, grad_tau=gt)


if __name__ == "__main__":
    if not ref.available():
        sys.exit("oracle/_ref/libdotref.so missing: run `make -C oracle` first")
    sinkhorn_cases()
    bidi_cases()
