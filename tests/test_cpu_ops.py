"""CPU: the eight torch.ops.dot operators on CPU tensors (the reference's
src/sinkhorn/torch_cpu.cpp and src/bidirectional_softmax/torch_cpu.cpp).

Checked against the golden vectors of the reference's compiled CPU kernels
(tests/golden, written by make_golden.py from oracle/_ref), against the numpy
oracle on shapes the fixtures do not cover, for the reference's CPU-op
semantics (dual_forward ignores tol; the implicit adjoint stops at 1e-6), and
through the public API with the reference's own CPU tests.  Tolerances as the
GPU suite: plans 1e-5, gradients 1e-4 (norm-wise relative).
"""

import numpy as np
import pytest
import torch

import dot_amd
from dot_amd import _ops
from conftest import load_golden, rel_err, sum_err
from oracle import bidirectional_softmax as obs
from oracle import sinkhorn as osk

FWD_TOL, GRAD_TOL = 1e-5, 1e-4


def _t(x):
    return None if x is None else torch.from_numpy(np.ascontiguousarray(x))


# ---------------------------------------------------------------------------
# Golden vectors of the reference's CPU kernels
# ---------------------------------------------------------------------------
def test_forward_golden_6x9():
    g = load_golden("sk_fwd_6x9")
    la, lga, lgb = _t(g["log_alpha"]), _t(g["log_a"]), _t(g["log_b"])
    tau, T = float(g["tau"]), int(g["n_iters"])
    assert rel_err(_ops.sinkhorn(la, tau, T, lga, lgb), g["P"]) < FWD_TOL
    assert np.abs(_ops.sinkhorn_log(la, tau, T, lga, lgb).numpy() - g["logP"]).max() < 1e-4
    P, used, conv = _ops.sinkhorn_dual_forward(la, tau, T, 1e-6, lga, lgb)
    assert rel_err(P, g["P"]) < FWD_TOL
    # the CPU op ignores tol and method (torch_cpu.cpp:115-151)
    assert int(used) == T and int(conv) == 0
    _, used, conv = _ops.sinkhorn_dual_forward(la, tau, T, 0.0, lga, lgb, False, 2)
    assert int(used) == T and int(conv) == 1


def test_forward_golden_small_reg():
    g = load_golden("sk_fwd_smallreg")
    P = _ops.sinkhorn(_t(-g["cost"]), float(g["tau"]), int(g["n_iters"]))
    assert rel_err(P, g["P"]) < FWD_TOL


def test_implicit_golden_c1():
    # the CPU adjoint stops once the largest change is below 1e-6
    g = load_golden("sk_c1")
    C = g["cost"]
    P, grad, gtau = _ops.sinkhorn_with_grads_implicit(_t(-C), _t(C), float(g["tau"]), int(g["n_iters"]),
                                                      int(g["backward_iters"]))
    assert rel_err(P, g["P"]) < FWD_TOL
    assert rel_err(grad, g["grad_cpu"]) < GRAD_TOL
    terms = grad.numpy() * -C / float(g["tau"])
    assert sum_err(gtau, g["grad_tau_cpu"], terms) < GRAD_TOL


def test_grads_golden_8x16():
    g = load_golden("sk_grads_8x16")
    la, lga, lgb, G = _t(g["log_alpha"]), _t(g["log_a"]), _t(g["log_b"]), _t(g["grad_P"])
    tau, T, BT = float(g["tau"]), int(g["n_iters"]), int(g["backward_iters"])
    P, gi, gti = _ops.sinkhorn_with_grads_implicit(la, G, tau, T, BT, lga, lgb)
    assert rel_err(P, g["P"]) < FWD_TOL
    assert rel_err(gi, g["grad_implicit_cpu"]) < GRAD_TOL
    terms = lambda gr: gr.numpy() * g["log_alpha"] / tau
    assert sum_err(gti, g["grad_tau_implicit_cpu"], terms(gi)) < GRAD_TOL
    Pu, gu, gtu = _ops.sinkhorn_with_grads_unrolled(la, G, tau, T, lga, lgb)
    assert rel_err(Pu, g["P_unrolled"]) < FWD_TOL
    assert rel_err(gu, g["grad_unrolled"]) < GRAD_TOL
    assert sum_err(gtu, g["grad_tau_unrolled"], terms(gu) / tau) < GRAD_TOL


def test_unrolled_golden_48x64():
    g = load_golden("sk_unrolled_48x64")
    C = g["cost"]
    P, gu, gtu = _ops.sinkhorn_with_grads_unrolled(_t(-C), _t(C), float(g["tau"]), int(g["n_iters"]))
    assert rel_err(P, g["P"]) < FWD_TOL
    assert rel_err(gu, g["grad_unrolled"]) < GRAD_TOL


@pytest.mark.parametrize("name", ["bidi_varlen", "bidi_full", "bidi_64x80"])
def test_bidi_golden(name):
    g = load_golden(name)
    s, ln, tau = _t(g["sim"]), _t(g["lengths"]), float(g["tau"])
    out, r, c = _ops.bidirectional_softmax(s, tau, ln)
    assert rel_err(out, g["out"]) < FWD_TOL
    assert rel_err(r, g["row_sm"]) < FWD_TOL and rel_err(c, g["col_sm"]) < FWD_TOL
    gs, gt = _ops.bidirectional_softmax_backward(s, out, _t(g["grad_out"]), r, c, tau, ln)
    assert rel_err(gs, g["grad_sim"]) < GRAD_TOL
    assert sum_err(gt, g["grad_tau"], gs.numpy() * g["sim"] / tau) < GRAD_TOL


def test_bidi_golden_temperatures():
    g = load_golden("bidi_diag")
    s, ln, G = _t(g["sim"]), _t(g["lengths"]), _t(g["grad_out"])
    for name, tau in (("sharp", 0.1), ("soft", 10.0)):
        out, r, c = _ops.bidirectional_softmax(s, tau, ln)
        assert rel_err(out, g["out_" + name]) < FWD_TOL
        gs, _ = _ops.bidirectional_softmax_backward(s, out, G, r, c, tau, ln)
        # the exact gradient is 0 here (diagonal sim, ones upstream); both sides
        # hold ~1e-9 of rounding noise, so only an absolute bound means anything
        assert gs.abs().max() < 1e-6 and np.abs(g["grad_sim_" + name]).max() < 1e-6


# ---------------------------------------------------------------------------
# Oracle on shapes the fixtures do not cover
# ---------------------------------------------------------------------------
SHAPES = [(1, 1, 1), (2, 1, 7), (3, 7, 1), (2, 37, 29), (1, 130, 90), (4, 33, 64)]


@pytest.mark.parametrize("shape", SHAPES)
def test_forward_and_grads_match_oracle(shape):
    B, M, N = shape
    rng = np.random.default_rng(M * 31 + N)
    la = (-rng.random(shape)).astype(np.float32)
    e = -np.log(rng.random((B, M)))
    lga = np.log(e / e.sum(1, keepdims=True)).astype(np.float32)
    e = -np.log(rng.random((B, N)))
    lgb = np.log(e / e.sum(1, keepdims=True)).astype(np.float32)
    G = rng.standard_normal(shape).astype(np.float32)
    for tau, T in ((0.1, 30), (1.0, 5)):
        P = _ops.sinkhorn(_t(la), tau, T, _t(lga), _t(lgb))
        assert rel_err(P, osk.dual_forward(la, tau, T, 0.0, lga, lgb).P) < FWD_TOL
        Pu, gu, gtu = _ops.sinkhorn_with_grads_unrolled(_t(la), _t(G), tau, T, _t(lga), _t(lgb))
        ru = osk.with_grads_unrolled(la, G, tau, T, lga, lgb)
        assert rel_err(gu, ru[1]) < GRAD_TOL
        assert sum_err(gtu, ru[2], gu.numpy() * la / tau) < GRAD_TOL


def test_spectral_preflight_matches_oracle():
    rng = np.random.default_rng(5)
    for shape in ((3, 37, 29), (1, 64, 200)):
        la = (0.5 * rng.standard_normal(shape)).astype(np.float32)
        for tau, n_power in ((0.4, 5), (1.5, 8)):
            est = _ops.sinkhorn_spectral_preflight(_t(la), tau, n_power)
            assert rel_err(est, osk.spectral_preflight_tau(la, tau, n_power)) < FWD_TOL


def test_bidi_matches_oracle_with_ragged_lengths():
    rng = np.random.default_rng(9)
    s = rng.standard_normal((3, 17, 23)).astype(np.float32)
    ln = np.array([[17, 23], [0, 5], [9, 40]], np.int32)  # empty rows; a length past the tensor
    g = rng.standard_normal(s.shape).astype(np.float32)
    out, r, c = _ops.bidirectional_softmax(_t(s), 0.7, _t(ln))
    clamped = np.minimum(ln, [17, 23]).astype(np.int32)
    ro, rr, rc = obs.forward(s, 0.7, clamped)
    assert rel_err(out, ro) < FWD_TOL
    gs, gt = _ops.bidirectional_softmax_backward(_t(s), out, _t(g), r, c, 0.7, _t(ln))
    rg = obs.backward(s, ro, g, rr, rc, 0.7, clamped)
    assert rel_err(gs, rg[0]) < GRAD_TOL


def test_results_do_not_depend_on_the_thread_count():
    rng = np.random.default_rng(3)
    la = _t((-rng.random((3, 200, 70))).astype(np.float32))
    G = _t(rng.standard_normal((3, 200, 70)).astype(np.float32))
    threads = torch.get_num_threads()
    try:
        torch.set_num_threads(1)
        one = _ops.sinkhorn_with_grads_implicit(la, G, 0.1, 20, 20)
        torch.set_num_threads(max(threads, 4))
        many = _ops.sinkhorn_with_grads_implicit(la, G, 0.1, 20, 20)
    finally:
        torch.set_num_threads(threads)
    for x, y in zip(one, many):
        assert torch.equal(x, y)


def test_argument_errors():
    x = torch.rand(2, 4, 4)
    with pytest.raises(RuntimeError, match="tau must be > 0"):
        _ops.sinkhorn(x, 0.0, 5)
    with pytest.raises(RuntimeError, match="3D"):
        _ops.sinkhorn(x[0], 1.0, 5)
    with pytest.raises(RuntimeError, match="log_a must have shape"):
        _ops.sinkhorn(x, 1.0, 5, torch.zeros(2, 5))
    with pytest.raises(RuntimeError, match="grad_P must match"):
        _ops.sinkhorn_with_grads_implicit(x, torch.zeros(2, 4, 5), 1.0, 5, 5)
    with pytest.raises(RuntimeError, match="lengths must be int32"):
        _ops.bidirectional_softmax(x, 1.0, torch.ones(2, 2))


# ---------------------------------------------------------------------------
# Public API on CPU tensors: the reference's CPU tests (test_sinkhorn.py)
# ---------------------------------------------------------------------------
def test_ref_sinkhorn_doubly_stochastic_cpu():
    cost = torch.rand(2, 10, 10)
    res = dot_amd.sinkhorn(cost, reg=0.1, n_iters=100)
    P = res.transport_plan
    assert torch.allclose(P.sum(-1), torch.full((2, 10), 0.1), atol=1e-3)
    assert torch.allclose(P.sum(-2), torch.full((2, 10), 0.1), atol=1e-3)
    assert res.n_iters_used == 100 and res.converged is False  # CPU path: converged = tol == 0


def test_ref_gradients_flow_cpu():
    for mode in ("implicit", "unrolled"):
        cost = torch.rand(2, 8, 8, requires_grad=True)
        res = dot_amd.sinkhorn(cost, reg=0.5, n_iters=30, backward_mode=mode)
        res.cost.sum().backward()
        assert cost.grad is not None and torch.isfinite(cost.grad).all()


def test_ref_differentiable_reg_matches_finite_difference_cpu():
    # test_sinkhorn.py:400-416
    cost = torch.eye(5).unsqueeze(0)
    eps = torch.tensor(0.2, requires_grad=True)
    dot_amd.sinkhorn(cost, reg=eps, n_iters=80).cost.sum().backward()
    d = 1e-3
    plus = dot_amd.sinkhorn(cost, reg=float(eps.detach() + d), n_iters=80).cost.sum().item()
    minus = dot_amd.sinkhorn(cost, reg=float(eps.detach() - d), n_iters=80).cost.sum().item()
    assert eps.grad.item() > 0
    assert abs(eps.grad.item() - (plus - minus) / (2 * d)) < 5e-2


def test_ref_from_scores_and_modules_cpu():
    la = torch.randn(2, 6, 6)
    P = dot_amd.sinkhorn_from_scores(la, tau=0.5, n_iters=50)
    logP = dot_amd.sinkhorn_from_scores(la, tau=0.5, n_iters=50, return_log=True)
    assert torch.allclose(P, logP.exp(), atol=1e-6)
    m = dot_amd.Sinkhorn(reg=0.5, n_iters=40)
    assert m(torch.rand(6, 6)).transport_plan.shape == (6, 6)
    out = dot_amd.bidirectional_softmax(torch.randn(2, 5, 7), tau=0.5)
    assert out.shape == (2, 5, 7) and torch.isfinite(out).all()


def test_ref_cpu_cuda_paths_agree_on_auto_iterations():
    # n_iters='auto' runs the spectral preflight on CPU tensors too
    cost = torch.rand(2, 12, 12)
    res = dot_amd.sinkhorn(cost, reg=0.5, n_iters="auto", tol=1e-4)
    assert 3 <= res.n_iters_used <= 1000
