"""GPU parity of the bidirectional softmax: HIP kernels against the oracle, the
golden fixtures and, at the C2 size, the float64 closed form and its autograd."""

import numpy as np
import pytest
import torch

import dot_amd
from dot_amd import _ops
from conftest import load_golden, rel_err, sum_err
from oracle import bidirectional_softmax as obs

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)
FWD_TOL, GRAD_TOL = 1e-5, 1e-4


def _t(x):
    return torch.as_tensor(np.ascontiguousarray(x)).to(DEV)


@pytest.mark.parametrize("name", ["bidi_varlen", "bidi_full", "bidi_64x80"])
def test_ops_match_golden(name):
    g = load_golden(name)
    tau = float(g["tau"])
    sim, ln = _t(g["sim"]), _t(g["lengths"])
    out, r, c = _ops.bidirectional_softmax(sim, tau, ln)
    assert rel_err(out, g["out"]) < FWD_TOL
    assert rel_err(r, g["row_sm"]) < FWD_TOL
    assert rel_err(c, g["col_sm"]) < FWD_TOL
    gs, gt = _ops.bidirectional_softmax_backward(sim, out, _t(g["grad_out"]), r, c, tau, ln)
    assert rel_err(gs, g["grad_sim"]) < GRAD_TOL
    assert sum_err(gt, g["grad_tau"], gs.cpu().numpy() * g["sim"] / tau) < GRAD_TOL
    # the fused autograd path (statistics instead of saved buffers)
    x = sim.clone().requires_grad_(True)
    P = dot_amd.bidirectional_softmax(x, tau, ln)
    P.backward(_t(g["grad_out"]))
    assert rel_err(P, g["out"]) < FWD_TOL
    assert rel_err(x.grad, g["grad_sim"]) < GRAD_TOL


SHAPES = [
    # (B, L1, L2, tau, lengths or None)
    (1, 1, 1, 1.0, None),
    (2, 7, 9, 0.3, [[7, 9], [3, 2]]),
    (3, 33, 130, 2.0, [[33, 130], [0, 130], [33, 0]]),
    (2, 256, 256, 1.0, None),
    (2, 100, 1023, 0.5, [[100, 1023], [61, 999]]),
    (1, 512, 4096, 1.0, None),
    (1, 300, 4093, 0.8, [[250, 4000]]),
    (4, 1500, 64, 1.0, [[1500, 64], [1, 1], [700, 10], [1499, 63]]),
    # rows longer than 4096 columns (strips x chunks tiles); L2 % 4 != 0: scalar loads
    (2, 40, 4097, 1.0, [[40, 4097], [17, 3000]]),
    (1, 64, 6000, 0.7, None),
    (2, 33, 8192, 1.3, [[33, 8192], [20, 6001]]),
    (1, 16, 5001, 1.0, [[16, 4500]]),
]


@pytest.mark.parametrize("B,L1,L2,tau,lengths", SHAPES)
def test_forward_backward_match_oracle(B, L1, L2, tau, lengths):
    rng = np.random.default_rng(B + L1 + L2)
    s = (2.0 * rng.standard_normal((B, L1, L2))).astype(np.float32)
    g = rng.standard_normal((B, L1, L2)).astype(np.float32)
    ln = np.array(lengths if lengths is not None else [[L1, L2]] * B, np.int32)
    out_o, r_o, c_o = obs.forward(s, tau, ln)
    gs_o, gt_o = obs.backward(s, out_o, g, r_o, c_o, tau, ln)
    out, r, c = _ops.bidirectional_softmax(_t(s), tau, _t(ln))
    assert rel_err(out, out_o) < FWD_TOL
    assert rel_err(r, r_o) < FWD_TOL and rel_err(c, c_o) < FWD_TOL
    gs, gt = _ops.bidirectional_softmax_backward(_t(s), out, _t(g), r, c, tau, _t(ln))
    assert rel_err(gs, gs_o) < GRAD_TOL
    assert sum_err(gt, gt_o, gs_o * s / tau) < GRAD_TOL
    x = _t(s).requires_grad_(True)
    P = dot_amd.bidirectional_softmax(x, tau, _t(ln))
    P.backward(_t(g))
    assert rel_err(P, out_o) < FWD_TOL
    assert rel_err(x.grad, gs_o) < GRAD_TOL
    # padding is exactly zero
    for b in range(B):
        l1, l2 = ln[b]
        for T in (P.detach(), r, c, gs, x.grad):
            assert (T[b, l1:, :] == 0).all() and (T[b, :, l2:] == 0).all()


def test_config_c2_full_size_against_float64_closed_form():
    B, L1, L2 = 32, 1024, 1024
    sim = torch.randn(B, L1, L2, generator=torch.Generator().manual_seed(1)).to(DEV)
    G = torch.randn(B, L1, L2, generator=torch.Generator().manual_seed(2)).to(DEV)
    x = sim.clone().requires_grad_(True)
    P = dot_amd.bidirectional_softmax(x, 1.0)
    P.backward(G)
    x64 = sim.double().requires_grad_(True)
    ref = torch.sqrt(1e-9 + torch.softmax(x64, dim=2) * torch.softmax(x64, dim=1))
    ref.backward(G.double())
    assert rel_err(P, ref) < FWD_TOL
    assert rel_err(x.grad, x64.grad) < GRAD_TOL
    assert (P >= 0).all() and (P <= 1).all()
    # the drop-in operator path agrees with the fused autograd path
    out, r, c = _ops.bidirectional_softmax(sim, 1.0, torch.tensor([[L1, L2]] * B, dtype=torch.int32, device=DEV))
    assert rel_err(out, P) < 1e-6


# The reference's own GPU tests (tests/test_bidirectional_softmax.py), re-expressed
def test_reference_shape_and_range():  # :15-31
    sim = torch.randn(2, 10, 15, device=DEV)
    P = dot_amd.bidirectional_softmax(sim, tau=1.0)
    assert P.shape == (2, 10, 15) and (P >= 0).all() and (P <= 1).all()


def test_reference_backward():  # :54-66
    sim = torch.randn(2, 8, 12, device=DEV, requires_grad=True)
    dot_amd.bidirectional_softmax(sim, tau=1.0).sum().backward()
    assert sim.grad is not None and sim.grad.shape == sim.shape


def test_reference_variable_lengths():  # :85-106
    sim = torch.randn(2, 10, 15, device=DEV)
    lengths = torch.tensor([[8, 12], [6, 10]], dtype=torch.int32, device=DEV)
    P = dot_amd.bidirectional_softmax_with_lengths(sim, lengths, tau=1.0)
    assert (P[0, 8:, :] == 0).all() and (P[0, :, 12:] == 0).all()
    assert (P[1, 6:, :] == 0).all() and (P[1, :, 10:] == 0).all()


def test_reference_temperature_effect():  # :158-177
    sim = torch.zeros(1, 5, 5, device=DEV)
    sim[0, torch.arange(5), torch.arange(5)] = 10.0
    sharp = dot_amd.bidirectional_softmax(sim, tau=0.1)
    soft = dot_amd.bidirectional_softmax(sim, tau=10.0)
    assert sharp[0].diag().sum() > soft[0].diag().sum()


def test_unbatched_and_module():
    sim = torch.randn(10, 15, device=DEV)
    P = dot_amd.bidirectional_softmax(sim, tau=1.0)
    assert P.shape == (10, 15)
    Q = dot_amd.BidirectionalSoftmax(tau=0.5)(sim.unsqueeze(0))
    assert Q.shape == (1, 10, 15)


def test_op_argument_errors():
    sim = torch.randn(2, 4, 4, device=DEV)
    with pytest.raises(RuntimeError, match="int32"):
        _ops.bidirectional_softmax(sim, 1.0, torch.ones(2, 2, dtype=torch.int64, device=DEV))
    with pytest.raises(RuntimeError, match=r"\[B, 2\]"):
        _ops.bidirectional_softmax(sim, 1.0, torch.ones(2, 3, dtype=torch.int32, device=DEV))
    with pytest.raises(RuntimeError, match="tau must be > 0"):
        _ops.bidirectional_softmax(sim, 0.0, torch.ones(2, 2, dtype=torch.int32, device=DEV))


@pytest.mark.gpu
def test_reference_cpu_cuda_consistency():
    """test_bidirectional_softmax.py's test_cpu_cuda_consistency, plus the
    backward: the CPU operators and the HIP kernels agree."""
    torch.manual_seed(3)
    for B, L1, L2 in ((2, 8, 10), (3, 33, 70)):
        sim_cpu = torch.randn(B, L1, L2)
        G = torch.randn(B, L1, L2)
        outs = []
        for dev in ("cpu", DEV):
            s = sim_cpu.detach().to(dev).clone().requires_grad_(True)
            P = dot_amd.bidirectional_softmax(s, tau=1.0)
            P.backward(G.to(dev))
            outs.append((P.detach().cpu(), s.grad.cpu()))
        assert torch.allclose(outs[0][0], outs[1][0], atol=1e-5)
        assert rel_err(outs[1][1], outs[0][1]) < 1e-4


def test_batch_above_65535():
    """Batch elements spill from grid y into grid z beyond 65535: forward and
    backward at B = 70001 against the oracle, ragged lengths included."""
    rng = np.random.default_rng(65536)
    B, L1, L2, tau = 70001, 3, 5, 0.9
    s = rng.standard_normal((B, L1, L2)).astype(np.float32)
    g = rng.standard_normal((B, L1, L2)).astype(np.float32)
    ln = np.stack([rng.integers(0, L1 + 1, B), rng.integers(0, L2 + 1, B)], 1).astype(np.int32)
    ln[-1] = [L1, L2]
    out_o, r_o, c_o = obs.forward(s, tau, ln)
    gs_o, gt_o = obs.backward(s, out_o, g, r_o, c_o, tau, ln)
    out, r, c = _ops.bidirectional_softmax(_t(s), tau, _t(ln))
    assert rel_err(out, out_o) < FWD_TOL and rel_err(c, c_o) < FWD_TOL
    gs, gt = _ops.bidirectional_softmax_backward(_t(s), out, _t(g), r, c, tau, _t(ln))
    assert rel_err(gs, gs_o) < GRAD_TOL
    # grad_tau of 70001 tiny elements: where one valid row meets a few valid
    # columns its terms nearly cancel, and float32 itself lands up to ~4e-4 of
    # sum|terms| from float64 (the oracle's float32 run shows the same figure),
    # so each element is held to max(1e-4, 2x the float32 spread)
    o32, r32, c32 = obs.forward(s, tau, ln, dtype=np.float32)
    _, gt32 = obs.backward(s, o32, g, r32, c32, tau, ln, dtype=np.float32)
    terms = gs_o * s / tau
    spread = sum_err(gt32, gt_o, terms)
    assert sum_err(gt, gt_o, terms) < max(GRAD_TOL, 2 * spread), spread
    x = _t(s).requires_grad_(True)
    P = dot_amd.bidirectional_softmax(x, tau, _t(ln))
    P.backward(_t(g))
    assert rel_err(P, out_o) < FWD_TOL and rel_err(x.grad, gs_o) < GRAD_TOL
    assert rel_err(x.grad[-1:], gs_o[-1:]) < GRAD_TOL
