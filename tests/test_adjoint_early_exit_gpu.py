"""GPU parity of the implicit adjoint's early end (register-resident and
persistent tiers).

The reference's GPU op runs exactly backward_iters Gauss-Seidel sweeps
(src/sinkhorn/kernels.cu:1715-1718); this build ends a batch element's sweeps
once they have converged (sk::AdjointStop: a fixed point, a geometric bound on
what the remaining sweeps could change below the rounding of the mu update's
operands, or the sweeps' fp32 rounding floor).  These tests hold the early
end to the float64 oracle run at the FULL sweep count (gradients 1e-4,
north_star), to the same kernels run with DOT_AMD_EXACT_SWEEPS=1 (1e-5), and
check the sweep counts each result reports.  The BASELINE configurations run
at their real shapes, regs and sweep counts: C1 and C3 whole batches, C4 and
C5 one element (their forwards at a fixed count that the float64 forward has
long converged by: C4 100 iterations, C5 60).
"""

import numpy as np
import pytest
import torch

import dot_amd
from conftest import load_golden, rel_err
from oracle import sinkhorn as osk

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)
GRAD_TOL, FWD_TOL = 1e-4, 1e-5


def _t(x):
    return torch.as_tensor(np.ascontiguousarray(x)).to(DEV)


def _dirichlet(rng, B, n):
    e = -np.log(rng.random((B, n)))
    return (e / e.sum(1, keepdims=True)).astype(np.float32)


def _run(C, tau, T, BT, a=None, b=None, tol=0.0):
    """dot.sinkhorn fwd + cost.sum().backward() on the device."""
    leaf = C.clone().requires_grad_(True)
    res = dot_amd.sinkhorn(leaf, reg=tau, n_iters=T, tol=tol, backward_iters=BT, a=a, b=b)
    res.cost.sum().backward()
    return res, leaf.grad


def _oracle_grad(Cn, tau, T, BT, a=None, b=None):
    """dL/dC = P - dL/dlog_alpha for L = cost.sum(), float64, exactly BT sweeps."""
    lga = None if a is None else np.log(a)
    lgb = None if b is None else np.log(b)
    f = osk.dual_forward(-Cn, tau, T, 0.0, lga, lgb)
    gla, _, sweeps = osk.implicit_backward(-Cn, f.P, Cn, tau, BT)
    assert (sweeps == BT).all()
    return f.P, f.P - gla


TIERS = {"resident": {}, "persistent": {"DOT_AMD_RESIDENT": "0"}}


@pytest.mark.parametrize("tier", sorted(TIERS))
@pytest.mark.parametrize("B,M,N,tau,T,BT,nonuni", [
    (4, 512, 512, 0.1, 40, 200, False),
    (3, 300, 257, 0.3, 60, 150, True),
    (2, 64, 1000, 0.5, 30, 100, True),
    (5, 96, 128, 0.05, 200, 300, True),
])
def test_early_end_matches_the_full_count(tier, B, M, N, tau, T, BT, nonuni, monkeypatch):
    """Each tier with and without DOT_AMD_EXACT_SWEEPS: the exact run reports
    BT sweeps per element, the default run at most BT, and both gradients
    match the float64 oracle at the full BT sweeps and each other."""
    print(f"[early-end] tier={tier} B={B} M={M} N={N} tau={tau} T={T} BT={BT}", flush=True)
    rng = np.random.default_rng(B * 1000 + M + N)
    Cn = rng.random((B, M, N)).astype(np.float32)
    a = _dirichlet(rng, B, M) if nonuni else None
    b = _dirichlet(rng, B, N) if nonuni else None
    for k, v in TIERS[tier].items():
        monkeypatch.setenv(k, v)
    lt = lambda x: None if x is None else _t(x)
    C = _t(Cn)
    res, g = _run(C, tau, T, BT, lt(a), lt(b))
    monkeypatch.setenv("DOT_AMD_EXACT_SWEEPS", "1")
    res_x, g_x = _run(C, tau, T, BT, lt(a), lt(b))
    monkeypatch.delenv("DOT_AMD_EXACT_SWEEPS")
    Po, go = _oracle_grad(Cn, tau, T, BT, a, b)
    sweeps = res.adjoint_sweeps
    print(f"[early-end] sweeps {sweeps}", flush=True)
    assert res_x.adjoint_sweeps == [BT] * B
    assert len(sweeps) == B and all(1 <= s <= BT for s in sweeps)
    assert rel_err(res.transport_plan, Po) < FWD_TOL
    assert rel_err(g, go) < GRAD_TOL
    assert rel_err(g_x, go) < GRAD_TOL
    assert rel_err(g, g_x.cpu().numpy()) < 1e-5
    # the element's workgroups decide together and the same way on every run
    res2, g2 = _run(C, tau, T, BT, lt(a), lt(b))
    assert res2.adjoint_sweeps == sweeps and torch.equal(g2, g)


def test_solution_after_one_sweep_ends_within_a_few():
    """A row-constant upstream gradient (G_ik = g_i) is solved by the first
    sweep (lambda = g, mu = 0 up to rounding): the later sweeps only move
    within the rounding, which ends the adjoint within a few sweeps, and
    grad_log_alpha = P (G - lambda - mu) / tau is 0 up to that rounding."""
    rng = np.random.default_rng(5)
    B, M, N = 3, 256, 384
    C = _t(rng.random((B, M, N)).astype(np.float32))
    leaf = C.clone().requires_grad_(True)
    res = dot_amd.sinkhorn(leaf, reg=0.2, n_iters=50, tol=0)
    g = torch.as_tensor(rng.standard_normal((B, M, 1)).astype(np.float32)).to(DEV)
    (res.transport_plan * g).sum().backward()
    assert max(res.adjoint_sweeps) <= 8, res.adjoint_sweeps
    assert leaf.grad.abs().max().item() <= 1e-6 * res.transport_plan.abs().max().item() / 0.2 * g.abs().max().item()


def test_config_c1_full_count_against_golden():
    """C1 (8 x 64^2, reg 1, 100 iterations, 100 sweeps): the reference's own
    CPU kernels' gradient after exactly 100 sweeps (golden fixture)."""
    gd = load_golden("sk_c1")
    res, g = _run(_t(gd["cost"]), 1.0, 100, 100)
    print(f"[early-end] C1 sweeps {res.adjoint_sweeps}", flush=True)
    assert rel_err(res.transport_plan, gd["P"]) < FWD_TOL
    assert rel_err(g, gd["P"] - gd["grad_fixed"]) < GRAD_TOL


def _c3_cost():
    g = torch.Generator().manual_seed(3)
    x, y = torch.randn(64, 512, 64, generator=g), torch.randn(64, 512, 64, generator=g)
    C = torch.cdist(x.to(DEV), y.to(DEV)).square()
    return (C / C.amax(dim=(-2, -1), keepdim=True)).contiguous()


def test_config_c3_whole_batch_full_count():
    """C3 (64 x 512^2, reg 0.1, tol 1e-6, 200 sweeps), all 64 elements: the
    plan at the run's own iteration count and the cost gradient against the
    float64 oracle's 200-sweep adjoint."""
    C = _c3_cost()
    res, g = _run(C, 0.1, 200, 200, tol=1e-6)
    T = res.n_iters_used
    sweeps = res.adjoint_sweeps
    print(f"[early-end] C3 T_f={T} sweeps min {min(sweeps)} max {max(sweeps)}", flush=True)
    Po, go = _oracle_grad(C.cpu().numpy(), 0.1, T, 200)
    assert rel_err(res.transport_plan, Po) < FWD_TOL
    assert rel_err(g, go) < GRAD_TOL
    assert max(sweeps) < 200


def test_config_c4_one_element_full_count():
    """C4 (1024 x 2048, reg 0.05, Dirichlet marginals, 500 sweeps), element 0,
    persistent tier; forward at 100 iterations (the float64 forward stops at 7
    under tol 1e-6)."""
    g = torch.Generator().manual_seed(4)
    Cf = torch.rand(16, 1024, 2048, generator=g)
    ea, eb = -torch.log(torch.rand(16, 1024, generator=g)), -torch.log(torch.rand(16, 2048, generator=g))
    a, b = (ea / ea.sum(-1, keepdim=True))[:1], (eb / eb.sum(-1, keepdim=True))[:1]
    Cn = Cf[:1].numpy()
    res, gr = _run(_t(Cn), 0.05, 100, 500, _t(a.numpy()), _t(b.numpy()))
    print(f"[early-end] C4 sweeps {res.adjoint_sweeps}", flush=True)
    Po, go = _oracle_grad(Cn, 0.05, 100, 500, a.numpy(), b.numpy())
    assert rel_err(res.transport_plan, Po) < FWD_TOL
    assert rel_err(gr, go) < GRAD_TOL
    assert res.adjoint_sweeps[0] < 500


def test_config_c5_one_element_full_count():
    """C5 (4096^2, reg 0.02, 1000 sweeps), element 0, persistent tier; forward
    at 60 iterations (a documented subset of the 1000: the oracle's float64
    forward at 4096^2 takes ~0.2 s per iteration on the host)."""
    g = torch.Generator().manual_seed(5)
    x, y = torch.randn(4, 4096, 128, generator=g), torch.randn(4, 4096, 128, generator=g)
    C = torch.cdist(x[:1].to(DEV), y[:1].to(DEV))
    C = (C / C.amax(dim=(-2, -1), keepdim=True)).contiguous()
    res, gr = _run(C, 0.02, 60, 1000)
    print(f"[early-end] C5 sweeps {res.adjoint_sweeps}", flush=True)
    Po, go = _oracle_grad(C.cpu().numpy(), 0.02, 60, 1000)
    assert rel_err(res.transport_plan, Po) < FWD_TOL
    assert rel_err(gr, go) < GRAD_TOL
    assert res.adjoint_sweeps[0] < 1000


@pytest.mark.parametrize("B", [128, 300])
def test_c3_shape_at_larger_batches(B):
    """C3's shape, inputs and solver at B = 128 (persistent forward) and B =
    300 (per-iteration forward sweeps); both adjoints run as slabs of the
    register-resident adjoint (64 elements each at 512 x 512), which end
    early: the forward's stop count, and the first and last element of the
    first and last slab against the float64 oracle (plan at the run's count,
    cost gradient after the full 200 sweeps)."""
    g = torch.Generator().manual_seed(3)
    x, y = torch.randn(B, 512, 64, generator=g), torch.randn(B, 512, 64, generator=g)
    C = torch.cdist(x.to(DEV), y.to(DEV)).square()
    C = (C / C.amax(dim=(-2, -1), keepdim=True)).contiguous()
    res, gr = _run(C, 0.1, 200, 200, tol=1e-6)
    T = res.n_iters_used
    sweeps = res.adjoint_sweeps
    print(f"[early-end] C3 shape B={B}: T_f={T} sweeps min {min(sweeps)} max {max(sweeps)}", flush=True)
    assert res.converged and abs(T - 5) <= 1
    Cn = C.cpu().numpy()
    for b in (0, 63, 64, B - 1):
        Po, go = _oracle_grad(Cn[b:b + 1], 0.1, T, 200)
        assert rel_err(res.transport_plan[b:b + 1], Po) < FWD_TOL, b
        assert rel_err(gr[b:b + 1], go) < GRAD_TOL, b
    assert max(sweeps) < 200


def test_persistent_slabs_beyond_the_cus(monkeypatch):
    """More batch elements than CUs at rows of 1025-4096 columns: the
    adjoint runs as slabs of the persistent adjoint (one element per CU),
    each ending its elements' sweeps early.  Elements at the slabs' edges
    against the float64 oracle at the full sweep count; the exact run reports
    every sweep."""
    cus = torch.cuda.get_device_properties(DEV).multi_processor_count
    B, M, N, tau, T, BT = cus + 44, 64, 1100, 0.3, 60, 150
    print(f"[early-end] persistent slabs B={B} M={M} N={N}", flush=True)
    rng = np.random.default_rng(77)
    Cn = rng.random((B, M, N)).astype(np.float32)
    a, b = _dirichlet(rng, B, M), _dirichlet(rng, B, N)
    C = _t(Cn)
    res, g = _run(C, tau, T, BT, _t(a), _t(b))
    sweeps = res.adjoint_sweeps
    print(f"[early-end] slab sweeps min {min(sweeps)} max {max(sweeps)}", flush=True)
    assert len(sweeps) == B and all(1 <= s < BT for s in sweeps)
    for e in (0, cus - 1, cus, B - 1):
        Po, go = _oracle_grad(Cn[e:e + 1], tau, T, BT, a[e:e + 1], b[e:e + 1])
        assert rel_err(res.transport_plan[e:e + 1], Po) < FWD_TOL, e
        assert rel_err(g[e:e + 1], go) < GRAD_TOL, e
    monkeypatch.setenv("DOT_AMD_EXACT_SWEEPS", "1")
    res_x, g_x = _run(C, tau, T, BT, _t(a), _t(b))
    assert res_x.adjoint_sweeps == [BT] * B
    assert rel_err(g, g_x.cpu().numpy()) < 1e-5
