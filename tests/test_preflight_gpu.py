"""GPU parity of the spectral preflight (n_iters='auto'): the HIP sweeps
against the oracle, and the reference's own preflight tests
(tests/test_sinkhorn.py:840-910 of the reference)."""

import math

import numpy as np
import pytest
import torch

import dot_amd
from dot_amd import _ops
from oracle import sinkhorn as osk

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)


@pytest.mark.parametrize("B,M,N,tau,n_power,scale", [
    (2, 64, 64, 0.1, 5, 0.1),
    (3, 130, 70, 0.5, 8, 1.0),      # rows not a multiple of 4: scalar row layout
    (1, 300, 4096, 0.2, 5, 0.3),
    (4, 512, 512, 0.05, 8, 0.02),
    (2, 1000, 257, 1.0, 3, 2.0),
    # rows longer than 4096 columns: strips x chunks tiles; 4097 takes scalar loads
    (2, 40, 4500, 0.2, 5, 0.3),
    (1, 33, 4097, 0.5, 4, 1.0),
    (1, 130, 8192, 0.1, 6, 0.1),
])
def test_preflight_matches_oracle(B, M, N, tau, n_power, scale):
    rng = np.random.default_rng(B + M + N)
    X = (scale * rng.standard_normal((B, M, N))).astype(np.float32)
    est = _ops.sinkhorn_spectral_preflight(torch.from_numpy(X).to(DEV), tau, n_power).cpu().numpy()
    ref = osk.spectral_preflight_tau(X, tau, n_power)
    assert est.shape == (B,) and est.dtype == np.float32
    np.testing.assert_allclose(est, ref, rtol=1e-5, atol=1e-6)


def test_preflight_is_deterministic_and_batch_independent():
    rng = np.random.default_rng(3)
    X = torch.from_numpy((0.3 * rng.standard_normal((3, 200, 300))).astype(np.float32)).to(DEV)
    a = _ops.sinkhorn_spectral_preflight(X, 0.1, 8)
    b = _ops.sinkhorn_spectral_preflight(X, 0.1, 8)
    assert torch.equal(a, b)
    # element b of a batch sees the start vector of index b
    one = _ops.sinkhorn_spectral_preflight(X[:1].contiguous(), 0.1, 8)
    assert torch.equal(one, a[:1])


def test_auto_iterations_on_long_rows():
    # n_iters='auto' end to end on rows longer than 4096 columns: the count the
    # preflight predicts, then the forward at that count
    rng = np.random.default_rng(5)
    C = torch.from_numpy((0.2 * rng.random((2, 24, 5000))).astype(np.float32)).to(DEV)
    predicted = dot_amd.spectral_preflight(-C, 0.1, tol=1e-6)
    tau_est = osk.spectral_preflight_tau(-C.cpu().numpy(), 0.1, 5)
    assert predicted.shape == (2,) and (predicted >= 1).all()
    res = dot_amd.sinkhorn(C, reg=0.1, n_iters="auto", tol=1e-6)
    assert 1 <= res.n_iters_used <= int(predicted.max())
    assert torch.isfinite(res.transport_plan).all() and np.all(tau_est < 1.0)


def test_preflight_argument_errors():
    X = torch.zeros(1, 4, 4, device=DEV)
    with pytest.raises(RuntimeError, match="n_power must be >= 1"):
        _ops.sinkhorn_spectral_preflight(X, 0.1, 0)
    with pytest.raises(RuntimeError, match="tau must be > 0"):
        _ops.sinkhorn_spectral_preflight(X, 0.0, 5)
    with pytest.raises(RuntimeError, match="3D"):
        _ops.sinkhorn_spectral_preflight(X[0], 0.1, 5)


# --- the reference's preflight tests (test_sinkhorn.py:78-108, :840-910) ----
def _easy(n, scale=0.1, seed=0):
    gen = torch.Generator(device=DEV).manual_seed(seed)
    return scale * torch.randn((1, n, n), device=DEV, generator=gen).abs()


def _moderate(n, scale=0.005, seed=0):
    gen = torch.Generator(device=DEV).manual_seed(seed)
    x = torch.randn((n, 2), device=DEV, generator=gen)
    y = torch.randn((n, 2), device=DEV, generator=gen)
    return (scale * torch.cdist(x, y, p=2).square()).unsqueeze(0)


def _hard(n, scale):
    x = torch.linspace(-1.0, 1.0, n, device=DEV).unsqueeze(1)
    return (scale * torch.cdist(x, x, p=2).square()).unsqueeze(0)


def test_reference_preflight_returns_per_batch_predictions():  # :840-857
    cost = torch.cat([_easy(64, scale=0.1, seed=0), _easy(64, scale=0.2, seed=1)], dim=0)
    predicted = dot_amd.spectral_preflight(-cost, 0.1, tol=1e-6)
    assert isinstance(predicted, torch.Tensor)
    assert predicted.shape == (2,)
    assert predicted.dtype == torch.int64


def test_reference_preflight_validation_matrix():  # :860-893
    cases = [
        ("easy", 1.0, 100, lambda: _easy(100, scale=0.1, seed=0)),
        ("easy", 0.1, 500, lambda: _easy(500, scale=0.1, seed=0)),
        ("moderate", 0.01, 500, lambda: _moderate(500, scale=0.005, seed=0)),
        ("hard", 0.001, 500, lambda: _hard(500, scale=0.18)),
        ("easy", 0.1, 2000, lambda: _easy(2000, scale=0.1, seed=0)),
        ("moderate", 0.01, 2000, lambda: _moderate(2000, scale=0.005, seed=0)),
        ("hard", 0.001, 2000, lambda: _hard(2000, scale=0.25)),
    ]
    conservative = within_2x = 0
    failures = []
    for label, eps, n, factory in cases:
        cost = factory()
        predicted = dot_amd.spectral_preflight(-cost, eps, tol=1e-6)
        predicted_iters = int(predicted.max().item()) if torch.is_tensor(predicted) else int(predicted)
        actual_iters = dot_amd.sinkhorn(cost, reg=eps, n_iters=400, tol=1e-6).n_iters_used
        if predicted_iters >= actual_iters:
            conservative += 1
        else:
            failures.append(f"{label} eps={eps} n={n} predicted={predicted_iters} actual={actual_iters}")
        if predicted_iters <= 2 * actual_iters:
            within_2x += 1
        else:
            failures.append(f"{label} eps={eps} n={n} ratio={predicted_iters / actual_iters:.2f}")
    assert conservative >= math.ceil(0.95 * len(cases)), failures
    assert within_2x >= math.ceil(0.90 * len(cases)), failures


def test_reference_sinkhorn_auto_matches_converged_solution():  # :896-910
    cost = _moderate(256, scale=0.005, seed=0)
    predicted = dot_amd.spectral_preflight(-cost, 0.01, tol=1e-6)
    predicted_iters = int(predicted.max().item()) if torch.is_tensor(predicted) else int(predicted)
    auto = dot_amd.sinkhorn(cost, reg=0.01, n_iters="auto", tol=1e-6)
    converged = dot_amd.sinkhorn(cost, reg=0.01, n_iters=400, tol=1e-6)
    assert auto.n_iters_used is not None
    assert converged.n_iters_used is not None
    assert predicted_iters >= converged.n_iters_used
    assert auto.n_iters_used <= predicted_iters
