"""CPU: host-side logic of the package — the operator schemas, the drop-in
package name, argument validation and result types.  No kernel runs here."""

import pytest
import torch

import dot
import dot_amd
from dot_amd import _ops
from dot_amd.sinkhorn import _prepare_marginal, _resolve_iters

# The reference's schemas, src/sinkhorn/registry.cpp:31-56 and
# src/bidirectional_softmax/registry.cpp:31-34.
REFERENCE_SCHEMAS = {
    "sinkhorn": "dot::sinkhorn(Tensor log_alpha, float tau, int n_iters, Tensor? log_a=None, Tensor? log_b=None) -> Tensor",
    "sinkhorn_log": "dot::sinkhorn_log(Tensor log_alpha, float tau, int n_iters, Tensor? log_a=None, Tensor? log_b=None) -> Tensor",
    "sinkhorn_dual_forward": (
        "dot::sinkhorn_dual_forward(Tensor log_alpha, float tau, int n_iters, float tol=0., Tensor? log_a=None, "
        "Tensor? log_b=None, bool return_log=False, int method=0, float omega=1.5, int anderson_k=5, "
        "float mixing_beta=1., float lr=1., float beta1=0.90000000000000002, float beta2=0.999, "
        "float eps_adam=1e-08, bool bias_correction=True, float reg_start=-1., int schedule=0) -> Tensor[]"),
    "sinkhorn_spectral_preflight": "dot::sinkhorn_spectral_preflight(Tensor log_alpha, float tau, int n_power=8) -> Tensor",
    "sinkhorn_with_grads_unrolled": "dot::sinkhorn_with_grads_unrolled(Tensor log_alpha, Tensor grad_P, float tau, int n_iters, Tensor? log_a=None, Tensor? log_b=None) -> Tensor[]",
    "sinkhorn_with_grads_implicit": "dot::sinkhorn_with_grads_implicit(Tensor log_alpha, Tensor grad_P, float tau, int n_iters, int backward_iters, Tensor? log_a=None, Tensor? log_b=None) -> Tensor[]",
    "bidirectional_softmax": "dot::bidirectional_softmax(Tensor sim, float tau, Tensor lengths) -> Tensor[]",
    "bidirectional_softmax_backward": "dot::bidirectional_softmax_backward(Tensor sim, Tensor output, Tensor grad_output, Tensor row_softmax, Tensor col_softmax, float tau, Tensor lengths) -> Tensor[]",
}


def _norm(schema: str) -> str:
    return " ".join(schema.replace("0.90000000000000002", "0.9").split())


@pytest.mark.parametrize("name", sorted(REFERENCE_SCHEMAS))
def test_reference_schemas_are_registered_verbatim(name):
    op = getattr(torch.ops.dot, name)
    schema = str(op.default._schema)
    assert _norm(schema) == _norm(REFERENCE_SCHEMAS[name])
    assert getattr(_ops, name) is op


def test_drop_in_package_name():
    assert dot.sinkhorn is dot_amd.sinkhorn
    assert dot.bidirectional_softmax is dot_amd.bidirectional_softmax
    assert dot._ops.sinkhorn_dual_forward is torch.ops.dot.sinkhorn_dual_forward
    for name in ("sinkhorn", "sinkhorn_from_scores", "spectral_preflight", "SinkhornResult", "Sinkhorn",
                 "SinkhornFromScores", "bidirectional_softmax", "bidirectional_softmax_with_lengths",
                 "BidirectionalSoftmax"):
        assert hasattr(dot, name) and name in dot.__all__


def test_sinkhorn_result_fields():
    r = dot.SinkhornResult(transport_plan=torch.zeros(1))
    assert r.cost is None and r.converged is True and r.n_iters_used is None


def test_prepare_marginal_validation():  # dot/sinkhorn.py:1259-1281
    assert _prepare_marginal(None, 2, 3, "a", "cpu", torch.float32) is None
    m = _prepare_marginal(torch.tensor([0.2, 0.3, 0.5]), 2, 3, "a", "cpu", torch.float32)
    assert m.shape == (2, 3)
    with pytest.raises(ValueError, match="shape"):
        _prepare_marginal(torch.ones(4) / 4, 2, 3, "a", "cpu", torch.float32)
    with pytest.raises(ValueError, match="strictly positive"):
        _prepare_marginal(torch.tensor([0.0, 0.5, 0.5]), 2, 3, "b", "cpu", torch.float32)
    with pytest.raises(ValueError, match="sum to 1"):
        _prepare_marginal(torch.tensor([0.2, 0.2, 0.2]), 2, 3, "b", "cpu", torch.float32)


def test_max_iter_alias():
    assert _resolve_iters(20, None) == 20
    assert _resolve_iters(20, 100) == 100
    assert _resolve_iters(None, 7) == 7
    with pytest.raises(ValueError, match="not both"):
        _resolve_iters(50, 100)
    m = dot.Sinkhorn(reg=1.0, max_iter=100)  # README.md:43 spelling
    assert m.n_iters == 100
    assert dot.Sinkhorn(reg=1.0, n_iters=30).n_iters == 30


def test_validation_errors_before_any_kernel():
    C = torch.rand(2, 4, 5)
    with pytest.raises(ValueError, match="n_iters must be an int"):
        dot.sinkhorn(C, n_iters="many")
    with pytest.raises(ValueError, match="strictly positive"):
        dot.sinkhorn(C, a=torch.zeros(4))
    with pytest.raises(ValueError, match="backward_mode"):
        dot.sinkhorn(C, backward_mode="sideways")
    with pytest.raises(ValueError, match="Unsupported method"):
        dot.sinkhorn(C, method="lbfgs")
    with pytest.raises(ValueError, match="only supports n, m <= 100"):
        dot.sinkhorn(torch.rand(1, 101, 3), method="newton")
    # the reference's solver branches reject the unrolled backward (sinkhorn.py:1533-1690)
    with pytest.raises(ValueError, match="only supports implicit backward"):
        dot.sinkhorn(C, method="anderson", backward_mode="unrolled")
    with pytest.raises(ValueError, match="schedule is only supported with implicit backward"):
        dot.sinkhorn(C, schedule="cosine", backward_mode="unrolled")
    with pytest.raises(ValueError, match="spectral_preflight requires tol > 0"):
        dot.spectral_preflight(-C, 0.1, tol=0)


def test_sinkhorn_result_deferred_counts():
    """HIP results fill converged / n_iters_used on first read; the dataclass
    behaves as one with plain fields (repr, asdict, equality, copy, pickle)."""
    import copy
    import dataclasses
    import pickle

    calls = []

    def resolve():
        calls.append(1)
        return 7, True

    P = torch.rand(2, 3, 4)
    r = dot.SinkhornResult._deferred(P, P.sum((-2, -1)), resolve)
    assert calls == []
    assert r.n_iters_used == 7 and isinstance(r.n_iters_used, int)
    assert r.converged is True and calls == [1]
    assert dataclasses.asdict(r)["n_iters_used"] == 7
    assert "n_iters_used=7" in repr(r)
    r2 = pickle.loads(pickle.dumps(r))
    assert r2.n_iters_used == 7 and r2.converged is True and calls == [1]
    assert copy.copy(r).n_iters_used == 7
    # assigning one field settles the pair first, so the other keeps its value
    r3 = dot.SinkhornResult._deferred(P, None, lambda: (3, False))
    r3.converged = True
    assert r3.converged is True and r3.n_iters_used == 3
    r4 = dot.SinkhornResult._deferred(P, None, lambda: (5, True))
    assert pickle.loads(pickle.dumps(r4)).n_iters_used == 5
    # vars() never shows placeholder values: the fields are absent until resolved
    r5 = dot.SinkhornResult._deferred(P, None, lambda: (9, False))
    assert "n_iters_used" not in vars(r5) and "converged" not in vars(r5)
    assert r5.converged is False
    assert vars(r5)["n_iters_used"] == 9 and vars(r5)["converged"] is False
    r6 = dot.SinkhornResult._deferred(P, None, lambda: (4, True))
    assert copy.copy(r6).n_iters_used == 4 and r6 == dot.SinkhornResult(P, None, True, 4)


def test_anderson_ring_limit_message():
    from dot_amd.sinkhorn import MAX_ANDERSON_RING, _check_anderson_ring
    _check_anderson_ring(MAX_ANDERSON_RING, 1000)  # at the limit: accepted
    _check_anderson_ring(1000, MAX_ANDERSON_RING)  # the ring holds min(k, n_iters)
    with pytest.raises(ValueError, match="anderson_k <= 64"):
        _check_anderson_ring(MAX_ANDERSON_RING + 1, MAX_ANDERSON_RING + 1)
    assert f"#define DOT_SK_MAX_ANDERSON {MAX_ANDERSON_RING}" in open(
        __import__("os").path.join(__import__("os").path.dirname(__file__), "..", "include", "dot_amd.h")).read()
