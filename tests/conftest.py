"""Shared test setup.

Markers:
  gpu — needs a HIP device; these are the parity tests of the HIP kernels
        against the CPU oracle and the golden fixtures.

CPU tests cover the oracle against the golden fixtures and independent
closed forms, the host-side logic of the package, and the C ABI library's
symbols and argument checks.
"""

import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)
GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X); runs the HIP kernels")


def pytest_collection_modifyitems(config, items):
    import torch

    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no HIP device in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


def load_golden(name):
    with np.load(os.path.join(GOLDEN, name + ".npz"), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def rel_err(actual, expected):
    """Norm-wise relative error max|a - e| / max|e| (elementwise relative error is
    meaningless for entries like exp(-50))."""
    a = np.asarray(actual.detach().cpu() if hasattr(actual, "detach") else actual, dtype=np.float64)
    e = np.asarray(expected.detach().cpu() if hasattr(expected, "detach") else expected,
                   dtype=np.float64)
    assert a.shape == e.shape, (a.shape, e.shape)
    scale = np.abs(e).max() if e.size else 0.0
    if scale == 0.0:
        return float(np.abs(a).max()) if a.size else 0.0
    return float(np.abs(a - e).max() / scale)


def sum_err(actual, expected, terms):
    """Error of a reduction judged against the magnitude of its terms: for
    grad_tau = -sum(grad * log_alpha) / tau the result can be orders of
    magnitude smaller than the terms it cancels, so max|a - e| is divided by
    sum|terms| per batch element instead of |e|."""
    a = np.asarray(actual.detach().cpu() if hasattr(actual, "detach") else actual, dtype=np.float64)
    e = np.asarray(expected.detach().cpu() if hasattr(expected, "detach") else expected,
                   dtype=np.float64)
    t = np.asarray(terms.detach().cpu() if hasattr(terms, "detach") else terms, dtype=np.float64)
    scale = np.abs(t).reshape(t.shape[0], -1).sum(axis=1)
    return float((np.abs(a - e) / np.maximum(scale, 1e-30)).max())


@pytest.fixture
def golden():
    return load_golden
