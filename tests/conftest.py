import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))

# A persistent decode launch whose hand-off times out raises instead of
# falling back to the per-phase kernels, so that a broken hand-off fails the
# test that caused it (the fallback has its own test).
os.environ.setdefault("MG_PERSIST_STRICT", "1")

# Logit tolerance |gpu - oracle| <= TOL * (1 + |oracle|): the north-star bound,
# five times tighter than the reference's own GPU check (src/bin/mesh-gpt.rs:357-366).
TOL = 1e-4


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (run with -m gpu)")


def pytest_collection_modifyitems(config, items):
    # GPU tests run where a GPU exists; on a machine without /dev/kfd they are
    # skipped with a reason rather than silently passing.
    if os.path.exists("/dev/kfd"):
        return
    skip = pytest.mark.skip(reason="no AMD GPU on this machine (/dev/kfd absent)")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


def assert_close(actual, expected, tol=TOL, what="values"):
    actual = np.asarray(actual, dtype=np.float64)
    expected = np.asarray(expected, dtype=np.float64)
    assert actual.shape == expected.shape, f"{what}: shape {actual.shape} vs {expected.shape}"
    bound = tol * (1.0 + np.abs(expected))
    err = np.abs(actual - expected)
    bad = ~(err <= bound)
    if bad.any():
        i = np.unravel_index(np.argmax(np.where(bad, err / bound, 0)), err.shape)
        raise AssertionError(f"{what}: {bad.sum()} of {err.size} outside {tol}*(1+|ref|); worst at {i}: "
                             f"got {actual[i]!r}, expected {expected[i]!r}")
    return float((err / bound).max()) if err.size else 0.0
