import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLDEN = os.path.join(ROOT, "tests", "golden")
for p in (ROOT, GOLDEN):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built libsaga_amd.so")


def pytest_collection_modifyitems(config, items):
    try:
        import torch
        has_gpu = torch.cuda.is_available()
    except Exception:  # pragma: no cover
        has_gpu = False
    if has_gpu:
        return
    skip = pytest.mark.skip(reason="no GPU in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


def rel_l2(a, b):
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))


def set_diff_outside_band(sel_a, sel_b, x, t, band):
    """Positions selected by exactly one side whose logit is farther than
    `band` from the threshold (a near-tie may flip with rounding)."""
    a = set(int(i) for i in sel_a)
    b = set(int(i) for i in sel_b)
    return [i for i in a ^ b if abs(float(x[i]) - float(t)) > band]


@pytest.fixture
def golden():
    def load(name):
        return np.load(os.path.join(GOLDEN, "fixtures", f"{name}.npz"))
    return load
