"""Shared test helpers (paths, fixtures, error metrics)."""
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "dracomancer-llmengine_amd")
GOLDEN = os.path.join(ROOT, "tests", "golden")
for _p in (PKG, ROOT, GOLDEN):
    if _p not in sys.path:
        sys.path.insert(0, _p)


def golden(name):
    path = os.path.join(GOLDEN, name)
    if not os.path.exists(path):
        pytest.fail(f"golden fixture {name} missing (tests/golden/gen_golden.py writes it)")
    return np.load(path, allow_pickle=False)


def rel_err(a, b):
    """Normwise relative error max|a-b| / max|b| (floored at 1e-30)."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30))


def bits_equal(a, b):
    a = np.ascontiguousarray(a)
    b = np.ascontiguousarray(b)
    return a.shape == b.shape and a.dtype == b.dtype and a.tobytes() == b.tobytes()
