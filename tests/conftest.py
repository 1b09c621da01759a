import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU (run on the GPU box)")


@pytest.fixture(scope="session")
def ow():
    import opworks_amd

    opworks_amd.lib()
    return opworks_amd


@pytest.fixture(scope="session")
def orc():
    from tests import oracle

    oracle.lib()
    return oracle


def bits(a: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def framework_close(actual, expected, tol=1e-5):
    """The reference's unit-test criterion |a - e| <= tol * (1 + |e|) (tests/unit/framework.cu:45-48)."""
    a = np.asarray(actual, np.float64)
    e = np.asarray(expected, np.float64)
    return bool(np.all(np.isfinite(a)) and np.all(np.abs(a - e) <= tol * (1 + np.abs(e))))


def max_rel(actual, expected, floor=1e-30):
    a = np.asarray(actual, np.float64)
    e = np.asarray(expected, np.float64)
    return float(np.max(np.abs(a - e) / np.maximum(np.abs(e), floor))) if a.size else 0.0
