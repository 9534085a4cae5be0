import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libprichs_hip.so)")


@pytest.fixture(scope="session")
def orc():
    """The CPU oracle (test infrastructure), built on first use."""
    from oracle import oracle as O

    O.build()
    return O


@pytest.fixture(scope="session")
def cuda():
    """Device handle for GPU tests; fails loudly when no GPU is visible."""
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test selected but no HIP device is visible")
    from prichs_amd import _lib

    _lib.load()
    return torch.device("cuda")


def rel_err(a, b) -> float:
    """max |a - b| / max |b| (0 when both are zero)."""
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    den = np.abs(b).max() if b.size else 0.0
    num = np.abs(a - b).max() if a.size else 0.0
    return float(num / den) if den > 0 else float(num)


def row_rel_err(a, b):
    """Per-row bar: max over rows r of max |a[r] - b[r]| / max |b[r]| (rows whose
    reference is all zero count their absolute error).  Returns (worst error,
    worst row), so a wrong result confined to a few small-magnitude rows
    cannot hide under the magnitude of the others."""
    a = np.asarray(a, dtype=np.float64).reshape(len(a), -1)
    b = np.asarray(b, dtype=np.float64).reshape(len(b), -1)
    if a.size == 0:
        return 0.0, -1
    num = np.abs(a - b).max(axis=1)
    den = np.abs(b).max(axis=1)
    err = np.where(den > 0, num / np.where(den > 0, den, 1.0), num)
    r = int(np.argmax(err))
    return float(err[r]), r
