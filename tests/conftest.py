import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libzenith_hip.so)")


@pytest.fixture(scope="session")
def dev():
    """cuda:0 with the HIP library loaded; skips only when no GPU exists.
    A missing or broken library is an error, not a skip."""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU in this environment")
    import zenith_amd

    zenith_amd.load_library()
    return torch.device("cuda:0")


def fp16_tol(y, ref, atol=2e-3, rtol=1e-2):
    """North-star bar for fp16 outputs vs the fp32 CPU path:
    |y - ref| <= 2e-3 + 1e-2 * |ref| elementwise. Returns (ok, worst excess)."""
    import numpy as np

    y = np.asarray(y, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    excess = np.abs(y - ref) - (atol + rtol * np.abs(ref))
    return bool(np.all(excess <= 0)), float(excess.max(initial=-1.0))
