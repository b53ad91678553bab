import os
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built libvte_amd.so")


@pytest.fixture(scope="session")
def hip():
    """Initialised HIPRuntime on device 0.  Fails (does not skip) without a GPU:
    GPU tests are selected with -m gpu only where one is present."""
    from vte_amd.bridge import HIPRuntime
    rt = HIPRuntime()
    assert rt.initialize(), "HIP initialisation failed: no GPU visible"
    rt._prevent_host_copies = False
    yield rt
    rt.cleanup()


@pytest.fixture(scope="session")
def K():
    from vte_amd.kernels import kernels
    return kernels()


def rel_l2(a, b) -> float:
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))
