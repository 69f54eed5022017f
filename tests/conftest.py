import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
for p in (REPO, REPO / "qwen3.5-0.8b_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libqwen35.so)")


@pytest.fixture(scope="session")
def oracle_weights():
    import torch
    from oracle.weights import WeightDict
    torch.set_grad_enabled(False)
    return WeightDict(0)


@pytest.fixture(scope="session")
def golden():
    import numpy as np
    d = REPO / "tests" / "golden"
    return {n: np.load(d / f"{n}.npz") for n in ("config0_greedy", "config0_chunk_prefill", "config0_online", "mtp_k2")}


@pytest.fixture(scope="session", autouse=True)
def _torch_hip_first():
    """Initialise torch's HIP runtime before any test loads libqwen35.so: the tests use torch
    for device buffers, and a process whose first HIP user was the library can leave torch
    without a device."""
    try:
        import torch
        if torch.cuda.is_available():
            torch.zeros(1, device="cuda")
    except ImportError:
        pass
    yield
