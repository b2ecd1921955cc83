import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
for p in (REPO / "torque-mlx_amd", REPO):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X); runs through libtorque_hip.so")


@pytest.fixture(scope="session")
def hip_device():
    """The HIP device; fails (does not skip) when the library or GPU is missing."""
    import torch

    import torque_hip

    torque_hip._lib.load()
    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    return torch.device("cuda", 0)
