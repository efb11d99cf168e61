"""Pytest configuration: the ``gpu`` marker and the repository root on sys.path."""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device) and the built library")
    config.addinivalue_line("markers", "slow: long CPU test")


def pytest_collection_modifyitems(config, items):
    """GPU tests fail loudly, never skip, when a device is present but the library is not."""
    return None


@pytest.fixture(scope="session")
def hip_device():
    import torch
    if not torch.cuda.is_available():
        if os.environ.get("EXACTSAMPLE_REQUIRE_GPU") == "1":
            raise RuntimeError("a HIP device is required")
        pytest.skip("no HIP device")
    return torch.device("cuda", 0)
