import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X); run with -m gpu")


@pytest.fixture(scope="session")
def pkg():
    import __graft_entry__

    return __graft_entry__.load_package()


@pytest.fixture(scope="session")
def dev(pkg):
    import torch

    assert torch.cuda.is_available(), "GPU test run without a visible HIP device"
    pkg._lib.load()  # fail loudly if the native library is missing
    return torch.device("cuda:0")
