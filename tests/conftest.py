import pathlib
import sys

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X); runs the product kernels")
    config.addinivalue_line("markers", "slow: CPU oracle checks at full workload sizes")


@pytest.fixture(scope="session")
def gpu():
    """The HIP device; a GPU test fails (never skips) without one."""
    import torch
    assert torch.cuda.is_available(), "GPU test run without a HIP device"
    from polyhedral_amd import _lib
    _lib.lib()
    return torch.device("cuda", 0)
