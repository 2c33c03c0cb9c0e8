import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parent.parent
if str(REPO) not in sys.path:
    sys.path.insert(0, str(REPO))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X / gfx950)")


@pytest.fixture(scope="session")
def gpu():
    """The ROCm device, with the native library loaded (fails loudly if it is not)."""
    import torch
    if not torch.cuda.is_available():
        pytest.fail("gpu test run without a visible ROCm device")
    from tokenfactory_amd import _native
    _native.load()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    return dev
