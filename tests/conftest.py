import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if REPO not in sys.path:
    sys.path.insert(0, REPO)

import pyasc_amd  # noqa: E402

# Reference-style tests do `import asc, asc2` unchanged.
pyasc_amd.install_aliases()


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device) and the built libasc_hip.so")


@pytest.fixture(scope="session")
def device():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU test selected but no HIP device is visible")
    from pyasc_amd import _native
    _native.load_library()
    return torch.device("cuda", 0)
