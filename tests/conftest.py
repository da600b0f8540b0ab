import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X); runs the C-ABI kernels")


@pytest.fixture(scope="session")
def gpu():
    """The HIP device used by the gpu tests; fails loudly when none is visible."""
    import torch

    if not torch.cuda.is_available():
        pytest.fail("gpu test run without a visible HIP device")
    from mentat_amd._lib import get_lib

    get_lib()  # raises if libmentat_hip.so is missing
    return torch.device("cuda", 0)
