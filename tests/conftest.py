import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


@pytest.fixture(scope="session")
def device():
    """The GPU for `-m gpu` tests.  A missing GPU or library is a failure, not a skip."""
    import torch

    from flicker_amd import _lib

    assert torch.cuda.is_available(), "gpu-marked test run without a visible GPU"
    _lib.lib()  # raises HipLibraryMissing if the HIP library was not built
    return torch.device("cuda:0")
