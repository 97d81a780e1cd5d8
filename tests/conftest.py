import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture(scope="session")
def gpu():
    """The GPU device; skips when this machine has none (the CPU container).
    On a GPU machine a missing library is an error, not a skip."""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU on this machine")
    from gfx950_gluon_tutorials_amd import _lib

    _lib.load()  # raises if the HIP library is not built
    return torch.device("cuda:0")
