import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if REPO not in sys.path:
    sys.path.insert(0, REPO)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built HIP library")


@pytest.fixture(scope="session")
def gpu():
    """Skip unless a GPU is present; fail loudly if the HIP library is missing."""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")
    from hrm_flashrenderer_amd import _lib

    _lib.load()  # raises if the library is not built: no silent fallback
    return torch.device("cuda", 0)
