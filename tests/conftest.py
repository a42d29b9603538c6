import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP GPU (MI355X); parity of the HIP kernels")


def _gpu_available() -> bool:
    try:
        import torch

        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(scope="session")
def gpu():
    """cuda:0 as a torch.device; GPU tests fail loudly if the HIP library is absent."""
    if not _gpu_available():
        pytest.skip("no HIP device visible")
    import torch

    from langtrain_studio_amd import _lib

    _lib.load()  # raises if libltkv.so is missing: there is no fallback
    return torch.device("cuda", 0)
