import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built library")


def _gpu_available() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(scope="session")
def device():
    """The GPU for parity tests. A gpu-marked test fails (does not skip) when no
    GPU or no built library is there: the product path has no fallback."""
    import torch
    if not _gpu_available():
        pytest.fail("no GPU visible; gpu tests need an MI355X")
    from nanopd_amd import _lib
    _lib.load()
    return torch.device("cuda:0")
