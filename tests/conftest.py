import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; run with -m gpu")


@pytest.fixture(scope="session")
def orc():
    from oracle import oracle as O
    return O.get()


@pytest.fixture(scope="session")
def gpu_ready():
    """The product library on a live GPU. Fails (never skips) when absent:
    a GPU test that cannot reach the HIP path must not pass."""
    import torch
    from dianoia_amd import _lib
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a HIP device (run them on the MI355X box)")
    lib = _lib.load()
    assert lib.lab_gpu_init() == 1, "lab_gpu_init failed on a GPU box"
    return lib
