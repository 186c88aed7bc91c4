import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if REPO not in sys.path:
    sys.path.insert(0, REPO)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture(scope="session")
def dev():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test collected on a machine without a GPU (run with -m 'not gpu')")
    from sparsesnn_amd import _lib

    _lib.load()  # fail loudly when the HIP library is not built
    return torch.device("cuda:0")


@pytest.fixture
def env():
    """Set environment variables for one test (the library reads its routing switches per call);
    restored afterwards."""
    saved = {}

    def set_(k, v):
        saved.setdefault(k, os.environ.get(k))
        os.environ[k] = str(v)

    yield set_
    for k, v in saved.items():
        if v is None:
            os.environ.pop(k, None)
        else:
            os.environ[k] = v
