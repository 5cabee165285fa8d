import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libhses.so on the GPU)")


@pytest.fixture(scope="session")
def oracle():
    """ctypes handle of the CPU oracle (built on demand with gcc)."""
    from tests import oracle_lib
    return oracle_lib.load()


@pytest.fixture(scope="session")
def hses_gpu():
    """Initialised libhses on cuda:0; fails loudly if the library is missing."""
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU test collected without a GPU")
    from hyperscalees_amd import kernels
    kernels.init(0)
    return kernels
