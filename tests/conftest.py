import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: runs HIP kernels on an MI355X (gfx950)")


@pytest.fixture(scope="session")
def oracle():
    from oracle import pyoracle

    pyoracle.lib()
    return pyoracle


@pytest.fixture(scope="session")
def cuda():
    import torch

    if not torch.cuda.is_available():
        raise RuntimeError("GPU test selected but no HIP device is visible")
    torch.cuda.init()
    return torch.device("cuda", 0)


@pytest.fixture(scope="session")
def ncm():
    """The HIP library (raises if it was not built)."""
    import ncmorph_amd
    from ncmorph_amd import _lib

    _lib.lib()
    return ncmorph_amd
