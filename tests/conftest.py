import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


@pytest.fixture(scope="session")
def oracle():
    from oracle import oracle as O
    O.build()
    return O


@pytest.fixture(scope="session")
def hip():
    """The hi-rocm library on a real GPU; fails (does not skip) without one."""
    import torch
    from hi_amd import _lib
    assert torch.cuda.is_available(), "GPU test run without a GPU"
    _lib.load()
    return _lib
