import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


def _gpu_available() -> bool:
    try:
        import torch

        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(scope="session")
def dev():
    if not _gpu_available():
        pytest.skip("no GPU")
    import torch

    from lisa_amd import _lib

    _lib.load()  # fail loudly if the library is missing
    return torch.device("cuda:0")


@pytest.fixture(scope="session")
def oracle():
    from oracle import oracle as O

    O.build()
    return O




@pytest.fixture
def force_path():
    """force_path(name, value): select a dispatch path through the library's
    explicit override entry point for the duration of one test."""
    from lisa_amd import _lib

    used = set()

    def set_(name, value):
        used.add(name)
        _lib.set_path_override(name, value)

    yield set_
    for name in used:
        _lib.set_path_override(name, None)
