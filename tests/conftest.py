import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if REPO not in sys.path:
    sys.path.insert(0, REPO)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture(scope="session")
def built_library():
    """Path of liblsfa_gfx950.so, building it in-tree first if it is missing."""
    from lightserve_amd import _lib
    if not os.path.exists(_lib.library_path()):
        from lightserve_amd.csrc import build
        build.build()
    return _lib.library_path()


@pytest.fixture(scope="session")
def gpu():
    """Skips unless a GPU is present; returns the device."""
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU in this process")
    from lightserve_amd import _lib
    _lib.load()  # fail loudly (not skip) if the native library is missing
    return torch.device("cuda", 0)
