"""pytest configuration: repo root on sys.path, the ``gpu`` marker, shared device fixtures."""
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP GPU (MI355X); runs the hand-written kernels")


@pytest.fixture(scope="session")
def built_library():
    """libpitch_amd.so, built in-tree first if no build is present (hipcc cross-compiles without a GPU)."""
    from pitch_amd import _lib
    if not _lib.LIB_PATH.exists():
        from pitch_amd.build import build
        build()
    return _lib.LIB_PATH


@pytest.fixture(scope="session")
def device():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no HIP device visible")
    return torch.device("cuda", 0)


@pytest.fixture(scope="session")
def q(device):
    """The codec on cuda:0 with the default seed (PITCH.shared in the reference's tests)."""
    import pitch_amd
    return pitch_amd.PITCH(device=device)
