import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (run with -m gpu on the GPU box)")
    config.addinivalue_line("markers", "slow: long-running CPU test")


@pytest.fixture(scope="session")
def lib():
    from spinnv2_amd.runtime import load_library

    return load_library()


@pytest.fixture(scope="session")
def gpu(lib):
    """The GPU runtime; GPU tests fail loudly (never silently fall back) when
    the library or the device is missing."""
    from spinnv2_amd.runtime import device_available

    assert device_available(), "no HIP device visible to libspkv2_mi355x.so"
    return lib
