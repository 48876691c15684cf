import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the HIP C ABI)")


@pytest.fixture(scope="session")
def hip():
    """The hip device, set current; the test fails loudly if the native library is missing."""
    from lumen_amd import native

    if native.device_count() < 1:
        pytest.fail("no HIP device visible to a gpu-marked test")
    native.set_device(0)
    return "hip:0"
