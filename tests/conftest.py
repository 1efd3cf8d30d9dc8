import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libsharplight_hip on cuda:0)")


@pytest.fixture(scope="session")
def device():
    """The HIP device the gpu tests run on. Fails (never skips) when no device is usable: a gpu test
    that cannot reach the GPU must not pass quietly."""
    from sharplight_amd import native
    n = native.device_count()
    if n < 1:
        pytest.fail("no HIP device visible to libsharplight_hip")
    native.set_device(0)
    return native.device_props(0)
