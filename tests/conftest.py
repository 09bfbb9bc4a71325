"""Pytest configuration: the `gpu` marker and shared fixtures.

Tests marked `gpu` need an MI355X (they call the HIP layer through its C-ABI);
everything else runs on the CPU. A `gpu` test that finds no usable GPU fails
rather than skips, so a missing device can never pass as success.
"""

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP GPU (MI355X); run with -m gpu")


@pytest.fixture(scope="session")
def gpu():
    from nert_amd import device

    if not device.gpu_available():
        pytest.fail("no usable HIP device: " + (device.last_error() if device.LIB_PATH.exists() else "library not built"))
    return device
