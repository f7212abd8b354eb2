import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the HIP backend)")


@pytest.fixture(scope="session")
def gpu():
    """Fails (not skips) when a gpu-marked test runs without a usable GPU."""
    import porch_amd as porch

    if not porch.is_available():
        pytest.fail("porch_amd: HIP backend unavailable on a GPU test run")
    return porch
