import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the HIP library)")


@pytest.fixture(scope="session")
def gpu():
    """Initialises device 0 through the C ABI.  On a GPU run a missing device
    or library is an error, never a skip."""
    from pegaflow_amd import runtime

    runtime.init(0)
    return runtime
