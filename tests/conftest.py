import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device) and the built library")


@pytest.fixture(scope="session")
def ctx():
    """A HipContext on cuda:0 (GPU tests only; fails loudly without a device)."""
    from headshot_amd.context import HipContext
    return HipContext("cuda:0")
