import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and libsynaptik_hip.so")


@pytest.fixture(scope="session")
def ctx():
    """One HIP context for the whole GPU session (one process per GPU)."""
    from synaptik_amd.native import HipContext
    c = HipContext(0)
    yield c
    c.close()
