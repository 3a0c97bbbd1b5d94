import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


# The runtime's environment switches (SHK_HIP_CONCURRENT=0, SHK_HIP_GRAPHS=0, SHK_HIP_FOLD_FINISH=0)
# turn off features whose defaults some tests assert; those tests skip under them, the rest run
# unchanged.
TWO_STREAMS_OFF = os.environ.get("SHK_HIP_CONCURRENT", "")[:1] == "0"
GRAPHS_OFF = os.environ.get("SHK_HIP_GRAPHS", "")[:1] == "0"
needs_two_streams = pytest.mark.skipif(TWO_STREAMS_OFF, reason="SHK_HIP_CONCURRENT=0 turns the "
                                                                "two-stream schedule off")
needs_graph_default = pytest.mark.skipif(GRAPHS_OFF, reason="SHK_HIP_GRAPHS=0 turns the graph "
                                                             "default off")
FOLD_OFF = os.environ.get("SHK_HIP_FOLD_FINISH", "")[:1] == "0"
needs_fold = pytest.mark.skipif(FOLD_OFF, reason="SHK_HIP_FOLD_FINISH=0 keeps every step a launch "
                                                 "of its own")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and libsynaptik_hip.so")


@pytest.fixture(scope="session")
def ctx():
    """One HIP context for the whole GPU session (one process per GPU)."""
    from synaptik_amd.native import HipContext
    c = HipContext(0)
    yield c
    c.close()
