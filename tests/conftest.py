import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU (run with -m gpu on the GPU host)")


@pytest.fixture
def announce(request):
    """Print (and flush) the case name before a GPU step, so a fault can be attributed."""

    def _say(msg=""):
        print(f"[case] {request.node.name} {msg}", flush=True)

    return _say
