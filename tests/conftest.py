import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) device and libmoc_amd.so")


def pytest_collection_modifyitems(config, items):
    # GPU tests print the case they are about to run, so a box that dies mid-run
    # still names it in the captured tail.
    for item in items:
        if item.get_closest_marker("gpu"):
            item.user_properties.append(("gpu", True))


@pytest.fixture(autouse=True)
def _announce_gpu_case(request):
    if request.node.get_closest_marker("gpu"):
        print(f"\n[gpu-case] {request.node.nodeid}", flush=True)
        sys.stdout.flush()
    yield
