import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP library)")


def pytest_collection_modifyitems(config, items):
    # GPU tests print their case before running so a lost box still names it.
    for item in items:
        if item.get_closest_marker("gpu"):
            item.add_marker(pytest.mark.timeout(300))


@pytest.fixture(autouse=True)
def _announce_gpu_case(request):
    if request.node.get_closest_marker("gpu"):
        print(f"\n[gpu case] {request.node.nodeid}", flush=True)
    yield
