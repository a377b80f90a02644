import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built HIP library")


def pytest_collection_modifyitems(config, items):
    # GPU tests print the case they run first, so a box that dies mid-run still
    # names it in the captured output.
    for item in items:
        if item.get_closest_marker("gpu") is not None:
            item.add_marker(pytest.mark.usefixtures("_announce_case"))


@pytest.fixture
def _announce_case(request):
    print(f"\n[case] {request.node.nodeid}", flush=True)
    sys.stdout.flush()
    yield
