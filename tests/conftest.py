import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (ROCm) GPU and the built HIP library")


def _gpu_available():
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


def pytest_collection_modifyitems(config, items):
    if _gpu_available():
        return
    skip = pytest.mark.skip(reason="no GPU in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def oracle():
    from oracle import oracle as module
    return module


@pytest.fixture
def dispatch():
    """Forces kernel choices of the library for one test (``vh_set_dispatch_override``,
    e.g. ``dispatch(scan_pack="2x2")``); every override is cleared when the test ends."""
    from visionhope_amd.utils import hip

    lib = hip.load_library()

    def force(**values):
        for name, value in values.items():
            hip.check(lib.vh_set_dispatch_override(name.encode(), str(value).encode()), "vh_set_dispatch_override")

    yield force
    lib.vh_clear_dispatch_overrides()


@pytest.fixture(scope="session")
def device():
    import torch
    return torch.device("cuda:0")
