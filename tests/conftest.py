import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and runs the HIP kernels")


@pytest.fixture(scope="session")
def gpu_ctx():
    import rns8_amd

    ctx = rns8_amd.Context()
    yield ctx
    ctx.close()


def pytest_runtest_setup(item):
    # name the case before any GPU work so a failing run says which one it was
    if item.get_closest_marker("gpu") is not None:
        print(f"\n[gpu case] {item.nodeid}", flush=True)
