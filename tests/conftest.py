import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and libinvision_hip.so")


@pytest.fixture(scope="session")
def hiplib():
    """The native library, initialised on device 0.  GPU tests only."""
    from invision_amd import hip, quicknn_hip

    lib = hip.load()  # raises HipLibraryError if the .so is missing: no fallback
    print(f"[gpu] {quicknn_hip.device_info()}", flush=True)
    yield lib
    quicknn_hip.shutdown()


def pytest_runtest_setup(item):
    if "gpu" in item.keywords:
        print(f"\n[gpu-test] {item.nodeid}", flush=True)
