"""Shared test setup.

Markers: `gpu` — needs an MI355X (run with -m gpu).  Everything else runs on a
CPU-only machine.  GPU tests do not skip when the device is missing or broken:
the `device` fixture fails them with the library's own reason, so a GPU run
can never pass without the native kernels having run.
"""

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT / "triton-metal_amd"))
sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a usable gfx950 device (run with -m gpu)")


@pytest.fixture(scope="session")
def core():
    from triton_metal import _core
    return _core


@pytest.fixture(scope="session")
def device(core):
    """The GPU tests' gate: the device must have passed the library's probe."""
    if not core.is_usable():
        pytest.fail("no usable gfx950 device: " + str(core.unusable_reason()))
    return core.device_name()


@pytest.fixture(autouse=True)
def _announce(request):
    """Name each test before it runs, so a run that dies mid-test says which."""
    if request.node.get_closest_marker("gpu"):
        print(f"\n[gpu-test] {request.node.nodeid}", flush=True)
    yield
