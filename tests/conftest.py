import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through liblancius_hip on the device)")


@pytest.fixture(scope="session")
def dev():
    """The lancius_hip context on GPU 0.  A GPU test on a machine without a
    GPU fails here (the product path has no CPU fallback)."""
    from lancius_amd import Device, device_count

    n = device_count()
    assert n >= 1, "no GPU visible to HIP: gpu tests need an MI355X"
    d = Device(0)
    yield d
    d.close()


@pytest.fixture(scope="session")
def glib():
    from lancius_amd import graph_lib

    return graph_lib()


def case(msg: str) -> None:
    """Print and flush the name of the case about to touch the GPU."""
    sys.stdout.write(f"[case] {msg}\n")
    sys.stdout.flush()
