import json
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


def top2_margin(logits) -> float:
    """Smallest gap, over rows, between a row's largest and second-largest
    value: how far a first-max-wins argmax is from flipping."""
    import numpy as np

    x = np.asarray(logits, dtype=np.float64)
    x = x.reshape(-1, x.shape[-1])
    top = np.sort(x, axis=1)[:, -2:]
    return float(np.min(top[:, 1] - top[:, 0]))


def record_parity(config: str, err: float, bound: float, **extra) -> None:
    """Print one parity measurement (normwise error against its bound and
    any extra fields, e.g. top-2 margins) and, when the environment variable
    LANCIUS_PARITY_LOG names a file, append it there as a JSON line."""
    row = {"config": config, "normwise_error": float(err), "bound": float(bound),
           "fraction_of_bound": float(err) / float(bound)}
    row.update(extra)
    sys.stdout.write(f"[parity] {json.dumps(row)}\n")
    sys.stdout.flush()
    path = os.environ.get("LANCIUS_PARITY_LOG")
    if path:
        with open(path, "a") as f:
            f.write(json.dumps(row) + "\n")


def case(msg: str) -> None:
    """Print and flush the name of the case about to touch the GPU."""
    sys.stdout.write(f"[case] {msg}\n")
    sys.stdout.flush()
