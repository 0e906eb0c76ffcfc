"""bench.py's command-line contract on a host without a GPU: more than one
GPU is refused with a message (this build measures one GPU), and a host with
no visible GPU exits with an error instead of a figure.  Neither case may
print anything on stdout, which carries only the one JSON line of a run."""
import subprocess
import sys
from pathlib import Path

import pytest

import torch

ROOT = Path(__file__).resolve().parents[1]


def _run(*args):
    return subprocess.run([sys.executable, str(ROOT / "bench.py"), *args], capture_output=True, text=True,
                          timeout=300, cwd=str(ROOT))


def test_bench_refuses_several_gpus():
    r = _run("--gpus", "2")
    assert r.returncode == 2
    assert r.stdout == ""
    assert "one GPU only" in r.stderr


@pytest.mark.skipif(torch.cuda.is_available(), reason="a GPU is visible: bench.py would measure it")
def test_bench_without_gpu_exits_with_error():
    r = _run("--steps", "1", "--warmup", "0")
    assert r.returncode == 1
    assert r.stdout == ""
    assert "no GPU visible" in r.stderr
