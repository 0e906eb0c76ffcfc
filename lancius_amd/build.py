"""Build the native libraries in-tree.

Products (next to this file):
  liblancius_hip.so    HIP kernels for gfx950 + the C device executor.
                       Exports only lancius_hip_*, lancius_device_*,
                       lancius_schedule_execute_device and kernel_matmul_f32.
  liblancius_graph.so  C graph IR / scheduler / planner with the reference's
                       names (a drop-in for the reference host library on the
                       graph path).

The test infrastructure (oracle/liboracle.so and, from /root/reference,
oracle/_ref/*) has its own recipe, oracle/Makefile; __graft_entry__.build()
runs both.

Usage: python -m lancius_amd.build  (or __graft_entry__.build()).
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
INCLUDE = ROOT / "include"
BUILD = PKG / "_build"

ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
HIPCC = str(ROCM / "bin" / "hipcc")
ARCH = "gfx950"

HIP_SOURCES = ["capi.hip", "gemm.hip", "attention.hip", "conv.hip", "rowops.hip", "reduce.hip", "pool.hip",
               "int8.hip", "io.hip", "chain.hip", "probe.hip", "basis.hip"]
HOST_C_SOURCES = ["host/graph_ir.c", "host/graph_plan.c", "host/graph_autodiff.c", "host/graph_io.c",
                  "host/basis_graph.c"]
DEVICE_C_SOURCES = ["host/device_exec.c", "host/basis_exec.c"]

HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-fvisibility=hidden",
    # Packed fp32 VALU instructions stay off: some of their forms have given
    # wrong results on these machines without any error.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]
C_FLAGS = ["-O2", "-std=gnu11", "-fPIC", "-Wall", "-Wextra", "-Wno-unused-parameter", f"-I{INCLUDE}"]

def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(
        line for line in proc.stdout.splitlines() if "packed-fp32-ops" not in line
    )  # hipcc's host pass does not know the GPU-only feature flag
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    if out.strip():
        sys.stderr.write(out + "\n")


def _compile_jobs(jobs: list[list[str]], workers: int) -> None:
    with cf.ThreadPoolExecutor(max_workers=workers) as ex:
        for fut in [ex.submit(_run, j) for j in jobs]:
            fut.result()


def build_hip(workers: int = 8) -> Path:
    BUILD.mkdir(exist_ok=True)
    jobs, objs = [], []
    for src in HIP_SOURCES:
        obj = BUILD / (Path(src).stem + ".hip.o")
        jobs.append([HIPCC, *HIP_FLAGS, "-c", str(CSRC / src), "-o", str(obj)])
        objs.append(obj)
    # The device executor only reads the graph structs, so the device library
    # works with graphs built by either host library.
    for src in DEVICE_C_SOURCES:
        obj = BUILD / (Path(src).stem + ".dev.o")
        jobs.append(["gcc", *C_FLAGS, "-fvisibility=hidden", "-c", str(CSRC / src), "-o", str(obj)])
        objs.append(obj)
    _compile_jobs(jobs, workers)
    out = PKG / "liblancius_hip.so"
    tmp = out.with_suffix(".so.tmp")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs),
          f"-Wl,-rpath,{ROCM / 'lib'}", "-Wl,--no-undefined"])
    os.replace(tmp, out)
    return out


def build_graph() -> Path:
    out = PKG / "liblancius_graph.so"
    tmp = out.with_suffix(".so.tmp")
    _run(["gcc", *C_FLAGS, "-shared", "-o", str(tmp), *[str(CSRC / s) for s in HOST_C_SOURCES],
          "-lm", "-pthread", "-Wl,--no-undefined"])
    os.replace(tmp, out)
    return out


def build_all(verbose: bool = True) -> dict[str, Path | None]:
    if shutil.which("gcc") is None:
        raise RuntimeError("gcc not found")
    if not Path(HIPCC).exists():
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    with cf.ThreadPoolExecutor(max_workers=2) as ex:
        f_hip = ex.submit(build_hip)
        f_graph = ex.submit(build_graph)
        res = {"liblancius_hip": f_hip.result(), "liblancius_graph": f_graph.result()}
    if verbose:
        for k, v in res.items():
            print(f"[build] {k}: {v}")
    return res


if __name__ == "__main__":
    build_all()
