"""The drop-in claim on the GPU: graphs that the reference's own library
builds, schedules and memory-plans (oracle/_ref/liblancius_ref.so, compiled
from the reference sources by oracle/Makefile) run through the device
executor unchanged.

Builders: bleeding/v11A1/src/ir/lancius_ir.c; schedule:
src/runtime/lancius_scheduler.c:12-59; plan:
src/runtime/lancius_memory_planner.c:33-182; fusion pass:
src/compiler/lancius_optimizer.c:15-41; autodiff: src/math/lancius_autodiff.c:44-207.
The device side is liblancius_hip (lancius_device_program_create and
lancius_schedule_execute_device, the counterpart of lancius_schedule_execute,
lancius_scheduler.c:311-362).  Outputs are compared with the reference's own
CPU runs of the same graphs (tests/golden/graph_outputs.npz,
train_outputs.npz).  The reference plan puts a tensor on a live one (its
offset-0 free-block defect), which the executor detects and replans around.
The reference library is loaded only as the caller of the boundary, never
for anything this repository's product computes.
"""
import ctypes as C
import ctypes.util
import os
import subprocess
from pathlib import Path

import numpy as np
import pytest

import oracle
from lancius_amd import DeviceProgram, abi, graphs
from tests.conftest import case
from tests.golden.make_golden import TRAIN_GRAPHS, TRAIN_SEEDS, train_feeds

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parents[1]
GOLD = Path(__file__).resolve().parent / "golden"
GO = np.load(GOLD / "graph_outputs.npz")
T = np.load(GOLD / "train_outputs.npz")
DROP_IN = ROOT / "oracle" / "_ref" / "drop_in"


def _ref():
    ref = oracle.ref_lib()
    assert ref is not None, "oracle/_ref/liblancius_ref.so is not built (build() compiles it from /root/reference)"
    return ref


def _schedule_and_plan(ref, g):
    """The reference's schedule and its fp32 plan (the planner sizes blocks by
    dtype, lancius_ir.h:75-78), dtype restored to fp64 afterwards."""
    abi.set_graph_dtype(g, abi.DTYPE_FP32)
    sched = ref.lancius_ir_schedule(g)
    plan = ref.lancius_build_memory_plan(sched, g)
    abi.set_graph_dtype(g, abi.DTYPE_FP64)
    assert sched and plan
    return sched, plan


def _run_program(dev, ref, bg, feeds, outputs):
    sched, plan = _schedule_and_plan(ref, bg.g)
    prog = DeviceProgram(dev, bg.g, sched, plan, 0)
    for name in bg.inputs:
        prog.upload(bg.node(name), np.asarray(feeds[name], np.float32))
    prog.run()
    got = {o: prog.download(bg.node(o)).reshape(abi.node_shape(bg.node(o))) for o in outputs}
    info = prog.info()
    am = prog.argmax(bg.node(outputs[0])) if bg.node(outputs[0]).contents.op == abi.OP["SOFTMAX"] else None
    prog.close()
    ref.lancius_memory_plan_destroy(plan)
    ref.lancius_schedule_destroy(sched)
    return got, info, am


def test_ref_mlp_graph(dev):
    ref = _ref()
    bg = graphs.build_mlp(ref)
    case("reference-built MLP graph")
    got, info, am = _run_program(dev, ref, bg, {n: GO[f"mlp_{n}"] for n in bg.inputs}, ["softmax"])
    assert oracle.normwise_error(got["softmax"], GO["mlp_softmax"]) <= oracle.tolerance(784)
    assert np.array_equal(am, oracle.argmax(GO["mlp_softmax"]))
    assert info["used_caller_plan"] + info["replanned"] == 1
    bg.destroy()


def test_ref_conv_graph_fused_by_reference_pass(dev):
    ref = _ref()
    bg = graphs.build_conv(ref, N=2, C_in=3, H=8, W=8, C_out=4)  # runs the reference's lancius_optimize_fusion
    ops = [bg.g.contents.nodes[i].contents.op for i in range(bg.g.contents.node_count)]
    assert abi.OP["CONV2D_RELU_FUSED"] in ops and abi.OP["NOP"] in ops
    case("reference-built conv graph")
    got, info, _ = _run_program(dev, ref, bg, {"x": GO["conv_x"], "w": GO["conv_w"]}, ["relu"])
    assert oracle.normwise_error(got["relu"], GO["conv_relu"]) <= oracle.tolerance(27)
    assert info["launches"] == 1
    bg.destroy()


def test_ref_block_graph(dev):
    ref = _ref()
    bg = graphs.build_block(ref, batch=2, S=32, d=64, H=4, F=256)
    case("reference-built transformer block graph")
    got, info, _ = _run_program(dev, ref, bg, {n: GO[f"block_{n}"] for n in bg.inputs}, list(bg.outputs))
    for name in bg.outputs:
        assert oracle.normwise_error(got[name], GO[f"block_out_{name}"]) <= oracle.tolerance(256), name
    # one grouped launch per wave: LN, QKV, attention, Wo, LN, FFN1, FFN2
    assert info["launches"] == 7, info
    bg.destroy()


TRAIN_K = {"mlp": 784, "cnn_fused": 4 * 32 * 32}


@pytest.mark.parametrize("name", sorted(TRAIN_K))
def test_ref_autodiff_training_graph(dev, name):
    """lancius_ir_autodiff of the reference library over its own forward
    graph: the loss and every input gradient on the device."""
    ref = _ref()
    t = graphs.build_training(ref, TRAIN_GRAPHS[name](ref))
    feeds = train_feeds(t, TRAIN_SEEDS[name])
    case(f"reference-built training graph {name}")
    got, info, _ = _run_program(dev, ref, t, feeds, list(t.outputs))
    stored = "cnn" if name == "cnn_fused" else name
    for out in t.outputs:
        err = oracle.normwise_error(got[out], T[f"{stored}_out_{out}"])
        assert err <= oracle.tolerance(TRAIN_K[name]), (name, out, err)
    t.destroy()


def test_ref_schedule_execute_device(dev):
    """The one-call drop-in on a reference-built, reference-scheduled graph
    with the reference's plan attached to the schedule
    (lancius_schedule_attach_pool, lancius_scheduler.c:416-420): fp64 inputs
    in runtime_data, the sink's runtime_data holds the result afterwards."""
    ref = _ref()
    bg = graphs.build_mlp(ref)
    keep = []
    for name in bg.inputs:
        arr = np.ascontiguousarray(GO[f"mlp_{name}"], dtype=np.float64)
        keep.append(arr)
        bg.node(name).contents.runtime_data = arr.ctypes.data_as(C.POINTER(C.c_double))
    sched, plan = _schedule_and_plan(ref, bg.g)
    ref.lancius_schedule_attach_pool(sched, None, plan)
    case("lancius_schedule_execute_device on a reference schedule")
    rc = dev.lib.lancius_schedule_execute_device(sched, bg.g, dev.ctx)
    assert rc == 0, dev.lib.lancius_hip_last_error()
    sm = bg.node("softmax")
    got = np.ctypeslib.as_array(sm.contents.runtime_data, shape=(64 * 10,)).reshape(64, 10).copy()
    assert oracle.normwise_error(got, GO["mlp_softmax"]) <= oracle.tolerance(784)
    libc = C.CDLL(ctypes.util.find_library("c"))
    libc.free(C.c_void_p(C.addressof(sm.contents.runtime_data.contents)))
    sm.contents.runtime_data = None
    for name in bg.inputs:
        bg.node(name).contents.runtime_data = None
    ref.lancius_schedule_attach_pool(sched, None, None)
    ref.lancius_memory_plan_destroy(plan)
    ref.lancius_schedule_destroy(sched)
    bg.destroy()


def test_drop_in_c_program(dev):
    """tests/integration/drop_in.c, the C program INTEGRATION.md section 2
    describes, compiled by oracle/Makefile against the reference headers and
    linked with the reference library and liblancius_hip.so: it builds the
    MLP, conv and block graphs with the reference builders, runs each on the
    reference's CPU executor and through lancius_schedule_execute_device,
    and exits 0 only when every sink agrees within the tolerance."""
    assert DROP_IN.exists(), "oracle/_ref/drop_in is not built (build() compiles it where /root/reference exists)"
    case("drop_in C program")
    env = dict(os.environ)
    env.setdefault("OMP_NUM_THREADS", "16")
    proc = subprocess.run([str(DROP_IN)], stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, timeout=100,
                          env=env)
    print(proc.stdout)
    assert proc.returncode == 0, proc.stdout
    assert proc.stdout.count("ok ") == 3, proc.stdout
