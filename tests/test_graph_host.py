"""The C host library (liblancius_graph): scheduler, planner and fusion pass
against the reference's own outputs (tests/golden/graphs.json, written by the
compiled reference) and against an independent model of the algorithm."""
import json
from pathlib import Path

import pytest

from lancius_amd import abi, graph_lib, graphs
from tests import graph_model

GOLD = json.loads((Path(__file__).resolve().parent / "golden" / "graphs.json").read_text())

BUILDERS = {
    "mlp": (lambda lib: graphs.build_mlp(lib), abi.DTYPE_FP32),
    "conv": (lambda lib: graphs.build_conv(lib), abi.DTYPE_FP32),
    "block": (lambda lib: graphs.build_block(lib), abi.DTYPE_FP32),
    "block_small": (lambda lib: graphs.build_block(lib, batch=2, S=32, d=64, H=4, F=256), abi.DTYPE_FP32),
    "relu_chain": (lambda lib: graphs.build_relu_chain(lib), abi.DTYPE_FP64),
    # autodiff training graphs (liblancius_graph's lancius_ir_autodiff)
    "train_mlp": (lambda lib: graphs.build_training(lib, graphs.build_mlp_ce(lib)), abi.DTYPE_FP32),
    "train_cnn": (lambda lib: graphs.build_training(lib, graphs.build_cnn_ce(lib, batch=4)), abi.DTYPE_FP32),
    "train_cnn_fused": (lambda lib: graphs.build_training(lib, graphs.build_cnn_ce(lib, batch=4, fuse=True)),
                        abi.DTYPE_FP32),
    "train_gradcheck": (lambda lib: graphs.build_training(lib, graphs.build_gradcheck(lib)), abi.DTYPE_FP32),
    "train_ops": (lambda lib: graphs.build_training(lib, graphs.build_ops_loss(lib)), abi.DTYPE_FP32),
}


def _graph_nodes(g):
    out = []
    for i in range(g.contents.node_count):
        n = g.contents.nodes[i].contents
        out.append((n.id, [n.inputs[j].contents.id for j in range(n.input_count)]))
    return out


@pytest.fixture(params=sorted(BUILDERS))
def built(request):
    lib = graph_lib()
    builder, dtype = BUILDERS[request.param]
    bg = builder(lib)
    lib.lancius_graph_set_dtype(bg.g, dtype)
    sched = lib.lancius_ir_schedule(bg.g)
    plan = lib.lancius_build_memory_plan(sched, bg.g)
    yield request.param, lib, bg, sched, plan
    lib.lancius_memory_plan_destroy(plan)
    lib.lancius_schedule_destroy(sched)
    bg.destroy()


def test_waves_match_reference(built):
    name, lib, bg, sched, plan = built
    assert abi.schedule_waves(sched) == GOLD[name]["waves"]
    assert lib.lancius_schedule_peak_memory(sched) == GOLD[name]["schedule_peak"]


def test_node_ops_match_reference(built):
    name, lib, bg, sched, plan = built
    ops = [bg.g.contents.nodes[i].contents.op for i in range(bg.g.contents.node_count)]
    assert ops == GOLD[name]["node_ops"]
    if "node_inputs" in GOLD[name]:  # training graphs: wiring and shapes too
        g = bg.g.contents
        assert [[g.nodes[i].contents.inputs[j].contents.id for j in range(g.nodes[i].contents.input_count)]
                for i in range(g.node_count)] == GOLD[name]["node_inputs"]
        assert [list(abi.node_shape(g.nodes[i])) for i in range(g.node_count)] == GOLD[name]["node_shapes"]
        assert bg.outputs == GOLD[name]["outputs"]


def test_model_reproduces_reference_plan(built):
    """The model with the reference's offset-0 free blocks gives the
    reference's offsets bit-for-bit: the algorithm is understood exactly."""
    name, lib, bg, sched, plan = built
    rec = GOLD[name]
    nodes = _graph_nodes(bg.g)
    peak, offs, _ = graph_model.plan(nodes, rec["node_ops"], rec["node_bytes"], rec["waves"], keep_offsets=False)
    assert peak == rec["peak"]
    for i, _ in nodes:
        if rec["is_pooled"][i]:
            assert offs[i] == rec["offsets"][i], (name, i)


def test_plan_matches_corrected_model(built):
    name, lib, bg, sched, plan = built
    rec = GOLD[name]
    nodes = _graph_nodes(bg.g)
    ids = bg.g.contents.next_id
    peak, offs, iv = graph_model.plan(nodes, rec["node_ops"], rec["node_bytes"], rec["waves"], keep_offsets=True)
    got_peak, got_offs, got_pooled = abi.plan_offsets(plan, ids)
    assert got_peak == peak
    assert got_pooled == rec["is_pooled"]
    for i, _ in nodes:
        if got_pooled[i]:
            assert got_offs[i] == offs[i], (name, i)
    assert graph_model.overlaps(iv, dict(enumerate(got_offs))) == []


def test_first_allocations_identical_to_reference(built):
    """Before the first reused block both planners take the same tail
    addresses, so every interval allocated from the tail agrees."""
    name, lib, bg, sched, plan = built
    rec = GOLD[name]
    ids = bg.g.contents.next_id
    _, got, _ = abi.plan_offsets(plan, ids)
    nodes = _graph_nodes(bg.g)
    _, _, iv = graph_model.plan(nodes, rec["node_ops"], rec["node_bytes"], rec["waves"], keep_offsets=True)
    first_free = min((t["birth"] for t in iv if any(a["death"] < t["birth"] for a in iv)), default=None)
    for t in iv:
        if first_free is None or t["birth"] < first_free:
            assert got[t["id"]] == rec["offsets"][t["id"]]


def test_reference_plan_overlaps_live_buffers():
    """Documents the reference planner defect the device executor guards
    against: in the MLP graph the second MATMUL is placed on its own live
    input (both at offset 0)."""
    rec = GOLD["mlp"]
    lib = graph_lib()
    bg = graphs.build_mlp(lib)
    nodes = _graph_nodes(bg.g)
    _, _, iv = graph_model.plan(nodes, rec["node_ops"], rec["node_bytes"], rec["waves"], keep_offsets=False)
    bad = graph_model.overlaps(iv, dict(enumerate(rec["offsets"])))
    mm2, relu = bg.node("mm2").contents.id, bg.node("relu").contents.id
    assert (relu, mm2) in bad or (mm2, relu) in bad
    bg.destroy()


def test_relu_chain_peak_16mib():
    # S9/examples/audit_memory_pool.c: 20 x ReLU on 1024^2 fp64 -> 16 MiB
    assert GOLD["relu_chain"]["peak"] == 16 * 1024 * 1024
    lib = graph_lib()
    bg = graphs.build_relu_chain(lib)
    sched = lib.lancius_ir_schedule(bg.g)
    plan = lib.lancius_build_memory_plan(sched, bg.g)
    assert plan.contents.peak_memory == 16 * 1024 * 1024
    lib.lancius_memory_plan_destroy(plan)
    lib.lancius_schedule_destroy(sched)
    bg.destroy()


def test_block_graph_shape():
    # 16 shared weights + 29 nodes per sequence, 17 waves at batch 4
    rec = GOLD["block"]
    assert len(rec["node_ops"]) == 132 and len(rec["waves"]) == 17


def test_fusion_pass():
    lib = graph_lib()
    bg = graphs.build_conv(lib, N=1, C_in=2, H=5, W=5, C_out=3)
    conv, relu = bg.node("conv").contents, bg.node("relu").contents
    assert conv.op == abi.OP["NOP"] and conv.input_count == 0
    assert relu.op == abi.OP["CONV2D_RELU_FUSED"] and relu.input_count == 2
    assert relu.inputs[0].contents.id == bg.node("x").contents.id
    assert (relu.stride, relu.pad, relu.kernel_h, relu.kernel_w) == (1, 1, 3, 3)
    assert abi.node_shape(bg.node("relu")) == (1, 3, 5, 5)
    bg.destroy()


def test_fusion_skips_shared_conv():
    lib = graph_lib()
    g = lib.lancius_graph_create()
    x = lib.lancius_input_4d(g, 1, 2, 5, 5)
    w = lib.lancius_input_4d(g, 3, 2, 3, 3)
    conv = lib.lancius_conv2d(g, x, w, 1, 1)
    r = lib.lancius_relu(g, conv)
    lib.lancius_add(g, conv, r)  # second consumer: no fusion
    lib.lancius_optimize_fusion(g)
    assert conv.contents.op == abi.OP["CONV2D"] and r.contents.op == abi.OP["RELU"]
    lib.lancius_graph_destroy(g)


def test_long_chain_waves():
    # B/examples/stress_test.c:110-141: a 10k-node chain gives 10001 waves
    lib = graph_lib()
    bg = graphs.build_relu_chain(lib, depth=10000, rows=1, cols=1)
    sched = lib.lancius_ir_schedule(bg.g)
    assert sched.contents.wave_count == 10001
    lib.lancius_schedule_destroy(sched)
    bg.destroy()


def test_cycle_stops_scheduling(capfd):
    lib = graph_lib()
    g = lib.lancius_graph_create()
    x = lib.lancius_input(g, 2, 2)
    a = lib.lancius_relu(g, x)
    b = lib.lancius_relu(g, a)
    a.contents.inputs[0] = b  # a <- b <- a
    sched = lib.lancius_ir_schedule(g)
    assert abi.schedule_waves(sched) == [[x.contents.id]]
    assert "Cycle" in capfd.readouterr().err
    lib.lancius_schedule_destroy(sched)
    lib.lancius_graph_destroy(g)


def test_builder_shape_checks():
    lib = graph_lib()
    g = lib.lancius_graph_create()
    a = lib.lancius_input(g, 3, 4)
    b = lib.lancius_input(g, 5, 2)
    assert not lib.lancius_matmul(g, a, b)
    assert lib.lancius_get_error() == -3
    x = lib.lancius_input_4d(g, 1, 3, 4, 4)
    w = lib.lancius_input_4d(g, 2, 4, 3, 3)
    assert not lib.lancius_conv2d(g, x, w, 1, 1)  # channel mismatch
    lib.lancius_graph_destroy(g)
