"""The device executor (lancius_hip_graph.h) on the config graphs, against the
reference's golden graph outputs and the fp64 oracle executor."""
import ctypes as C
import json
from pathlib import Path

import numpy as np
import pytest

import oracle
from lancius_amd import (DEVICE_GRAPH, DEVICE_KEEP_ALL, DEVICE_NO_CHAIN, DEVICE_NO_FUSION, DeviceProgram, HipError, abi,
                         graph_lib, graphs, prng)
from tests.conftest import case, record_parity, top2_margin

pytestmark = pytest.mark.gpu

GOLD = Path(__file__).resolve().parent / "golden"
GO = np.load(GOLD / "graph_outputs.npz")
PLANS = json.loads((GOLD / "graphs.json").read_text())


class Planned:
    """Graph + schedule + fp32 plan from liblancius_graph."""

    def __init__(self, bg, plan=True):
        self.lib = graph_lib()
        self.bg = bg
        self.lib.lancius_graph_set_dtype(bg.g, abi.DTYPE_FP32)
        self.sched = self.lib.lancius_ir_schedule(bg.g)
        self.plan = self.lib.lancius_build_memory_plan(self.sched, bg.g) if plan else None
        self.lib.lancius_graph_set_dtype(bg.g, abi.DTYPE_FP64)

    def program(self, dev, flags=0, plan="own"):
        p = {"own": self.plan, "none": None}.get(plan, plan) if isinstance(plan, str) else plan
        return DeviceProgram(dev, self.bg.g, self.sched, p, flags)

    def oracle_run(self, feeds):
        keep = []
        for name in self.bg.inputs:
            arr = np.ascontiguousarray(feeds[name], dtype=np.float64)
            keep.append(arr)
            self.bg.node(name).contents.runtime_data = arr.ctypes.data_as(C.POINTER(C.c_double))
        oracle.schedule_execute(self.sched)
        out = {}
        for i in range(self.bg.g.contents.node_count):
            n = self.bg.g.contents.nodes[i]
            if n.contents.runtime_data:
                out[n.contents.id] = np.ctypeslib.as_array(n.contents.runtime_data, shape=(abi.node_elems(n),)).copy()
        oracle.release(self.bg.g)
        for name in self.bg.inputs:
            self.bg.node(name).contents.runtime_data = None
        return out

    def close(self):
        if self.plan:
            self.lib.lancius_memory_plan_destroy(self.plan)
        self.lib.lancius_schedule_destroy(self.sched)
        self.bg.destroy()


def _plan_from_fixture(rec):
    ids = len(rec["offsets"])
    offs = (C.c_size_t * ids)(*rec["offsets"])
    pooled = (C.c_uint8 * ids)(*rec["is_pooled"])
    plan = abi.MemoryPlan(rec["peak"], C.cast(offs, C.POINTER(C.c_size_t)), C.cast(pooled, C.POINTER(C.c_uint8)))
    return plan, (offs, pooled)


def _feed(prog, bg, feeds):
    for name in bg.inputs:
        prog.upload(bg.node(name), np.asarray(feeds[name], np.float32))


# ---- MLP ----------------------------------------------------------------------------


@pytest.mark.parametrize("chain", [True, False])
def test_mlp_fused_matches_reference(dev, chain):
    """Default: the whole MLP is one lancius_hip_mlp2_f32 launch; with
    DEVICE_NO_CHAIN it is GEMM+bias+ReLU, GEMM+bias, softmax."""
    pl = Planned(graphs.build_mlp(graph_lib()))
    feeds = {n: GO[f"mlp_{n}"] for n in pl.bg.inputs}
    case(f"mlp fused, chain={chain}")
    prog = pl.program(dev, flags=0 if chain else DEVICE_NO_CHAIN)
    sm = pl.bg.node("softmax")
    for _ in range(3):  # the chain's arrival counters must come back to zero
        _feed(prog, pl.bg, feeds)
        prog.run()
        got = prog.download(sm)
        assert oracle.normwise_error(got, GO["mlp_softmax"]) <= oracle.tolerance(784)
        assert np.array_equal(prog.argmax(sm), oracle.argmax(GO["mlp_softmax"]))
    record_parity(f"mlp graph 64x784x256x10 softmax, chain={chain}", oracle.normwise_error(got, GO["mlp_softmax"]),
                  oracle.tolerance(784), argmax_exact=True, top2_margin_ref=top2_margin(GO["mlp_softmax"]),
                  top2_margin_dev=top2_margin(got.reshape(64, 10)))
    info = prog.info()
    if chain:
        assert info["launches"] == 1 and info["fused_nodes"] == 7
    else:
        assert info["launches"] == 3 and info["fused_nodes"] == 5
    prog.close()
    pl.close()


def test_mlp_unfused_uses_caller_plan(dev):
    pl = Planned(graphs.build_mlp(graph_lib()))
    feeds = {n: GO[f"mlp_{n}"] for n in pl.bg.inputs}
    case("mlp unfused, caller plan")
    prog = pl.program(dev, flags=DEVICE_NO_FUSION)
    info = prog.info()
    assert info["used_caller_plan"] == 1 and info["replanned"] == 0 and info["launches"] == 8
    # buffers sit at arena + plan offset
    base = prog.buffer(pl.bg.node("mm1")) - pl.plan.contents.offsets[pl.bg.node("mm1").contents.id]
    for name in ("bc1", "add1", "relu", "mm2", "add2", "softmax"):
        n = pl.bg.node(name)
        assert prog.buffer(n) == base + pl.plan.contents.offsets[n.contents.id]
    _feed(prog, pl.bg, feeds)
    prog.run()
    assert oracle.normwise_error(prog.download(pl.bg.node("softmax")), GO["mlp_softmax"]) <= oracle.tolerance(784)
    prog.close()
    pl.close()


def test_mlp_reference_plan_is_replanned(dev):
    # The reference plan puts the second MATMUL on its live input; the
    # executor detects it and plans its own arena.
    pl = Planned(graphs.build_mlp(graph_lib()))
    plan, keep = _plan_from_fixture(PLANS["mlp"])
    case("mlp reference plan")
    prog = pl.program(dev, flags=DEVICE_NO_FUSION, plan=C.pointer(plan))
    info = prog.info()
    assert info["replanned"] == 1 and info["used_caller_plan"] == 0
    _feed(prog, pl.bg, {n: GO[f"mlp_{n}"] for n in pl.bg.inputs})
    prog.run()
    assert oracle.normwise_error(prog.download(pl.bg.node("softmax")), GO["mlp_softmax"]) <= oracle.tolerance(784)
    prog.close()
    pl.close()


@pytest.mark.parametrize("stream", ["null", "own"])
def test_graph_replay_mlp(dev, stream):
    """LANCIUS_DEVICE_GRAPH: first run eager + capture, then replays; new
    inputs are uploaded and an unrelated split-K GEMM (which grows the
    context's workspace) runs on the caller's context between replays, and
    every replay is checked against the oracle."""
    from lancius_amd import Device

    d = dev if stream == "null" else Device(0, own_stream=True)
    pl = Planned(graphs.build_mlp(graph_lib()))
    case(f"mlp graph replay, {stream} stream")
    prog = pl.program(d, flags=DEVICE_GRAPH)
    sm = pl.bg.node("softmax")
    for rep in range(4):
        feeds = {"x": prng.uniform(500 + rep, (64, 784), -1.0, 1.0),
                 "W1": prng.normal(600 + rep, (784, 256), 0, 0.05), "b1": prng.normal(700 + rep, (1, 256), 0, 0.05),
                 "W2": prng.normal(800 + rep, (256, 10), 0, 0.05), "b2": prng.normal(900 + rep, (1, 10), 0, 0.05)}
        _feed(prog, pl.bg, feeds)
        prog.run()
        got = prog.download(sm)
        ref = pl.oracle_run(feeds)[sm.contents.id].reshape(64, 10)
        assert oracle.normwise_error(got, ref) <= oracle.tolerance(784), rep
        assert np.array_equal(prog.argmax(sm), oracle.argmax(ref)), rep
        # eager work on the same context between replays
        m, k, n = 64, 1024 * (rep + 1), 128
        a, b = prng.normal(rep, (m, k)), prng.normal(rep + 50, (k, n))
        da, db, dc = d.upload(a), d.upload(b), d.alloc(m * n * 4)
        d.gemm(dc, da, db, m, k, n)
        out = d.download(dc, (m, n))
        assert oracle.normwise_error(out, oracle.matmul(a, b)) <= oracle.tolerance(k), rep
        for buf in (da, db, dc):
            buf.free()
    prog.close()
    pl.close()
    if d is not dev:
        d.close()


def test_graph_replay_block_small(dev):
    pl = Planned(graphs.build_block(graph_lib(), batch=2, S=32, d=64, H=4, F=256))
    case("block small graph replay")
    prog = pl.program(dev, flags=DEVICE_GRAPH)
    for rep in range(3):
        feeds = _block_feeds(pl.bg, seed=3000 + 100 * rep)
        _feed(prog, pl.bg, feeds)
        prog.run()
        ref = pl.oracle_run(feeds)
        for name in pl.bg.outputs:
            n = pl.bg.node(name)
            assert oracle.normwise_error(prog.download(n).ravel(), ref[n.contents.id]) <= oracle.tolerance(256), rep
    prog.close()
    pl.close()


def test_schedule_execute_device_drop_in(dev):
    lib = graph_lib()
    bg = graphs.build_mlp(lib)
    keep = []
    for name in bg.inputs:
        arr = np.ascontiguousarray(GO[f"mlp_{name}"], dtype=np.float64)
        keep.append(arr)
        bg.node(name).contents.runtime_data = arr.ctypes.data_as(C.POINTER(C.c_double))
    sched = lib.lancius_ir_schedule(bg.g)
    case("lancius_schedule_execute_device")
    rc = dev.lib.lancius_schedule_execute_device(sched, bg.g, dev.ctx)
    assert rc == 0, dev.lib.lancius_hip_last_error()
    sm = bg.node("softmax")
    got = np.ctypeslib.as_array(sm.contents.runtime_data, shape=(64 * 10,)).reshape(64, 10).copy()
    assert oracle.normwise_error(got, GO["mlp_softmax"]) <= oracle.tolerance(784)
    assert sm.contents.rt.contents.buffer_owner == 3  # LANCIUS_MEMORY_OWNED_HEAP
    import ctypes.util

    libc = C.CDLL(ctypes.util.find_library("c"))
    libc.free(C.c_void_p(C.addressof(sm.contents.runtime_data.contents)))
    sm.contents.runtime_data = None
    for name in bg.inputs:
        bg.node(name).contents.runtime_data = None
    lib.lancius_schedule_destroy(sched)
    bg.destroy()


def test_unsupported_op_fails_loudly(dev):
    lib = graph_lib()
    g = lib.lancius_graph_create()
    x = lib.lancius_input(g, 4, 4)
    n = lib.lancius_relu(g, x)
    n.contents.op = abi.OP["EMBEDDING"]  # no executor branch in the reference either
    sched = lib.lancius_ir_schedule(g)
    case("unsupported op")
    with pytest.raises(HipError) as e:
        DeviceProgram(dev, g, sched, None, 0)
    assert e.value.code == -4
    lib.lancius_schedule_destroy(sched)
    lib.lancius_graph_destroy(g)


# ---- conv -----------------------------------------------------------------------------


def test_conv_graph_small_golden(dev):
    pl = Planned(graphs.build_conv(graph_lib(), N=2, C_in=3, H=8, W=8, C_out=4))
    case("conv graph small")
    prog = pl.program(dev)
    _feed(prog, pl.bg, {"x": GO["conv_x"], "w": GO["conv_w"]})
    prog.run()
    assert oracle.normwise_error(prog.download(pl.bg.node("relu")), GO["conv_relu"]) <= oracle.tolerance(27)
    assert prog.info()["launches"] == 1
    prog.close()
    pl.close()


def test_conv_graph_config(dev):
    pl = Planned(graphs.build_conv(graph_lib()))
    x = prng.normal(45, (32, 64, 56, 56))
    w = prng.normal(145, (128, 64, 3, 3), std=float(np.sqrt(2.0 / 576)))
    case("conv graph config")
    prog = pl.program(dev)
    _feed(prog, pl.bg, {"x": x, "w": w})
    prog.run()
    got = prog.download(pl.bg.node("relu"))
    ref = oracle.conv2d(x, w, 1, 1, True, images=(0, 2))
    assert oracle.normwise_error(got[:2], ref[:2]) <= oracle.tolerance(576)
    prog.close()
    pl.close()


def test_conv_graph_repacks_changed_filter(dev):
    """The executor keeps one packed copy of a conv filter the caller
    uploads (C_in % 16 == 0); a new upload and a write through
    lancius_device_buffer must both reach the next run."""
    N, C_in, H, W, C_out = 2, 16, 12, 12, 32
    pl = Planned(graphs.build_conv(graph_lib(), N=N, C_in=C_in, H=H, W=W, C_out=C_out))
    case("conv graph, filter re-uploaded")
    prog = pl.program(dev)
    x = prng.normal(700, (N, C_in, H, W))
    prog.upload(pl.bg.node("x"), x)
    for seed, how in ((1, "upload"), (2, "upload"), (3, "buffer")):
        w = prng.normal(710 + seed, (C_out, C_in, 3, 3), std=0.1)
        if how == "upload":
            prog.upload(pl.bg.node("w"), w)
        else:
            dev.write(prog.buffer(pl.bg.node("w")), w)
        prog.run()
        got = prog.download(pl.bg.node("relu"))
        assert oracle.normwise_error(got, oracle.conv2d(x, w, 1, 1, True)) <= oracle.tolerance(9 * C_in), (seed, how)
    prog.close()
    pl.close()


def test_conv_graph_filter_pointer_kept(dev):
    """A caller that takes the filter's device address once and writes
    through it before each later run (an in-place optimizer step, say) must
    see every write reach the forward conv, whose kernel reads a packed
    copy of the filter."""
    N, C_in, H, W, C_out = 2, 16, 12, 12, 32
    pl = Planned(graphs.build_conv(graph_lib(), N=N, C_in=C_in, H=H, W=W, C_out=C_out))
    case("conv graph, filter written through a kept pointer")
    prog = pl.program(dev)
    x = prng.normal(720, (N, C_in, H, W))
    prog.upload(pl.bg.node("x"), x)
    wptr = prog.buffer(pl.bg.node("w"))
    for seed in (1, 2, 3):
        w = prng.normal(730 + seed, (C_out, C_in, 3, 3), std=0.1)
        dev.write(wptr, w)
        prog.run()
        got = prog.download(pl.bg.node("relu"))
        assert oracle.normwise_error(got, oracle.conv2d(x, w, 1, 1, True)) <= oracle.tolerance(9 * C_in), seed
    # an upload after the pointer was handed out still reaches the next run
    w = prng.normal(740, (C_out, C_in, 3, 3), std=0.1)
    prog.upload(pl.bg.node("w"), w)
    prog.run()
    got = prog.download(pl.bg.node("relu"))
    assert oracle.normwise_error(got, oracle.conv2d(x, w, 1, 1, True)) <= oracle.tolerance(9 * C_in)
    prog.close()
    pl.close()


# ---- transformer block ----------------------------------------------------------------


def _block_feeds(bg, seed=1000):
    feeds = {}
    for i, name in enumerate(bg.inputs):
        shape = abi.node_shape(bg.node(name))
        if name.startswith("x"):
            feeds[name] = prng.normal(seed + i, shape)
        elif name in ("g1", "g2"):
            feeds[name] = 1.0 + prng.normal(seed + i, shape, 0, 0.02)
        else:
            feeds[name] = prng.normal(seed + i, shape, 0, 0.02)
    return feeds


def test_block_small_golden(dev):
    pl = Planned(graphs.build_block(graph_lib(), batch=2, S=32, d=64, H=4, F=256))
    feeds = {n: GO[f"block_{n}"] for n in pl.bg.inputs}
    case("block small fused")
    prog = pl.program(dev)
    _feed(prog, pl.bg, feeds)
    prog.run()
    for name in pl.bg.outputs:
        got = prog.download(pl.bg.node(name))
        assert oracle.normwise_error(got, GO[f"block_out_{name}"]) <= oracle.tolerance(256), name
    info = prog.info()
    # LN grouped, QKV grouped (6 GEMMs), attention grouped, Wo grouped,
    # LN grouped, FFN1 grouped, FFN2 grouped
    assert info["launches"] == 7, info
    prog.close()
    pl.close()


def test_block_small_every_node(dev):
    pl = Planned(graphs.build_block(graph_lib(), batch=2, S=32, d=64, H=4, F=256))
    feeds = {n: GO[f"block_{n}"] for n in pl.bg.inputs}
    ref = pl.oracle_run(feeds)
    case("block small keep-all")
    prog = pl.program(dev, flags=DEVICE_KEEP_ALL)
    _feed(prog, pl.bg, feeds)
    prog.run()
    for i in range(pl.bg.g.contents.node_count):
        n = pl.bg.g.contents.nodes[i]
        if n.contents.op in (abi.OP["INPUT"],):
            continue
        got = prog.download(n).ravel()
        assert oracle.normwise_error(got, ref[n.contents.id]) <= oracle.tolerance(256), abi.OP_NAME[n.contents.op]
    prog.close()
    pl.close()


@pytest.mark.parametrize("noncausal", [False, True])
def test_block_config_every_sequence(dev, noncausal):
    """Full config block (B=4, S=1024, d=1024, H=16, F=4096) on the device.
    All four sequences (every member of every grouped launch) are checked
    against the fp64 oracle executor on a batch-1 graph with the same
    weights; every sink is NaN-free."""
    lib = graph_lib()
    pl = Planned(graphs.build_block(lib, noncausal=noncausal))
    feeds = _block_feeds(pl.bg)
    case(f"block config noncausal={noncausal}")
    prog = pl.program(dev)
    _feed(prog, pl.bg, feeds)
    prog.run()
    got = {name: prog.download(pl.bg.node(name)) for name in pl.bg.outputs}
    info = prog.info()
    prog.close()
    pl.close()
    assert info["launches"] == 7, info
    for name, y in got.items():
        assert np.isfinite(y).all(), name
    one = Planned(graphs.build_block(lib, batch=1, noncausal=noncausal), plan=False)
    for seq in range(4):
        f1 = {n: feeds[n] for n in one.bg.inputs if n != "x0"}
        f1["x0"] = feeds[f"x{seq}"]
        ref = one.oracle_run(f1)[one.bg.node("y0").contents.id]
        err = oracle.normwise_error(got[f"y{seq}"].ravel(), ref)
        record_parity(f"transformer block B4 S1024 d1024 H16 F4096 noncausal={noncausal}, sequence {seq}", err,
                      oracle.tolerance(4096))
        assert err <= oracle.tolerance(4096), seq
    one.close()


# ---- aliases between fused launches ------------------------------------------------


@pytest.mark.parametrize("second", ["relu", "sink_alias"])
def test_mlp_chain_not_fused_through_shared_alias(dev, second):
    """h = ReLU(x.W1 + b1) reaches the second MATMUL through a RESHAPE that a
    second node also reads (a RELU, or a RESHAPE left as a sink).  h's
    buffer is read by more than the second GEMM, so the two-layer chain must
    not be fused into one launch: every sink comes back right."""
    lib = graph_lib()
    bg = graphs.BuiltGraph(lib, lib.lancius_graph_create())
    M, K1, N1, N2 = 8, 32, 64, 10
    shapes = {"x": (M, K1), "W1": (K1, N1), "b1": (1, N1), "W2": (N1, N2), "b2": (1, N2)}
    for name, shp in shapes.items():
        bg.nodes[name] = lib.lancius_input(bg.g, *shp)
        bg.inputs.append(name)
    n = bg.nodes
    a1 = lib.lancius_add(bg.g, lib.lancius_matmul(bg.g, n["x"], n["W1"]), lib.lancius_broadcast(bg.g, n["b1"], M, N1))
    h = lib.lancius_relu(bg.g, a1)
    hr = lib.lancius_reshape(bg.g, h, 2, M, N1, 0, 0)
    a2 = lib.lancius_add(bg.g, lib.lancius_matmul(bg.g, hr, n["W2"]), lib.lancius_broadcast(bg.g, n["b2"], M, N2))
    sm = lib.lancius_softmax(bg.g, a2)
    other = lib.lancius_relu(bg.g, hr) if second == "relu" else lib.lancius_reshape(bg.g, hr, 2, M, N1, 0, 0)
    n.update(softmax=sm, other=other)
    bg.outputs = ["softmax", "other"]
    pl = Planned(bg)
    feeds = {"x": prng.uniform(71, (M, K1), -1.0, 1.0), "W1": prng.normal(72, (K1, N1), 0, 0.2),
             "b1": prng.normal(73, (1, N1), 0, 0.2), "W2": prng.normal(74, (N1, N2), 0, 0.2),
             "b2": prng.normal(75, (1, N2), 0, 0.2)}
    case(f"mlp chain with a shared alias of h, second reader {second}")
    prog = pl.program(dev)
    _feed(prog, pl.bg, feeds)
    prog.run()
    hid = oracle.relu(oracle.matmul(feeds["x"], feeds["W1"]) + feeds["b1"].astype(np.float64))
    ref_sm = oracle.softmax(oracle.matmul(hid, feeds["W2"]) + feeds["b2"].astype(np.float64))
    assert oracle.normwise_error(prog.download(sm).reshape(M, N2), ref_sm) <= oracle.tolerance(K1)
    assert oracle.normwise_error(prog.download(other).reshape(M, N1), hid) <= oracle.tolerance(K1)
    assert prog.info()["launches"] >= 2
    prog.close()
    pl.close()
