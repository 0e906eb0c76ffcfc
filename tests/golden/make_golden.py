"""Writes the golden fixtures of tests/golden/ by running the REFERENCE's own
C code, compiled from /root/reference into oracle/_ref/liblancius_ref.so
(`python -m lancius_amd.build`).  Run in the build container only:

    python tests/golden/make_golden.py

Outputs (data only - inputs and the reference's outputs):
  kernels.npz        kernel_matmul / graph MATMUL, kernel_conv2d_fwd,
                     kernel_conv2d_relu_fwd, kernel_attention,
                     kernel_layernorm, kernel_gelu, graph SOFTMAX; graph
                     SUB, MUL, RELU_BWD, TRANSPOSE, SUM, SUM_AXIS0/1,
                     SOFTMAX_BWD, CROSS_ENTROPY(_BWD), MAXPOOL2D(_BWD) and
                     kernel_conv2d_bwd_in/_w
  graphs.json        lancius_ir_schedule waves and lancius_build_memory_plan
                     offsets/peaks of the config graphs (fp32 dtypes, as the
                     device plans them) and of the 20 x ReLU chain (fp64)
  graph_outputs.npz  sink values of reference CPU graph runs (scratch-arena
                     executor, B/src/runtime/lancius_scheduler.c:311-362)
  train_outputs.npz  loss and every input gradient of the reference's
                     autodiff training graphs (B/src/math/lancius_autodiff.c)
                     run by the same executor, for the inputs train_feeds()
                     regenerates from the seeds in TRAIN_SEEDS (the fused
                     CNN graph is checked to give the unfused graph's values
                     and is not stored twice); their structure and fp32 plans
                     go to graphs.json as train_<name>
Inputs come from lancius_amd.prng with the seeds written next to them.
"""
from __future__ import annotations

import ctypes as C
import json
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

import oracle  # noqa: E402
from lancius_amd import abi, graphs, prng  # noqa: E402

OUT = Path(__file__).resolve().parent
_D = C.POINTER(C.c_double)


def p(a):
    return a.ctypes.data_as(_D)


def f32(a):
    """fp32-representable values widened to fp64 (what the device sees)."""
    return np.ascontiguousarray(np.asarray(a, np.float32), dtype=np.float64)


def run_ref_graph(ref, bg: graphs.BuiltGraph, feeds: dict[str, np.ndarray]) -> dict[str, np.ndarray]:
    keep = []
    for name in bg.inputs:
        arr = np.ascontiguousarray(feeds[name], dtype=np.float64)
        keep.append(arr)
        bg.node(name).contents.runtime_data = p(arr)
    sched = ref.lancius_ir_schedule(bg.g)
    arena = ref.lancius_arena_create(64 << 20)
    ref.lancius_schedule_execute(sched, arena)
    out = {}
    for name in bg.outputs:
        n = bg.node(name)
        e = abi.node_elems(n)
        out[name] = np.ctypeslib.as_array(n.contents.runtime_data, shape=(e,)).copy().reshape(abi.node_shape(n))
    for name in bg.inputs:
        bg.node(name).contents.runtime_data = None
    ref.lancius_schedule_destroy(sched)
    ref.lancius_arena_destroy(arena)
    return out


def plan_record(ref, bg: graphs.BuiltGraph, dtype: int) -> dict:
    abi.set_graph_dtype(bg.g, dtype)
    sched = ref.lancius_ir_schedule(bg.g)
    plan = ref.lancius_build_memory_plan(sched, bg.g)
    ids = bg.g.contents.next_id
    peak, offsets, pooled = abi.plan_offsets(plan, ids)
    waves = abi.schedule_waves(sched)
    rec = {
        "waves": waves,
        "peak": peak,
        "offsets": offsets,
        "is_pooled": pooled,
        "schedule_peak": ref.lancius_schedule_peak_memory(sched),
        "node_ops": [bg.g.contents.nodes[i].contents.op for i in range(bg.g.contents.node_count)],
        "node_bytes": [abi.node_elems(bg.g.contents.nodes[i]) * (4 if dtype == abi.DTYPE_FP32 else 8)
                       for i in range(bg.g.contents.node_count)],
    }
    ref.lancius_memory_plan_destroy(plan)
    ref.lancius_schedule_destroy(sched)
    abi.set_graph_dtype(bg.g, abi.DTYPE_FP64)
    return rec


def main() -> None:
    ref = oracle.ref_lib()
    if ref is None:
        raise SystemExit("oracle/_ref/liblancius_ref.so not built (needs /root/reference)")
    k = {}

    # graph MATMUL (the path the scheduler runs) and kernel_matmul
    k["mm_a"], k["mm_b"] = f32(prng.normal(1, (7, 13))), f32(prng.normal(2, (13, 5)))
    out = np.zeros((7, 5))
    ref.kernel_matmul(p(out), p(k["mm_a"]), p(k["mm_b"]), 7, 13, 5)
    k["mm_kernel_out"] = out
    bg = graphs.BuiltGraph(ref, ref.lancius_graph_create())
    a = graphs._inp(bg, "a", 7, 13)
    b = graphs._inp(bg, "b", 13, 5)
    bg.nodes["mm"] = ref.lancius_matmul(bg.g, a, b)
    bg.outputs = ["mm"]
    k["mm_graph_out"] = run_ref_graph(ref, bg, {"a": k["mm_a"], "b": k["mm_b"]})["mm"]
    bg.destroy()

    # conv2d
    k["conv_x"], k["conv_w"] = f32(prng.normal(3, (2, 3, 7, 7))), f32(prng.normal(4, (5, 3, 3, 3)))
    for name, fn in (("conv_s1p1", ref.kernel_conv2d_fwd), ("conv_relu_s1p1", ref.kernel_conv2d_relu_fwd)):
        out = np.zeros((2, 5, 7, 7))
        fn(p(out), p(k["conv_x"]), p(k["conv_w"]), 2, 3, 7, 7, 5, 3, 3, 1, 1)
        k[name] = out
    k["conv_x2"], k["conv_w2"] = f32(prng.normal(5, (1, 2, 9, 8))), f32(prng.normal(6, (3, 2, 5, 5)))
    out = np.zeros((1, 3, 5, 4))
    ref.kernel_conv2d_fwd(p(out), p(k["conv_x2"]), p(k["conv_w2"]), 1, 2, 9, 8, 3, 5, 5, 2, 2)
    k["conv_s2p2"] = out

    # attention (causal, [S, H, D])
    for tag, (S, H, D), seed in (("attn", (17, 2, 8), 7), ("attn2", (64, 4, 16), 8)):
        q, kk, v = (f32(prng.uniform(seed + i, (S, H, D), -1.0, 1.0)) for i in range(3))
        out = np.zeros((S, H, D))
        ref.kernel_attention(p(out), p(q), p(kk), p(v), S, H, D)
        k[f"{tag}_q"], k[f"{tag}_k"], k[f"{tag}_v"], k[f"{tag}_out"] = q, kk, v, out

    # layernorm, gelu
    k["ln_x"] = f32(prng.normal(9, (5, 12), mean=0.3, std=2.0))
    k["ln_g"], k["ln_b"] = f32(prng.normal(10, (12,), 1.0, 0.2)), f32(prng.normal(11, (12,), 0.0, 0.2))
    out = np.zeros((5, 12))
    ref.kernel_layernorm(p(out), p(k["ln_x"]), p(k["ln_g"]), p(k["ln_b"]), 5, 12, 1e-5)
    k["ln_out"] = out
    gx = prng.normal(12, (64,), std=4.0)
    gx[:8] = [0.0, 150.0, -150.0, 100.0, -100.0, 99.5, -0.5, 3.0]
    k["gelu_x"] = f32(gx)
    out = np.zeros(64)
    ref.kernel_gelu(p(out), p(k["gelu_x"]), 64)
    k["gelu_out"] = out

    # graph SOFTMAX
    k["softmax_x"] = f32(prng.normal(13, (4, 10), std=3.0))
    bg = graphs.BuiltGraph(ref, ref.lancius_graph_create())
    a = graphs._inp(bg, "a", 4, 10)
    bg.nodes["sm"] = ref.lancius_softmax(bg.g, a)
    bg.outputs = ["sm"]
    k["softmax_out"] = run_ref_graph(ref, bg, {"a": k["softmax_x"]})["sm"]
    bg.destroy()
    training_op_vectors(ref, k)
    int8_vectors(ref, k)
    decode_vectors(ref, k)
    np.savez_compressed(OUT / "kernels.npz", **k)

    # schedules and plans
    recs = {}
    for name, builder, dtype in (
        ("mlp", lambda: graphs.build_mlp(ref), abi.DTYPE_FP32),
        ("conv", lambda: graphs.build_conv(ref), abi.DTYPE_FP32),
        ("block", lambda: graphs.build_block(ref), abi.DTYPE_FP32),
        ("block_small", lambda: graphs.build_block(ref, batch=2, S=32, d=64, H=4, F=256), abi.DTYPE_FP32),
        ("relu_chain", lambda: graphs.build_relu_chain(ref), abi.DTYPE_FP64),
    ):
        bg = builder()
        recs[name] = plan_record(ref, bg, dtype)
        bg.destroy()
    (OUT / "graphs.json").write_text(json.dumps(recs, indent=0, sort_keys=True))

    # reference CPU graph runs
    go = {}
    bg = graphs.build_mlp(ref)
    feeds = {"x": f32(prng.uniform(42, (64, 784), -1.0, 1.0)), "W1": f32(prng.normal(142, (784, 256), 0, 0.02)),
             "b1": f32(prng.normal(242, (1, 256), 0, 0.02)), "W2": f32(prng.normal(342, (256, 10), 0, 0.02)),
             "b2": f32(prng.normal(442, (1, 10), 0, 0.02))}
    res = run_ref_graph(ref, bg, feeds)
    go.update({f"mlp_{n}": v for n, v in feeds.items()})
    go["mlp_softmax"] = res["softmax"]
    bg.destroy()

    bg = graphs.build_conv(ref, N=2, C_in=3, H=8, W=8, C_out=4)
    feeds = {"x": f32(prng.normal(46, (2, 3, 8, 8))), "w": f32(prng.normal(47, (4, 3, 3, 3), 0, 0.47))}
    res = run_ref_graph(ref, bg, feeds)
    go.update({f"conv_{n}": v for n, v in feeds.items()})
    go["conv_relu"] = res["relu"]
    bg.destroy()

    bg = graphs.build_block(ref, batch=2, S=32, d=64, H=4, F=256)
    feeds = {}
    for i, name in enumerate(bg.inputs):
        shape = abi.node_shape(bg.node(name))
        if name.startswith("x"):
            feeds[name] = f32(prng.normal(1000 + i, shape))
        elif name in ("g1", "g2"):
            feeds[name] = f32(1.0 + prng.normal(1000 + i, shape, 0, 0.02))
        else:
            feeds[name] = f32(prng.normal(1000 + i, shape, 0, 0.02))
    res = run_ref_graph(ref, bg, feeds)
    go.update({f"block_{n}": v for n, v in feeds.items()})
    go.update({f"block_out_{n}": v for n, v in res.items()})
    bg.destroy()
    np.savez_compressed(OUT / "graph_outputs.npz", **go)

    # training graphs: structure and plan of the reference's autodiff graphs,
    # and loss + gradients of reference CPU runs
    tr = {}
    trec = {}
    for name, fwd in TRAIN_GRAPHS.items():
        t = graphs.build_training(ref, fwd(ref))
        trec[name] = plan_record(ref, t, abi.DTYPE_FP32)
        trec[name]["node_inputs"] = [
            [t.g.contents.nodes[i].contents.inputs[j].contents.id for j in range(t.g.contents.nodes[i].contents.input_count)]
            for i in range(t.g.contents.node_count)]
        trec[name]["node_shapes"] = [list(abi.node_shape(t.g.contents.nodes[i])) for i in range(t.g.contents.node_count)]
        trec[name]["outputs"] = list(t.outputs)
        feeds = train_feeds(t, TRAIN_SEEDS[name])
        res = run_ref_graph(ref, t, feeds)
        if name == "cnn_fused":
            # the fused graph computes the same values as the unfused one (up
            # to the order in which the reference's OpenMP threads add their
            # kernel_conv2d_bwd_w partials, lancius_kernels.c:128-131)
            for n, v in res.items():
                np.testing.assert_allclose(v, tr[f"cnn_out_{n}"], rtol=1e-9, atol=1e-12)
        else:
            tr.update({f"{name}_out_{n}": v for n, v in res.items()})
        t.destroy()
    recs.update({f"train_{k}": v for k, v in trec.items()})
    (OUT / "graphs.json").write_text(json.dumps(recs, indent=0, sort_keys=True))
    np.savez_compressed(OUT / "train_outputs.npz", **tr)
    model_vectors(ref)
    print("fixtures written to", OUT)


def _ref_graph_from_records(ref, recs: list[dict]):
    """The graph of parsed v9 records rebuilt with the reference's own
    builders, as its loader does (lancius_serialize.c:137-201) plus BROADCAST,
    which that loader skips (:175-176); weights bound as its loader binds
    them (:221-240).  Returns (graph, file id -> node, arrays to keep)."""
    I8 = C.POINTER(C.c_int8)
    g = ref.lancius_graph_create()
    by_id, keep = {}, []
    for r in recs:
        op, s, m = r["op"], r["shape"], r["meta"]
        ins = [by_id.get(i) for i in r["inputs"]]
        if op == abi.OP["INPUT"]:
            n = ref.lancius_input_4d(g, *s) if r["ndim"] == 4 else ref.lancius_input(g, s[0], s[1])
        elif op in (abi.OP["CONV2D"], abi.OP["CONV2D_RELU_FUSED"]):
            n = ref.lancius_conv2d(g, ins[0], ins[1], m[2], m[3])
            n.contents.op = op
        elif op == abi.OP["MAXPOOL2D"]:
            n = ref.lancius_maxpool2d(g, ins[0], m[0], m[2])
        elif op == abi.OP["FLATTEN"]:
            n = ref.lancius_flatten(g, ins[0])
        elif op == abi.OP["MATMUL"]:
            n = ref.lancius_matmul(g, ins[0], ins[1])
        elif op == abi.OP["ADD"]:
            n = ref.lancius_add(g, ins[0], ins[1])
        elif op == abi.OP["RELU"]:
            n = ref.lancius_relu(g, ins[0])
        elif op == abi.OP["BROADCAST"]:
            n = ref.lancius_broadcast(g, ins[0], s[0], s[1])
        elif op == abi.OP["CROSS_ENTROPY"]:
            n = ref.lancius_cross_entropy(g, ins[0], ins[1])
        elif op == abi.OP["NOP"]:
            continue
        else:
            raise ValueError(f"op {op} not rebuilt here")
        n.contents.kernel_h, n.contents.kernel_w, n.contents.stride, n.contents.pad = m
        for d in range(4):
            n.contents.axes[d] = r["axes"][d]
        by_id[r["id"]] = n
        if r["weights"] is not None:
            w = np.ascontiguousarray(r["weights"])
            keep.append(w)
            n.contents.dtype = r["dtype"]
            n.contents.scale = r["scale"]
            if r["dtype"] == abi.DTYPE_INT8:
                n.contents.runtime_data_int8 = w.ctypes.data_as(I8)
            else:
                n.contents.runtime_data = p(w)
    return g, by_id, keep


def _node_values(n) -> np.ndarray:
    return np.ctypeslib.as_array(n.contents.runtime_data, shape=(abi.node_elems(n),)).copy().reshape(
        abi.node_shape(n))


def model_vectors(ref) -> None:
    """Model-file fixtures under tests/golden/:
      models/ref_<io graph>.lancius  lancius_graph_save of the reference on
                                     graphs.build_io_graph graphs (v10 bytes)
      model_io.npz  lenet_logits: stable/v9S/pytorch_lenet.lancius, re-laid
                    as v10 by oracle.model_file, read by the reference's own
                    lancius_graph_load and run by its executor on
                    parity_input.bin (the shipped lancius_out.bin is these
                    logits in fp32 from the v9 build);
                    cifar_logits / cifar_loss: stable/v9S/cifar10_lenet.lancius
                    (int8 image and filters, BROADCAST, CROSS_ENTROPY over
                    its stored batch) rebuilt with the reference's builders
                    and run by its executor."""
    import tempfile

    from oracle import model_file as mf

    models = OUT / "models"
    for name in graphs.IO_GRAPHS:
        bg = graphs.build_io_graph(ref, name)
        ref.lancius_graph_save(bg.g, str(models / f"ref_{name}.lancius").encode())
        for i in range(bg.g.contents.node_count):  # the reference's int8 copies are left to the process
            bg.g.contents.nodes[i].contents.runtime_data = None
        bg.destroy()
    out = {}
    recs = mf.read_records((models / "pytorch_lenet.lancius").read_bytes(), 9)
    with tempfile.TemporaryDirectory() as tmp:
        path = Path(tmp) / "lenet_v10.lancius"
        path.write_bytes(mf.write_records(recs, 10))
        g = ref.lancius_graph_load(str(path).encode())
    nodes = [g.contents.nodes[i] for i in range(g.contents.node_count)]
    x_node = [n for n in nodes if n.contents.op == abi.OP["INPUT"] and n.contents.ndim == 4
              and not n.contents.runtime_data][0]  # examples/parity_runner.c:14-18
    y_node = [n for n in nodes if n.contents.ndim == 2 and n.contents.shape[1] == 10
              and n.contents.op != abi.OP["INPUT"]][-1]
    x = np.fromfile(models / "parity_input.bin", dtype="<f4").astype(np.float64)
    x_node.contents.runtime_data = p(x)
    sched = ref.lancius_ir_schedule(g)
    arena = ref.lancius_arena_create(16 << 20)
    ref.lancius_schedule_execute(sched, arena)
    out["lenet_logits"] = _node_values(y_node).ravel()
    shipped = np.fromfile(models / "lancius_out.bin", dtype="<f4")
    print("lenet logits vs shipped lancius_out.bin:", oracle.normwise_error(shipped, out["lenet_logits"]))
    x_node.contents.runtime_data = None
    ref.lancius_schedule_destroy(sched)
    ref.lancius_arena_destroy(arena)

    recs = mf.read_records((models / "cifar10_lenet.lancius").read_bytes(), 9)
    g, by_id, keep = _ref_graph_from_records(ref, recs)
    sched = ref.lancius_ir_schedule(g)
    arena = ref.lancius_arena_create(64 << 20)
    ref.lancius_schedule_execute(sched, arena)
    out["cifar_logits"] = _node_values(by_id[20])
    out["cifar_loss"] = _node_values(by_id[22]).ravel()
    print("cifar loss", out["cifar_loss"])
    ref.lancius_schedule_destroy(sched)
    ref.lancius_arena_destroy(arena)
    np.savez_compressed(OUT / "model_io.npz", **out)


def ref_op(ref, shapes: dict[str, tuple], build, feeds: dict[str, np.ndarray]) -> np.ndarray:
    """Output of one reference graph node `build(graph, inputs)` over INPUTs of
    the given shapes, run by the reference's scratch-arena executor."""
    bg = graphs.BuiltGraph(ref, ref.lancius_graph_create())
    ins = {name: graphs._inp(bg, name, *shape) for name, shape in shapes.items()}
    bg.nodes["out"] = build(bg.g, ins)
    bg.outputs = ["out"]
    out = run_ref_graph(ref, bg, feeds)["out"]
    bg.destroy()
    return out


def training_op_vectors(ref, k: dict) -> None:
    """Golden vectors of the training/reduction dispatch branches
    (lancius_scheduler.c:68-104,236-304; lancius_vision_ops.c:82-190) and of
    kernel_conv2d_bwd_in/_w (lancius_kernels.c:62-136)."""
    R, Cc = 6, 9
    a, b = f32(prng.normal(20, (R, Cc))), f32(prng.normal(21, (R, Cc)))
    a[0, :3] = [0.0, -0.0, 1e-30]  # RELU_BWD decides on fwd > 0
    k["ew_a"], k["ew_b"] = a, b
    two = {"a": (R, Cc), "b": (R, Cc)}
    feeds = {"a": a, "b": b}
    k["sub_out"] = ref_op(ref, two, lambda g, i: ref.lancius_sub(g, i["a"], i["b"]), feeds)
    k["mul_out"] = ref_op(ref, two, lambda g, i: ref.lancius_mul(g, i["a"], i["b"]), feeds)
    k["relu_bwd_out"] = ref_op(ref, two, lambda g, i: ref.lancius_relu_bwd(g, i["b"], i["a"]), feeds)
    one = {"a": (R, Cc)}
    k["transpose_out"] = ref_op(ref, one, lambda g, i: ref.lancius_transpose(g, i["a"]), {"a": a})
    k["sum_out"] = ref_op(ref, one, lambda g, i: ref.lancius_sum(g, i["a"]), {"a": a})
    k["sum_axis0_out"] = ref_op(ref, one, lambda g, i: ref.lancius_sum_axis0(g, i["a"]), {"a": a})
    k["sum_axis1_out"] = ref_op(ref, one, lambda g, i: ref.lancius_sum_axis1(g, i["a"]), {"a": a})
    y = np.exp(a - a.max(1, keepdims=True))
    y = f32(y / y.sum(1, keepdims=True))
    k["softmax_bwd_y"] = y
    k["softmax_bwd_out"] = ref_op(ref, two, lambda g, i: ref.lancius_softmax_bwd(g, i["b"], i["a"]),
                                  {"a": y, "b": b})
    # cross-entropy: one-hot targets, plus a row with no 1.0 and a row with two
    t = np.zeros((R, Cc))
    t[np.arange(R), [3, 0, 8, 5, 5, 1]] = 1.0
    t[4] = 0.0
    t[5, 7] = 1.0
    x = f32(prng.normal(22, (R, Cc), std=3.0))
    k["ce_x"], k["ce_y"] = x, t
    k["ce_out"] = ref_op(ref, two, lambda g, i: ref.lancius_cross_entropy(g, i["a"], i["b"]), {"a": x, "b": t})
    k["ce_g"] = np.array([[0.75]])
    k["ce_bwd_out"] = ref_op(ref, {"a": (R, Cc), "b": (R, Cc), "g": (1, 1)},
                             lambda g, i: ref.lancius_cross_entropy_bwd(g, i["a"], i["b"], i["g"]),
                             {"a": x, "b": t, "g": k["ce_g"]})
    # conv backward, kernel level: stride 1 pad 1 and stride 2 pad 2
    for tag, (N, Ci, H, W, Co, KH, KW, st, pd), seed in (("s1p1", (2, 3, 7, 6, 4, 3, 3, 1, 1), 23),
                                                        ("s2p2", (1, 2, 9, 8, 3, 5, 5, 2, 2), 24)):
        Ho, Wo = (H + 2 * pd - KH) // st + 1, (W + 2 * pd - KW) // st + 1
        xx, ww = f32(prng.normal(seed, (N, Ci, H, W))), f32(prng.normal(seed + 50, (Co, Ci, KH, KW)))
        gg = f32(prng.normal(seed + 100, (N, Co, Ho, Wo)))
        dx, dw = np.zeros((N, Ci, H, W)), np.zeros((Co, Ci, KH, KW))
        ref.kernel_conv2d_bwd_in(p(dx), p(gg), p(ww), N, Ci, H, W, Co, Ho, Wo, KH, KW, st, pd)
        ref.kernel_conv2d_bwd_w(p(dw), p(gg), p(xx), N, Ci, H, W, Co, Ho, Wo, KH, KW, st, pd)
        k[f"cbwd_{tag}_x"], k[f"cbwd_{tag}_w"], k[f"cbwd_{tag}_g"] = xx, ww, gg
        k[f"cbwd_{tag}_dx"], k[f"cbwd_{tag}_dw"] = dx, dw
    # max pooling: overlapping 3/2 windows with ties, and 2/2 windows, one of
    # which holds nothing above -1e9 (its gradient goes to plane (0,0))
    xp = f32(np.round(prng.normal(25, (2, 3, 9, 7)) * 2.0) / 2.0)  # many ties
    xp[1, 2, 2:4, 2:4] = -2e9
    k["pool_x"] = xp
    for tag, (K, st) in (("k3s2", (3, 2)), ("k2s2", (2, 2))):
        Ho, Wo = (9 - K) // st + 1, (7 - K) // st + 1
        k[f"pool_{tag}_out"] = ref_op(ref, {"x": (2, 3, 9, 7)}, lambda g, i: ref.lancius_maxpool2d(g, i["x"], K, st),
                                      {"x": xp})
        gp = f32(prng.normal(26, (2, 3, Ho, Wo)))
        k[f"pool_{tag}_g"] = gp
        k[f"pool_{tag}_dx"] = ref_op(ref, {"g": (2, 3, Ho, Wo), "x": (2, 3, 9, 7)},
                                     lambda g, i: ref.lancius_maxpool2d_bwd(g, i["g"], i["x"], K, st),
                                     {"g": gp, "x": xp})


def int8_vectors(ref, k: dict) -> None:
    """Golden vectors of the int8 path: the int8 MATMUL branch
    (lancius_scheduler.c:195-220), lancius_quantize_graph + the int8 conv route
    (lancius_quantize.c, lancius_vision_ops.c:16-57, also fused with ReLU),
    and kernel_conv2d_int8_fwd on given int8 tensors."""
    I8 = C.POINTER(C.c_int8)
    # MATMUL with an int8 B (its scale set on the node, as a loader would)
    M, K, N = 9, 37, 11
    a = f32(prng.normal(30, (M, K), std=1.5))
    a[0, 0] = 0.5 * float(np.max(np.abs(a)))  # exact .5 quotients appear in rows
    bq = (np.round(prng.uniform(31, (K, N), -127.4, 127.4))).astype(np.int8)
    scale_b = 0.0173
    bg = graphs.BuiltGraph(ref, ref.lancius_graph_create())
    na = graphs._inp(bg, "a", M, K)
    nb = graphs._inp(bg, "b", K, N)
    bg.nodes["out"] = ref.lancius_matmul(bg.g, na, nb)
    bg.outputs = ["out"]
    nb.contents.runtime_data_int8 = bq.ctypes.data_as(I8)
    nb.contents.scale = scale_b
    k["i8mm_a"], k["i8mm_bq"], k["i8mm_scale_b"] = a, bq, np.array(scale_b)
    k["i8mm_out"] = run_ref_graph(ref, bg, {"a": a, "b": bq.astype(np.float64) * scale_b})["out"]
    nb.contents.runtime_data_int8 = None
    bg.destroy()
    # conv through lancius_quantize_graph, unfused and fused with ReLU
    for tag, fuse in (("i8conv", False), ("i8conv_relu", True)):
        x = f32(prng.normal(32, (2, 5, 9, 8)))
        w = f32(prng.normal(33, (6, 5, 3, 3), std=0.3))
        bg = graphs.BuiltGraph(ref, ref.lancius_graph_create())
        nx = graphs._inp(bg, "x", 2, 5, 9, 8)
        nw = graphs._inp(bg, "w", 6, 5, 3, 3)
        conv = ref.lancius_conv2d(bg.g, nx, nw, 1, 1)
        bg.nodes["out"] = ref.lancius_relu(bg.g, conv) if fuse else conv
        if fuse:
            ref.lancius_optimize_fusion(bg.g)
        bg.outputs = ["out"]
        keep = [np.ascontiguousarray(x), np.ascontiguousarray(w)]
        nx.contents.runtime_data = p(keep[0])
        nw.contents.runtime_data = p(keep[1])
        ref.lancius_quantize_graph(bg.g)
        wq = np.ctypeslib.as_array(nw.contents.runtime_data_int8, shape=(w.size,)).copy().reshape(w.shape)
        k[f"{tag}_x"], k[f"{tag}_w"], k[f"{tag}_wq"] = x, w, wq
        k[f"{tag}_scale_w"] = np.array(nw.contents.scale)
        sched = ref.lancius_ir_schedule(bg.g)
        arena = ref.lancius_arena_create(64 << 20)
        ref.lancius_schedule_execute(sched, arena)
        n = bg.node("out")
        k[f"{tag}_out"] = np.ctypeslib.as_array(n.contents.runtime_data, shape=(abi.node_elems(n),)).copy().reshape(
            abi.node_shape(n))
        ref.lancius_schedule_destroy(sched)
        ref.lancius_arena_destroy(arena)
        bg.destroy()  # frees the reference's int8 copies
    # kernel_conv2d_int8_fwd on given int8 tensors, stride 2 pad 2
    xq = np.round(prng.uniform(34, (1, 3, 11, 10), -127.4, 127.4)).astype(np.int8)
    xq.flat[0] = 127  # so that re-quantizing xq * 0.01 returns xq
    wq = np.round(prng.uniform(35, (4, 3, 5, 5), -127.4, 127.4)).astype(np.int8)
    out = np.zeros((1, 4, 6, 5))
    ref.kernel_conv2d_int8_fwd(p(out), xq.ctypes.data_as(I8), wq.ctypes.data_as(I8), 0.01, 0.002,
                               1, 3, 11, 10, 4, 5, 5, 2, 2)
    k["i8k_xq"], k["i8k_wq"], k["i8k_out"] = xq, wq, out


def decode_vectors(ref, k: dict) -> None:
    """Golden vectors of the decode-side family: kernel_rmsnorm, kernel_swiglu,
    kernel_rope, kernel_gqa, kernel_attention_kv_cache (lancius_kernels.c:
    248-272, 338-448) and the RMSNORM / SWIGLU / GQA / ROPE scheduler branches
    (lancius_scheduler.c:134-165)."""
    x = f32(prng.normal(40, (5, 12), 0.3, 2.0))
    g = f32(prng.normal(41, (12,), 1.0, 0.2))
    out = np.zeros((5, 12))
    ref.kernel_rmsnorm(p(out), p(x), p(g), 5, 12, 1e-5)
    k["rms_x"], k["rms_g"], k["rms_out"] = x, g, out
    gate = f32(prng.normal(42, (64,), std=5.0))
    gate[:4] = [0.0, 80.0, -80.0, -700.0]
    up = f32(prng.normal(43, (64,)))
    out = np.zeros(64)
    ref.kernel_swiglu(p(out), p(gate), p(up), 64)
    k["swiglu_gate"], k["swiglu_up"], k["swiglu_out"] = gate, up, out
    # rope: q and k [1, 7, 3, 8] rotated in place, positions from 5
    q = f32(prng.normal(44, (1, 7, 3, 8)))
    kk = f32(prng.normal(45, (1, 7, 3, 8)))
    qr, kr = q.copy(), kk.copy()
    ref.kernel_rope(p(qr), p(kr), 1, 7, 3, 8, 5)
    k["rope_q"], k["rope_k"], k["rope_q_out"], k["rope_k_out"] = q, kk, qr, kr
    # gqa: q [9, 6, 8], k/v [9, 2, 8], causal
    q = f32(prng.uniform(46, (9, 6, 8), -1.0, 1.0))
    kv = [f32(prng.uniform(47 + i, (9, 2, 8), -1.0, 1.0)) for i in range(2)]
    out = np.zeros((9, 6, 8))
    ref.kernel_gqa(p(out), p(q), p(kv[0]), p(kv[1]), 9, 6, 2, 8)
    k["gqa_q"], k["gqa_k"], k["gqa_v"], k["gqa_out"] = q, kv[0], kv[1], out
    # kv-cache decode: one query [4 heads x 16], caches [13, 4, 16]
    q = f32(prng.uniform(49, (4, 16), -1.0, 1.0))
    kc, vc = f32(prng.uniform(50, (13, 4, 16), -1.0, 1.0)), f32(prng.uniform(51, (13, 4, 16), -1.0, 1.0))
    out = np.zeros((4, 16))
    ref.kernel_attention_kv_cache(p(out), p(q), p(kc), p(vc), 13, 4, 16)
    k["kvc_q"], k["kvc_k"], k["kvc_v"], k["kvc_out"] = q, kc, vc, out
    # scheduler branches
    k["node_rms_out"] = ref_op(ref, {"x": (5, 12), "g": (1, 12)}, lambda gg, i: ref.lancius_rmsnorm(gg, i["x"], i["g"]),
                               {"x": k["rms_x"], "g": k["rms_g"][None, :]})
    k["node_swiglu_out"] = ref_op(ref, {"a": (8, 8), "b": (8, 8)}, lambda gg, i: ref.lancius_swiglu(gg, i["a"], i["b"]),
                                  {"a": gate.reshape(8, 8), "b": up.reshape(8, 8)})

    def gqa_node(gg, i):
        q3 = ref.lancius_reshape(gg, i["q"], 3, 9, 6, 8, 0)
        k3 = ref.lancius_reshape(gg, i["k"], 3, 9, 2, 8, 0)
        v3 = ref.lancius_reshape(gg, i["v"], 3, 9, 2, 8, 0)
        return ref.lancius_gqa(gg, q3, k3, v3, 6, 2)

    k["node_gqa_out"] = ref_op(ref, {"q": (9, 48), "k": (9, 16), "v": (9, 16)}, gqa_node,
                               {"q": k["gqa_q"].reshape(9, 48), "k": k["gqa_k"].reshape(9, 16),
                                "v": k["gqa_v"].reshape(9, 16)})

    def rope_node(gg, i):
        x3 = ref.lancius_reshape(gg, i["x"], 3, 7, 3, 16, 0)
        n = ref.lancius_relu(gg, x3)  # a unary node of x3's shape, re-opcoded: the reference has no ROPE builder
        n.contents.op = abi.OP["ROPE"]
        return n

    xr = f32(prng.normal(52, (7, 48)))
    k["node_rope_x"] = xr
    k["node_rope_out"] = ref_op(ref, {"x": (7, 48)}, rope_node, {"x": xr})


TRAIN_GRAPHS = {
    "mlp": lambda lib: graphs.build_mlp_ce(lib, batch=64, d_in=784, hidden=128, classes=10),
    "cnn": lambda lib: graphs.build_cnn_ce(lib, batch=4),
    "cnn_fused": lambda lib: graphs.build_cnn_ce(lib, batch=4, fuse=True),
    "gradcheck": graphs.build_gradcheck,
    "ops": graphs.build_ops_loss,
}
TRAIN_SEEDS = {"mlp": 5000, "cnn": 6000, "cnn_fused": 6000, "gradcheck": 7000, "ops": 8000}


def train_feeds(t, seed: int) -> dict[str, np.ndarray]:
    """Seeded inputs of a training graph: one-hot targets Y, He-scaled 4-D
    weights, N(0, 0.05) matrices, N(0,1) data."""
    feeds = {}
    for i, name in enumerate(t.inputs):
        shape = abi.node_shape(t.node(name))
        s = seed + 17 * i
        if name == "Y":
            rows, classes = shape
            lab = (prng.uniform(s, (rows,), 0.0, 1.0) * classes).astype(np.int64) % classes
            y = np.zeros(shape)
            y[np.arange(rows), lab] = 1.0
            feeds[name] = y
        elif name.startswith("W") and len(shape) == 4:
            fan_in = shape[1] * shape[2] * shape[3]
            feeds[name] = f32(prng.normal(s, shape, 0.0, float(np.sqrt(2.0 / fan_in))))
        elif name.startswith(("W", "b")):
            feeds[name] = f32(prng.normal(s, shape, 0.0, 0.05))
        else:
            feeds[name] = f32(prng.normal(s, shape))
    return feeds


if __name__ == "__main__":
    if sys.argv[1:] == ["models"]:  # only the model-file fixtures
        _ref = oracle.ref_lib()
        if _ref is None:
            raise SystemExit("oracle/_ref/liblancius_ref.so not built (needs /root/reference)")
        model_vectors(_ref)
    else:
        main()
