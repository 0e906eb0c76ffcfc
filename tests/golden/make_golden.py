"""Writes the golden fixtures of tests/golden/ by running the REFERENCE's own
C code, compiled from /root/reference into oracle/_ref/liblancius_ref.so
(`python -m lancius_amd.build`).  Run in the build container only:

    python tests/golden/make_golden.py

Outputs (data only - inputs and the reference's outputs):
  kernels.npz        kernel_matmul / graph MATMUL, kernel_conv2d_fwd,
                     kernel_conv2d_relu_fwd, kernel_attention,
                     kernel_layernorm, kernel_gelu, graph SOFTMAX
  graphs.json        lancius_ir_schedule waves and lancius_build_memory_plan
                     offsets/peaks of the config graphs (fp32 dtypes, as the
                     device plans them) and of the 20 x ReLU chain (fp64)
  graph_outputs.npz  sink values of reference CPU graph runs (scratch-arena
                     executor, B/src/runtime/lancius_scheduler.c:311-362)
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
    print("fixtures written to", OUT)


if __name__ == "__main__":
    main()
