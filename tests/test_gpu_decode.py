"""The decode-side family on the device (RMSNorm, SwiGLU, RoPE, GQA
attention including a key sequence longer than the queries, split-KV decode
attention with per-sequence cache lengths) and the RMSNORM / SWIGLU / GQA /
ROPE nodes through the executor, against the oracle and the compiled
reference's golden outputs.  Tolerance as everywhere:
1e-4 * max(1, sqrt(K)/32) with K the longest reduction."""
import ctypes as C
from pathlib import Path

import numpy as np
import pytest

import oracle
from lancius_amd import DeviceProgram, abi, graph_lib, graphs, prng
from tests.conftest import case

pytestmark = pytest.mark.gpu

K = np.load(Path(__file__).resolve().parent / "golden" / "kernels.npz")


def f64(a):
    return np.asarray(a, np.float32).astype(np.float64)


def up(dev, a):
    return dev.upload(np.ascontiguousarray(a, dtype=np.float32))


@pytest.mark.parametrize("rows,hidden", [(5, 12), (64, 4096), (1000, 257), (1, 1), (7, 1000), (3, 2052)])
def test_rmsnorm(dev, rows, hidden):
    x, g = prng.normal(200 + hidden, (rows, hidden), 0.3, 2.0), prng.normal(201, (hidden,), 1.0, 0.2)
    if (rows, hidden) == (5, 12):
        x, g = K["rms_x"], K["rms_g"]
    dx, dg, do = up(dev, x), up(dev, g), dev.alloc(4 * rows * hidden)
    case(f"rmsnorm {rows}x{hidden}")
    dev.rmsnorm(do, dx, dg, rows, hidden)
    got = dev.download(do, (rows, hidden))
    ref = K["rms_out"] if (rows, hidden) == (5, 12) else oracle.rmsnorm(f64(x), f64(g))
    assert oracle.normwise_error(got, ref) <= oracle.tolerance(hidden)
    for b in (dx, dg, do):
        b.free()


def test_swiglu(dev):
    gate, upv = K["swiglu_gate"], K["swiglu_up"]
    dg, du, do = up(dev, gate), up(dev, upv), dev.alloc(4 * 64)
    case("swiglu golden")
    dev.swiglu(do, dg, du, 64)
    assert oracle.normwise_error(dev.download(do, (64,)), K["swiglu_out"]) <= 1e-6
    n = 1 << 22
    gate2, up2 = prng.normal(210, (n,), std=4.0), prng.normal(211, (n,))
    dg2, du2, do2 = up(dev, gate2), up(dev, up2), dev.alloc(4 * n)
    dev.swiglu(do2, dg2, du2, n)
    assert oracle.normwise_error(dev.download(do2, (n,)), oracle.swiglu(f64(gate2), f64(up2))) <= 1e-6
    for b in (dg, du, do, dg2, du2, do2):
        b.free()


@pytest.mark.parametrize("count,batch,S,H,hd,pos", [(2, 1, 7, 3, 8, 5), (2, 1, 4096, 8, 128, 0), (1, 3, 33, 4, 64, 1000)])
def test_rope(dev, count, batch, S, H, hd, pos):
    if (S, hd) == (7, 8):
        x = np.concatenate([K["rope_q"].ravel(), K["rope_k"].ravel()])
        ref = np.concatenate([K["rope_q_out"].ravel(), K["rope_k_out"].ravel()])
    else:
        x = prng.normal(220 + S, (count * batch * S * H * hd,))
        ref = oracle.rope(f64(x), count, batch, S, H, hd, pos)
    dx = up(dev, x)
    case(f"rope count={count} batch={batch} S={S} H={H} hd={hd} pos={pos}")
    dev.rope(dx, dx, count, batch, S, H, hd, pos)  # in place, as the node does
    assert oracle.normwise_error(dev.download(dx, (x.size,)), ref) <= 1e-6
    dx.free()


def _gqa(dev, B, Sq, Skv, Hq, Hkv, D, causal, seed, q=None, k=None, v=None):
    q = prng.uniform(seed, (B, Sq, Hq, D), -1.0, 1.0) if q is None else q
    k = prng.uniform(seed + 1, (B, Skv, Hkv, D), -1.0, 1.0) if k is None else k
    v = prng.uniform(seed + 2, (B, Skv, Hkv, D), -1.0, 1.0) if v is None else v
    dq, dk, dv, do = up(dev, q), up(dev, k), up(dev, v), dev.alloc(4 * q.size)
    case(f"attention_gqa B={B} Sq={Sq} Skv={Skv} Hq={Hq} Hkv={Hkv} D={D} causal={causal}")
    dev.attention_gqa(do, dq, dk, dv, B, Sq, Skv, Hq, Hkv, D, causal)
    got = dev.download(do, q.shape)
    for b in (dq, dk, dv, do):
        b.free()
    return q, k, v, got


def test_gqa_golden(dev):
    q, k, v = K["gqa_q"][None], K["gqa_k"][None], K["gqa_v"][None]
    *_, got = _gqa(dev, 1, 9, 9, 6, 2, 8, True, 0, q, k, v)
    assert oracle.normwise_error(got[0], K["gqa_out"]) <= oracle.tolerance(9)


@pytest.mark.parametrize("B,Sq,Skv,Hq,Hkv,D,causal", [
    (1, 300, 300, 16, 4, 64, True),     # GQA prefill, fused D = 64 kernel
    (2, 128, 1000, 8, 2, 64, True),     # queries after a 872-token history
    (2, 65, 190, 8, 8, 64, False),      # non-causal, ragged lengths
    (1, 50, 80, 6, 3, 40, True),        # other head dim: row kernel
    (1, 1, 513, 4, 1, 64, True),        # one query over a cache (MQA)
    (2, 300, 300, 16, 4, 128, True),    # GQA prefill at D = 128: the fused kernel, 32-key blocks
    (2, 128, 1000, 8, 2, 128, True),    # D = 128 after an 872-token history
    (1, 77, 200, 8, 4, 128, False),     # D = 128 non-causal, ragged
    (2, 96, 500, 8, 2, 32, True),       # D = 32 with history
    (1, 130, 130, 6, 2, 96, True),      # D = 96
])
def test_gqa_shapes(dev, B, Sq, Skv, Hq, Hkv, D, causal):
    q, k, v, got = _gqa(dev, B, Sq, Skv, Hq, Hkv, D, causal, 230 + Sq + Skv)
    ref = oracle.attention_gqa(f64(q), f64(k), f64(v), causal)
    assert oracle.normwise_error(got, ref) <= oracle.tolerance(max(Skv, D))


def _decode(dev, B, Skv, Hq, Hkv, D, lens, seed, q=None, k=None, v=None):
    q = prng.uniform(seed, (B, Hq, D), -1.0, 1.0) if q is None else q
    k = prng.uniform(seed + 1, (B, Skv, Hkv, D), -1.0, 1.0) if k is None else k
    v = prng.uniform(seed + 2, (B, Skv, Hkv, D), -1.0, 1.0) if v is None else v
    dq, dk, dv, do = up(dev, q), up(dev, k), up(dev, v), dev.alloc(4 * q.size)
    dl = dev.upload(np.asarray(lens, np.int32)) if lens is not None else None
    dev.fill(do, float("nan"), q.size)  # every output element must be written
    case(f"attention_decode B={B} Skv={Skv} Hq={Hq} Hkv={Hkv} D={D} lens={lens is not None}")
    dev.attention_decode(do, dq, dk, dv, dl, B, Skv, Hq, Hkv, D)
    got = dev.download(do, q.shape)
    assert np.isfinite(got).all(), f"{np.count_nonzero(~np.isfinite(got))} outputs not written"
    for b in (dq, dk, dv, do, dl):
        if b is not None:
            b.free()
    return q, k, v, got


def test_decode_golden(dev):
    q, k, v = K["kvc_q"].reshape(1, 4, 16), K["kvc_k"][None], K["kvc_v"][None]
    *_, got = _decode(dev, 1, 13, 4, 4, 16, None, 0, q, k, v)
    assert oracle.normwise_error(got.reshape(4, 16), K["kvc_out"]) <= oracle.tolerance(13)


@pytest.mark.parametrize("B,Skv,Hq,Hkv,D,lens", [
    (1, 4096, 32, 8, 128, None),
    (8, 1000, 8, 8, 64, None),
    (4, 777, 16, 2, 64, [777, 1, 0, 300]),
    (2, 64, 64, 1, 128, [64, 63]),
    (3, 5000, 4, 4, 96, [4999, 5000, 2500]),
    (2, 300, 6, 2, 37, None),
    (1, 1000, 8, 1, 100, [999]),
    (2, 2000, 32, 2, 80, [1500, 2000]),
    (16, 4096, 32, 8, 128, None),
])
def test_decode_shapes(dev, B, Skv, Hq, Hkv, D, lens):
    q, k, v, got = _decode(dev, B, Skv, Hq, Hkv, D, lens, 240 + Skv)
    ref = oracle.attention_decode(f64(q), f64(k), f64(v), lens)
    assert oracle.normwise_error(got, ref) <= oracle.tolerance(max(Skv, D))


def test_decode_deterministic(dev):
    B, Skv, Hq, Hkv, D = 2, 3000, 8, 2, 64
    q = prng.uniform(250, (B, Hq, D), -1.0, 1.0)
    k, v = prng.uniform(251, (B, Skv, Hkv, D), -1.0, 1.0), prng.uniform(252, (B, Skv, Hkv, D), -1.0, 1.0)
    outs = [_decode(dev, B, Skv, Hq, Hkv, D, None, 0, q, k, v)[3] for _ in range(3)]
    assert all(np.array_equal(outs[0], o) for o in outs[1:])


def test_decode_rejects_unsupported(dev):
    from lancius_amd import HipError

    case("attention_decode D=256 refused")
    with pytest.raises(HipError) as e:
        dev.attention_decode(None, None, None, None, None, 1, 4, 1, 1, 256)
    assert e.value.code in (-2, -3)


# ---- nodes through the executor ----------------------------------------------------


def _run_nodes(dev, build, feeds, out_name):
    lib = graph_lib()
    bg = graphs.BuiltGraph(lib, lib.lancius_graph_create())
    ins = {name: graphs._inp(bg, name, *a.shape) for name, a in feeds.items()}
    bg.nodes[out_name] = build(lib, bg.g, ins)
    bg.outputs = [out_name]
    lib.lancius_graph_set_dtype(bg.g, abi.DTYPE_FP32)
    sched = lib.lancius_ir_schedule(bg.g)
    plan = lib.lancius_build_memory_plan(sched, bg.g)
    prog = DeviceProgram(dev, bg.g, sched, plan)
    for name, a in feeds.items():
        prog.upload(bg.node(name), np.asarray(a, np.float32))
    prog.run()
    got = prog.download(bg.node(out_name))
    prog.close()
    lib.lancius_memory_plan_destroy(plan)
    lib.lancius_schedule_destroy(sched)
    bg.destroy()
    return got


def test_decode_nodes_on_device(dev):
    case("RMSNORM / SWIGLU / GQA / ROPE nodes")
    got = _run_nodes(dev, lambda L, g, i: L.lancius_rmsnorm(g, i["x"], i["g"]),
                     {"x": K["rms_x"], "g": K["rms_g"][None, :]}, "out")
    assert oracle.normwise_error(got, K["node_rms_out"]) <= oracle.tolerance(12)
    got = _run_nodes(dev, lambda L, g, i: L.lancius_swiglu(g, i["a"], i["b"]),
                     {"a": K["swiglu_gate"].reshape(8, 8), "b": K["swiglu_up"].reshape(8, 8)}, "out")
    assert oracle.normwise_error(got, K["node_swiglu_out"]) <= 1e-6

    def gqa(L, g, i):
        return L.lancius_gqa(g, L.lancius_reshape(g, i["q"], 3, 9, 6, 8, 0), L.lancius_reshape(g, i["k"], 3, 9, 2, 8, 0),
                             L.lancius_reshape(g, i["v"], 3, 9, 2, 8, 0), 6, 2)

    got = _run_nodes(dev, gqa, {"q": K["gqa_q"].reshape(9, 48), "k": K["gqa_k"].reshape(9, 16),
                                "v": K["gqa_v"].reshape(9, 16)}, "out")
    assert oracle.normwise_error(got, K["node_gqa_out"]) <= oracle.tolerance(9)

    def rope(L, g, i):
        n = L.lancius_relu(g, L.lancius_reshape(g, i["x"], 3, 7, 3, 16, 0))
        n.contents.op = abi.OP["ROPE"]  # no builder in the reference either (a loader makes these nodes)
        return n

    got = _run_nodes(dev, rope, {"x": K["node_rope_x"]}, "out")
    assert oracle.normwise_error(got, K["node_rope_out"]) <= 1e-6
