"""The BASIS interfaces on the device: the memory API (include/basis/core/
memory.h, declared and never implemented by the reference) on HBM, and the
device executor for BASIS static graphs (include/basis/stage6_ir/graph.h),
against the fp64 oracle.

The reference has no executor for these graphs, so the oracle is the
textbook meaning of each op: MATMUL a.b, ADD a+b, BROADCAST_ADD a + bias
row, RELU max(x,0), TANH tanh(x), all in fp64.  Bar: normwise error within
1e-4 * max(1, sqrt(K)/32) for the longest reduction K.
"""
import ctypes as C

import numpy as np
import pytest

import oracle
from lancius_amd import ACT_NONE, ACT_RELU, ACT_TANH, HipError, graph_lib, prng
from lancius_amd.basis import KEEP_ALL, Graph, Program, declare_device
from tests.conftest import case

pytestmark = pytest.mark.gpu

TOL_ELEMENTWISE = 1e-6


# ---- memory API -----------------------------------------------------------


def test_arena_bump_alignment_growth_and_reset(dev):
    lib = declare_device(dev.lib)
    case("basis_arena")
    a = lib.basis_arena_create(4096)
    assert a
    assert lib.lancius_basis_arena_capacity(a) == 4096
    p1 = lib.basis_arena_alloc(a, 100, 0)
    p2 = lib.basis_arena_alloc(a, 100, 1024)
    p3 = lib.basis_arena_alloc(a, 8, 8)
    assert p1 % 256 == 0 and p2 % 1024 == 0 and p3 % 8 == 0
    assert p1 < p2 < p3 and p3 - p1 < 4096  # one block
    big = lib.basis_arena_alloc(a, 1 << 20, 0)  # does not fit: a new block
    assert big and lib.lancius_basis_arena_capacity(a) >= 4096 + (1 << 20)
    # the memory is real HBM: a round trip through it
    x = prng.normal(1, (1 << 18,))
    assert dev.lib.lancius_hip_upload(dev.ctx, big, x.ctypes.data_as(C.c_void_p), x.nbytes) == 0
    y = np.empty_like(x)
    assert dev.lib.lancius_hip_download(dev.ctx, y.ctypes.data_as(C.c_void_p), big, y.nbytes) == 0
    assert np.array_equal(x, y)
    cap = lib.lancius_basis_arena_capacity(a)
    lib.basis_arena_reset(a)
    assert lib.basis_arena_alloc(a, 100, 0) == p1  # rewound, blocks kept
    assert lib.basis_arena_alloc(a, 4000, 0) != 0  # next block reused after the first fills
    assert lib.lancius_basis_arena_capacity(a) == cap
    assert not lib.basis_arena_alloc(a, 16, 3)  # alignment not a power of two
    lib.basis_arena_destroy(a)
    lib.basis_arena_destroy(None)


def test_pool_reuse_and_bad_frees(dev):
    lib = declare_device(dev.lib)
    case("basis_pool")
    p = lib.basis_pool_create(1000, 4)  # objects rounded to 1024 bytes
    assert p
    objs = [lib.basis_pool_alloc(p) for _ in range(5)]  # two chunks
    assert len(set(objs)) == 5 and all(o % 256 == 0 for o in objs)
    assert objs[1] - objs[0] == 1024
    assert lib.lancius_basis_pool_capacity(p) == 2 * 4 * 1024
    lib.basis_pool_free(p, objs[2])
    assert lib.basis_pool_alloc(p) == objs[2]
    lib.basis_pool_free(p, objs[3])
    lib.basis_pool_free(p, objs[3])  # twice: the second is ignored
    lib.basis_pool_free(p, objs[0] + 8)  # not an object start: ignored
    lib.basis_pool_free(p, None)
    again = [lib.basis_pool_alloc(p) for _ in range(2)]
    assert again[0] == objs[3] and again[1] not in objs
    assert not lib.basis_pool_create(0, 4)
    lib.basis_pool_destroy(p)


# ---- tanh and bias + activation kernels --------------------------------------


@pytest.mark.parametrize("rows,cols", [(64, 48), (7, 13), (1, 4), (300, 1000)])
@pytest.mark.parametrize("act", [ACT_NONE, ACT_RELU, ACT_TANH])
def test_bias_act(dev, rows, cols, act):
    a = prng.normal(rows + cols, (rows, cols), std=2.0)
    b = prng.normal(act + 7, (cols,))
    da, db, do = dev.upload(a), dev.upload(b), dev.alloc(rows * cols * 4)
    case(f"bias_act {rows}x{cols} act={act}")
    dev.bias_act(do, da, db, rows, cols, act)
    got = dev.download(do, (rows, cols))
    ref = a.astype(np.float64) + b.astype(np.float64)[None, :]
    ref = np.maximum(ref, 0) if act == ACT_RELU else np.tanh(ref) if act == ACT_TANH else ref
    assert oracle.normwise_error(got, ref) <= TOL_ELEMENTWISE
    for x in (da, db, do):
        x.free()


def test_tanh_elementwise_and_special_values(dev):
    x = np.concatenate([prng.normal(9, (1001,), std=4.0),
                        np.array([0.0, -0.0, 30.0, -30.0, np.inf, -np.inf, np.nan], np.float32)]).astype(np.float32)
    dx, do = dev.upload(x), dev.alloc(x.size * 4)
    case("tanh")
    dev.tanh(do, dx, x.size)
    got = dev.download(do, (x.size,))
    ref = np.tanh(x.astype(np.float64))
    fin = np.isfinite(ref)
    assert np.max(np.abs(got[fin] - ref[fin])) <= 2e-7
    assert got[-3] == 1.0 and got[-2] == -1.0 and np.isnan(got[-1])
    for b in (dx, do):
        b.free()


# ---- executor ------------------------------------------------------------------


def _mlp_graph(M=64, K=784, H=256, O=10):
    g = Graph(graph_lib())
    ids = {"x": g.input("x", M, K), "W1": g.input("W1", K, H), "b1": g.input("b1", 1, H)}
    ids["h"] = g.matmul(ids["x"], ids["W1"])
    ids["hb"] = g.broadcast_add(ids["h"], ids["b1"])
    ids["ht"] = g.tanh(ids["hb"])
    ids["W2"], ids["b2"] = g.input("W2", H, O), g.input("b2", 1, O)
    ids["y"] = g.matmul(ids["ht"], ids["W2"])
    ids["yb"] = g.broadcast_add(ids["y"], ids["b2"])
    ids["out"] = g.relu(ids["yb"])
    return g, ids


def _feeds(g, ids, seed):
    f = {}
    for name, i in ids.items():
        n = g.node(i)
        if n.op == 0:
            f[name] = prng.normal(seed + i, (n.rows, n.cols), std=0.1 if name.startswith(("W", "b")) else 1.0)
    return f


def _mlp_ref(f):
    d = {k: v.astype(np.float64) for k, v in f.items()}
    ht = np.tanh(oracle.matmul(f["x"], f["W1"]) + d["b1"])
    return ht, np.maximum(oracle.matmul(ht, f["W2"]) + d["b2"], 0.0)


@pytest.mark.parametrize("M,flags,launches", [
    (64, 0, 1),         # the whole MLP in one lancius_hip_mlp2_ex_f32 call
    (96, 0, 2),         # batch above the chain kernel's limit: two fused GEMMs
    (64, KEEP_ALL, 6),  # every node its own launch and buffer
])
def test_mlp_graph(dev, M, flags, launches):
    g, ids = _mlp_graph(M=M)
    f = _feeds(g, ids, 300)
    prog = Program(dev, g, flags)
    for name, arr in f.items():
        prog.upload(ids[name], arr)
    case(f"basis mlp M={M} flags={flags}")
    prog.run()
    ht_ref, out_ref = _mlp_ref(f)
    got = prog.download(ids["out"])
    assert oracle.normwise_error(got, out_ref) <= oracle.tolerance(784)
    assert prog.info()["launches"] == launches
    if flags & KEEP_ALL:
        assert oracle.normwise_error(prog.download(ids["ht"]), ht_ref) <= oracle.tolerance(784)
        assert prog.buffer(ids["h"]) is not None
    else:
        assert prog.buffer(ids["h"]) is None  # absorbed into a fused launch
        with pytest.raises(HipError) as e:
            prog.download(ids["h"])
        assert e.value.code == -4
    prog.close()
    g.close()


def test_residual_and_unfused_ops(dev):
    """x.W + b -> relu -> + x is one GEMM (bias, ReLU, residual); an ADD of
    two inputs, TANH and RELU of an input and a BROADCAST_ADD -> TANH of an
    input run as their own kernels."""
    g = Graph(graph_lib())
    x, W, b = g.input("x", 96, 64), g.input("W", 64, 64), g.input("b", 1, 64)
    h = g.relu(g.broadcast_add(g.matmul(x, W), b))
    r = g.add(h, x)
    u, v = g.input("u", 96, 64), g.input("v", 96, 64)
    s = g.add(u, v)
    t = g.tanh(u)
    q = g.relu(v)
    bt = g.tanh(g.broadcast_add(u, b))
    f = {i: prng.normal(500 + i, (g.node(i).rows, g.node(i).cols)) for i in (x, W, b, u, v)}
    prog = Program(dev, g)
    for i, arr in f.items():
        prog.upload(i, arr)
    case("basis residual + unfused")
    prog.run()
    d = {i: a.astype(np.float64) for i, a in f.items()}
    ref_r = np.maximum(oracle.matmul(f[x], f[W]) + d[b], 0.0) + d[x]
    assert oracle.normwise_error(prog.download(r), ref_r) <= oracle.tolerance(64)
    assert oracle.normwise_error(prog.download(s), d[u] + d[v]) <= TOL_ELEMENTWISE
    assert oracle.normwise_error(prog.download(t), np.tanh(d[u])) <= TOL_ELEMENTWISE
    assert np.array_equal(prog.download(q), np.maximum(f[v], 0))
    assert oracle.normwise_error(prog.download(bt), np.tanh(d[u] + d[b])) <= TOL_ELEMENTWISE
    # GEMM(+bias, ReLU, residual), ADD, TANH, RELU, bias+TANH
    assert prog.info()["launches"] == 5
    prog.close()
    g.close()


def test_hidden_layer_read_twice_is_not_one_mlp_launch(dev):
    """The hidden activation feeds both the second MATMUL and a residual ADD,
    so it must be materialised: two GEMM chains, the second with the
    residual in its epilogue, not one MLP launch."""
    g = Graph(graph_lib())
    x, W1, W2 = g.input("x", 32, 48), g.input("W1", 48, 64), g.input("W2", 64, 64)
    h = g.tanh(g.matmul(x, W1))
    out = g.add(g.relu(g.matmul(h, W2)), h)
    f = {i: prng.normal(800 + i, (g.node(i).rows, g.node(i).cols), std=0.2) for i in (x, W1, W2)}
    prog = Program(dev, g)
    for i, arr in f.items():
        prog.upload(i, arr)
    case("basis mlp with a shared hidden layer")
    prog.run()
    ht = np.tanh(oracle.matmul(f[x], f[W1]))
    ref = np.maximum(oracle.matmul(ht, f[W2]), 0.0) + ht
    assert oracle.normwise_error(prog.download(out), ref) <= oracle.tolerance(64)
    assert oracle.normwise_error(prog.download(h), ht) <= oracle.tolerance(48)
    assert prog.info()["launches"] == 2
    prog.close()
    g.close()


def test_residual_computed_later_is_not_fused(dev):
    """ADD(chain, z) where z comes after the MATMUL cannot be the GEMM's
    residual (it does not exist yet when the GEMM runs)."""
    g = Graph(graph_lib())
    x, W, u = g.input("x", 32, 32), g.input("W", 32, 32), g.input("u", 32, 32)
    m = g.matmul(x, W)
    z = g.tanh(u)
    r = g.add(m, z)
    f = {i: prng.normal(700 + i, (32, 32)) for i in (x, W, u)}
    prog = Program(dev, g)
    for i, arr in f.items():
        prog.upload(i, arr)
    case("basis late residual")
    prog.run()
    ref = oracle.matmul(f[x], f[W]) + np.tanh(f[u].astype(np.float64))
    assert oracle.normwise_error(prog.download(r), ref) <= oracle.tolerance(32)
    assert prog.info()["launches"] == 3
    prog.close()
    g.close()


def test_program_rejects_bad_requests(dev):
    g, ids = _mlp_graph(M=4, K=8, H=8, O=2)
    prog = Program(dev, g)
    case("basis refusals")
    with pytest.raises(HipError) as e:
        prog.upload(ids["h"], np.zeros((4, 8), np.float32))  # absorbed node
    assert e.value.code == -4
    with pytest.raises(HipError) as e:
        prog.upload(ids["x"], np.zeros(5, np.float32))  # wrong count
    assert e.value.code == -3
    with pytest.raises(HipError) as e:
        prog.upload(99, np.zeros(1, np.float32))
    assert e.value.code == -3
    prog.close()
    # a hand-edited graph whose MATMUL reads a later node is refused
    g.g.contents.nodes[ids["h"]].input_ids[1] = ids["out"]
    with pytest.raises(HipError) as e:
        Program(dev, g)
    assert e.value.code == -3
    g.close()
