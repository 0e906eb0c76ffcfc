"""Parity of the training / reduction kernels (C ABI) and of the autodiff
training graphs through the device executor, against the fp64 oracle and the
reference's golden outputs.

Bar: normwise error max|y - y_ref| / max|y_ref| <= 1e-4 * max(1, sqrt(K)/32)
with K the longest reduction feeding the value; exact for TRANSPOSE, SUB,
MUL, RELU_BWD and MAXPOOL2D (no arithmetic beyond one fp32 op).
"""
import ctypes as C
from pathlib import Path

import numpy as np
import pytest

import oracle
from lancius_amd import DeviceProgram, abi, graph_lib, graphs, prng
from tests.conftest import case
from tests.golden.make_golden import TRAIN_GRAPHS, TRAIN_SEEDS, train_feeds

pytestmark = pytest.mark.gpu

GOLD = Path(__file__).resolve().parent / "golden"
K = np.load(GOLD / "kernels.npz")
T = np.load(GOLD / "train_outputs.npz")


def up(dev, a):
    return dev.upload(np.ascontiguousarray(a, dtype=np.float32))


def down(dev, buf, shape):
    return dev.download(buf, shape).astype(np.float64)


def f32(a):
    return np.asarray(a, np.float32).astype(np.float64)


# ---- elementwise ------------------------------------------------------------------


@pytest.mark.parametrize("n", [1, 3, 4, 1001, 4096 * 1024 + 3])
def test_sub_mul_relu_bwd(dev, n):
    a, b = prng.normal(100 + n % 97, (n,)), prng.normal(200 + n % 89, (n,))
    a[: min(n, 3)] = [0.0, -0.0, 1e-30][: min(n, 3)]
    da, db, dout = up(dev, a), up(dev, b), dev.alloc(4 * n)
    case(f"sub/mul/relu_bwd n={n}")
    dev.sub(dout, da, db, n)
    np.testing.assert_array_equal(dev.download(dout, (n,)), (a - b).astype(np.float32))
    dev.mul(dout, da, db, n)
    np.testing.assert_array_equal(dev.download(dout, (n,)), (a * b).astype(np.float32))
    dev.relu_bwd(dout, db, da, n)  # gradient b where forward a > 0
    np.testing.assert_array_equal(dev.download(dout, (n,)), np.where(a > 0, b, 0).astype(np.float32))
    for x in (da, db, dout):
        x.free()


def test_elementwise_golden(dev):
    a, b = K["ew_a"], K["ew_b"]
    n = a.size
    da, db, dout = up(dev, a), up(dev, b), dev.alloc(4 * n)
    case("sub/mul/relu_bwd golden")
    dev.sub(dout, da, db, n)
    assert oracle.normwise_error(down(dev, dout, a.shape), K["sub_out"]) <= 1e-7
    dev.mul(dout, da, db, n)
    assert oracle.normwise_error(down(dev, dout, a.shape), K["mul_out"]) <= 1e-7
    dev.relu_bwd(dout, db, da, n)
    np.testing.assert_array_equal(down(dev, dout, a.shape), K["relu_bwd_out"].astype(np.float32))
    for x in (da, db, dout):
        x.free()


# ---- transpose and sums ------------------------------------------------------------


@pytest.mark.parametrize("R,Cc", [(1, 1), (6, 9), (64, 64), (65, 130), (1000, 3), (3, 1000), (1024, 4096)])
def test_transpose(dev, R, Cc):
    a = prng.normal(300 + R + Cc, (R, Cc))
    da, dout = up(dev, a), dev.alloc(4 * R * Cc)
    case(f"transpose {R}x{Cc}")
    dev.transpose(dout, da, R, Cc)
    np.testing.assert_array_equal(dev.download(dout, (Cc, R)), a.T)
    da.free()
    dout.free()


@pytest.mark.parametrize("n", [0, 1, 5, 4096, 4097, 10_000_003])
def test_sum(dev, n):
    a = prng.normal(400 + n % 101, (max(n, 1),))[:n]
    da, dout = up(dev, a if n else np.zeros(1)), dev.alloc(4)
    case(f"sum n={n}")
    dev.sum(dout, da, n)
    got = float(dev.download(dout, (1,))[0])
    want = oracle.sum_all(a)
    # fp64 accumulation: only the final fp32 rounding
    assert abs(got - want) <= 1e-6 * max(1.0, abs(want))
    dev.sum(dout, da, n)
    assert float(dev.download(dout, (1,))[0]) == got  # fixed order: bit-identical
    da.free()
    dout.free()


@pytest.mark.parametrize("R,Cc", [(0, 5), (1, 7), (64, 128), (64, 10), (4096, 1024), (100_000, 3), (3, 5000)])
def test_sum_axes(dev, R, Cc):
    a = prng.normal(500 + R % 97 + Cc, (max(R, 1), Cc))[:R]
    da = up(dev, a if R else np.zeros((1, Cc)))
    d0, d1 = dev.alloc(4 * Cc), dev.alloc(4 * max(R, 1))
    case(f"sum_axis0/1 {R}x{Cc}")
    dev.sum_axis0(d0, da, R, Cc)
    got0 = down(dev, d0, (1, Cc))
    want0 = oracle.sum_axis0(a) if R else np.zeros((1, Cc))
    assert np.max(np.abs(got0 - want0)) <= 1e-6 * max(1.0, np.max(np.abs(want0)))
    if R:
        dev.sum_axis1(d1, da, R, Cc)
        got1 = down(dev, d1, (R, 1))
        want1 = oracle.sum_axis1(a)
        assert np.max(np.abs(got1 - want1)) <= 1e-6 * max(1.0, np.max(np.abs(want1)))
    for x in (da, d0, d1):
        x.free()


def test_sums_golden(dev):
    a = K["ew_a"]
    R, Cc = a.shape
    da, d0, d1, ds, dt = up(dev, a), dev.alloc(4 * Cc), dev.alloc(4 * R), dev.alloc(4), dev.alloc(4 * a.size)
    case("transpose/sum golden")
    dev.transpose(dt, da, R, Cc)
    np.testing.assert_array_equal(down(dev, dt, (Cc, R)), K["transpose_out"].astype(np.float32))
    dev.sum(ds, da, a.size)
    dev.sum_axis0(d0, da, R, Cc)
    dev.sum_axis1(d1, da, R, Cc)
    assert oracle.normwise_error(down(dev, ds, (1, 1)), K["sum_out"]) <= 1e-7
    assert oracle.normwise_error(down(dev, d0, (1, Cc)), K["sum_axis0_out"]) <= 1e-7
    assert oracle.normwise_error(down(dev, d1, (R, 1)), K["sum_axis1_out"]) <= 1e-7
    for x in (da, d0, d1, ds, dt):
        x.free()


# ---- softmax backward and cross-entropy -------------------------------------------


@pytest.mark.parametrize("R,Cc", [(6, 9), (64, 10), (33, 1000), (4096, 1024)])
def test_softmax_bwd(dev, R, Cc):
    x = prng.normal(600 + R, (R, Cc))
    y = oracle.softmax(x).astype(np.float32)
    dy = prng.normal(601 + R, (R, Cc))
    dyy, ddy, dout = up(dev, y), up(dev, dy), dev.alloc(4 * R * Cc)
    case(f"softmax_bwd {R}x{Cc}")
    dev.softmax_bwd(dout, ddy, dyy, R, Cc)
    assert oracle.normwise_error(down(dev, dout, (R, Cc)), oracle.softmax_bwd(dy, y)) <= oracle.tolerance(Cc)
    for b in (dyy, ddy, dout):
        b.free()


def test_cross_entropy_golden(dev):
    x, y, g = K["ce_x"], K["ce_y"], K["ce_g"]
    R, Cc = x.shape
    dx, dyy, dg, dl, dout = up(dev, x), up(dev, y), up(dev, g), dev.alloc(4), dev.alloc(4 * x.size)
    case("cross_entropy golden")
    dev.cross_entropy(dl, dx, dyy, R, Cc)
    assert oracle.normwise_error(down(dev, dl, (1, 1)), K["ce_out"]) <= oracle.tolerance(Cc)
    dev.cross_entropy_bwd(dout, dx, dyy, dg, R, Cc)
    assert oracle.normwise_error(down(dev, dout, (R, Cc)), K["ce_bwd_out"]) <= oracle.tolerance(Cc)
    for b in (dx, dyy, dg, dl, dout):
        b.free()


@pytest.mark.parametrize("R,Cc", [(1, 2), (64, 10), (1000, 1000), (8192, 10)])
def test_cross_entropy(dev, R, Cc):
    x = prng.normal(700 + R, (R, Cc), std=3.0)
    lab = (prng.uniform(701 + R, (R,), 0, 1) * Cc).astype(np.int64) % Cc
    y = np.zeros((R, Cc), np.float32)
    y[np.arange(R), lab] = 1.0
    dx, dyy, dg, dl, dout = up(dev, x), up(dev, y), up(dev, np.array([1.7])), dev.alloc(4), dev.alloc(4 * R * Cc)
    case(f"cross_entropy {R}x{Cc}")
    dev.cross_entropy(dl, dx, dyy, R, Cc)
    got = float(dev.download(dl, (1,))[0])
    assert abs(got - oracle.cross_entropy(x, y)) <= oracle.tolerance(Cc) * max(1.0, oracle.cross_entropy(x, y))
    dev.cross_entropy_bwd(dout, dx, dyy, dg, R, Cc)
    want = oracle.cross_entropy_bwd(x, y, float(np.float32(1.7)))
    assert oracle.normwise_error(down(dev, dout, (R, Cc)), want) <= oracle.tolerance(Cc)
    for b in (dx, dyy, dg, dl, dout):
        b.free()


# ---- conv backward ------------------------------------------------------------------


def _conv_bwd(dev, N, Ci, H, W, Co, KH, KW, st, pd, seed, x=None, w=None, g=None):
    Ho, Wo = (H + 2 * pd - KH) // st + 1, (W + 2 * pd - KW) // st + 1
    x = prng.normal(seed, (N, Ci, H, W)) if x is None else x
    w = prng.normal(seed + 1, (Co, Ci, KH, KW), 0, float(np.sqrt(2.0 / (Ci * KH * KW)))) if w is None else w
    g = prng.normal(seed + 2, (N, Co, Ho, Wo)) if g is None else g
    dx_, dw_, dg_ = up(dev, x), up(dev, w), up(dev, g)
    ddx, ddw = dev.alloc(4 * x.size), dev.alloc(4 * w.size)
    case(f"conv bwd N={N} Ci={Ci} {H}x{W} Co={Co} K={KH}x{KW} s={st} p={pd}")
    dev.conv2d_bwd_input(ddx, dg_, dw_, N, Ci, H, W, Co, Ho, Wo, KH, KW, st, pd)
    dev.conv2d_bwd_weight(ddw, dg_, dx_, N, Ci, H, W, Co, Ho, Wo, KH, KW, st, pd)
    got_dx, got_dw = down(dev, ddx, x.shape), down(dev, ddw, w.shape)
    for b in (dx_, dw_, dg_, ddx, ddw):
        b.free()
    return x, w, g, got_dx, got_dw


@pytest.mark.parametrize("tag,stride,pad", [("s1p1", 1, 1), ("s2p2", 2, 2)])
def test_conv_backward_golden(dev, tag, stride, pad):
    x, w, g = K[f"cbwd_{tag}_x"], K[f"cbwd_{tag}_w"], K[f"cbwd_{tag}_g"]
    N, Ci, H, W = x.shape
    Co, _, KH, KW = w.shape
    *_, got_dx, got_dw = _conv_bwd(dev, N, Ci, H, W, Co, KH, KW, stride, pad, 0, x, w, g)
    assert oracle.normwise_error(got_dx, K[f"cbwd_{tag}_dx"]) <= oracle.tolerance(Co * KH * KW)
    assert oracle.normwise_error(got_dw, K[f"cbwd_{tag}_dw"]) <= oracle.tolerance(N * g.shape[2] * g.shape[3])


@pytest.mark.parametrize("shape", [
    (2, 3, 8, 8, 4, 3, 3, 1, 0),       # test_grad_check.c
    (4, 3, 32, 32, 16, 5, 5, 1, 2),    # train_cifar10.c conv1 (C_out = 16: k-major dgrad needs C_in % 4)
    (4, 16, 16, 16, 32, 5, 5, 1, 2),   # train_cifar10.c conv2 (k-major dgrad)
    (2, 64, 14, 14, 128, 3, 3, 1, 1),  # 3x3 k-major dgrad
    (2, 5, 11, 9, 7, 3, 3, 2, 1),      # stride 2: direct dgrad
    (1, 4, 10, 12, 6, 3, 5, 1, 1),     # non-square filter: direct dgrad
    (1, 2, 6, 6, 3, 3, 3, 1, 3),       # pad > K - 1: direct dgrad
    (3, 8, 7, 7, 5, 1, 1, 1, 0),       # 1x1
    (2, 6, 16, 16, 8, 3, 3, 2, 1),     # stride 2, H_out * W_out % 4 == 0: direct-load wgrad
    (2, 20, 12, 12, 130, 3, 3, 1, 1),  # two channel tiles of 128, J = 180 (a partial column tile)
])
def test_conv_backward_shapes(dev, shape):
    N, Ci, H, W, Co, KH, KW, st, pd = shape
    x, w, g, got_dx, got_dw = _conv_bwd(dev, N, Ci, H, W, Co, KH, KW, st, pd, seed=800 + sum(shape))
    ref_dx = oracle.conv2d_bwd_input(f32(g), f32(w), x.shape, st, pd)
    ref_dw = oracle.conv2d_bwd_weight(f32(g), f32(x), w.shape, st, pd)
    assert oracle.normwise_error(got_dx, ref_dx) <= oracle.tolerance(Co * KH * KW)
    assert oracle.normwise_error(got_dw, ref_dw) <= oracle.tolerance(N * g.shape[2] * g.shape[3])


def test_conv_backward_config_size(dev):
    """The conv config (N32, 64->128, 56x56, 3x3, pad 1) through both
    backward kernels, checked by the adjoint identity on the full size and
    against the oracle on two images' worth of the weight gradient."""
    N, Ci, H, W, Co = 32, 64, 56, 56, 128
    x, w, g, got_dx, got_dw = _conv_bwd(dev, N, Ci, H, W, Co, 3, 3, 1, 1, seed=900)
    y = oracle.conv2d(f32(x), f32(w), 1, 1)
    lhs = float(np.sum(y * f32(g)))
    scale = float(np.sum(np.abs(y * f32(g))))
    assert abs(float(np.sum(f32(x) * got_dx)) - lhs) <= 1e-5 * scale
    assert abs(float(np.sum(f32(w) * got_dw)) - lhs) <= 1e-5 * scale
    ref_dx0 = oracle.conv2d_bwd_input(f32(g[:1]), f32(w), (1, Ci, H, W), 1, 1)
    assert oracle.normwise_error(got_dx[:1], ref_dx0) <= oracle.tolerance(Co * 9)


def test_conv_wgrad_deterministic(dev):
    N, Ci, H, W, Co = 8, 16, 20, 20, 32
    g = prng.normal(950, (N, Co, H, W))
    x = prng.normal(951, (N, Ci, H, W))
    dx_, dg_, ddw = up(dev, x), up(dev, g), dev.alloc(4 * Co * Ci * 9)
    case("conv wgrad determinism")
    outs = []
    for _ in range(3):
        dev.conv2d_bwd_weight(ddw, dg_, dx_, N, Ci, H, W, Co, H, W, 3, 3, 1, 1)
        outs.append(dev.download(ddw, (Co, Ci, 3, 3)))
    assert all(np.array_equal(outs[0], o) for o in outs[1:])
    for b in (dx_, dg_, ddw):
        b.free()


# ---- max pooling ----------------------------------------------------------------------


@pytest.mark.parametrize("tag,k,s", [("k3s2", 3, 2), ("k2s2", 2, 2)])
def test_maxpool_golden(dev, tag, k, s):
    x = K["pool_x"]
    N, Cc, H, W = x.shape
    g = K[f"pool_{tag}_g"]
    Ho, Wo = g.shape[2], g.shape[3]
    dx_, dg_, dout, ddx = up(dev, x), up(dev, g), dev.alloc(4 * N * Cc * Ho * Wo), dev.alloc(4 * x.size)
    case(f"maxpool golden {tag}")
    dev.maxpool2d(dout, dx_, N, Cc, H, W, k, s)
    np.testing.assert_array_equal(down(dev, dout, g.shape), K[f"pool_{tag}_out"].astype(np.float32))
    dev.maxpool2d_bwd(ddx, dg_, dx_, N, Cc, H, W, Ho, Wo, k, s)
    assert oracle.normwise_error(down(dev, ddx, x.shape), K[f"pool_{tag}_dx"]) <= 1e-6
    for b in (dx_, dg_, dout, ddx):
        b.free()


@pytest.mark.parametrize("shape", [(4, 16, 32, 32, 2, 2), (2, 3, 9, 9, 3, 1), (1, 1, 5, 5, 5, 1), (32, 64, 56, 56, 3, 2)])
def test_maxpool_shapes(dev, shape):
    N, Cc, H, W, k, s = shape
    Ho, Wo = (H - k) // s + 1, (W - k) // s + 1
    x = np.round(prng.normal(1000 + H, (N, Cc, H, W)) * 4) / 4  # ties
    g = prng.normal(1001 + H, (N, Cc, Ho, Wo))
    dx_, dg_, dout, ddx = up(dev, x), up(dev, g), dev.alloc(4 * N * Cc * Ho * Wo), dev.alloc(4 * x.size)
    case(f"maxpool {shape}")
    dev.maxpool2d(dout, dx_, N, Cc, H, W, k, s)
    np.testing.assert_array_equal(down(dev, dout, (N, Cc, Ho, Wo)), oracle.maxpool2d(f32(x), k, s))
    dev.maxpool2d_bwd(ddx, dg_, dx_, N, Cc, H, W, Ho, Wo, k, s)
    ref = oracle.maxpool2d_bwd(f32(g), f32(x), k, s)
    assert oracle.normwise_error(down(dev, ddx, x.shape), ref) <= 1e-6
    for b in (dx_, dg_, dout, ddx):
        b.free()


# ---- training graphs on the device executor ----------------------------------------

# longest reduction feeding any output of each graph (for the tolerance)
TRAIN_K = {"mlp": 784, "cnn": 4 * 32 * 32, "cnn_fused": 4 * 32 * 32, "gradcheck": 144, "ops": 8}


def _train_program(dev, name, flags=0):
    lib = graph_lib()
    t = graphs.build_training(lib, TRAIN_GRAPHS[name](lib))
    lib.lancius_graph_set_dtype(t.g, abi.DTYPE_FP32)
    sched = lib.lancius_ir_schedule(t.g)
    plan = lib.lancius_build_memory_plan(sched, t.g)
    prog = DeviceProgram(dev, t.g, sched, plan, flags)
    return lib, t, sched, plan, prog


@pytest.mark.parametrize("name", sorted(TRAIN_GRAPHS))
def test_training_graph_on_device(dev, name):
    lib, t, sched, plan, prog = _train_program(dev, name)
    feeds = train_feeds(t, TRAIN_SEEDS[name])
    case(f"training graph {name}: {prog.info()['launches']} launches")
    for inp in t.inputs:
        prog.upload(t.node(inp), np.asarray(feeds[inp], np.float32))
    prog.run()
    stored = "cnn" if name == "cnn_fused" else name
    for out in t.outputs:
        got = prog.download(t.node(out)).reshape(abi.node_shape(t.node(out)))
        err = oracle.normwise_error(got, T[f"{stored}_out_{out}"])
        assert err <= oracle.tolerance(TRAIN_K[name]), (name, out, err)
    prog.close()
    lib.lancius_memory_plan_destroy(plan)
    lib.lancius_schedule_destroy(sched)
    t.destroy()


def test_training_step_drop_in(dev):
    """lancius_schedule_execute_device on the MNIST training graph: host fp64
    inputs bound to runtime_data in, loss and gradients written back to
    runtime_data (the reference executor's contract)."""
    lib = graph_lib()
    t = graphs.build_training(lib, TRAIN_GRAPHS["mlp"](lib))
    feeds = train_feeds(t, TRAIN_SEEDS["mlp"])
    keep = []
    for inp in t.inputs:
        arr = np.ascontiguousarray(feeds[inp], dtype=np.float64)
        keep.append(arr)
        t.node(inp).contents.runtime_data = arr.ctypes.data_as(C.POINTER(C.c_double))
    sched = lib.lancius_ir_schedule(t.g)
    case("training step drop-in")
    rc = dev.lib.lancius_schedule_execute_device(sched, t.g, dev.ctx)
    assert rc == 0, dev.lib.lancius_hip_last_error()
    import ctypes.util

    libc = C.CDLL(ctypes.util.find_library("c"))
    for out in t.outputs:
        n = t.node(out)
        got = np.ctypeslib.as_array(n.contents.runtime_data, shape=(abi.node_elems(n),)).copy()
        assert oracle.normwise_error(got, T[f"mlp_out_{out}"].ravel()) <= oracle.tolerance(784), out
        libc.free(C.c_void_p(C.addressof(n.contents.runtime_data.contents)))
        n.contents.runtime_data = None
    for inp in t.inputs:
        t.node(inp).contents.runtime_data = None
    lib.lancius_schedule_destroy(sched)
    t.destroy()
