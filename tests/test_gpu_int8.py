"""The int8 path on the device (C ABI and the executor) against the oracle and
the compiled reference's golden outputs.

The int32 sums are exact and the quantizer runs in fp64 like the reference,
so int8 values must match bit for bit and every output equals the
reference's fp64 value rounded once to fp32 (normwise error <= 1e-6, the
fp32 rounding plus the fp32 epilogue).
"""
import ctypes as C
from pathlib import Path

import numpy as np
import pytest

import oracle
from lancius_amd import ACT_NONE, ACT_RELU, DEVICE_GRAPH, DeviceProgram, abi, graph_lib, graphs, prng
from tests.conftest import case

pytestmark = pytest.mark.gpu

K = np.load(Path(__file__).resolve().parent / "golden" / "kernels.npz")
TOL = 1e-6


def f64(a):
    return np.asarray(a, np.float32).astype(np.float64)


@pytest.mark.parametrize("n", [1, 7, 4096, 1_000_003])
def test_quantize_bit_exact(dev, n):
    x = prng.normal(70 + n % 13, (n,), std=3.0)
    dx, dq, ds = dev.upload(x), dev.alloc(n), dev.alloc(8)
    case(f"quantize_i8 n={n}")
    dev.quantize_i8(dq, ds, dx, n)
    q = dev.download(dq, (n,), np.int8)
    s = float(dev.download(ds, (1,), np.float64)[0])
    rq, rs = oracle.quantize_i8(f64(x))
    assert s == rs
    np.testing.assert_array_equal(q, rq)
    for b in (dx, dq, ds):
        b.free()


@pytest.mark.parametrize("top", [381.0, 127.0 / 8, 100.0])
def test_quantize_exact_halves(dev, top):
    """x / scale exactly k + 0.5 (scale = top / 127 is 3, 1/8 or 100/127):
    the reference rounds the fp64 quotient half away from zero, so a
    multiply by 1 / scale that lands a hair below the half must not decide
    these.  The remaining entries sit one float step either side of them."""
    sc = top / 127.0
    halves = np.array([(k + 0.5) * sc for k in range(-127, 127)], np.float64)
    x = np.concatenate([[top], halves.astype(np.float32), np.nextafter(halves.astype(np.float32), np.float32(np.inf)),
                        np.nextafter(halves.astype(np.float32), np.float32(-np.inf))]).astype(np.float32)
    n = x.size
    dx, dq, ds = dev.upload(x), dev.alloc(n), dev.alloc(8)
    case(f"quantize_i8 exact halves top={top}")
    dev.quantize_i8(dq, ds, dx, n)
    q = dev.download(dq, (n,), np.int8)
    rq, rs = oracle.quantize_i8(f64(x))
    assert float(dev.download(ds, (1,), np.float64)[0]) == rs
    np.testing.assert_array_equal(q, rq)
    for b in (dx, dq, ds):
        b.free()


def test_quantize_all_zero(dev):
    dx, dq, ds = dev.upload(np.zeros(100, np.float32)), dev.alloc(100), dev.alloc(8)
    case("quantize_i8 zeros")
    dev.quantize_i8(dq, ds, dx, 100)
    assert float(dev.download(ds, (1,), np.float64)[0]) == 1e-8
    assert not dev.download(dq, (100,), np.int8).any()
    for b in (dx, dq, ds):
        b.free()


def _gemm_i8(dev, a, bq, sb, bias=None, act=ACT_NONE, res=None):
    M, Kd = a.shape
    N = bq.shape[1]
    da, db, dc = dev.upload(a), dev.upload(bq), dev.alloc(4 * M * N)
    dbias = dev.upload(bias) if bias is not None else None
    dres = dev.upload(res) if res is not None else None
    case(f"gemm_i8 M={M} K={Kd} N={N}")
    dev.gemm_i8(dc, da, db, sb, M, Kd, N, bias=dbias, act=act, residual=dres)
    got = dev.download(dc, (M, N))
    for b in (da, db, dc, dbias, dres):
        if b is not None:
            b.free()
    return got


def test_gemm_i8_golden(dev):
    got = _gemm_i8(dev, K["i8mm_a"].astype(np.float32), K["i8mm_bq"], float(K["i8mm_scale_b"]))
    assert oracle.normwise_error(got, K["i8mm_out"]) <= TOL


@pytest.mark.parametrize("M,Kd,N", [(1, 1, 1), (64, 784, 128), (130, 70, 201), (257, 300, 129), (1024, 1024, 1024),
                                    (33, 4096, 50),
                                    # 256 x 256 tiles (one per CU or more): exact and ragged edges
                                    (4096, 128, 4096), (3900, 130, 3950)])
def test_gemm_i8_shapes(dev, M, Kd, N):
    a = prng.normal(80 + M, (M, Kd))
    bq = np.round(prng.uniform(81 + N, (Kd, N), -127.4, 127.4)).astype(np.int8)
    got = _gemm_i8(dev, a, bq, 0.0123)
    assert oracle.normwise_error(got, oracle.matmul_i8(f64(a), bq, 0.0123)) <= TOL


@pytest.mark.parametrize("M,Kd,N", [(96, 200, 72), (3850, 40, 4000)])
def test_gemm_i8_epilogue(dev, M, Kd, N):
    a = prng.normal(90, (M, Kd))
    bq = np.round(prng.uniform(91, (Kd, N), -127.4, 127.4)).astype(np.int8)
    bias, res = prng.normal(92, (N,)), prng.normal(93, (M, N))
    got = _gemm_i8(dev, a, bq, 0.004, bias=bias, act=ACT_RELU, res=res)
    ref = np.maximum(oracle.matmul_i8(f64(a), bq, 0.004) + f64(bias)[None, :], 0.0) + f64(res)
    assert oracle.normwise_error(got, ref) <= TOL


def test_gemm_i8_big_tiles_every_element(dev):
    """256 x 256 tiles (240 of them) over 11 k-tiles of 128: an odd count,
    ragged M and N; C starts as NaN, so an unwritten element fails."""
    M, Kd, N = 4000, 1400, 3790
    a = prng.normal(94, (M, Kd))
    bq = np.round(prng.uniform(95, (Kd, N), -127.4, 127.4)).astype(np.int8)
    da, db = dev.upload(a), dev.upload(bq)
    dc = dev.upload(np.full((M, N), np.nan, np.float32))
    case(f"gemm_i8 M={M} K={Kd} N={N} NaN-filled")
    dev.gemm_i8(dc, da, db, 0.0021, M, Kd, N)
    got = dev.download(dc, (M, N))
    for b in (da, db, dc):
        b.free()
    assert np.isfinite(got).all()
    # the oracle's quantizer, then the integer product through float64 BLAS:
    # every partial sum is an integer below 2^53, so it is exact in any order
    qa, sa = oracle.quantize_i8(f64(a).ravel())
    ref = (qa.reshape(M, Kd).astype(np.float64) @ bq.astype(np.float64)) * (sa * 0.0021)
    assert oracle.normwise_error(got, ref) <= TOL


@pytest.mark.parametrize("M,Kd,N", [(4096, 4096, 4096), (4000, 2000, 3790), (4096, 512, 4096)])
def test_gemm_i8_big_tiles_bit_exact(dev, M, Kd, N):
    """256 x 256 tiles over 32, 16 and 4 k-tiles (ragged M, N and K at the
    second).  C starts as NaN.  Every element must equal the exact integer
    product scaled in fp64 and rounded once to fp32, bit for bit."""
    a = prng.normal(120 + M, (M, Kd))
    bq = np.round(prng.uniform(121 + N, (Kd, N), -127.4, 127.4)).astype(np.int8)
    da, db = dev.upload(a), dev.upload(bq)
    dc = dev.upload(np.full((M, N), np.nan, np.float32))
    case(f"gemm_i8 M={M} K={Kd} N={N} NaN-filled, bits")
    dev.gemm_i8(dc, da, db, 0.0021, M, Kd, N)
    got = dev.download(dc, (M, N))
    for b in (da, db, dc):
        b.free()
    # integer partial sums below 2^53 are exact in float64 in any order
    qa, sa = oracle.quantize_i8(f64(a).ravel())
    ref = ((qa.reshape(M, Kd).astype(np.float64) @ bq.astype(np.float64)) * (sa * 0.0021)).astype(np.float32)
    np.testing.assert_array_equal(got, ref)


def test_gemm_i8_big_tiles_epilogue(dev):
    """The 256 x 256 kernel's staged epilogue: bias, ReLU and residual on
    ragged edges, with an even number of k-tiles."""
    M, Kd, N = 3850, 1000, 4000
    a = prng.normal(122, (M, Kd))
    bq = np.round(prng.uniform(123, (Kd, N), -127.4, 127.4)).astype(np.int8)
    bias, res = prng.normal(124, (N,)), prng.normal(125, (M, N))
    got = _gemm_i8(dev, a, bq, 0.004, bias=bias, act=ACT_RELU, res=res)
    ref = np.maximum(oracle.matmul_i8(f64(a), bq, 0.004) + f64(bias)[None, :], 0.0) + f64(res)
    assert np.isfinite(got).all()
    assert oracle.normwise_error(got, ref) <= TOL


@pytest.mark.parametrize("M,Kd,N", [(130, 70, 201), (4000, 1400, 3790), (33, 4096, 50), (4000, 2000, 3790)])
def test_gemm_i8_packed_weight_bit_identical(dev, M, Kd, N):
    """lancius_hip_i8_pack_weight once + lancius_hip_gemm_i8p_f32 gives the
    bits of lancius_hip_gemm_i8_f32 (which packs on every call)."""
    a = prng.normal(96 + M, (M, Kd))
    bq = np.round(prng.uniform(97 + N, (Kd, N), -127.4, 127.4)).astype(np.int8)
    bias = prng.normal(98, (N,))
    da, db, dbias = dev.upload(a), dev.upload(bq), dev.upload(bias)
    dpk = dev.alloc(dev.i8_packed_bytes(Kd, N))
    c1, c2 = dev.alloc(4 * M * N), dev.alloc(4 * M * N)
    case(f"gemm_i8p M={M} K={Kd} N={N}")
    dev.i8_pack_weight(dpk, db, Kd, N)
    dev.gemm_i8(c1, da, db, 0.0031, M, Kd, N, bias=dbias, act=ACT_RELU)
    for _ in range(2):
        dev.gemm_i8p(c2, da, dpk, 0.0031, M, Kd, N, bias=dbias, act=ACT_RELU)
        np.testing.assert_array_equal(dev.download(c2, (M, N)), dev.download(c1, (M, N)))
    for b in (da, db, dbias, dpk, c1, c2):
        b.free()


def _conv_i8(dev, x, wq, sw, stride, pad, act=ACT_NONE):
    N, Ci, H, W = x.shape
    Co, _, KH, KW = wq.shape
    Ho, Wo = (H + 2 * pad - KH) // stride + 1, (W + 2 * pad - KW) // stride + 1
    dx, dw, do = dev.upload(x.astype(np.float32)), dev.upload(wq), dev.alloc(4 * N * Co * Ho * Wo)
    case(f"conv2d_i8 N={N} Ci={Ci} {H}x{W} Co={Co} K={KH}x{KW} s={stride} p={pad}")
    dev.conv2d_i8(do, dx, dw, sw, None, N, Ci, H, W, Co, KH, KW, stride, pad, act)
    got = dev.download(do, (N, Co, Ho, Wo))
    for b in (dx, dw, do):
        b.free()
    return got


def test_conv_i8_golden(dev):
    for tag, act in (("i8conv", ACT_NONE), ("i8conv_relu", ACT_RELU)):
        got = _conv_i8(dev, K[f"{tag}_x"], K[f"{tag}_wq"], float(K[f"{tag}_scale_w"]), 1, 1, act)
        assert oracle.normwise_error(got, K[f"{tag}_out"]) <= TOL, tag
    got = _conv_i8(dev, K["i8k_xq"].astype(np.float64) * 0.01, K["i8k_wq"], 0.002, 2, 2)
    assert oracle.normwise_error(got, K["i8k_out"]) <= TOL


@pytest.mark.parametrize("shape", [(2, 3, 32, 32, 16, 5, 5, 1, 2), (4, 16, 16, 16, 32, 5, 5, 1, 2),
                                   (2, 64, 28, 28, 128, 3, 3, 1, 1), (1, 20, 13, 11, 7, 3, 3, 2, 0),
                                   (3, 8, 9, 9, 5, 1, 1, 1, 0), (1, 130, 7, 7, 33, 3, 3, 1, 1),
                                   # filter too large for the LDS-resident kernel: the staged implicit GEMM
                                   (1, 300, 9, 9, 40, 3, 3, 1, 1)])
def test_conv_i8_shapes(dev, shape):
    N, Ci, H, W, Co, KH, KW, st, pd = shape
    x = prng.normal(100 + sum(shape), (N, Ci, H, W))
    wq = np.round(prng.uniform(101 + sum(shape), (Co, Ci, KH, KW), -127.4, 127.4)).astype(np.int8)
    got = _conv_i8(dev, x, wq, 0.003, st, pd)
    assert oracle.normwise_error(got, oracle.conv2d_i8(f64(x), wq, 0.003, st, pd)) <= TOL


def test_conv_i8_bench_shape_bit_exact(dev):
    """The bench conv (N32, 64 -> 128, 56 x 56, 3 x 3, pad 1): 1568 tiles of
    128 x 64 pixels.  The output starts as NaN; every element must equal the
    exact integer sum over the quantized operands times scale_w * scale_x in
    fp64, rounded once to fp32, bit for bit."""
    N, Ci, H, W, Co = 32, 64, 56, 56, 128
    x = prng.normal(130, (N, Ci, H, W))
    wq = np.round(prng.uniform(131, (Co, Ci, 3, 3), -127.4, 127.4)).astype(np.int8)
    sw = 0.0017
    dx, dw = dev.upload(x.astype(np.float32)), dev.upload(wq)
    do = dev.upload(np.full((N, Co, H, W), np.nan, np.float32))
    case(f"conv2d_i8 N={N} Ci={Ci} {H}x{W} Co={Co} 3x3 p1 NaN-filled, bits")
    dev.conv2d_i8(do, dx, dw, sw, None, N, Ci, H, W, Co, 3, 3, 1, 1, ACT_NONE)
    got = dev.download(do, (N, Co, H, W))
    for b in (dx, dw, do):
        b.free()
    assert np.isfinite(got).all()
    qx, sx = oracle.quantize_i8(f64(x).ravel())
    xp = np.zeros((N, H + 2, W + 2, Ci))
    xp[:, 1:-1, 1:-1, :] = qx.reshape(N, Ci, H, W).transpose(0, 2, 3, 1)
    acc = np.zeros((N * H * W, Co))
    for kh in range(3):
        for kw in range(3):
            # integer sums below 2^53 are exact in float64 in any order
            acc += xp[:, kh:kh + H, kw:kw + W, :].reshape(-1, Ci) @ wq[:, :, kh, kw].astype(np.float64).T
    ref = (acc * (sw * sx)).astype(np.float32).reshape(N, H, W, Co).transpose(0, 3, 1, 2)
    np.testing.assert_array_equal(got, ref)


def _conv_i8_exact(x, wq, sw, stride, pad, bias=None, relu=False):
    """The exact int8 conv: integer sums over the quantized operands (exact
    in float64), times scale_w * scale_x in fp64, rounded once to fp32, then
    the fp32 bias add and ReLU of the kernel's epilogue."""
    N, Ci, H, W = x.shape
    Co, _, KH, KW = wq.shape
    Ho, Wo = (H + 2 * pad - KH) // stride + 1, (W + 2 * pad - KW) // stride + 1
    qx, sx = oracle.quantize_i8(f64(x).ravel())
    xp = np.zeros((N, H + 2 * pad, W + 2 * pad, Ci))
    xp[:, pad:pad + H, pad:pad + W, :] = qx.reshape(N, Ci, H, W).transpose(0, 2, 3, 1)
    acc = np.zeros((N * Ho * Wo, Co))
    for kh in range(KH):
        for kw in range(KW):
            win = xp[:, kh:kh + stride * (Ho - 1) + 1:stride, kw:kw + stride * (Wo - 1) + 1:stride, :]
            acc += win.reshape(-1, Ci) @ wq[:, :, kh, kw].astype(np.float64).T
    v = (acc * (sw * sx)).astype(np.float32)
    if bias is not None:
        v = v + bias.astype(np.float32)[None, :]
    if relu:
        v = np.where(v > 0, v, np.float32(0))
    return v.reshape(N, Ho, Wo, Co).transpose(0, 3, 1, 2)


# (N, Ci, H, W, Co, K, stride, pad): the LDS-resident kernel with 128-channel
# blocks (two of them for 200 channels), 64-channel blocks with 7 x 7 taps
# over 16 channels (two taps per k-step), stride 2, and 32-channel blocks.
EXACT = [(3, 64, 20, 20, 128, 3, 1, 1), (2, 32, 14, 14, 200, 3, 1, 1), (2, 16, 10, 10, 70, 7, 1, 3),
         (2, 48, 15, 17, 96, 3, 2, 1), (1, 20, 9, 9, 30, 5, 1, 2)]


@pytest.mark.parametrize("N,Ci,H,W,Co,Kk,stride,pad", EXACT)
def test_conv_i8_bit_exact_bias_relu(dev, N, Ci, H, W, Co, Kk, stride, pad):
    x = prng.normal(140 + Co, (N, Ci, H, W))
    wq = np.round(prng.uniform(141 + Co, (Co, Ci, Kk, Kk), -127.4, 127.4)).astype(np.int8)
    bias = prng.normal(142 + Co, (Co,), 0.0, 0.5)
    sw = 0.0023
    Ho, Wo = (H + 2 * pad - Kk) // stride + 1, (W + 2 * pad - Kk) // stride + 1
    dx, dw, db = dev.upload(x.astype(np.float32)), dev.upload(wq), dev.upload(bias.astype(np.float32))
    do = dev.upload(np.full((N, Co, Ho, Wo), np.nan, np.float32))
    case(f"conv2d_i8 N={N} Ci={Ci} {H}x{W} Co={Co} {Kk}x{Kk} s={stride} p={pad} bias+relu, bits")
    dev.conv2d_i8(do, dx, dw, sw, db, N, Ci, H, W, Co, Kk, Kk, stride, pad, ACT_RELU)
    got = dev.download(do, (N, Co, Ho, Wo))
    for b in (dx, dw, db, do):
        b.free()
    np.testing.assert_array_equal(got, _conv_i8_exact(x, wq, sw, stride, pad, bias, True))


# ---- through the device executor ------------------------------------------------------


def test_int8_conv_graph_on_device(dev):
    """lancius_quantize_graph + the executor: the filter uploads as int8, the
    image (also quantized by the pass, as in the reference) stays an fp32
    activation quantized by the conv itself."""
    lib = graph_lib()
    for tag, fuse in (("i8conv", False), ("i8conv_relu", True)):
        bg = graphs.BuiltGraph(lib, lib.lancius_graph_create())
        nx = graphs._inp(bg, "x", 2, 5, 9, 8)
        nw = graphs._inp(bg, "w", 6, 5, 3, 3)
        conv = lib.lancius_conv2d(bg.g, nx, nw, 1, 1)
        out = lib.lancius_relu(bg.g, conv) if fuse else conv
        if fuse:
            lib.lancius_optimize_fusion(bg.g)
        keep = [np.ascontiguousarray(K[f"{tag}_x"]), np.ascontiguousarray(K[f"{tag}_w"])]
        nx.contents.runtime_data = keep[0].ctypes.data_as(C.POINTER(C.c_double))
        nw.contents.runtime_data = keep[1].ctypes.data_as(C.POINTER(C.c_double))
        lib.lancius_quantize_graph(bg.g)
        wq = np.ctypeslib.as_array(nw.contents.runtime_data_int8, shape=(keep[1].size,)).copy()
        np.testing.assert_array_equal(wq.reshape(K[f"{tag}_wq"].shape), K[f"{tag}_wq"])
        lib.lancius_graph_set_dtype(bg.g, abi.DTYPE_FP32)
        assert nw.contents.dtype == abi.DTYPE_INT8  # quantized weights keep their dtype
        sched = lib.lancius_ir_schedule(bg.g)
        plan = lib.lancius_build_memory_plan(sched, bg.g)
        case(f"int8 conv graph {tag}")
        prog = DeviceProgram(dev, bg.g, sched, plan)
        prog.upload(nx, K[f"{tag}_x"].astype(np.float32))
        prog.upload(nw, wq)
        with pytest.raises(TypeError):
            prog.upload(nw, np.zeros(3, np.int32))
        prog.run()
        got = prog.download(out)
        assert oracle.normwise_error(got, K[f"{tag}_out"]) <= TOL, tag
        prog.close()
        lib.lancius_memory_plan_destroy(plan)
        lib.lancius_schedule_destroy(sched)
        nx.contents.runtime_data = None
        nw.contents.runtime_data = None
        bg.destroy()


def test_int8_matmul_drop_in(dev):
    """lancius_schedule_execute_device on a MATMUL whose B carries an int8
    copy and scale (lancius_scheduler.c:192-195): the int8 bytes upload, the
    result comes back to runtime_data."""
    lib = graph_lib()
    a, bq, sb = K["i8mm_a"], K["i8mm_bq"], float(K["i8mm_scale_b"])
    g = lib.lancius_graph_create()
    na, nb = lib.lancius_input(g, *a.shape), lib.lancius_input(g, *bq.shape)
    mm = lib.lancius_matmul(g, na, nb)
    keep = [np.ascontiguousarray(a), np.ascontiguousarray(bq.astype(np.float64) * sb), np.ascontiguousarray(bq)]
    na.contents.runtime_data = keep[0].ctypes.data_as(C.POINTER(C.c_double))
    nb.contents.runtime_data = keep[1].ctypes.data_as(C.POINTER(C.c_double))
    nb.contents.runtime_data_int8 = keep[2].ctypes.data_as(C.POINTER(C.c_int8))
    nb.contents.scale = sb
    sched = lib.lancius_ir_schedule(g)
    case("int8 matmul drop-in")
    rc = dev.lib.lancius_schedule_execute_device(sched, g, dev.ctx)
    assert rc == 0, dev.lib.lancius_hip_last_error()
    got = np.ctypeslib.as_array(mm.contents.runtime_data, shape=(a.shape[0] * bq.shape[1],)).copy()
    assert oracle.normwise_error(got, K["i8mm_out"].ravel()) <= TOL
    import ctypes.util

    libc = C.CDLL(ctypes.util.find_library("c"))
    libc.free(C.c_void_p(C.addressof(mm.contents.runtime_data.contents)))
    mm.contents.runtime_data = None
    na.contents.runtime_data = nb.contents.runtime_data = None
    nb.contents.runtime_data_int8 = None
    lib.lancius_schedule_destroy(sched)
    lib.lancius_graph_destroy(g)


def test_int8_matmul_program_repacks_changed_weights(dev):
    """A program keeps one packed copy of an int8 MATMUL weight.  A new
    upload, and a write through lancius_device_buffer, must both reach the
    next run."""
    lib = graph_lib()
    M, Kd, N = 96, 300, 130
    g = lib.lancius_graph_create()
    na, nb = lib.lancius_input(g, M, Kd), lib.lancius_input(g, Kd, N)
    mm = lib.lancius_matmul(g, na, nb)
    lib.lancius_graph_set_dtype(g, abi.DTYPE_FP32)
    nb.contents.dtype = abi.DTYPE_INT8
    nb.contents.scale = 0.004
    sched = lib.lancius_ir_schedule(g)
    case("int8 matmul program, weight re-uploaded")
    prog = DeviceProgram(dev, g, sched)
    a = prng.normal(99, (M, Kd))
    prog.upload(na, a)
    for seed, how in ((1, "upload"), (2, "upload"), (3, "buffer")):
        bq = np.round(prng.uniform(200 + seed, (Kd, N), -127.4, 127.4)).astype(np.int8)
        if how == "upload":
            prog.upload(nb, bq)
        else:
            dev.write(prog.buffer(nb), bq)
        prog.run()
        got = prog.download(mm).reshape(M, N)
        assert oracle.normwise_error(got, oracle.matmul_i8(f64(a), bq, 0.004)) <= TOL, (seed, how)
    prog.close()
    lib.lancius_schedule_destroy(sched)
    lib.lancius_graph_destroy(g)


def test_int8_matmul_program_weight_pointer_kept(dev):
    """The int8 weight's device address taken once, then written before
    each of several runs: every write must reach the product, whose kernel
    reads a packed copy of the weight."""
    lib = graph_lib()
    M, Kd, N = 96, 300, 130
    g = lib.lancius_graph_create()
    na, nb = lib.lancius_input(g, M, Kd), lib.lancius_input(g, Kd, N)
    mm = lib.lancius_matmul(g, na, nb)
    lib.lancius_graph_set_dtype(g, abi.DTYPE_FP32)
    nb.contents.dtype = abi.DTYPE_INT8
    nb.contents.scale = 0.004
    sched = lib.lancius_ir_schedule(g)
    case("int8 matmul program, weight written through a kept pointer")
    prog = DeviceProgram(dev, g, sched)
    a = prng.normal(98, (M, Kd))
    prog.upload(na, a)
    bptr = prog.buffer(nb)
    for seed in (11, 12, 13):
        bq = np.round(prng.uniform(200 + seed, (Kd, N), -127.4, 127.4)).astype(np.int8)
        dev.write(bptr, bq)
        prog.run()
        got = prog.download(mm).reshape(M, N)
        assert oracle.normwise_error(got, oracle.matmul_i8(f64(a), bq, 0.004)) <= TOL, seed
    prog.close()
    lib.lancius_schedule_destroy(sched)
    lib.lancius_graph_destroy(g)


def test_int8_matmul_program_graph_replay(dev):
    """An int8 MATMUL program run as a recorded graph (the quantizer's two
    launches and the product replayed): each replay takes a new A, whose
    scale differs, and is checked against the oracle, with eager int8 work
    on the same context in between."""
    lib = graph_lib()
    M, Kd, N = 200, 512, 260
    g = lib.lancius_graph_create()
    na, nb = lib.lancius_input(g, M, Kd), lib.lancius_input(g, Kd, N)
    mm = lib.lancius_matmul(g, na, nb)
    lib.lancius_graph_set_dtype(g, abi.DTYPE_FP32)
    nb.contents.dtype = abi.DTYPE_INT8
    nb.contents.scale = 0.004
    sched = lib.lancius_ir_schedule(g)
    case("int8 matmul program as a recorded graph")
    prog = DeviceProgram(dev, g, sched, flags=DEVICE_GRAPH)
    bq = np.round(prng.uniform(230, (Kd, N), -127.4, 127.4)).astype(np.int8)
    prog.upload(nb, bq)
    for rep in range(4):
        a = prng.normal(240 + rep, (M, Kd), std=1.0 + rep)
        prog.upload(na, a)
        prog.run()
        got = prog.download(mm).reshape(M, N)
        assert oracle.normwise_error(got, oracle.matmul_i8(f64(a), bq, 0.004)) <= TOL, rep
        x = prng.normal(250 + rep, (4096,))
        dx, dq, ds = dev.upload(x), dev.alloc(4096), dev.alloc(8)
        dev.quantize_i8(dq, ds, dx, 4096)
        np.testing.assert_array_equal(dev.download(dq, (4096,), np.int8), oracle.quantize_i8(f64(x))[0])
        for b in (dx, dq, ds):
            b.free()
    prog.close()
    lib.lancius_schedule_destroy(sched)
    lib.lancius_graph_destroy(g)
