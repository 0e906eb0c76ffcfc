"""Benchmark of the Lancius hot path on one MI355X.

Headline (its largest square case): one fp32 GEMM
C = A.B with M = N = K = 4096, A and B ~ N(0,1) (SplitMix64, seed 43), inputs
resident in HBM.  A step is one GEMM launch; `value` is GFLOP/s = 2MNK /
(seconds per step), timed with HIP events on the stream the kernel runs on.

The same JSON line carries:
  roofline      the GEMM against the fp32 MFMA peak (157.3 TFLOP/s)
  cpu_baseline  the reference's own graph MATMUL node (IKJ, one thread by
                construction, B/src/runtime/lancius_scheduler.c:222-234),
                compiled from source into oracle/_ref, timed on this host on
                a bounded row sample of the same product
  all_configs   every other BASELINE.json config measured in this run:
                GEMM 1024^3 / 2048^3 / 16x4096x4096, attention B8 H16 D64
                S512/S2048 causal/non-causal, conv 3x3 N32 64->128 56^2 +ReLU
                and its two backward convolutions, the MLP and transformer-block
                graphs through the device executor (forward latency), and the
                training steps (autodiff graphs) of the MNIST MLP and CIFAR CNN
                examples.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--quick] [--no-cpu]
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import platform
import shutil
import sys
import tempfile
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

from lancius_amd import (DEVICE_GRAPH, DEVICE_NO_CHAIN, Device, DeviceProgram, abi, device_count, graph_lib,  # noqa: E402
                         graphs, prng)

PEAK_FP32_MFMA = 157.3  # TFLOP/s, MI355X dense fp32 matrix
PEAK_HBM = 8000.0       # GB/s
PEAK_INT8_MFMA = 5000.0  # TOPS, MI355X dense int8 matrix
METRIC = "GFLOP/s + % of fp32 MFMA peak (GEMM/attn/conv); graph fwd latency ms"
TRAFFIC_FILE = ROOT / "profiles" / "traffic.json"
# Algorithmic flops of one training step (forward + every gradient):
# MNIST MLP B64: 3 GEMMs per layer (fwd, dX, dW) of 64x784x128 and 64x128x10
MLP_TRAIN_GFLOP = 3 * 2.0 * (64 * 784 * 128 + 64 * 128 * 10) / 1e9
# CIFAR CNN B32: 3 convolutions per conv layer (fwd, dgrad, wgrad) + 3 GEMMs per FC layer
CNN_TRAIN_GFLOP = 3 * 2.0 * (32 * 16 * 32 * 32 * 3 * 25 + 32 * 32 * 16 * 16 * 16 * 25
                             + 32 * 2048 * 120 + 32 * 120 * 10) / 1e9


def log(msg: str) -> None:
    sys.stderr.write(f"[bench] {msg}\n")
    sys.stderr.flush()


def time_steps(dev: Device, fn, steps: int, warmup: int, settle_ms: float = 40.0, info: dict | None = None) -> float:
    """Average ms per call of fn over `steps` calls, HIP events on the
    context stream, after `warmup` untimed calls and, with settle_ms > 0,
    enough further untimed calls for about settle_ms of GPU work (at most
    4000): the clock drops while the host prepares a case and settles again
    over tens of milliseconds of load (with at most 500, a 21 us case
    settled for 10 ms and timed about 10% slow).  info["settle_launches"]
    receives the number of those further calls."""
    for _ in range(warmup):
        fn()
    dev.synchronize()
    settled = 0
    if settle_ms > 0:
        dev.timer_start()
        fn()
        one = max(dev.timer_stop(), 1e-3)
        settled = 1 + min(4000, int(settle_ms / one))
        for _ in range(settled - 1):
            fn()
        dev.synchronize()
    if info is not None:
        info["settle_launches"] = settled
    dev.timer_start()
    for _ in range(steps):
        fn()
    ms = dev.timer_stop()
    dev.synchronize()
    return ms / steps


def gemm_case(dev, M, K, N, seed, steps, warmup, settle_ms=40.0, info=None):
    A = dev.upload(prng.normal(seed, (M, K)))
    B = dev.upload(prng.normal(seed + 1000, (K, N)))
    Cb = dev.alloc(M * N * 4)
    ms = time_steps(dev, lambda: dev.gemm(Cb, A, B, M, K, N), steps, warmup, settle_ms, info)
    for b in (A, B, Cb):
        b.free()
    flops = 2.0 * M * N * K
    nbytes = 4.0 * (M * K + K * N + M * N)
    return ms, flops, nbytes


def attention_case(dev, B, S, H, D, causal, seed, steps, warmup):
    shape = (B, S, H, D)
    q, k, v = (dev.upload(prng.normal(seed + i, shape)) for i in range(3))
    o = dev.alloc(int(np.prod(shape)) * 4)
    ms = time_steps(dev, lambda: dev.attention(o, q, k, v, B, S, H, D, causal=causal), steps, warmup)
    for b in (q, k, v, o):
        b.free()
    flops = 4.0 * B * H * D * (S * (S + 1) / 2 if causal else S * S)
    return ms, flops, 16.0 * B * S * H * D


def conv_case(dev, steps, warmup, packed=True):
    """The conv config + ReLU.  packed: the filter re-laid once
    (lancius_hip_conv2d_pack_weight, as the device executor does for an
    uploaded filter) and lancius_hip_conv2d_packed_f32 timed; otherwise
    lancius_hip_conv2d_f32, which re-lays the OIHW filter inside every call."""
    N, C_in, H, W, C_out = 32, 64, 56, 56, 128
    x = dev.upload(prng.normal(45, (N, C_in, H, W)))
    w = dev.upload(prng.normal(145, (C_out, C_in, 3, 3), std=float(np.sqrt(2.0 / (9 * C_in)))))
    o = dev.alloc(N * C_out * H * W * 4)
    bufs = [x, w, o]
    if packed:
        pk = dev.alloc(dev.conv2d_packed_bytes(C_out, C_in, 3, 3))
        bufs.append(pk)
        dev.conv2d_pack_weight(pk, w, C_out, C_in, 3, 3)
        ms = time_steps(dev, lambda: dev.conv2d_packed(o, x, pk, None, N, C_in, H, W, C_out, 3, 3, 1, 1, 1), steps,
                        warmup)
    else:
        ms = time_steps(dev, lambda: dev.conv2d(o, x, w, None, N, C_in, H, W, C_out, 3, 3, 1, 1, 1), steps, warmup)
    for b in bufs:
        b.free()
    flops = 2.0 * N * C_out * H * W * C_in * 9
    return ms, flops, 4.0 * (N * C_in * H * W + C_out * C_in * 9 + N * C_out * H * W)


def decode_cases(dev, steps, warmup) -> dict:
    """Decode-side family at LLM shapes: split-KV decode attention (HBM-bound:
    the K and V caches read once), GQA prefill with a history, RMSNorm, RoPE,
    SwiGLU."""
    out = {}
    B, Skv, Hq, Hkv, D = 16, 4096, 32, 8, 128
    q = dev.upload(prng.uniform(60, (B, Hq, D), -1.0, 1.0))
    k = dev.upload(prng.uniform(61, (B, Skv, Hkv, D), -1.0, 1.0))
    v = dev.upload(prng.uniform(62, (B, Skv, Hkv, D), -1.0, 1.0))
    o = dev.alloc(B * Hq * D * 4)
    t = time_steps(dev, lambda: dev.attention_decode(o, q, k, v, None, B, Skv, Hq, Hkv, D), steps, warmup)
    nb = 4.0 * (2 * B * Skv * Hkv * D + 2 * B * Hq * D)
    out[f"attention_decode_B{B}_kv{Skv}_Hq{Hq}_Hkv{Hkv}_D{D}"] = {
        "ms": round(t, 4), "GB/s": round(nb / t / 1e6, 1), "frac_hbm": round(nb / t / 1e6 / PEAK_HBM, 4)}
    for b in (q, k, v, o):
        b.free()
    for D in (64, 128):
        B, Sq, Skv, Hq, Hkv = 4, 1024, 2048, 32, 8
        q = dev.upload(prng.uniform(63, (B, Sq, Hq, D), -1.0, 1.0))
        k = dev.upload(prng.uniform(64, (B, Skv, Hkv, D), -1.0, 1.0))
        v = dev.upload(prng.uniform(65, (B, Skv, Hkv, D), -1.0, 1.0))
        o = dev.alloc(B * Sq * Hq * D * 4)
        t = time_steps(dev, lambda: dev.attention_gqa(o, q, k, v, B, Sq, Skv, Hq, Hkv, D, True), steps, warmup)
        # causal with a 1024-token history: query i sees 1024 + i + 1 keys
        flops = 4.0 * B * Hq * D * sum(Skv - Sq + i + 1 for i in range(Sq))
        out[f"attention_gqa_prefill_B{B}_q{Sq}_kv{Skv}_Hq{Hq}_Hkv{Hkv}_D{D}"] = {
            "ms": round(t, 4), "GFLOP/s": round(flops / t / 1e6, 1),
            "frac_fp32_mfma": round(flops / t / 1e9 / PEAK_FP32_MFMA, 4)}
        for b in (q, k, v, o):
            b.free()
    for D in (32, 128):  # the SDPA config at other head dims (same B, S, H)
        for causal in (True, False):
            name = f"attention_B8_H16_D{D}_S2048_{'causal' if causal else 'noncausal'}"
            t, f, _ = attention_case(dev, 8, 2048, 16, D, causal, 44, steps, warmup)
            out[name] = {"ms": round(t, 4), "GFLOP/s": round(f / t / 1e6, 1),
                         "frac_fp32_mfma": round(f / t / 1e9 / PEAK_FP32_MFMA, 4)}
    # one sequence, and four of S=768: grids too small to fill the CUs
    # with 128-query tiles (the 64-query kernel)
    for B, S, causal in ((1, 512, True), (1, 512, False), (4, 768, True)):
        t, f, _ = attention_case(dev, B, S, 16, 64, causal, 44, steps, warmup)
        out[f"attention_B{B}_H16_D64_S{S}_{'causal' if causal else 'noncausal'}"] = {
            "ms": round(t, 4), "GFLOP/s": round(f / t / 1e6, 1),
            "frac_fp32_mfma": round(f / t / 1e9 / PEAK_FP32_MFMA, 4)}
    rows, hid = 4096, 4096
    x = dev.upload(prng.normal(66, (rows, hid)))
    g = dev.upload(np.ones((hid,), np.float32))
    y = dev.alloc(rows * hid * 4)
    t = time_steps(dev, lambda: dev.rmsnorm(y, x, g, rows, hid), steps, warmup)
    nb = 8.0 * rows * hid
    out["rmsnorm_4096x4096"] = {"ms": round(t, 4), "GB/s": round(nb / t / 1e6, 1),
                                "frac_hbm": round(nb / t / 1e6 / PEAK_HBM, 4)}
    u = dev.upload(prng.normal(67, (rows, hid)))
    t = time_steps(dev, lambda: dev.swiglu(y, x, u, rows * hid), steps, warmup)
    u.free()
    nb = 12.0 * rows * hid
    out["swiglu_4096x4096"] = {"ms": round(t, 4), "GB/s": round(nb / t / 1e6, 1),
                               "frac_hbm": round(nb / t / 1e6 / PEAK_HBM, 4)}
    # q and k of a 4096-token, 32-head, 128-dim layer (2 x 64 MiB)
    S, H, hd = 4096, 32, 128
    t = time_steps(dev, lambda: dev.rope(y, x, 2, 1, S, H // 2, hd), steps, warmup)
    nb = 8.0 * 2 * S * (H // 2) * hd
    out["rope_q_k_S4096_H16_hd128"] = {"ms": round(t, 4), "GB/s": round(nb / t / 1e6, 1),
                                       "frac_hbm": round(nb / t / 1e6 / PEAK_HBM, 4)}
    for b in (x, g, y):
        b.free()
    return out


LOAD_LAYERS, LOAD_DIM = 4, 4096  # stored weights: 4 x 4096 x 4096 fp64 = 512 MiB in a v10 file


def write_load_models(tmpdir: Path) -> tuple[Path, Path]:
    """An MLP whose weights are stored in the file, saved as v10 (fp64) and as
    a v2 container with fp32 weights."""
    lib = graph_lib()
    bg = graphs.BuiltGraph(lib, lib.lancius_graph_create())
    h = graphs._inp(bg, "x", 64, LOAD_DIM)
    for i in range(LOAD_LAYERS):
        w = graphs._inp(bg, f"W{i}", LOAD_DIM, LOAD_DIM)
        graphs._bind(bg, f"W{i}", prng.normal(800 + i, (LOAD_DIM, LOAD_DIM), 0, 0.02))
        h = lib.lancius_matmul(bg.g, h, w)
    v10, v2 = tmpdir / "mlp.lancius", tmpdir / "mlp_fp32.lancius2"
    lib.lancius_graph_save(bg.g, str(v10).encode())
    if lib.lancius_graph_save_v2(bg.g, str(v2).encode(), abi.DTYPE_FP32) != 0:
        raise RuntimeError("lancius_graph_save_v2 failed")
    bg.destroy()
    return v10, v2


def model_load_cases(dev, v10: Path, v2: Path) -> dict:
    """File -> HBM arena: lancius_graph_load_mapped (parse; the v2 CRC-32 over
    the whole file), program creation, lancius_device_upload_weights (pread
    into pinned buffers, H2D copies, fp64 -> fp32 on the device).  The files
    were just written, so reads come from the page cache; best of 3."""
    lib = graph_lib()
    out = {}
    for tag, path in (("v10_fp64", v10), ("v2_fp32", v2)):
        best = None
        for _ in range(3):
            t0 = time.perf_counter()
            wm = abi.WeightMap()
            g = lib.lancius_graph_load_mapped(str(path).encode(), C.byref(wm))
            t1 = time.perf_counter()
            lib.lancius_graph_set_dtype(g, abi.DTYPE_FP32)
            sched = lib.lancius_ir_schedule(g)
            plan = lib.lancius_build_memory_plan(sched, g)
            prog = DeviceProgram(dev, g, sched, plan)
            t2 = time.perf_counter()
            prog.upload_weights(path, wm)
            t3 = time.perf_counter()
            times = (t1 - t0, t2 - t1, t3 - t2, t3 - t0)
            if best is None or times[3] < best[3]:
                best = times
            prog.close()
            lib.lancius_memory_plan_destroy(plan)
            lib.lancius_schedule_destroy(sched)
            lib.lancius_weight_map_free(C.byref(wm))
            lib.lancius_graph_destroy(g)
        size = path.stat().st_size
        out[f"model_load_{tag}_{LOAD_LAYERS}x{LOAD_DIM}x{LOAD_DIM}"] = {
            "file_MiB": round(size / 2 ** 20, 1), "parse_ms": round(best[0] * 1e3, 2),
            "program_ms": round(best[1] * 1e3, 2), "upload_ms": round(best[2] * 1e3, 2),
            "total_ms": round(best[3] * 1e3, 2), "file_GB/s": round(size / best[3] / 1e9, 2),
            "upload_GB/s": round(size / best[2] / 1e9, 2)}
    return out


def cpu_model_load(ref, v10: Path) -> dict:
    """The reference's lancius_graph_load on the same v10 file (fread into
    malloc'd fp64 buffers), page cache warm, best of 3."""
    import ctypes.util

    libc = C.CDLL(ctypes.util.find_library("c"))
    best = None
    for _ in range(3):
        t0 = time.perf_counter()
        g = ref.lancius_graph_load(str(v10).encode())
        dt = time.perf_counter() - t0
        if not g:
            raise RuntimeError("reference lancius_graph_load failed")
        best = dt if best is None else min(best, dt)
        for i in range(g.contents.node_count):  # its graph_destroy leaves the weights to the caller
            n = g.contents.nodes[i]
            if n.contents.runtime_data:
                libc.free(C.c_void_p(C.addressof(n.contents.runtime_data.contents)))
                n.contents.runtime_data = None
        ref.lancius_graph_destroy(g)
    size = v10.stat().st_size
    return {"ms": round(best * 1e3, 2), "GB/s": round(size / best / 1e9, 2), "file_MiB": round(size / 2 ** 20, 1),
            "note": "reference lancius_graph_load (lancius_serialize.c:65-259) into host fp64, page cache warm"}


def int8_cases(dev, steps, warmup) -> dict:
    """The int8 path at the headline GEMM and conv shapes: one call = dynamic
    per-tensor quantization of the fp32 activation + int8 MFMA product with
    int32 accumulation, fp32 out.  TOPS counts 2MNK.  The GEMM's int8 weight
    is packed once (lancius_hip_i8_pack_weight, as the device executor keeps
    it per weight); the call that re-lays it every time is reported beside."""
    out = {}
    n = 4096
    a = dev.upload(prng.normal(43, (n, n)))
    b = dev.upload(np.round(prng.uniform(1043, (n, n), -127.4, 127.4)).astype(np.int8))
    c = dev.alloc(n * n * 4)
    pk = dev.alloc(dev.i8_packed_bytes(n, n))
    dev.i8_pack_weight(pk, b, n, n)
    ops = 2.0 * n ** 3
    t = time_steps(dev, lambda: dev.gemm_i8p(c, a, pk, 0.01, n, n, n), steps, warmup)
    t_repack = time_steps(dev, lambda: dev.gemm_i8(c, a, b, 0.01, n, n, n), steps, warmup)
    out["gemm_i8_4096"] = {"ms": round(t, 4), "TOPS": round(ops / t / 1e9, 1),
                           "frac_int8_mfma": round(ops / t / 1e9 / PEAK_INT8_MFMA, 4),
                           "ms_repacking_B_each_call": round(t_repack, 4),
                           "note": "quantizes A (fp32 -> int8) each call; B packed once per weight"}
    for buf in (a, b, c, pk):
        buf.free()
    N, C_in, H, W, C_out = 32, 64, 56, 56, 128
    x = dev.upload(prng.normal(45, (N, C_in, H, W)))
    w = dev.upload(np.round(prng.uniform(145, (C_out, C_in, 3, 3), -127.4, 127.4)).astype(np.int8))
    o = dev.alloc(N * C_out * H * W * 4)
    t = time_steps(dev, lambda: dev.conv2d_i8(o, x, w, 0.001, None, N, C_in, H, W, C_out, 3, 3, 1, 1, 1), steps,
                   warmup)
    ops = 2.0 * N * C_out * H * W * C_in * 9
    # 14.8 G ops over >= 77 MB (fp32 activation in, fp32 output out, int8
    # filter) is ~190 ops per byte, below the int8 MFMA ridge (5.0 P / 8 TB/s
    # = 625): HBM is this call's roofline, so both fractions are reported.
    nbytes = 4.0 * (N * C_in * H * W + N * C_out * H * W) + C_out * C_in * 9
    out["conv3x3_N32_64to128_56x56_relu_i8"] = {"ms": round(t, 4), "TOPS": round(ops / t / 1e9, 1),
                                                "frac_int8_mfma": round(ops / t / 1e9 / PEAK_INT8_MFMA, 4),
                                                "GB/s": round(nbytes / t / 1e6, 1),
                                                "frac_hbm": round(nbytes / t / 1e6 / PEAK_HBM, 4),
                                                "bound": "hbm"}
    for buf in (x, w, o):
        buf.free()
    return out


def conv_bwd_cases(dev, steps, warmup) -> dict:
    """Input and weight gradients of the conv config (the two backward
    convolutions of a training step); same 2*N*C_out*H*W*C_in*9 flops each."""
    N, C_in, H, W, C_out = 32, 64, 56, 56, 128
    x = dev.upload(prng.normal(50, (N, C_in, H, W)))
    w = dev.upload(prng.normal(150, (C_out, C_in, 3, 3), std=float(np.sqrt(2.0 / (9 * C_in)))))
    g = dev.upload(prng.normal(250, (N, C_out, H, W)))
    dx, dw = dev.alloc(N * C_in * H * W * 4), dev.alloc(C_out * C_in * 9 * 4)
    flops = 2.0 * N * C_out * H * W * C_in * 9
    out = {}
    t = time_steps(dev, lambda: dev.conv2d_bwd_input(dx, g, w, N, C_in, H, W, C_out, H, W, 3, 3, 1, 1), steps, warmup)
    out["conv3x3_N32_64to128_56x56_bwd_input"] = {"ms": round(t, 4), "GFLOP/s": round(flops / t / 1e6, 1),
                                                  "frac_fp32_mfma": round(flops / t / 1e9 / PEAK_FP32_MFMA, 4)}
    t = time_steps(dev, lambda: dev.conv2d_bwd_weight(dw, g, x, N, C_in, H, W, C_out, H, W, 3, 3, 1, 1), steps,
                   warmup)
    out["conv3x3_N32_64to128_56x56_bwd_weight"] = {"ms": round(t, 4), "GFLOP/s": round(flops / t / 1e6, 1),
                                                   "frac_fp32_mfma": round(flops / t / 1e9 / PEAK_FP32_MFMA, 4)}
    for b in (x, w, g, dx, dw):
        b.free()
    return out


def train_feeds(t, seed: int) -> dict:
    """Synthetic training-step inputs: one-hot Y, He-scaled conv weights,
    N(0, 0.05) matrices and biases, N(0, 1) data."""
    feeds = {}
    for i, name in enumerate(t.inputs):
        shape = abi.node_shape(t.node(name))
        if name == "Y":
            lab = (prng.uniform(seed + i, (shape[0],), 0.0, 1.0) * shape[1]).astype(np.int64) % shape[1]
            y = np.zeros(shape, np.float32)
            y[np.arange(shape[0]), lab] = 1.0
            feeds[name] = y
        elif name.startswith("W") and len(shape) == 4:
            feeds[name] = prng.normal(seed + i, shape, 0.0, float(np.sqrt(2.0 / np.prod(shape[1:]))))
        elif name.startswith(("W", "b")):
            feeds[name] = prng.normal(seed + i, shape, 0.0, 0.05)
        else:
            feeds[name] = prng.normal(seed + i, shape)
    return feeds


def train_case(dev, fwd_builder, steps, warmup, flags=0):
    """One training step = the whole autodiff graph (forward, loss, every
    gradient) through the device executor."""
    lib = graph_lib()
    t = graphs.build_training(lib, fwd_builder(lib))
    lib.lancius_graph_set_dtype(t.g, abi.DTYPE_FP32)
    sched = lib.lancius_ir_schedule(t.g)
    plan = lib.lancius_build_memory_plan(sched, t.g)
    prog = DeviceProgram(dev, t.g, sched, plan, flags)
    feeds = train_feeds(t, 77)
    for name in t.inputs:
        prog.upload(t.node(name), feeds[name])
    ms = time_steps(dev, prog.run, steps, warmup)
    info = prog.info()
    prog.close()
    lib.lancius_memory_plan_destroy(plan)
    lib.lancius_schedule_destroy(sched)
    t.destroy()
    return ms, info


def rowop_cases(dev, steps, warmup) -> dict:
    """Memory-bound kernels at the transformer block's shapes; GB/s counts
    each tensor read and written once."""
    out = {}
    rows, hid = 4096, 1024
    x = dev.upload(prng.normal(47, (rows, hid)))
    g = dev.upload(np.ones((hid,), np.float32))
    b = dev.upload(np.zeros((hid,), np.float32))
    y = dev.alloc(rows * hid * 4)
    t = time_steps(dev, lambda: dev.layernorm(y, x, g, b, rows, hid), steps, warmup)
    nb = 8.0 * rows * hid
    out["layernorm_4096x1024"] = {"ms": round(t, 4), "GB/s": round(nb / t / 1e6, 1),
                                  "frac_hbm": round(nb / t / 1e6 / PEAK_HBM, 4)}
    t = time_steps(dev, lambda: dev.softmax(y, None, x, rows, hid), steps, warmup)
    out["softmax_4096x1024"] = {"ms": round(t, 4), "GB/s": round(nb / t / 1e6, 1),
                                "frac_hbm": round(nb / t / 1e6 / PEAK_HBM, 4)}
    for buf in (x, g, b, y):
        buf.free()
    # HBM-sized rows (256 MiB in, 256 MiB out: past the 256 MB MALL)
    rows, hid = 16384, 4096
    x = dev.upload(prng.normal(46, (rows, hid)))
    g = dev.upload(np.ones((hid,), np.float32))
    b = dev.upload(np.zeros((hid,), np.float32))
    y = dev.alloc(rows * hid * 4)
    nb = 8.0 * rows * hid
    for name, fn in (("layernorm", lambda: dev.layernorm(y, x, g, b, rows, hid)),
                     ("softmax", lambda: dev.softmax(y, None, x, rows, hid)),
                     ("rmsnorm", lambda: dev.rmsnorm(y, x, g, rows, hid))):
        t = time_steps(dev, fn, steps, warmup)
        out[f"{name}_{rows}x{hid}"] = {"ms": round(t, 4), "GB/s": round(nb / t / 1e6, 1),
                                       "frac_hbm": round(nb / t / 1e6 / PEAK_HBM, 4)}
    n = 4096 * 4096
    u = dev.upload(prng.normal(48, (n,)))
    v = dev.upload(prng.normal(49, (n,)))
    w = dev.alloc(n * 4)
    t = time_steps(dev, lambda: dev.gelu(w, u, n), steps, warmup)
    out["gelu_4096x4096"] = {"ms": round(t, 4), "GB/s": round(8.0 * n / t / 1e6, 1),
                             "frac_hbm": round(8.0 * n / t / 1e6 / PEAK_HBM, 4)}
    t = time_steps(dev, lambda: dev.add(w, u, v, n), steps, warmup)
    out["add_4096x4096"] = {"ms": round(t, 4), "GB/s": round(12.0 * n / t / 1e6, 1),
                            "frac_hbm": round(12.0 * n / t / 1e6 / PEAK_HBM, 4)}
    for buf in (x, g, b, y, u, v, w):
        buf.free()
    return out


def bridge_case(dev, n=4096) -> dict:
    """kernel_matmul_f32 (host pointers): includes both host->device copies and
    the copy back, so it is PCIe-bound; never the headline."""
    a = prng.normal(43, (n, n))
    bm = prng.normal(1043, (n, n))
    c = np.empty((n, n), np.float32)
    vp = C.c_void_p
    dev.lib.kernel_matmul_f32(c.ctypes.data_as(vp), a.ctypes.data_as(vp), bm.ctypes.data_as(vp), n, n, n)
    t0 = time.perf_counter()
    reps = 3
    for _ in range(reps):
        dev.lib.kernel_matmul_f32(c.ctypes.data_as(vp), a.ctypes.data_as(vp), bm.ctypes.data_as(vp), n, n, n)
    dt = (time.perf_counter() - t0) / reps
    return {"ms": round(dt * 1e3, 3), "GFLOP/s": round(2.0 * n ** 3 / dt / 1e9, 1),
            "note": "host-pointer bridge, PCIe copies of A, B and C included (wall clock)"}


def basis_case(dev, steps, warmup) -> dict:
    """The MLP as a BASIS static graph (include/basis/stage6_ir/graph.h):
    x . W1 + b1 -> tanh -> . W2 + b2 -> relu through lancius_basis_program_*
    (one fused two-layer launch)."""
    from lancius_amd.basis import Graph, Program

    g = Graph(graph_lib())
    x, w1, b1 = g.input("x", 64, 784), g.input("W1", 784, 256), g.input("b1", 1, 256)
    h = g.tanh(g.broadcast_add(g.matmul(x, w1), b1))
    w2, b2 = g.input("W2", 256, 10), g.input("b2", 1, 10)
    g.relu(g.broadcast_add(g.matmul(h, w2), b2))
    prog = Program(dev, g)
    for i, seed in ((x, 42), (w1, 142), (b1, 242), (w2, 342), (b2, 442)):
        n = g.node(i)
        prog.upload(i, prng.normal(seed, (n.rows, n.cols), 0, 0.02 if i != x else 1.0))
    t = time_steps(dev, prog.run, steps, warmup)
    info = prog.info()
    prog.close()
    g.close()
    return {"fwd_latency_ms": round(t, 4), "launches": info["launches"], "GFLOP/s": round(26.02e6 / t / 1e6, 1),
            "arena_KiB": round(info["arena_bytes"] / 1024, 1)}


def graph_case(dev, bg, feeds, steps, warmup, flags=0):
    lib = graph_lib()
    lib.lancius_graph_set_dtype(bg.g, abi.DTYPE_FP32)
    sched = lib.lancius_ir_schedule(bg.g)
    plan = lib.lancius_build_memory_plan(sched, bg.g)
    prog = DeviceProgram(dev, bg.g, sched, plan, flags)
    for name in bg.inputs:
        prog.upload(bg.node(name), feeds[name])
    ms = time_steps(dev, prog.run, steps, warmup)
    info = prog.info()
    prog.close()
    lib.lancius_memory_plan_destroy(plan)
    lib.lancius_schedule_destroy(sched)
    return ms, info


def cpu_baseline(M, K, N, target_s: float = 12.0) -> dict | None:
    """The reference graph MATMUL node on a row sample of the headline GEMM."""
    try:
        import oracle
    except Exception as e:  # pragma: no cover - reported, not fatal
        log(f"cpu baseline unavailable: {e}")
        return None
    ref = oracle.ref_lib()
    kind = "reference"
    a_full = prng.normal(43, (M, K)).astype(np.float64)
    b = np.ascontiguousarray(prng.normal(1043, (K, N)).astype(np.float64))

    def run(rows: int) -> float:
        a = np.ascontiguousarray(a_full[:rows])
        if ref is not None:
            g = ref.lancius_graph_create()
            na, nb = ref.lancius_input(g, rows, K), ref.lancius_input(g, K, N)
            ref.lancius_matmul(g, na, nb)
            na.contents.runtime_data = a.ctypes.data_as(C.POINTER(C.c_double))
            nb.contents.runtime_data = b.ctypes.data_as(C.POINTER(C.c_double))
            sched = ref.lancius_ir_schedule(g)
            arena = ref.lancius_arena_create(rows * N * 8 + (1 << 20))
            t0 = time.perf_counter()
            ref.lancius_schedule_execute(sched, arena)
            dt = time.perf_counter() - t0
            na.contents.runtime_data = None
            nb.contents.runtime_data = None
            ref.lancius_schedule_destroy(sched)
            ref.lancius_arena_destroy(arena)
            ref.lancius_graph_destroy(g)
            return dt
        oracle.set_threads(1)
        t0 = time.perf_counter()
        oracle.matmul(a, b, rows=(0, rows))
        return time.perf_counter() - t0

    if ref is None:
        kind = "port"
    probe_rows = 32
    dt = run(probe_rows)
    rows = int(min(M, max(probe_rows, probe_rows * target_s / max(dt, 1e-6))))
    rows = max(probe_rows, (rows // 32) * 32)
    dt = run(rows)
    gflops = 2.0 * rows * K * N / dt / 1e9
    cpu = platform.processor() or ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    other = {}
    if ref is not None:
        other.update(cpu_config_baselines(ref))
        other.update(cpu_next_row_baselines(ref))
        for name, builder in (("train_step_mnist_mlp_B64_784x128x10", lambda l: graphs.build_mlp_ce(l)),
                              ("train_step_cifar_cnn_B32", lambda l: graphs.build_cnn_ce(l, batch=32))):
            other[name] = {"step_latency_ms": round(cpu_train_step_ms(ref, builder), 3),
                           "note": "reference scratch-arena executor (lancius_schedule_execute), its own "
                                   "OpenMP threading, median of 3"}
    return {"value": round(gflops, 3), "unit": "GFLOP/s", "cores": 1, "kind": kind, "other_configs": other,
            "sample": f"rows 0-{rows - 1} of the {M}x{K}x{N} fp64 product through the "
                      f"{'reference' if kind == 'reference' else 'oracle'} graph MATMUL node (IKJ, 1 thread), "
                      f"{dt:.1f} s on {cpu} ({os.cpu_count()} logical CPUs visible)"}


def _omp_threads() -> int:
    """OpenMP threads the reference's parallel kernels run with here (the
    reference library and this process share one libgomp)."""
    try:
        return int(C.CDLL("libgomp.so.1").omp_get_max_threads())
    except OSError:
        return int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))


def _ref_graph_ms(ref, bg, feeds: dict, reps: int) -> float:
    """Median wall time of lancius_schedule_execute (the reference's scratch
    arena executor, B/src/runtime/lancius_scheduler.c:311-362) on a graph the
    reference library built, fresh intermediates each run."""
    keep = {k: np.ascontiguousarray(v, dtype=np.float64) for k, v in feeds.items()}
    for name in bg.inputs:
        bg.node(name).contents.runtime_data = keep[name].ctypes.data_as(C.POINTER(C.c_double))
    sched = ref.lancius_ir_schedule(bg.g)
    arena = ref.lancius_arena_create(512 << 20)
    times = []
    for _ in range(reps):
        g = bg.g.contents
        for i in range(g.node_count):
            n = g.nodes[i]
            if n.contents.op not in (abi.OP["INPUT"], abi.OP["CONST"]):
                n.contents.runtime_data = None
        t0 = time.perf_counter()
        ref.lancius_schedule_execute(sched, arena)
        times.append(time.perf_counter() - t0)
        ref.lancius_arena_reset(arena)
    ref.lancius_arena_destroy(arena)
    ref.lancius_schedule_destroy(sched)
    for name in bg.inputs:
        bg.node(name).contents.runtime_data = None
    return sorted(times)[len(times) // 2] * 1e3


def cpu_config_baselines(ref) -> dict:
    """The reference's own CPU path for every other config, on this host:
    graph MATMUL nodes (one thread by construction, lancius_scheduler.c:226-233),
    kernel_attention and kernel_conv2d_relu_fwd (OpenMP, all threads this
    process has), and the MLP and transformer-block graphs through the
    reference's executor.  Sizes that would take tens of seconds run on a
    stated sample; the extrapolation is stated with them."""
    threads = _omp_threads()
    D = C.POINTER(C.c_double)
    out = {}
    for name, (m, k, n) in (("gemm_1024", (1024, 1024, 1024)), ("gemm_2048", (2048, 2048, 2048)),
                            ("gemm_16x4096x4096", (16, 4096, 4096))):
        log(f"cpu {name}")
        bg = graphs.BuiltGraph(ref, ref.lancius_graph_create())
        a, b = bg.nodes["a"], bg.nodes["b"] = ref.lancius_input(bg.g, m, k), ref.lancius_input(bg.g, k, n)
        bg.inputs = ["a", "b"]
        ref.lancius_matmul(bg.g, a, b)
        ms = _ref_graph_ms(ref, bg, {"a": prng.normal(43, (m, k)), "b": prng.normal(1043, (k, n))},
                           1 if m * n * k >= 1 << 33 else 3)
        bg.destroy()
        out[name] = {"ms": round(ms, 2), "GFLOP/s": round(2.0 * m * n * k / ms / 1e6, 3), "cores": 1,
                     "note": "reference graph MATMUL node (IKJ, one thread), whole product"}
    for S in (512, 2048):
        log(f"cpu attention S={S}")
        B, H, Dh = 8, 16, 64
        seqs = B if S == 512 else 1
        q, k, v = (np.ascontiguousarray(prng.normal(44 + j, (seqs, S, H, Dh)), dtype=np.float64) for j in range(3))
        o = np.zeros_like(q)
        t0 = time.perf_counter()
        for b in range(seqs):
            ref.kernel_attention(o[b].ctypes.data_as(D), q[b].ctypes.data_as(D), k[b].ctypes.data_as(D),
                                 v[b].ctypes.data_as(D), S, H, Dh)
        dt = (time.perf_counter() - t0) * B / seqs
        flops = 4.0 * B * H * Dh * S * (S + 1) / 2
        out[f"attention_B8_H16_D64_S{S}_causal"] = {
            "ms": round(dt * 1e3, 1), "GFLOP/s": round(flops / dt / 1e9, 3), "cores": threads,
            "note": ("kernel_attention (causal; masked keys still computed, so the non-causal variant, "
                     "which has no reference kernel, costs the same), one call per sequence, "
                     + ("all 8 sequences" if seqs == B else "1 of the 8 sequences timed, x8"))}
    log("cpu conv")
    x = np.ascontiguousarray(prng.normal(45, (32, 64, 56, 56)), dtype=np.float64)
    w = np.ascontiguousarray(prng.normal(145, (128, 64, 3, 3), std=float(np.sqrt(2.0 / 576))), dtype=np.float64)
    y = np.zeros((32, 128, 56, 56))
    t0 = time.perf_counter()
    ref.kernel_conv2d_relu_fwd(y.ctypes.data_as(D), x.ctypes.data_as(D), w.ctypes.data_as(D), 32, 64, 56, 56, 128,
                               3, 3, 1, 1)
    dt = time.perf_counter() - t0
    out["conv3x3_N32_64to128_56x56_relu"] = {
        "ms": round(dt * 1e3, 1), "GFLOP/s": round(2.0 * 32 * 128 * 56 * 56 * 64 * 9 / dt / 1e9, 3),
        "cores": threads, "note": "kernel_conv2d_relu_fwd, whole batch"}
    log("cpu mlp graph")
    bg = graphs.build_mlp(ref)
    feeds = {"x": prng.uniform(1, (64, 784), -1.0, 1.0), "W1": prng.normal(2, (784, 256), 0, 0.02),
             "b1": np.zeros((1, 256)), "W2": prng.normal(3, (256, 10), 0, 0.02), "b2": np.zeros((1, 10))}
    ms = _ref_graph_ms(ref, bg, feeds, 7)
    bg.destroy()
    out["mlp_graph_64x784x256x10"] = {"fwd_latency_ms": round(ms, 3), "cores": threads,
                                      "note": "reference executor on the reference-built graph, median of 7"}
    log("cpu transformer block (one sequence)")
    bg = graphs.build_block(ref, batch=1)
    feeds = {}
    for i, name in enumerate(bg.inputs):
        shape = abi.node_shape(bg.node(name))
        feeds[name] = (prng.normal(1000 + i, shape) if name.startswith("x")
                       else 1.0 + prng.normal(1000 + i, shape, 0, 0.02) if name in ("g1", "g2")
                       else prng.normal(1000 + i, shape, 0, 0.02))
    ms = _ref_graph_ms(ref, bg, feeds, 1)
    bg.destroy()
    out["transformer_block_B4_S1024_d1024_H16_F4096"] = {
        "fwd_latency_ms": round(4 * ms, 1), "one_sequence_ms": round(ms, 1), "cores": threads,
        "GFLOP/s": round(27.925 / ms * 1e3, 3),
        "note": ("reference executor on the reference-built block graph with batch 1 (one of the 4 "
                 "sequences, which share only the weights), x4; MATMUL nodes one thread, attention OpenMP")}
    return out


def cpu_next_row_baselines(ref) -> dict:
    """The reference's own CPU kernels for the bench lines of the rows past
    the hot path (conv backward, the int8 path, the decode-side family), on
    this host, each at its bench shape or a stated sample extrapolated
    linearly.  Threads: the reference's OpenMP kernels run with every thread
    this process has; the int8 MATMUL branch and kernel_rope have no
    parallel loop (one thread)."""
    threads = _omp_threads()
    D = C.POINTER(C.c_double)
    I8 = C.POINTER(C.c_int8)
    out = {}

    def timed(fn) -> float:
        t0 = time.perf_counter()
        fn()
        return time.perf_counter() - t0

    # conv backward (B/src/math/lancius_kernels.c:62-136) on 4 of the 32 images
    log("cpu conv backward")
    N, Cin, H, W, Cout, n_s = 32, 64, 56, 56, 128, 4
    x = np.ascontiguousarray(prng.normal(50, (n_s, Cin, H, W)), dtype=np.float64)
    w = np.ascontiguousarray(prng.normal(150, (Cout, Cin, 3, 3), std=float(np.sqrt(2.0 / 576))), dtype=np.float64)
    g = np.ascontiguousarray(prng.normal(250, (n_s, Cout, H, W)), dtype=np.float64)
    dx, dw = np.zeros_like(x), np.zeros_like(w)
    flops = 2.0 * N * Cout * H * W * Cin * 9
    for name, fn in (("bwd_input", lambda: ref.kernel_conv2d_bwd_in(dx.ctypes.data_as(D), g.ctypes.data_as(D),
                                                                     w.ctypes.data_as(D), n_s, Cin, H, W, Cout, H, W,
                                                                     3, 3, 1, 1)),
                     ("bwd_weight", lambda: ref.kernel_conv2d_bwd_w(dw.ctypes.data_as(D), g.ctypes.data_as(D),
                                                                     x.ctypes.data_as(D), n_s, Cin, H, W, Cout, H, W,
                                                                     3, 3, 1, 1))):
        dt = timed(fn) * N / n_s
        out[f"conv3x3_N32_64to128_56x56_{name}"] = {
            "ms": round(dt * 1e3, 1), "GFLOP/s": round(flops / dt / 1e9, 3), "cores": threads,
            "note": f"kernel_conv2d_{'bwd_in' if name == 'bwd_input' else 'bwd_w'}, {n_s} of the {N} images timed, "
                    f"x{N // n_s}"}
    # int8 MATMUL branch (lancius_scheduler.c:195-220): quantize A, int32
    # sums, one thread, through the reference executor on a row sample of
    # the 4096^3 product
    log("cpu int8 matmul")
    n, rows = 4096, 16  # its B walk strides N per k: ~0.13 s per row here
    a = np.ascontiguousarray(prng.normal(43, (rows, n)), dtype=np.float64)
    bq = np.round(prng.uniform(1043, (n, n), -127.4, 127.4)).astype(np.int8)
    bg = graphs.BuiltGraph(ref, ref.lancius_graph_create())
    na, nb = ref.lancius_input(bg.g, rows, n), ref.lancius_input(bg.g, n, n)
    ref.lancius_matmul(bg.g, na, nb)
    nb.contents.runtime_data_int8 = bq.ctypes.data_as(I8)
    nb.contents.scale = 0.01
    na.contents.runtime_data = a.ctypes.data_as(D)
    sched = ref.lancius_ir_schedule(bg.g)
    arena = ref.lancius_arena_create(rows * n * 8 + (1 << 20))
    dt = timed(lambda: ref.lancius_schedule_execute(sched, arena)) * n / rows
    ref.lancius_arena_destroy(arena)
    ref.lancius_schedule_destroy(sched)
    na.contents.runtime_data = None
    nb.contents.runtime_data_int8 = None
    bg.destroy()
    out["gemm_i8_4096"] = {"ms": round(dt * 1e3, 1), "TOPS": round(2.0 * n ** 3 / dt / 1e12, 5), "cores": 1,
                           "note": f"reference int8 MATMUL branch (executor), rows 0-{rows - 1} of 4096 timed, "
                                   f"x{n // rows}"}
    # kernel_conv2d_int8_fwd (lancius_kernels.c:177-210) on 8 of the 32 images
    log("cpu int8 conv")
    n_s = 8
    xq = np.round(prng.uniform(45, (n_s, Cin, H, W), -127.4, 127.4)).astype(np.int8)
    wq = np.round(prng.uniform(145, (Cout, Cin, 3, 3), -127.4, 127.4)).astype(np.int8)
    y = np.zeros((n_s, Cout, H, W))
    dt = timed(lambda: ref.kernel_conv2d_int8_fwd(y.ctypes.data_as(D), xq.ctypes.data_as(I8), wq.ctypes.data_as(I8),
                                                  0.01, 0.001, n_s, Cin, H, W, Cout, 3, 3, 1, 1)) * N / n_s
    out["conv3x3_N32_64to128_56x56_relu_i8"] = {
        "ms": round(dt * 1e3, 1), "TOPS": round(flops / dt / 1e12, 5), "cores": threads,
        "note": f"kernel_conv2d_int8_fwd on int8 tensors (the quantization pass not timed), {n_s} of the {N} "
                f"images timed, x{N // n_s}"}
    # kernel_attention_kv_cache (lancius_kernels.c:338-379): batch 1 and
    # Hq = Hkv, so the B16 Hq32/Hkv8 decode runs as 16 calls with 32 K/V
    # heads (the same flops, four times the cache bytes); 2 calls timed
    log("cpu decode attention")
    B, Skv, Hq, Dh, n_s = 16, 4096, 32, 128, 2
    q = np.ascontiguousarray(prng.uniform(60, (Hq * Dh,), -1.0, 1.0), dtype=np.float64)
    kc = np.ascontiguousarray(prng.uniform(61, (Skv, Hq * Dh), -1.0, 1.0), dtype=np.float64)
    vc = np.ascontiguousarray(prng.uniform(62, (Skv, Hq * Dh), -1.0, 1.0), dtype=np.float64)
    o = np.zeros(Hq * Dh)
    dt = timed(lambda: [ref.kernel_attention_kv_cache(o.ctypes.data_as(D), q.ctypes.data_as(D), kc.ctypes.data_as(D),
                                                      vc.ctypes.data_as(D), Skv, Hq, Dh) for _ in range(n_s)]) * B / n_s
    out["attention_decode_B16_kv4096_Hq32_Hkv8_D128"] = {
        "ms": round(dt * 1e3, 1), "GFLOP/s": round(4.0 * B * Hq * Skv * Dh / dt / 1e9, 3), "cores": 1,
        "note": f"kernel_attention_kv_cache (one thread, fp64), Hkv = Hq = 32 (no grouped form), {n_s} of the "
                f"{B} sequences timed, x{B // n_s}"}
    # kernel_gqa (lancius_kernels.c:407-448): keys = queries (no history),
    # so the prefill's 1024 queries run over 1024 keys; one sequence of 4
    for Dh in (64, 128):
        log(f"cpu gqa D={Dh}")
        Bq, Sq, Hq, Hkv = 4, 1024, 32, 8
        q = np.ascontiguousarray(prng.uniform(63, (Sq, Hq * Dh), -1.0, 1.0), dtype=np.float64)
        k = np.ascontiguousarray(prng.uniform(64, (Sq, Hkv * Dh), -1.0, 1.0), dtype=np.float64)
        v = np.ascontiguousarray(prng.uniform(65, (Sq, Hkv * Dh), -1.0, 1.0), dtype=np.float64)
        o = np.zeros_like(q)
        dt = timed(lambda: ref.kernel_gqa(o.ctypes.data_as(D), q.ctypes.data_as(D), k.ctypes.data_as(D),
                                          v.ctypes.data_as(D), Sq, Hq, Hkv, Dh)) * Bq
        fl = 4.0 * Bq * Hq * Dh * Sq * (Sq + 1) / 2
        out[f"attention_gqa_prefill_B4_q1024_Hq32_Hkv8_D{Dh}"] = {
            "ms": round(dt * 1e3, 1), "GFLOP/s": round(fl / dt / 1e9, 3), "cores": threads,
            "note": "kernel_gqa, causal over the 1024 queries only (it has no key history: the GPU case's 1024 "
                    "earlier keys are not in this figure), 1 of the 4 sequences timed, x4"}
    # row ops at the bench shapes
    log("cpu rmsnorm / swiglu / rope")
    rows, hid = 4096, 4096
    x = np.ascontiguousarray(prng.normal(66, (rows, hid)), dtype=np.float64)
    u = np.ascontiguousarray(prng.normal(67, (rows, hid)), dtype=np.float64)
    gm = np.ones(hid)
    y = np.zeros_like(x)
    dt = timed(lambda: ref.kernel_rmsnorm(y.ctypes.data_as(D), x.ctypes.data_as(D), gm.ctypes.data_as(D), rows, hid,
                                          1e-5))
    out["rmsnorm_4096x4096"] = {"ms": round(dt * 1e3, 2), "GB/s": round(16.0 * rows * hid / dt / 1e9, 2),
                                "cores": threads, "note": "kernel_rmsnorm, fp64 (16 bytes per element read + written)"}
    dt = timed(lambda: ref.kernel_swiglu(y.ctypes.data_as(D), x.ctypes.data_as(D), u.ctypes.data_as(D), rows * hid))
    out["swiglu_4096x4096"] = {"ms": round(dt * 1e3, 2), "GB/s": round(24.0 * rows * hid / dt / 1e9, 2),
                               "cores": threads, "note": "kernel_swiglu, fp64"}
    S, H, hd, s_rows = 4096, 16, 128, 512
    qk = np.ascontiguousarray(prng.normal(68, (2, s_rows, H, hd)), dtype=np.float64)
    dt = timed(lambda: ref.kernel_rope(qk[0].ctypes.data_as(D), qk[1].ctypes.data_as(D), 1, s_rows, H, hd, 0)) * S / s_rows
    out["rope_q_k_S4096_H16_hd128"] = {"ms": round(dt * 1e3, 1), "GB/s": round(16.0 * 2 * S * H * hd / dt / 1e9, 3),
                                       "cores": 1, "note": f"kernel_rope (one thread, pow/cos/sin per element pair), "
                                                           f"{s_rows} of the {S} positions timed, x{S // s_rows}"}
    return out


def cpu_train_step_ms(ref, builder) -> float:
    """One training step of the reference's own autodiff graph on its CPU
    executor (graph, autodiff and executor all the reference's C)."""
    t = graphs.build_training(ref, builder(ref))
    feeds = {k: np.ascontiguousarray(v, dtype=np.float64) for k, v in train_feeds(t, 77).items()}
    for name in t.inputs:
        t.node(name).contents.runtime_data = feeds[name].ctypes.data_as(C.POINTER(C.c_double))
    sched = ref.lancius_ir_schedule(t.g)
    arena = ref.lancius_arena_create(512 << 20)
    times = []
    for _ in range(3):
        g = t.g.contents
        for i in range(g.node_count):  # fresh intermediates each step, as train_mnist.c:160-166 does
            n = g.nodes[i]
            if n.contents.op not in (abi.OP["INPUT"], abi.OP["CONST"]):
                n.contents.runtime_data = None
        t0 = time.perf_counter()
        ref.lancius_schedule_execute(sched, arena)
        times.append(time.perf_counter() - t0)
        ref.lancius_arena_reset(arena)
    ref.lancius_arena_destroy(arena)
    ref.lancius_schedule_destroy(sched)
    for name in t.inputs:
        t.node(name).contents.runtime_data = None
    t.destroy()
    return sorted(times)[1] * 1e3


PROFILE_CASES = {
    # name: (what it runs, callable(dev, reps) -> ms per call)
    "gemm4096": "fp32 GEMM 4096^3 (the headline)",
    "gemm_skinny": "fp32 GEMM 16x4096x4096",
    "conv": "conv 3x3 N32 64->128 56x56 + ReLU",
    "attn_s512_causal": "SDPA B8 H16 D64 S512 causal",
    "attn_s2048_causal": "SDPA B8 H16 D64 S2048 causal",
    "attn_s2048_noncausal": "SDPA B8 H16 D64 S2048 non-causal",
    "gemm_i8": "int8 GEMM 4096^3: quantize A + int8 product, weight packed once",
    "conv_i8": "int8 conv 3x3 N32 64->128 56x56 + ReLU: quantize + implicit-GEMM int8 conv",
    "gemm1024": "fp32 GEMM 1024^3",
    "block": "transformer block B4 S1024 d1024 H16 F4096 forward through the device executor",
    "copy": "HBM copy probe (1 GiB read + 1 GiB written per launch)",
}


def profile_case(dev, name: str, reps: int) -> float:
    """One config on its own, `reps` timed calls after a settle period, for
    rocprofv3 passes whose dispatches are the kernel of interest; the "copy"
    case (the HBM copy probe) calibrates the byte counters."""
    if name == "copy":
        dev.peak_probe("hbm")
        return 0.0
    if name == "gemm4096":
        return gemm_case(dev, 4096, 4096, 4096, 43, reps, 2, settle_ms=60.0)[0]
    if name == "gemm_skinny":
        return gemm_case(dev, 16, 4096, 4096, 43, reps, 2)[0]
    if name == "conv":
        return conv_case(dev, reps, 2)[0]
    if name == "gemm_i8":
        n = 4096
        a = dev.upload(prng.normal(43, (n, n)))
        b = dev.upload(np.round(prng.uniform(1043, (n, n), -127.4, 127.4)).astype(np.int8))
        c, pk = dev.alloc(n * n * 4), dev.alloc(dev.i8_packed_bytes(n, n))
        dev.i8_pack_weight(pk, b, n, n)
        t = time_steps(dev, lambda: dev.gemm_i8p(c, a, pk, 0.01, n, n, n), reps, 2)
        for buf in (a, b, c, pk):
            buf.free()
        return t
    if name == "conv_i8":
        N, C_in, H, W, C_out = 32, 64, 56, 56, 128
        x = dev.upload(prng.normal(45, (N, C_in, H, W)))
        w = dev.upload(np.round(prng.uniform(145, (C_out, C_in, 3, 3), -127.4, 127.4)).astype(np.int8))
        o = dev.alloc(N * C_out * H * W * 4)
        t = time_steps(dev, lambda: dev.conv2d_i8(o, x, w, 0.001, None, N, C_in, H, W, C_out, 3, 3, 1, 1, 1), reps, 2)
        for buf in (x, w, o):
            buf.free()
        return t
    if name == "gemm1024":
        return gemm_case(dev, 1024, 1024, 1024, 43, reps, 2)[0]
    if name == "block":
        bg = graphs.build_block(graph_lib())
        feeds = {}
        for i, nm in enumerate(bg.inputs):
            shape = abi.node_shape(bg.node(nm))
            feeds[nm] = (prng.normal(46 + 1000 * i, shape) if nm.startswith("x") else np.ones(shape, np.float32)
                         if nm in ("g1", "g2") else prng.normal(46 + 1000 * i, shape, 0, 0.02))
        t, _ = graph_case(dev, bg, feeds, reps, 2)
        bg.destroy()
        return t
    S = 512 if "s512" in name else 2048
    return attention_case(dev, 8, S, 16, 64, name.endswith("_causal"), 44, reps, 2)[0]


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    # The GPU clock settles over the first ~50 ms of MFMA load (4096^3 launches
    # shorten from 1.27 to 1.02 ms); the headline adds untimed launches for
    # about 60 ms of load after the warm-up, so the timed ones run in the
    # steady state whatever --warmup is.
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--quick", action="store_true", help="headline only (no other configs)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--profile-case", choices=sorted(PROFILE_CASES),
                    help="run one config only (for rocprofv3 passes): " +
                         "; ".join(f"{k}: {v}" for k, v in PROFILE_CASES.items()))
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: --gpus {args.gpus} is not supported in this build "
              f"(every workload here fits one MI355X; the multi-GPU split is a design, not code)",
              file=sys.stderr)
        return 2
    if device_count() < 1:
        print("bench.py: no GPU visible to HIP", file=sys.stderr)
        return 1
    # stdout carries exactly one JSON line: everything else the libraries
    # print (loader and pass messages) goes to stderr
    sys.stdout.flush()
    json_out = os.fdopen(os.dup(1), "w")
    os.dup2(2, 1)
    dev = Device(0)
    if args.profile_case:
        ms = profile_case(dev, args.profile_case, args.steps)
        dev.close()
        json_out.write(json.dumps({"profile_case": args.profile_case, "ms": round(ms, 4)}) + "\n")
        json_out.flush()
        return 0
    M = N = K = 4096
    log("device ceilings")
    measured_mfma = dev.peak_probe("mfma")
    measured_hbm = dev.peak_probe("hbm")
    measured_hbm_read = dev.peak_probe("hbm_read")
    log("headline gemm 4096^3")
    # args.warmup untimed launches, then further untimed launches for about
    # 60 ms of MFMA load (counted in the JSON as settle_launches): with few
    # warm-up launches the timed ones would otherwise run during the clock
    # ramp (1.3 ms per launch at the start against 1.02 ms settled).
    head_info: dict = {}
    ms, flops, nbytes = gemm_case(dev, M, K, N, 43, args.steps, args.warmup, settle_ms=60.0, info=head_info)
    gflops = flops / (ms * 1e-3) / 1e9
    traffic = None
    if TRAFFIC_FILE.exists():
        traffic = json.loads(TRAFFIC_FILE.read_text()).get("gemm_f32_direct 4096^3")
    result = {
        "metric": METRIC,
        "value": round(gflops, 1),
        "unit": "GFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "settle_launches": head_info.get("settle_launches", 0),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic: SplitMix64 seed 43, A,B ~ N(0,1) fp32, resident in HBM",
        "config": {"workload": "gemm_f32 C=A.B row-major M=N=K=4096 (BASELINE.json configs[1])",
                   "M": M, "N": N, "K": K, "parallelism": "1 GPU"},
        "roofline": {"bound": "mfma", "achieved": round(flops / (ms * 1e-3) / 1e12, 2), "peak": PEAK_FP32_MFMA,
                     "unit": "TFLOP/s", "frac": round(flops / (ms * 1e-3) / 1e12 / PEAK_FP32_MFMA, 4),
                     "traffic": traffic, "algorithmic_bytes": nbytes,
                     "measured_peak": round(measured_mfma, 2),
                     "frac_of_measured_peak": round(flops / (ms * 1e-3) / 1e12 / measured_mfma, 4)},
        "device_ceilings": {"fp32_mfma_TFLOPs_measured": round(measured_mfma, 2),
                            "fp32_mfma_TFLOPs_spec": PEAK_FP32_MFMA,
                            "hbm_copy_GBs_measured": round(measured_hbm, 1),
                            "hbm_read_GBs_measured": round(measured_hbm_read, 1), "hbm_GBs_spec": PEAK_HBM},
    }
    extra = {}
    load_dir, load_files = None, None
    if not args.quick:
        steps = max(5, args.steps)
        for name, (m, k, n) in (("gemm_1024", (1024, 1024, 1024)), ("gemm_2048", (2048, 2048, 2048)),
                                ("gemm_16x4096x4096", (16, 4096, 4096))):
            log(name)
            t, f, b = gemm_case(dev, m, k, n, 43, steps, 3)
            extra[name] = {"ms": round(t, 4), "GFLOP/s": round(f / t / 1e6, 1),
                           "frac_fp32_mfma": round(f / t / 1e9 / PEAK_FP32_MFMA, 4),
                           "GB/s": round(b / t / 1e6, 1), "frac_hbm": round(b / t / 1e6 / PEAK_HBM, 4)}
        for S in (512, 2048):
            for causal in (True, False):
                name = f"attention_B8_H16_D64_S{S}_{'causal' if causal else 'noncausal'}"
                log(name)
                t, f, b = attention_case(dev, 8, S, 16, 64, causal, 44, steps, 3)
                extra[name] = {"ms": round(t, 4), "GFLOP/s": round(f / t / 1e6, 1),
                               "frac_fp32_mfma": round(f / t / 1e9 / PEAK_FP32_MFMA, 4)}
        log("conv")
        t, f, b = conv_case(dev, steps, 3)
        tw, _, _ = conv_case(dev, steps, 3, packed=False)
        extra["conv3x3_N32_64to128_56x56_relu"] = {
            "ms": round(t, 4), "GFLOP/s": round(f / t / 1e6, 1), "frac_fp32_mfma": round(f / t / 1e9 / PEAK_FP32_MFMA, 4),
            "ms_relaying_w_each_call": round(tw, 4),
            "note": "filter packed once per weight, as the device executor does for an uploaded filter; "
                    "ms_relaying_w_each_call re-lays the OIHW filter inside every call"}
        log("decode-side family")
        extra.update(decode_cases(dev, steps, 3))
        log("int8 path")
        extra.update(int8_cases(dev, steps, 3))
        log("conv backward")
        extra.update(conv_bwd_cases(dev, steps, 3))
        log("row and elementwise kernels")
        extra.update(rowop_cases(dev, max(20, steps), 5))
        log("model files to HBM")
        load_dir = Path(tempfile.mkdtemp(prefix="lancius_load_"))
        load_files = write_load_models(load_dir)
        extra.update(model_load_cases(dev, *load_files))
        log("host-pointer bridge")
        extra["kernel_matmul_f32_host_bridge_4096"] = bridge_case(dev)
        log("mlp graph")
        sdev = Device(0, own_stream=True)  # hipGraph replay on a capturable stream
        lib = graph_lib()
        bg = graphs.build_mlp(lib)
        feeds = {"x": prng.uniform(42, (64, 784), -1.0, 1.0), "W1": prng.normal(142, (784, 256), 0, 0.02),
                 "b1": np.zeros((1, 256), np.float32), "W2": prng.normal(342, (256, 10), 0, 0.02),
                 "b2": np.zeros((1, 10), np.float32)}
        # a forward is a few microseconds: 200 timed forwards (each a whole
        # run of the program) keep the stream's start-up latency out of the
        # per-forward figure (at 20 it adds about 0.4 us)
        small = max(200, steps)
        t, info = graph_case(dev, bg, feeds, small, 5)
        tg, _ = graph_case(sdev, bg, feeds, small, 5, DEVICE_GRAPH)
        tu, info_u = graph_case(dev, bg, feeds, small, 5, DEVICE_NO_CHAIN)
        bg.destroy()
        extra["mlp_graph_64x784x256x10"] = {"fwd_latency_ms": round(t, 4), "launches": info["launches"],
                                            "timed_forwards": small,
                                            "GFLOP/s": round(26.02e6 / t / 1e6, 1),
                                            "fwd_latency_ms_hipgraph": round(tg, 4),
                                            "fwd_latency_ms_unchained": round(tu, 4),
                                            "launches_unchained": info_u["launches"]}
        log("basis graph")
        extra["basis_mlp_graph_64x784x256x10_tanh"] = basis_case(dev, small, 5)
        log("transformer block graph")
        bg = graphs.build_block(lib)
        feeds = {}
        for i, name in enumerate(bg.inputs):
            shape = abi.node_shape(bg.node(name))
            if name.startswith("x"):
                feeds[name] = prng.normal(46 + 1000 * i, shape)
            elif name in ("g1", "g2"):
                feeds[name] = np.ones(shape, np.float32)
            else:
                feeds[name] = prng.normal(46 + 1000 * i, shape, 0, 0.02)
        t, info = graph_case(dev, bg, feeds, 10, 3)
        tg, _ = graph_case(sdev, bg, feeds, 10, 3, DEVICE_GRAPH)
        bg.destroy()
        extra["transformer_block_B4_S1024_d1024_H16_F4096"] = {
            "fwd_latency_ms": round(t, 3), "fwd_latency_ms_hipgraph": round(tg, 3), "launches": info["launches"],
            "GFLOP/s": round(111.7e9 / t / 1e6, 1), "arena_MiB": round(info["arena_bytes"] / 2 ** 20, 1)}
        for name, builder, gflop in (
                ("train_step_mnist_mlp_B64_784x128x10", lambda l: graphs.build_mlp_ce(l), MLP_TRAIN_GFLOP),
                ("train_step_cifar_cnn_B32", lambda l: graphs.build_cnn_ce(l, batch=32), CNN_TRAIN_GFLOP)):
            log(name)
            t, info = train_case(dev, builder, max(20, steps), 5)
            tg, _ = train_case(sdev, builder, max(20, steps), 5, DEVICE_GRAPH)
            extra[name] = {"step_latency_ms": round(t, 4), "step_latency_ms_hipgraph": round(tg, 4),
                           "launches": info["launches"], "GFLOP/s": round(gflop / t * 1e3, 1),
                           "arena_MiB": round(info["arena_bytes"] / 2 ** 20, 2)}
        result["all_configs"] = extra
        sdev.close()
    dev.close()
    if not args.no_cpu:
        log("cpu baseline")
        result["cpu_baseline"] = cpu_baseline(M, K, N)
        if load_files and result["cpu_baseline"] and result["cpu_baseline"]["kind"] == "reference":
            import oracle

            result["cpu_baseline"]["other_configs"][f"model_load_v10_fp64_{LOAD_LAYERS}x{LOAD_DIM}x{LOAD_DIM}"] = \
                cpu_model_load(oracle.ref_lib(), load_files[0])
    if load_dir is not None:
        shutil.rmtree(load_dir, ignore_errors=True)
    sys.stdout.flush()
    json_out.write(json.dumps(result) + "\n")
    json_out.flush()
    return 0


if __name__ == "__main__":
    sys.exit(main())
