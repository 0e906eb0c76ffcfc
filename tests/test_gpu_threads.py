"""Several host threads driving the device at once, each through its own
context on its own stream: the reference runs the nodes of one wave on a
pthread pool (bleeding/v11A1/src/runtime/lancius_scheduler.c:405-411), so
the entry points must be callable concurrently.  Workspaces, arrival
counters and the last-error message are per context or per thread; the
kernels here include the skinny GEMM (its split-K slices meet through the
context's arrival counters), the MLP chain (same) and the grouped attention.
Every thread's results must match its own first round bit for bit (all
kernels are run-to-run deterministic) and the first round must match the
oracle."""
import threading

import numpy as np
import pytest

import oracle
from lancius_amd import ACT_RELU, Device, DeviceProgram, graph_lib, graphs, prng
from tests.conftest import case

pytestmark = pytest.mark.gpu

THREADS = 4
ROUNDS = 8


def _worker(tid, bg, start, results, errors):
    try:
        dev = Device(0, own_stream=True)
        M, K, N = 384, 512, 320
        A, B, bias = prng.normal(300 + tid, (M, K)), prng.normal(310 + tid, (K, N)), prng.normal(320 + tid, (N,))
        As, Bs = prng.normal(330 + tid, (16, 2048)), prng.normal(340 + tid, (2048, 1024))
        Bq, S, H, D = 2, 256, 4, 64
        q, k, v = (prng.normal(350 + tid + 10 * i, (Bq, S, H, D)) for i in range(3))
        d = {n: dev.upload(x) for n, x in (("A", A), ("B", B), ("bias", bias), ("As", As), ("Bs", Bs), ("q", q),
                                              ("k", k), ("v", v))}
        C1, C2, O = dev.alloc(4 * M * N), dev.alloc(4 * 16 * 1024), dev.alloc(4 * q.size)
        prog = DeviceProgram(dev, bg.g, bg.sched, None, 0)
        feeds = {n: prng.normal(360 + tid + i, tuple(bg.node(n).contents.shape[:2])) for i, n in enumerate(bg.inputs)}
        for n, x in feeds.items():
            prog.upload(bg.node(n), x)
        start.wait()
        rounds = []
        for _ in range(ROUNDS):
            dev.gemm(C1, d["A"], d["B"], M, K, N, bias=d["bias"], act=ACT_RELU)
            dev.gemm(C2, d["As"], d["Bs"], 16, 2048, 1024)
            dev.attention(O, d["q"], d["k"], d["v"], Bq, S, H, D, causal=True)
            prog.run()
            rounds.append((dev.download(C1, (M, N)), dev.download(C2, (16, 1024)),
                           dev.download(O, q.shape), prog.download(bg.node("softmax")).reshape(64, 10)))
        prog.close()
        for b in list(d.values()) + [C1, C2, O]:
            b.free()
        dev.close()
        results[tid] = (rounds, (A, B, bias, As, Bs, q, k, v, feeds))
    except Exception as e:  # re-raised by the main thread
        errors[tid] = e


def test_concurrent_contexts_from_host_threads():
    lib = graph_lib()
    built = []
    for _ in range(THREADS):
        bg = graphs.build_mlp(lib)
        bg.sched = lib.lancius_ir_schedule(bg.g)
        built.append(bg)
    start = threading.Barrier(THREADS)
    results, errors = [None] * THREADS, [None] * THREADS
    case(f"{THREADS} host threads, own contexts and streams, {ROUNDS} rounds of GEMM / skinny GEMM / attention / MLP")
    threads = [threading.Thread(target=_worker, args=(t, built[t], start, results, errors)) for t in range(THREADS)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=100)
    assert not any(t.is_alive() for t in threads), "a device thread did not finish"
    for e in errors:
        if e is not None:
            raise e
    for tid in range(THREADS):
        rounds, (A, B, bias, As, Bs, q, k, v, feeds) = results[tid]
        for r in rounds[1:]:
            for got, first in zip(r, rounds[0]):
                np.testing.assert_array_equal(got, first)
        c1, c2, o, sm = rounds[0]
        ref1 = np.maximum(oracle.matmul(A, B) + np.asarray(bias, np.float64)[None, :], 0.0)
        assert oracle.normwise_error(c1, ref1) <= oracle.tolerance(512), tid
        assert oracle.normwise_error(c2, oracle.matmul(As, Bs)) <= oracle.tolerance(2048), tid
        ref_o = oracle.attention(q, k, v, True)
        assert oracle.normwise_error(o, ref_o) <= oracle.tolerance(256), tid
        h = np.maximum(oracle.matmul(feeds["x"], feeds["W1"]) + np.asarray(feeds["b1"], np.float64), 0.0)
        ref_sm = oracle.softmax(oracle.matmul(h, feeds["W2"]) + np.asarray(feeds["b2"], np.float64))
        assert oracle.normwise_error(sm, ref_sm) <= oracle.tolerance(784), tid
    for bg in built:
        lib.lancius_schedule_destroy(bg.sched)
        bg.destroy()
