"""lancius_hip_gemm_f32_noalloc (include/lancius_hip.h): the GEMM with its
split-K partial sums in the library's fixed per-GPU scratch array instead of
the context workspace.  It has no counterpart in the reference; it is for
callers that cannot allocate device memory.  Called through the C ABI, on
calls in a row of decreasing size, its output must equal
lancius_hip_gemm_f32's bit for bit (same kernels, same split choice) and the
fp64 oracle within the GEMM tolerance; a shape whose partials exceed the
scratch is refused with -3 before any launch; and the calls leave the
device's free memory unchanged."""
import ctypes as C

import numpy as np
import pytest

import oracle
from lancius_amd import ACT_GELU, ACT_NONE, ACT_RELU, Device, prng
from tests.conftest import case

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 32 << 20  # LANCIUS_HIP_NOALLOC_SCRATCH_BYTES


def _hip_free_bytes() -> int:
    hip = C.CDLL("libamdhip64.so")
    free, total = C.c_size_t(), C.c_size_t()
    assert hip.hipMemGetInfo(C.byref(free), C.byref(total)) == 0
    return free.value


def _noalloc(d, Cb, A, B, M, K, N, bias=None, act=ACT_NONE, R=None) -> int:
    v = lambda b: None if b is None else C.c_void_p(int(b))  # noqa: E731
    return d.lib.lancius_hip_gemm_f32_noalloc(d.ctx, v(Cb), v(A), v(B), M, K, N, v(bias), act, v(R))


# (M, K, N, act): skinny split-K (16 K slices, 4 MiB of partials), tiled
# split-K with k-groups and ragged edges, a small skinny split, no split.
CALLS = [(16, 4096, 4096, ACT_RELU), (520, 1100, 500, ACT_GELU), (8, 1024, 768, ACT_NONE), (64, 64, 64, ACT_NONE)]


def test_noalloc_gemm_matches_gemm_f32():
    d = Device(0)  # a fresh context: its workspace is empty
    first = True
    for i, (M, K, N, act) in enumerate(CALLS):
        A, B = prng.normal(700 + i, (M, K)), prng.normal(800 + i, (K, N))
        bias, R = prng.normal(900 + i, (N,)), prng.normal(950 + i, (M, N))
        dA, dB, db, dR = d.upload(A), d.upload(B), d.upload(bias), d.upload(R)
        c_ref, c_new = d.alloc(M * N * 4), d.alloc(M * N * 4)
        d.fill(c_new, float("nan"), M * N)
        d.synchronize()
        case(f"gemm_f32_noalloc call {i}: M={M} K={K} N={N} act={act}")
        free_before = _hip_free_bytes()
        rc = _noalloc(d, c_new, dA, dB, M, K, N, db, act, dR)
        assert rc == 0, d.lib.lancius_hip_last_error()
        d.synchronize()
        if not first:  # the first call on the device may load the code object and its scratch
            assert _hip_free_bytes() == free_before, "the no-alloc entry point allocated device memory"
        first = False
        got = d.download(c_new, (M, N))
        d.gemm(c_ref, dA, dB, M, K, N, bias=db, act=act, residual=dR)
        want = d.download(c_ref, (M, N))
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), i
        ref = oracle.matmul(A, B) + bias.astype(np.float64)[None, :]
        ref = oracle.relu(ref) if act == ACT_RELU else oracle.gelu(ref) if act == ACT_GELU else ref
        ref = ref + R.astype(np.float64)
        assert oracle.normwise_error(got, ref) <= oracle.tolerance(K), i
        for b in (dA, dB, db, dR, c_ref, c_new):
            b.free()
    d.close()


def test_noalloc_gemm_refuses_beyond_scratch(dev):
    """32 x 16384 x 16384 splits K into 64 partial sums of 2 MiB (128 MiB),
    more than the scratch: -3 with a message, and C is not touched."""
    M, K, N = 32, 16384, 16384
    assert 64 * M * N * 4 > SCRATCH_BYTES
    dA, dB, dC = dev.alloc(M * K * 4), dev.alloc(K * N * 4), dev.alloc(M * N * 4)
    dev.fill(dA, 1.0, M * K)
    dev.fill(dB, 1.0, K * N)
    dev.fill(dC, 7.0, M * N)
    case("gemm_f32_noalloc beyond its scratch")
    rc = _noalloc(dev, dC, dA, dB, M, K, N)
    assert rc == -3
    assert b"scratch" in dev.lib.lancius_hip_last_error()
    assert (dev.download(dC, (M, N)) == 7.0).all()
    # the same shape through the allocating entry point works
    dev.gemm(dC, dA, dB, M, K, N)
    assert (dev.download(dC, (M, N)) == float(K)).all()
    for b in (dA, dB, dC):
        b.free()


def test_noalloc_gemm_under_capture():
    """The first no-alloc calls of a fresh context made inside a stream
    capture: the recorded graph, replayed several times with eager work of
    the same context between the replays, gives lancius_hip_gemm_f32's
    output bit for bit on every replay (the scratch's address and its zeroed
    counters come from context creation, not from the first call)."""
    d = Device(0, own_stream=True)
    shapes = [(16, 4096, 4096, ACT_RELU), (520, 1100, 500, ACT_GELU)]
    bufs = []
    for i, (M, K, N, act) in enumerate(shapes):
        A, B = prng.normal(1700 + i, (M, K)), prng.normal(1800 + i, (K, N))
        bias = prng.normal(1900 + i, (N,))
        dA, dB, db = d.upload(A), d.upload(B), d.upload(bias)
        c_ref, c_new = d.alloc(M * N * 4), d.alloc(M * N * 4)
        d.gemm(c_ref, dA, dB, M, K, N, bias=db, act=act)
        bufs.append((M, K, N, act, dA, dB, db, c_ref, c_new))
    d.synchronize()
    want = [d.download(b[7], (b[0], b[2])) for b in bufs]
    case("gemm_f32_noalloc captured into a graph")
    assert d.lib.lancius_hip_capture_begin(d.ctx) == 0, d.lib.lancius_hip_last_error()
    rcs = [_noalloc(d, c_new, dA, dB, M, K, N, db, act) for (M, K, N, act, dA, dB, db, _, c_new) in bufs]
    graph = C.c_void_p()
    rc_end = d.lib.lancius_hip_capture_end(d.ctx, C.byref(graph))
    assert rcs == [0, 0] and rc_end == 0, d.lib.lancius_hip_last_error()
    for rep in range(3):
        for (M, K, N, act, dA, dB, db, c_ref, c_new) in bufs:
            d.fill(c_new, float("nan"), M * N)
        # eager work of the same context between replays (its own split-K)
        M, K, N, act, dA, dB, db, c_ref, _ = bufs[1]
        d.gemm(c_ref, dA, dB, M, K, N, bias=db, act=act)
        d.synchronize()
        assert d.lib.lancius_hip_graph_launch(graph, d.ctx) == 0, d.lib.lancius_hip_last_error()
        d.synchronize()
        for j, b in enumerate(bufs):
            got = d.download(b[8], (b[0], b[2]))
            assert np.array_equal(got.view(np.uint32), want[j].view(np.uint32)), (rep, j)
    d.lib.lancius_hip_graph_destroy(graph)
    for b in bufs:
        for buf in b[4:]:
            buf.free()
    d.close()
