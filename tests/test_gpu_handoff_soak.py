"""Repeat-call soak of every kernel that hands partial results from one
workgroup to another inside a launch (sc1 stores written through to the
point of coherence, vmcnt(0), a relaxed agent-scope add on an arrival
counter, and the last arriver reading the partials back with sc1 loads):

  * the one-launch skinny GEMM (K slices summed by the last workgroup of a
    column block);
  * the stream-K conv (a tile's k shares summed by the last sharer);
  * split-KV decode attention (key-range partials merged by the last range);
  * the small-batch MLP chain (hidden-tile partials, K-range partials).

A latent ordering fault in that hand-off would show as a rare result that
differs from the others.  Each kernel is called about 200 times on several
shapes and seeded inputs; every call's output must equal, bit for bit, the
first call's output for the same input, and the first call of each input is
checked against the fp64 oracle.  The first mismatch fails the test with
the call that produced it.  The host-side counterpart in the reference is
S9/examples/audit_threadpool_parity.c:12-75 (repeat runs of one graph on a
thread pool must agree)."""
import numpy as np
import pytest

import oracle
from lancius_amd import ACT_GELU, ACT_NONE, ACT_RELU, prng
from tests.conftest import case

pytestmark = pytest.mark.gpu

REPEATS = 10  # calls per input after the first


def _up(dev, a):
    return dev.upload(np.ascontiguousarray(a, dtype=np.float32))


def _same_bits(got, first, what):
    if not np.array_equal(got.view(np.uint32), first.view(np.uint32)):
        diff = np.count_nonzero(got.view(np.uint32) != first.view(np.uint32))
        raise AssertionError(f"{what}: {diff} elements differ from the first call")


# 4 shapes x 5 inputs x (1 + 10) calls = 220 launches; every shape splits K
# (K / 512 slices), one has N % 4 != 0 (scalar B loads), one M = 32.
SKINNY = [(16, 4096, 4096, ACT_NONE), (8, 2048, 1000, ACT_RELU), (32, 8192, 520, ACT_GELU), (5, 3000, 301, ACT_NONE)]


@pytest.mark.parametrize("M,K,N,act", SKINNY)
def test_soak_skinny_gemm(dev, M, K, N, act):
    dC = dev.alloc(M * N * 4)
    for s in range(5):
        seed = 5000 + 10 * s + M
        A, B, bias = prng.normal(seed, (M, K)), prng.normal(seed + 1, (K, N)), prng.normal(seed + 2, (N,))
        dA, dB, db = _up(dev, A), _up(dev, B), _up(dev, bias)
        first = None
        for r in range(REPEATS + 1):
            case(f"soak skinny gemm M={M} K={K} N={N} act={act} input {s} call {r}")
            dev.fill(dC, float("nan"), M * N)
            dev.gemm(dC, dA, dB, M, K, N, bias=db, act=act)
            got = dev.download(dC, (M, N))
            if first is None:
                first = got
                ref = oracle.matmul(A, B) + bias.astype(np.float64)[None, :]
                ref = oracle.relu(ref) if act == ACT_RELU else oracle.gelu(ref) if act == ACT_GELU else ref
                assert oracle.normwise_error(got, ref) <= oracle.tolerance(K), (s, r)
            else:
                _same_bits(got, first, f"skinny gemm input {s} call {r}")
        for b in (dA, dB, db):
            b.free()
    dC.free()


# Tile counts a little over a whole number per CU on a 256-CU part, so the
# last tiles are shared (stream-K): 294 (128x64 tiles), 282 (64x64 tiles)
# and the bench conv's 1568; a small grid split over all CUs (26 tiles, each
# shared 4 ways).  5 / 5 / 2 / 3 inputs x 11 calls.
CONV = [(6, 16, 56, 56, 128, 5), (23, 32, 28, 28, 64, 5), (32, 64, 56, 56, 128, 2), (1, 128, 28, 28, 256, 3)]


@pytest.mark.parametrize("N,C_in,H,W,C_out,inputs", CONV)
def test_soak_stream_k_conv(dev, N, C_in, H, W, C_out, inputs):
    n_out = N * C_out * H * W
    do = dev.alloc(n_out * 4)
    for s in range(inputs):
        seed = 6000 + 10 * s + C_in
        x = prng.normal(seed, (N, C_in, H, W))
        w = prng.normal(seed + 1, (C_out, C_in, 3, 3), 0, np.sqrt(2.0 / (9 * C_in)))
        bias = prng.normal(seed + 2, (C_out,), 0, 0.1)
        dx, dw, db = _up(dev, x), _up(dev, w), _up(dev, bias)
        first = None
        for r in range(REPEATS + 1):
            case(f"soak stream-K conv N={N} C_in={C_in} {H}x{W} C_out={C_out} input {s} call {r}")
            dev.fill(do, float("nan"), n_out)
            dev.conv2d(do, dx, dw, db, N, C_in, H, W, C_out, 3, 3, 1, 1, act=ACT_RELU)
            got = dev.download(do, (N, C_out, H, W))
            if first is None:
                first = got
                if s == 0:  # the oracle on one input per shape (fp64 conv of the whole batch)
                    ref = oracle.relu(oracle.conv2d(x, w, 1, 1, False) + bias.astype(np.float64)[None, :, None, None])
                    assert oracle.normwise_error(got, ref) <= oracle.tolerance(9 * C_in)
                else:
                    assert np.isfinite(got).all()
            else:
                _same_bits(got, first, f"conv input {s} call {r}")
        for b in (dx, dw, db):
            b.free()
    do.free()


# Several key ranges per (sequence, K/V head): the last range to arrive
# merges the partials.  4 shapes x 5 inputs x 11 calls.
DECODE = [(16, 4096, 32, 8, 128, None), (4, 8192, 8, 8, 64, None), (3, 5000, 4, 4, 96, [4999, 5000, 2500]),
          (8, 2048, 16, 2, 128, [2048, 1, 700, 1999, 0, 1024, 2047, 513])]


@pytest.mark.parametrize("B,Skv,Hq,Hkv,D,lens", DECODE)
def test_soak_decode_merge(dev, B, Skv, Hq, Hkv, D, lens):
    do = dev.alloc(4 * B * Hq * D)
    dl = dev.upload(np.asarray(lens, np.int32)) if lens is not None else None
    for s in range(5):
        seed = 7000 + 10 * s + D
        q = prng.uniform(seed, (B, Hq, D), -1.0, 1.0)
        k = prng.uniform(seed + 1, (B, Skv, Hkv, D), -1.0, 1.0)
        v = prng.uniform(seed + 2, (B, Skv, Hkv, D), -1.0, 1.0)
        dq, dk, dv = _up(dev, q), _up(dev, k), _up(dev, v)
        first = None
        for r in range(REPEATS + 1):
            case(f"soak decode B={B} Skv={Skv} Hq={Hq} Hkv={Hkv} D={D} input {s} call {r}")
            dev.fill(do, float("nan"), B * Hq * D)
            dev.attention_decode(do, dq, dk, dv, dl, B, Skv, Hq, Hkv, D)
            got = dev.download(do, (B, Hq, D))
            if first is None:
                first = got
                ref = oracle.attention_decode(q, k, v, lens)
                if lens is not None:  # an empty cache gives zeros on both sides
                    assert np.isfinite(got).all()
                assert oracle.normwise_error(got, ref) <= oracle.tolerance(Skv), (s, r)
            else:
                _same_bits(got, first, f"decode input {s} call {r}")
        for b in (dq, dk, dv):
            b.free()
    for b in (do, dl):
        if b is not None:
            b.free()


# The MNIST MLP (16-row blocks handed to the last tile), K1 = 4096 (four K
# ranges per hidden tile, then the row-block hand-off) and a long-K shape
# that runs mlp2_split.  3 shapes x 6 inputs x 11 calls.
MLP = [(64, 784, 256, 10, ACT_RELU), (64, 4096, 256, 10, ACT_RELU), (16, 9000, 64, 32, ACT_GELU)]


@pytest.mark.parametrize("M,K1,N1,N2,act", MLP)
def test_soak_mlp_chain(dev, M, K1, N1, N2, act):
    out, am = dev.alloc(M * N2 * 4), dev.alloc(M * 4)
    for s in range(6):
        seed = 8000 + 10 * s + K1
        x = prng.uniform(seed, (M, K1), -1.0, 1.0)
        w1, w2 = prng.normal(seed + 1, (K1, N1), 0, 0.05), prng.normal(seed + 2, (N1, N2), 0, 0.1)
        b1, b2 = prng.normal(seed + 3, (N1,), 0, 0.05), prng.normal(seed + 4, (N2,), 0, 0.05)
        dx, dw1, dw2, db1, db2 = (_up(dev, a) for a in (x, w1, w2, b1, b2))
        first = first_idx = None
        for r in range(REPEATS + 1):
            case(f"soak mlp chain M={M} K1={K1} N1={N1} N2={N2} input {s} call {r}")
            dev.fill(out, float("nan"), M * N2)
            dev.mlp2(out, am, dx, dw1, db1, act, dw2, db2, M, K1, N1, N2, True)
            got = dev.download(out, (M, N2))
            idx = dev.download(am, (M,), np.int32)
            if first is None:
                first, first_idx = got, idx
                h = oracle.matmul(x, w1) + b1.astype(np.float64)[None, :]
                h = oracle.relu(h) if act == ACT_RELU else oracle.gelu(h)
                ref = oracle.softmax(oracle.matmul(h, w2) + b2.astype(np.float64)[None, :])
                assert oracle.normwise_error(got, ref) <= oracle.tolerance(K1), (s, r)
                assert np.array_equal(idx, oracle.argmax(ref)), (s, r)
            else:
                _same_bits(got, first, f"mlp chain input {s} call {r}")
                assert np.array_equal(idx, first_idx), (s, r)
        for b in (dx, dw1, dw2, db1, db2):
            b.free()
    for b in (out, am):
        b.free()

