"""lancius_hip_mlp2_f32 / lancius_hip_mlp2_ex_f32: two dense layers (each
with bias and activation) and a row softmax in one launch, against the fp64
oracle of the unfused chain (MATMUL, bias, activation, MATMUL, bias,
activation, SOFTMAX, first-maximum argmax).  Tolerance as for the GEMM of
the longest reduction, 1e-4 * max(1, sqrt(K1)/32); argmax bit-exact."""
import numpy as np
import pytest

import oracle
from lancius_amd import ACT_GELU, ACT_NONE, ACT_RELU, ACT_TANH, HipError, prng
from tests.conftest import case

pytestmark = pytest.mark.gpu


def _act(h, act):
    if act == ACT_RELU:
        return oracle.relu(h)
    if act == ACT_GELU:
        return oracle.gelu(h)
    if act == ACT_TANH:
        return np.tanh(h)
    return h


def reference(x, w1, b1, act, w2, b2, softmax, act2=ACT_NONE):
    h = oracle.matmul(x, w1)
    if b1 is not None:
        h = h + b1.astype(np.float64)[None, :]
    y = oracle.matmul(_act(h, act), w2)
    if b2 is not None:
        y = y + b2.astype(np.float64)[None, :]
    y = _act(y, act2)
    return oracle.softmax(y) if softmax else y


def run(dev, M, K1, N1, N2, act, bias, softmax, seed, act2=None):
    x = prng.uniform(seed, (M, K1), -1.0, 1.0)
    w1 = prng.normal(seed + 1, (K1, N1), 0, 0.05)
    w2 = prng.normal(seed + 2, (N1, N2), 0, 0.1)
    b1 = prng.normal(seed + 3, (N1,), 0, 0.05) if bias else None
    b2 = prng.normal(seed + 4, (N2,), 0, 0.05) if bias else None
    bufs = {k: dev.upload(v) for k, v in (("x", x), ("w1", w1), ("w2", w2)) if v is not None}
    db1 = dev.upload(b1) if bias else None
    db2 = dev.upload(b2) if bias else None
    out, am = dev.alloc(M * N2 * 4), dev.alloc(M * 4)
    case(f"mlp2 M={M} K1={K1} N1={N1} N2={N2} act={act},{act2} bias={bias} softmax={softmax}")
    dev.mlp2(out, am, bufs["x"], bufs["w1"], db1, act, bufs["w2"], db2, M, K1, N1, N2, softmax, act2)
    got = dev.download(out, (M, N2))
    idx = dev.download(am, (M,), np.int32) if softmax else None
    for b in list(bufs.values()) + [db1, db2, out, am]:
        if b is not None:
            b.free()
    return got, idx, reference(x, w1, b1, act, w2, b2, softmax, ACT_NONE if act2 is None else act2)


@pytest.mark.parametrize("M,K1,N1,N2,act,bias,softmax", [
    (64, 784, 256, 10, ACT_RELU, True, True),   # the MNIST MLP
    (64, 784, 128, 10, ACT_RELU, True, True),
    (1, 1, 1, 1, ACT_NONE, False, True),
    (7, 100, 64, 5, ACT_GELU, True, True),
    (33, 300, 128, 64, ACT_RELU, False, True),
    (64, 17, 100, 7, ACT_NONE, True, False),
    (50, 1000, 96, 33, ACT_GELU, False, False),
    (64, 4096, 64, 64, ACT_RELU, True, True),
    (16, 9000, 64, 10, ACT_RELU, True, True),    # K ranges of several staged chunks
    (13, 301, 250, 9, ACT_TANH, True, True),     # K ranges and N1 not multiples of 4
    (64, 400, 256, 10, ACT_RELU, True, True),    # 7 blocks of 16 k per wave: groups of 8
    (64, 1500, 128, 32, ACT_RELU, True, True),   # 32 tiles, K > 1024: four K ranges per tile
    (40, 1200, 352, 10, ACT_GELU, True, True),   # 66 tiles: three K ranges per tile
    (20, 2001, 250, 9, ACT_TANH, True, True),    # four K ranges, K1 and N1 not multiples of 4 (scalar loads)
    # hidden layers wider than 256: 16-column tiles, K split for K > 1024
    # while the grid is under 256 workgroups
    (16, 300, 512, 16, ACT_RELU, True, True),
    (4, 2000, 2048, 4, ACT_GELU, True, True),    # 128 tiles: two K ranges
    (3, 77, 1000, 8, ACT_RELU, False, False),   # K too short to split
    (1, 100, 8192, 1, ACT_RELU, True, False),   # 512 tiles: no split
])
def test_mlp2_matches_unfused_chain(dev, M, K1, N1, N2, act, bias, softmax):
    got, idx, ref = run(dev, M, K1, N1, N2, act, bias, softmax, 40 + M + K1)
    assert oracle.normwise_error(got, ref) <= oracle.tolerance(max(K1, N1))
    if softmax:
        assert np.array_equal(idx, oracle.argmax(ref))


@pytest.mark.parametrize("M,K1,N1,N2,act,act2,bias,softmax", [
    (64, 784, 256, 10, ACT_TANH, ACT_RELU, True, False),  # the BASIS example MLP
    (64, 784, 256, 10, ACT_TANH, ACT_TANH, True, True),
    (5, 33, 64, 64, ACT_GELU, ACT_GELU, False, False),
    (64, 128, 128, 64, ACT_NONE, ACT_RELU, True, True),
])
def test_mlp2_second_activation(dev, M, K1, N1, N2, act, act2, bias, softmax):
    got, idx, ref = run(dev, M, K1, N1, N2, act, bias, softmax, 90 + N1 + act2, act2)
    assert oracle.normwise_error(got, ref) <= oracle.tolerance(max(K1, N1))
    if softmax:
        assert np.array_equal(idx, oracle.argmax(ref))


def test_mlp2_repeatable(dev):
    """Fixed reduction orders and counters that return to zero: repeated
    calls give identical bits."""
    outs = [run(dev, 64, 784, 256, 10, ACT_RELU, True, True, 7)[0] for _ in range(3)]
    assert all(np.array_equal(outs[0], o) for o in outs[1:])


def test_mlp2_limits(dev):
    case("mlp2 limits")
    for M, K1, N1, N2 in ((65, 8, 8, 8), (8, 8, 8, 65), (64, 8, 257, 8), (8, 8, 200, 64), (64, (1 << 22) + 1, 8, 8),
                          (8, 1 << 25, 16, 8)):
        with pytest.raises(HipError) as e:
            dev.mlp2(1, None, 1, 1, None, ACT_NONE, 1, None, M, K1, N1, N2)
        assert e.value.code == -3
    with pytest.raises(HipError) as e:
        dev.mlp2(1, None, 1, 1, None, ACT_NONE, 1, None, 8, 8, 8, 8, act2=7)
    assert e.value.code != 0
