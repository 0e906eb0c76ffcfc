"""Pins the fp64 oracle (oracle/liboracle.so) before it is trusted: golden
vectors written by the reference's own compiled C (tests/golden/kernels.npz,
graph_outputs.npz), closed forms, and textbook formulas that a dropped term,
a wrong sign or a transposed operand would break."""
from pathlib import Path

import numpy as np
import pytest

import oracle
from lancius_amd import graph_lib, graphs, prng

GOLD = Path(__file__).resolve().parent / "golden"
K = np.load(GOLD / "kernels.npz")
GO = np.load(GOLD / "graph_outputs.npz")


def close(a, b, rel=1e-12):
    return oracle.normwise_error(a, b) <= rel


# ---- golden vectors of the compiled reference ---------------------------------


def test_matmul_golden():
    assert close(oracle.matmul(K["mm_a"], K["mm_b"]), K["mm_graph_out"])
    assert close(oracle.matmul(K["mm_a"], K["mm_b"]), K["mm_kernel_out"])


def test_conv_golden():
    assert close(oracle.conv2d(K["conv_x"], K["conv_w"], 1, 1, False), K["conv_s1p1"])
    assert close(oracle.conv2d(K["conv_x"], K["conv_w"], 1, 1, True), K["conv_relu_s1p1"])
    assert close(oracle.conv2d(K["conv_x2"], K["conv_w2"], 2, 2, False), K["conv_s2p2"])


@pytest.mark.parametrize("tag", ["attn", "attn2"])
def test_attention_golden(tag):
    got = oracle.attention(K[f"{tag}_q"], K[f"{tag}_k"], K[f"{tag}_v"], causal=True)
    assert close(got, K[f"{tag}_out"])


def test_layernorm_gelu_softmax_golden():
    assert close(oracle.layernorm(K["ln_x"], K["ln_g"], K["ln_b"]), K["ln_out"])
    assert close(oracle.gelu(K["gelu_x"]), K["gelu_out"])
    assert close(oracle.softmax(K["softmax_x"]), K["softmax_out"])


def _run_oracle_graph(bg, feeds):
    lib = graph_lib()
    keep = []
    import ctypes as C

    for name in bg.inputs:
        arr = np.ascontiguousarray(feeds[name], dtype=np.float64)
        keep.append(arr)
        bg.node(name).contents.runtime_data = arr.ctypes.data_as(C.POINTER(C.c_double))
    sched = lib.lancius_ir_schedule(bg.g)
    oracle.schedule_execute(sched)
    out = {}
    from lancius_amd import abi

    for name in bg.outputs:
        n = bg.node(name)
        out[name] = np.ctypeslib.as_array(n.contents.runtime_data, shape=(abi.node_elems(n),)).copy().reshape(
            abi.node_shape(n))
    oracle.release(bg.g)
    for name in bg.inputs:
        bg.node(name).contents.runtime_data = None
    lib.lancius_schedule_destroy(sched)
    return out


def test_graph_executor_mlp_golden():
    bg = graphs.build_mlp(graph_lib())
    feeds = {n: GO[f"mlp_{n}"] for n in bg.inputs}
    out = _run_oracle_graph(bg, feeds)
    assert close(out["softmax"], GO["mlp_softmax"])
    bg.destroy()


def test_graph_executor_conv_golden():
    bg = graphs.build_conv(graph_lib(), N=2, C_in=3, H=8, W=8, C_out=4)
    out = _run_oracle_graph(bg, {"x": GO["conv_x"], "w": GO["conv_w"]})
    assert close(out["relu"], GO["conv_relu"])
    bg.destroy()


def test_graph_executor_block_golden():
    bg = graphs.build_block(graph_lib(), batch=2, S=32, d=64, H=4, F=256)
    out = _run_oracle_graph(bg, {n: GO[f"block_{n}"] for n in bg.inputs})
    for name in bg.outputs:
        assert close(out[name], GO[f"block_out_{name}"]), name
    bg.destroy()


# ---- closed forms and textbook formulas --------------------------------------------


def test_matmul_closed_forms():
    a = np.array([[-1, 2, 3], [4, -5, 6]], float)
    assert oracle.matmul(a, np.ones((3, 4))).tolist() == [[4] * 4, [5] * 4]  # S9/examples/audit_ffi.c:52-61
    x = prng.normal(3, (9, 9)).astype(float)
    assert np.array_equal(oracle.matmul(x, np.eye(9)), x)
    a, b = prng.normal(4, (6, 5)).astype(float), prng.normal(5, (5, 7)).astype(float)
    assert close(oracle.matmul(a, b), a @ b, 1e-14)
    assert close(oracle.matmul(a, b, rows=(2, 4))[2:4], (a @ b)[2:4], 1e-14)


def test_matmul_nan_inf():
    x = np.ones((32, 32))
    w = np.where(np.arange(1024).reshape(32, 32) % 2 == 0, np.nan, np.inf)
    out = oracle.relu(oracle.matmul(x, w))
    assert int(np.sum(~np.isfinite(out))) == 512  # S9/examples/audit_nan_injection.c


def _conv_im2col(x, w, stride, pad):
    N, C, H, W = x.shape
    O, _, KH, KW = w.shape
    xp = np.pad(x, ((0, 0), (0, 0), (pad, pad), (pad, pad)))
    Ho, Wo = (H + 2 * pad - KH) // stride + 1, (W + 2 * pad - KW) // stride + 1
    cols = np.empty((N, C * KH * KW, Ho * Wo))
    for c in range(C):
        for i in range(KH):
            for j in range(KW):
                patch = xp[:, c, i:i + stride * Ho:stride, j:j + stride * Wo:stride]
                cols[:, (c * KH + i) * KW + j, :] = patch.reshape(N, -1)
    return np.einsum("ok,nkp->nop", w.reshape(O, -1), cols).reshape(N, O, Ho, Wo)


@pytest.mark.parametrize("stride,pad,k", [(1, 1, 3), (2, 0, 3), (1, 2, 5), (3, 1, 2)])
def test_conv_equals_im2col_gemm(stride, pad, k):
    x = prng.normal(6, (2, 3, 9, 11)).astype(float)
    w = prng.normal(7, (4, 3, k, k)).astype(float)
    assert close(oracle.conv2d(x, w, stride, pad), _conv_im2col(x, w, stride, pad), 1e-13)


def test_conv_constant_input():
    # every output pixel away from the border sums all taps: value = sum(w[o])
    x = np.full((1, 2, 6, 6), 2.0)
    w = prng.normal(8, (3, 2, 3, 3)).astype(float)
    out = oracle.conv2d(x, w, 1, 1)
    assert np.allclose(out[0, :, 2, 2], 2.0 * w.reshape(3, -1).sum(1), rtol=1e-13)


def _naive_attention(q, k, v, causal):
    S, H, D = q.shape
    out = np.empty_like(q)
    for h in range(H):
        s = q[:, h, :] @ k[:, h, :].T / np.sqrt(D)
        if causal:
            s = np.where(np.triu(np.ones((S, S), bool), 1), -1e9, s)
        p = np.exp(s - s.max(1, keepdims=True))
        out[:, h, :] = (p / p.sum(1, keepdims=True)) @ v[:, h, :]
    return out


@pytest.mark.parametrize("causal", [True, False])
def test_attention_textbook(causal):
    # S9/examples/audit_flash_attention.c:9-49 (naive O(S^2)); the non-causal
    # variant has no reference kernel, only the textbook formula.
    q, k, v = (prng.uniform(20 + i, (40, 3, 16), -1, 1).astype(float) for i in range(3))
    assert close(oracle.attention(q, k, v, causal=causal), _naive_attention(q, k, v, causal), 1e-13)


def test_attention_special_cases():
    q, k = prng.normal(30, (12, 2, 8)).astype(float), prng.normal(31, (12, 2, 8)).astype(float)
    v = np.full((12, 2, 8), -1.25)
    assert np.allclose(oracle.attention(q, k, v), -1.25, rtol=1e-14)  # V constant => out constant
    v = prng.normal(32, (1, 2, 8)).astype(float)
    assert np.allclose(oracle.attention(q[:1], k[:1], v), v, rtol=1e-14)  # S = 1 => v0
    v = prng.normal(33, (12, 2, 8)).astype(float)
    prefix = np.cumsum(v, axis=0) / np.arange(1, 13)[:, None, None]
    assert close(oracle.attention(np.zeros_like(q), k, v, causal=True), prefix, 1e-14)  # q = 0


def test_layernorm_closed_forms():
    x = np.full((3, 8), 7.0)
    b = prng.normal(40, (8,)).astype(float)
    assert np.array_equal(oracle.layernorm(x, np.ones(8), b), np.broadcast_to(b, (3, 8)))  # constant row => beta
    x = prng.normal(41, (4, 50)).astype(float)
    ref = (x - x.mean(1, keepdims=True)) / np.sqrt(x.var(1, keepdims=True) + 1e-5)
    assert close(oracle.layernorm(x, np.ones(50), np.zeros(50)), ref, 1e-13)


def test_gelu_closed_forms():
    out = oracle.gelu(np.array([0.0, 150.0, -150.0, np.nan]))
    assert out[0] == 0.0 and out[1] == 100.0 and out[2] == 0.0 and np.isnan(out[3])
    x = np.linspace(-6, 6, 101)
    ref = 0.5 * x * (1 + np.tanh(np.sqrt(2 / np.pi) * (x + 0.044715 * x ** 3)))
    assert close(oracle.gelu(x), ref, 1e-14)


def test_softmax_argmax_closed_forms():
    x = np.zeros((2, 10))
    assert np.allclose(oracle.softmax(x), 0.1, rtol=1e-15)  # audit_internals: uniform 0.1 x 10
    x = prng.normal(50, (6, 7)).astype(float)
    assert np.allclose(oracle.softmax(x).sum(1), 1.0, rtol=1e-14)
    t = np.array([[1, 5, 5, 2], [-3e9, -2e9, -4e9, -5e9], [0, 0, 0, 0.0]])
    assert oracle.argmax(t).tolist() == [1, 0, 0]  # first max; all <= -1e9 => 0


def test_broadcast_add_relu():
    a = np.arange(5.0)
    assert np.array_equal(oracle.broadcast(a, 3, 5), np.tile(a, (3, 1)))
    assert np.array_equal(oracle.broadcast(np.array([2.5]), 2, 4), np.full((2, 4), 2.5))
    x = np.array([-1.0, 0.0, 2.0, np.nan])
    assert oracle.relu(x).tolist() == [0.0, 0.0, 2.0, 0.0]
    assert oracle.add(x[:3], x[:3]).tolist() == [-2.0, 0.0, 4.0]


def test_prng_documented_values():
    # SplitMix64 seeded with 0: first outputs of the published algorithm.
    z = prng.splitmix64(0, 3)
    assert [int(v) for v in z] == [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F]
    u = prng.uniform(42, (100000,), dtype=np.float64)
    assert 0.49 < u.mean() < 0.51 and u.min() >= 0.0 and u.max() < 1.0
    n = prng.normal(42, (200001,), dtype=np.float64)
    assert abs(n.mean()) < 0.01 and abs(n.std() - 1.0) < 0.01
