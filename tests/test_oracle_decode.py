"""The oracle's decode-side family (RMSNorm, SwiGLU, RoPE, GQA attention,
KV-cache decode attention), pinned by the compiled reference's kernels and
scheduler branches (tests/golden/kernels.npz) and by closed forms: RoPE is a
rotation (norms kept, undone at the negated position), GQA with Hkv = Hq is
plain causal attention, decode equals the last row of causal attention over
the cache, and a longer key sequence shifts the causal diagonal."""
from pathlib import Path

import numpy as np
import pytest

import oracle
from lancius_amd import prng

K = np.load(Path(__file__).resolve().parent / "golden" / "kernels.npz")


def close(got, ref, tol=1e-12):
    assert oracle.normwise_error(got, ref) <= tol


def test_rmsnorm_swiglu_golden():
    close(oracle.rmsnorm(K["rms_x"], K["rms_g"]), K["rms_out"])
    close(oracle.rmsnorm(K["rms_x"], K["rms_g"]), K["node_rms_out"])
    close(oracle.swiglu(K["swiglu_gate"], K["swiglu_up"]), K["swiglu_out"])
    close(oracle.swiglu(K["swiglu_gate"], K["swiglu_up"]).reshape(8, 8), K["node_swiglu_out"])


def test_rope_golden_and_rotation():
    both = np.concatenate([K["rope_q"].ravel(), K["rope_k"].ravel()])
    got = oracle.rope(both, 2, 1, 7, 3, 8, 5)
    close(got[:168].reshape(K["rope_q"].shape), K["rope_q_out"])
    close(got[168:].reshape(K["rope_k"].shape), K["rope_k_out"])
    # the ROPE node: [S, H, 2 hd] buffer = q block then k block (lancius_scheduler.c:153-165)
    close(oracle.rope(K["node_rope_x"].ravel(), 2, 1, 7, 3, 8, 0).reshape(7, 3, 16), K["node_rope_out"])
    # a rotation: pair norms kept, the inverse rotation restores the input
    x = prng.normal(70, (2, 5, 3, 8)).astype(np.float64)
    y = oracle.rope(x, 1, 2, 5, 3, 8, 11)
    np.testing.assert_allclose(np.hypot(y[..., 0::2], y[..., 1::2]), np.hypot(x[..., 0::2], x[..., 1::2]),
                               rtol=1e-13)
    back = np.empty_like(y)
    for s in range(5):  # position s + 11 undone by -(s + 11)
        back[:, s] = oracle.rope(y[:, s:s + 1].copy(), 1, 2, 1, 3, 8, -(s + 11))[:, 0]
    np.testing.assert_allclose(back, x, atol=1e-12)


def test_gqa_golden_and_closed_forms():
    q, k, v = K["gqa_q"][None], K["gqa_k"][None], K["gqa_v"][None]
    close(oracle.attention_gqa(q, k, v)[0], K["gqa_out"])
    close(oracle.attention_gqa(q, k, v)[0], K["node_gqa_out"])
    # Hkv = Hq: the causal attention oracle
    q2 = prng.normal(71, (2, 10, 4, 8)).astype(np.float64)
    k2, v2 = prng.normal(72, (2, 10, 4, 8)).astype(np.float64), prng.normal(73, (2, 10, 4, 8)).astype(np.float64)
    close(oracle.attention_gqa(q2, k2, v2), oracle.attention(q2, k2, v2, causal=True))
    # GQA = MHA with each K/V head repeated over its group
    kg, vg = k2[:, :, :2], v2[:, :, :2]
    close(oracle.attention_gqa(q2, kg, vg), oracle.attention(q2, np.repeat(kg, 2, axis=2), np.repeat(vg, 2, axis=2)))
    # 3 queries against 10 keys = the last 3 rows of 10-query causal attention
    close(oracle.attention_gqa(q2[:, 7:], k2, v2), oracle.attention(q2, k2, v2, causal=True)[:, 7:])


def test_decode_golden_and_closed_forms():
    q, kc, vc = K["kvc_q"].reshape(1, 4, 16), K["kvc_k"][None], K["kvc_v"][None]
    close(oracle.attention_decode(q, kc, vc).reshape(4, 16), K["kvc_out"])
    # the last row of causal attention over the cache
    B, S, Hq, Hkv, D = 3, 20, 8, 2, 16
    qs = prng.normal(74, (B, S, Hq, D)).astype(np.float64)
    ks, vs = prng.normal(75, (B, S, Hkv, D)).astype(np.float64), prng.normal(76, (B, S, Hkv, D)).astype(np.float64)
    full = oracle.attention_gqa(qs, ks, vs)
    close(oracle.attention_decode(qs[:, -1], ks, vs), full[:, -1])
    # per-sequence lengths: the first len keys only; an empty cache gives zeros
    lens = np.array([20, 7, 0], np.int32)
    got = oracle.attention_decode(qs[:, -1], ks, vs, lens)
    close(got[0], full[0, -1])
    close(got[1], oracle.attention_decode(qs[1:2, -1], ks[1:2, :7], vs[1:2, :7])[0])
    assert not got[2].any()
