"""One parity case for every kernel variant the dispatch can reach that the
config-level tests do not already launch: the staged GEMM configurations
with transposed, unaligned or short-K operands, the skinny GEMM's
transposed-A and scalar-B forms, row kernels at every register width, the
decode kernel at every head-group width with and without float4 loads, the
direct and implicit-GEMM convs with filters other than 3x3, the staged
weight-gradient kernel, the unaligned small-batch MLP chains, the scalar
tail of the elementwise kernels and the device-ceiling probes.  Each case
names the variant it is there for; a kernel trace of the GPU suite lists
every kernel of liblancius_hip.so as launched.  Tolerance as everywhere:
1e-4 * max(1, sqrt(K)/32) with K the longest reduction."""
import numpy as np
import pytest

import oracle
from lancius_amd import ACT_GELU, ACT_NONE, ACT_RELU, prng
from tests.conftest import case

pytestmark = pytest.mark.gpu


def _up(dev, a):
    return dev.upload(np.ascontiguousarray(a, dtype=np.float32))


def _band_rows(M, band=128):
    rows = {0, M - 1}
    for b in range((M + band - 1) // band):
        rows.add(min(M - 1, b * band + (41 * b + 7) % band))
    return np.asarray(sorted(rows))


def _gemm_ex_case(dev, M, K, N, ta, tb, seed, act=ACT_GELU):
    A, B, bias = prng.normal(seed, (M, K)), prng.normal(seed + 1, (K, N)), prng.normal(seed + 2, (N,))
    dA = _up(dev, A.T if ta else A)
    dB = _up(dev, B.T if tb else B)
    db, dC = _up(dev, bias), dev.alloc(M * N * 4)
    dev.fill(dC, float("nan"), M * N)
    case(f"gemm_ex M={M} K={K} N={N} ta={ta} tb={tb} act={act}")
    dev.gemm_ex(dC, dA, dB, M, K, N, trans_a=ta, trans_b=tb, bias=db, act=act)
    got = dev.download(dC, (M, N))
    for b in (dA, dB, db, dC):
        b.free()
    assert np.isfinite(got).all()
    rows = _band_rows(M) if M * N > 1_000_000 else np.arange(M)
    ref = oracle.matmul(A[rows], B) + bias.astype(np.float64)[None, :]
    ref = oracle.gelu(ref) if act == ACT_GELU else oracle.relu(ref) if act == ACT_RELU else ref
    assert oracle.normwise_error(got[rows], ref) <= oracle.tolerance(K)


# (M, K, N, ta, tb, variant)
STAGED = [
    # 128x128/16 tiles (>= 256 of them) with transposed operands, float4 and scalar loads
    (2048, 260, 2048, True, False, "cfg 6, A^T, float4"),
    (2048, 260, 2048, False, True, "cfg 6, B^T, float4"),
    (2048, 260, 2048, True, True, "cfg 6, A^T B^T, float4"),
    (2048, 259, 2050, True, False, "cfg 6, A^T, scalar"),
    (2046, 259, 2048, False, True, "cfg 6, B^T, scalar"),
    (2046, 260, 2050, True, True, "cfg 6, A^T B^T, scalar"),
    # plain operands, >= 768 tiles, K % 4 != 0: the scalar 128x128/16 kernel
    (3600, 101, 3600, False, False, "cfg 6, plain, scalar"),
    # 128x128/32 with 2 k-groups, split K, scalar loads
    (520, 2101, 500, False, False, "cfg 7, split, scalar"),
    # 128x128/32 with 4 k-groups (256..383 tiles), K < 256 float4 and scalar
    (2048, 72, 2048, False, False, "cfg 8, float4"),
    (2048, 73, 2048, False, False, "cfg 8, scalar"),
    # 64x64/64 with 4 k-groups, unsplit (K < 256), float4 and scalar
    (600, 100, 700, False, False, "cfg 9, float4"),
    (601, 101, 703, False, False, "cfg 9, scalar"),
    # 64x64/16 split K with transposed operands and scalar loads
    (100, 1001, 90, True, False, "cfg 2, A^T, split, scalar"),
    (100, 1001, 90, False, True, "cfg 2, B^T, split, scalar"),
    (100, 1001, 90, True, True, "cfg 2, A^T B^T, split, scalar"),
]


@pytest.mark.parametrize("M,K,N,ta,tb,variant", STAGED, ids=[s[-1] for s in STAGED])
def test_gemm_staged_variants(dev, M, K, N, ta, tb, variant):
    _gemm_ex_case(dev, M, K, N, ta, tb, seed=1300 + M + K + N)


@pytest.mark.parametrize("M", [16, 32])
@pytest.mark.parametrize("ta", [False, True])
@pytest.mark.parametrize("N", [256, 258])
@pytest.mark.parametrize("K", [400, 3000])
def test_gemm_skinny_variants(dev, M, ta, N, K):
    """M <= 16 / 17..32 rows, A or A^T, float4 or scalar B and C, one K
    slice or several summed inside the launch."""
    _gemm_ex_case(dev, M, K, N, ta, False, seed=1400 + M + N + K, act=ACT_RELU)


@pytest.mark.parametrize("op", ["layernorm", "softmax", "rmsnorm"])
@pytest.mark.parametrize("cols", [400, 2000])
def test_row_kernel_widths(dev, op, cols):
    """Rows of 257..512 and 1025..2048 floats: the two- and eight-piece
    register kernels."""
    rows = 37
    x = prng.normal(1500 + cols, (rows, cols), 0.3, 2.0)
    g, b = prng.normal(1501, (cols,), 1.0, 0.1), prng.normal(1502, (cols,), 0.0, 0.1)
    dx, dg, db, do = _up(dev, x), _up(dev, g), _up(dev, b), dev.alloc(4 * x.size)
    case(f"{op} {rows}x{cols}")
    if op == "layernorm":
        dev.layernorm(do, dx, dg, db, rows, cols)
        ref = oracle.layernorm(x, g, b)
    elif op == "softmax":
        dev.softmax(do, None, dx, rows, cols)
        ref = oracle.softmax(x)
    else:
        dev.rmsnorm(do, dx, dg, rows, cols)
        ref = oracle.rmsnorm(x, g)
    got = dev.download(do, x.shape)
    for t in (dx, dg, db, do):
        t.free()
    assert oracle.normwise_error(got, ref) <= oracle.tolerance(cols)


@pytest.mark.parametrize("D", [37, 64, 101, 128])
@pytest.mark.parametrize("G", [1, 2, 4, 8])
def test_decode_variants(dev, D, G):
    """Four or eight values per lane (D <= 64 / D > 64), float4 or scalar
    row pieces (D % 4), query heads per K/V head 1, 2, 4 and 8 (the head
    chunk of a workgroup), several key ranges merged in the launch."""
    B, Skv, Hkv = 2, 600, 2
    Hq = Hkv * G
    q = prng.uniform(1600 + D, (B, Hq, D), -1.0, 1.0)
    k = prng.uniform(1601 + D, (B, Skv, Hkv, D), -1.0, 1.0)
    v = prng.uniform(1602 + D, (B, Skv, Hkv, D), -1.0, 1.0)
    lens = np.asarray([Skv, 257], np.int32)
    dq, dk, dv, do, dl = _up(dev, q), _up(dev, k), _up(dev, v), dev.alloc(4 * q.size), dev.upload(lens)
    dev.fill(do, float("nan"), q.size)
    case(f"decode D={D} G={G}")
    dev.attention_decode(do, dq, dk, dv, dl, B, Skv, Hq, Hkv, D)
    got = dev.download(do, q.shape)
    for t in (dq, dk, dv, do, dl):
        t.free()
    assert oracle.normwise_error(got, oracle.attention_decode(q, k, v, lens)) <= oracle.tolerance(Skv)


# (N, C_in, H, W, C_out, K, stride, pad, variant)
CONVS = [
    (2, 16, 20, 20, 128, 5, 1, 2, "direct 128x64 tiles, 5x5 filter"),
    (2, 16, 21, 19, 64, 1, 1, 0, "direct 64x64 tiles, 1x1 filter"),
    (2, 16, 20, 20, 100, 3, 1, 1, "direct 128x64 tiles, a partial channel block (bias rows past C_out)"),
    (3, 32, 13, 17, 36, 3, 1, 1, "direct 64x64 tiles, a partial channel block"),
    (2, 3, 20, 20, 128, 5, 1, 2, "implicit GEMM 128x64 tiles, OIHW filter"),
    (2, 3, 20, 20, 64, 5, 2, 1, "implicit GEMM 64x64 tiles, OIHW filter"),
    (2, 6, 15, 15, 96, 3, 1, 1, "implicit GEMM 128x64 tiles, 3x3 OIHW filter"),
    # grids under half the CUs: every workgroup an equal share of the
    # (tile, k-tile) units, a tile split 2, 4, 8 ways, the last sharer adding
    (1, 64, 56, 56, 128, 3, 1, 1, "direct, small grid split 2 ways (49 tiles)"),
    (1, 128, 28, 28, 256, 3, 1, 1, "direct, small grid split 4 ways (26 tiles)"),
    (1, 256, 14, 14, 512, 3, 1, 1, "direct, small grid split 8 ways (16 tiles)"),
    (1, 80, 23, 23, 100, 3, 1, 1, "direct, small grid split 2 ways, ragged tiles"),
]


@pytest.mark.parametrize("N,C_in,H,W,C_out,K,stride,pad,variant", CONVS, ids=[c[-1] for c in CONVS])
def test_conv_variants(dev, N, C_in, H, W, C_out, K, stride, pad, variant):
    x = prng.normal(1700 + C_in, (N, C_in, H, W))
    w = prng.normal(1701 + C_out, (C_out, C_in, K, K), 0, float(np.sqrt(2.0 / (C_in * K * K))))
    bias = prng.normal(1702, (C_out,), 0, 0.1)
    Ho, Wo = (H + 2 * pad - K) // stride + 1, (W + 2 * pad - K) // stride + 1
    dx, dw, db, do = _up(dev, x), _up(dev, w), _up(dev, bias), dev.alloc(4 * N * C_out * Ho * Wo)
    dev.fill(do, float("nan"), N * C_out * Ho * Wo)
    case(f"conv {variant}")
    dev.conv2d(do, dx, dw, db, N, C_in, H, W, C_out, K, K, stride, pad, act=ACT_RELU)
    got = dev.download(do, (N, C_out, Ho, Wo))
    for t in (dx, dw, db, do):
        t.free()
    ref = oracle.relu(oracle.conv2d(x, w, stride, pad, False) + bias.astype(np.float64)[None, :, None, None])
    assert oracle.normwise_error(got, ref) <= oracle.tolerance(C_in * K * K)


def test_conv_wgrad_staged_128(dev):
    """Weight gradient with more than 64 output channels and H_out * W_out
    not a multiple of 4: the register-staged kernel at 128 x 64 tiles."""
    N, Ci, H, W, Co = 2, 8, 7, 7, 96
    x, g = prng.normal(1800, (N, Ci, H, W)), prng.normal(1801, (N, Co, H, W))
    dx_, dg_, dw_ = _up(dev, x), _up(dev, g), dev.alloc(4 * Co * Ci * 9)
    case("conv wgrad staged 128x64")
    dev.conv2d_bwd_weight(dw_, dg_, dx_, N, Ci, H, W, Co, H, W, 3, 3, 1, 1)
    got = dev.download(dw_, (Co, Ci, 3, 3))
    for t in (dx_, dg_, dw_):
        t.free()
    ref = oracle.conv2d_bwd_weight(g.astype(np.float32), x.astype(np.float32), (Co, Ci, 3, 3), 1, 1)
    assert oracle.normwise_error(got, ref) <= oracle.tolerance(N * H * W)


# (M, K1, N1, N2, variant): scalar x / W1 loads (K1 % 4 != 0)
CHAINS = [(64, 785, 256, 10, "mlp2_tiles, groups of 13"), (64, 1021, 128, 10, "mlp2_tiles, groups of 16"),
          (16, 9001, 64, 32, "mlp2_split")]


@pytest.mark.parametrize("M,K1,N1,N2,variant", CHAINS, ids=[c[-1] for c in CHAINS])
def test_mlp_chain_scalar_variants(dev, M, K1, N1, N2, variant):
    x = prng.uniform(1900 + K1, (M, K1), -1.0, 1.0)
    w1, w2 = prng.normal(1901, (K1, N1), 0, 0.05), prng.normal(1902, (N1, N2), 0, 0.1)
    b1, b2 = prng.normal(1903, (N1,), 0, 0.05), prng.normal(1904, (N2,), 0, 0.05)
    dx, dw1, dw2, db1, db2 = (_up(dev, a) for a in (x, w1, w2, b1, b2))
    out, am = dev.alloc(M * N2 * 4), dev.alloc(M * 4)
    case(f"mlp chain {variant} M={M} K1={K1} N1={N1} N2={N2}")
    dev.mlp2(out, am, dx, dw1, db1, ACT_RELU, dw2, db2, M, K1, N1, N2, True)
    got, idx = dev.download(out, (M, N2)), dev.download(am, (M,), np.int32)
    for t in (dx, dw1, dw2, db1, db2, out, am):
        t.free()
    h = oracle.relu(oracle.matmul(x, w1) + b1.astype(np.float64)[None, :])
    ref = oracle.softmax(oracle.matmul(h, w2) + b2.astype(np.float64)[None, :])
    assert oracle.normwise_error(got, ref) <= oracle.tolerance(K1)
    assert np.array_equal(idx, oracle.argmax(ref))


def test_tanh_scalar_tail(dev):
    """1001 elements: float4 body plus the scalar kernel for the last one."""
    x = prng.normal(2000, (1001,), 0.0, 3.0)
    dx, do = _up(dev, x), dev.alloc(4 * x.size)
    case("tanh 1001")
    dev.tanh(do, dx, x.size)
    got = dev.download(do, x.shape)
    for t in (dx, do):
        t.free()
    assert np.max(np.abs(got - np.tanh(x.astype(np.float32).astype(np.float64)))) <= 2e-7


@pytest.mark.parametrize("which,low", [("mfma", 50.0), ("hbm", 1000.0), ("hbm_read", 1000.0)])
def test_device_ceiling_probes(dev, which, low):
    """The bench's ceiling probes (MFMA-only kernel in TFLOP/s, 1 GiB copy and
    read in GB/s) run and report a plausible rate."""
    case(f"peak probe {which}")
    assert dev.peak_probe(which) > low


def test_conv_input_beyond_2gib(dev):
    """An input over 2 GiB (1040 images of 64 x 90 x 90): the conv runs as
    launches over runs of whole images under 2 GiB each (the direct kernel's
    32-bit offsets), 1035 images and then 5.  Images on both sides of the
    split carry random data and are checked against the oracle; the rest
    hold a constant, and every output must be finite."""
    N, C_in, H, W, C_out = 1040, 64, 90, 90, 64
    img = C_in * H * W
    assert N * img * 4 >= 1 << 31
    per = ((1 << 31) - 65) // (img * 4)
    sample = [0, per - 1, per, N - 1]
    w = prng.normal(2100, (C_out, C_in, 3, 3), 0, float(np.sqrt(2.0 / (9 * C_in))))
    dx, dw, do = dev.alloc(4 * N * img), _up(dev, w), dev.alloc(4 * N * C_out * H * W)
    dev.fill(dx, 0.25, N * img)
    dev.fill(do, float("nan"), N * C_out * H * W)
    xs = {}
    for i, n in enumerate(sample):
        xs[n] = prng.normal(2110 + i, (1, C_in, H, W))
        dev.write(int(dx) + 4 * n * img, np.ascontiguousarray(xs[n], np.float32))
    case(f"conv input beyond 2 GiB: N={N} C_in={C_in} {H}x{W} C_out={C_out}")
    dev.conv2d(do, dx, dw, None, N, C_in, H, W, C_out, 3, 3, 1, 1, act=ACT_RELU)
    dev.synchronize()
    for n in sample:
        got = dev.download(int(do) + 4 * n * C_out * H * W, (1, C_out, H, W))
        ref = oracle.conv2d(xs[n], w, 1, 1, True)
        assert oracle.normwise_error(got, ref) <= oracle.tolerance(9 * C_in), n
    # a constant image's interior is the filter sum times the constant (ReLU of it)
    mid = dev.download(int(do) + 4 * (N // 2) * C_out * H * W, (C_out, H, W))
    want = np.maximum(0.25 * w.astype(np.float32).astype(np.float64).sum(axis=(1, 2, 3)), 0.0)
    assert np.allclose(mid[:, 1:-1, 1:-1], want[:, None, None], rtol=1e-5, atol=1e-6)
    big = dev.download(do, (N * C_out * H * W,))
    assert np.isfinite(big).all()
    for b in (dx, dw, do):
        b.free()
