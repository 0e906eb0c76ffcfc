"""Parity of every HIP kernel, called through the C ABI, against the fp64 CPU
oracle on identical seeded fp32 inputs.

Bar: normwise error max|y - y_ref| / max|y_ref| <=
1e-4 * max(1, sqrt(K)/32), K the longest reduction; argmax/indices bit-exact.
"""
import numpy as np
import pytest

import oracle
from lancius_amd import ACT_GELU, ACT_NONE, ACT_RELU, HipError, prng
from tests.conftest import case, record_parity

pytestmark = pytest.mark.gpu

TOL_ELEMENTWISE = 1e-6  # fp32 rounding of one op (GELU's tanh included)


def _upload(dev, *arrs):
    return [dev.upload(np.ascontiguousarray(a, dtype=np.float32)) for a in arrs]


def _gemm_case(dev, M, K, N, seed, bias=False, act=ACT_NONE, residual=False, rows=None, row_list=None):
    """C is filled with NaN before the call, so an element the kernel never
    writes shows up in the finite check of the caller.  rows = (r0, r1) or
    row_list = [r, ...] restricts the fp64 oracle (and the returned pair) to
    those rows of the full product."""
    A = prng.normal(seed, (M, K))
    B = prng.normal(seed + 1000, (K, N))
    bv = prng.normal(seed + 2000, (N,)) if bias else None
    R = prng.normal(seed + 3000, (M, N)) if residual else None
    dA, dB = _upload(dev, A, B)
    dbias = dev.upload(bv) if bias else None
    dR = dev.upload(R) if residual else None
    dC = dev.alloc(M * N * 4)
    dev.fill(dC, float("nan"), M * N)
    case(f"gemm M={M} K={K} N={N} bias={bias} act={act} res={residual}")
    dev.gemm(dC, dA, dB, M, K, N, bias=dbias, act=act, residual=dR)
    got = dev.download(dC, (M, N))
    assert np.isfinite(got).all(), f"{np.count_nonzero(~np.isfinite(got))} elements of C not written"
    if row_list is not None:
        sel = np.asarray(row_list)
        ref = oracle.matmul(A[sel], B)
        Rs = R[sel] if residual else None
    else:
        ref = oracle.matmul(A, B, rows=rows)
        sel = slice(*rows) if rows else slice(None)
        ref = ref[sel]
        Rs = R[sel] if residual else None
    if bias:
        ref = ref + bv.astype(np.float64)[None, :]
    if act == ACT_RELU:
        ref = oracle.relu(ref)
    elif act == ACT_GELU:
        ref = oracle.gelu(ref)
    if residual:
        ref = ref + Rs.astype(np.float64)
    for b in (dA, dB, dC, dbias, dR):
        if b is not None:
            b.free()
    return got[sel], ref


def band_rows(M, band=128, per_band=2):
    """per_band rows of every band-row tile band of an M-row output, at
    offsets that differ from band to band, plus the first and last row."""
    rows = {0, M - 1}
    for b in range((M + band - 1) // band):
        for j in range(per_band):
            rows.add(min(M - 1, b * band + (37 * b + 61 * j + 5) % band))
    return sorted(rows)


@pytest.mark.parametrize("M,K,N", [(1, 1, 1), (7, 13, 5), (64, 784, 256), (64, 256, 10), (130, 70, 200),
                                   (257, 129, 131), (33, 64, 96), (300, 1000, 260)])
def test_gemm_shapes(dev, M, K, N):
    got, ref = _gemm_case(dev, M, K, N, seed=100 + M + K + N)
    assert oracle.normwise_error(got, ref) <= oracle.tolerance(K)


@pytest.mark.parametrize("act", [ACT_NONE, ACT_RELU, ACT_GELU])
@pytest.mark.parametrize("bias,residual", [(True, False), (True, True), (False, True)])
def test_gemm_epilogues(dev, act, bias, residual):
    got, ref = _gemm_case(dev, 96, 200, 160, seed=7, bias=bias, act=act, residual=residual)
    assert oracle.normwise_error(got, ref) <= oracle.tolerance(200)


@pytest.mark.parametrize("act", [ACT_NONE, ACT_RELU, ACT_GELU])
@pytest.mark.parametrize("bias,residual", [(True, True), (False, True), (True, False)])
def test_gemm_direct_epilogues(dev, act, bias, residual):
    """The 128x128 direct kernel (>= 768 tiles) with every epilogue: whole
    tiles take the unchecked store path, the last tile-row (3000 = 23 x 128
    + 56) and tile-column (4000 = 31 x 128 + 32) the bounded one, each
    loading a block's residual values before its stores.  Rows sampled from
    every 128-row band, the edge band's included."""
    M, K, N = 3000, 256, 4000
    rows = band_rows(M) + [2944, 2999]
    got, ref = _gemm_case(dev, M, K, N, seed=61, bias=bias, act=act, residual=residual, row_list=sorted(set(rows)))
    assert oracle.normwise_error(got, ref) <= oracle.tolerance(K)


@pytest.mark.parametrize("M,K,N", [(1024, 1024, 1024), (16, 4096, 4096)])
def test_gemm_config_full(dev, M, K, N):
    got, ref = _gemm_case(dev, M, K, N, seed=43)
    err = oracle.normwise_error(got, ref)
    record_parity(f"gemm {M}x{K}x{N} (every element)", err, oracle.tolerance(K))
    assert err <= oracle.tolerance(K)


@pytest.mark.parametrize("n", [2048, 4096])
def test_gemm_config_every_band(dev, n):
    """Every element is written (NaN-filled C comes back finite), and two
    rows of every 128-row tile band, across all columns (so every 128x128
    tile), are exact fp64 oracle rows of the full product: the XCD
    renumbering and raster of the tiles cannot drop or misplace a tile."""
    got, ref = _gemm_case(dev, n, n, n, seed=43, row_list=band_rows(n))
    err = oracle.normwise_error(got, ref)
    record_parity(f"gemm {n}^3 (two rows of every 128-row band)", err, oracle.tolerance(n))
    assert err <= oracle.tolerance(n)


@pytest.mark.parametrize("M,K,N", [
    (2048, 1000, 2048),  # direct loads, 64x64 tiles, 2 k-groups; K crosses a 16-deep k-tile
    (1000, 1028, 1100),  # direct loads, 64x64 tiles, 4 k-groups, ragged edges
    (3000, 4096, 1500),  # direct loads, 128x128 tiles, 4 k-groups, ragged edges
    (2048, 72, 3072),    # K < 256: staged, 384 tiles of 128^2 with 2 k-groups
    (2000, 40, 2990),    # 384 tiles, N % 4 != 0: scalar loads
    (520, 2100, 500),    # 20 tiles, K >= 2048: 2 k-groups with split K, ragged edges
    (600, 300, 700),     # 64x64 tiles with 4 k-groups (staged), ragged edges
    (601, 301, 703),     # same, K % 4 != 0: scalar loads
])
def test_gemm_tile_paths(dev, M, K, N):
    """Each default tile path of the GEMM dispatch (k-groups reduce their
    accumulators through LDS before the epilogue), with bias, GELU and a
    residual; rows of every 128-row band for the two largest products."""
    rows = band_rows(M) if M * N >= 4_000_000 else None
    got, ref = _gemm_case(dev, M, K, N, seed=120 + M + N, bias=True, act=ACT_GELU, residual=True, row_list=rows)
    assert oracle.normwise_error(got, ref) <= oracle.tolerance(K)


@pytest.mark.parametrize("M,K,N,act", [(100, 2000, 120, ACT_NONE), (33, 1500, 64, ACT_GELU),
                                       (16, 4096, 260, ACT_RELU), (5, 777, 9, ACT_NONE),
                                       (24, 1024, 200, ACT_GELU), (8, 200, 64, ACT_RELU), (32, 2052, 4100, ACT_NONE),
                                       (1, 4096, 4096, ACT_NONE)])
def test_gemm_split_k(dev, M, K, N, act):
    # grids this small split K; partials are summed in a fixed order
    got, ref = _gemm_case(dev, M, K, N, seed=61, bias=True, act=act, residual=True)
    assert oracle.normwise_error(got, ref) <= oracle.tolerance(K)


@pytest.mark.parametrize("M,K,N", [(16, 4096, 4096), (32, 8192, 1000), (5, 3000, 77)])
def test_gemm_skinny_fused_split_repeatable(dev, M, K, N):
    """The skinny kernel adds its K slices inside the launch (partials through
    the point of coherence, the last-arriving workgroup reduces in slice
    order): eight calls in a row give the same bits, and the oracle's values."""
    A, B = prng.normal(31 + M, (M, K)), prng.normal(32 + N, (K, N))
    bv, R = prng.normal(33, (N,)), prng.normal(34, (M, N))
    dA, dB, db, dR = _upload(dev, A, B, bv, R)
    dC = dev.alloc(M * N * 4)
    case(f"skinny fused split M={M} K={K} N={N} x8")
    outs = []
    for _ in range(8):
        dev.fill(dC, float("nan"), M * N)
        dev.gemm(dC, dA, dB, M, K, N, bias=db, act=ACT_RELU, residual=dR)
        outs.append(dev.download(dC, (M, N)))
    for o in outs[1:]:
        assert np.array_equal(o.view(np.uint32), outs[0].view(np.uint32))
    ref = oracle.relu(oracle.matmul(A, B) + bv.astype(np.float64)[None, :]) + R.astype(np.float64)
    assert oracle.normwise_error(outs[0], ref) <= oracle.tolerance(K)
    for b in (dA, dB, db, dR, dC):
        b.free()


@pytest.mark.parametrize("M,K,N", [
    (16, 4096, 4096),   # the skinny config: 64 column blocks x 8 K slices
    (1, 100, 4096),     # one row; one K slice of 100 rows (two waves)
    (17, 1000, 4100),   # two row tiles (rows 17..31 absent); N % 64 = 4: a partial last column block
    (32, 16, 8192),     # K = 16: seven of the eight waves hold no rows
    (24, 8200, 4096),   # 17 K slices: the reducer adds them in two batches of loads
])
def test_gemm_skinny_wide(dev, M, K, N):
    """M <= 32 and N >= 4096 through the B-streaming skinny kernel.  C is
    NaN-filled, so every element must be written; bias, GELU and a
    residual; every row is checked against the fp64 oracle, and two calls
    give the same bits."""
    got, ref = _gemm_case(dev, M, K, N, seed=150 + M + K, bias=True, act=ACT_GELU, residual=True)
    assert oracle.normwise_error(got, ref) <= oracle.tolerance(K)
    again, _ = _gemm_case(dev, M, K, N, seed=150 + M + K, bias=True, act=ACT_GELU, residual=True)
    assert np.array_equal(got.view(np.uint32), again.view(np.uint32))


@pytest.mark.parametrize("M,K,N", [(64, 4096, 2048), (48, 2048, 4096), (33, 4096, 2050)])
def test_gemm_rows_33_to_64_as_two_skinny_products(dev, M, K, N):
    """32 < M <= 64 with B of at least 32 MiB: rows 0-31 and 32..M-1 run as
    two skinny products (A, C and the residual offset by 32 rows).  C is
    NaN-filled; bias, GELU and a residual; every row against the oracle;
    M = 33 leaves a one-row second product, N % 4 != 0 the scalar-B path."""
    got, ref = _gemm_case(dev, M, K, N, seed=160 + M + K, bias=True, act=ACT_GELU, residual=True)
    assert oracle.normwise_error(got, ref) <= oracle.tolerance(K)


@pytest.mark.parametrize("M,K,N", [(128, 2048, 4096), (4096, 1024, 96)])
def test_gemm_mid_grids_split_k(dev, M, K, N):
    """128 to 191 tiles of 64 x 64 run the split-K tiled kernels (partials
    added by the reduce kernel) rather than the k-group kernel: every
    element against the oracle, with bias, GELU and a residual."""
    got, ref = _gemm_case(dev, M, K, N, seed=165 + M + K, bias=True, act=ACT_GELU, residual=True)
    assert oracle.normwise_error(got, ref) <= oracle.tolerance(K)


@pytest.mark.parametrize("M,K,N", [(768, 2048, 4096), (4096, 2048, 768)])
def test_gemm_k_groups_192_to_255_big_tiles(dev, M, K, N):
    """K >= 2048 with 192 to 255 tiles of 128 x 128: the k-group kernel at
    64 x 64 tiles, two k-groups.  C NaN-filled, bias and a residual, two rows
    of every 128-row band against the oracle (every column)."""
    got, ref = _gemm_case(dev, M, K, N, seed=168 + M, bias=True, residual=True, row_list=band_rows(M))
    assert np.isfinite(got).all()
    assert oracle.normwise_error(got, ref) <= oracle.tolerance(K)


def test_gemm_skinny_grouped(dev):
    """A grouped call (blockIdx.z = member) through the skinny kernel: each
    member against its own oracle product."""
    M, K, N, n = 8, 512, 4096, 3
    As = [prng.normal(170 + i, (M, K)) for i in range(n)]
    Bs = [prng.normal(180 + i, (K, N)) for i in range(n)]
    dAs, dBs = [dev.upload(a) for a in As], [dev.upload(b) for b in Bs]
    dCs = [dev.alloc(M * N * 4) for _ in range(n)]
    for c in dCs:
        dev.fill(c, float("nan"), M * N)
    case(f"skinny grouped x{n} M={M} K={K} N={N}")
    dev.gemm_grouped(dCs, dAs, dBs, M, K, N)
    for i in range(n):
        got = dev.download(dCs[i], (M, N))
        assert np.isfinite(got).all()
        assert oracle.normwise_error(got, oracle.matmul(As[i], Bs[i])) <= oracle.tolerance(K)
    for b in dAs + dBs + dCs:
        b.free()


@pytest.mark.parametrize("M,K,N", [(32, 784, 128), (32, 128, 10), (17, 300, 77), (3, 1000, 1), (64, 784, 128),
                                   (64, 128, 10), (48, 300, 77), (40, 4096, 4096)])
def test_gemm_small_m_and_ragged_n(dev, M, K, N):
    # M <= 32: the B-streaming kernel, N % 4 != 0 through its scalar-B path;
    # 33..64: the tiled kernel with split K
    got, ref = _gemm_case(dev, M, K, N, seed=90 + M + N, bias=True, act=ACT_RELU, residual=True)
    assert oracle.normwise_error(got, ref) <= oracle.tolerance(K)


@pytest.mark.parametrize("M,K,N", [(64, 784, 128), (784, 64, 128), (128, 64, 784), (64, 128, 784), (130, 70, 201),
                                   (300, 1000, 260), (1024, 1024, 1024), (7, 13, 5), (2048, 120, 10), (32, 500, 130),
                                   (16, 4096, 4096)])
@pytest.mark.parametrize("ta,tb", [(True, False), (False, True), (True, True)])
def test_gemm_transposed_operands(dev, M, K, N, ta, tb):
    """A given as A^T [K][M] and/or B as B^T [N][K] (what an absorbed
    TRANSPOSE node hands the GEMM)."""
    A = prng.normal(91 + M, (M, K))
    B = prng.normal(92 + N, (K, N))
    bv = prng.normal(93, (N,))
    dA = dev.upload(np.ascontiguousarray(A.T) if ta else A)
    dB = dev.upload(np.ascontiguousarray(B.T) if tb else B)
    db, dC = dev.upload(bv), dev.alloc(M * N * 4)
    case(f"gemm_ex M={M} K={K} N={N} ta={ta} tb={tb}")
    dev.gemm_ex(dC, dA, dB, M, K, N, trans_a=ta, trans_b=tb, bias=db, act=ACT_GELU)
    got = dev.download(dC, (M, N))
    ref = oracle.gelu(oracle.matmul(A, B) + bv.astype(np.float64)[None, :])
    for b in (dA, dB, db, dC):
        b.free()
    assert oracle.normwise_error(got, ref) <= oracle.tolerance(K)


def test_gemm_split_k_grouped_deterministic(dev):
    M, K, N, G = 50, 3000, 40, 3
    As = [prng.normal(70 + g, (M, K)) for g in range(G)]
    Bs = [prng.normal(80 + g, (K, N)) for g in range(G)]
    dA, dB = _upload(dev, *As), _upload(dev, *Bs)
    dC = [dev.alloc(M * N * 4) for _ in range(G)]
    case("gemm split-k grouped")
    dev.gemm_grouped(dC, dA, dB, M, K, N)
    first = [dev.download(c, (M, N)) for c in dC]
    dev.gemm_grouped(dC, dA, dB, M, K, N)
    for g in range(G):
        again = dev.download(dC[g], (M, N))
        assert np.array_equal(first[g].view(np.uint32), again.view(np.uint32))
        assert oracle.normwise_error(again, oracle.matmul(As[g], Bs[g])) <= oracle.tolerance(K)


def test_gemm_grouped(dev):
    M, K, N, G = 200, 96, 136, 5
    As = [prng.normal(500 + g, (M, K)) for g in range(G)]
    Bs = [prng.normal(600 + g % 2, (K, N)) for g in range(G)]
    bs = [prng.normal(700 + g, (N,)) for g in range(G)]
    Rs = [prng.normal(800 + g, (M, N)) for g in range(G)]
    dA = _upload(dev, *As)
    dB = _upload(dev, *Bs)
    db = _upload(dev, *bs)
    dR = _upload(dev, *Rs)
    dC = [dev.alloc(M * N * 4) for _ in range(G)]
    case("gemm grouped")
    dev.gemm_grouped(dC, dA, dB, M, K, N, biases=db, act=ACT_RELU, residuals=dR)
    for g in range(G):
        ref = oracle.relu(oracle.matmul(As[g], Bs[g]) + bs[g].astype(np.float64)) + Rs[g]
        got = dev.download(dC[g], (M, N))
        assert oracle.normwise_error(got, ref) <= oracle.tolerance(K), g


def test_gemm_grouped_direct_kgroups(dev):
    """A grouped launch through the direct-load k-group kernel (64x64
    tiles, 4 k-groups; grid.z = member) with each member's own B, bias and
    residual, NaN-filled outputs, and repeat calls bit-identical."""
    M, K, N, G = 520, 300, 600, 3
    As = [prng.normal(900 + g, (M, K)) for g in range(G)]
    Bs = [prng.normal(910 + g, (K, N)) for g in range(G)]
    bs = [prng.normal(920 + g, (N,)) for g in range(G)]
    Rs = [prng.normal(930 + g, (M, N)) for g in range(G)]
    dA, dB, db, dR = _upload(dev, *As), _upload(dev, *Bs), _upload(dev, *bs), _upload(dev, *Rs)
    dC = [dev.alloc(M * N * 4) for _ in range(G)]
    for c in dC:
        dev.fill(c, float("nan"), M * N)
    case("gemm grouped, direct k-groups")
    dev.gemm_grouped(dC, dA, dB, M, K, N, biases=db, act=ACT_GELU, residuals=dR)
    first = [dev.download(dC[g], (M, N)) for g in range(G)]
    dev.gemm_grouped(dC, dA, dB, M, K, N, biases=db, act=ACT_GELU, residuals=dR)
    for g in range(G):
        assert np.isfinite(first[g]).all(), g
        ref = oracle.gelu(oracle.matmul(As[g], Bs[g]) + bs[g].astype(np.float64)) + Rs[g]
        assert oracle.normwise_error(first[g], ref) <= oracle.tolerance(K), g
        assert np.array_equal(first[g].view(np.uint32), dev.download(dC[g], (M, N)).view(np.uint32)), g
    for b in dA + dB + db + dR + dC:
        b.free()


def test_gemm_deterministic(dev):
    M = K = N = 512
    A, B = prng.normal(1, (M, K)), prng.normal(2, (K, N))
    dA, dB = _upload(dev, A, B)
    dC = dev.alloc(M * N * 4)
    case("gemm determinism")
    dev.gemm(dC, dA, dB, M, K, N)
    first = dev.download(dC, (M, N))
    dev.gemm(dC, dA, dB, M, K, N)
    second = dev.download(dC, (M, N))
    assert np.array_equal(first.view(np.uint32), second.view(np.uint32))


def test_gemm_nan_inf_propagation(dev):
    # S9/examples/audit_nan_injection.c:13-50: ones . (NaN/Inf alternating)
    # -> MATMUL NaN in even columns, Inf in odd; ReLU maps NaN to 0 -> 512 of
    # 1024 outputs stay non-finite.
    x = np.ones((32, 32), np.float32)
    w = np.where(np.arange(32 * 32).reshape(32, 32) % 2 == 0, np.nan, np.inf).astype(np.float32)
    dx, dw = _upload(dev, x, w)
    dC = dev.alloc(32 * 32 * 4)
    case("gemm nan/inf")
    dev.gemm(dC, dx, dw, 32, 32, 32, act=ACT_RELU)
    got = dev.download(dC, (32, 32))
    assert int(np.sum(~np.isfinite(got))) == 512
    assert np.all(got[:, 0::2] == 0.0) and np.all(np.isposinf(got[:, 1::2]))


def test_kernel_matmul_f32_bridge(dev):
    # The reference-declared host-pointer symbol (lancius_kernels.h:55);
    # audit_ffi closed form: [[-1,2,3],[4,-5,6]] . ones(3,4) = rows of 4 and 5.
    import ctypes as C

    a = np.array([[-1, 2, 3], [4, -5, 6]], np.float32)
    b = np.ones((3, 4), np.float32)
    out = np.zeros((2, 4), np.float32)
    case("kernel_matmul_f32 bridge")
    dev.lib.kernel_matmul_f32(out.ctypes.data_as(C.c_void_p), a.ctypes.data_as(C.c_void_p),
                              b.ctypes.data_as(C.c_void_p), 2, 3, 4)
    assert dev.lib.lancius_hip_last_status() == 0
    assert out.tolist() == [[4, 4, 4, 4], [5, 5, 5, 5]]


def test_kernel_matmul_f32_bridge_4096(dev):
    """The host-pointer bridge at the bench's 4096^3 (host A and B staged
    in, C staged out on every call): every element comes back finite from a
    NaN-filled host C, and two rows of every 128-row band are exact fp64
    oracle rows."""
    import ctypes as C

    n = 4096
    A = np.ascontiguousarray(prng.normal(47, (n, n)), np.float32)
    B = np.ascontiguousarray(prng.normal(1047, (n, n)), np.float32)
    out = np.full((n, n), np.nan, np.float32)
    case("kernel_matmul_f32 bridge 4096^3")
    dev.lib.kernel_matmul_f32(out.ctypes.data_as(C.c_void_p), A.ctypes.data_as(C.c_void_p),
                              B.ctypes.data_as(C.c_void_p), n, n, n)
    assert dev.lib.lancius_hip_last_status() == 0, dev.lib.lancius_hip_last_error()
    assert np.isfinite(out).all()
    sel = np.asarray(band_rows(n))
    err = oracle.normwise_error(out[sel], oracle.matmul(A[sel], B))
    record_parity("kernel_matmul_f32 bridge 4096^3 (two rows of every 128-row band)", err, oracle.tolerance(n))
    assert err <= oracle.tolerance(n)


# ---- attention ---------------------------------------------------------------


def _attn_case(dev, B, S, H, D, causal, seed, batches=None, rows=None, row_list=None):
    """The output is NaN-filled before the call and must come back finite
    everywhere; the oracle covers batches [b0, b1) and rows (r0, r1) or the
    rows in row_list (all by default)."""
    q = prng.normal(seed, (B, S, H, D))
    k = prng.normal(seed + 1, (B, S, H, D))
    v = prng.normal(seed + 2, (B, S, H, D))
    dq, dk, dv = _upload(dev, q, k, v)
    do = dev.alloc(q.nbytes)
    dev.fill(do, float("nan"), q.size)
    case(f"attention B={B} S={S} H={H} D={D} causal={causal}")
    dev.attention(do, dq, dk, dv, B, S, H, D, causal=causal)
    got = dev.download(do, q.shape)
    assert np.isfinite(got).all(), f"{np.count_nonzero(~np.isfinite(got))} output elements not written"
    ref = oracle.attention(q, k, v, causal=causal, batches=batches, rows=rows, row_list=row_list)
    for b in (dq, dk, dv, do):
        b.free()
    bs = slice(*batches) if batches else slice(None)
    rs = np.asarray(row_list) if row_list is not None else slice(*rows) if rows else slice(None)
    return got[bs][:, rs], ref[bs][:, rs]


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("B,S,H,D", [(1, 1, 1, 64), (1, 17, 2, 8), (2, 65, 3, 64), (1, 130, 2, 64),
                                     (1, 200, 2, 32), (2, 256, 4, 64)])
def test_attention_shapes(dev, B, S, H, D, causal):
    got, ref = _attn_case(dev, B, S, H, D, causal, seed=900 + S)
    assert oracle.normwise_error(got, ref) <= oracle.tolerance(max(S, D))


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("D", [32, 96, 128])
@pytest.mark.parametrize("B,S,H", [(1, 1, 2), (2, 77, 3), (1, 300, 2), (2, 129, 1)])
def test_attention_head_dims(dev, B, S, H, D, causal):
    """The MFMA kernel at head dims other than 64 (32 and 96/128 use 64- and
    32-key blocks), ragged query tiles included."""
    got, ref = _attn_case(dev, B, S, H, D, causal, seed=950 + S + D)
    assert oracle.normwise_error(got, ref) <= oracle.tolerance(max(S, D))


@pytest.mark.parametrize("D", [20, 64, 128, 160])
@pytest.mark.parametrize("causal", [True, False])
def test_attention_misaligned_and_odd_dims(dev, D, causal):
    """Operands 4 bytes past a 16-byte boundary (and D = 20, 160) take the
    row kernel: the output row in registers up to D = 128, in memory above."""
    B, S, H = 2, 70, 3
    q, k, v = (prng.normal(960 + j + D, (B, S, H, D)) for j in range(3))
    n = q.size
    dq, dk, dv, do = (dev.alloc(4 * (n + 1)) for _ in range(4))
    for buf, a in ((dq, q), (dk, k), (dv, v)):
        dev.write(int(buf) + 4, np.ascontiguousarray(a, np.float32))
    dev.fill(int(do) + 4, float("nan"), n)
    case(f"attention misaligned D={D} causal={causal}")
    dev.attention(int(do) + 4, int(dq) + 4, int(dk) + 4, int(dv) + 4, B, S, H, D, causal=causal)
    got = dev.download(int(do) + 4, q.shape)
    assert np.isfinite(got).all()
    ref = oracle.attention(q, k, v, causal=causal)
    assert oracle.normwise_error(got, ref) <= oracle.tolerance(max(S, D))
    for b in (dq, dk, dv, do):
        b.free()


@pytest.mark.parametrize("causal", [True, False])
def test_attention_config_s512(dev, causal):
    """The whole S=512 config (every batch, head and row) against the oracle."""
    got, ref = _attn_case(dev, 8, 512, 16, 64, causal, seed=44)
    err = oracle.normwise_error(got, ref)
    record_parity(f"sdpa B8 H16 D64 S512 causal={causal} (every element)", err, oracle.tolerance(512))
    assert err <= oracle.tolerance(512)


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("B,S,H", [(4, 768, 16), (1, 512, 16), (2, 300, 8), (3, 64, 5)])
def test_attention_small_grids(dev, B, S, H, causal):
    """D = 64 grids of at most three 64-query tiles per CU run the 64-query
    kernel (4-wave workgroups, one LDS buffer, three resident a CU; causal
    long and short tiles paired): every element against the oracle, the
    output NaN-filled first.  B4 H16 S=768 is three tiles per CU on 256 CUs,
    B1 S=512 fewer workgroups than CUs, S=300 a ragged last tile."""
    got, ref = _attn_case(dev, B, S, H, 64, causal, seed=970 + S)
    assert oracle.normwise_error(got, ref) <= oracle.tolerance(S)


def tile_rows(S, tile=128):
    """First, last and one varying row of every tile-row query tile."""
    rows = set()
    for t in range((S + tile - 1) // tile):
        lo, hi = t * tile, min(S, (t + 1) * tile) - 1
        rows.update((lo, hi, min(hi, lo + (29 * t + 11) % tile)))
    return sorted(rows)


@pytest.mark.parametrize("causal", [True, False])
def test_attention_config_s2048_every_tile(dev, causal):
    """S=2048: every element written, and three rows of every 128-query tile
    of every (batch, head) against the oracle, so the causal task order
    (long and short tiles paired, XCD-spread) cannot drop a tile."""
    got, ref = _attn_case(dev, 8, 2048, 16, 64, causal, seed=44, row_list=tile_rows(2048))
    err = oracle.normwise_error(got, ref)
    record_parity(f"sdpa B8 H16 D64 S2048 causal={causal} (three rows of every query tile)", err,
                  oracle.tolerance(2048))
    assert err <= oracle.tolerance(2048)


def test_attention_closed_forms(dev):
    # V constant => output constant; S = 1 => out = v0 (audit_flash_attention semantics)
    B, S, H, D = 1, 96, 2, 64
    q = prng.normal(5, (B, S, H, D))
    k = prng.normal(6, (B, S, H, D))
    v = np.full((B, S, H, D), 0.375, np.float32)
    dq, dk, dv = _upload(dev, q, k, v)
    do = dev.alloc(q.nbytes)
    case("attention closed forms")
    dev.attention(do, dq, dk, dv, B, S, H, D, causal=True)
    assert np.allclose(dev.download(do, q.shape), 0.375, rtol=0, atol=1e-6)
    # q = 0 with causal mask: output row i is the mean of v[0..i]
    v = prng.normal(8, (B, S, H, D))
    dev.write(dq, np.zeros_like(q))
    dev.write(dv, v)
    dev.attention(do, dq, dk, dv, B, S, H, D, causal=True)
    prefix_mean = np.cumsum(v.astype(np.float64), axis=1) / np.arange(1, S + 1)[None, :, None, None]
    assert oracle.normwise_error(dev.download(do, q.shape), prefix_mean) <= 1e-5


def test_attention_grouped(dev):
    G, S, H, D = 4, 192, 4, 64
    qs = [prng.normal(10 + g, (S, H, D)) for g in range(G)]
    ks = [prng.normal(20 + g, (S, H, D)) for g in range(G)]
    vs = [prng.normal(30 + g, (S, H, D)) for g in range(G)]
    dq, dk, dv = _upload(dev, *qs), _upload(dev, *ks), _upload(dev, *vs)
    do = [dev.alloc(qs[0].nbytes) for _ in range(G)]
    case("attention grouped")
    dev.attention_grouped(do, dq, dk, dv, S, H, D, causal=True)
    for g in range(G):
        ref = oracle.attention(qs[g], ks[g], vs[g], causal=True)
        assert oracle.normwise_error(dev.download(do[g], (S, H, D)), ref) <= oracle.tolerance(S)


# ---- conv2d ------------------------------------------------------------------


def _conv_case(dev, N, C_in, H, W, C_out, KH, KW, stride, pad, relu, seed, images=None):
    """The output is NaN-filled before the call and must come back finite."""
    x = prng.normal(seed, (N, C_in, H, W))
    w = prng.normal(seed + 1, (C_out, C_in, KH, KW), std=float(np.sqrt(2.0 / (KH * KW * C_in))))
    dx, dw = _upload(dev, x, w)
    Ho, Wo = (H + 2 * pad - KH) // stride + 1, (W + 2 * pad - KW) // stride + 1
    do = dev.alloc(N * C_out * Ho * Wo * 4)
    dev.fill(do, float("nan"), N * C_out * Ho * Wo)
    case(f"conv N={N} C_in={C_in} {H}x{W} C_out={C_out} k={KH}x{KW} s={stride} p={pad} relu={relu}")
    dev.conv2d(do, dx, dw, None, N, C_in, H, W, C_out, KH, KW, stride, pad, ACT_RELU if relu else ACT_NONE)
    got = dev.download(do, (N, C_out, Ho, Wo))
    assert np.isfinite(got).all(), f"{np.count_nonzero(~np.isfinite(got))} output elements not written"
    ref = oracle.conv2d(x, w, stride, pad, relu, images=images)
    for b in (dx, dw, do):
        b.free()
    sel = slice(*images) if images else slice(None)
    return got[sel], ref[sel]


@pytest.mark.parametrize("N,C_in,H,W,C_out,KH,KW,stride,pad,relu", [
    (1, 1, 5, 5, 1, 3, 3, 1, 1, False),
    (2, 3, 7, 7, 5, 3, 3, 1, 1, True),
    (2, 3, 9, 8, 4, 3, 3, 2, 0, False),
    (1, 4, 6, 6, 8, 1, 1, 1, 0, True),
    (2, 3, 11, 10, 6, 5, 5, 2, 2, True),
    (3, 16, 14, 14, 130, 3, 3, 1, 1, True),
    (1, 8, 32, 32, 64, 3, 3, 1, 1, False),
])
def test_conv_shapes(dev, N, C_in, H, W, C_out, KH, KW, stride, pad, relu):
    got, ref = _conv_case(dev, N, C_in, H, W, C_out, KH, KW, stride, pad, relu, seed=300 + H + C_out)
    assert oracle.normwise_error(got, ref) <= oracle.tolerance(C_in * KH * KW)


def test_conv_config_full(dev):
    """The whole conv config (all 32 images, every channel and pixel)."""
    got, ref = _conv_case(dev, 32, 64, 56, 56, 128, 3, 3, 1, 1, True, seed=45)
    err = oracle.normwise_error(got, ref)
    record_parity("conv 3x3 N32 64->128 56x56 + ReLU (every element)", err, oracle.tolerance(64 * 9))
    assert err <= oracle.tolerance(64 * 9)


@pytest.mark.parametrize("N,C_in,H,W,C_out", [(32, 64, 56, 56, 128), (6, 16, 56, 56, 128), (23, 32, 28, 28, 64)])
def test_conv_stream_k_repeatable(dev, N, C_in, H, W, C_out):
    """Grids a little over a whole number of tiles per CU share their last
    tiles between workgroups (1568, 294 and 282 tiles here); whichever
    workgroup arrives last adds the shares in k order, so repeat calls give
    identical bits, and the result matches the oracle."""
    x = prng.normal(460 + N, (N, C_in, H, W))
    w = prng.normal(461 + N, (C_out, C_in, 3, 3), std=float(np.sqrt(2.0 / (9 * C_in))))
    dx, dw = _upload(dev, x, w)
    do = dev.alloc(N * C_out * H * W * 4)
    dev.fill(do, float("nan"), N * C_out * H * W)
    case(f"conv stream-K N={N} C_in={C_in} {H}x{W} C_out={C_out}")
    outs = []
    for _ in range(3):
        dev.conv2d(do, dx, dw, None, N, C_in, H, W, C_out, 3, 3, 1, 1, ACT_RELU)
        outs.append(dev.download(do, (N, C_out, H, W)))
    assert np.isfinite(outs[0]).all()
    for o in outs[1:]:
        assert np.array_equal(outs[0].view(np.uint32), o.view(np.uint32))
    img = (N - 2, N)
    ref = oracle.conv2d(x, w, 1, 1, True, images=img)
    assert oracle.normwise_error(outs[0][slice(*img)], ref[slice(*img)]) <= oracle.tolerance(9 * C_in)
    for b in (dx, dw, do):
        b.free()


@pytest.mark.parametrize("N,C_in,H,W,C_out,KH,KW,stride,pad,act", [
    (4, 32, 28, 28, 64, 3, 3, 1, 1, ACT_RELU),   # direct kernel
    (2, 16, 15, 13, 36, 5, 5, 2, 2, ACT_NONE),   # 5x5, stride 2, runtime filter size
    (32, 64, 56, 56, 128, 3, 3, 1, 1, ACT_RELU),  # the config (stream-K grid)
])
def test_conv_packed_weight_bit_identical(dev, N, C_in, H, W, C_out, KH, KW, stride, pad, act):
    """lancius_hip_conv2d_pack_weight once + lancius_hip_conv2d_packed_f32
    gives the bits of lancius_hip_conv2d_f32 (which re-lays w every call)."""
    Ho, Wo = (H + 2 * pad - KH) // stride + 1, (W + 2 * pad - KW) // stride + 1
    x = prng.normal(470 + C_in, (N, C_in, H, W))
    w = prng.normal(471 + C_in, (C_out, C_in, KH, KW), std=float(np.sqrt(2.0 / (KH * KW * C_in))))
    b = prng.normal(472 + C_in, (C_out,))
    dx, dw, db = _upload(dev, x, w, b)
    packed = dev.alloc(dev.conv2d_packed_bytes(C_out, C_in, KH, KW))
    o1, o2 = dev.alloc(N * C_out * Ho * Wo * 4), dev.alloc(N * C_out * Ho * Wo * 4)
    case(f"conv packed N={N} C_in={C_in} {H}x{W} C_out={C_out} k={KH}x{KW} s={stride}")
    dev.conv2d(o1, dx, dw, db, N, C_in, H, W, C_out, KH, KW, stride, pad, act)
    dev.conv2d_pack_weight(packed, dw, C_out, C_in, KH, KW)
    dev.conv2d_packed(o2, dx, packed, db, N, C_in, H, W, C_out, KH, KW, stride, pad, act)
    a, c = dev.download(o1, (N, C_out, Ho, Wo)), dev.download(o2, (N, C_out, Ho, Wo))
    assert np.isfinite(a).all()
    assert np.array_equal(a.view(np.uint32), c.view(np.uint32))
    for buf in (dx, dw, db, packed, o1, o2):
        buf.free()


def test_conv_packed_weight_shape_limits(dev):
    case("conv packed limits")
    for C_out, C_in in ((4, 3), (6, 16)):  # C_in % 16 != 0, C_out % 4 != 0
        with pytest.raises(HipError) as e:
            dev.conv2d_pack_weight(1, 1, C_out, C_in, 3, 3)
        assert e.value.code == -3
        with pytest.raises(HipError) as e:
            dev.conv2d_packed(1, 1, 1, None, 1, C_in, 8, 8, C_out, 3, 3, 1, 1)
        assert e.value.code == -3


def test_conv_bias(dev):
    N, C_in, H, W, C_out = 2, 4, 9, 9, 6
    x = prng.normal(71, (N, C_in, H, W))
    w = prng.normal(72, (C_out, C_in, 3, 3))
    b = prng.normal(73, (C_out,))
    dx, dw, db = _upload(dev, x, w, b)
    do = dev.alloc(N * C_out * H * W * 4)
    case("conv bias")
    dev.conv2d(do, dx, dw, db, N, C_in, H, W, C_out, 3, 3, 1, 1, ACT_RELU)
    ref = oracle.relu(oracle.conv2d(x, w, 1, 1, False) + b.astype(np.float64)[None, :, None, None])
    assert oracle.normwise_error(dev.download(do, (N, C_out, H, W)), ref) <= oracle.tolerance(36)


# ---- row and elementwise ops -----------------------------------------------------


@pytest.mark.parametrize("rows,hidden", [(4096, 1024), (7, 100), (3, 256), (5, 4096), (2, 1), (9, 1500), (3, 4100)])
def test_layernorm(dev, rows, hidden):
    x = prng.normal(11, (rows, hidden), mean=0.5, std=2.0)
    g = prng.normal(12, (hidden,), mean=1.0, std=0.1)
    b = prng.normal(13, (hidden,), std=0.1)
    dx, dg, db = _upload(dev, x, g, b)
    do = dev.alloc(x.nbytes)
    case(f"layernorm {rows}x{hidden}")
    dev.layernorm(do, dx, dg, db, rows, hidden)
    ref = oracle.layernorm(x, g, b)
    assert oracle.normwise_error(dev.download(do, x.shape), ref) <= oracle.tolerance(hidden)


@pytest.mark.parametrize("rows,hidden", [(1024, 1024), (9, 1500), (5, 1001)])
def test_layernorm_grouped(dev, rows, hidden):
    """Three LayerNorms of one shape in one launch (the executor's launch
    for one wave's LAYERNORM nodes), each with its own gamma and beta; equal
    bit for bit to the single call, member by member (1001 columns: the
    three-pass kernel once per member)."""
    xs = [prng.normal(30 + j, (rows, hidden), mean=0.5, std=2.0) for j in range(3)]
    gs = [prng.normal(40 + j, (hidden,), mean=1.0, std=0.1) for j in range(3)]
    bs = [prng.normal(50 + j, (hidden,), std=0.1) for j in range(3)]
    dx, dg, db = [dev.upload(a) for a in xs], [dev.upload(a) for a in gs], [dev.upload(a) for a in bs]
    dos, d1 = [dev.alloc(4 * rows * hidden) for _ in range(3)], dev.alloc(4 * rows * hidden)
    case(f"layernorm grouped x3 {rows}x{hidden}")
    dev.layernorm_grouped(dos, dx, dg, db, rows, hidden)
    for j in range(3):
        got = dev.download(dos[j], (rows, hidden))
        assert oracle.normwise_error(got, oracle.layernorm(xs[j], gs[j], bs[j])) <= oracle.tolerance(hidden)
        dev.layernorm(d1, dx[j], dg[j], db[j], rows, hidden)
        assert np.array_equal(got.view(np.uint32), dev.download(d1, (rows, hidden)).view(np.uint32))
    for b in dx + dg + db + dos + [d1]:
        b.free()


def test_layernorm_constant_row_gives_beta(dev):
    x = np.full((4, 1024), 3.25, np.float32)
    g = prng.normal(1, (1024,))
    b = prng.normal(2, (1024,))
    dx, dg, db = _upload(dev, x, g, b)
    do = dev.alloc(x.nbytes)
    case("layernorm constant row")
    dev.layernorm(do, dx, dg, db, 4, 1024)
    assert np.allclose(dev.download(do, x.shape), np.broadcast_to(b, x.shape), atol=1e-6, rtol=0)


@pytest.mark.parametrize("rows,cols", [(64, 10), (5, 1), (3, 200), (1000, 37), (8, 1024), (4, 4096), (6, 2000),
                                       (2, 4104)])
def test_softmax_argmax(dev, rows, cols):
    x = prng.normal(21, (rows, cols), std=3.0)
    dx = dev.upload(x)
    dp = dev.alloc(x.nbytes)
    di = dev.alloc(rows * 4)
    case(f"softmax {rows}x{cols}")
    dev.softmax(dp, di, dx, rows, cols)
    probs = dev.download(dp, x.shape)
    idx = dev.download(di, (rows,), np.int32)
    ref = oracle.softmax(x)
    assert oracle.normwise_error(probs, ref) <= oracle.tolerance(cols)
    ref_idx = oracle.argmax(ref)
    assert np.array_equal(idx, ref_idx)


def test_softmax_ties_first_max(dev):
    x = np.zeros((4, 10), np.float32)
    x[1, 3] = x[1, 7] = 2.0
    x[2, 9] = 1.0
    dx = dev.upload(x)
    dp = dev.alloc(x.nbytes)
    di = dev.alloc(16)
    case("softmax ties")
    dev.softmax(dp, di, dx, 4, 10)
    assert dev.download(di, (4,), np.int32).tolist() == [0, 3, 9, 0]
    assert np.allclose(dev.download(dp, x.shape)[0], 0.1, atol=1e-7)


def test_softmax_ties_first_max_register_rows(dev):
    """Ties inside one float4 piece, across pieces of one lane and across
    lanes (lane 0's piece 1 holds column 257, lane 1's piece 0 column 4)."""
    x = np.zeros((4, 1024), np.float32)
    x[1, 700] = x[1, 300] = 2.0
    x[2, 5] = x[2, 6] = 1.5
    x[3, 257] = x[3, 4] = 3.0
    dx = dev.upload(x)
    dp = dev.alloc(x.nbytes)
    di = dev.alloc(16)
    case("softmax ties 4x1024")
    dev.softmax(dp, di, dx, 4, 1024)
    assert dev.download(di, (4,), np.int32).tolist() == [0, 300, 5, 4]


def test_elementwise(dev):
    n = 1_000_003
    a = prng.normal(31, (n,), std=60.0)
    a[:6] = [np.nan, np.inf, -np.inf, 150.0, -150.0, 0.0]
    b = prng.normal(32, (n,))
    da, db = _upload(dev, a, b)
    do = dev.alloc(a.nbytes)
    case("elementwise add/relu/gelu/copy")
    dev.add(do, da, db, n)
    assert oracle.normwise_error(dev.download(do, (n,))[6:], oracle.add(a, b)[6:]) <= TOL_ELEMENTWISE
    dev.relu(do, da, n)
    got = dev.download(do, (n,))
    assert got[0] == 0.0 and np.isposinf(got[1]) and got[2] == 0.0
    assert np.array_equal(got[3:], oracle.relu(a)[3:].astype(np.float32))
    dev.gelu(do, da, n)
    got = dev.download(do, (n,))
    ref = oracle.gelu(a)
    assert np.isnan(got[0]) and got[1] == 100.0 and got[2] == 0.0 and got[3] == 100.0 and got[4] == 0.0
    assert got[5] == 0.0
    assert oracle.normwise_error(got[1:], ref[1:]) <= TOL_ELEMENTWISE
    dev.copy(do, db, n)
    assert np.array_equal(dev.download(do, (n,)), b)


def test_broadcast_fill(dev):
    row = prng.normal(41, (37,))
    dr = dev.upload(row)
    do = dev.alloc(50 * 37 * 4)
    case("broadcast/fill")
    dev.broadcast(do, dr, 50, 37, 37)
    assert np.array_equal(dev.download(do, (50, 37)), np.broadcast_to(row, (50, 37)))
    dev.broadcast(do, dr, 50, 37, 1)
    assert np.all(dev.download(do, (50, 37)) == row[0])
    dev.fill(do, 2.5, 50 * 37)
    assert np.all(dev.download(do, (50, 37)) == 2.5)
