// fp32 GEMM on the gfx950 matrix cores: C[M,N] = epilogue(A[M,K] . B[K,N]),
// row-major, no transposes - the layout of the graph MATMUL node
// (bleeding/v11A1/src/runtime/lancius_scheduler.c:222-234, which reads
// M = a.shape[0], K = a.shape[1], N = b.shape[1]).
//
// Design:
//  * 256 threads = 4 wave64s arranged WGM x WGN; each wave owns a
//    (BM/WGM) x (BN/WGN) block of C held in v_mfma_f32_32x32x2_f32
//    accumulators (16 fp32 per lane per 32x32 sub-tile).
//  * A and B tiles are staged in LDS in k-major order (A is transposed on the
//    way in), so the MFMA operand of lane l - element (row l%32, k l/32) - is
//    one conflict-free 32-float row segment.  Two LDS buffers: the global loads
//    of tile k+1 are issued before the MFMAs of tile k and written to the other
//    buffer after them, one barrier per k-tile.
//  * The epilogue adds bias[n], applies ReLU/GELU and adds a residual before
//    the single store of C (the BROADCAST + ADD + activation nodes of a graph).
//  * Workgroup ids are renumbered XCD-contiguously and rastered in groups of
//    tile-rows so that each XCD's L2 sees a compact set of A/B panels.
#include <algorithm>
#include <mutex>

#include "common.hpp"
#include "kernels.hpp"

namespace lancius {
namespace {

struct GemmParams {
    float* C[LANCIUS_HIP_MAX_GROUP];
    const float* A[LANCIUS_HIP_MAX_GROUP];
    const float* R[LANCIUS_HIP_MAX_GROUP];     // residuals (may be null)
    const float* B[LANCIUS_HIP_MAX_GROUP];
    const float* bias[LANCIUS_HIP_MAX_GROUP];  // may be null
    int M, N, K;
    int act;
    uint32_t tiles_m, tiles_n;
    float* ws;   // split-K partials [count][splits][M][N]
    unsigned* counters;  // fused skinny split-K: one arrival counter per (group, column block), zero between launches
    int splits;  // K ranges (blockIdx.y), 1 = no split
    int kchunk;  // K per split, a multiple of the k-tile
};

constexpr int kThreads = 256;

// SPLIT: the workgroup reduces K range [y*kchunk, (y+1)*kchunk) and stores its
// raw partial sums; splitk_reduce adds the partials in order y = 0, 1, ...
// (a fixed order, so results are run-to-run identical) and applies the
// epilogue.
// TA: A is given transposed, stored [K][M] (element (m,k) at A[k*M + m]);
// TB: B is given transposed, stored [N][K] (element (k,n) at B[n*K + k]).
// The LDS tiles are the same k-major tiles either way; only the global-load
// pattern changes (a transposed operand is read along its contiguous axis).
// KG > 1: the workgroup has KG groups of 4 waves over the same C tile; group
// g takes k-pairs g, g + KG, g + 2 KG, ... of every k-tile, and at the end
// groups 1 .. KG-1 pass their accumulators through LDS to group 0, which adds
// them in group order (fixed, so run-to-run identical) and runs the epilogue.
// It puts 8 or 16 waves on a CU when the grid has only one workgroup per CU.
template <int BM, int BN, int BK, int WGM, int WGN, bool VEC, bool SPLIT, int OCC = 1, bool TA = false,
          bool TB = false, int KG = 1>
__global__ void __launch_bounds__(kThreads * KG, OCC) gemm_f32_mfma(const GemmParams p) {
    static_assert(WGM * WGN == 4, "4 waves per k-group");
    constexpr int NT = kThreads * KG;
    constexpr int WM = BM / WGM, WN = BN / WGN;
    constexpr int TM = WM / 32, TN = WN / 32;
    static_assert(TM >= 1 && TN >= 1 && WM % 32 == 0 && WN % 32 == 0, "wave tile is a multiple of 32");
    static_assert(BK % 4 == 0, "BK multiple of 4");
    constexpr int KPG = BK / 2 / KG;  // k-pairs per group per k-tile
    static_assert(KPG >= 1 && KPG * KG * 2 == BK, "k-pairs split evenly over the groups");
    // AMK: A[M][K] loaded along k is kept m-major in LDS (Am[m][k], a
    // 16-byte store per float4); k-group g takes k in [g*BK/KG, (g+1)*BK/KG)
    // and lane half h of its MFMAs the h-th half of that range: a lane's A
    // operands for a whole k-tile are BK/(8 KG) 16-byte reads instead of
    // BK/(2 KG) 4-byte reads, and the k-major transpose on the store (four
    // 4-byte writes per float4) goes away.  Any pairing of k between A and B
    // is valid as long as both use the same one.  The pitch BK+4 keeps 16
    // consecutive rows on distinct 16-byte bank groups.
    constexpr bool AMK = VEC && !TA && (BK / KG) % 8 == 0;
    constexpr int LDA = BM + 4;  // As[k][m]
    constexpr int LDB = BN + 4;  // Bs[k][n]
    constexpr int LDK = BK + 4;  // Am[m][k]
    constexpr int A_STAGE = AMK ? BM * LDK : BK * LDA;
    constexpr int STAGE = 2 * (A_STAGE + BK * LDB);
    constexpr int RED = KG > 1 ? 4 * TM * TN * 16 * 64 : 0;  // one group's accumulators
    __shared__ __attribute__((aligned(16))) float smem[STAGE > RED ? STAGE : RED];
    float(*As)[BK][LDA] = reinterpret_cast<float(*)[BK][LDA]>(smem);
    float(*Am)[BM][LDK] = reinterpret_cast<float(*)[BM][LDK]>(smem);
    float(*Bs)[BK][LDB] = reinterpret_cast<float(*)[BK][LDB]>(smem + 2 * A_STAGE);

    const int g = blockIdx.z;
    const float* __restrict__ A = p.A[g];
    const float* __restrict__ B = p.B[g];
    float* __restrict__ C = p.C[g];
    const float* __restrict__ R = p.R[g];
    const int M = p.M, N = p.N, K = p.K;

    const uint32_t ntiles = p.tiles_m * p.tiles_n;
    uint32_t tm_id, tn_id;
    grouped_tile(xcd_contiguous_id(blockIdx.x, ntiles), p.tiles_m, p.tiles_n, 4, tm_id, tn_id);
    const int m0 = (int)tm_id * BM;
    const int n0 = (int)tn_id * BN;

    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const int kg = KG > 1 ? wave >> 2 : 0, wl = wave & 3;
    const int wm = wl / WGN, wn = wl % WGN;
    const int lr = lane & 31, lk = lane >> 5;

    // ---- global -> register staging -------------------------------------
    constexpr int A_VEC = VEC ? (BM * BK / 4) / NT : 0;
    constexpr int B_VEC = VEC ? (BK * BN / 4) / NT : 0;
    constexpr int A_SCL = VEC ? 0 : (BM * BK) / NT;
    constexpr int B_SCL = VEC ? 0 : (BK * BN) / NT;
    static_assert(!VEC || (A_VEC * NT * 4 == BM * BK && B_VEC * NT * 4 == BK * BN), "even split");
    static_assert(VEC || (A_SCL * NT == BM * BK && B_SCL * NT == BK * BN), "even split");
    f32x4 a_v[A_VEC > 0 ? A_VEC : 1];
    f32x4 b_v[B_VEC > 0 ? B_VEC : 1];
    float a_s[A_SCL > 0 ? A_SCL : 1];
    float b_s[B_SCL > 0 ? B_SCL : 1];

    // A tile (rows m0.., k0..): along k from A[M][K], along m from A^T[K][M].
    // B tile (k0.., cols n0..): along n from B[K][N], along k from B^T[N][K].
    // Branch-free: every load reads a clamped, in-bounds address, so one
    // k-tile is one basic block and a load past the last k-tile is harmless.
    // Rows of A past M and columns of B past N then hold copies of the last
    // row / column; they only reach rows and columns of C that are never
    // stored.  Elements past K must be zero: store_tile clears them in the
    // one k-tile that crosses K (a uniform branch), so no select waits on a
    // load in the other tiles.
    // AMK: float4 idx of the A tile -> (row, k chunk).  A wave's 64 float4
    // cover 64/KQ rows x all KQ chunks, as with row-major order, but lanes
    // of one chunk take consecutive rows, so a 16-lane group stores 16 rows
    // of one chunk: the same distinct 16-byte bank slots as the operand
    // reads (row-major order put 4 lanes on one 64-byte row segment and
    // conflicted 2-way at the BK+4 pitch).
    constexpr int KQ = BK / 4, RPW = 64 / KQ;
    static_assert(!AMK || (64 % KQ == 0 && (BM * KQ) % 64 == 0), "whole waves of A rows");
    auto a_rk = [&](int idx, int& r, int& kq) {
        if constexpr (AMK) {
            r = (idx / 64) * RPW + (idx % 64) % RPW;
            kq = (idx % 64) / RPW;
        } else {
            r = idx / KQ;
            kq = idx % KQ;
        }
    };
    auto load_tile = [&](int k0) {
        if constexpr (VEC) {
#pragma unroll
            for (int i = 0; i < A_VEC; ++i) {
                const int idx = tid + i * NT;
                if constexpr (!TA) {
                    int r, kq;
                    a_rk(idx, r, kq);
                    const int gm = m0 + r, gk = k0 + 4 * kq;
                    a_v[i] = *(const f32x4*)(A + (size_t)min(gm, M - 1) * K + min(gk, K - 4));
                } else {
                    const int kr = idx / (BM / 4), mq = idx % (BM / 4);
                    const int gk = k0 + kr, gm = m0 + 4 * mq;
                    a_v[i] = *(const f32x4*)(A + (size_t)min(gk, K - 1) * M + min(gm, M - 4));
                }
            }
#pragma unroll
            for (int i = 0; i < B_VEC; ++i) {
                const int idx = tid + i * NT;
                if constexpr (!TB) {
                    const int kr = idx / (BN / 4), nq = idx % (BN / 4);
                    const int gk = k0 + kr, gn = n0 + 4 * nq;
                    b_v[i] = *(const f32x4*)(B + (size_t)min(gk, K - 1) * N + min(gn, N - 4));
                } else {
                    const int c = idx / (BK / 4), kq = idx % (BK / 4);
                    const int gn = n0 + c, gk = k0 + 4 * kq;
                    b_v[i] = *(const f32x4*)(B + (size_t)min(gn, N - 1) * K + min(gk, K - 4));
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < A_SCL; ++i) {
                const int idx = tid + i * NT;
                if constexpr (!TA) {
                    const int r = idx / BK, kk = idx % BK;
                    const int gm = m0 + r, gk = k0 + kk;
                    a_s[i] = A[(size_t)min(gm, M - 1) * K + min(gk, K - 1)];
                } else {
                    const int kr = idx / BM, r = idx % BM;
                    const int gk = k0 + kr, gm = m0 + r;
                    a_s[i] = A[(size_t)min(gk, K - 1) * M + min(gm, M - 1)];
                }
            }
#pragma unroll
            for (int i = 0; i < B_SCL; ++i) {
                const int idx = tid + i * NT;
                if constexpr (!TB) {
                    const int kr = idx / BN, n = idx % BN;
                    const int gk = k0 + kr, gn = n0 + n;
                    b_s[i] = B[(size_t)min(gk, K - 1) * N + min(gn, N - 1)];
                } else {
                    const int c = idx / BK, kk = idx % BK;
                    const int gn = n0 + c, gk = k0 + kk;
                    b_s[i] = B[(size_t)min(gn, N - 1) * K + min(gk, K - 1)];
                }
            }
        }
    };

    auto clear_past_k = [&](int k0) {
        const f32x4 z4 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < A_VEC; ++i) {
            const int idx = tid + i * NT;
            int r, kq;
            a_rk(idx, r, kq);
            const int gk = !TA ? k0 + 4 * kq : k0 + idx / (BM / 4);
            if (gk >= K) a_v[i] = z4;
        }
#pragma unroll
        for (int i = 0; i < B_VEC; ++i) {
            const int idx = tid + i * NT;
            const int gk = !TB ? k0 + idx / (BN / 4) : k0 + 4 * (idx % (BK / 4));
            if (gk >= K) b_v[i] = z4;
        }
#pragma unroll
        for (int i = 0; i < A_SCL; ++i) {
            const int idx = tid + i * NT;
            const int gk = !TA ? k0 + idx % BK : k0 + idx / BM;
            if (gk >= K) a_s[i] = 0.0f;
        }
#pragma unroll
        for (int i = 0; i < B_SCL; ++i) {
            const int idx = tid + i * NT;
            const int gk = !TB ? k0 + idx / BN : k0 + idx % BK;
            if (gk >= K) b_s[i] = 0.0f;
        }
    };

    auto store_tile = [&](int buf, int k0) {
        if (k0 + BK > K) clear_past_k(k0);
        if constexpr (VEC) {
#pragma unroll
            for (int i = 0; i < A_VEC; ++i) {
                const int idx = tid + i * NT;
                if constexpr (AMK) {
                    int r, kq;
                    a_rk(idx, r, kq);
                    *(f32x4*)&Am[buf][r][4 * kq] = a_v[i];
                } else if constexpr (!TA) {
                    int r, kq;
                    a_rk(idx, r, kq);
                    As[buf][4 * kq + 0][r] = a_v[i].x;
                    As[buf][4 * kq + 1][r] = a_v[i].y;
                    As[buf][4 * kq + 2][r] = a_v[i].z;
                    As[buf][4 * kq + 3][r] = a_v[i].w;
                } else {
                    const int kr = idx / (BM / 4), mq = idx % (BM / 4);
                    *(f32x4*)&As[buf][kr][4 * mq] = a_v[i];
                }
            }
#pragma unroll
            for (int i = 0; i < B_VEC; ++i) {
                const int idx = tid + i * NT;
                if constexpr (!TB) {
                    const int kr = idx / (BN / 4), nq = idx % (BN / 4);
                    *(f32x4*)&Bs[buf][kr][4 * nq] = b_v[i];
                } else {
                    const int c = idx / (BK / 4), kq = idx % (BK / 4);
                    Bs[buf][4 * kq + 0][c] = b_v[i].x;
                    Bs[buf][4 * kq + 1][c] = b_v[i].y;
                    Bs[buf][4 * kq + 2][c] = b_v[i].z;
                    Bs[buf][4 * kq + 3][c] = b_v[i].w;
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < A_SCL; ++i) {
                const int idx = tid + i * NT;
                if constexpr (!TA)
                    As[buf][idx % BK][idx / BK] = a_s[i];
                else
                    As[buf][idx / BM][idx % BM] = a_s[i];
            }
#pragma unroll
            for (int i = 0; i < B_SCL; ++i) {
                const int idx = tid + i * NT;
                if constexpr (!TB)
                    Bs[buf][idx / BN][idx % BN] = b_s[i];
                else
                    Bs[buf][idx % BK][idx / BK] = b_s[i];
            }
        }
    };

    f32x16 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    int kt0 = 0, kt1 = (K + BK - 1) / BK;
    if constexpr (SPLIT) {
        kt0 = (int)blockIdx.y * (p.kchunk / BK);
        kt1 = min(kt1, kt0 + p.kchunk / BK);
    }
    load_tile(kt0 * BK);
    store_tile(0, kt0 * BK);
    __syncthreads();

    for (int kt = kt0; kt < kt1; ++kt) {
        const int cur = (kt - kt0) & 1;
        load_tile((kt + 1) * BK);  // past the end on the last tile: clamped, unused
        // keep the global loads first: they have the whole k-tile to land
        __builtin_amdgcn_sched_barrier(0);
        // Fragments of k-pair kp+1 are read from LDS before the MFMAs of kp in
        // program order (the compiler may sink the reads after them; the
        // other waves on the SIMD cover that latency - pinning the order
        // measured no faster).
        if constexpr (AMK) {
            // group kg, lane half lk: k = kb + kp, kp = 0 .. KH-1
            constexpr int KH = BK / KG / 2;
            const int kb = kg * (BK / KG) + lk * KH;
            f32x4 av[TM][KH / 4];
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int h = 0; h < KH / 4; ++h) av[i][h] = *(const f32x4*)&Am[cur][wm * WM + i * 32 + lr][kb + 4 * h];
            float bf[2][TN];
#pragma unroll
            for (int j = 0; j < TN; ++j) bf[0][j] = Bs[cur][kb][wn * WN + j * 32 + lr];
#pragma unroll
            for (int kp = 0; kp < KH; ++kp) {
                const int c = kp & 1;
                if (kp + 1 < KH) {
#pragma unroll
                    for (int j = 0; j < TN; ++j) bf[c ^ 1][j] = Bs[cur][kb + kp + 1][wn * WN + j * 32 + lr];
                }
#pragma unroll
                for (int i = 0; i < TM; ++i)
#pragma unroll
                    for (int j = 0; j < TN; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[i][kp / 4][kp % 4], bf[c][j], acc[i][j],
                                                                         0, 0, 0);
                // The next tile's LDS store (see the k-major path below for
                // why mid-tile): a quarter in with one k-group (4096^3:
                // 133.5 -> 134.7 TFLOP/s against halfway; three quarters in
                // measured 132.4); with k-groups after the first k-pair of
                // four (2048^3: 115.3 -> 117.7) and halfway through eight (a
                // quarter in cost 1024^3 6%).
                if (kp == (KG == 1 && KH >= 8 ? KH / 4 - 1 : KH == 4 ? 0 : KH > 1 ? KH / 2 - 1 : 0)) {
                    __builtin_amdgcn_sched_barrier(0);
                    store_tile(cur ^ 1, (kt + 1) * BK);
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
            __syncthreads();
            continue;
        }
        // group kg: k rows 2 (kg + KG j) + lk, j = 0 .. KPG-1
        float af[2][TM], bf[2][TN];
        const int kf = 2 * kg + lk;
#pragma unroll
        for (int i = 0; i < TM; ++i) af[0][i] = As[cur][kf][wm * WM + i * 32 + lr];
#pragma unroll
        for (int j = 0; j < TN; ++j) bf[0][j] = Bs[cur][kf][wn * WN + j * 32 + lr];
#pragma unroll
        for (int kp = 0; kp < KPG; ++kp) {
            const int c = kp & 1;
            if (kp + 1 < KPG) {
                const int kr = kf + 2 * KG * (kp + 1);
#pragma unroll
                for (int i = 0; i < TM; ++i) af[c ^ 1][i] = As[cur][kr][wm * WM + i * 32 + lr];
#pragma unroll
                for (int j = 0; j < TN; ++j) bf[c ^ 1][j] = Bs[cur][kr][wn * WN + j * 32 + lr];
            }
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[c][i], bf[c][j], acc[i][j], 0, 0, 0);
            // The next tile goes to the other buffer (last read before the
            // previous barrier) halfway through this one: its loads have had
            // half a tile of MFMAs to land, and the LDS writes spread over
            // the tile instead of bunching before the barrier (4096^3 at the
            // settled clock: 125 -> 130 TFLOP/s).
            if (kp == (KPG > 1 ? KPG / 2 - 1 : 0)) {
                __builtin_amdgcn_sched_barrier(0);
                store_tile(cur ^ 1, (kt + 1) * BK);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        __syncthreads();
    }

    if constexpr (KG > 1) {
        // groups 1 .. KG-1 hand their sums to group 0 one at a time (the
        // staging buffers are free after the last barrier of the k loop)
        for (int s = 1; s < KG; ++s) {
            if (kg == s) {
#pragma unroll
                for (int i = 0; i < TM; ++i)
#pragma unroll
                    for (int j = 0; j < TN; ++j)
#pragma unroll
                        for (int r = 0; r < 16; ++r) smem[(((wl * TM + i) * TN + j) * 16 + r) * 64 + lane] = acc[i][j][r];
            }
            __syncthreads();
            if (kg == 0) {
#pragma unroll
                for (int i = 0; i < TM; ++i)
#pragma unroll
                    for (int j = 0; j < TN; ++j)
#pragma unroll
                        for (int r = 0; r < 16; ++r) acc[i][j][r] += smem[(((wl * TM + i) * TN + j) * 16 + r) * 64 + lane];
            }
            if (s + 1 < KG) __syncthreads();
        }
        if (kg != 0) return;
    }

    // ---- epilogue: bias, activation, residual, one store -----------------
    // Accumulator layout of v_mfma_f32_32x32x2_f32: register r of lane l holds
    // row 8*(r/4) + 4*(l/32) + r%4, column l%32 of the 32x32 sub-tile.
    if constexpr (SPLIT) {
        float* __restrict__ part = p.ws + ((size_t)g * p.splits + blockIdx.y) * (size_t)M * N;
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const int col = n0 + wn * WN + j * 32 + lr;
            if (col >= N) continue;
#pragma unroll
            for (int i = 0; i < TM; ++i) {
                const int rbase = m0 + wm * WM + i * 32 + 4 * lk;
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int row = rbase + 8 * (r >> 2) + (r & 3);
                    if (row < M) part[(size_t)row * N + col] = acc[i][j][r];
                }
            }
        }
        return;
    }
    // (the activation chosen once per launch, as in gemm_f32_direct)
    const float* __restrict__ bias = p.bias[g];
    with_act(p.act, [&](auto act_c) {
        constexpr int ACT = decltype(act_c)::value;
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const int col = n0 + wn * WN + j * 32 + lr;
            if (col >= N) continue;
            const float bv = bias ? bias[col] : 0.0f;
#pragma unroll
            for (int i = 0; i < TM; ++i) {
                const int rbase = m0 + wm * WM + i * 32 + 4 * lk;
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int row = rbase + 8 * (r >> 2) + (r & 3);
                    if (row < M) {
                        const size_t o = (size_t)row * N + col;
                        const float v = act_fixed<ACT>(acc[i][j][r] + bv);
                        C[o] = R ? v + R[o] : v;
                    }
                }
            }
        }
    });
}

// 128x128 tiles, k-tiles of 16, 4 waves of 64x64, with both operand tiles
// loaded straight from global memory into LDS (16-byte buffer loads with the
// LDS as destination, gfx950): no register staging and no LDS store
// instructions, and the next k-tile's loads have a whole k-tile of MFMAs to
// land before the barrier that precedes their first read.  The two LDS
// buffers are separate arrays and the loop is unrolled by two, so every
// access names its buffer statically.
//  * A (rows m0.., float4 chunks c of 4 k) lives m-major, 64 bytes per row;
//    chunk c of row r sits at chunk c ^ ((r >> 2) & 3), so the 16-byte
//    operand reads of 16 consecutive rows hit 16 different bank groups.
//  * B (rows k, columns n0..) lives k-major, 512 bytes per row; chunk c of
//    row k sits at chunk c ^ (8 * ((k >> 3) & 1)): the two lane halves, which
//    read rows 8 apart, land on disjoint banks.
//  * Elements past K are zero because their loads use an offset past the
//    buffer's end (which returns 0); rows past M and columns past N read the
//    last row / column and only reach entries of C that are never stored.
// Requires A, B non-transposed and float4-aligned (K, N multiples of 4) and
// both operands under 2 GiB.  A and B use the same k pairing as the AMK
// path: lane half h of the MFMAs takes k in [8h, 8h + 8).
template <int OCC>
__global__ void __launch_bounds__(256, OCC) gemm_f32_direct(const GemmParams p) {
    constexpr int BM = 128, BN = 128, BK = 16;
    constexpr int WM = 64, WN = 64, TM = 2, TN = 2;
    typedef __attribute__((address_space(3))) void lds_void;
    __shared__ __attribute__((aligned(16))) float As0[BM * BK];
    __shared__ __attribute__((aligned(16))) float As1[BM * BK];
    __shared__ __attribute__((aligned(16))) float Bs0[BK * BN];
    __shared__ __attribute__((aligned(16))) float Bs1[BK * BN];

    const int g = blockIdx.z;
    const float* __restrict__ A = p.A[g];
    const float* __restrict__ B = p.B[g];
    float* __restrict__ C = p.C[g];
    const float* __restrict__ R = p.R[g];
    const int M = p.M, N = p.N, K = p.K;
    const uint32_t ntiles = p.tiles_m * p.tiles_n;
    uint32_t tm_id, tn_id;
    grouped_tile(xcd_contiguous_id(blockIdx.x, ntiles), p.tiles_m, p.tiles_n, 4, tm_id, tn_id);
    const int m0 = (int)tm_id * BM;
    const int n0 = (int)tn_id * BN;

    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int wm = wave >> 1, wn = wave & 1;
    const int lr = lane & 31, lk = lane >> 5;

    const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(A), 0, (int)((size_t)M * K * sizeof(float)), kBufferRsrcWord3);
    const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(B), 0, (int)((size_t)K * N * sizeof(float)), kBufferRsrcWord3);
    constexpr int kOut = 0x7ffffff0;  // an offset past the end of any operand: the load returns 0

    // This lane's two chunks of each tile (instruction i of wave w fills LDS
    // chunks (2w + i) * 64 + lane).  Byte offsets at k0 = 0; per k-tile A
    // moves 64 bytes and B 16 rows.
    int a_row[2], a_k[2], b_kr[2];
    int a_off0[2], b_off0[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int q = (2 * wave + i) * 64 + lane;
        const int row = q >> 2, c = (q & 3) ^ ((row >> 2) & 3);
        a_row[i] = row;
        a_k[i] = 4 * c;
        a_off0[i] = (min(m0 + row, M - 1) * K + 4 * c) * (int)sizeof(float);
        const int kr = q >> 5, lc = (q & 31) ^ (((kr >> 3) & 1) << 3);
        b_kr[i] = kr;
        b_off0[i] = (kr * N + min(n0 + 4 * lc, N - 4)) * (int)sizeof(float);
    }
    auto load_tile = [&](float* As, float* Bs, int kt) {
        const int k0 = kt * BK;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int ao = k0 + a_k[i] < K ? a_off0[i] + k0 * (int)sizeof(float) : kOut;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_void*)(As + (2 * wave + i) * 256), 16, ao, 0, 0, 0);
            const int bo = k0 + b_kr[i] < K ? b_off0[i] + k0 * N * (int)sizeof(float) : kOut;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, (lds_void*)(Bs + (2 * wave + i) * 256), 16, bo, 0, 0, 0);
        }
        // (compute places them between its first MFMAs)
    };

    f32x16 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    // operand addresses (floats) of this lane, fixed over the k loop
    int a_rd[TM][2];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int row = wm * WM + i * 32 + lr, c = 2 * lk + h;
            a_rd[i][h] = row * BK + 4 * (c ^ ((row >> 2) & 3));
        }
    int b_rd[TN];
#pragma unroll
    for (int j = 0; j < TN; ++j) {
        const int n = wn * WN + j * 32 + lr;
        b_rd[j] = 8 * lk * BN + 4 * ((n >> 2) ^ (lk << 3)) + (n & 3);
    }
    auto compute = [&](const float* As, const float* Bs) {
        f32x4 av[TM][2];
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int h = 0; h < 2; ++h) av[i][h] = *(const f32x4*)(As + a_rd[i][h]);
#pragma unroll
        for (int kp = 0; kp < 8; ++kp) {
            float bf[TN];
#pragma unroll
            for (int j = 0; j < TN; ++j) bf[j] = Bs[b_rd[j] + kp * BN];
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[i][kp / 4][kp % 4], bf[j], acc[i][j], 0, 0, 0);
        }
        // the k-tile's four loads one after each of the first four MFMAs
        // (the scheduler would otherwise sink them to the wait before the
        // barrier)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
            __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // global load
        }
        __builtin_amdgcn_sched_group_barrier(0x008, TM * TN * 8 - 4, 0);
        __builtin_amdgcn_sched_barrier(0);
    };

    // k-tiles in pairs; when their count is odd the last pair's second tile
    // lies wholly past K, loads as zeros and adds nothing.
    const int pairs = (K + 2 * BK - 1) / (2 * BK);
    load_tile(As0, Bs0, 0);
    __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
    __syncthreads();
    for (int pr = 0; pr < pairs; ++pr) {
        load_tile(As1, Bs1, 2 * pr + 1);
        compute(As0, Bs0);
        __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
        __syncthreads();
        // (unconditional, so the loads share the MFMAs' block: past K they
        // read zeros, and the wait below covers them)
        load_tile(As0, Bs0, 2 * pr + 2);
        compute(As1, Bs1);
        __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
        __syncthreads();
    }

    // ---- epilogue: bias, activation, residual, one store -----------------
    // The activation is chosen once per launch and a tile wholly inside C
    // takes a copy without bounds checks: per element, a four-way switch
    // and the row check made the unrolled epilogue thousands of branchy
    // instructions, fetched by every CU at once at the end of the launch.
    const float* __restrict__ bias = p.bias[g];
    const int cb = n0 + wn * WN + lr;
    float bv[TN];
#pragma unroll
    for (int j = 0; j < TN; ++j) bv[j] = bias && cb + 32 * j < N ? bias[cb + 32 * j] : 0.0f;
    const bool full = m0 + BM <= M && n0 + BN <= N;
    with_act(p.act, [&](auto act_c) {
        constexpr int ACT = decltype(act_c)::value;
        if (full) {
            // one 32 x 32 block at a time (a scheduling barrier between
            // blocks keeps the residual loads from all being hoisted at once)
#pragma unroll
            for (int j = 0; j < TN; ++j)
#pragma unroll
                for (int i = 0; i < TM; ++i) {
                    const size_t o0 = (size_t)(m0 + wm * WM + i * 32 + 4 * lk) * N + cb + 32 * j;
                    float* __restrict__ cp = C + o0;
                    if (R) {
                        const float* __restrict__ rp = R + o0;
#pragma unroll
                        for (int r = 0; r < 16; ++r) {
                            const size_t ro = (size_t)(8 * (r >> 2) + (r & 3)) * N;
                            cp[ro] = act_fixed<ACT>(acc[i][j][r] + bv[j]) + rp[ro];
                        }
                    } else {
#pragma unroll
                        for (int r = 0; r < 16; ++r)
                            cp[(size_t)(8 * (r >> 2) + (r & 3)) * N] = act_fixed<ACT>(acc[i][j][r] + bv[j]);
                    }
                    __builtin_amdgcn_sched_barrier(0);
                }
            return;
        }
        // a tile on the edge of C: the same blocks with bounds, the block's
        // residual values loaded before its stores
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const int col = cb + 32 * j;
            if (col >= N) continue;
#pragma unroll
            for (int i = 0; i < TM; ++i) {
                const int rbase = m0 + wm * WM + i * 32 + 4 * lk;
                float rv[16];
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int row = rbase + 8 * (r >> 2) + (r & 3);
                    rv[r] = R && row < M ? R[(size_t)row * N + col] : 0.0f;
                }
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int row = rbase + 8 * (r >> 2) + (r & 3);
                    if (row < M) {
                        const float v = act_fixed<ACT>(acc[i][j][r] + bv[j]);
                        C[(size_t)row * N + col] = R ? v + rv[r] : v;
                    }
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    });
}

// The direct-load pipeline of gemm_f32_direct for grids too small to give
// every CU several tiles: BM x BM tiles (BM = 128, or 64 for the smallest
// products) and KG k-groups of 4 waves in one workgroup.  Group g takes
// k-tiles g, g + KG, g + 2 KG, ... with its own pair of LDS buffers (same
// layouts and swizzles as gemm_f32_direct, scaled to BM), so a CU runs 4 KG
// waves on its tile instead of 4.  At the end the groups' sums are added
// through LDS in the fixed order (g0 + g1) + (g2 + g3), every wave taking a
// share of the tile's epilogue: results are run-to-run identical.
template <int BM, int KG, int BK = 16>
__global__ void __launch_bounds__(256 * KG, 1) gemm_f32_direct_kg(const GemmParams p) {
    constexpr int BN = BM;
    static_assert(BK == 16 || BK == 32, "k-tile");
    constexpr int WM = BM / 2, WN = BN / 2, TM = WM / 32, TN = WN / 32;
    constexpr int AI = BM * BK / 1024, BI = BN * BK / 1024;  // 16-byte loads per wave per k-tile
    constexpr int ACH = BK / 4;                                // 16-byte chunks of an A row
    constexpr int ASZ = BM * BK, BSZ = BK * BN;
    constexpr int STAGE = KG * 2 * (ASZ + BSZ);
    constexpr int RED = 2 * BM * BN;  // partial tiles in LDS at once
    static_assert(KG == 2 || KG == 4, "k-groups");
    typedef __attribute__((address_space(3))) void lds_void;
    __shared__ __attribute__((aligned(16))) float smem[STAGE > RED ? STAGE : RED];

    const int g = blockIdx.z;
    const float* __restrict__ A = p.A[g];
    const float* __restrict__ B = p.B[g];
    float* __restrict__ C = p.C[g];
    const float* __restrict__ R = p.R[g];
    const int M = p.M, N = p.N, K = p.K;
    const uint32_t ntiles = p.tiles_m * p.tiles_n;
    uint32_t tm_id, tn_id;
    grouped_tile(xcd_contiguous_id(blockIdx.x, ntiles), p.tiles_m, p.tiles_n, 4, tm_id, tn_id);
    const int m0 = (int)tm_id * BM;
    const int n0 = (int)tn_id * BN;

    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int grp = wave >> 2, gw = wave & 3;
    const int wm = gw >> 1, wn = gw & 1;
    const int lr = lane & 31, lk = lane >> 5;
    float* const As0 = smem + grp * 2 * (ASZ + BSZ);
    float* const As1 = As0 + ASZ;
    float* const Bs0 = As1 + ASZ;
    float* const Bs1 = Bs0 + BSZ;

    const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(A), 0, (int)((size_t)M * K * sizeof(float)), kBufferRsrcWord3);
    const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(B), 0, (int)((size_t)K * N * sizeof(float)), kBufferRsrcWord3);
    constexpr int kOut = 0x7ffffff0;  // an offset past the end of any operand: the load returns 0

    // A chunks: instruction i of wave gw fills chunks (AI gw + i) * 64 + lane
    // (row q / ACH, chunk (q % ACH) ^ aswz(row)); B chunks likewise (row
    // q / (BN / 4), chunk swizzled by 8 for the rows the second lane half
    // reads).  With BK = 16 a row is 4 chunks (4 rows per 256 bytes of
    // banks) and aswz(r) = (r >> 2) & 3; with BK = 32 it is 8 chunks (2 rows
    // per 256 bytes) and aswz(r) = (r >> 1) & 7: either way the 16-byte
    // reads of 16 consecutive rows at one chunk hit 16 different bank groups.
    auto aswz = [](int row) { return BK == 16 ? (row >> 2) & 3 : (row >> 1) & 7; };
    constexpr int BHALF = BK / 2;  // B row of the second lane half's first k
    int a_k[AI], a_off0[AI], b_kr[BI], b_off0[BI];
#pragma unroll
    for (int i = 0; i < AI; ++i) {
        const int q = (AI * gw + i) * 64 + lane;
        const int row = q / ACH, c = (q % ACH) ^ aswz(row);
        a_k[i] = 4 * c;
        a_off0[i] = (min(m0 + row, M - 1) * K + 4 * c) * (int)sizeof(float);
    }
#pragma unroll
    for (int i = 0; i < BI; ++i) {
        const int q = (BI * gw + i) * 64 + lane;
        const int kr = q / (BN / 4), lc = (q % (BN / 4)) ^ (((kr / BHALF) & 1) << 3);
        b_kr[i] = kr;
        b_off0[i] = (kr * N + min(n0 + 4 * lc, N - 4)) * (int)sizeof(float);
    }
    auto load_tile = [&](float* As, float* Bs, int kt) {
        const int k0 = kt * BK;
#pragma unroll
        for (int i = 0; i < AI; ++i) {
            const int ao = pick(k0 + a_k[i] < K, a_off0[i] + k0 * (int)sizeof(float), kOut);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_void*)(As + (AI * gw + i) * 256), 16, ao, 0, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < BI; ++i) {
            const int bo = pick(k0 + b_kr[i] < K, b_off0[i] + k0 * N * (int)sizeof(float), kOut);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, (lds_void*)(Bs + (BI * gw + i) * 256), 16, bo, 0, 0, 0);
        }
    };

    f32x16 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    // lane half lk of the MFMAs takes k in [lk BK/2, (lk + 1) BK/2) of the
    // k-tile (A chunks lk BK/8 .., B rows lk BK/2 ..)
    constexpr int AH = BK / 8;  // A chunks per lane half
    int a_rd[TM][AH];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int h = 0; h < AH; ++h) {
            const int row = wm * WM + i * 32 + lr, c = AH * lk + h;
            a_rd[i][h] = row * BK + 4 * (c ^ aswz(row));
        }
    int b_rd[TN];
#pragma unroll
    for (int j = 0; j < TN; ++j) {
        const int n = wn * WN + j * 32 + lr;
        b_rd[j] = BHALF * lk * BN + 4 * ((n >> 2) ^ (lk << 3)) + (n & 3);
    }
    // one global load after each of the k-tile's first MFMAs
    auto compute = [&](const float* As, const float* Bs) {
        f32x4 av[TM][AH];
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int h = 0; h < AH; ++h) av[i][h] = *(const f32x4*)(As + a_rd[i][h]);
#pragma unroll
        for (int kp = 0; kp < BK / 2; ++kp) {
            float bf[TN];
#pragma unroll
            for (int j = 0; j < TN; ++j) bf[j] = Bs[b_rd[j] + kp * BN];
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[i][kp / 4][kp % 4], bf[j], acc[i][j], 0, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < AI + BI; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
            __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // global load
        }
        __builtin_amdgcn_sched_group_barrier(0x008, TM * TN * BK / 2 - (AI + BI), 0);
        __builtin_amdgcn_sched_barrier(0);
    };

    // this group's k-tiles grp, grp + KG, ... in pairs; the groups run the
    // same number of steps, k-tiles past K load as zeros and add nothing
    const int ktiles = (K + BK - 1) / BK;
    const int steps = (ktiles + KG - 1) / KG;
    const int pairs = (steps + 1) / 2;
    load_tile(As0, Bs0, grp);
    __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
    __syncthreads();
    for (int pr = 0; pr < pairs; ++pr) {
        load_tile(As1, Bs1, grp + KG * (2 * pr + 1));
        compute(As0, Bs0);
        __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
        __syncthreads();
        load_tile(As0, Bs0, grp + KG * (2 * pr + 2));
        compute(As1, Bs1);
        __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
        __syncthreads();
    }

    // (g0 + g1) + (g2 + g3) through LDS: a group's sums are BM x BN floats,
    // stored per (wave, register quad, lane) as 16-byte pieces.  The last
    // two partial tiles (g0 + g1 and g2 + g3 with four groups, g0 and g1
    // with two) go to two LDS slots, and every wave of the workgroup adds
    // and stores its share of the pieces: the epilogue's stores spread over
    // all the waves instead of group 0's four (measured against group 0
    // alone, same box: 1024^3 22.8 -> 21.2 us, four grouped 1024x4096x1024
    // 255.8 -> 249.5, four grouped 1024^3 72.5 -> 70.8).
    constexpr int QUADS = TM * TN * 4;
    auto put = [&](int slot) {
        float* dst = smem + slot * BM * BN + gw * QUADS * 256;
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j)
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    *(f32x4*)(dst + (((i * TN + j) * 4 + q) * 64 + lane) * 4) =
                        f32x4{acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
    };
    if constexpr (KG == 4) {
        auto add = [&](int slot) {
            const float* src = smem + slot * BM * BN + gw * QUADS * 256;
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j)
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const f32x4 v = *(const f32x4*)(src + (((i * TN + j) * 4 + q) * 64 + lane) * 4);
                        acc[i][j][4 * q] += v.x;
                        acc[i][j][4 * q + 1] += v.y;
                        acc[i][j][4 * q + 2] += v.z;
                        acc[i][j][4 * q + 3] += v.w;
                    }
        };
        if (grp & 1) put(grp >> 1);
        __syncthreads();
        if (!(grp & 1)) add(grp >> 1);
        __syncthreads();
        if (!(grp & 1)) put(grp >> 1);
    } else {
        put(grp);
    }
    __syncthreads();

    // piece pi = (source wave pw, accumulator (i, j), quad q): lane l's four
    // values are rows 8q + 4(l/32) + 0..3, column l%32 of accumulator (i, j)
    // of wave pw's WM x WN block
    // Bias and residual values are all requested before the first store (a
    // load issued after a store waits for it: loads and stores complete in
    // order), and the activation is chosen once per launch.
    constexpr int NP = 4 * QUADS, NW = 4 * KG, T = NP / NW;
    const float* __restrict__ bias = p.bias[g];
    const int w = grp * 4 + gw;
    int col[T], rbase[T];
    float bv[T], rv[T][4];
#pragma unroll
    for (int t = 0; t < T; ++t) {
        const int pi = w + NW * t;
        const int pw = pi / QUADS, rest = pi % QUADS;
        const int i = (rest / 4) / TN, j = (rest / 4) % TN, q = rest % 4;
        col[t] = n0 + (pw & 1) * WN + j * 32 + lr;
        rbase[t] = m0 + (pw >> 1) * WM + i * 32 + 8 * q + 4 * lk;
        bv[t] = bias && col[t] < N ? bias[col[t]] : 0.0f;
#pragma unroll
        for (int s = 0; s < 4; ++s)
            rv[t][s] = R && col[t] < N && rbase[t] + s < M ? R[(size_t)(rbase[t] + s) * N + col[t]] : 0.0f;
    }
    with_act(p.act, [&](auto act_c) {
        constexpr int ACT = decltype(act_c)::value;
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const int pi = w + NW * t;
            const f32x4 s0 = *(const f32x4*)(smem + (pi * 64 + lane) * 4);
            const f32x4 s1 = *(const f32x4*)(smem + BM * BN + (pi * 64 + lane) * 4);
            const float sum[4] = {s0.x + s1.x, s0.y + s1.y, s0.z + s1.z, s0.w + s1.w};
            if (col[t] >= N) continue;
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                const int row = rbase[t] + s;
                if (row < M) {
                    const float v = act_fixed<ACT>(sum[s] + bv[t]);
                    C[(size_t)row * N + col[t]] = R ? v + rv[t][s] : v;
                }
            }
        }
    });
}

// Skinny GEMM (M <= 16*MT): the product is bound by reading B once from
// HBM (or, for tiny problems, by latency), so the kernel is organised around
// that stream.
//  * A workgroup of WAVES waves owns 64 columns and a K slice of 64*WAVES
//    rows; each wave takes 64 of those rows.  Lane l's MFMA k index l/16
//    stands for rows k0 + 16(l/16) + s of step s = 0..15 (any bijection of k
//    serves, as long as A and B use the same one), so a lane's A operands
//    for the whole slice are 16 consecutive floats of one A row: four float4
//    loads from L2 (A is small and shared), no LDS staging, no barrier.
//  * A loads are issued first, then all 16 B loads, and step s waits only
//    for its own B rows: the MFMAs run while later rows are in flight
//    instead of after the whole slice has arrived (the grid is one round of
//    workgroups, so there is nothing else to overlap them with).
//  * VB: every B load is a float4: lane l reads row k0 + 16(l/16) + s,
//    columns c0 + 4(l%16) .. +3, so 16 lanes stream 256 contiguous bytes of a
//    row and a wave keeps 16 KB in flight.  Otherwise (N % 4 != 0 or
//    unaligned B) the same four columns are four bounds-checked scalar loads.
//    Component j feeds its own v_mfma_f32_16x16x4_f32, whose column index
//    l%16 then stands for column c0 + 4(l%16) + j; the four MFMAs cover the
//    64 columns.
//  * VA: A rows are float4-loadable (K % 4 == 0, A 16-byte aligned, not
//    transposed); otherwise the 16 values are scalar loads (TA: A given
//    transposed, [K][M]).
//  * The waves' partial sums are added through LDS in wave order.  With
//    several K slices each workgroup stores its partial sums, and the K
//    slices are added in slice order y = 0, 1, ... (fixed, so results are
//    run-to-run identical):
//    - FUSED: in this launch, by the workgroup that arrives last at its
//      column block's counter.  An agent-scope release/acquire pair would
//      write back and invalidate the XCD's whole L2 (measured 4x slower), so
//      the partials instead go through the point of coherence: stored with
//      the device-scope cache policy (sc1: written through), the wave waits
//      for the stores to complete before the counter's atomic add, and the
//      last workgroup reads them back with sc1 loads (which miss in L2).
//      Workgroup-scope fences order the accesses; the sc1 accesses carry the
//      coherence.  The last workgroup resets the counter to zero, so
//      counters are zero between launches.
//    - otherwise a separate reduce kernel adds them (splitk_reduce*).
template <int MT, bool VB, bool TA, bool FUSED, int WAVES>
__global__ void __launch_bounds__(64 * WAVES) gemm_skinny_f32(const GemmParams p) {
    constexpr int KW = 64;           // K rows per wave
    constexpr int KS = KW * WAVES;   // K rows per workgroup
    constexpr int STEPS = 16;        // MFMA k-steps per wave
    constexpr int ROWS = 16 * MT;
    constexpr int NT = 64 * WAVES;   // threads
    __shared__ __attribute__((aligned(16))) float red[WAVES][ROWS][64];

    const int g = blockIdx.z, split = blockIdx.y, cb = blockIdx.x;
    const int M = p.M, N = p.N, K = p.K;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int kq = lane >> 4, cq = lane & 15;
    const int c0 = cb * 64;
    const int col4 = c0 + 4 * cq;
    const int kbase = split * KS + wave * KW + 16 * kq;  // this lane's 16 rows: kbase .. kbase + 15
    const float* __restrict__ A = p.A[g];
    const float* __restrict__ B = p.B[g];

    // A operands first: av[t][s] = A[16t + cq][kbase + s].  The float4 loads
    // go through buffer resources with past-the-end offsets for elements
    // that do not exist (the load returns 0): a branch around each load, as
    // hipcc compiles a plain guarded load, costs as much as the load.
    constexpr int kOut = 0x7ffffff0;
    float av[MT][STEPS];
    const bool va = !TA && (K % 4 == 0) && (((uintptr_t)A & 15u) == 0) && (size_t)M * K < ((size_t)1 << 29);
    const __amdgpu_buffer_rsrc_t ra =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(A), 0, va ? M * K * (int)sizeof(float) : 0,
                                          kBufferRsrcWord3);
#pragma unroll
    for (int t = 0; t < MT; ++t) {
        const int m = 16 * t + cq;
        if (va) {
#pragma unroll
            for (int q = 0; q < STEPS / 4; ++q) {
                const int k = kbase + 4 * q;
                const f32x4 x = __builtin_bit_cast(
                    f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                               ra, pick((m < M) & (k < K), (m * K + k) * (int)sizeof(float), kOut), 0, 0));
                av[t][4 * q] = x.x;
                av[t][4 * q + 1] = x.y;
                av[t][4 * q + 2] = x.z;
                av[t][4 * q + 3] = x.w;
            }
        } else {
#pragma unroll
            for (int s = 0; s < STEPS; ++s) {
                const int k = kbase + s;
                av[t][s] = (m < M && k < K) ? (TA ? A[(size_t)k * M + m] : A[(size_t)m * K + k]) : 0.0f;
            }
        }
    }
    // then every B load of the slice (VB: a buffer over the slice's rows,
    // rows past K past its end)
    f32x4 bv[STEPS];
    const int k_slice = split * KS;
    const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(B + (size_t)k_slice * N), 0, VB ? min(KS, K - k_slice) * N * (int)sizeof(float) : 0,
        kBufferRsrcWord3);
#pragma unroll
    for (int s = 0; s < STEPS; ++s) {
        const int k = kbase + s;
        if constexpr (VB) {
            bv[s] = __builtin_bit_cast(
                f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                           rb, pick(col4 < N, ((k - k_slice) * N + col4) * (int)sizeof(float), kOut), 0, 0));
        } else {
            const float* row = B + (size_t)k * N;
            const bool kin = k < K;
            bv[s] = f32x4{(kin && col4 < N) ? row[col4] : 0.f, (kin && col4 + 1 < N) ? row[col4 + 1] : 0.f,
                          (kin && col4 + 2 < N) ? row[col4 + 2] : 0.f, (kin && col4 + 3 < N) ? row[col4 + 3] : 0.f};
        }
    }
    // every load of the slice is in flight before the first MFMA (the
    // scheduler would otherwise place each load next to its MFMA)
    __builtin_amdgcn_sched_barrier(0);

    f32x4 acc[MT][4];
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[t][j] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < STEPS; ++s) {
#pragma unroll
        for (int t = 0; t < MT; ++t) {
            acc[t][0] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[t][s], bv[s].x, acc[t][0], 0, 0, 0);
            acc[t][1] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[t][s], bv[s].y, acc[t][1], 0, 0, 0);
            acc[t][2] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[t][s], bv[s].z, acc[t][2], 0, 0, 0);
            acc[t][3] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[t][s], bv[s].w, acc[t][3], 0, 0, 0);
        }
    }
    // Accumulator (t, j), register r of lane l: row 16t + 4(l/16) + r,
    // column c0 + 4(l%16) + j.
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r)
            *(f32x4*)&red[wave][16 * t + 4 * kq + r][4 * cq] =
                f32x4{acc[t][0][r], acc[t][1][r], acc[t][2][r], acc[t][3][r]};
    __syncthreads();

    // ROWS x 16 float4 groups of the tile; thread e4 < ROWS*16 owns group e4
    // (row e4 / 16, columns c0 + 4 (e4 % 16) .. +3); the waves' sums are
    // added in wave order.
    constexpr int GROUPS = ROWS * 16;
    static_assert(GROUPS <= NT, "one float4 group per thread");
    const int e4 = tid;
    const int row = e4 / 16, col = c0 + 4 * (e4 % 16), cc = 4 * (e4 % 16);
    const bool mine = e4 < GROUPS && row < M && col < N;
    f32x4 v = f32x4{0.f, 0.f, 0.f, 0.f};
    if (mine) {
        v = *(const f32x4*)&red[0][row][cc];
#pragma unroll
        for (int w = 1; w < WAVES; ++w) v += *(const f32x4*)&red[w][row][cc];
    }

    const float* __restrict__ bias = p.bias[g];
    const float* __restrict__ R = p.R[g];
    float* __restrict__ C = p.C[g];
    const size_t MN = (size_t)M * N;
    if constexpr (FUSED) {
        if (p.splits > 1) {
            // This group's partials as a raw buffer: 16-byte loads and stores
            // with the device-scope cache policy (sc1) the coherence needs.
            const __amdgpu_buffer_rsrc_t part = __builtin_amdgcn_make_buffer_rsrc(
                p.ws + (size_t)g * p.splits * MN, 0, (int)(p.splits * MN * sizeof(float)), kBufferRsrcWord3);
            // 1. this K slice's partial sums, written through to the point of coherence
            if (mine) {
                const int off = (int)(((size_t)split * MN + (size_t)row * N + col) * sizeof(float));
                if constexpr (VB) {
                    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), part, off, 0, kCachePolicySc1);
                } else {
                    const float o[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        if (col + j < N)
                            __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, o[j]), part,
                                                                  off + 4 * j, 0, kCachePolicySc1);
                }
            }
            // 2. arrival: the stores have completed before the counter moves
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
            __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
            __shared__ int s_last;
            __syncthreads();
            unsigned* ctr = p.counters + (size_t)g * gridDim.x + cb;
            if (tid == 0)
                s_last = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                         (unsigned)(p.splits - 1);
            __syncthreads();
            if (!s_last) return;
            __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
            // 3. the last workgroup adds the slices in order y = 0, 1, ... and
            //    runs the epilogue; the loads of up to kLoadsInFlight slices
            //    are issued before the first add
            if (mine) {
                constexpr int kLoadsInFlight = 16;
                const int off = (int)(((size_t)row * N + col) * sizeof(float));
                const int step = (int)(MN * sizeof(float));
                f32x4 sum = f32x4{0.f, 0.f, 0.f, 0.f};
                for (int y0 = 0; y0 < p.splits; y0 += kLoadsInFlight) {
                    f32x4 pv[kLoadsInFlight];
#pragma unroll
                    for (int t = 0; t < kLoadsInFlight; ++t) {
                        if (y0 + t >= p.splits) break;
                        if constexpr (VB) {
                            pv[t] = __builtin_bit_cast(
                                f32x4, __builtin_amdgcn_raw_buffer_load_b128(part, off + (y0 + t) * step, 0,
                                                                             kCachePolicySc1));
                        } else {
#pragma unroll
                            for (int j = 0; j < 4; ++j)
                                pv[t][j] = col + j < N ? __builtin_bit_cast(
                                                             float, __builtin_amdgcn_raw_buffer_load_b32(
                                                                        part, off + (y0 + t) * step + 4 * j, 0,
                                                                        kCachePolicySc1))
                                                       : 0.0f;
                        }
                    }
#pragma unroll
                    for (int t = 0; t < kLoadsInFlight; ++t) {
                        if (y0 + t >= p.splits) break;
                        sum = (y0 + t == 0) ? pv[t] : sum + pv[t];
                    }
                }
                v = sum;
            }
            if (tid == 0) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    if (!mine) return;
    float o[4] = {v.x, v.y, v.z, v.w};
    const bool direct = p.splits == 1 || FUSED;
    float* dst = direct ? C + (size_t)row * N + col
                        : p.ws + ((size_t)g * p.splits + split) * MN + (size_t)row * N + col;
    if (direct) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            if (!VB && col + j >= N) break;
            float y = o[j] + (bias ? bias[col + j] : 0.0f);
            y = apply_act(y, p.act);
            if (R) y += R[(size_t)row * N + col + j];
            o[j] = y;
        }
    }
    if constexpr (VB) {
        *(f32x4*)dst = f32x4{o[0], o[1], o[2], o[3]};
    } else {
#pragma unroll
        for (int j = 0; j < 4; ++j)
            if (col + j < N) dst[j] = o[j];
    }
}

// Sums split-K partials in split order and applies the epilogue.
__global__ void __launch_bounds__(256) splitk_reduce(const GemmParams p, int count) {
    const size_t MN = (size_t)p.M * p.N;
    const size_t total = (size_t)count * MN;
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total; idx += stride) {
        const int g = (int)(idx / MN);
        const size_t e = idx - (size_t)g * MN;
        const float* part = p.ws + (size_t)g * p.splits * MN + e;
        float s = 0.0f;
        for (int y = 0; y < p.splits; ++y) s += part[(size_t)y * MN];
        const int col = (int)(e % p.N);
        if (p.bias[g]) s += p.bias[g][col];
        s = apply_act(s, p.act);
        if (p.R[g]) s += p.R[g][e];
        p.C[g][e] = s;
    }
}

// SPLITS: the configuration can be chosen for a split K (grids under 256
// tiles); VECS: with float4 operand loads (false where the dispatch sends
// every float4-shaped case of the configuration to a direct kernel).  Only
// the variants the dispatch can reach are built.
template <int BM, int BN, int BK, int WGM, int WGN, int OCC = 1, bool TA = false, bool TB = false, int KG = 1,
          bool SPLITS = true, bool VECS = true>
int launch_cfg(lancius_hip_ctx* ctx, GemmParams& p, int count, bool vec) {
    constexpr int SOCC = KG > 1 ? OCC : 1;  // occupancy hint of the split and scalar variants
    p.tiles_m = (uint32_t)((p.M + BM - 1) / BM);
    p.tiles_n = (uint32_t)((p.N + BN - 1) / BN);
    dim3 grid(p.tiles_m * p.tiles_n, (unsigned)p.splits, (unsigned)count);
    const bool split = p.splits > 1;
    LANCIUS_REQUIRE((SPLITS || !split) && (VECS || !vec), LANCIUS_HIP_ERR_INTERNAL,
                    "gemm: configuration %dx%d/%d without this variant (split %d, vec %d)", BM, BN, BK, (int)split,
                    (int)vec);
    const dim3 block(kThreads * KG);
    if constexpr (SPLITS && VECS) {
        if (vec && split) {
            hipLaunchKernelGGL((gemm_f32_mfma<BM, BN, BK, WGM, WGN, true, true, SOCC, TA, TB, KG>), grid, block, 0,
                               ctx->stream, p);
            goto launched;
        }
    }
    if constexpr (VECS) {
        if (vec) {
            hipLaunchKernelGGL((gemm_f32_mfma<BM, BN, BK, WGM, WGN, true, false, OCC, TA, TB, KG>), grid, block, 0,
                               ctx->stream, p);
            goto launched;
        }
    }
    if constexpr (SPLITS) {
        if (split) {
            hipLaunchKernelGGL((gemm_f32_mfma<BM, BN, BK, WGM, WGN, false, true, SOCC, TA, TB, KG>), grid, block, 0,
                               ctx->stream, p);
            goto launched;
        }
    }
    hipLaunchKernelGGL((gemm_f32_mfma<BM, BN, BK, WGM, WGN, false, false, SOCC, TA, TB, KG>), grid, block, 0,
                       ctx->stream, p);
launched:
    if (int rc = check_launch("gemm_f32_mfma")) return rc;
    if (split) {
        const size_t total = (size_t)count * p.M * p.N;
        const unsigned blocks = (unsigned)std::min<size_t>((total + 255) / 256, 4096);
        hipLaunchKernelGGL(splitk_reduce, dim3(blocks), dim3(256), 0, ctx->stream, p, count);
        if (int rc = check_launch("splitk_reduce")) return rc;
    }
    return 0;
}

// Transposed operands are built for the two default tile shapes only.
// Configurations 6 and 8 run grids of at least 256 tiles, which never split
// K; with plain operands, configuration 6's float4 case is the direct
// kernel's (the dispatch sends operands beyond its 2 GiB offsets to the
// scalar variant).
template <bool TA, bool TB>
int launch_by_cfg(lancius_hip_ctx* ctx, GemmParams& p, int count, bool vec, int cfg) {
    if constexpr (TA || TB) {
        if (cfg == 2) return launch_cfg<64, 64, 16, 2, 2, 1, TA, TB>(ctx, p, count, vec);
        return launch_cfg<128, 128, 16, 2, 2, 4, TA, TB, 1, false>(ctx, p, count, vec);
    } else {
        switch (cfg) {
            case 2: return launch_cfg<64, 64, 16, 2, 2>(ctx, p, count, vec);
            case 7: return launch_cfg<128, 128, 32, 2, 2, 2, false, false, 2>(ctx, p, count, vec);
            case 8: return launch_cfg<128, 128, 32, 2, 2, 1, false, false, 4, false>(ctx, p, count, vec);
            case 9: return launch_cfg<64, 64, 64, 2, 2, 1, false, false, 4>(ctx, p, count, vec);
            default: return launch_cfg<128, 128, 16, 2, 2, 4, false, false, 1, false, false>(ctx, p, count, vec);  // 6
        }
    }
}

// Waves per workgroup of the skinny kernel (K rows per workgroup = 64 x
// waves).  8 measured best on MI355X: 16x4096x4096 15.9 us against 16.4 /
// 15.9 at 4 / 16 waves, 16x8192x8192 51.5 against 57.3 / 53.1, 8x1024x768
// 7.8 against 8.7 / 8.6.
constexpr int kSkinnyWaves = 8;

template <int MT, bool TA, int WAVES>
void launch_skinny(lancius_hip_ctx* ctx, const GemmParams& p, dim3 grid, bool vb, bool fused) {
    const dim3 block(64 * WAVES);
    if (vb && fused)
        hipLaunchKernelGGL((gemm_skinny_f32<MT, true, TA, true, WAVES>), grid, block, 0, ctx->stream, p);
    else if (fused)
        hipLaunchKernelGGL((gemm_skinny_f32<MT, false, TA, true, WAVES>), grid, block, 0, ctx->stream, p);
    else if (vb)
        hipLaunchKernelGGL((gemm_skinny_f32<MT, true, TA, false, WAVES>), grid, block, 0, ctx->stream, p);
    else
        hipLaunchKernelGGL((gemm_skinny_f32<MT, false, TA, false, WAVES>), grid, block, 0, ctx->stream, p);
}

template <bool TA>
void launch_skinny_rows(lancius_hip_ctx* ctx, const GemmParams& p, dim3 grid, bool vb, bool fused, int mt) {
    if (mt == 1) return launch_skinny<1, TA, kSkinnyWaves>(ctx, p, grid, vb, fused);
    return launch_skinny<2, TA, kSkinnyWaves>(ctx, p, grid, vb, fused);  // 32 rows x 16 float4 groups: 512 threads
}

bool aligned16(const void* ptr) { return ((uintptr_t)ptr & 15u) == 0; }

// Scratch of lancius_hip_gemm_f32_noalloc: split-K partial sums, then
// kScratchCounters arrival counters (zero between launches).  Each GPU the
// library runs on holds its own copy of this array until the process ends.
// Host code never uses the name itself (on the host it only stands for the
// symbol): the per-device address comes from hipGetSymbolAddress, below.
constexpr size_t kNoallocScratchBytes = LANCIUS_HIP_NOALLOC_SCRATCH_BYTES;
constexpr size_t kScratchCounters = 16384;
constexpr size_t kScratchPartialBytes = kNoallocScratchBytes - kScratchCounters * sizeof(unsigned);
static __device__ __align__(256) unsigned char scratch[kNoallocScratchBytes];

constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxScratchDevices];  // device address of `scratch`, by device index

__global__ void zero_words(unsigned* p, size_t n) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        p[i] = 0u;
}

// Where a GEMM puts split-K partial sums and arrival counters: the context's
// workspace and counters (grown on demand), or a fixed buffer.
struct SplitStore {
    void* partials = nullptr;  // null: the context workspace
    size_t partial_bytes = 0;
    unsigned* counters = nullptr;
    size_t n_counters = 0;
};

// The calling device's scratch; its address is resolved (and its counters
// cleared by a kernel, not a memset, so a caller may capture the call) once
// per device, with that device current (the caller has bound ctx->device).
}  // namespace

// Resolves the scratch's address on the context's device (which is
// current) and clears its counters, once per device; lancius_hip_ctx_create
// calls it, so a lancius_hip_gemm_f32_noalloc call, under stream capture
// or not, never does more than read the cached address.  The clearing runs
// on a private stream and is waited for here, outside any capture.
int noalloc_scratch_init(lancius_hip_ctx* ctx) {
    if (ctx->device < 0 || ctx->device >= kMaxScratchDevices) return 0;  // the entry point reports it
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_ptr[ctx->device]) return 0;
    void* p = nullptr;
    LANCIUS_HIP_TRY(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
    LANCIUS_REQUIRE(p != nullptr, LANCIUS_HIP_ERR_INTERNAL, "gemm_f32_noalloc: no address for the scratch");
    hipStream_t s = nullptr;
    LANCIUS_HIP_TRY(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "hipStreamCreateWithFlags");
    hipLaunchKernelGGL(zero_words, dim3(16), dim3(256), 0, s, (unsigned*)((char*)p + kScratchPartialBytes),
                       kScratchCounters);
    hipError_t e = hipGetLastError();
    const hipError_t e2 = hipStreamSynchronize(s);
    const hipError_t e3 = hipStreamDestroy(s);
    if (e == hipSuccess) e = e2 != hipSuccess ? e2 : e3;
    if (e != hipSuccess) return from_hip(e, "noalloc scratch init");
    g_scratch_ptr[ctx->device] = p;
    return 0;
}

namespace {

int noalloc_scratch(lancius_hip_ctx* ctx, SplitStore* out) {
    LANCIUS_REQUIRE(ctx->device >= 0 && ctx->device < kMaxScratchDevices, LANCIUS_HIP_ERR_UNSUPPORTED,
                    "gemm_f32_noalloc: device index %d beyond %d", ctx->device, kMaxScratchDevices);
    void* p;
    {
        std::lock_guard<std::mutex> lock(g_scratch_mu);
        p = g_scratch_ptr[ctx->device];
    }
    LANCIUS_REQUIRE(p != nullptr, LANCIUS_HIP_ERR_INTERNAL,
                    "gemm_f32_noalloc: the scratch of device %d was not set up by lancius_hip_ctx_create",
                    ctx->device);
    out->partials = p;
    out->partial_bytes = kScratchPartialBytes;
    out->counters = (unsigned*)((char*)out->partials + kScratchPartialBytes);
    out->n_counters = kScratchCounters;
    return 0;
}

// Device memory for `bytes` of split-K partials: the context workspace, or
// the fixed buffer of `st`, with a clear error when the shape needs more.
int partials(lancius_hip_ctx* ctx, const SplitStore* st, size_t bytes, void** out) {
    if (!st || !st->partials) return workspace(ctx, bytes, out);
    *out = nullptr;
    LANCIUS_REQUIRE(bytes <= st->partial_bytes, LANCIUS_HIP_ERR_SHAPE,
                    "gemm_f32_noalloc: this shape splits K into partial sums of %zu bytes, more than the %zu-byte "
                    "scratch (use lancius_hip_gemm_f32)",
                    bytes, st->partial_bytes);
    *out = st->partials;
    return 0;
}

// `n` zero arrival counters: the context's, or those of `st`.
int arrival_counters(lancius_hip_ctx* ctx, const SplitStore* st, size_t n, unsigned** out) {
    if (!st || !st->partials) return counters(ctx, n, out);
    *out = nullptr;
    LANCIUS_REQUIRE(n <= st->n_counters, LANCIUS_HIP_ERR_SHAPE,
                    "gemm_f32_noalloc: %zu column blocks need more than the scratch's %zu counters", n,
                    st->n_counters);
    *out = st->counters;
    return 0;
}

constexpr int kBK = 16;
constexpr size_t kMaxSplitBytes = (size_t)256 << 20;

// fixed: when not null, split-K partials and arrival counters go to its
// buffers instead of the context's, and nothing is allocated.
int gemm_dispatch(lancius_hip_ctx* ctx, size_t count, float* const* C, const float* const* A,
                  const float* const* B, size_t M, size_t K, size_t N, int ta, int tb, const float* const* bias,
                  int act, const float* const* residual, const SplitStore* fixed = nullptr) {
    LANCIUS_REQUIRE(ctx && C && A && B, LANCIUS_HIP_ERR_NULL_PTR, "gemm: NULL argument");
    LANCIUS_REQUIRE(count >= 1 && count <= LANCIUS_HIP_MAX_GROUP, LANCIUS_HIP_ERR_SHAPE, "gemm: group count %zu",
                    count);
    LANCIUS_REQUIRE(M > 0 && N > 0 && K > 0, LANCIUS_HIP_ERR_SHAPE, "gemm: empty shape M=%zu K=%zu N=%zu", M, K, N);
    LANCIUS_REQUIRE(M < (1u << 30) && N < (1u << 30) && K < (1u << 30), LANCIUS_HIP_ERR_SHAPE,
                    "gemm: dimension too large");
    LANCIUS_REQUIRE(act >= LANCIUS_HIP_ACT_NONE && act <= LANCIUS_HIP_ACT_TANH, LANCIUS_HIP_ERR_UNSUPPORTED,
                    "gemm: activation %d", act);
    if (int rc = bind_device(ctx)) return rc;
    ta = ta != 0;
    tb = tb != 0;
    // 32 < M <= 64 with a large B: rows 0-31 and the rest as two skinny
    // products (B read twice from HBM) beat the tiled kernels, which read it
    // once but keep most CUs idle.  Measured: 64x4096x4096 48.0 -> 39.5 us,
    // 48x4096x4096 46.9 -> 34.8 us; at B of 16 MiB and less it measured
    // slower (64x4096x1024 17.9 -> 22.2 us, 64x1024x1024 11.6 -> 19.7 us).
    if (M > 32 && M <= 64 && !ta && !tb && K * N >= ((size_t)1 << 23)) {
        const float* a2[LANCIUS_HIP_MAX_GROUP];
        float* c2[LANCIUS_HIP_MAX_GROUP];
        const float* r2[LANCIUS_HIP_MAX_GROUP];
        for (size_t g = 0; g < count; ++g) {
            LANCIUS_REQUIRE(C[g] && A[g] && B[g], LANCIUS_HIP_ERR_NULL_PTR, "gemm: NULL operand in group %zu", g);
            a2[g] = A[g] + 32 * K;
            c2[g] = C[g] + 32 * N;
            r2[g] = residual && residual[g] ? residual[g] + 32 * N : nullptr;
        }
        if (int rc = gemm_dispatch(ctx, count, C, A, B, 32, K, N, 0, 0, bias, act, residual, fixed)) return rc;
        return gemm_dispatch(ctx, count, c2, a2, B, M - 32, K, N, 0, 0, bias, act, residual ? r2 : nullptr, fixed);
    }

    GemmParams p{};
    // float4 global loads run along each operand's contiguous axis
    bool vec = ((ta ? M : K) % 4 == 0) && ((tb ? K : N) % 4 == 0);
    // skinny: float4 B rows (a K slice of up to 1024 rows within 32-bit
    // buffer offsets) and float4 C / partial stores
    bool vb = N % 4 == 0 && N < ((size_t)1 << 19);
    for (size_t g = 0; g < count; ++g) {
        LANCIUS_REQUIRE(C[g] && A[g] && B[g], LANCIUS_HIP_ERR_NULL_PTR, "gemm: NULL operand in group %zu", g);
        p.C[g] = C[g];
        p.A[g] = A[g];
        p.B[g] = B[g];
        p.bias[g] = bias ? bias[g] : nullptr;
        p.R[g] = residual ? residual[g] : nullptr;
        vec = vec && aligned16(A[g]) && aligned16(B[g]);
        vb = vb && aligned16(B[g]) && aligned16(C[g]);
    }
    p.M = (int)M;
    p.N = (int)N;
    p.K = (int)K;
    p.act = act;

    // M <= 32 (B not transposed): the B-streaming skinny kernel, one
    // workgroup per (64 columns, 64 x waves K rows), the K slices added
    // inside the launch.  Measured on MI355X it beats the tiled kernel up to
    // M = 32 (16x4096x4096: 22 vs 34 us with the first skinny design;
    // 32x2048x120: 10.6 vs 13.6 us) and loses at M = 64 with four row tiles
    // (64x4096x4096: 43 vs 38 us; 64x784x256: 13.0 vs 11.8 us).
    if (M <= 32 && !tb) {
        const int mt = M <= 16 ? 1 : 2;
        const size_t splits = (K + 64 * kSkinnyWaves - 1) / (64 * kSkinnyWaves);
        const size_t col_blocks = (N + 63) / 64;
        const size_t ws_bytes = splits > 1 ? count * splits * M * N * sizeof(float) : 0;
        if (ws_bytes <= kMaxSplitBytes && splits < 65536 && col_blocks < kMaxGridX) {
            // the K slices are added inside the launch (see gemm_skinny_f32)
            const bool fused = splits > 1;
            if (splits > 1) {
                void* ws = nullptr;
                if (int rc = partials(ctx, fixed, ws_bytes, &ws)) return rc;
                p.ws = (float*)ws;
                if (fused)
                    if (int rc = arrival_counters(ctx, fixed, count * col_blocks, &p.counters)) return rc;
            }
            p.splits = (int)splits;
            const dim3 grid((unsigned)col_blocks, (unsigned)splits, (unsigned)count);
            if (ta)
                launch_skinny_rows<true>(ctx, p, grid, vb, fused, mt);
            else
                launch_skinny_rows<false>(ctx, p, grid, vb, fused, mt);
            if (int rc = check_launch("gemm_skinny_f32")) return rc;
            return ok();
        }
    }

    // Configurations (BM x BN / BK, k-groups): 2 = 64x64/16, 6 = 128x128/16
    // built for 4 workgroups per CU, 7 = 128x128/32 x2, 8 = 128x128/32 x4,
    // 9 = 64x64/64 x4.  Chosen by the number of 128x128 tiles (one per CU
    // fills the chip once), measured on MI355X:
    //  * >= 768: 6 (4096^3: 112 TFLOP/s);
    //  * 384 .. 767: 7 (two 8-wave workgroups per CU);
    //  * 256 .. 383: 8, 16 waves on the CU's one tile (2048^3: 205 -> 190
    //    us; 4096x1024x1024: 110 -> 103 us);
    //  * fewer, K >= 2048: 7 with split-K (1024x4096x1024: 137 -> 103 us);
    //  * fewer, shorter K: 9 (1024^3: 38.9 -> 34.0 us), or 2 for small
    //    grids and transposed operands.
    // Split-K when the grid still leaves CUs idle and K is long enough:
    // enough K ranges for ~512 workgroups, each >= 128 deep.
    const size_t big_tiles = count * ((M + 127) / 128) * ((N + 127) / 128);
    const size_t t64 = count * ((M + 63) / 64) * ((N + 63) / 64);
    const bool plain = !ta && !tb;
    int cfg;
    if (big_tiles >= 768)
        cfg = 6;
    else if (big_tiles >= 384)
        cfg = plain ? 7 : 6;
    else if (big_tiles >= 256)
        cfg = plain ? 8 : 6;
    else if (plain && K >= 2048 && big_tiles >= 16)
        cfg = 7;
    else if (plain && t64 >= 64)
        cfg = 9;
    else
        cfg = 2;
    const bool small = cfg == 2 || cfg == 9;
    const size_t bm = small ? 64 : 128;
    const size_t bn = bm;
    const size_t bk = cfg == 9 ? 64 : cfg == 7 || cfg == 8 ? 32 : kBK;
    const size_t tiles = count * ((M + bm - 1) / bm) * ((N + bn - 1) / bn);
    const size_t ktiles = (K + bk - 1) / bk;
    size_t splits = 1;
    if (tiles < 256 && K >= 256) splits = std::min<size_t>({(512 + tiles - 1) / tiles, K / 128, 16});
    splits = std::max<size_t>(1, std::min(splits, ktiles));
    size_t chunk_tiles = (ktiles + splits - 1) / splits;
    splits = (ktiles + chunk_tiles - 1) / chunk_tiles;  // no empty K range
    while (splits > 1 && count * splits * M * N * sizeof(float) > kMaxSplitBytes) {
        splits = (splits + 1) / 2;
        chunk_tiles = (ktiles + splits - 1) / splits;
        splits = (ktiles + chunk_tiles - 1) / chunk_tiles;
    }
    p.splits = (int)splits;
    p.kchunk = (int)(chunk_tiles * bk);
    // 128x128 tiles loaded straight into LDS (gemm_f32_direct)
    if (cfg == 6 && splits == 1 && vec && !ta && !tb &&
        M * K * sizeof(float) < ((size_t)1 << 31) && K * N * sizeof(float) < ((size_t)1 << 31)) {
        p.tiles_m = (uint32_t)((M + 127) / 128);
        p.tiles_n = (uint32_t)((N + 127) / 128);
        // the k-tile's four loads one after each of the first four MFMAs
        // (measured 143.0 -> 144.4 TFLOP/s at 4096^3; a burst before the
        // MFMAs, or one load per 2, 4 or 7 MFMAs, ran slower)
        hipLaunchKernelGGL(gemm_f32_direct<4>, dim3(p.tiles_m * p.tiles_n, 1, (unsigned)count), dim3(256), 0, ctx->stream, p);
        if (int rc = check_launch("gemm_f32_direct")) return rc;
        return ok();
    }
    // Grids that give a CU about one 128 x 128 tile (or one 64 x 64 tile):
    // the direct-load pipeline with the K loop spread over k-groups of
    // 4 waves inside the workgroup (gemm_f32_direct_kg)
    if (vec && plain && M * K * sizeof(float) < ((size_t)1 << 31) && K * N * sizeof(float) < ((size_t)1 << 31) &&
        K >= 256 && big_tiles < 768) {
        // 64 x 64 tiles, with 4 k-groups when that gives about one tile per
        // CU and 2 otherwise; 128 x 128 tiles with 4 k-groups (16 waves, 100
        // registers each) for K >= 2048 with >= 192 of them.
        // Measured on MI355X (old dispatch -> this): 1024^3 27.0 -> 23.7 us,
        // 2048^3 146.0 -> 135.6, 4096x1024x1024 82.4 -> 71.3,
        // 1024x4096x1024 84.4 -> 76.4, 4096x4096x1024 275.2 -> 257.3,
        // 3000x1000x2000 145.8 -> 104.3.  The 128 x 128 tiles with 4 k-groups
        // of 16-deep k-tiles against 2 k-groups of 32-deep ones (one box, the
        // two builds alternated): 2048^3 131.3 -> 129.0 us, 2048x4096x2048
        // 251.1 -> 246.7, 2048x2048x4096 259.3 -> 254.2, four grouped
        // 1024x4096x1024 (bias and residual) 259.8 -> 251.4.  At K = 1024 they
        // lose to 64 x 64 tiles unless the grid is exactly 256 of them (3072 x
        // 1024 x 1024: 54.9 -> 69.2 us; 4096 x 1024 x 1024: 70.5 -> 69.9).
        // (128 x 128 tiles from 256 of them: with 192 to 255 the 64 x 64
        // tiles measured faster, 768x4096x4096 245.5 -> 195.5 us and
        // 4096x2048x768 127.7 -> 101.8 us, one box, builds alternated)
        const int bm_kg = K >= 2048 && big_tiles >= 256 ? 128 : 64;
        const int kg = bm_kg == 128 || t64 <= 384 ? 4 : 2;
        const size_t kg_tiles = count * ((M + bm_kg - 1) / bm_kg) * ((N + bm_kg - 1) / bm_kg);
        // at least 192 tiles: with 128 to 191 the split-K tiled kernels
        // below are faster (128x4096x4096 72.0 -> 52.2 us, 4096x4096x128
        // 74.6 -> 51.3 us, 96x4096x4096 71.5 -> 51.5 us, 128x2048x4096 38.1
        // -> 35.0 us; 192 tiles, e.g. 192x4096x4096, measured 71.7 against
        // 84.0 us split)
        if (kg_tiles >= 192) {
            p.tiles_m = (uint32_t)((M + bm_kg - 1) / bm_kg);
            p.tiles_n = (uint32_t)((N + bm_kg - 1) / bm_kg);
            // k-tiles of 16: with 32 (half the barriers per k) the 64 x 64
            // tiles measured no better (1024^3 23.9 -> 24.3 us, four grouped
            // 72.1 -> 72.7 us), and 128 x 128 tiles with 4 k-groups would
            // need 256 KB of LDS
            void (*kern)(const GemmParams) = bm_kg == 128 ? gemm_f32_direct_kg<128, 4>
                                                          : (kg == 2 ? gemm_f32_direct_kg<64, 2> : gemm_f32_direct_kg<64, 4>);
            hipLaunchKernelGGL(kern, dim3(p.tiles_m * p.tiles_n, 1, (unsigned)count), dim3(256 * kg), 0,
                               ctx->stream, p);
            if (int rc = check_launch("gemm_f32_direct_kg")) return rc;
            return ok();
        }
    }
    if (splits > 1) {
        void* ws = nullptr;
        if (int rc = partials(ctx, fixed, count * splits * M * N * sizeof(float), &ws)) return rc;
        p.ws = (float*)ws;
    }
    // plain configuration-6 operands beyond the direct kernel's offsets: scalar loads
    if (cfg == 6 && plain) vec = false;
    int rc;
    if (ta && tb)
        rc = launch_by_cfg<true, true>(ctx, p, (int)count, vec, cfg);
    else if (ta)
        rc = launch_by_cfg<true, false>(ctx, p, (int)count, vec, cfg);
    else if (tb)
        rc = launch_by_cfg<false, true>(ctx, p, (int)count, vec, cfg);
    else
        rc = launch_by_cfg<false, false>(ctx, p, (int)count, vec, cfg);
    return rc ? rc : ok();
}

}  // namespace
}  // namespace lancius

using namespace lancius;

extern "C" {

int lancius_hip_gemm_f32(lancius_hip_ctx* ctx, float* C, const float* A, const float* B, size_t M, size_t K,
                         size_t N, const float* bias, int act, const float* residual) {
    float* c1[1] = {C};
    const float* a1[1] = {A};
    const float* b1[1] = {B};
    const float* s1[1] = {bias};
    const float* r1[1] = {residual};
    return gemm_dispatch(ctx, 1, c1, a1, b1, M, K, N, 0, 0, s1, act, r1);
}

int lancius_hip_gemm_f32_noalloc(lancius_hip_ctx* ctx, float* C, const float* A, const float* B, size_t M,
                                 size_t K, size_t N, const float* bias, int act, const float* residual) {
    LANCIUS_REQUIRE(ctx != nullptr, LANCIUS_HIP_ERR_NULL_PTR, "gemm_f32_noalloc: NULL context");
    if (int rc = bind_device(ctx)) return rc;
    SplitStore st;
    if (int rc = noalloc_scratch(ctx, &st)) return rc;
    float* c1[1] = {C};
    const float* a1[1] = {A};
    const float* b1[1] = {B};
    const float* s1[1] = {bias};
    const float* r1[1] = {residual};
    return gemm_dispatch(ctx, 1, c1, a1, b1, M, K, N, 0, 0, s1, act, r1, &st);
}

int lancius_hip_gemm_grouped_f32(lancius_hip_ctx* ctx, size_t count, float* const* C, const float* const* A,
                                 const float* const* B, size_t M, size_t K, size_t N, const float* const* bias,
                                 int act, const float* const* residual) {
    return gemm_dispatch(ctx, count, C, A, B, M, K, N, 0, 0, bias, act, residual);
}

int lancius_hip_gemm_ex_f32(lancius_hip_ctx* ctx, float* C, const float* A, const float* B, size_t M, size_t K,
                            size_t N, int trans_a, int trans_b, const float* bias, int act, const float* residual) {
    float* c1[1] = {C};
    const float* a1[1] = {A};
    const float* b1[1] = {B};
    const float* s1[1] = {bias};
    const float* r1[1] = {residual};
    return gemm_dispatch(ctx, 1, c1, a1, b1, M, K, N, trans_a, trans_b, s1, act, r1);
}

int lancius_hip_gemm_grouped_ex_f32(lancius_hip_ctx* ctx, size_t count, float* const* C, const float* const* A,
                                    const float* const* B, size_t M, size_t K, size_t N, int trans_a, int trans_b,
                                    const float* const* bias, int act, const float* const* residual) {
    return gemm_dispatch(ctx, count, C, A, B, M, K, N, trans_a, trans_b, bias, act, residual);
}

}  // extern "C"
