// Two dense layers and a row softmax in one launch, for the small-batch MLP
// graphs (B/examples/train_mnist.c:149-158 builds x -> MATMUL -> +b -> RELU ->
// MATMUL -> +b -> SOFTMAX with 64 rows).  At that size every kernel of the
// unfused chain (split-K GEMM, its reduce, GEMM, reduce, softmax) is a few
// microseconds of work behind a fixed launch cost, so the chain is bound by
// its number of dependent launches.  See mlp2_fused for the design.
#include <math.h>

#include <algorithm>

#include "common.hpp"
#include "kernels.hpp"

namespace lancius {
namespace {

struct ChainParams {
    const float* x;   // [M][K1]
    const float* w1;  // [K1][N1]
    const float* b1;  // [N1] or null
    const float* w2;  // [N1][N2]
    const float* b2;  // [N2] or null
    float* out;       // [M][N2]: probabilities (softmax) or y
    int32_t* argmax;  // [M] or null
    float* ypart;     // [tiles_n][M][N2]: each column tile's share of y
    unsigned* counters;  // one arrival counter per row block, zero between launches
    int M, K1, N1, N2, act1, act2, softmax;
    int vec;  // K1 and N1 multiples of 4, x and W1 16-byte aligned: float4 loads
    int tiles_n;
};

// Workgroup (column tile t of 16 columns of h, row block b of 16 rows):
//  1. h[b, t] = act1(x[b] . W1[:, t] + b1[t]) over the whole K1: the x row
//     block and the W1 column slab are staged in LDS (in K chunks of kFKC),
//     the 4 waves take a quarter of each chunk's k-steps with
//     v_mfma_f32_16x16x4_f32 and add their accumulators through LDS in wave
//     order;
//  2. y_t = h[b, t] . W2[t rows, :], the tile's share of the second layer,
//     stored for the row block's reducer;
//  3. the workgroup that arrives last at row block b's counter adds the
//     tiles' shares in tile order, adds b2, applies act2, and runs each row's
//     softmax and first-maximum argmax (one thread per row).
// One hand-off between workgroups (through the point of coherence,
// kernels.hpp); every sum runs in a fixed order, so repeated calls give
// identical bits.
// Limits of the chain (the small-batch regime it is for; lancius_hip.h):
// rows, outputs, hidden values M * N1 and second-layer weights N1 * N2.
constexpr int kMaxRows = 64;
constexpr int kMaxOut = 64;
constexpr int kMaxH = 16384;
constexpr int kMaxW2 = 8192;
constexpr int kFR = 16;     // rows of h per workgroup
constexpr int kFC = 16;     // columns of h per workgroup
constexpr int kFKC = 1024;  // K staged per chunk
constexpr int kXP = kFKC + 4;  // x rows in LDS: lanes read rows r at k-steps (r*kXP + k) mod 64 distinct

__global__ void __launch_bounds__(256) mlp2_fused(const ChainParams p) {
    __shared__ __attribute__((aligned(16))) float Xs[kFR][kXP];    // x rows of the block, current K chunk
    __shared__ __attribute__((aligned(16))) float Wsl[kFKC][kFC];  // W1 columns of the tile, current K chunk
    __shared__ float red[4][kFR][kFC + 1];
    __shared__ float Hs[kFR][kFC + 1];
    __shared__ float W2s[kFC][64];
    __shared__ float Ys[kFR][64];
    __shared__ int s_flag;

    const int tn = (int)blockIdx.x % p.tiles_n, rb = (int)blockIdx.x / p.tiles_n;
    const int n0 = tn * kFC, m0 = rb * kFR;
    const int M = p.M, K1 = p.K1, N1 = p.N1, N2 = p.N2;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int li = lane & 15, lq = lane >> 4;

    // W2 rows of this tile, needed after phase 1: loaded first
    for (int i = tid; i < kFC * N2; i += 256) {
        const int k = i / N2, j = i % N2;
        W2s[k][j] = n0 + k < N1 ? p.w2[(size_t)(n0 + k) * N2 + j] : 0.0f;
    }

    f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int kc = 0; kc < K1; kc += kFKC) {
        const int kn = min(kFKC, K1 - kc);  // k of this chunk
        if (kc > 0) __syncthreads();        // the previous chunk's reads are done
        // x rows m0.. of the chunk (float4 along k) and W1 columns n0.. (one
        // float4 per k and quarter of the 16 columns): every load of the
        // chunk is issued before the first LDS store.
        constexpr int kPer = kFR * kFKC / 4 / 256;  // float4 of each operand per thread
        const int xq = (kn + 3) / 4;
        f32x4 xv[kPer], wv[kPer];
#pragma unroll
        for (int u = 0; u < kPer; ++u) {
            const int i = tid + 256 * u;
            const int r = i / xq, k = 4 * (i % xq);
            f32x4 v = f32x4{0.f, 0.f, 0.f, 0.f};
            if (i < kFR * xq && m0 + r < M) {
                const float* src = p.x + (size_t)(m0 + r) * K1 + kc + k;
                if (p.vec && k + 4 <= kn) {
                    v = *(const f32x4*)src;
                } else {
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        if (k + j < kn) v[j] = src[j];
                }
            }
            xv[u] = v;
            const int kw = i >> 2, c = 4 * (i & 3);
            f32x4 w = f32x4{0.f, 0.f, 0.f, 0.f};
            if (kw < kn) {
                const float* src = p.w1 + (size_t)(kc + kw) * N1 + n0 + c;
                if (p.vec && n0 + c + 4 <= N1) {
                    w = *(const f32x4*)src;
                } else {
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        if (n0 + c + j < N1) w[j] = src[j];
                }
            }
            wv[u] = w;
        }
#pragma unroll
        for (int u = 0; u < kPer; ++u) {
            const int i = tid + 256 * u;
            if (i < kFR * xq) {
                const int r = i / xq, k = 4 * (i % xq);
                Xs[r][k] = xv[u].x, Xs[r][k + 1] = xv[u].y, Xs[r][k + 2] = xv[u].z, Xs[r][k + 3] = xv[u].w;
            }
            if ((i >> 2) < kn) *(f32x4*)&Wsl[i >> 2][4 * (i & 3)] = wv[u];
        }
        __syncthreads();
        // wave w takes k-steps w, w + 4, ...; lane l holds A[row l%16][k + l/16]
        // and B[k + l/16][column l%16]; eight steps' LDS reads are issued
        // before their MFMAs
        const int steps = (kn + 3) / 4;
        for (int s0 = wave; s0 < steps; s0 += 32) {
            float a[8], b[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int k = 4 * (s0 + 4 * u) + lq;
                a[u] = k < kn ? Xs[li][k] : 0.0f;
                b[u] = k < kn ? Wsl[k][li] : 0.0f;
            }
#pragma unroll
            for (int u = 0; u < 8; ++u) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[u], b[u], acc, 0, 0, 0);
        }
    }
    // register r of lane l: row 4(l/16) + r, column l%16
#pragma unroll
    for (int r = 0; r < 4; ++r) red[wave][4 * lq + r][li] = acc[r];
    __syncthreads();
    {
        const int r = tid >> 4, c = tid & 15;  // 256 threads = 16 x 16
        const float v = ((red[0][r][c] + red[1][r][c]) + red[2][r][c]) + red[3][r][c];
        float h = 0.0f;
        if (m0 + r < M && n0 + c < N1) h = apply_act(v + (p.b1 ? p.b1[n0 + c] : 0.0f), p.act1);
        Hs[r][c] = h;  // rows past M and columns past N1 hold 0
    }
    __syncthreads();
    // this tile's share of y for the block's rows
    const size_t MN2 = (size_t)M * N2;
    const __amdgpu_buffer_rsrc_t ypart = coherent_buffer(p.ypart, (size_t)p.tiles_n * MN2 * sizeof(float));
    for (int i = tid; i < kFR * N2; i += 256) {
        const int r = i / N2, j = i % N2;
        if (m0 + r >= M) continue;
        float a = 0.0f;
#pragma unroll
        for (int k = 0; k < kFC; ++k) a += Hs[r][k] * W2s[k][j];
        store_coherent(ypart, (int)(((size_t)tn * MN2 + (size_t)(m0 + r) * N2 + j) * sizeof(float)), a);
    }
    if (!arrive_last(p.counters + rb, (unsigned)p.tiles_n, &s_flag)) return;
    reset_arrival(p.counters + rb);

    // the block's rows: y = sum of the tiles' shares in tile order + b2
    {
        constexpr int kChunk = 16;
        for (int i = tid; i < kFR * N2; i += 256) {
            const int r = i / N2, j = i % N2;
            if (m0 + r >= M) continue;
            const int off = (int)(((size_t)(m0 + r) * N2 + j) * sizeof(float));
            float y = 0.0f;
            for (int t0 = 0; t0 < p.tiles_n; t0 += kChunk) {
                float t[kChunk];
#pragma unroll
                for (int c = 0; c < kChunk; ++c)
                    t[c] = t0 + c < p.tiles_n
                               ? load_coherent(ypart, off + (int)((size_t)(t0 + c) * MN2 * sizeof(float)))
                               : 0.0f;
#pragma unroll
                for (int c = 0; c < kChunk; ++c)
                    if (t0 + c < p.tiles_n) y = (t0 + c == 0) ? t[c] : y + t[c];
            }
            Ys[r][j] = apply_act(y + (p.b2 ? p.b2[j] : 0.0f), p.act2);
        }
    }
    __syncthreads();
    // One thread per row: the reference's serial loops, max, exp, sum,
    // divide (lancius_scheduler.c:284-294), then the first maximum scanning
    // with '>' from -1e9 (B/examples/train_mnist.c:206-209).
    if (tid < kFR && m0 + tid < M) {
        const int r = m0 + tid;
        const float* yr = Ys[tid];
        float* o = p.out + (size_t)r * N2;
        if (!p.softmax) {
            for (int j = 0; j < N2; ++j) o[j] = yr[j];
        } else {
            float m = yr[0];
            for (int j = 1; j < N2; ++j) m = fmaxf(m, yr[j]);
            float sum = 0.0f;
            for (int j = 0; j < N2; ++j) sum += expf(yr[j] - m);
            float best = -1e9f;
            int bi = 0;
            for (int j = 0; j < N2; ++j) {
                const float pv = expf(yr[j] - m) / sum;
                o[j] = pv;
                if (pv > best) {
                    best = pv;
                    bi = j;
                }
            }
            if (p.argmax) p.argmax[r] = bi;
        }
    }
}

}  // namespace
}  // namespace lancius

using namespace lancius;

extern "C" int lancius_hip_mlp2_f32(lancius_hip_ctx* ctx, float* out, int32_t* argmax, const float* x,
                                    const float* w1, const float* b1, int act1, const float* w2, const float* b2,
                                    size_t M, size_t K1, size_t N1, size_t N2, int softmax) {
    return lancius_hip_mlp2_ex_f32(ctx, out, argmax, x, w1, b1, act1, w2, b2, LANCIUS_HIP_ACT_NONE, M, K1, N1, N2,
                                   softmax);
}

extern "C" int lancius_hip_mlp2_ex_f32(lancius_hip_ctx* ctx, float* out, int32_t* argmax, const float* x,
                                       const float* w1, const float* b1, int act1, const float* w2, const float* b2,
                                       int act2, size_t M, size_t K1, size_t N1, size_t N2, int softmax) {
    LANCIUS_REQUIRE(ctx && out && x && w1 && w2, LANCIUS_HIP_ERR_NULL_PTR, "mlp2: NULL argument");
    LANCIUS_REQUIRE(M >= 1 && M <= (size_t)kMaxRows && N2 >= 1 && N2 <= (size_t)kMaxOut && N1 >= 1 && K1 >= 1 &&
                        M * N1 <= (size_t)kMaxH && N1 * N2 <= (size_t)kMaxW2 && K1 < (1u << 30),
                    LANCIUS_HIP_ERR_SHAPE, "mlp2: M=%zu K1=%zu N1=%zu N2=%zu outside the fused chain's limits", M, K1,
                    N1, N2);
    LANCIUS_REQUIRE(act1 >= LANCIUS_HIP_ACT_NONE && act1 <= LANCIUS_HIP_ACT_TANH && act2 >= LANCIUS_HIP_ACT_NONE &&
                        act2 <= LANCIUS_HIP_ACT_TANH,
                    LANCIUS_HIP_ERR_UNSUPPORTED, "mlp2: activations %d, %d", act1, act2);
    if (int rc = bind_device(ctx)) return rc;
    ChainParams p{};
    p.x = x;
    p.w1 = w1;
    p.b1 = b1;
    p.w2 = w2;
    p.b2 = b2;
    p.out = out;
    p.argmax = softmax ? argmax : nullptr;
    p.M = (int)M;
    p.K1 = (int)K1;
    p.N1 = (int)N1;
    p.N2 = (int)N2;
    p.act1 = act1;
    p.act2 = act2;
    p.softmax = softmax ? 1 : 0;
    p.vec = K1 % 4 == 0 && N1 % 4 == 0 && ((uintptr_t)x & 15u) == 0 && ((uintptr_t)w1 & 15u) == 0;
    p.tiles_n = (int)((N1 + kFC - 1) / kFC);
    const size_t row_blocks = (M + kFR - 1) / kFR;
    void* ws = nullptr;
    if (int rc = workspace(ctx, (size_t)p.tiles_n * M * N2 * sizeof(float), &ws)) return rc;
    p.ypart = (float*)ws;
    if (int rc = counters(ctx, row_blocks, &p.counters)) return rc;
    hipLaunchKernelGGL(mlp2_fused, dim3((unsigned)(p.tiles_n * row_blocks)), dim3(256), 0, ctx->stream, p);
    if (int rc = check_launch("mlp2_fused")) return rc;
    return ok();
}
