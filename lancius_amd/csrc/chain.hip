// Two dense layers and a row softmax in two launches, for the small-batch MLP
// graphs (B/examples/train_mnist.c:149-158 builds x -> MATMUL -> +b -> RELU ->
// MATMUL -> +b -> SOFTMAX with 64 rows).  At that size every kernel of the
// unfused chain (split-K GEMM, its reduce, GEMM, reduce, softmax) is a few
// microseconds of work behind a fixed ~9 us launch cost, so the chain is
// bound by its number of dependent launches.
//  * mlp2_partials: workgroup (column tile t, K range s) computes the
//    64 x 64 tile of x . W1 over its K range with 32x32x2 MFMAs and stores
//    the partial.
//  * mlp2_tail (one workgroup per row): adds the row's partials in K-range
//    order, applies b1 and the activation into LDS, computes y = h . W2 + b2
//    (W2 staged in LDS), then the row's softmax with the first-maximum
//    argmax, exactly as softmax_rows does.
// The kernel boundary orders the two phases.  (Joining them in one launch
// with "last workgroup continues" arrival counters needs device-scope
// release/acquire fences, which write back and invalidate the XCD's L2 on
// this part: measured 91 us against 26 us for the unfused chain.)
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
    float* part;      // [splits][M][N1]
    int M, K1, N1, N2, act1, act2, softmax;
    int splits, kchunk, tiles_n;
};

constexpr int kT = 64;   // phase-1 tile: up to 64 rows x 64 columns
constexpr int kK = 16;   // k-tile
constexpr int kMaxH = 16384;  // M * N1 floats of h in LDS
constexpr int kMaxW2 = 8192;  // N1 * N2 floats of W2 in LDS

__global__ void __launch_bounds__(256) mlp2_partials(const ChainParams p) {
    __shared__ __attribute__((aligned(16))) float As[2][kK][kT + 4];
    __shared__ __attribute__((aligned(16))) float Bs[2][kK][kT + 4];

    const int tn = (int)blockIdx.x % p.tiles_n, sp = (int)blockIdx.x / p.tiles_n;
    const int n0 = tn * kT;
    const int M = p.M, K1 = p.K1, N1 = p.N1;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int wm = wave >> 1, wn = wave & 1, lr = lane & 31, lk = lane >> 5;
    const int kb = sp * p.kchunk, ke = min(K1, kb + p.kchunk);

    // staging: thread -> 4 consecutive k of row tid/4 (A), 4 consecutive
    // columns of k-row tid/16 (B); bounds-checked scalar loads.
    float ar[4], br[4];
    auto load = [&](int k0) {
        const int r = tid >> 2, ka = k0 + 4 * (tid & 3);
#pragma unroll
        for (int j = 0; j < 4; ++j) ar[j] = (r < M && ka + j < ke) ? p.x[(size_t)r * K1 + ka + j] : 0.0f;
        const int kr = k0 + (tid >> 4), c = n0 + 4 * (tid & 15);
#pragma unroll
        for (int j = 0; j < 4; ++j) br[j] = (kr < ke && c + j < N1) ? p.w1[(size_t)kr * N1 + c + j] : 0.0f;
    };
    auto store = [&](int buf) {
        const int r = tid >> 2, ka = 4 * (tid & 3);
#pragma unroll
        for (int j = 0; j < 4; ++j) As[buf][ka + j][r] = ar[j];
        const int kr = tid >> 4, c = 4 * (tid & 15);
#pragma unroll
        for (int j = 0; j < 4; ++j) Bs[buf][kr][c + j] = br[j];
    };
    f32x16 acc;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = 0.0f;
    const int nk = (ke - kb + kK - 1) / kK;
    if (nk > 0) {
        load(kb);
        store(0);
    }
    __syncthreads();
    for (int t = 0; t < nk; ++t) {
        const int cur = t & 1;
        const bool more = t + 1 < nk;
        if (more) load(kb + (t + 1) * kK);
#pragma unroll
        for (int kp = 0; kp < kK / 2; ++kp) {
            const float a = As[cur][2 * kp + lk][wm * 32 + lr];
            const float b = Bs[cur][2 * kp + lk][wn * 32 + lr];
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, acc, 0, 0, 0);
        }
        if (more) store(cur ^ 1);
        __syncthreads();
    }
    // register r of lane l: row 8(r/4) + 4(l/32) + r%4, column l%32 of the wave's 32x32 block
    float* dst = p.part + (size_t)sp * M * N1;
    const int col = n0 + wn * 32 + lr;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int row = wm * 32 + 8 * (r >> 2) + 4 * lk + (r & 3);
        if (row < M && col < N1) dst[(size_t)row * N1 + col] = acc[r];
    }
}

constexpr int kMaxSplits = 8;

// One workgroup per row r: h[r] = act(sum of the K-range partials in order
// + b1) in LDS, y[r] = h[r] . W2 + b2 with W2 staged in LDS (four k-quarters
// per output column added in order), then the row's softmax and argmax.
__global__ void __launch_bounds__(256) mlp2_tail(const ChainParams p) {
    __shared__ float Hs[kMaxH];
    __shared__ float Ws[kMaxW2];
    __shared__ float red[4][kT];
    const int r = (int)blockIdx.x;
    const int M = p.M, N1 = p.N1, N2 = p.N2;
    const int tid = threadIdx.x, lane = tid & 63, q = tid >> 6;

    for (int k = tid; k < N1; k += 256) {
        float t[kMaxSplits];
#pragma unroll
        for (int s = 0; s < kMaxSplits; ++s) t[s] = s < p.splits ? p.part[((size_t)s * M + r) * N1 + k] : 0.0f;
        float v = 0.0f;
#pragma unroll
        for (int s = 0; s < kMaxSplits; ++s) v += t[s];
        if (p.b1) v += p.b1[k];
        Hs[k] = apply_act(v, p.act1);
    }
    for (int i = tid; i < N1 * N2; i += 256) Ws[i] = p.w2[i];
    __syncthreads();
    const int kq = (N1 + 3) / 4, k0 = q * kq, k1 = min(N1, k0 + kq);
    if (lane < N2) {
        float a0 = 0.0f, a1 = 0.0f;
        int k = k0;
        for (; k + 1 < k1; k += 2) {
            a0 += Hs[k] * Ws[k * N2 + lane];
            a1 += Hs[k + 1] * Ws[(k + 1) * N2 + lane];
        }
        if (k < k1) a0 += Hs[k] * Ws[k * N2 + lane];
        red[q][lane] = a0 + a1;
    }
    __syncthreads();
    if (q != 0) return;
    float v = -INFINITY;
    if (lane < N2) v = apply_act(((red[0][lane] + red[1][lane]) + (red[2][lane] + red[3][lane])) + (p.b2 ? p.b2[lane] : 0.0f), p.act2);
    float* o = p.out + (size_t)r * N2;
    if (!p.softmax) {
        if (lane < N2) o[lane] = v;
        return;
    }
    float m = v;
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
    const float e = lane < N2 ? expf(v - m) : 0.0f;
    float sum = e;
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) sum += __shfl_xor(sum, off);
    const float pv = e / sum;
    if (lane < N2) o[lane] = pv;
    if (p.argmax) {
        // first index of the largest probability, scanning with '>' from -1e9
        float best = lane < N2 && pv > -1e9f ? pv : -1e9f;
        int bi = lane < N2 && pv > -1e9f ? lane : 0x7fffffff;
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) {
            const float ob = __shfl_xor(best, off);
            const int oi = __shfl_xor(bi, off);
            if (ob > best || (ob == best && oi < bi)) {
                best = ob;
                bi = oi;
            }
        }
        if (lane == 0) p.argmax[r] = bi == 0x7fffffff ? 0 : bi;
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
    LANCIUS_REQUIRE(M >= 1 && M <= (size_t)kT && N2 >= 1 && N2 <= (size_t)kT && N1 >= 1 && K1 >= 1 &&
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
    p.tiles_n = (int)((N1 + kT - 1) / kT);
    // K ranges of whole k-tiles, about 128 deep, at most 8: the tail
    // workgroup reads splits * M * N1 partials, the first launch wants
    // enough workgroups to finish quickly.
    size_t splits = std::max<size_t>(1, std::min<size_t>(kMaxSplits, (K1 + 127) / 128));
    const size_t kchunk = ((K1 + splits - 1) / splits + kK - 1) / kK * kK;
    splits = (K1 + kchunk - 1) / kchunk;
    p.splits = (int)splits;
    p.kchunk = (int)kchunk;
    void* ws = nullptr;
    if (int rc = workspace(ctx, splits * M * N1 * sizeof(float), &ws)) return rc;
    p.part = (float*)ws;
    hipLaunchKernelGGL(mlp2_partials, dim3((unsigned)(p.tiles_n * splits)), dim3(256), 0, ctx->stream, p);
    if (int rc = check_launch("mlp2_partials")) return rc;
    hipLaunchKernelGGL(mlp2_tail, dim3((unsigned)M), dim3(256), 0, ctx->stream, p);
    if (int rc = check_launch("mlp2_tail")) return rc;
    return ok();
}
