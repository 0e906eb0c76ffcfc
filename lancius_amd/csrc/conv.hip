// conv2d (NCHW input, OIHW weights) as an implicit GEMM on the gfx950 matrix
// cores, with bias and ReLU fused into the store.
//
// Semantics: bleeding/v11A1/src/math/lancius_kernels.c:28-60 (kernel_conv2d_fwd)
// and :140-173 (kernel_conv2d_relu_fwd): cross-correlation, zero padding by
// bounds test (:156-158), H_out = (H + 2 pad - K_h)/stride + 1 (:143-144),
// ReLU on store (:168).  The reference has no bias; the device adds bias[co]
// when one is given (NULL otherwise).
//
// GEMM view: Out[co][P] = sum_k W[co][k] * X[k][P] with k = (ci, kh, kw) and
// P = (n, ho, wo) running over every output pixel of the batch.  The OIHW
// weight tensor already is the row-major [C_out][C_in*K_h*K_w] A operand.  The
// B operand is never materialised: each k-tile of the im2col matrix is
// gathered from the NCHW input straight into LDS (zero outside the padded
// image), consecutive threads taking consecutive pixels so the gathers
// coalesce along W.  The MFMA tiling, double-buffered LDS and k-major layout
// are those of the GEMM kernel; the epilogue writes Out[n][co][ho][wo], where
// lanes 0..31 of a register cover 32 consecutive pixels of one channel.
#include "common.hpp"
#include "kernels.hpp"

namespace lancius {
namespace {

struct ConvParams {
    float* out;
    const float* in;
    const float* w;
    const float* bias;
    int N, C_in, H, W, C_out, KH, KW, stride, pad, Ho, Wo;
    int Kdim;          // C_in * KH * KW
    long long Ptotal;  // N * Ho * Wo
    int act;
    uint32_t tiles_m, tiles_n;
};

constexpr int kThreads = 256;

// KH_T/KW_T > 0 fixes the filter size at compile time (cheap k decomposition);
// 0 means runtime values.
template <int BM, int BN, int BK, int WGM, int WGN, int KH_T, int KW_T>
__global__ void __launch_bounds__(kThreads) conv2d_implicit_gemm(const ConvParams p) {
    constexpr int WM = BM / WGM, WN = BN / WGN;
    constexpr int TM = WM / 32, TN = WN / 32;
    constexpr int LDA = BM + 4;
    constexpr int LDB = BN + 4;
    __shared__ __attribute__((aligned(16))) float As[2][BK][LDA];
    __shared__ __attribute__((aligned(16))) float Bs[2][BK][LDB];

    const int KH = KH_T > 0 ? KH_T : p.KH;
    const int KW = KW_T > 0 ? KW_T : p.KW;
    const int KHW = KH * KW;
    const int H = p.H, W = p.W, Ho = p.Ho, Wo = p.Wo;
    const int HWo = Ho * Wo;
    const int Kdim = p.Kdim;
    const int C_out = p.C_out;

    const uint32_t ntiles = p.tiles_m * p.tiles_n;
    uint32_t tm_id, tn_id;
    grouped_tile(xcd_contiguous_id(blockIdx.x, ntiles), p.tiles_m, p.tiles_n, 2, tm_id, tn_id);
    const int m0 = (int)tm_id * BM;            // first output channel
    const long long P0 = (long long)tn_id * BN;  // first output pixel

    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const int wm = wave / WGN, wn = wave % WGN;
    const int lr = lane & 31, lk = lane >> 5;

    // The pixel this thread gathers for (fixed for the whole k loop).
    static_assert(kThreads % BN == 0 || BN % kThreads == 0, "pixel mapping");
    constexpr int B_ELEMS = BK * BN / kThreads;
    constexpr int K_STEP = kThreads / BN;  // k rows covered per pass
    static_assert(B_ELEMS * kThreads == BK * BN && K_STEP >= 1, "even B split");
    const int pp = tid % BN;
    const int kk0 = tid / BN;
    const long long P = P0 + pp;
    const bool p_valid = P < p.Ptotal;
    int n_img = 0, hi0 = 0, wi0 = 0;
    if (p_valid) {
        n_img = (int)(P / HWo);
        const int rem = (int)(P - (long long)n_img * HWo);
        const int ho = rem / Wo, wo = rem - (rem / Wo) * Wo;
        hi0 = ho * p.stride - p.pad;
        wi0 = wo * p.stride - p.pad;
    }
    const float* __restrict__ x_img = p.in + (size_t)n_img * p.C_in * H * W;
    const float* __restrict__ wgt = p.w;

    constexpr int A_ELEMS = BM * BK / kThreads;
    static_assert(A_ELEMS * kThreads == BM * BK, "even A split");
    float a_s[A_ELEMS];
    float b_s[B_ELEMS];

    auto load_tile = [&](int k0) {
#pragma unroll
        for (int i = 0; i < A_ELEMS; ++i) {
            const int idx = tid + i * kThreads;
            const int r = idx / BK, c = idx % BK;
            const int co = m0 + r, k = k0 + c;
            a_s[i] = (co < C_out && k < Kdim) ? wgt[(size_t)co * Kdim + k] : 0.0f;
        }
#pragma unroll
        for (int i = 0; i < B_ELEMS; ++i) {
            const int k = k0 + kk0 + i * K_STEP;
            float v = 0.0f;
            if (p_valid && k < Kdim) {
                const int ci = k / KHW;
                const int r = k - ci * KHW;
                const int kh = r / KW, kw = r - (r / KW) * KW;
                const int hi = hi0 + kh, wi = wi0 + kw;
                if (hi >= 0 && hi < H && wi >= 0 && wi < W) v = x_img[((size_t)ci * H + hi) * W + wi];
            }
            b_s[i] = v;
        }
    };
    auto store_tile = [&](int buf) {
#pragma unroll
        for (int i = 0; i < A_ELEMS; ++i) {
            const int idx = tid + i * kThreads;
            As[buf][idx % BK][idx / BK] = a_s[i];
        }
#pragma unroll
        for (int i = 0; i < B_ELEMS; ++i) Bs[buf][kk0 + i * K_STEP][pp] = b_s[i];
    };

    f32x16 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    const int ktiles = (Kdim + BK - 1) / BK;
    load_tile(0);
    store_tile(0);
    __syncthreads();
    for (int kt = 0; kt < ktiles; ++kt) {
        const int cur = kt & 1;
        const bool more = kt + 1 < ktiles;
        if (more) load_tile((kt + 1) * BK);
#pragma unroll
        for (int kp = 0; kp < BK / 2; ++kp) {
            float af[TM], bf[TN];
#pragma unroll
            for (int i = 0; i < TM; ++i) af[i] = As[cur][2 * kp + lk][wm * WM + i * 32 + lr];
#pragma unroll
            for (int j = 0; j < TN; ++j) bf[j] = Bs[cur][2 * kp + lk][wn * WN + j * 32 + lr];
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
        if (more) store_tile(cur ^ 1);
        __syncthreads();
    }

    // Epilogue: register r of lane l is channel row 8*(r/4)+4*(l/32)+r%4,
    // pixel column l%32 of its 32x32 sub-tile.
    const float* __restrict__ bias = p.bias;
    const int act = p.act;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
        const long long Pc = P0 + wn * WN + j * 32 + lr;
        if (Pc >= p.Ptotal) continue;
        const int n_o = (int)(Pc / HWo);
        const int pix = (int)(Pc - (long long)n_o * HWo);
        float* obase = p.out + (size_t)n_o * C_out * HWo + pix;
#pragma unroll
        for (int i = 0; i < TM; ++i) {
            const int cbase = m0 + wm * WM + i * 32 + 4 * lk;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int co = cbase + 8 * (r >> 2) + (r & 3);
                if (co < C_out) {
                    float v = acc[i][j][r] + (bias ? bias[co] : 0.0f);
                    obase[(size_t)co * HWo] = apply_act(v, act);
                }
            }
        }
    }
}

template <int BM, int BN, int KH_T, int KW_T>
int launch(lancius_hip_ctx* ctx, ConvParams& p) {
    p.tiles_m = (uint32_t)((p.C_out + BM - 1) / BM);
    p.tiles_n = (uint32_t)((p.Ptotal + BN - 1) / BN);
    const size_t grid = (size_t)p.tiles_m * p.tiles_n;
    LANCIUS_REQUIRE(grid < kMaxGridX, LANCIUS_HIP_ERR_SHAPE, "conv2d: too many tiles");
    constexpr int WGM = BM >= 128 ? 2 : 1;
    constexpr int WGN = 4 / WGM;
    hipLaunchKernelGGL((conv2d_implicit_gemm<BM, BN, 16, WGM, WGN, KH_T, KW_T>), dim3((unsigned)grid),
                       dim3(kThreads), 0, ctx->stream, p);
    return check_launch("conv2d_implicit_gemm");
}

}  // namespace
}  // namespace lancius

using namespace lancius;

extern "C" int lancius_hip_conv2d_f32(lancius_hip_ctx* ctx, float* out, const float* in, const float* w,
                                      const float* bias, size_t N, size_t C_in, size_t H, size_t W, size_t C_out,
                                      size_t K_h, size_t K_w, size_t stride, size_t pad, int act) {
    LANCIUS_REQUIRE(ctx && out && in && w, LANCIUS_HIP_ERR_NULL_PTR, "conv2d: NULL argument");
    LANCIUS_REQUIRE(N && C_in && H && W && C_out && K_h && K_w && stride, LANCIUS_HIP_ERR_SHAPE,
                    "conv2d: empty shape");
    LANCIUS_REQUIRE(H + 2 * pad >= K_h && W + 2 * pad >= K_w, LANCIUS_HIP_ERR_SHAPE,
                    "conv2d: spatial dimensions underflow");
    LANCIUS_REQUIRE(act == LANCIUS_HIP_ACT_NONE || act == LANCIUS_HIP_ACT_RELU, LANCIUS_HIP_ERR_UNSUPPORTED,
                    "conv2d: activation %d", act);
    LANCIUS_REQUIRE(C_in * K_h * K_w < (1u << 30) && H * W < (1u << 30) && C_out < (1u << 30) &&
                        N * C_in * H * W < ((size_t)1 << 40),
                    LANCIUS_HIP_ERR_SHAPE, "conv2d: shape too large");
    if (int rc = bind_device(ctx)) return rc;
    ConvParams p{};
    p.out = out;
    p.in = in;
    p.w = w;
    p.bias = bias;
    p.N = (int)N;
    p.C_in = (int)C_in;
    p.H = (int)H;
    p.W = (int)W;
    p.C_out = (int)C_out;
    p.KH = (int)K_h;
    p.KW = (int)K_w;
    p.stride = (int)stride;
    p.pad = (int)pad;
    p.Ho = (int)((H + 2 * pad - K_h) / stride + 1);
    p.Wo = (int)((W + 2 * pad - K_w) / stride + 1);
    p.Kdim = (int)(C_in * K_h * K_w);
    p.Ptotal = (long long)N * p.Ho * p.Wo;
    p.act = act;
    int rc;
    if (C_out > 64) {
        if (K_h == 3 && K_w == 3)
            rc = launch<128, 128, 3, 3>(ctx, p);
        else
            rc = launch<128, 128, 0, 0>(ctx, p);
    } else {
        if (K_h == 3 && K_w == 3)
            rc = launch<32, 128, 3, 3>(ctx, p);
        else
            rc = launch<32, 128, 0, 0>(ctx, p);
    }
    return rc ? rc : ok();
}
