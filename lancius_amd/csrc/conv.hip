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
// coalesce along W.  The MFMA tiling, double-buffered LDS and LDS layouts
// are those of the GEMM kernel; the epilogue writes Out[n][co][ho][wo], where
// lanes 0..31 of a register cover 32 consecutive pixels of one channel.
#include <algorithm>
#include <atomic>

#include "common.hpp"
#include "kernels.hpp"

namespace lancius {
namespace {

struct ConvParams {
    float* out;
    const float* in;
    const float* w;
    const float* wt;   // weights re-laid per output channel: wt[(co*KH*KW + tap)*C_in + ci] (CI_INNER path)
    const float* bias;
    int N, C_in, H, W, C_out, KH, KW, stride, pad, Ho, Wo;
    int Kdim;          // C_in * KH * KW
    long long Ptotal;  // N * Ho * Wo
    int act;
    uint32_t tiles_m, tiles_n;
    // conv2d_direct's split of the tiles: workgroups [0, sk_dp) take whole
    // tiles [0, sk_dp); sk_wgs more share the rest by (tile, k-tile) units
    int sk_dp, sk_wgs;
    float* sk_part;       // 2 * sk_wgs slots of one tile's sums
    unsigned* sk_ctr;     // one arrival counter per shared tile, zero between launches
    // weights the launch lays out in the workspace first: 0 none (wt or w
    // ready), 1 the forward per-channel layout of w, 2 dgrad's flipped
    // weights of w_src (the conv being differentiated has C_in and C_out
    // swapped against this one)
    int prep;
    const float* w_src;
};

constexpr int kThreads = 256;

// KH_T/KW_T > 0 fixes the filter size at compile time (cheap k decomposition);
// 0 means runtime values.
template <int BM, int BN, int BK, int WGM, int WGN, int KH_T, int KW_T, bool CI_INNER>
__global__ void __launch_bounds__(kThreads) conv2d_implicit_gemm(const ConvParams p) {
    constexpr int WM = BM / WGM, WN = BN / WGN;
    constexpr int TM = WM / 32, TN = WN / 32;
    constexpr int LDA = BM + 4;
    constexpr int LDB = BN + 4;
    // CI_INNER stages the filter tile m-major (Am[co][k], pitch BK+4: 16
    // consecutive rows on distinct 16-byte bank groups) and lane half h of
    // every MFMA takes k in [h*BK/2, (h+1)*BK/2), so a lane reads its A
    // operands for a whole k-tile with BK/8 16-byte reads; B reads the
    // matching rows.  Otherwise the filter tile is k-major (As[k][co]).
    constexpr int LDK = BK + 4;
    constexpr int A_STAGE = CI_INNER ? BM * LDK : BK * LDA;
    static_assert(!CI_INNER || BK % 8 == 0, "k halves of whole float4");
    __shared__ __attribute__((aligned(16))) float smem[2 * A_STAGE + 2 * BK * LDB];
    float(*As)[BK][LDA] = reinterpret_cast<float(*)[BK][LDA]>(smem);
    float(*Am)[BM][LDK] = reinterpret_cast<float(*)[BM][LDK]>(smem);
    float(*Bs)[BK][LDB] = reinterpret_cast<float(*)[BK][LDB]>(smem + 2 * A_STAGE);

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
    constexpr int A4 = BM * BK / 4;                        // float4 of one A tile
    constexpr int A_VEC = (A4 + kThreads - 1) / kThreads;  // float4 per thread (CI_INNER)
    float a_s[CI_INNER ? 1 : A_ELEMS];
    f32x4 a_v[A_VEC];
    float b_s[B_ELEMS];

    // CI_INNER: the reduction runs over (kh, kw, ci) with ci innermost, so a
    // k-tile is BK channels of one filter tap: one bounds test per tile and
    // channel addresses base + ci*H*W.  Otherwise k = (ci, kh, kw) as stored.
    const int ctiles = p.C_in / BK;
    const size_t HW = (size_t)H * W;
    auto load_tile = [&](int kt) {
        if constexpr (CI_INNER) {
            const int tap = kt / ctiles;
            const int ci0 = (kt - tap * ctiles) * BK;
            const int kh = tap / KW, kw = tap - (tap / KW) * KW;
            // A tile straight from the per-channel weights: rows co, float4
            // along ci.  Rows past C_out re-read the last row (they only
            // reach output channels that are never stored); threads past
            // the tile re-read its last float4 and store nothing.
            const float* wrow = p.wt + (size_t)tap * p.C_in + ci0;
#pragma unroll
            for (int i = 0; i < A_VEC; ++i) {
                const int idx = min(tid + i * kThreads, A4 - 1);
                const int r = idx / (BK / 4), kq = idx % (BK / 4);
                const int co = min(m0 + r, C_out - 1);
                a_v[i] = *(const f32x4*)(wrow + (size_t)co * KHW * p.C_in + 4 * kq);
            }
            const int hi = hi0 + kh, wi = wi0 + kw;
            const bool inside = p_valid && hi >= 0 && hi < H && wi >= 0 && wi < W;
            const float* src = x_img + (inside ? (size_t)hi * W + wi : 0) + (size_t)(ci0 + kk0) * HW;
#pragma unroll
            for (int i = 0; i < B_ELEMS; ++i) b_s[i] = inside ? src[(size_t)(i * K_STEP) * HW] : 0.0f;
        } else {
            const int k0 = kt * BK;
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
        }
    };
    auto store_tile = [&](int buf) {
        if constexpr (CI_INNER) {
#pragma unroll
            for (int i = 0; i < A_VEC; ++i) {
                const int idx = tid + i * kThreads;
                if (idx < A4) *(f32x4*)&Am[buf][idx / (BK / 4)][4 * (idx % (BK / 4))] = a_v[i];
            }
        } else {
#pragma unroll
            for (int i = 0; i < A_ELEMS; ++i) {
                const int idx = tid + i * kThreads;
                As[buf][idx % BK][idx / BK] = a_s[i];
            }
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

    const int ktiles = CI_INNER ? KHW * ctiles : (Kdim + BK - 1) / BK;
    load_tile(0);
    store_tile(0);
    __syncthreads();
    for (int kt = 0; kt < ktiles; ++kt) {
        const int cur = kt & 1;
        const bool more = kt + 1 < ktiles;
        if (more) load_tile(kt + 1);
        if constexpr (CI_INNER) {
            // lane half lk: k = lk*KH + kp
            constexpr int KH2 = BK / 2;
            f32x4 av[TM][KH2 / 4];
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int h = 0; h < KH2 / 4; ++h) av[i][h] = *(const f32x4*)&Am[cur][wm * WM + i * 32 + lr][lk * KH2 + 4 * h];
#pragma unroll
            for (int kp = 0; kp < KH2; ++kp) {
                float bf[TN];
#pragma unroll
                for (int j = 0; j < TN; ++j) bf[j] = Bs[cur][lk * KH2 + kp][wn * WN + j * 32 + lr];
#pragma unroll
                for (int i = 0; i < TM; ++i)
#pragma unroll
                    for (int j = 0; j < TN; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[i][kp / 4][kp % 4], bf[j], acc[i][j], 0, 0, 0);
            }
            if (more) store_tile(cur ^ 1);
            __syncthreads();
            continue;
        }
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
    // pixel column l%32 of its 32x32 sub-tile.  The tile's bias goes through
    // LDS (free after the loop's last barrier), four values per read: a bias
    // load from global memory issued after a store would wait for that store,
    // since a wave's loads and stores complete in order.  The activation is
    // chosen once per launch.
    if (threadIdx.x < BM) smem[threadIdx.x] = p.bias && m0 + (int)threadIdx.x < C_out ? p.bias[m0 + threadIdx.x] : 0.0f;
    __syncthreads();
    with_act(p.act, [&](auto act_c) {
        constexpr int ACT = decltype(act_c)::value;
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const long long Pc = P0 + wn * WN + j * 32 + lr;
            if (Pc >= p.Ptotal) continue;
            const int n_o = (int)(Pc / HWo);
            const int pix = (int)(Pc - (long long)n_o * HWo);
            float* obase = p.out + (size_t)n_o * C_out * HWo + pix;
#pragma unroll
            for (int i = 0; i < TM; ++i) {
                const int cl = wm * WM + i * 32 + 4 * lk;  // the lane's first channel row in the tile
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const f32x4 b4 = *(const f32x4*)&smem[cl + 8 * q];
                    const float bq[4] = {b4.x, b4.y, b4.z, b4.w};
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const int co = m0 + cl + 8 * q + e;
                        if (co < C_out) obase[(size_t)co * HWo] = act_fixed<ACT>(acc[i][j][4 * q + e] + bq[e]);
                    }
                }
            }
        }
    });
}

// The per-channel path (C_in % 16 == 0, weights re-laid as wt) with both
// operand tiles loaded straight from global memory into LDS (buffer loads
// with LDS destination, gfx950), as the GEMM's direct kernel: no register
// staging, the next k-tile's loads issued ahead of the current one's MFMAs.
// BM (64 or 128) output channels x BN pixels per workgroup, 4 waves of
// BM/2 x BN/2, k-tiles of 16 channels of one filter tap.
//  * A: rows co of wt (16 floats of the tap's channel run), 16-byte loads,
//    m-major in LDS with chunk c of row r at c ^ ((r >> 2) & 3).
//  * B: the im2col tile, k-major: one wave instruction fills 64 pixels of
//    one k-row with 4-byte loads.  A lane's pixel is fixed, so per filter tap
//    it computes one base offset; a tap outside the (padded) image, a pixel
//    past the batch and every load of a k-tile past the end use an offset
//    past the input's end and read 0.
// Requires the input and wt below 2 GiB.
template <int BM, int BN, int KH_T, int KW_T>
__global__ void __launch_bounds__(kThreads, 2) conv2d_direct(const ConvParams p) {
    constexpr int BK = 16, WM = BM / 2, WN = BN / 2, TM = WM / 32, TN = WN / 32;
    constexpr int A_INSTR = BM * BK / 4 / 256;  // 16-byte instructions per wave per k-tile
    constexpr int B_INSTR = BK * BN / 256;      // 4-byte instructions per wave per k-tile
    typedef __attribute__((address_space(3))) void lds_void;
    __shared__ __attribute__((aligned(16))) float As0[BM * BK];
    __shared__ __attribute__((aligned(16))) float As1[BM * BK];
    __shared__ __attribute__((aligned(16))) float Bs0[BK * BN];
    __shared__ __attribute__((aligned(16))) float Bs1[BK * BN];
    __shared__ int s_flag;
    __shared__ __attribute__((aligned(16))) float s_bias[BM];

    const int KH = KH_T > 0 ? KH_T : p.KH;
    const int KW = KW_T > 0 ? KW_T : p.KW;
    const int KHW = KH * KW;
    const int H = p.H, W = p.W, Ho = p.Ho, Wo = p.Wo;
    const int HWo = Ho * Wo;
    const int C_in = p.C_in, C_out = p.C_out;
    const unsigned HW4 = (unsigned)(H * W) * 4u;
    const uint32_t ntiles = p.tiles_m * p.tiles_n;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    const int lr = lane & 31, lk = lane >> 5;

    const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(p.in), 0, (int)((size_t)p.N * C_in * H * W * sizeof(float)), kBufferRsrcWord3);
    const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(p.wt), 0, (int)((size_t)C_out * KHW * C_in * sizeof(float)), kBufferRsrcWord3);
    constexpr unsigned kOut = 0x7ffffff0u;  // past the end of either operand: the load returns 0

    // Per-tile lane state (setup): B instruction j of wave w fills k-row
    // ((4j + w) * 64) / BN, pixels ((4j + w) * 64) % BN + lane, so a lane's
    // pixel is the same for every j; A instruction i of wave w fills chunks
    // (A_INSTR * w + i) * 64 + lane.
    const int b_pix = BN == 64 ? lane : (wave & 1) * 64 + lane;
    int a_c[A_INSTR];
#pragma unroll
    for (int i = 0; i < A_INSTR; ++i) {
        const int q = (A_INSTR * wave + i) * 64 + lane;
        a_c[i] = (q & 3) ^ (((q >> 2) >> 2) & 3);
    }
    int m0 = 0, hi0 = 0, wi0 = 0, a_row[A_INSTR];
    long long P0 = 0;
    bool p_valid = false;
    unsigned img_base = 0;
    auto setup = [&](uint32_t t) {
        uint32_t tm_id, tn_id;
        grouped_tile(t, p.tiles_m, p.tiles_n, 2, tm_id, tn_id);
        m0 = (int)tm_id * BM;
        P0 = (long long)tn_id * BN;
        const long long P = P0 + b_pix;
        p_valid = P < p.Ptotal;
        int n_img = 0;
        hi0 = wi0 = 0;
        if (p_valid) {
            n_img = (int)(P / HWo);
            const int rem = (int)(P - (long long)n_img * HWo);
            const int ho = rem / Wo, wo = rem - (rem / Wo) * Wo;
            hi0 = ho * p.stride - p.pad;
            wi0 = wo * p.stride - p.pad;
        }
        img_base = (unsigned)n_img * (unsigned)C_in * HW4;
#pragma unroll
        for (int i = 0; i < A_INSTR; ++i) a_row[i] = min(m0 + (((A_INSTR * wave + i) * 64 + lane) >> 2), C_out - 1);
    };
    const int ctiles = C_in / BK;
    const int ktiles = KHW * ctiles;
    auto load_tile = [&](float* As, float* Bs, int kt, int kend) {
        const bool live = kt < kend;
        const int tap = live ? kt / ctiles : 0;
        const int ci0 = (kt - tap * ctiles) * BK;
        const int kh = tap / KW, kw = tap - (tap / KW) * KW;
#pragma unroll
        for (int i = 0; i < A_INSTR; ++i) {
            const unsigned ao =
                live ? (unsigned)(((a_row[i] * KHW + tap) * C_in + ci0 + 4 * a_c[i]) * (int)sizeof(float)) : kOut;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rw, (lds_void*)(As + (A_INSTR * wave + i) * 256), 16, (int)ao, 0,
                                                     0, 0);
        }
        const int hi = hi0 + kh, wi = wi0 + kw;
        const bool inside = live & p_valid & ((unsigned)hi < (unsigned)H) & ((unsigned)wi < (unsigned)W);
        const unsigned pix = img_base + (unsigned)(hi * W + wi) * 4u + (unsigned)ci0 * HW4;
#pragma unroll
        for (int j = 0; j < B_INSTR; ++j) {
            const int row = ((4 * j + wave) * 64) / BN;
            const unsigned bo = (unsigned)pick(inside, (int)(pix + (unsigned)row * HW4), (int)kOut);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (lds_void*)(Bs + (4 * j + wave) * 64), 4, (int)bo, 0, 0, 0);
        }
    };

    f32x16 acc[TM][TN];
    int a_rd[TM][2];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int row = wm * WM + i * 32 + lr, c = 2 * lk + h;
            a_rd[i][h] = row * BK + 4 * (c ^ ((row >> 2) & 3));
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
            for (int j = 0; j < TN; ++j) bf[j] = Bs[(8 * lk + kp) * BN + wn * WN + j * 32 + lr];
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[i][kp / 4][kp % 4], bf[j], acc[i][j], 0, 0, 0);
        }
        // the k-tile's loads one after each of the first MFMAs
#pragma unroll
        for (int i = 0; i < A_INSTR + B_INSTR; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
        }
        __builtin_amdgcn_sched_group_barrier(0x008, TM * TN * 8 - A_INSTR - B_INSTR, 0);
        __builtin_amdgcn_sched_barrier(0);
    };
    // acc = the tile's sums over k-tiles [kbeg, kend), in pairs (a pair's
    // second tile past kend loads zeros)
    auto run = [&](int kbeg, int kend) {
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
        const int pairs = (kend - kbeg + 1) / 2;
        load_tile(As0, Bs0, kbeg, kend);
        __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
        __syncthreads();
        for (int pr = 0; pr < pairs; ++pr) {
            load_tile(As1, Bs1, kbeg + 2 * pr + 1, kend);
            compute(As0, Bs0);
            __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
            __syncthreads();
            load_tile(As0, Bs0, kbeg + 2 * pr + 2, kend);  // past the end: zeros
            compute(As1, Bs1);
            __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
            __syncthreads();
        }
    };

    // register r of lane l: channel row 8(r/4) + 4(l/32) + r%4, pixel l%32
    // The tile's bias goes through LDS, read four values at a time: a
    // wave's loads and stores complete in order, so a bias load from global
    // memory issued after a store waits for that store (one such load per
    // element made the epilogue a chain of store round trips).  The
    // activation is chosen once per launch.
    auto store = [&]() {
        if (tid < BM) s_bias[tid] = p.bias && m0 + tid < C_out ? p.bias[m0 + tid] : 0.0f;
        __syncthreads();
        with_act(p.act, [&](auto act_c) {
            constexpr int ACT = decltype(act_c)::value;
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                const long long Pc = P0 + wn * WN + j * 32 + lr;
                if (Pc >= p.Ptotal) continue;
                const int n_o = (int)(Pc / HWo);
                const int pix = (int)(Pc - (long long)n_o * HWo);
                float* obase = p.out + (size_t)n_o * C_out * HWo + pix;
#pragma unroll
                for (int i = 0; i < TM; ++i) {
                    const int cl = wm * WM + i * 32 + 4 * lk;  // the lane's first channel row in the tile
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const f32x4 b4 = *(const f32x4*)&s_bias[cl + 8 * q];
                        const float bq[4] = {b4.x, b4.y, b4.z, b4.w};
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const int co = m0 + cl + 8 * q + e;
                            if (co < C_out) obase[(size_t)co * HWo] = act_fixed<ACT>(acc[i][j][4 * q + e] + bq[e]);
                        }
                    }
                }
            }
        });
    };

    // Whole tiles: workgroups [0, sk_dp) take tiles [0, sk_dp) (each XCD a
    // contiguous run).
    // Stream-K: workgroup s of sk_wgs takes the s-th equal share of the
    // remaining tiles' (tile, k-tile) units, in tile order.  A tile split
    // between workgroups is finished by the one that arrives last at its
    // counter: each share's sums go to its workgroup's slot (2s for the
    // first tile of its range, 2s + 1 for the last) through the point of
    // coherence, and the last re-reads all shares, its own included, and
    // adds them in k order, so the sum does not depend on which came last;
    // then it runs the epilogue.  Every workgroup of the launch is resident
    // at once (the host sizes the grid to the CUs), and none waits for
    // another.  Unit counts are 32-bit (the host checks U * sk_wgs).
    // One loop body serves both kinds of workgroup (a whole tile is one
    // pass), so the kernel holds one copy of the k loop and the epilogue.
    const int S = p.sk_wgs, s = (int)blockIdx.x - p.sk_dp;
    const int U = ((int)ntiles - p.sk_dp) * ktiles;
    int t_rel, kbeg, kend, u = 0, uend = 0;
    if (s < 0) {
        t_rel = (int)xcd_contiguous_id(blockIdx.x, (uint32_t)p.sk_dp) - p.sk_dp;
        kbeg = 0;
        kend = ktiles;
    } else {
        u = s * U / S;
        uend = (s + 1) * U / S;
        t_rel = u / ktiles;
        kbeg = u - t_rel * ktiles;
        kend = min(ktiles, uend - t_rel * ktiles);
        u = t_rel * ktiles + kend;
    }
    constexpr int QUADS = TM * TN * 4;  // 16-byte pieces of a lane's sums
    for (;;) {
        setup((uint32_t)(p.sk_dp + t_rel));
        run(kbeg, kend);
        bool out = true;
        if (kbeg != 0 || kend != ktiles) {
            // slot: 4 waves x QUADS x 64 lanes x 16 bytes = QUADS * 4096 bytes
            const __amdgpu_buffer_rsrc_t part = coherent_buffer(p.sk_part, (size_t)2 * S * QUADS * 4096);
            auto owner = [&](int v) { return ((v + 1) * S - 1) / U; };
            auto slot_off = [&](int w) {
                const int first = w * U / S / ktiles;
                return ((2 * w + (t_rel == first ? 0 : 1)) * QUADS * 256 + wave * QUADS * 64 + lane) * 16;
            };
            const int mine = slot_off(s);
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j)
#pragma unroll
                    for (int q = 0; q < 4; ++q)
                        store_coherent4(part, mine + ((i * TN + j) * 4 + q) * 64 * 16,
                                        f32x4{acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2],
                                              acc[i][j][4 * q + 3]});
            const int w_lo = owner(t_rel * ktiles), w_hi = owner((t_rel + 1) * ktiles - 1);
            out = arrive_last(p.sk_ctr + t_rel, (unsigned)(w_hi - w_lo + 1), &s_flag);
            if (out) {
                reset_arrival(p.sk_ctr + t_rel);
#pragma unroll
                for (int i = 0; i < TM; ++i)
#pragma unroll
                    for (int j = 0; j < TN; ++j)
#pragma unroll
                        for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
                for (int w = w_lo; w <= w_hi; ++w) {
                    const int off = slot_off(w);
#pragma unroll
                    for (int i = 0; i < TM; ++i)
#pragma unroll
                        for (int j = 0; j < TN; ++j)
#pragma unroll
                            for (int q = 0; q < 4; ++q) {
                                const f32x4 v = load_coherent4(part, off + ((i * TN + j) * 4 + q) * 64 * 16);
                                acc[i][j][4 * q] += v.x;
                                acc[i][j][4 * q + 1] += v.y;
                                acc[i][j][4 * q + 2] += v.z;
                                acc[i][j][4 * q + 3] += v.w;
                            }
                }
            }
        }
        if (out) store();
        if (u >= uend) break;
        t_rel = u / ktiles;
        kbeg = 0;
        kend = min(ktiles, uend - t_rel * ktiles);
        u = t_rel * ktiles + kend;
    }
}

// wt[(co*KHW + tap)*C_in + ci] = w[(co*C_in + ci)*KHW + tap]: the OIHW
// weights re-laid with the reduction index (tap, ci) major and C_out
// contiguous, so the conv's A tiles are plain float4 row copies.
__global__ void __launch_bounds__(256) conv_weights_per_co(float* __restrict__ wt, const float* __restrict__ w,
                                                           int C_out, int C_in, int KHW) {
    const size_t total = (size_t)C_out * C_in * KHW;
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t d = (size_t)blockIdx.x * blockDim.x + threadIdx.x; d < total; d += stride) {
        const int ci = (int)(d % C_in);
        const size_t r = d / C_in;
        const int tap = (int)(r % KHW), co = (int)(r / KHW);
        wt[d] = w[((size_t)co * C_in + ci) * KHW + tap];
    }
}

// ---- backward ------------------------------------------------------------
//
// Input gradient at stride 1 is itself a convolution: dx = conv(dy, w') with
// w'[ci][co][kh][kw] = w[co][ci][K_h-1-kh][K_w-1-kw] and padding K-1-pad,
// since dx[ih] = sum_kh dy[ih + pad - kh] w[kh].  The flipped weights are
// written straight into the layout the forward kernel reads: per output
// channel ((ci, tap) rows, C_out contiguous) when the forward kernel takes
// that path, OIHW otherwise.
__global__ void __launch_bounds__(256) dgrad_weights(float* __restrict__ wt, const float* __restrict__ w, int C_out,
                                                     int C_in, int KH, int KW, int per_co) {
    const int KHW = KH * KW;
    const size_t total = (size_t)C_out * C_in * KHW;
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t s = (size_t)blockIdx.x * blockDim.x + threadIdx.x; s < total; s += stride) {
        const int tap = (int)(s % KHW);
        const size_t r = s / KHW;
        const int ci = (int)(r % C_in), co = (int)(r / C_in);
        const int kh = tap / KW, kw = tap - (tap / KW) * KW;
        const int ftap = (KH - 1 - kh) * KW + (KW - 1 - kw);  // tap of the flipped filter
        const float v = w[s];
        // flipped conv: output channel ci, input channel co
        if (per_co)
            wt[((size_t)ci * KHW + ftap) * C_out + co] = v;
        else
            wt[((size_t)ci * C_out + co) * KHW + ftap] = v;
    }
}

// Any stride: one thread per dx element, summing over (co, kh, kw) in the
// reference's order (lancius_kernels.c:62-91 accumulates per output element
// over co, then ho/wo; the terms are the same).
__global__ void __launch_bounds__(256) dgrad_direct(float* __restrict__ dx, const float* __restrict__ dy,
                                                    const float* __restrict__ w, int N, int C_in, int H, int W,
                                                    int C_out, int Ho, int Wo, int KH, int KW, int stride, int pad) {
    const size_t total = (size_t)N * C_in * H * W;
    const size_t step = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += step) {
        const int iw = (int)(i % W);
        const int ih = (int)((i / W) % H);
        const int ci = (int)((i / ((size_t)W * H)) % C_in);
        const int n = (int)(i / ((size_t)W * H * C_in));
        float acc = 0.0f;
        for (int co = 0; co < C_out; ++co) {
            const float* g = dy + ((size_t)n * C_out + co) * Ho * Wo;
            const float* wk = w + ((size_t)co * C_in + ci) * KH * KW;
            for (int kh = 0; kh < KH; ++kh) {
                const int hn = ih + pad - kh;
                if (hn < 0 || hn % stride) continue;
                const int ho = hn / stride;
                if (ho >= Ho) continue;
                for (int kw = 0; kw < KW; ++kw) {
                    const int wn = iw + pad - kw;
                    if (wn < 0 || wn % stride) continue;
                    const int wo = wn / stride;
                    if (wo >= Wo) continue;
                    acc += g[(size_t)ho * Wo + wo] * wk[kh * KW + kw];
                }
            }
        }
        dx[i] = acc;
    }
}

// Weight gradient as a GEMM on the matrix cores:
//   dW[co][j] = sum_P dY[co][P] * X[j][P],  j = (ci, kh, kw), P = (n, ho, wo)
// with dY[co][P] = dy[n][co][ho][wo] and X[j][P] the im2col value
// x[n][ci][ho*stride-pad+kh][wo*stride-pad+kw] (0 outside the image).  The
// reduction over P (N*H_out*W_out, ~10^5 at the conv config) is split across
// blockIdx.y; wgrad_reduce adds the partials in a fixed order.
struct WgradParams {
    float* dw;
    float* ws;
    const float* dy;
    const float* x;
    int N, C_in, H, W, C_out, Ho, Wo, KH, KW, stride, pad;
    int J;             // C_in * KH * KW
    long long Ptotal;  // N * Ho * Wo
    long long pchunk;  // pixels per split (multiple of BK)
    int splits;
    uint32_t tiles_m, tiles_n;
};

// BK pixels per k-tile: lanes run along BK consecutive pixels of a row, so
// BK = 64 makes each load instruction one 256-byte run per row.
template <int BM, int BN, int BK>
__global__ void __launch_bounds__(256) conv2d_wgrad_mfma(const WgradParams p) {
    constexpr int WGM = 2, WGN = 2;
    constexpr int WM = BM / WGM, WN = BN / WGN;
    constexpr int TM = WM / 32, TN = WN / 32;
    constexpr int LDA = BM + 4, LDB = BN + 4;
    __shared__ __attribute__((aligned(16))) float As[2][BK][LDA];
    __shared__ __attribute__((aligned(16))) float Bs[2][BK][LDB];

    const uint32_t tile = blockIdx.x;
    const int m0 = (int)(tile / p.tiles_n) * BM;  // first output channel
    const int j0 = (int)(tile % p.tiles_n) * BN;  // first (ci, kh, kw)
    const int split = blockIdx.y;
    const long long pbeg = (long long)split * p.pchunk;
    const long long pend = pbeg + p.pchunk < p.Ptotal ? pbeg + p.pchunk : p.Ptotal;

    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const int wm = wave / WGN, wn = wave % WGN;
    const int lr = lane & 31, lk = lane >> 5;

    // Loader mapping: lanes along the pixel index (contiguous in memory).
    const int kk = tid % BK;
    const int row0 = tid / BK;                      // 0 .. 256/BK - 1
    constexpr int RSTEP = 256 / BK;                 // rows covered per pass
    constexpr int A_PER = BM / RSTEP;               // channels per thread
    constexpr int B_PER = BN / RSTEP;               // j per thread
    const int HWo = p.Ho * p.Wo, KHW = p.KH * p.KW;
    // The (ci, kh, kw) of each j this thread loads never changes.
    int b_off[B_PER], b_dh[B_PER], b_dw[B_PER];
#pragma unroll
    for (int i = 0; i < B_PER; ++i) {
        const int j = j0 + row0 + RSTEP * i;
        if (j < p.J) {
            const int ci = j / KHW, t = j - (j / KHW) * KHW;
            const int kh = t / p.KW, kw = t - (t / p.KW) * p.KW;
            b_off[i] = ci * p.H * p.W;
            b_dh[i] = kh - p.pad;
            b_dw[i] = kw - p.pad;
        } else {
            b_off[i] = -1;
            b_dh[i] = b_dw[i] = 0;
        }
    }
    float a_s[A_PER], b_s[B_PER];
    auto load_tile = [&](long long kt) {
        const long long P = pbeg + kt * BK + kk;
        const bool valid = P < pend;
        int n = 0, ho = 0, wo = 0;
        if (valid) {
            n = (int)(P / HWo);
            const int pix = (int)(P - (long long)n * HWo);
            ho = pix / p.Wo;
            wo = pix - ho * p.Wo;
        }
        const float* g = p.dy + ((size_t)n * p.C_out) * HWo + (size_t)ho * p.Wo + wo;
#pragma unroll
        for (int i = 0; i < A_PER; ++i) {
            const int co = m0 + row0 + RSTEP * i;
            a_s[i] = (valid && co < p.C_out) ? g[(size_t)co * HWo] : 0.0f;
        }
        const float* xi = p.x + (size_t)n * p.C_in * p.H * p.W;
        const int hb = ho * p.stride, wb = wo * p.stride;
#pragma unroll
        for (int i = 0; i < B_PER; ++i) {
            const int hi = hb + b_dh[i], wi = wb + b_dw[i];
            b_s[i] = (valid && b_off[i] >= 0 && hi >= 0 && hi < p.H && wi >= 0 && wi < p.W)
                         ? xi[(size_t)b_off[i] + (size_t)hi * p.W + wi]
                         : 0.0f;
        }
    };
    auto store_tile = [&](int buf) {
#pragma unroll
        for (int i = 0; i < A_PER; ++i) As[buf][kk][row0 + RSTEP * i] = a_s[i];
#pragma unroll
        for (int i = 0; i < B_PER; ++i) Bs[buf][kk][row0 + RSTEP * i] = b_s[i];
    };

    f32x16 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    const long long ktiles = pend > pbeg ? (pend - pbeg + BK - 1) / BK : 0;
    if (ktiles > 0) {
        load_tile(0);
        store_tile(0);
    }
    __syncthreads();
    for (long long kt = 0; kt < ktiles; ++kt) {
        const int cur = (int)(kt & 1);
        const bool more = kt + 1 < ktiles;
        if (more) load_tile(kt + 1);
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

    // Register r of lane l: channel row 8(r/4) + 4(l/32) + r%4, column l%32.
    float* dst = p.splits == 1 ? p.dw : p.ws + (size_t)split * p.C_out * p.J;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
        const int col = j0 + wn * WN + j * 32 + lr;
        if (col >= p.J) continue;
#pragma unroll
        for (int i = 0; i < TM; ++i) {
            const int cbase = m0 + wm * WM + i * 32 + 4 * lk;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int co = cbase + 8 * (r >> 2) + (r & 3);
                if (co < p.C_out) dst[(size_t)co * p.J + col] = acc[i][j][r];
            }
        }
    }
}

// Weight gradient with both operand tiles loaded straight from global memory
// into LDS (buffer loads with the LDS as destination), the forward direct
// GEMM's pipeline (gemm.hip, gemm_f32_direct): BM x 64 tiles (BM = 128 or
// 64), k-tiles of 16 pixels, 4 waves of (BM/2) x 32, two separate LDS
// buffers and the k loop unrolled by two.  Both operands run along the
// pixel index, so both live m-major, 64 bytes per row, chunk c (4 pixels)
// of row r at chunk c ^ ((r >> 2) & 3): the 16-byte operand reads of 16
// consecutive rows hit 16 different bank groups.  Lane half h of the MFMAs
// takes pixels [8h, 8h + 8) of the k-tile, the same for both operands.
//  * dY rows (channels m0..) load as 16-byte chunks: HWo % 4 == 0 keeps a
//    chunk of 4 pixels inside one image and 16-byte aligned.  Instruction i
//    of wave w fills LDS chunks (A_INSTR w + i) * 64 + lane; every
//    instruction of a lane reads the same pixel chunk (rows 16 apart share
//    the swizzle), so the lane tracks one (image, pixel) pair.
//  * X im2col rows (j = (ci, kh, kw) from j0) load 4 bytes per lane:
//    instruction t = w + 4 i writes words 64 t + lane, rows 4 t + lane/16,
//    whose swizzle is (4 t + ...) >> 2 & 3 = w: the lane's pixel is again
//    one per k-tile, tracked as (image, ho, wo) and advanced by 16 pixels a
//    k-tile without a division.  Taps outside the image, pixels past the
//    split's range and j past J use an offset past the buffer's end (the
//    load returns 0); channel rows past C_out read the last row and reach
//    only entries that are never stored.
// Requires HWo % 4 == 0, HWo >= 16 and dY, X under 2 GiB.
template <int BM>
__global__ void __launch_bounds__(256, 2) conv2d_wgrad_direct(const WgradParams p) {
    constexpr int BN = 64, BK = 16;
    constexpr int WM = BM / 2, WN = BN / 2, TM = WM / 32, TN = WN / 32;
    constexpr int A_INSTR = BM * BK / 4 / 64 / 4;  // 16-byte loads of dY per wave per k-tile
    constexpr int B_INSTR = BN * BK / 64 / 4;      // 4-byte loads of X per wave per k-tile
    static_assert(A_INSTR >= 1 && B_INSTR == 4 && TN == 1, "tile shape");
    typedef __attribute__((address_space(3))) void lds_void;
    __shared__ __attribute__((aligned(16))) float As0[BM * BK];
    __shared__ __attribute__((aligned(16))) float As1[BM * BK];
    __shared__ __attribute__((aligned(16))) float Bs0[BN * BK];
    __shared__ __attribute__((aligned(16))) float Bs1[BN * BK];

    const uint32_t tile = blockIdx.x;
    const int m0 = (int)(tile / p.tiles_n) * BM;  // first output channel
    const int j0 = (int)(tile % p.tiles_n) * BN;  // first (ci, kh, kw)
    const long long pbeg = (long long)blockIdx.y * p.pchunk;
    const int prange = (int)((pbeg + p.pchunk < p.Ptotal ? pbeg + p.pchunk : p.Ptotal) - pbeg);
    const int HWo = p.Ho * p.Wo, HW = p.H * p.W, KHW = p.KH * p.KW;

    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int wm = wave >> 1, wn = wave & 1;
    const int lr = lane & 31, lk = lane >> 5;

    const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(p.dy), 0, (int)((size_t)p.N * p.C_out * HWo * sizeof(float)), kBufferRsrcWord3);
    const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(p.x), 0, (int)((size_t)p.N * p.C_in * HW * sizeof(float)), kBufferRsrcWord3);
    constexpr int kOut = 0x7ffffff0;  // an offset past the end of any operand: the load returns 0

    // dY: this lane's rows and pixel chunk
    int a_rowoff[A_INSTR];
    const int qa = A_INSTR * wave * 64 + lane;
    const int a_c = (qa & 3) ^ ((qa >> 4) & 3);
#pragma unroll
    for (int i = 0; i < A_INSTR; ++i) a_rowoff[i] = min(m0 + ((qa >> 2) + 16 * i), p.C_out - 1) * HWo;
    int a_rel = 4 * a_c;  // pixel of the chunk, relative to pbeg
    int a_n, a_pix;
    {
        const long long P = pbeg + a_rel;
        a_n = (int)(P / HWo);
        a_pix = (int)(P - (long long)a_n * HWo);
    }
    // X: this lane's four rows j and its pixel
    int b_cioff[B_INSTR], b_dh[B_INSTR], b_dw[B_INSTR];
#pragma unroll
    for (int i = 0; i < B_INSTR; ++i) {
        const int j = j0 + 16 * i + 4 * wave + (lane >> 4);
        if (j < p.J) {
            const int ci = j / KHW, t = j - ci * KHW;
            const int kh = t / p.KW, kw = t - kh * p.KW;
            b_cioff[i] = ci * HW;
            b_dh[i] = kh - p.pad;
            b_dw[i] = kw - p.pad;
        } else {
            b_cioff[i] = -1;
            b_dh[i] = b_dw[i] = 0;
        }
    }
    int b_rel = 4 * (((lane & 15) >> 2) ^ wave) + (lane & 3);
    int b_n, b_ho, b_wo;
    {
        const long long P = pbeg + b_rel;
        b_n = (int)(P / HWo);
        const int pix = (int)(P - (long long)b_n * HWo);
        b_ho = pix / p.Wo;
        b_wo = pix - b_ho * p.Wo;
    }

    // Issues the loads of the next k-tile into (As, Bs) and advances the
    // lane's pixels by one k-tile.
    auto load_tile = [&](float* As, float* Bs) {
        const bool a_in = a_rel < prange;
#pragma unroll
        for (int i = 0; i < A_INSTR; ++i) {
            const int ao = pick(a_in, ((a_n * p.C_out) * HWo + a_rowoff[i] + a_pix) * (int)sizeof(float), kOut);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_void*)(As + (A_INSTR * wave + i) * 256), 16, ao, 0, 0,
                                                     0);
        }
        const bool b_in = b_rel < prange;
        const int hb = b_ho * p.stride, wb = b_wo * p.stride, xbase = b_n * p.C_in * HW;
#pragma unroll
        for (int i = 0; i < B_INSTR; ++i) {
            const int hi = hb + b_dh[i], wi = wb + b_dw[i];
            const bool in = b_in & (b_cioff[i] >= 0) & ((unsigned)hi < (unsigned)p.H) & ((unsigned)wi < (unsigned)p.W);
            const int bo = pick(in, (xbase + b_cioff[i] + hi * p.W + wi) * (int)sizeof(float), kOut);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, (lds_void*)(Bs + (wave + 4 * i) * 64), 4, bo, 0, 0, 0);
        }
        // keep the loads ahead of the MFMAs that follow
        __builtin_amdgcn_sched_barrier(0);
        a_rel += BK;
        a_pix += BK;
        if (a_pix >= HWo) {
            a_pix -= HWo;
            ++a_n;
        }
        b_rel += BK;
        b_wo += BK;
        while (b_wo >= p.Wo) {
            b_wo -= p.Wo;
            if (++b_ho == p.Ho) {
                b_ho = 0;
                ++b_n;
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

    // operand addresses (floats) of this lane, fixed over the k loop
    int a_rd[TM][2], b_rd[TN][2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int c = 2 * lk + h;
#pragma unroll
        for (int i = 0; i < TM; ++i) {
            const int row = wm * WM + i * 32 + lr;
            a_rd[i][h] = row * BK + 4 * (c ^ ((row >> 2) & 3));
        }
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const int row = wn * WN + j * 32 + lr;
            b_rd[j][h] = row * BK + 4 * (c ^ ((row >> 2) & 3));
        }
    }
    auto compute = [&](const float* As, const float* Bs) {
        f32x4 av[TM][2], bv[TN][2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
#pragma unroll
            for (int i = 0; i < TM; ++i) av[i][h] = *(const f32x4*)(As + a_rd[i][h]);
#pragma unroll
            for (int j = 0; j < TN; ++j) bv[j][h] = *(const f32x4*)(Bs + b_rd[j][h]);
        }
#pragma unroll
        for (int kp = 0; kp < 8; ++kp)
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[i][kp / 4][kp % 4], bv[j][kp / 4][kp % 4],
                                                                     acc[i][j], 0, 0, 0);
    };

    // k-tiles in pairs; when their count is odd the last pair's second tile
    // lies wholly past the range, loads as zeros and adds nothing.
    const int pairs = (prange + 2 * BK - 1) / (2 * BK);
    load_tile(As0, Bs0);
    __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
    __syncthreads();
    for (int pr = 0; pr < pairs; ++pr) {
        load_tile(As1, Bs1);
        compute(As0, Bs0);
        __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
        __syncthreads();
        if (pr + 1 < pairs) load_tile(As0, Bs0);
        compute(As1, Bs1);
        __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
        __syncthreads();
    }

    // Register r of lane l: channel row 8(r/4) + 4(l/32) + r%4, column l%32.
    float* dst = p.splits == 1 ? p.dw : p.ws + (size_t)blockIdx.y * p.C_out * p.J;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
        const int col = j0 + wn * WN + j * 32 + lr;
        if (col >= p.J) continue;
#pragma unroll
        for (int i = 0; i < TM; ++i) {
            const int cbase = m0 + wm * WM + i * 32 + 4 * lk;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int co = cbase + 8 * (r >> 2) + (r & 3);
                if (co < p.C_out) dst[(size_t)co * p.J + col] = acc[i][j][r];
            }
        }
    }
}

// A workgroup per 64 consecutive weights: lane l of wave g adds splits g,
// g+4, g+8, ... of weight l in order (a wave reads 256 contiguous bytes of a
// split's partials), then wave 0 adds the four sums in wave order: a fixed
// order, so results are identical from run to run.  (One wave per weight,
// its lanes on 64 splits a whole partial array apart, read a cache line per
// 4-byte value: 29.7 us for 85 splits of 73728 weights.)
__global__ void __launch_bounds__(256) wgrad_reduce(float* __restrict__ dw, const float* __restrict__ ws, size_t n,
                                                    int splits) {
    __shared__ float part[4][64];
    const int lane = threadIdx.x & 63, g = threadIdx.x >> 6;
    const size_t i = (size_t)blockIdx.x * 64 + lane;
    float s = 0.0f;
    if (i < n)
        for (int k = g; k < splits; k += 4) s += ws[(size_t)k * n + i];
    part[g][lane] = s;
    __syncthreads();
    if (g == 0 && i < n) dw[i] = ((part[0][lane] + part[1][lane]) + part[2][lane]) + part[3][lane];
}

template <int BM, int BN, int KH_T, int KW_T>
int launch(lancius_hip_ctx* ctx, ConvParams& p) {
    p.tiles_m = (uint32_t)((p.C_out + BM - 1) / BM);
    p.tiles_n = (uint32_t)((p.Ptotal + BN - 1) / BN);
    const size_t grid = (size_t)p.tiles_m * p.tiles_n;
    LANCIUS_REQUIRE(grid < kMaxGridX, LANCIUS_HIP_ERR_SHAPE, "conv2d: too many tiles");
    constexpr int WGM = BM >= 64 ? 2 : 1;
    constexpr int WGN = 4 / WGM;
    // The filter re-laid per output channel (taps outer, input channels
    // inner) feeds conv2d_direct (64- and 128-channel tiles: whole tiles,
    // plus a stream-K share of the rest when the tiles are not a multiple
    // of the CUs) and the A loads of the 32 x 128 implicit GEMM; every other
    // launch reads OIHW.  conv2d_direct addresses the input and the filter
    // with 32-bit offsets: the callers split the batch so that a launch's
    // input stays under 2 GiB (one image beyond that takes the OIHW path).
    constexpr bool kDirect = (BM == 64 || BM == 128) && (BN == 64 || BN == 128);
    const bool per_co = p.C_in % 16 == 0 && p.C_out % 4 == 0 &&
                        (size_t)p.N * p.C_in * p.H * p.W * sizeof(float) < LANCIUS_HIP_CONV_PACKED_MAX_BYTES &&
                        (size_t)p.C_out * p.Kdim * sizeof(float) < LANCIUS_HIP_CONV_PACKED_MAX_BYTES;
    const bool direct = kDirect && per_co;
    const bool wt_layout = per_co && (kDirect || BM == 32);
    LANCIUS_REQUIRE(p.prep != 0 || wt_layout, LANCIUS_HIP_ERR_SHAPE,
                    "conv2d_packed: an image of %d x %d x %d or the filter is beyond 2 GiB (use lancius_hip_conv2d_f32)",
                    p.C_in, p.H, p.W);
    void (*kern)(const ConvParams) = nullptr;
    if constexpr (kDirect) kern = conv2d_direct<BM, BN, KH_T, KW_T>;
    p.sk_dp = (int)grid;
    p.sk_wgs = 0;
    size_t part_bytes = 0;
    if (direct) {
        // resident workgroups per CU, per instantiation (host threads may
        // race to fill it in: they all store the same value)
        static std::atomic<int> slot;
        int occ = slot.load(std::memory_order_relaxed);
        if (occ == 0) {
            if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, kern, kThreads, 0) != hipSuccess || occ < 1) occ = 1;
            slot.store(occ, std::memory_order_relaxed);
        }
        // When tiles / CUs is a little above an integer n (at most n + 1/4)
        // and every workgroup is resident at once, whole tiles alone would
        // leave some CUs n + 1 tiles and the rest n: instead (n - 1) * CUs
        // workgroups take whole tiles and one per CU shares the rest, about
        // 1 + (tiles - n CUs) / CUs tiles each.  Measured at N32 64->128 56^2:
        // forward 140.4 -> 135.8 us, dgrad 150.3 -> 143.6 us; with 2, 3 or 6
        // sharing workgroups per CU it ran slower (each shared tile costs a
        // hand-off through the point of coherence), and larger remainders
        // are faster as whole tiles (N33: 6.32 tiles per CU 141.0 against
        // 143.7 us; N31: 5.93, 122.7 against 141.3).
        const size_t cus = (size_t)cu_count(ctx), per = grid / cus, rem = grid % cus;
        const size_t units = (grid - (per > 0 ? per - 1 : 0) * cus) * (size_t)p.Kdim / 16;
        // Grids under half the CUs (small batches): every workgroup takes an
        // equal share of all (tile, k-tile) units, each share at least 18
        // k-tiles and a tile split at most 8 ways (the finishing workgroup
        // reads every share through the point of coherence, about 30 GB/s
        // for one workgroup).  Measured with the filter re-laid in the call:
        // N1 64->128 56^2 30.8 -> 25.9 us, N2 30.9 -> 26.8, N1 128->256 28^2
        // 55.7 -> 32.0, N1 256->512 14^2 107.6 -> 46.6, N2 64->64 56^2 21.1
        // -> 17.2; shares of at least 8 or 12 k-tiles measured slower at 56^2.
        const size_t sk_small =
            std::min(cus, grid * std::min<size_t>(8, std::max<size_t>(1, (size_t)p.Kdim / 16 / 18)));
        if (per == 0 && sk_small >= 2 * grid && units >= 4 * sk_small && units * sk_small < ((size_t)1 << 31)) {
            p.sk_dp = 0;
            p.sk_wgs = (int)sk_small;
            part_bytes = 2 * sk_small * BM * BN * sizeof(float);
        } else if (per >= 1 && per <= (size_t)occ && rem != 0 && rem <= cus / 4 && units * cus < ((size_t)1 << 31)) {
            p.sk_dp = (int)((per - 1) * cus);
            p.sk_wgs = (int)cus;
            part_bytes = 2 * cus * BM * BN * sizeof(float);
        }
    }
    const size_t wcount = (size_t)p.C_out * p.Kdim;
    const size_t wbytes = (p.prep == 1 && wt_layout) || p.prep == 2 ? (wcount * sizeof(float) + 255) / 256 * 256 : 0;
    if (wbytes + part_bytes > 0) {
        void* ws = nullptr;
        if (int rc = workspace(ctx, wbytes + part_bytes, &ws)) return rc;
        p.sk_part = (float*)((char*)ws + wbytes);
        const unsigned wgrid = (unsigned)std::min<size_t>((wcount + 255) / 256, 2048);
        if (p.prep == 1 && wt_layout) {
            p.wt = (const float*)ws;
            hipLaunchKernelGGL(conv_weights_per_co, dim3(wgrid), dim3(256), 0, ctx->stream, (float*)ws, p.w, p.C_out,
                               p.C_in, p.KH * p.KW);
            if (int rc = check_launch("conv_weights_per_co")) return rc;
        } else if (p.prep == 2) {
            hipLaunchKernelGGL(dgrad_weights, dim3(wgrid), dim3(256), 0, ctx->stream, (float*)ws, p.w_src, p.C_in,
                               p.C_out, p.KH, p.KW, (int)wt_layout);
            if (int rc = check_launch("conv2d_dgrad_weights")) return rc;
            if (wt_layout)
                p.wt = (const float*)ws;
            else
                p.w = (const float*)ws;
        }
    }
    if (direct) {
        if (p.sk_wgs > 0)
            if (int rc = counters(ctx, grid - (size_t)p.sk_dp, &p.sk_ctr)) return rc;
        hipLaunchKernelGGL(kern, dim3((unsigned)(p.sk_dp + p.sk_wgs)), dim3(kThreads), 0, ctx->stream, p);
        return check_launch("conv2d_direct");
    }
    if constexpr (BM == 32) {
        if (wt_layout) {
            hipLaunchKernelGGL((conv2d_implicit_gemm<BM, BN, 16, WGM, WGN, KH_T, KW_T, true>), dim3((unsigned)grid),
                               dim3(kThreads), 0, ctx->stream, p);
            return check_launch("conv2d_implicit_gemm");
        }
    }
    hipLaunchKernelGGL((conv2d_implicit_gemm<BM, BN, 16, WGM, WGN, KH_T, KW_T, false>), dim3((unsigned)grid),
                       dim3(kThreads), 0, ctx->stream, p);
    return check_launch("conv2d_implicit_gemm");
}

int default_tile(size_t C_out) { return C_out > 64 ? 1 : C_out > 32 ? 2 : 3; }

template <int KH_T, int KW_T>
int launch_tile(lancius_hip_ctx* ctx, ConvParams& p, int tile);

// One launch per run of images whose input stays under 2 GiB (the direct
// kernel's 32-bit input offsets); the images of a conv are independent, so
// the split changes no result.  p describes the whole batch.
int launch_batches(lancius_hip_ctx* ctx, const ConvParams& p, int tile) {
    const size_t img_in = (size_t)p.C_in * p.H * p.W, img_out = (size_t)p.C_out * p.Ho * p.Wo;
    const size_t per = std::max<size_t>(1, std::min<size_t>((size_t)p.N, (LANCIUS_HIP_CONV_PACKED_MAX_BYTES - 1) /
                                                                           (img_in * sizeof(float))));
    for (size_t n0 = 0; n0 < (size_t)p.N; n0 += per) {
        ConvParams q = p;
        q.N = (int)std::min<size_t>(per, (size_t)p.N - n0);
        q.in = p.in + n0 * img_in;
        q.out = p.out + n0 * img_out;
        q.Ptotal = (long long)q.N * p.Ho * p.Wo;
        const int rc = (p.KH == 3 && p.KW == 3) ? launch_tile<3, 3>(ctx, q, tile) : launch_tile<0, 0>(ctx, q, tile);
        if (rc) return rc;
    }
    return 0;
}

template <int KH_T, int KW_T>
int launch_tile(lancius_hip_ctx* ctx, ConvParams& p, int tile) {
    switch (tile) {
        case 1: return launch<128, 64, KH_T, KW_T>(ctx, p);
        case 2: return launch<64, 64, KH_T, KW_T>(ctx, p);
        default: return launch<32, 128, KH_T, KW_T>(ctx, p);
    }
}

}  // namespace
}  // namespace lancius

using namespace lancius;

namespace {

// The forward conv with the filter as OIHW w (re-laid per call when the
// kernels want it per output channel) or, with w null, already packed.
int conv2d_entry(lancius_hip_ctx* ctx, float* out, const float* in, const float* w, const float* packed,
                 const float* bias, size_t N, size_t C_in, size_t H, size_t W, size_t C_out, size_t K_h, size_t K_w,
                 size_t stride, size_t pad, int act) {
    LANCIUS_REQUIRE(ctx && out && in && (w || packed), LANCIUS_HIP_ERR_NULL_PTR, "conv2d: NULL argument");
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
    p.wt = packed;
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
    p.prep = packed ? 0 : 1;
    // Tiles (C_out x pixels): 0 = 128x128, 1 = 128x64, 2 = 64x64, 3 = 32x128,
    // the one whose channel extent covers C_out with the least padding.
    // 128x64 measured best on the N32 64->128 56x56 config (with the direct
    // loads 100.9 TFLOP/s against 89.6 for 128x128): twice the workgroups, a
    // shorter tail; 64x64 for its dgrad (64 output channels: 238 -> 204 us
    // against 32x128).
    const int rc = launch_batches(ctx, p, default_tile(C_out));
    return rc ? rc : ok();
}

}  // namespace

extern "C" int lancius_hip_conv2d_f32(lancius_hip_ctx* ctx, float* out, const float* in, const float* w,
                                      const float* bias, size_t N, size_t C_in, size_t H, size_t W, size_t C_out,
                                      size_t K_h, size_t K_w, size_t stride, size_t pad, int act) {
    LANCIUS_REQUIRE(w, LANCIUS_HIP_ERR_NULL_PTR, "conv2d: NULL weights");
    return conv2d_entry(ctx, out, in, w, nullptr, bias, N, C_in, H, W, C_out, K_h, K_w, stride, pad, act);
}

extern "C" size_t lancius_hip_conv2d_packed_bytes(size_t C_out, size_t C_in, size_t K_h, size_t K_w) {
    return C_out * C_in * K_h * K_w * sizeof(float);
}

extern "C" int lancius_hip_conv2d_pack_weight(lancius_hip_ctx* ctx, float* packed, const float* w, size_t C_out,
                                              size_t C_in, size_t K_h, size_t K_w) {
    LANCIUS_REQUIRE(ctx && packed && w, LANCIUS_HIP_ERR_NULL_PTR, "conv2d_pack_weight: NULL argument");
    LANCIUS_REQUIRE(C_out && C_in && K_h && K_w && C_in % 16 == 0 && C_out % 4 == 0 &&
                        C_out * C_in * K_h * K_w < ((size_t)1 << 31),
                    LANCIUS_HIP_ERR_SHAPE, "conv2d_pack_weight: C_out=%zu C_in=%zu (need C_in %% 16 == 0, C_out %% 4 == 0)",
                    C_out, C_in);
    if (int rc = bind_device(ctx)) return rc;
    const size_t total = C_out * C_in * K_h * K_w;
    hipLaunchKernelGGL(conv_weights_per_co, dim3((unsigned)std::min<size_t>((total + 255) / 256, 2048)), dim3(256), 0,
                       ctx->stream, packed, w, (int)C_out, (int)C_in, (int)(K_h * K_w));
    if (int rc = check_launch("conv_weights_per_co")) return rc;
    return ok();
}

extern "C" int lancius_hip_conv2d_packed_f32(lancius_hip_ctx* ctx, float* out, const float* in, const float* packed,
                                             const float* bias, size_t N, size_t C_in, size_t H, size_t W,
                                             size_t C_out, size_t K_h, size_t K_w, size_t stride, size_t pad,
                                             int act) {
    LANCIUS_REQUIRE(packed, LANCIUS_HIP_ERR_NULL_PTR, "conv2d_packed: NULL weights");
    LANCIUS_REQUIRE(C_in % 16 == 0 && C_out % 4 == 0, LANCIUS_HIP_ERR_SHAPE,
                    "conv2d_packed: C_out=%zu C_in=%zu (need C_in %% 16 == 0, C_out %% 4 == 0)", C_out, C_in);
    return conv2d_entry(ctx, out, in, nullptr, packed, bias, N, C_in, H, W, C_out, K_h, K_w, stride, pad, act);
}

extern "C" int lancius_hip_conv2d_bwd_input_f32(lancius_hip_ctx* ctx, float* dx, const float* dy, const float* w,
                                                size_t N, size_t C_in, size_t H, size_t W, size_t C_out,
                                                size_t H_out, size_t W_out, size_t K_h, size_t K_w, size_t stride,
                                                size_t pad) {
    LANCIUS_REQUIRE(ctx && dx && dy && w, LANCIUS_HIP_ERR_NULL_PTR, "conv2d_bwd_input: NULL argument");
    LANCIUS_REQUIRE(K_h && K_w && stride, LANCIUS_HIP_ERR_SHAPE, "conv2d_bwd_input: empty filter or stride 0");
    LANCIUS_REQUIRE(C_in * K_h * K_w < (1u << 30) && C_out * K_h * K_w < (1u << 30) && H * W < (1u << 30) &&
                        H_out * W_out < (1u << 30) && N * C_in * H * W < ((size_t)1 << 40) &&
                        N * C_out * H_out * W_out < ((size_t)1 << 40),
                    LANCIUS_HIP_ERR_SHAPE, "conv2d_bwd_input: shape too large");
    const size_t total = N * C_in * H * W;
    if (total == 0) return ok();
    if (int rc = bind_device(ctx)) return rc;
    // Stride 1, square filter, the shapes of a real forward conv
    // (H = H_out + K - 1 - 2 pad, pad <= K - 1): the forward implicit GEMM
    // over flipped weights.  Anything else: the direct kernel.
    const bool as_conv = stride == 1 && K_h == K_w && pad + 1 <= K_h && H_out > 0 && W_out > 0 &&
                         H + 2 * pad + 1 == H_out + K_h && W + 2 * pad + 1 == W_out + K_w;
    if (!as_conv) {
        const unsigned grid = (unsigned)std::max<size_t>(1, std::min<size_t>((total + 255) / 256, 16384));
        hipLaunchKernelGGL(dgrad_direct, dim3(grid), dim3(256), 0, ctx->stream, dx, dy, w, (int)N, (int)C_in, (int)H,
                           (int)W, (int)C_out, (int)H_out, (int)W_out, (int)K_h, (int)K_w, (int)stride, (int)pad);
        return check_launch("conv2d_dgrad_direct");
    }
    ConvParams p{};
    p.out = dx;
    p.in = dy;
    p.bias = nullptr;
    p.N = (int)N;
    p.C_in = (int)C_out;  // the flipped conv reads dy's channels
    p.H = (int)H_out;
    p.W = (int)W_out;
    p.C_out = (int)C_in;
    p.KH = (int)K_h;
    p.KW = (int)K_w;
    p.stride = 1;
    p.pad = (int)(K_h - 1 - pad);
    p.Ho = (int)H;
    p.Wo = (int)W;
    p.Kdim = (int)(C_out * K_h * K_w);
    p.Ptotal = (long long)N * H * W;
    p.act = LANCIUS_HIP_ACT_NONE;
    p.prep = 2;  // the launch lays out the flipped weights of w
    p.w_src = w;
    const int rc = launch_batches(ctx, p, default_tile((size_t)p.C_out));
    return rc ? rc : ok();
}

extern "C" int lancius_hip_conv2d_bwd_weight_f32(lancius_hip_ctx* ctx, float* dw, const float* dy, const float* x,
                                                 size_t N, size_t C_in, size_t H, size_t W, size_t C_out,
                                                 size_t H_out, size_t W_out, size_t K_h, size_t K_w, size_t stride,
                                                 size_t pad) {
    LANCIUS_REQUIRE(ctx && dw && dy && x, LANCIUS_HIP_ERR_NULL_PTR, "conv2d_bwd_weight: NULL argument");
    LANCIUS_REQUIRE(K_h && K_w && stride, LANCIUS_HIP_ERR_SHAPE, "conv2d_bwd_weight: empty filter or stride 0");
    LANCIUS_REQUIRE(C_in * K_h * K_w < (1u << 30) && C_out < (1u << 30) && H * W < (1u << 30) &&
                        C_in * H * W < (1u << 31) && H_out * W_out < (1u << 30) &&
                        N * C_in * H * W < ((size_t)1 << 40) &&
                        N * C_out * H_out * W_out < ((size_t)1 << 40),
                    LANCIUS_HIP_ERR_SHAPE, "conv2d_bwd_weight: shape too large");
    const size_t J = C_in * K_h * K_w;
    if (C_out * J == 0) return ok();
    if (int rc = bind_device(ctx)) return rc;
    // 128 x 64 tiles (two 32 x 32 MFMA blocks per wave) when C_out > 64,
    // else 64 x 64 (one)
    const int BM = C_out > 64 ? 128 : 64, BN = 64;
    WgradParams p{};
    p.dw = dw;
    p.dy = dy;
    p.x = x;
    p.N = (int)N;
    p.C_in = (int)C_in;
    p.H = (int)H;
    p.W = (int)W;
    p.C_out = (int)C_out;
    p.Ho = (int)H_out;
    p.Wo = (int)W_out;
    p.KH = (int)K_h;
    p.KW = (int)K_w;
    p.stride = (int)stride;
    p.pad = (int)pad;
    p.J = (int)J;
    p.Ptotal = (long long)(N * H_out * W_out);
    p.tiles_m = (uint32_t)((C_out + BM - 1) / BM);
    p.tiles_n = (uint32_t)((J + BN - 1) / BN);
    const size_t tiles = (size_t)p.tiles_m * p.tiles_n;
    LANCIUS_REQUIRE(tiles < kMaxGridX, LANCIUS_HIP_ERR_SHAPE, "conv2d_bwd_weight: too many tiles");
    // Split the pixel reduction so the grid is one full round of resident
    // workgroups (CUs x workgroups per CU by LDS), each >= 256 pixels deep:
    // a partial second round costs the time of a whole one.  k-tiles of 32
    // pixels (16: 64-byte runs per load; 64: 70 KB of LDS, fewer workgroups
    // per CU).  At the N32 64->128 56x56 config: 64 x 64 tiles, 57 splits
    // (1026 workgroups for 1024 slots) 0.239 ms; 128 x 64 tiles, 85 splits
    // (765 for 768) 0.216 ms.
    // conv2d_wgrad_direct: k-tiles of 16 pixels taken in pairs (so the
    // split length is a multiple of 32), splits for three workgroups per CU
    // (N32 64->128 56x56: 0.1477 ms at two, 0.1450 at three, 0.1461 at four;
    // the staged kernel 0.1939)
    const size_t HWo = H_out * W_out;
    const bool direct = HWo % 4 == 0 && HWo >= 16 &&
                        N * C_out * HWo * sizeof(float) < ((size_t)1 << 31) - 64 &&
                        N * C_in * H * W * sizeof(float) < ((size_t)1 << 31) - 64;
    constexpr int bk = 32;
    const long long ktiles = (p.Ptotal + bk - 1) / bk;
    long long splits;
    {
        const size_t lds = (size_t)2 * bk * ((BM + 4) + (BN + 4)) * sizeof(float);
        const size_t per_cu = direct ? 3 : std::max<size_t>(1, std::min<size_t>(8, 163840 / lds));
        const size_t slots = (size_t)cu_count(ctx) * per_cu;
        splits = std::max<long long>(1, std::min<long long>((long long)std::max<size_t>(1, slots / tiles),
                                                            ktiles * bk / 256));
    }
    splits = std::max<long long>(1, std::min<long long>({splits, std::max<long long>(ktiles, 1), 65535}));
    while (splits > 1 && (size_t)splits * C_out * J * sizeof(float) > ((size_t)1 << 28)) splits = (splits + 1) / 2;
    const long long chunk_tiles = (std::max<long long>(ktiles, 1) + splits - 1) / splits;
    p.pchunk = chunk_tiles * bk;
    p.splits = (int)((std::max<long long>(ktiles, 1) + chunk_tiles - 1) / chunk_tiles);
    if (p.splits > 1) {
        void* ws = nullptr;
        if (int rc = workspace(ctx, (size_t)p.splits * C_out * J * sizeof(float), &ws)) return rc;
        p.ws = (float*)ws;
    }
    const dim3 grid((unsigned)tiles, (unsigned)p.splits);
    if (direct && BM == 128)
        hipLaunchKernelGGL(conv2d_wgrad_direct<128>, grid, dim3(256), 0, ctx->stream, p);
    else if (direct)
        hipLaunchKernelGGL(conv2d_wgrad_direct<64>, grid, dim3(256), 0, ctx->stream, p);
    else if (BM == 128)
        hipLaunchKernelGGL((conv2d_wgrad_mfma<128, 64, bk>), grid, dim3(256), 0, ctx->stream, p);
    else
        hipLaunchKernelGGL((conv2d_wgrad_mfma<64, 64, bk>), grid, dim3(256), 0, ctx->stream, p);
    if (int rc = check_launch("conv2d_wgrad_mfma")) return rc;
    if (p.splits > 1) {
        const size_t n = C_out * J;
        LANCIUS_REQUIRE((n + 63) / 64 < kMaxGridX, LANCIUS_HIP_ERR_SHAPE, "conv2d_bwd_weight: %zu weights", n);
        hipLaunchKernelGGL(wgrad_reduce, dim3((unsigned)((n + 63) / 64)), dim3(256), 0, ctx->stream, dw,
                           (const float*)p.ws, n, p.splits);
        if (int rc = check_launch("conv2d_wgrad_reduce")) return rc;
    }
    return ok();
}
