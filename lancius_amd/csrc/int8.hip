// The int8 path of the scheduler and the vision router on the gfx950 int8
// matrix cores (v_mfma_i32_32x32x32_i8, 16 int8 per lane, int32 accumulate).
//
// Semantics (bleeding/v11A1/src/runtime/lancius_scheduler.c:195-220 and
// lancius_vision_ops.c:16-57 with lancius_kernels.c:177-210):
//  * the fp activation is quantized per tensor on the fly:
//      scale = max|x| / 127 (1e-8 when the tensor is all zero),
//      q = (int8) round(x / scale)   (round half away from zero, in fp64);
//  * the weight is int8 with its own per-tensor scale (lancius_quantize.c:6-31
//    for conv filters; any int8 B for MATMUL);
//  * out = (double) sum_k q_a * q_b (int32) * scale_a * scale_b.
// The int32 sums are exact, so the device output equals the reference's
// fp64 value rounded once to fp32.
//
// Layouts: both MFMA operands are staged k-contiguous, so one lane's 16
// int8 are one 16-byte LDS read.  The GEMM quantizes A [M][K] row-major
// (k-contiguous) and re-lays B [K][N] as B^T [N][K]; the conv quantizes its
// NCHW input into NHWC with the channels padded to a multiple of 16, and
// re-lays the OIHW weights as [C_out][(kh, kw, ci)] with the same padding,
// so a k-run of 16 is 16 channels of one filter tap at one pixel: a single
// 16-byte gather.  The padded weight bytes are zero, which makes whatever
// the padded activation bytes hold irrelevant.
#include <algorithm>

#include "common.hpp"
#include "kernels.hpp"

namespace lancius {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int kThreads = 256;
constexpr int kMaxBlocks = 512;

// ---- quantization ------------------------------------------------------------

// Per-workgroup max|x| (order-independent, so the result does not depend on
// the grid).  vec: x is 16-byte aligned; four float4 loads per thread are in
// flight per step.
__global__ void __launch_bounds__(kThreads) absmax_partials(float* __restrict__ part, const float* __restrict__ x,
                                                            size_t n, int vec) {
    __shared__ float s[kThreads / 64];
    float m = 0.0f;
    const size_t T = (size_t)gridDim.x * kThreads, t0 = (size_t)blockIdx.x * kThreads + threadIdx.x;
    size_t tail = 0;
    if (vec) {
        const size_t n4 = n / 4;
        const f32x4* __restrict__ x4 = (const f32x4*)x;
        size_t i = t0;
        for (; i + 3 * T < n4; i += 4 * T) {
            const f32x4 a = x4[i], b = x4[i + T], c = x4[i + 2 * T], d = x4[i + 3 * T];
            m = fmaxf(m, fmaxf(fmaxf(fmaxf(fabsf(a.x), fabsf(a.y)), fmaxf(fabsf(a.z), fabsf(a.w))),
                               fmaxf(fmaxf(fabsf(b.x), fabsf(b.y)), fmaxf(fabsf(b.z), fabsf(b.w)))));
            m = fmaxf(m, fmaxf(fmaxf(fmaxf(fabsf(c.x), fabsf(c.y)), fmaxf(fabsf(c.z), fabsf(c.w))),
                               fmaxf(fmaxf(fabsf(d.x), fabsf(d.y)), fmaxf(fabsf(d.z), fabsf(d.w)))));
        }
        for (; i < n4; i += T) {
            const f32x4 a = x4[i];
            m = fmaxf(m, fmaxf(fmaxf(fabsf(a.x), fabsf(a.y)), fmaxf(fabsf(a.z), fabsf(a.w))));
        }
        tail = 4 * n4;
    }
    for (size_t i = tail + t0; i < n; i += T) m = fmaxf(m, fabsf(x[i]));
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
    if ((threadIdx.x & 63) == 0) s[threadIdx.x >> 6] = m;
    __syncthreads();
    if (threadIdx.x == 0) part[blockIdx.x] = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
}

// The per-tensor scale from the partial maxima, computed by every
// workgroup of the consuming kernel (all threads must call it):
// scale = max|x| / 127, or 1e-8 for an all-zero tensor (fp64, as the
// reference).  Workgroup 0 also stores it at scale_out[0], and the other
// operand's host-given scale at scale_out[1] when `other` >= 0, for the
// GEMM epilogue and the caller.
__device__ double scale_from_partials(const float* __restrict__ part, int parts, double* __restrict__ scale_out,
                                      double other) {
    __shared__ float s[kThreads / 64];
    float m = 0.0f;
    for (int i = threadIdx.x; i < parts; i += kThreads) m = fmaxf(m, part[i]);
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
    if ((threadIdx.x & 63) == 0) s[threadIdx.x >> 6] = m;
    __syncthreads();
    m = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
    const double sc = m > 0.0f ? (double)m / 127.0 : 1e-8;
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        scale_out[0] = sc;
        if (other >= 0.0) scale_out[1] = other;
    }
    return sc;
}

// The reference's quantized value: (int8) round(x / scale), the quotient
// rounded to fp64 first, halves away from zero.  Fast path in fp32:
// r = x * fl32(1 / scale) is within 1.5e-5 of x / scale (|x / scale| <=
// 127.5, two roundings of 2^-24 relative), so when r's fraction is farther
// than 1e-4 from one half, round(r) is the reference's integer.  The rest -
// values near a half, NaN, and scales below 1e-30 whose reciprocal would
// overflow fp32 - take the fp64 division.
struct Quantizer {
    double scale;
    float inv;
    bool fast;
    __device__ explicit Quantizer(double s) : scale(s), inv((float)(1.0 / s)), fast(s >= 1e-30) {}
    __device__ __forceinline__ int8_t operator()(float v) const {
        if (fast) {
            const float r = v * inv;
            const float a = fabsf(r);
            if (fabsf(a - floorf(a) - 0.5f) >= 1e-4f) return (int8_t)(int)roundf(r);
        }
        return (int8_t)(int)round((double)v / scale);
    }
    __device__ __forceinline__ uint32_t pack4(float a, float b, float c, float d) const {
        return (uint32_t)(uint8_t)(*this)(a) | (uint32_t)(uint8_t)(*this)(b) << 8 |
               (uint32_t)(uint8_t)(*this)(c) << 16 | (uint32_t)(uint8_t)(*this)(d) << 24;
    }
};

// Row-major copy: q[i] = quant(x[i]).
__global__ void __launch_bounds__(kThreads) quantize_flat(int8_t* __restrict__ q, const float* __restrict__ x,
                                                          const float* __restrict__ part, int parts,
                                                          double* __restrict__ scale_out, size_t n) {
    const Quantizer quant(scale_from_partials(part, parts, scale_out, -1.0));
    const size_t step = (size_t)gridDim.x * kThreads;
    for (size_t i = (size_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += step) q[i] = quant(x[i]);
}

// Conv weights for the implicit GEMM: OIHW int8 -> [C_out][Kp] with
// k = (kh, kw, ci), Cp channels per tap; zero for ci >= C_in and for
// k >= KHW * Cp.  Element d of wblocks * kThreads per step.
struct ConvWeightsI8 {
    int8_t* wt;
    const int8_t* w;
    int C_out, C_in, KHW, Cp, Kp, blocks;
};
__device__ __forceinline__ void conv_weights_i8_part(const ConvWeightsI8& cw, int block) {
    const size_t total = (size_t)cw.C_out * cw.Kp;
    const size_t step = (size_t)cw.blocks * kThreads;
    for (size_t d = (size_t)block * kThreads + threadIdx.x; d < total; d += step) {
        const int k = (int)(d % cw.Kp), co = (int)(d / cw.Kp);
        const int tap = k / cw.Cp, ci = k - (k / cw.Cp) * cw.Cp;
        cw.wt[d] = (tap < cw.KHW && ci < cw.C_in) ? cw.w[((size_t)co * cw.C_in + ci) * cw.KHW + tap] : (int8_t)0;
    }
}

// NCHW fp32 -> NHWC int8 with Cp >= C channels per pixel (padding bytes 0),
// through a 64 (channels) x 64 (pixels) LDS tile: reads coalesce along the
// pixels of a channel plane (VEC, H*W % 4 == 0 and x 16-byte aligned: one
// float4 of 4 pixels per load, through a buffer whose past-the-end offset
// stands for channels and pixels that do not exist, so no load sits behind
// a branch); each write is 4 channels of one pixel packed into 32 bits, 16
// lanes covering 64 channels of a pixel.  Workgroups past the activation's
// tiles re-lay the conv weights (the two are independent: one launch).
template <bool VEC>
__global__ void __launch_bounds__(kThreads) quantize_nchw_to_nhwc(int8_t* __restrict__ q, const float* __restrict__ x,
                                                                  const float* __restrict__ part, int parts,
                                                                  double* __restrict__ scale_out, double other, int N,
                                                                  int C, int HW, int Cp, int tiles_p, int tiles_c,
                                                                  const ConvWeightsI8 cw) {
    const int qblocks = N * tiles_p * tiles_c;
    if ((int)blockIdx.x >= qblocks) {
        conv_weights_i8_part(cw, (int)blockIdx.x - qblocks);
        return;
    }
    __shared__ int8_t t[64][65];
    const Quantizer quant(scale_from_partials(part, parts, scale_out, other));
    const int tile = blockIdx.x;
    const int n = tile / (tiles_p * tiles_c);
    const int rem = tile - n * tiles_p * tiles_c;
    const int c0 = (rem / tiles_p) * 64, p0 = (rem % tiles_p) * 64;
    const float* xn = x + (size_t)n * C * HW;
    if constexpr (VEC) {
        constexpr int kOut = 0x7ffffff0;
        const __amdgpu_buffer_rsrc_t xb = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<float*>(xn), 0, C * HW * (int)sizeof(float), kBufferRsrcWord3);
        f32x4 v[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int idx = threadIdx.x + kThreads * i;
            const int cl = idx >> 4, p = p0 + 4 * (idx & 15), c = c0 + cl;
            v[i] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                 xb, pick((c < C) & (p < HW), (c * HW + p) * (int)sizeof(float), kOut),
                                                 0, 0));
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int idx = threadIdx.x + kThreads * i;
            const int cl = idx >> 4, pl = 4 * (idx & 15);
#pragma unroll
            for (int e = 0; e < 4; ++e) t[cl][pl + e] = quant(v[i][e]);  // zeros past C and HW quantize to 0
        }
    } else {
        const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int c = c0 + ty + 4 * i, p = p0 + tx;
            t[ty + 4 * i][tx] = (c < C && p < HW) ? quant(xn[(size_t)c * HW + p]) : (int8_t)0;
        }
    }
    __syncthreads();
    int8_t* qn = q + (size_t)n * HW * Cp;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int idx = threadIdx.x + kThreads * i;
        const int pl = idx >> 4, cq = idx & 15;
        const int p = p0 + pl, c = c0 + 4 * cq;
        if (p < HW && c < Cp) {
            const uint32_t v = (uint32_t)(uint8_t)t[4 * cq][pl] | (uint32_t)(uint8_t)t[4 * cq + 1][pl] << 8 |
                               (uint32_t)(uint8_t)t[4 * cq + 2][pl] << 16 | (uint32_t)(uint8_t)t[4 * cq + 3][pl] << 24;
            *(uint32_t*)(qn + (size_t)p * Cp + c) = v;
        }
    }
}

// B [K][N] int8 -> B^T [N][Kp] int8 (k zero-padded to Kp, a multiple of
// 128), one 128 (k) x 128 (n) tile per workgroup.  Reads: 16-byte runs of a
// k-row (vec: N % 16 == 0 and B 16-byte aligned; otherwise byte loads with
// bounds), kept in LDS as T[n/4][k] words of 4 n-bytes.  Writes: a thread
// takes 4 columns n x 16 rows k, transposes the 16 x 4 bytes in registers and
// stores four 16-byte runs of B^T rows; 8 lanes cover 128 contiguous bytes.
__global__ void __launch_bounds__(kThreads) transpose_i8(int8_t* __restrict__ bt, const int8_t* __restrict__ b, int K,
                                                         int N, int Kp, int tiles_n, int vec) {
    constexpr int P = 130;  // words per T row (2-way bank aliasing on the writes)
    __shared__ uint32_t T[32 * P];
    const int k0 = (blockIdx.x / tiles_n) * 128, n0 = (blockIdx.x % tiles_n) * 128;
    const int tid = threadIdx.x;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int idx = tid + kThreads * i;
        const int k = idx >> 3, c = idx & 7;
        const int gk = k0 + k, gn = n0 + 16 * c;
        v4i w = {0, 0, 0, 0};
        if (gk < K) {
            if (vec) {
                if (gn < N) w = *(const v4i*)(b + (size_t)gk * N + gn);
            } else {
                uint32_t u[4] = {0, 0, 0, 0};
#pragma unroll
                for (int e = 0; e < 16; ++e)
                    if (gn + e < N) u[e >> 2] |= (uint32_t)(uint8_t)b[(size_t)gk * N + gn + e] << (8 * (e & 3));
                w = v4i{(int)u[0], (int)u[1], (int)u[2], (int)u[3]};
            }
        }
#pragma unroll
        for (int d = 0; d < 4; ++d) T[(4 * c + d) * P + k] = (uint32_t)w[d];
    }
    __syncthreads();
    const int nq = tid >> 3, kb = tid & 7;
    uint32_t w[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) w[i] = T[nq * P + 16 * kb + i];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int n = n0 + 4 * nq + j;
        if (n >= N) break;
        v4i o;
#pragma unroll
        for (int m = 0; m < 4; ++m)
            o[m] = (int)(((w[4 * m] >> (8 * j)) & 0xffu) | ((w[4 * m + 1] >> (8 * j)) & 0xffu) << 8 |
                         ((w[4 * m + 2] >> (8 * j)) & 0xffu) << 16 | ((w[4 * m + 3] >> (8 * j)) & 0xffu) << 24);
        *(v4i*)(bt + (size_t)n * Kp + k0 + 16 * kb) = o;
    }
}

// A [M][K] fp32 -> [M][Kp] int8, zeros past K (Kp a multiple of 128, so a
// row is D = Kp/4 words).  Each thread writes whole 32-bit words (vec: K % 4
// == 0 and A 16-byte aligned, one float4 per word), four words per trip with
// their loads issued together; rows shorter than the workgroup share it,
// 256/D rows at a time.
__global__ void __launch_bounds__(kThreads) quantize_rows_padded(int8_t* __restrict__ q, const float* __restrict__ x,
                                                                 const float* __restrict__ part, int parts,
                                                                 double* __restrict__ scale_out, double other,
                                                                 size_t M, int K, int Kp, int vec) {
    const Quantizer quant(scale_from_partials(part, parts, scale_out, other));
    const int D = Kp / 4;
    const int rows_per = D >= kThreads ? 1 : kThreads / D;
    const int sub = D >= kThreads ? 0 : (int)threadIdx.x / D;
    const int d0 = D >= kThreads ? (int)threadIdx.x : (int)threadIdx.x % D;
    const int dstep = D >= kThreads ? kThreads : D;
    if (sub >= rows_per) return;
    for (size_t r = (size_t)blockIdx.x * rows_per + sub; r < M; r += (size_t)gridDim.x * rows_per) {
        const float* __restrict__ xr = x + r * K;
        uint32_t* __restrict__ qr = (uint32_t*)(q + r * Kp);
        for (int d = d0; d < D; d += 4 * dstep) {
            if (vec) {
                f32x4 v[4];
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const int k = 4 * (d + u * dstep);
                    v[u] = k < K ? *(const f32x4*)(xr + k) : f32x4{0.f, 0.f, 0.f, 0.f};
                }
#pragma unroll
                for (int u = 0; u < 4; ++u)
                    if (d + u * dstep < D) qr[d + u * dstep] = quant.pack4(v[u].x, v[u].y, v[u].z, v[u].w);
            } else {
                for (int u = 0; u < 4 && d + u * dstep < D; ++u) {
                    const int k = 4 * (d + u * dstep);
                    uint32_t packed = 0;
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (k + e < K) packed |= (uint32_t)(uint8_t)quant(xr[k + e]) << (8 * e);
                    qr[d + u * dstep] = packed;
                }
            }
        }
    }
}

// ---- int8 GEMM / implicit-GEMM conv on v_mfma_i32_32x32x32_i8 ---------------

struct I8Params {
    float* C;
    const int8_t* A;     // [M][Kp] k-contiguous (quantized activation or conv weights)
    const int8_t* B;     // GEMM: B^T [N][Kp]; conv: NHWC activation with Cp channels
    const float* bias;   // per output column (GEMM) / channel (conv); may be null
    const float* R;      // residual (GEMM only); may be null
    const double* scale_a;  // device scalar
    const double* scale_b;  // device scalar
    int M, N, Kp;        // Kp: padded k extent (multiple of the k-tile)
    int act;
    uint32_t tiles_m, tiles_n;
    // conv geometry (CONV == true): N = N_img * Ho * Wo pixels
    int H, W, Cp, KW, KHW, stride, pad, Ho, Wo, HWo;
    int out_channels;    // conv: C_out (M) for the NCHW store
};

// CONV selects the B-operand gather (im2col over NHWC) and the NCHW store;
// otherwise B rows come from B^T and C is row-major [M][N].  WGM x WGN waves
// each own a (BM/WGM) x (BN/WGN) sub-tile; BK int8 of k per tile.
//
// A k-tile's global loads are issued two tiles ahead of its use (two
// register sets, even and odd tiles, and an LDS double buffer): at the LDS
// store of tile t+1 the loads of tile t+2 stay in flight.  The implicit-GEMM
// conv and GEMMs with fewer than ~240 256 x 256 tiles use this kernel; large
// GEMMs use gemm_i8_direct.
template <int BM, int BN, int WGM, int WGN, int BK, bool CONV, int MINW = 8 / (WGM * WGN)>
__global__ void __launch_bounds__(64 * WGM * WGN, MINW) gemm_i8_mfma(const I8Params p) {
    constexpr int LDK = BK + 16;
    constexpr int NT = 64 * WGM * WGN;
    constexpr int WM = BM / WGM, WN = BN / WGN;
    constexpr int TM = WM / 32, TN = WN / 32;
    static_assert(BK % 32 == 0, "k-tile of whole MFMA steps");
    __shared__ __attribute__((aligned(16))) int8_t As[2][BM][LDK];
    __shared__ __attribute__((aligned(16))) int8_t Bs[2][BN][LDK];

    const uint32_t ntiles = p.tiles_m * p.tiles_n;
    uint32_t tm_id, tn_id;
    grouped_tile(xcd_contiguous_id(blockIdx.x, ntiles), p.tiles_m, p.tiles_n, 4, tm_id, tn_id);
    const int m0 = (int)tm_id * BM, n0 = (int)tn_id * BN;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int wm = wave / WGN, wn = wave % WGN;
    const int lr = lane & 31, lh = lane >> 5;

    // Each thread moves 16-byte chunks: chunk c of a tile row is k bytes
    // [16c, 16c+16).  A tile: BM rows x CH chunks, B tile: BN rows x CH chunks.
    constexpr int CH = BK / 16;
    constexpr int A_LD = BM * CH / NT, B_LD = BN * CH / NT;
    static_assert(A_LD * NT == BM * CH && B_LD * NT == BN * CH, "even split");
    v4i a0[A_LD], b0[B_LD], a1[A_LD], b1[B_LD];

    // Rows past M (A) or N (B) are loaded from row M-1 / N-1 instead of
    // being zeroed: they only reach accumulator rows / columns that the
    // epilogue never stores, and the loads need no branch.  k is padded
    // with zeros to Kp in both operands.
    const int8_t* a_row[A_LD];
#pragma unroll
    for (int i = 0; i < A_LD; ++i) {
        const int idx = tid + i * NT;
        a_row[i] = p.A + (size_t)min(m0 + idx / CH, p.M - 1) * p.Kp + 16 * (idx % CH);
    }
    const int8_t* b_row[B_LD];
    // conv: the pixel of each B row this thread loads (fixed for the k loop)
    int pix_n[B_LD], pix_h[B_LD], pix_w[B_LD];
#pragma unroll
    for (int i = 0; i < B_LD; ++i) {
        const int idx = tid + i * NT;
        const int row = idx / CH;
        if constexpr (!CONV) {
            b_row[i] = p.B + (size_t)min(n0 + row, p.N - 1) * p.Kp + 16 * (idx % CH);
        } else {
            const int P = n0 + row;
            if (P < p.N) {
                const int img = P / p.HWo, rem = P - (P / p.HWo) * p.HWo;
                const int ho = rem / p.Wo, wo = rem - (rem / p.Wo) * p.Wo;
                pix_n[i] = img;
                pix_h[i] = ho * p.stride - p.pad;
                pix_w[i] = wo * p.stride - p.pad;
            } else {
                pix_n[i] = -1;
                pix_h[i] = pix_w[i] = 0;
            }
        }
    }

    // Every load is unconditional, so the compiler's wait counts see one
    // path: a load skipped on some path made it wait for all outstanding
    // loads at the LDS store, the look-ahead tile included.  The conv gather
    // loads the image's first pixel for taps outside the image and zeroes
    // them at the store (bit i of *bin).
    auto load_tile = [&](int k0, v4i* av, v4i* bv, unsigned* bin) {
#pragma unroll
        for (int i = 0; i < A_LD; ++i) av[i] = *(const v4i*)(a_row[i] + k0);
        if constexpr (CONV) *bin = 0;
#pragma unroll
        for (int i = 0; i < B_LD; ++i) {
            if constexpr (!CONV) {
                bv[i] = *(const v4i*)(b_row[i] + k0);
            } else {
                // k = (tap, channel run): 16 channels of one tap at one pixel
                const int k = k0 + 16 * ((tid + i * NT) % CH);
                const int tap = k / p.Cp, c = k - (k / p.Cp) * p.Cp;
                const int kh = tap / p.KW, kw = tap - (tap / p.KW) * p.KW;
                const int hi = pix_h[i] + kh, wi = pix_w[i] + kw;
                const bool in = pix_n[i] >= 0 && tap < p.KHW && hi >= 0 && hi < p.H && wi >= 0 && wi < p.W;
                const size_t off = in ? (((size_t)pix_n[i] * p.H + hi) * p.W + wi) * p.Cp + c : 0;
                bv[i] = *(const v4i*)(p.B + off);
                *bin |= (unsigned)in << i;
            }
        }
    };
    auto store_tile = [&](int buf, const v4i* av, const v4i* bv, unsigned bin) {
#pragma unroll
        for (int i = 0; i < A_LD; ++i) {
            const int idx = tid + i * NT;
            *(v4i*)&As[buf][idx / CH][16 * (idx % CH)] = av[i];
        }
#pragma unroll
        for (int i = 0; i < B_LD; ++i) {
            const int idx = tid + i * NT;
            v4i v = bv[i];
            if constexpr (CONV) {
                if (!((bin >> i) & 1u)) v = v4i{0, 0, 0, 0};
            }
            *(v4i*)&Bs[buf][idx / CH][16 * (idx % CH)] = v;
        }
    };

    v16i acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;

    auto compute = [&](int buf) {
#pragma unroll
        for (int ks = 0; ks < BK / 32; ++ks) {
            // lane half h holds k bytes [32ks + 16h, +16) of its row / column
            v4i af[TM], bf[TN];
#pragma unroll
            for (int i = 0; i < TM; ++i) af[i] = *(const v4i*)&As[buf][wm * WM + i * 32 + lr][32 * ks + 16 * lh];
#pragma unroll
            for (int j = 0; j < TN; ++j) bf[j] = *(const v4i*)&Bs[buf][wn * WN + j * 32 + lr][32 * ks + 16 * lh];
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
    };

    // Even tiles live in (a0, b0) and LDS buffer 0, odd tiles in (a1, b1)
    // and buffer 1.
    // Past the last tile the loads re-read the last tile (never stored).
    const int ktiles = p.Kp / BK;
    unsigned in0 = 0, in1 = 0;
    load_tile(0, a0, b0, &in0);
    load_tile(min(1, ktiles - 1) * BK, a1, b1, &in1);
    store_tile(0, a0, b0, in0);
    __syncthreads();
    // Pairs of tiles per trip, the odd last tile after the loop (an exit in
    // the middle of the trip made the compiler rotate the loop and keep two
    // copies of the accumulators).
    int kt = 0;
    for (; kt + 1 < ktiles; kt += 2) {
        load_tile(min(kt + 2, ktiles - 1) * BK, a0, b0, &in0);
        compute(0);
        __builtin_amdgcn_sched_barrier(0);
        store_tile(1, a1, b1, in1);  // waits for tile kt+1 only
        __syncthreads();
        load_tile(min(kt + 3, ktiles - 1) * BK, a1, b1, &in1);
        compute(1);
        __builtin_amdgcn_sched_barrier(0);
        if (kt + 2 < ktiles) store_tile(0, a0, b0, in0);
        __syncthreads();
    }
    if (kt < ktiles) compute(0);

    // int32 -> (double) * scale_a * scale_b -> fp32, then bias / act / residual.
    // Register r of lane l: row 8(r/4) + 4(l/32) + r%4, column l%32.
    const double scale = p.scale_a[0] * p.scale_b[0];
#pragma unroll
    for (int j = 0; j < TN; ++j) {
        const int col = n0 + wn * WN + j * 32 + lr;
        if (col >= p.N) continue;
        float* obase = nullptr;
        if constexpr (CONV) {
            const int img = col / p.HWo, pix = col - (col / p.HWo) * p.HWo;
            obase = p.C + (size_t)img * p.out_channels * p.HWo + pix;
        }
#pragma unroll
        for (int i = 0; i < TM; ++i) {
            const int rbase = m0 + wm * WM + i * 32 + 4 * lh;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = rbase + 8 * (r >> 2) + (r & 3);
                if (row >= p.M) continue;
                float v = (float)((double)acc[i][j][r] * scale);
                if constexpr (CONV) {
                    if (p.bias) v += p.bias[row];
                    obase[(size_t)row * p.HWo] = apply_act(v, p.act);
                } else {
                    if (p.bias) v += p.bias[col];
                    v = apply_act(v, p.act);
                    const size_t o = (size_t)row * p.N + col;
                    if (p.R) v += p.R[o];
                    p.C[o] = v;
                }
            }
        }
    }
}

// The int8 conv as a loop over output pixels with the filter resident in
// LDS.  A workgroup holds ROWS = 32 TM output channels of the filter
// ([ROWS][Kp] int8; the LDS row stride, ldw bytes, is an odd number of
// 16-byte chunks, so the 16-byte fragment reads of 8 consecutive rows fall
// on distinct bank groups) for the whole launch.  Each wave takes tiles of
// 32 consecutive output pixels, all ROWS channels (TM accumulators of
// 32 x 32), and gathers its pixel operands straight from the NHWC int8
// activation into registers: one 16-byte buffer load per lane per k-step
// (lane half h: k bytes [32 ks + 16 h, +16) = 16 channels of one tap at the
// lane's pixel), kConvI8Ring k-steps ahead; taps outside the image, and k
// past the filter's KHW * Cp, load from an offset past the buffer's end
// (zeros).  After the prologue the filter is read-only, so the k loop has
// no barrier.  One workgroup of 8 waves per CU: workgroup b serves
// output-channel block b % co_blocks and an equal share of its consecutive
// pixel tiles (they share input rows in the CU's L1), dealt to the waves
// one per SIMD first; a wave issues its next tile's first loads before its
// current tile's stores.  The epilogue computes what gemm_i8_mfma's does
// (fp64 scale, fp32 result, bias, ReLU, NCHW store), so both kernels give
// the same bits.
// Requires Kp % (32 kConvI8Ring) == 0, Kp <= kConvI8MaxKp, ROWS * ldw + 32 <= kConvI8Lds, KHW <= 64
// and the activation under 2 GiB - 64 (b_bytes: its size; the past-the-end
// offset lies beyond it).
constexpr int kConvI8Lds = 78848;
constexpr int kConvI8Threads = 512;  // 8 waves, one workgroup per CU
constexpr int kConvI8Ring = 3;
constexpr int kConvI8MaxKp = 2400;  // whole rings; 32 rows of it fit kConvI8Lds
constexpr int kConvI8KtPad = 2 * kConvI8Ring + 2;

template <int TM, int TN>
__global__ void __launch_bounds__(kConvI8Threads, 2) conv_i8_direct(const I8Params p, int co_blocks, int ldw,
                                                                     int b_bytes) {
    constexpr int ROWS = 32 * TM, PX = 32 * TN, NT = kConvI8Threads, NW = NT / 64;
    __shared__ __attribute__((aligned(16))) int8_t wl[kConvI8Lds];
    __shared__ __attribute__((aligned(16))) float bl[ROWS];
    __shared__ int2 kt[kConvI8MaxKp / 16 + kConvI8KtPad];
    const int cb = (int)blockIdx.x % co_blocks;
    const int wg = (int)blockIdx.x / co_blocks, wgs = (int)gridDim.x / co_blocks;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lr = lane & 31, lh = lane >> 5;
    const int Kp = p.Kp, chunks = Kp / 16;

    // k-step s, lane half h: k = 32 s + 16 h is channel c of tap (kh, kw);
    // kt[2 s + h] = (tap, input offset of the tap and channel relative to
    // the pixel's top-left tap), tap 64 for k past the filter (the table
    // runs a ring and one entry past Kp: the loads issued ahead of the
    // loop's end)
    for (int i = tid; i < Kp / 16 + kConvI8KtPad; i += NT) {
        const int k = 16 * i, tap = k / p.Cp, c = k - tap * p.Cp;
        const int kh = tap / p.KW, kw = tap - kh * p.KW;
        kt[i] = int2{tap < p.KHW ? tap : 64, (kh * p.W + kw) * p.Cp + c};
    }
    for (int r = tid; r < ROWS; r += NT) bl[r] = p.bias && cb * ROWS + r < p.M ? p.bias[cb * ROWS + r] : 0.0f;
    __syncthreads();

    const __amdgpu_buffer_rsrc_t rb =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<int8_t*>(p.B), 0, b_bytes, kBufferRsrcWord3);
    constexpr int kOut = 0x7ffffff0;
    const int KH = p.KHW / p.KW;
    const int ksteps = Kp / 32;
    const int tiles = (p.N - 1) / PX + 1;

    // The current tile: PX output pixels from t * PX; B fragment j holds
    // pixel t * PX + 32 j + l%32 of this lane (pv: it exists), with its
    // image, offset in the image's plane, the input offset of its top-left
    // tap (base) and which taps lie inside the image (bit tap of inside).
    // ls / e walk the k-step table one load ahead.  A workgroup takes an
    // equal share of consecutive tiles (its waves share input rows in L1),
    // dealt to the waves one per SIMD first (waves w and w + 4 share a
    // SIMD).
    const int t_end = (int)((long long)(wg + 1) * tiles / wgs);
    const int slot = (wave & 3) * 2 + (wave >> 2);
    int t = (int)((long long)wg * tiles / wgs) + slot;
    bool pv[TN];
    int img[TN], pix[TN], base[TN];
    uint64_t inside[TN];
    int ls = 0;
    int2 e = int2{64, 0};
    auto setup = [&]() {
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const int P = t * PX + 32 * j + lr;
            pv[j] = P < p.N;
            img[j] = pix[j] = 0;
            int hi0 = 0, wi0 = 0;
            if (pv[j]) {
                img[j] = P / p.HWo;
                pix[j] = P - img[j] * p.HWo;
                const int ho = pix[j] / p.Wo, wo = pix[j] - (pix[j] / p.Wo) * p.Wo;
                hi0 = ho * p.stride - p.pad;
                wi0 = wo * p.stride - p.pad;
            }
            uint64_t in_mask = 0;
            for (int kh = 0, tap = 0; kh < KH; ++kh)
                for (int kw = 0; kw < p.KW; ++kw, ++tap) {
                    const bool in = pv[j] && hi0 + kh >= 0 && hi0 + kh < p.H && wi0 + kw >= 0 && wi0 + kw < p.W;
                    in_mask |= (uint64_t)in << tap;
                }
            inside[j] = in_mask;
            base[j] = ((img[j] * p.H + hi0) * p.W + wi0) * p.Cp;
        }
        ls = 0;
        e = kt[lh];
    };
    v4i bq[kConvI8Ring][TN];
    auto next_loads = [&](v4i* dst) {
        const int2 cur = e;
        e = kt[2 * ++ls + lh];
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const bool in = (inside[j] >> (cur.x & 63)) & (uint64_t)(cur.x < 64);
            const int off = pick(in, base[j] + cur.y, kOut);
            dst[j] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(rb, off, 0, 0));
        }
    };
    // the first ring of loads, issued in slot order as the loop issues them
    // (so the wait counts at the loop head agree on every edge)
    auto prime = [&]() {
#pragma unroll
        for (int u = 0; u < kConvI8Ring; ++u) {
            next_loads(bq[u]);
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    if (t < t_end) {
        setup();
        prime();
    }

    // The filter block into LDS while the first tile's loads are in flight:
    // TPR threads per row, each taking every TPR-th 16-byte chunk, 10 loads
    // in flight at a time (every workgroup reads the same block: loads
    // issued one at a time made this a chain of L2 round trips).
    {
        constexpr int TPR = NT / ROWS;
        const int r = tid / TPR, co = cb * ROWS + r;
        const int8_t* src = p.A + (size_t)min(co, p.M - 1) * Kp;
        for (int c0 = tid % TPR; c0 < chunks; c0 += 10 * TPR) {
            v4i v[10];
#pragma unroll
            for (int j = 0; j < 10; ++j) {
                const int c = c0 + j * TPR;
                v[j] = c < chunks && co < p.M ? *(const v4i*)(src + 16 * c) : v4i{0, 0, 0, 0};
            }
#pragma unroll
            for (int j = 0; j < 10; ++j) {
                const int c = c0 + j * TPR;
                if (c < chunks) *(v4i*)(wl + r * ldw + 16 * c) = v[j];
            }
        }
    }
    __syncthreads();

    const double scale = p.scale_a[0] * p.scale_b[0];
    const int8_t* const a_lane = wl + lr * ldw + 16 * lh;
    while (t < t_end) {
        v16i acc[TM][TN];
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;
        // the filter fragments of k-step s + 1 are read while the MFMAs of
        // step s run (past the last step: padding inside the LDS array)
        v4i a[TM];
#pragma unroll
        for (int i = 0; i < TM; ++i) a[i] = *(const v4i*)(a_lane + i * 32 * ldw);
        for (int ks = 0; ks < ksteps; ks += kConvI8Ring) {
#pragma unroll
            for (int u = 0; u < kConvI8Ring; ++u) {
                v4i an[TM];
#pragma unroll
                for (int i = 0; i < TM; ++i) an[i] = *(const v4i*)(a_lane + i * 32 * ldw + 32 * (ks + u + 1));
#pragma unroll
                for (int i = 0; i < TM; ++i)
#pragma unroll
                    for (int j = 0; j < TN; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[i], bq[u][j], acc[i][j], 0, 0, 0);
                // refill the slot with k-step ks + u + ring (past the last
                // k-step the table says tap 64: zero loads, never used)
                next_loads(bq[u]);
#pragma unroll
                for (int i = 0; i < TM; ++i) a[i] = an[i];
                // next step's fragment reads first, then the MFMAs, then the loads
                __builtin_amdgcn_sched_group_barrier(0x100, TM + 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x008, TM * TN, 0);
                __builtin_amdgcn_sched_group_barrier(0x020, TN, 0);
                __builtin_amdgcn_sched_barrier(0);
            }
        }

        // The next tile's first loads go out before this tile's stores: a
        // wave's loads and stores retire in issue order, so loads issued
        // after the stores would wait for all of them.
        bool out_pv[TN];
        int out_img[TN], out_pix[TN];
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            out_pv[j] = pv[j];
            out_img[j] = img[j];
            out_pix[j] = pix[j];
        }
        t += NW;
        if (t < t_end) {
            setup();
            prime();
        }

        // register r of accumulator (i, j), lane l: channel 8(4i + r/4) +
        // 4(l/32) + r%4 of the block, pixel 32 j + l%32 of the tile.  The row
        // pointer steps 8 rows per register quad (no per-row offsets stay
        // live across tiles), a quad's four biases are one LDS read, and
        // blocks wholly inside C_out store without a per-row check (the
        // int8 conv takes no activation but ReLU).
        const size_t hw = (size_t)p.HWo;
        const bool relu = p.act == kActRelu;
        const bool full = (cb + 1) * ROWS <= p.M;
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            if (!out_pv[j]) continue;
            float* o = p.C + ((size_t)out_img[j] * p.out_channels + cb * ROWS + 4 * lh) * hw + out_pix[j];
            auto quad = [&](int g, bool check) {
                const f32x4 bv = *(const f32x4*)(bl + 8 * g + 4 * lh);
#pragma unroll
                for (int s = 0; s < 4; ++s) {
                    float v = (float)((double)acc[g >> 2][j][4 * (g & 3) + s] * scale) + bv[s];
                    v = relu ? relu_ref(v) : v;
                    if (!check || cb * ROWS + 8 * g + 4 * lh + s < p.M) o[s * hw] = v;
                }
                o += 8 * hw;
            };
            if (full) {
#pragma unroll
                for (int g = 0; g < 4 * TM; ++g) quad(g, false);
            } else {
#pragma unroll
                for (int g = 0; g < 4 * TM; ++g) quad(g, true);
            }
        }
    }
}

// GEMM only: 256 x 256 tiles, one workgroup of 4 waves per CU, each wave
// a 128 x 128 block (16 accumulators of 32 x 32, so every 16-byte fragment
// read from LDS feeds 4 MFMAs).  Both operands are k-contiguous ([M][Kp]
// and B^T [N][Kp]) and are loaded straight into LDS with 16-byte buffer
// loads (LDS destination): k-tiles of 128 bytes, two static buffers, the
// loads of tile kt + 2 issued from the last k-step of tile kt over SPREAD
// k-steps (1 to 3).  In LDS a row
// is 8 chunks of 16 bytes, chunk c stored at slot c ^ ((row >> 1) & 7): the
// 16 rows one fragment read touches in a cycle fall on 16 distinct bank
// groups.  Fragments of k-step s + 1 are read while the MFMAs of step s run.
// Rows past M / N load as zeros (an offset past the buffer's end) and are
// never stored; an odd last k-tile is paired with an all-zero one.
// Requires (M + 1) * Kp and (N + 1) * Kp below 2^31 - 16.
template <int SPREAD>
__global__ void __launch_bounds__(256, 1) gemm_i8_direct(const I8Params p) {
    static_assert(SPREAD >= 1 && SPREAD <= 3, "loads spread over 1 to 3 k-steps");
    constexpr int BM = 256, BN = 256, BK = 128, TM = 4, TN = 4;
    constexpr int kTileBytes = BM * BK;  // one operand's k-tile (BM == BN)
    typedef __attribute__((address_space(3))) void lds_void;
    __shared__ __attribute__((aligned(16))) int8_t As0[kTileBytes];
    __shared__ __attribute__((aligned(16))) int8_t As1[kTileBytes];
    __shared__ __attribute__((aligned(16))) int8_t Bs0[kTileBytes];
    __shared__ __attribute__((aligned(16))) int8_t Bs1[kTileBytes];

    const uint32_t ntiles = p.tiles_m * p.tiles_n;
    uint32_t tm_id, tn_id;
    grouped_tile(xcd_contiguous_id(blockIdx.x, ntiles), p.tiles_m, p.tiles_n, 4, tm_id, tn_id);
    const int m0 = (int)tm_id * BM, n0 = (int)tn_id * BN;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    const int lr = lane & 31, lh = lane >> 5;
    const int Kp = p.Kp;

    const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<int8_t*>(p.A), 0, (int)((size_t)p.M * Kp), kBufferRsrcWord3);
    const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<int8_t*>(p.B), 0, (int)((size_t)p.N * Kp), kBufferRsrcWord3);
    // Offsets are 32-bit unsigned.  A row past M (N) starts at M * Kp, the
    // buffer's end, so it reads zeros at every k0 < Kp; the all-zero tail
    // tile adds kOut = 2^31 - 16 to in-range offsets (< 2^31 - Kp), which
    // lands past the end without wrapping (the host checks (M + 1) * Kp <
    // 2^31 - 16, and the same for N).
    constexpr unsigned kOut = 0x7ffffff0u;

    // Instruction i of wave w fills LDS chunks (4i + w) * 64 + lane: tile row
    // (4i + w) * 8 + lane / 8, slot lane % 8.  The slot's logical chunk is
    // the same for every i.
    const int sub_row = wave * 8 + (lane >> 3);
    const int chunk = (lane & 7) ^ (((wave & 1) * 4 + (lane >> 4)) & 7);
    unsigned a_off[8], b_off[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        a_off[i] = (unsigned)min(m0 + 32 * i + sub_row, p.M) * (unsigned)Kp + 16u * chunk;
        b_off[i] = (unsigned)min(n0 + 32 * i + sub_row, p.N) * (unsigned)Kp + 16u * chunk;
    }
    // Load i (0..7 A, 8..15 B) of k-tile kt, for lo <= i < hi.
    auto load_part = [&](int8_t* As, int8_t* Bs, int kt, int lo, int hi) {
        const unsigned k0 = kt * BK < Kp ? (unsigned)(kt * BK) : kOut;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            if (i < lo || i >= hi) continue;
            if (i < 8)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_void*)(As + (4 * i + wave) * 1024), 16,
                                                         (int)(a_off[i] + k0), 0, 0, 0);
            else
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, (lds_void*)(Bs + (4 * (i - 8) + wave) * 1024), 16,
                                                         (int)(b_off[i - 8] + k0), 0, 0, 0);
        }
    };
    // part q of SPREAD holds loads [lo(q), lo(q + 1))
    constexpr int kParts = SPREAD;
    auto lo = [](int q) { return 16 * q / kParts; };

    // fragment addresses (bytes) at k-step 0; step s reads chunk 2s + lh
    int a_rd[TM], b_rd[TN], a_sw[TM], b_sw[TN];
#pragma unroll
    for (int i = 0; i < TM; ++i) {
        const int row = wm * 128 + i * 32 + lr;
        a_rd[i] = row * BK;
        a_sw[i] = (row >> 1) & 7;
    }
#pragma unroll
    for (int j = 0; j < TN; ++j) {
        const int row = wn * 128 + j * 32 + lr;
        b_rd[j] = row * BK;
        b_sw[j] = (row >> 1) & 7;
    }

    v16i acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;

    auto read_frags = [&](const int8_t* As, const int8_t* Bs, int s, v4i* af, v4i* bf) {
        const int c = 2 * s + lh;
#pragma unroll
        for (int i = 0; i < TM; ++i) af[i] = *(const v4i*)(As + a_rd[i] + 16 * (c ^ a_sw[i]));
#pragma unroll
        for (int j = 0; j < TN; ++j) bf[j] = *(const v4i*)(Bs + b_rd[j] + 16 * (c ^ b_sw[j]));
    };
    auto mfmas = [&](const v4i* af, const v4i* bf) {
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[i], bf[j], acc[i][j], 0, 0, 0);
    };
    // One k-step: its 16 MFMAs with the next step's 8 fragment reads placed
    // one after each of the first 8 (the reads land while MFMAs run), and the
    // n global loads issued just before spread evenly over the 16 MFMAs.
    auto step = [&](const v4i* af, const v4i* bf, const int8_t* As, const int8_t* Bs, int s_next, v4i* an,
                    v4i* bn, int n = 0) {
        read_frags(As, Bs, s_next, an, bn);
        mfmas(af, bf);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                     // MFMA
            if (i < 8) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);          // LDS read
            if ((i + 1) * n / 16 > i * n / 16)
                __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);                 // global load
        }
        __builtin_amdgcn_sched_barrier(0);
    };
    // One k-tile in buffer X (fragments of its step 0 already in f0), with
    // tile kt + 1 landing in Y.  The barrier sits before the last step: by
    // then every wave holds all of X's fragments, so X can take tile kt + 2
    // and the last step's MFMAs cover the first reads of Y.  The loads of
    // tile kt + 2 start in that step (part 0) and the rest go with the first
    // steps of tile kt + 1, so no step issues more loads than the CU's
    // address unit takes in the step's MFMA time.
    v4i fa0[TM], fb0[TN], fa1[TM], fb1[TN];
    auto tile = [&](int8_t* Xa, int8_t* Xb, int8_t* Ya, int8_t* Yb, int kt) {
        if (kParts > 1) load_part(Ya, Yb, kt + 1, lo(1), lo(2));
        step(fa0, fb0, Xa, Xb, 1, fa1, fb1, kParts > 1 ? lo(2) - lo(1) : 0);
        if (kParts > 2) load_part(Ya, Yb, kt + 1, lo(2), lo(3));
        step(fa1, fb1, Xa, Xb, 2, fa0, fb0, kParts > 2 ? lo(3) - lo(2) : 0);
        step(fa0, fb0, Xa, Xb, 3, fa1, fb1);
        __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
        __syncthreads();
        load_part(Xa, Xb, kt + 2, 0, lo(1));
        step(fa1, fb1, Ya, Yb, 0, fa0, fb0, lo(1));
    };

    // k-tiles in pairs; tiles at or past Kp load as zeros (an odd count's
    // last pair adds nothing; the look-ahead past the end is never used).
    const int pairs = (Kp / BK + 1) / 2;
    load_part(As0, Bs0, 0, 0, 16);
    __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
    __syncthreads();
    load_part(As1, Bs1, 1, 0, lo(1));  // the rest in tile 0's first steps
    read_frags(As0, Bs0, 0, fa0, fb0);
    for (int pr = 0; pr < pairs; ++pr) {
        tile(As0, Bs0, As1, Bs1, 2 * pr);
        tile(As1, Bs1, As0, Bs0, 2 * pr + 1);
    }
    // the last look-ahead loads land before the workgroup ends
    __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);

    // int32 -> (double) * scale_a * scale_b -> fp32, then bias / act / residual.
    // Register r of lane l: row 8(r/4) + 4(l/32) + r%4, column l%32.
    // Epilogue staged through LDS (free now): each wave takes one of the four
    // 32 KB arrays and, per half of its block (64 rows x 128 columns), writes
    // the scaled values there, then reads whole rows back as float4 and
    // stores them with bias, activation and residual: 64 row-contiguous
    // 16-byte stores per lane instead of 256 scattered 4-byte ones.  Column
    // c of row r sits at c ^ (32 * ((r >> 2) & 1)), so the two lane halves
    // (rows 4 apart) write disjoint banks.
    __syncthreads();
    float* st = (float*)(wave == 0 ? As0 : wave == 1 ? As1 : wave == 2 ? Bs0 : Bs1);
    const double scale = p.scale_a[0] * p.scale_b[0];
    const bool vec = (p.N & 3) == 0 && ((uintptr_t)p.C & 15) == 0 && ((uintptr_t)p.R & 15) == 0 &&
                     ((uintptr_t)p.bias & 15) == 0;
    with_act(p.act, [&](auto act_c) {
        constexpr int ACT = decltype(act_c)::value;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
#pragma unroll
            for (int ii = 0; ii < 2; ++ii)
#pragma unroll
                for (int j = 0; j < TN; ++j)
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int lrow = ii * 32 + 8 * (r >> 2) + 4 * lh + (r & 3);
                        const int col = j * 32 + lr;
                        st[lrow * 128 + (col ^ (((lrow >> 2) & 1) << 5))] =
                            (float)((double)acc[2 * h + ii][j][r] * scale);
                    }
            // the wave reads back only what it wrote: LDS order within a wave
#pragma unroll 4
            for (int t = 0; t < 32; ++t) {
                const int idx = t * 64 + lane, lrow = idx >> 5, c4 = 4 * (idx & 31);
                const f32x4 v0 = *(const f32x4*)&st[lrow * 128 + (c4 ^ (((lrow >> 2) & 1) << 5))];
                const int row = m0 + wm * 128 + h * 64 + lrow, col = n0 + wn * 128 + c4;
                if (row >= p.M || col >= p.N) continue;
                const size_t o = (size_t)row * p.N + col;
                if (vec) {
                    f32x4 v = v0;
                    if (p.bias) v += *(const f32x4*)(p.bias + col);
#pragma unroll
                    for (int e = 0; e < 4; ++e) v[e] = act_fixed<ACT>(v[e]);
                    if (p.R) v += *(const f32x4*)(p.R + o);
                    *(f32x4*)(p.C + o) = v;
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        if (col + e >= p.N) break;
                        float v = v0[e];
                        if (p.bias) v += p.bias[col + e];
                        v = act_fixed<ACT>(v);
                        if (p.R) v += p.R[o + e];
                        p.C[o + e] = v;
                    }
                }
            }
        }
    });
}

unsigned grid_for(size_t work) {
    return (unsigned)std::max<size_t>(1, std::min<size_t>((work + kThreads - 1) / kThreads, 4096));
}

// Partial maxima of |x| into part (at most kMaxBlocks); returns their count.
int absmax_partials_launch(lancius_hip_ctx* ctx, float* part, const float* x, size_t n, int* parts) {
    const unsigned blocks = (unsigned)std::max<size_t>(1, std::min<size_t>((n + 8191) / 8192, kMaxBlocks));
    const int vec = ((uintptr_t)x & 15u) == 0;
    hipLaunchKernelGGL(absmax_partials, dim3(blocks), dim3(kThreads), 0, ctx->stream, part, x, n, vec);
    *parts = (int)blocks;
    return check_launch("absmax_partials");
}

size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

// k-tile of the int8 GEMMs: both operands are zero-padded in k to a
// multiple of it.
constexpr size_t kGemmBK = 128;

// B [K][N] int8 -> B^T [N][Kp] (the layout both int8 GEMM kernels read).
int pack_weight(lancius_hip_ctx* ctx, int8_t* bt, const int8_t* B, size_t K, size_t N) {
    const size_t Kp = align_up(K, kGemmBK);
    const int tiles_k = (int)(Kp / 128), tiles_n = (int)((N + 127) / 128);
    LANCIUS_REQUIRE((size_t)tiles_k * tiles_n < kMaxGridX, LANCIUS_HIP_ERR_SHAPE, "gemm_i8: B too large");
    const int bvec = N % 16 == 0 && ((uintptr_t)B & 15u) == 0;
    hipLaunchKernelGGL(transpose_i8, dim3((unsigned)(tiles_k * tiles_n)), dim3(kThreads), 0, ctx->stream, bt, B,
                       (int)K, (int)N, (int)Kp, tiles_n, bvec);
    return check_launch("transpose_i8");
}

int gemm_i8_check(size_t M, size_t K, size_t N, int act, double scale_b) {
    LANCIUS_REQUIRE(M > 0 && N > 0 && K > 0 && M < (1u << 30) && N < (1u << 30) && K < (1u << 30),
                    LANCIUS_HIP_ERR_SHAPE, "gemm_i8: shape M=%zu K=%zu N=%zu", M, K, N);
    LANCIUS_REQUIRE(act >= LANCIUS_HIP_ACT_NONE && act <= LANCIUS_HIP_ACT_TANH, LANCIUS_HIP_ERR_UNSUPPORTED,
                    "gemm_i8: activation %d", act);
    // scale_b is a host value; the kernel reads both scales from device memory
    LANCIUS_REQUIRE(scale_b >= 0.0, LANCIUS_HIP_ERR_SHAPE, "gemm_i8: negative scale");
    LANCIUS_REQUIRE(align_up(K, kGemmBK) * (M > N ? M : N) < ((size_t)1 << 36), LANCIUS_HIP_ERR_SHAPE,
                    "gemm_i8: operands too large");
    return 0;
}

// Workspace head: the two scales (doubles) and the absmax partials; A_q
// [M][Kp] starts at this offset.
size_t gemm_i8_a_offset() { return align_up(64 + kMaxBlocks * sizeof(float), 256); }

// Quantize A into the workspace, then the int8 product with B^T [N][Kp].
int gemm_i8_core(lancius_hip_ctx* ctx, char* ws, float* C, const float* A, const int8_t* bt, double scale_b,
                 size_t M, size_t K, size_t N, const float* bias, int act, const float* residual) {
    const size_t Kp = align_up(K, kGemmBK);
    double* scales = (double*)ws;
    float* part = (float*)(ws + 64);
    int8_t* aq = (int8_t*)(ws + gemm_i8_a_offset());
    int parts = 0;
    if (int rc = absmax_partials_launch(ctx, part, A, M * K, &parts)) return rc;
    // A_q [M][Kp]: row r holds quant(A[r][k]) for k < K, zeros after; the
    // kernel also stores scale_a (and scale_b) for the GEMM epilogue
    const int vec4 = K % 4 == 0 && ((uintptr_t)A & 15u) == 0;
    const size_t D = Kp / 4, rows_per = D >= (size_t)kThreads ? 1 : kThreads / D;
    const unsigned qblocks = (unsigned)std::min<size_t>((M + rows_per - 1) / rows_per, 2048);
    hipLaunchKernelGGL(quantize_rows_padded, dim3(qblocks), dim3(kThreads), 0, ctx->stream, aq, A, (const float*)part,
                       parts, scales, scale_b, M, (int)K, (int)Kp, vec4);
    if (int rc = check_launch("quantize_rows_padded")) return rc;
    I8Params p{};
    p.C = C;
    p.A = aq;
    p.B = bt;
    p.bias = bias;
    p.R = residual;
    p.scale_a = scales;
    p.scale_b = scales + 1;
    p.M = (int)M;
    p.N = (int)N;
    p.Kp = (int)Kp;
    p.act = act;
    // gemm_i8_direct (256 x 256 tiles, fewer bytes per MFMA) when they
    // still give every CU one and both operands are under 2 GiB, else
    // gemm_i8_mfma at 128 x 128 (more workgroups for small products; 64-bit
    // addressing)
    const bool fits31 = (M + 1) * Kp < ((size_t)1 << 31) - 16 && (N + 1) * Kp < ((size_t)1 << 31) - 16;
    const bool big = ((M + 255) / 256) * ((N + 255) / 256) >= 240 && fits31;
    const int BM = big ? 256 : 128, BN = BM;
    p.tiles_m = (uint32_t)((M + BM - 1) / BM);
    p.tiles_n = (uint32_t)((N + BN - 1) / BN);
    const size_t grid = (size_t)p.tiles_m * p.tiles_n;
    LANCIUS_REQUIRE(grid < kMaxGridX, LANCIUS_HIP_ERR_SHAPE, "gemm_i8: too many tiles");
    // the k-tile loads of gemm_i8_direct spread over three k-steps
    // (measured against one burst, one and two steps: kernel 67 -> 65 us)
    if (big)
        hipLaunchKernelGGL(gemm_i8_direct<3>, dim3((unsigned)grid), dim3(256), 0, ctx->stream, p);
    else
        hipLaunchKernelGGL((gemm_i8_mfma<128, 128, 2, 2, 128, false>), dim3((unsigned)grid), dim3(256), 0, ctx->stream,
                           p);
    return check_launch("gemm_i8_mfma");
}

}  // namespace
}  // namespace lancius

using namespace lancius;

extern "C" {

int lancius_hip_quantize_i8(lancius_hip_ctx* ctx, int8_t* q, double* scale, const float* x, size_t n) {
    LANCIUS_REQUIRE(ctx && q && scale && x, LANCIUS_HIP_ERR_NULL_PTR, "quantize_i8: NULL argument");
    if (int rc = bind_device(ctx)) return rc;
    void* ws = nullptr;
    if (int rc = workspace(ctx, kMaxBlocks * sizeof(float), &ws)) return rc;
    int parts = 0;
    if (int rc = absmax_partials_launch(ctx, (float*)ws, x, n, &parts)) return rc;
    // one workgroup at least: it stores the scale even for n == 0
    hipLaunchKernelGGL(quantize_flat, dim3(grid_for(n)), dim3(kThreads), 0, ctx->stream, q, x, (const float*)ws, parts,
                       scale, n);
    return check_launch("quantize_flat");
}

size_t lancius_hip_i8_packed_bytes(size_t K, size_t N) { return N * align_up(K, kGemmBK); }

int lancius_hip_i8_pack_weight(lancius_hip_ctx* ctx, int8_t* packed, const int8_t* B, size_t K, size_t N) {
    LANCIUS_REQUIRE(ctx && packed && B, LANCIUS_HIP_ERR_NULL_PTR, "i8_pack_weight: NULL argument");
    LANCIUS_REQUIRE(N > 0 && K > 0 && N < (1u << 30) && K < (1u << 30), LANCIUS_HIP_ERR_SHAPE,
                    "i8_pack_weight: shape K=%zu N=%zu", K, N);
    if (int rc = bind_device(ctx)) return rc;
    if (int rc = pack_weight(ctx, packed, B, K, N)) return rc;
    return ok();
}

int lancius_hip_gemm_i8p_f32(lancius_hip_ctx* ctx, float* C, const float* A, const int8_t* packed, double scale_b,
                             size_t M, size_t K, size_t N, const float* bias, int act, const float* residual) {
    LANCIUS_REQUIRE(ctx && C && A && packed, LANCIUS_HIP_ERR_NULL_PTR, "gemm_i8p: NULL argument");
    if (int rc = gemm_i8_check(M, K, N, act, scale_b)) return rc;
    if (int rc = bind_device(ctx)) return rc;
    const size_t Kp = align_up(K, kGemmBK);
    char* ws = nullptr;
    if (int rc = workspace(ctx, gemm_i8_a_offset() + M * Kp, (void**)&ws)) return rc;
    if (int rc = gemm_i8_core(ctx, ws, C, A, packed, scale_b, M, K, N, bias, act, residual)) return rc;
    return ok();
}

int lancius_hip_gemm_i8_f32(lancius_hip_ctx* ctx, float* C, const float* A, const int8_t* B, double scale_b,
                            size_t M, size_t K, size_t N, const float* bias, int act, const float* residual) {
    LANCIUS_REQUIRE(ctx && C && A && B, LANCIUS_HIP_ERR_NULL_PTR, "gemm_i8: NULL argument");
    if (int rc = gemm_i8_check(M, K, N, act, scale_b)) return rc;
    if (int rc = bind_device(ctx)) return rc;
    // workspace: scales | absmax partials | A_q [M][Kp] | B^T [N][Kp]
    const size_t Kp = align_up(K, kGemmBK);
    const size_t off_b = align_up(gemm_i8_a_offset() + M * Kp, 256);
    const size_t bytes = off_b + N * Kp;
    LANCIUS_REQUIRE(bytes < ((size_t)1 << 36), LANCIUS_HIP_ERR_SHAPE, "gemm_i8: operands too large");
    char* ws = nullptr;
    if (int rc = workspace(ctx, bytes, (void**)&ws)) return rc;
    int8_t* bt = (int8_t*)(ws + off_b);
    if (int rc = pack_weight(ctx, bt, B, K, N)) return rc;
    if (int rc = gemm_i8_core(ctx, ws, C, A, bt, scale_b, M, K, N, bias, act, residual)) return rc;
    return ok();
}

int lancius_hip_conv2d_i8_f32(lancius_hip_ctx* ctx, float* out, const float* in, const int8_t* w, double scale_w,
                              const float* bias, size_t N, size_t C_in, size_t H, size_t W, size_t C_out, size_t K_h,
                              size_t K_w, size_t stride, size_t pad, int act) {
    LANCIUS_REQUIRE(ctx && out && in && w, LANCIUS_HIP_ERR_NULL_PTR, "conv2d_i8: NULL argument");
    LANCIUS_REQUIRE(N && C_in && H && W && C_out && K_h && K_w && stride, LANCIUS_HIP_ERR_SHAPE,
                    "conv2d_i8: empty shape");
    LANCIUS_REQUIRE(H + 2 * pad >= K_h && W + 2 * pad >= K_w, LANCIUS_HIP_ERR_SHAPE,
                    "conv2d_i8: spatial dimensions underflow");
    LANCIUS_REQUIRE(act == LANCIUS_HIP_ACT_NONE || act == LANCIUS_HIP_ACT_RELU, LANCIUS_HIP_ERR_UNSUPPORTED,
                    "conv2d_i8: activation %d", act);
    const size_t Cp = align_up(C_in, 16);
    const size_t KHW = K_h * K_w;
    // conv_i8_direct when a block of at least 32 output channels of the
    // filter fits its LDS: TM = 4, 2 or 1 accumulators per wave (128, 64 or
    // 32 channels per workgroup), k padded to whole rings of k-steps.
    // Otherwise the LDS-staged implicit GEMM (gemm_i8_mfma, k-tiles of 64).
    const size_t xq_bytes = N * H * W * Cp;
    const size_t Kp_d = align_up(KHW * Cp, 32 * kConvI8Ring);
    const size_t ldw = Kp_d + ((Kp_d / 16) % 2 == 0 ? 16 : 0);
    int tm = C_out > 64 ? 4 : C_out > 32 ? 2 : 1;
    // (+32: the fragment reads one k-step past the end stay in the array)
    while (tm > 1 && 32 * tm * ldw + 32 > (size_t)kConvI8Lds) tm /= 2;
    const bool direct = 32 * tm * ldw + 32 <= (size_t)kConvI8Lds && Kp_d <= (size_t)kConvI8MaxKp && KHW <= 64 &&
                        xq_bytes < (size_t)0x7fffffc0;
    constexpr size_t BK = 64;
    const size_t Kp = direct ? Kp_d : align_up(KHW * Cp, BK);
    const size_t Ho = (H + 2 * pad - K_h) / stride + 1, Wo = (W + 2 * pad - K_w) / stride + 1;
    const size_t P = N * Ho * Wo;
    LANCIUS_REQUIRE(Kp < (1u << 30) && P < (1u << 31) && N * H * W * Cp < ((size_t)1 << 40) && C_out < (1u << 30),
                    LANCIUS_HIP_ERR_SHAPE, "conv2d_i8: shape too large");
    if (int rc = bind_device(ctx)) return rc;
    // workspace: scales | partials | weights [C_out][Kp] | NHWC activation (+16 B tail)
    const size_t off_part = 64, off_w = align_up(off_part + kMaxBlocks * sizeof(float), 256);
    const size_t off_x = align_up(off_w + C_out * Kp, 256);
    const size_t bytes = off_x + N * H * W * Cp + 16;
    char* ws = nullptr;
    if (int rc = workspace(ctx, bytes, (void**)&ws)) return rc;
    double* scales = (double*)ws;
    int8_t* wq = (int8_t*)(ws + off_w);
    int8_t* xq = (int8_t*)(ws + off_x);
    LANCIUS_REQUIRE(scale_w >= 0.0, LANCIUS_HIP_ERR_SHAPE, "conv2d_i8: negative scale");
    float* part = (float*)(ws + off_part);
    int parts = 0;
    if (int rc = absmax_partials_launch(ctx, part, in, N * C_in * H * W, &parts)) return rc;
    const int HW = (int)(H * W);
    const int tiles_p = (HW + 63) / 64, tiles_c = (int)((Cp + 63) / 64);
    LANCIUS_REQUIRE((size_t)N * tiles_p * tiles_c < kMaxGridX, LANCIUS_HIP_ERR_SHAPE, "conv2d_i8: input too large");
    // the activation quantized to NHWC and, in the same launch, the weights
    // re-laid k = (kh, kw, ci) and zero-padded to Kp
    ConvWeightsI8 cw{wq, w, (int)C_out, (int)C_in, (int)KHW, (int)Cp, (int)Kp, 0};
    cw.blocks = (int)std::min<size_t>(grid_for(C_out * Kp), 1024);
    const size_t qblocks = (size_t)N * tiles_p * tiles_c;
    LANCIUS_REQUIRE(qblocks + cw.blocks < kMaxGridX, LANCIUS_HIP_ERR_SHAPE, "conv2d_i8: input too large");
    const bool xvec = HW % 4 == 0 && ((uintptr_t)in & 15u) == 0 && C_in * (size_t)HW * sizeof(float) < ((size_t)1 << 31);
    hipLaunchKernelGGL(xvec ? quantize_nchw_to_nhwc<true> : quantize_nchw_to_nhwc<false>,
                       dim3((unsigned)(qblocks + cw.blocks)), dim3(kThreads), 0, ctx->stream, xq, in,
                       (const float*)part, parts, scales, scale_w, (int)N, (int)C_in, HW, (int)Cp, tiles_p, tiles_c,
                       cw);
    if (int rc = check_launch("quantize_nchw_to_nhwc")) return rc;
    constexpr int BM = 128, BN = 64;  // output channels x pixels per tile
    I8Params p{};
    p.C = out;
    p.A = wq;
    p.B = xq;
    p.bias = bias;
    p.scale_a = scales + 1;
    p.scale_b = scales;
    p.M = (int)C_out;
    p.N = (int)P;
    p.Kp = (int)Kp;
    p.act = act;
    p.H = (int)H;
    p.W = (int)W;
    p.Cp = (int)Cp;
    p.KW = (int)K_w;
    p.KHW = (int)KHW;
    p.stride = (int)stride;
    p.pad = (int)pad;
    p.Ho = (int)Ho;
    p.Wo = (int)Wo;
    p.HWo = (int)(Ho * Wo);
    p.out_channels = (int)C_out;
    if (direct) {
        // one workgroup per CU over the channel blocks (8 waves, each at
        // least one pixel tile of 32).  Tiles of 32 pixels (one B fragment
        // per k-step) measured 34.0 us per bench call against 35.0 for 64
        // (two fragments, half the filter reads per MFMA, fewer tiles to
        // overlap the stores of one with the MFMAs of the next).
        const int rows = 32 * tm;
        const size_t co_blocks = (C_out + rows - 1) / rows, tiles = (P + 31) / 32;
        const size_t wgs = std::max<size_t>(1, std::min<size_t>((tiles + 7) / 8, (size_t)cu_count(ctx) / co_blocks));
        LANCIUS_REQUIRE(co_blocks * wgs < kMaxGridX, LANCIUS_HIP_ERR_SHAPE, "conv2d_i8: too many channel blocks");
        void (*kern)(const I8Params, int, int, int) =
            tm == 4 ? conv_i8_direct<4, 1> : tm == 2 ? conv_i8_direct<2, 1> : conv_i8_direct<1, 1>;
        hipLaunchKernelGGL(kern, dim3((unsigned)(co_blocks * wgs)), dim3(kConvI8Threads), 0, ctx->stream, p, (int)co_blocks,
                           (int)ldw, (int)xq_bytes);
        return check_launch("conv_i8_direct");
    }
    p.tiles_m = (uint32_t)((C_out + BM - 1) / BM);
    p.tiles_n = (uint32_t)((P + BN - 1) / BN);
    const size_t grid = (size_t)p.tiles_m * p.tiles_n;
    LANCIUS_REQUIRE(grid < kMaxGridX, LANCIUS_HIP_ERR_SHAPE, "conv2d_i8: too many tiles");
    // 128 x 64 tiles, 4 workgroups per CU: the bench conv's 1568 tiles run
    // 40 us against 47 us for 784 tiles of 128 x 128 at 3 per CU (5 per CU
    // spilled and measured 41-43 us)
    hipLaunchKernelGGL((gemm_i8_mfma<BM, BN, 2, 2, (int)BK, true, 4>), dim3((unsigned)grid), dim3(kThreads), 0,
                       ctx->stream, p);
    return check_launch("conv2d_i8_mfma");
}

}  // extern "C"
