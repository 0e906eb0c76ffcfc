// Two dense layers and a row softmax in one launch, for the small-batch MLP
// graphs (B/examples/train_mnist.c:149-158 builds x -> MATMUL -> +b -> RELU ->
// MATMUL -> +b -> SOFTMAX with 64 rows).  At that size every kernel of the
// unfused chain (split-K GEMM, its reduce, GEMM, reduce, softmax) is a few
// microseconds of work behind a fixed launch cost, so the chain is bound by
// its number of dependent launches.  See mlp2_split and mlp2_tiles for the
// two designs.
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
    float* part;      // mlp2_split: [row_blocks][ks][16][16 tiles_n] partial h; mlp2_tiles: [tiles_n][M][N2] y shares
    float* hpart;     // mlp2_tiles with ks > 1: [row_blocks][tiles_n][ks][16 x 16] partial h tiles
    unsigned* counters;  // one arrival counter per row block (mlp2_tiles with ks > 1: then one per tile), zero between launches
    int M, K1, N1, N2, act1, act2, softmax;
    int tiles_n;  // 16-column tiles of h
    int ks;       // K ranges per tile
    int kchunk;   // K per range, a multiple of 4
};

// Limits of the chain (the small-batch regime it is for; lancius_hip.h):
// rows, outputs, hidden values M * N1, second-layer weights N1 * N2, and
// x and W1 each within kMaxOperand values (32-bit buffer offsets).
constexpr int kMaxRows = 64;
constexpr int kMaxOut = 64;
constexpr int kMaxH = 16384;
constexpr int kMaxW2 = 8192;
constexpr size_t kMaxOperand = size_t(1) << 28;
constexpr int kFR = 16;     // rows of h per workgroup
constexpr int kFC = 16;     // columns of h per workgroup
constexpr int kSplitMaxN1 = 256;  // mlp2_split: the reducer holds the block's whole h
constexpr int kMaxSplit = 4;      // K ranges per tile
constexpr int kSplitMaxTiles = 16;  // mlp2_split by default: at most 16 * kMaxSplit arrivals per row block
constexpr int kSplitMinK = 2048;    // and at least 256 KiB per workgroup of mlp2_tiles
constexpr int kTilesMinK = 128;     // mlp2_tiles: K per range (one MFMA trip of the four waves)
constexpr int kOut = 0x7ffffff0;  // a byte offset past the end of any operand: the load returns 0

// Every global read is a buffer load whose offset is pushed past the end of
// its operand where the element does not exist, so no load sits behind a
// branch: the launch is a few microseconds long, and per-load exec-mask
// branches cost as much as the loads themselves.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t operand(const float* base, size_t count) {
    // a null operand gets no records: every load from it returns 0
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), 0, base ? (int)(count * sizeof(float)) : 0,
                                             kBufferRsrcWord3);
}
__device__ __forceinline__ float load1(__amdgpu_buffer_rsrc_t r, unsigned off) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, 0));
}
// A buffer over `count` values at `base` (count <= 0 or a null base: no
// records).  Built from wave-uniform values it lives in scalar registers,
// and its range does the bounds checks of every load from it.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t range(const float* base, int count) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), 0,
                                             base && count > 0 ? count * (int)sizeof(float) : 0, kBufferRsrcWord3);
}
__device__ __forceinline__ f32x4 load4(__amdgpu_buffer_rsrc_t r, unsigned off) {
    return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0));
}

struct NoPrefetch {
    __device__ void operator()() const {}
};

// The 16 x 16 tile of x . W1 at rows m0.., columns n0.. over k in
// [kbeg, kend), one f32x4 of partial sums per wave (register r of lane l:
// row 4(l/16) + r, column l%16; the four waves' sums add up to the tile).
// The range is cut into blocks of 16 k and wave w takes a contiguous quarter
// of the blocks, so no operand is shared between waves and the loop has no
// workgroup barrier.  Per block, lane l = 16 q + i loads
//   x[m0 + i][k + 4q .. k + 4q + 3]        (one float4: the A operand of four
//                                          MFMAs, MFMA j taking k + 4q + j)
//   W1[k + l/4][n0 + 4(l%4) .. + 3]        (one float4: the block's 16 rows)
// and W1 goes through the wave's own 1 KB of LDS, rows permuted so that MFMA
// j's B operand, W1[k + 4q + j][n0 + i], is the 64 consecutive floats j*64
// + l: a conflict-free read, ordered after the write by the wave alone.  A
// group of G blocks is loaded at once (no load is conditional: past
// the range or the operand they read zeros past the end of their buffer,
// so the compiler's wait counts stay exact and block 0's MFMAs run while
// the later blocks arrive).  prefetch() issues right behind the first
// group's loads, so loads of its own share the trip to memory.
// VEC: K1 and N1 multiples of 4 (x and W1 rows hold whole float4s).
constexpr int kKB = 16;     // k per block
constexpr int kGroup = 16;  // blocks in flight per wave (the largest group)
constexpr int kSlot = kKB * kFC;  // one W1 block in LDS (floats)
constexpr int kFKC = 4 * kGroup * kKB;  // K that the four waves load in one group each

template <bool VEC, int G, class Prefetch>
__device__ __forceinline__ f32x4 hidden_tile(const ChainParams& p, float* wl, int m0, int n0, int kbeg, int kend,
                                             int wave, int lane, Prefetch prefetch) {
    const int li = lane & 15, lq = lane >> 4;
    const int M = p.M, K1 = p.K1, N1 = p.N1;
    const int nb = (kend - kbeg + kKB - 1) / kKB;
    const int b0 = wave * nb / 4, b1 = (wave + 1) * nb / 4;  // this wave's blocks
    const int kend_w = min(kend, kbeg + kKB * b1);          // and the end of their k
    const __amdgpu_buffer_rsrc_t xr = range(p.x, M * K1);
    const __amdgpu_buffer_rsrc_t wr = range(p.w1, kend_w * N1);  // W1 rows below the wave's end: zeros past it
    const bool row = m0 + li < M;
    const int c = n0 + 4 * (lane & 3);
    unsigned woff[VEC ? 1 : 4];
#pragma unroll
    for (int e = 0; e < (VEC ? 1 : 4); ++e)
        woff[e] = c + e < N1 ? ((unsigned)(lane >> 2) * (unsigned)N1 + (unsigned)(c + e)) * 4u : (unsigned)kOut;
    const int wpos = ((lane >> 2) & 3) * 64 + (lane >> 4) * 16 + 4 * (lane & 3);  // row l/4 permuted, column 4(l%4)
    f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
    f32x4 xv[G], wv[G];
    // block j of a group at g0: x at k = kbeg + 16 (g0 + j) + 4q, in range
    // while 16 j < lim (lim < 0 for rows past M); W1 rows 16 (g0 + j) on
    auto load_group = [&](int g0) {
        const int kq = kbeg + kKB * g0 + 4 * lq;
        const int lim = row ? kend_w - kq : -1;
        const unsigned xo = ((unsigned)(m0 + li) * (unsigned)K1 + (unsigned)kq) * 4u;
        const unsigned wstep = (unsigned)kKB * (unsigned)N1 * 4u;
        const unsigned wbase = (unsigned)(kbeg + kKB * g0) * (unsigned)N1 * 4u;
#pragma unroll
        for (int j = 0; j < G; ++j) {
            if constexpr (VEC) {
                xv[j] = load4(xr, (unsigned)pick(kKB * j < lim, (int)xo, kOut) + 64u * j);
                wv[j] = load4(wr, woff[0] + wbase + wstep * j);
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    xv[j][e] = load1(xr, (unsigned)pick(kKB * j + e < lim, (int)xo, kOut) + 64u * j + 4u * e);
                    wv[j][e] = load1(wr, woff[e] + wbase + wstep * j);
                }
            }
            __builtin_amdgcn_sched_barrier(0);  // issue in block order (block 0 lands first)
        }
    };
    auto run_group = [&](int g0) {
#pragma unroll
        for (int j = 0; j < G; ++j) {
            if (g0 + j >= b1) continue;  // uniform; no loads follow
            float* slot = wl + (j & 1) * kSlot;
            *(f32x4*)&slot[wpos] = wv[j];
            __builtin_amdgcn_wave_barrier();
            float b[4];
#pragma unroll
            for (int jj = 0; jj < 4; ++jj) b[jj] = slot[jj * 64 + lane];
#pragma unroll
            for (int jj = 0; jj < 4; ++jj) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(xv[j][jj], b[jj], acc, 0, 0, 0);
        }
    };
    // the first group, then prefetch() behind its loads (a K of up to kFKC
    // is one group per wave), then the rest
    load_group(b0);
    prefetch();
    __builtin_amdgcn_sched_barrier(0);  // the group's loads are all in flight before block 0's LDS write
    run_group(b0);
    for (int g0 = b0 + G; g0 < b1; g0 += G) {
        load_group(g0);
        __builtin_amdgcn_sched_barrier(0);
        run_group(g0);
    }
    return acc;
}

// Outputs of a 16-row block: row 4 w + g belongs to lanes 16 g .. 16 g + 15
// of wave w, and lane 16 g + c holds outputs c + 16 q, q < kOutPerLane
// (N2 <= 64), so every reduction over a row stays inside one DPP row of 16
// lanes and the four rows of a wave reduce together.
constexpr int kOutPerLane = kMaxOut / 16;

template <int kCtrl>
__device__ __forceinline__ int dpp_i(int v) {
    return __builtin_amdgcn_update_dpp(0, v, kCtrl, 0xf, 0xf, false);
}
template <int kCtrl>
__device__ __forceinline__ float dpp_f(float v) {
    return __builtin_bit_cast(float, dpp_i<kCtrl>(__builtin_bit_cast(int, v)));
}
// DPP controls: lane ^ 1 and lane ^ 2 within a quad, lane 7 - i within a
// half row of 8, lane 15 - i within a row of 16.  Once the quads agree, the
// half-row mirror pairs every lane with a lane of the other quad, and once
// the half rows agree the row mirror pairs it with the other half: both
// partners combine the same two values, so all 16 lanes end with identical
// bits.
constexpr int kQuadXor1 = 0xb1, kQuadXor2 = 0x4e, kHalfRowMirror = 0x141, kRowMirror = 0x140;

template <class Op>
__device__ __forceinline__ float row16(float v, Op op) {
    v = op(v, dpp_f<kQuadXor1>(v));
    v = op(v, dpp_f<kQuadXor2>(v));
    v = op(v, dpp_f<kHalfRowMirror>(v));
    return op(v, dpp_f<kRowMirror>(v));
}

// The first maximum of a row's values (the larger value, the smaller output
// index among equal ones): the same winner whichever of two lanes combines.
template <int kCtrl>
__device__ __forceinline__ void argmax_step(float& best, int& bi) {
    const float ob = dpp_f<kCtrl>(best);
    const int oi = dpp_i<kCtrl>(bi);
    const bool take = ob > best || (ob == best && oi < bi);
    best = take ? ob : best;
    bi = take ? oi : bi;
}

// The block's outputs from y (after b2 and act2; y[q] is output c + 16 q of
// this lane's row): the logits, or the reference's softmax
// (lancius_scheduler.c:284-294: m = the row's maximum, p = exp(y - m) /
// sum of exp(y - m)), then the first maximum of each row's p, as scanning
// with '>' from -1e9 finds it (B/examples/train_mnist.c:206-209): the
// largest p, the smallest output among equal ones, output 0 when no p
// exceeds -1e9.  Every lane runs the reductions (DPP reads no lane outside
// its row); only the stores are masked.  No LDS, no barrier.
__device__ __forceinline__ void finish_rows(const ChainParams& p, int m0, int wave, int lane,
                                            const float (&y)[kOutPerLane]) {
    const int N2 = p.N2, c = lane & 15;
    const int r = m0 + 4 * wave + (lane >> 4);
    const bool row_on = r < p.M;
    float* o = p.out + (size_t)r * N2;
    if (!p.softmax) {
#pragma unroll
        for (int q = 0; q < kOutPerLane; ++q)
            if (row_on && c + 16 * q < N2) o[c + 16 * q] = y[q];
        return;
    }
    // output groups q with 16 q >= N2 hold no output of any lane: skipped
    // (uniformly), so N2 <= 16 costs one exponential and one division
    float m = -INFINITY;
#pragma unroll
    for (int q = 0; q < kOutPerLane; ++q)
        if (16 * q < N2 && c + 16 * q < N2) m = fmaxf(m, y[q]);
    m = row16(m, [](float a, float b) { return fmaxf(a, b); });
    float e[kOutPerLane], s = 0.0f;
#pragma unroll
    for (int q = 0; q < kOutPerLane; ++q) {
        e[q] = 0.0f;
        if (16 * q >= N2) continue;
        if (c + 16 * q < N2) e[q] = expf(y[q] - m);
        s += e[q];
    }
    s = row16(s, [](float a, float b) { return a + b; });
    float best = -1e9f;
    int bi = 0;
#pragma unroll
    for (int q = 0; q < kOutPerLane; ++q) {
        if (16 * q >= N2) continue;
        const int j = c + 16 * q;
        const float prob = e[q] / s;
        if (row_on && j < N2) o[j] = prob;
        if (j < N2 && prob > best) {  // q ascending: the lane's first maximum
            best = prob;
            bi = j;
        }
    }
    if (!p.argmax) return;
    argmax_step<kQuadXor1>(best, bi);
    argmax_step<kQuadXor2>(best, bi);
    argmax_step<kHalfRowMirror>(best, bi);
    argmax_step<kRowMirror>(best, bi);
    if (row_on && c == 0) p.argmax[r] = bi;
}

// mlp2_split, for N1 <= kSplitMaxN1.  Workgroup (row block b of 16 rows,
// column tile t of 16 columns of h, K range q):
//  1. the tile's partial x[b] . W1[q range, t] (hidden_tile; the four waves'
//     sums added in wave order), stored for the row block's reducer;
//  2. the workgroup that arrives last at row block b's counter (of
//     tiles_n * ks) loads the block's partials together with W2, b1 and b2,
//     forms h = act1(sum of the ks partials in range order + b1) in LDS,
//     multiplies it by W2 with MFMAs (the waves split the output tiles, and
//     K where there are fewer than four output tiles, and their sums add in
//     wave order), adds b2, applies act2 and finishes the rows.
// The K split spreads the first layer, nearly all of the work and of the
// loaded bytes, over tiles_n * row_blocks * ks workgroups instead of
// tiles_n * row_blocks, and the second layer needs no hand-off of its own.
// It pays where there are few tiles and a long K (each workgroup of
// mlp2_tiles would stream 128 * K1 bytes): the reducer's loads bypass the
// caches (about 30 GB/s for one workgroup, measured) and arrivals at one
// counter serialise (about 45 ns each), so with many tiles (the
// 64 x 784 -> 256 MLP: 64 tiles, 256 arrivals) mlp2_tiles is faster (8.7
// against 13.1 us).  One hand-off between workgroups (through the point of
// coherence, kernels.hpp); every sum runs in a fixed order, so repeated
// calls give identical bits.
template <bool VEC>
__global__ void __launch_bounds__(256) mlp2_split(const ChainParams p) {
    // the waves' W1 slots, then the reducer's h and W2
    constexpr int kStage = kFR * (kSplitMaxN1 + 4) + kMaxW2;
    static_assert(kStage >= 4 * 2 * kSlot, "slots fit the staging area");
    __shared__ __attribute__((aligned(16))) float smem[kStage];
    __shared__ float red[4][kFR][kFC + 1];
    __shared__ float B2s[kMaxOut];
    __shared__ int s_flag;

    const int ks = p.ks, kq = (int)blockIdx.x % ks, rest = (int)blockIdx.x / ks;
    const int tn = rest % p.tiles_n, rb = rest / p.tiles_n;
    const int n0 = tn * kFC, m0 = rb * kFR;
    const int M = p.M, N1 = p.N1, N2 = p.N2;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int li = lane & 15, lq = lane >> 4;
    const int kbeg = kq * p.kchunk, kend = min(p.K1, kbeg + p.kchunk);

    const f32x4 acc = hidden_tile<VEC, kGroup>(p, smem + wave * 2 * kSlot, m0, n0, kbeg, kend, wave, lane, NoPrefetch{});
#pragma unroll
    for (int r = 0; r < 4; ++r) red[wave][4 * lq + r][li] = acc[r];
    __syncthreads();
    const int N1p = p.tiles_n * kFC;  // h columns, padded to the tiles
    const int blk = kFR * N1p;        // one range's partials of a block
    const __amdgpu_buffer_rsrc_t part = coherent_buffer(p.part, (size_t)(M + kFR - 1) / kFR * ks * blk * sizeof(float));
    {
        const int r = tid >> 4, c = tid & 15;  // 256 threads = 16 x 16
        const float v = ((red[0][r][c] + red[1][r][c]) + red[2][r][c]) + red[3][r][c];
        store_coherent(part, ((rb * ks + kq) * blk + r * N1p + n0 + c) * (int)sizeof(float), v);
    }
    if (!arrive_last(p.counters + rb, (unsigned)(p.tiles_n * ks), &s_flag)) return;
    reset_arrival(p.counters + rb);

    // The reducer.  Thread tid holds h elements e = 4 (tid + 256 g), g <
    // N1p / 64: row e / N1p, columns e % N1p .. +3.
    constexpr int kHG = kFR * kSplitMaxN1 / 4 / 256;  // float4 groups per thread
    constexpr int kW2T = kMaxW2 / 256;                // W2 values per thread
    f32x4 hp[kMaxSplit][kHG];
#pragma unroll
    for (int s = 0; s < kMaxSplit; ++s)
#pragma unroll
        for (int g = 0; g < kHG; ++g) {
            const int e = 4 * (tid + 256 * g);
            const bool in = s < ks && e < blk;
            hp[s][g] = load_coherent4(part, in ? ((rb * ks + s) * blk + e) * (int)sizeof(float) : kOut);
        }
    float w2v[kW2T];
    const __amdgpu_buffer_rsrc_t w2b = operand(p.w2, (size_t)N1 * N2);
#pragma unroll
    for (int u = 0; u < kW2T; ++u) {
        const int i = tid + 256 * u;
        w2v[u] = load1(w2b, i < N1 * N2 ? 4u * i : (unsigned)kOut);
    }
    const __amdgpu_buffer_rsrc_t b1b = operand(p.b1, (size_t)N1);
    f32x4 b1v[kHG];
#pragma unroll
    for (int g = 0; g < kHG; ++g) {
        const int e = 4 * (tid + 256 * g), c = e % N1p;
#pragma unroll
        for (int x = 0; x < 4; ++x) b1v[g][x] = load1(b1b, e < blk && c + x < N1 ? 4u * (c + x) : (unsigned)kOut);
    }
    const float b2r = load1(operand(p.b2, (size_t)N2), tid < N2 ? 4u * tid : (unsigned)kOut);

    // h and W2 in LDS (the staging area is free: every wave has passed the
    // arrival barrier).  Hs rows have pitch N1p + 4; W2s keeps W2's layout.
    const int ldh = N1p + 4;
    float* Hs = smem;
    float* W2s = smem + kFR * ldh;
    with_act(p.act1, [&](auto A) {
#pragma unroll
        for (int g = 0; g < kHG; ++g) {
            const int e = 4 * (tid + 256 * g);
            if (e >= blk) continue;
            const int r = e / N1p, c = e % N1p;
            f32x4 v = hp[0][g];
#pragma unroll
            for (int s = 1; s < kMaxSplit; ++s)
                if (s < ks) v += hp[s][g];
#pragma unroll
            for (int x = 0; x < 4; ++x) Hs[r * ldh + c + x] = act_fixed<decltype(A)::value>(v[x] + b1v[g][x]);
        }
    });
#pragma unroll
    for (int u = 0; u < kW2T; ++u) {
        const int i = tid + 256 * u;
        if (i < N1 * N2) W2s[i] = w2v[u];
    }
    if (tid < kMaxOut) B2s[tid] = b2r;
    __syncthreads();

    // y = h . W2: output tile t = w / parts of 16 outputs, K part w % parts
    const int ytiles = (N2 + 15) / 16;
    const int parts = ytiles == 1 ? 4 : ytiles == 2 ? 2 : 1;
    const int yt = wave / parts, part_k = wave % parts;
    const int steps = N1 / 4 + (N1 % 4 != 0);  // k-steps of 4 over N1
    const int per = (steps + parts - 1) / parts;
    f32x4 ya = f32x4{0.f, 0.f, 0.f, 0.f};
    if (yt < ytiles) {
        const int col = 16 * yt + li;
        const int s1 = min(steps, (part_k + 1) * per);
        for (int s = part_k * per; s < s1; s += 4) {
            // four steps' LDS reads ahead of their MFMAs (addresses past
            // N1 stay inside the staging area and are masked)
            float a[4], b[4];
#pragma unroll
            for (int x = 0; x < 4; ++x) {
                const int k = 4 * (s + x) + lq;
                const bool in = s + x < s1 && k < N1;
                a[x] = in ? Hs[li * ldh + k] : 0.0f;
                b[x] = in && col < N2 ? W2s[k * N2 + col] : 0.0f;
            }
#pragma unroll
            for (int x = 0; x < 4; ++x) ya = __builtin_amdgcn_mfma_f32_16x16x4f32(a[x], b[x], ya, 0, 0, 0);
        }
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) red[wave][4 * lq + r][li] = ya[r];
    __syncthreads();
    // y of this lane's row and outputs c + 16 q: the waves' K parts of the
    // output tile q added in wave order
    float y[kOutPerLane];
    {
        const int r = 4 * wave + lq;
#pragma unroll
        for (int q = 0; q < kOutPerLane; ++q) {
            y[q] = 0.0f;
            if (16 * q >= N2) continue;  // uniform
            const int j = li + 16 * q;
            float v = 0.0f;
            if (j < N2) {
                v = red[q * parts][r][li];
                for (int k = 1; k < parts; ++k) v += red[q * parts + k][r][li];
            }
            y[q] = apply_act(v + B2s[j], p.act2);
        }
    }
    finish_rows(p, m0, wave, lane, y);
}

// mlp2_tiles, for any N1 within the limits.  Workgroup (K range q of ks,
// column tile t of 16 columns of h, row block b of 16 rows):
//  1. the range's part of x[b] . W1[:, t] (hidden_tile; the four waves'
//     sums added in wave order); with ks > 1, stored, and the workgroup
//     that arrives last at tile (b, t)'s counter adds the ranges' parts in
//     range order;
//  2. h[b, t] = act1(that + b1[t]) and y_t = h[b, t] . W2[t rows, :], the
//     tile's share of the second layer, stored for the row block's reducer;
//  3. the workgroup that arrives last at row block b's counter adds the
//     tiles' shares in tile order, adds b2, applies act2 and finishes the
//     rows.
// The K ranges put ks workgroups on each tile, for a long K: a workgroup's
// loads arrive at about 80 GB/s after a first trip of over a microsecond,
// so a long K is faster spread over more CUs, at the price of one more
// hand-off (three more trips to memory).  Every sum runs in a fixed order,
// so repeated calls give identical bits.
template <bool VEC, int G>
__global__ void __launch_bounds__(256) mlp2_tiles(const ChainParams p) {
    __shared__ __attribute__((aligned(16))) float Wl[4][2 * kSlot];  // each wave's W1 slots
    __shared__ float red[4][kFR][kFC + 1];
    __shared__ float Hs[kFR][kFC + 1];
    __shared__ float W2s[kFC * kMaxOut];  // W2 rows of the tile, row pitch N2
    __shared__ float B2s[kMaxOut];
    __shared__ int s_flag;

    const int ks = p.ks, kq = (int)blockIdx.x % ks, tile = (int)blockIdx.x / ks;
    const int tn = tile % p.tiles_n, rb = tile / p.tiles_n;
    const int n0 = tn * kFC, m0 = rb * kFR;
    const int M = p.M, N1 = p.N1, N2 = p.N2;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int li = lane & 15, lq = lane >> 4;
    const int kbeg = kq * p.kchunk, kend = min(p.K1, kbeg + p.kchunk);

    // W2 rows n0.. (one contiguous run of kFC * N2 values), this thread's
    // b1 column and b2 output: loaded with the first K chunk, so the launch
    // makes one trip to memory for its inputs
    constexpr int kW2Per = kFC * kMaxOut / 256;
    float w2r[kW2Per], b1r = 0.0f, b2r = 0.0f;
    const f32x4 acc = hidden_tile<VEC, G>(p, Wl[wave], m0, n0, kbeg, kend, wave, lane, [&] {
        const int cols = min(kFC, N1 - n0);  // h columns of the tile
        const __amdgpu_buffer_rsrc_t w2b = range(p.w2 + (size_t)n0 * N2, cols * N2);  // its W2 rows
#pragma unroll
        for (int u = 0; u < kW2Per; ++u) w2r[u] = load1(w2b, 4u * tid + 1024u * u);
        b1r = load1(range(p.b1 + n0, cols), 4u * (tid & 15));
        b2r = load1(range(p.b2, N2), 4u * tid);
    });
#pragma unroll
    for (int r = 0; r < 4; ++r) red[wave][4 * lq + r][li] = acc[r];
#pragma unroll
    for (int u = 0; u < kW2Per; ++u) W2s[tid + 256 * u] = w2r[u];  // zeros past the tile's rows
    if (tid < kMaxOut) B2s[tid] = b2r;
    __syncthreads();
    {
        const int r = tid >> 4, c = tid & 15;  // 256 threads = 16 x 16
        float v = ((red[0][r][c] + red[1][r][c]) + red[2][r][c]) + red[3][r][c];
        if (ks > 1) {
            const int row_blocks = (M + kFR - 1) / kFR;
            const __amdgpu_buffer_rsrc_t hp =
                coherent_buffer(p.hpart, (size_t)row_blocks * p.tiles_n * ks * kFR * kFC * sizeof(float));
            store_coherent(hp, ((tile * ks + kq) * (kFR * kFC) + tid) * (int)sizeof(float), v);
            if (!arrive_last(p.counters + row_blocks + tile, (unsigned)ks, &s_flag)) return;
            reset_arrival(p.counters + row_blocks + tile);
            float t[kMaxSplit];
#pragma unroll
            for (int q = 0; q < kMaxSplit; ++q)
                t[q] = load_coherent(hp, q < ks ? ((tile * ks + q) * (kFR * kFC) + tid) * (int)sizeof(float) : kOut);
            v = t[0];
#pragma unroll
            for (int q = 1; q < kMaxSplit; ++q)
                if (q < ks) v += t[q];
        }
        float h = 0.0f;
        if (m0 + r < M && n0 + c < N1) h = apply_act(v + b1r, p.act1);
        Hs[r][c] = h;  // rows past M and columns past N1 hold 0
    }
    __syncthreads();
    // this tile's share of y for the lane's row and outputs c + 16 q
    const int MN2 = M * N2;
    const int r = 4 * wave + lq;  // of the block
    const bool row_on = m0 + r < M;
    const __amdgpu_buffer_rsrc_t ypart = coherent_buffer(p.part, (size_t)p.tiles_n * MN2 * sizeof(float));
#pragma unroll
    for (int q = 0; q < kOutPerLane; ++q) {
        if (16 * q >= N2) continue;  // uniform
        const int j = li + 16 * q;
        float a = 0.0f;
#pragma unroll
        for (int k = 0; k < kFC; ++k) a += Hs[r][k] * W2s[k * N2 + j];  // within W2s: j < 64
        store_coherent(ypart, row_on && j < N2 ? (tn * MN2 + (m0 + r) * N2 + j) * (int)sizeof(float) : kOut, a);
    }
    if (!arrive_last(p.counters + rb, (unsigned)p.tiles_n, &s_flag)) return;
    reset_arrival(p.counters + rb);

    // the block's rows: y = sum of the tiles' shares in tile order + b2
    // (loads past the last tile or outside the block fall outside the
    // buffer and return 0)
    constexpr int kChunk = 16;
    float y[kOutPerLane];
    int off[kOutPerLane];
#pragma unroll
    for (int q = 0; q < kOutPerLane; ++q) {
        const int j = li + 16 * q;
        y[q] = 0.0f;
        off[q] = row_on && j < N2 ? ((m0 + r) * N2 + j) * (int)sizeof(float) : kOut;
    }
    for (int t0 = 0; t0 < p.tiles_n; t0 += kChunk) {
        // every output group's loads of the chunk before any sum
        float t[kOutPerLane][kChunk];
#pragma unroll
        for (int q = 0; q < kOutPerLane; ++q) {
            if (16 * q >= N2) continue;  // uniform
#pragma unroll
            for (int c = 0; c < kChunk; ++c)
                t[q][c] = load_coherent(
                    ypart, off[q] != kOut && t0 + c < p.tiles_n ? off[q] + (t0 + c) * MN2 * (int)sizeof(float) : kOut);
        }
#pragma unroll
        for (int q = 0; q < kOutPerLane; ++q) {
            if (16 * q >= N2) continue;
#pragma unroll
            for (int c = 0; c < kChunk; ++c)
                if (t0 + c < p.tiles_n) y[q] = (t0 + c == 0) ? t[q][c] : y[q] + t[q][c];
        }
    }
#pragma unroll
    for (int q = 0; q < kOutPerLane; ++q)
        if (16 * q < N2) y[q] = apply_act(y[q] + B2s[li + 16 * q], p.act2);
    finish_rows(p, m0, wave, lane, y);
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
                        M * N1 <= (size_t)kMaxH && N1 * N2 <= (size_t)kMaxW2 && K1 * std::max(M, N1) <= kMaxOperand,
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
    const bool vec = K1 % 4 == 0 && N1 % 4 == 0 && ((uintptr_t)x & 15u) == 0 && ((uintptr_t)w1 & 15u) == 0;
    p.tiles_n = (int)((N1 + kFC - 1) / kFC);
    const size_t row_blocks = (M + kFR - 1) / kFR;
    const size_t tiles = row_blocks * (size_t)p.tiles_n;
    if (int rc = counters(ctx, row_blocks, &p.counters)) return rc;
    void* ws = nullptr;
    // mlp2_split for few tiles with a long K, mlp2_tiles otherwise
    if ((size_t)p.tiles_n * kFC <= (size_t)kSplitMaxN1 && tiles <= kSplitMaxTiles && K1 >= kSplitMinK) {
        // K ranges of at least 64 that bring the grid to about one
        // workgroup per CU
        int ks = (int)std::max<size_t>(1, std::min<size_t>(kMaxSplit, 256 / tiles));
        while (ks > 1 && K1 < (size_t)ks * 64) --ks;
        p.kchunk = (int)((K1 + ks - 1) / ks + 3) / 4 * 4;
        p.ks = (int)((K1 + p.kchunk - 1) / p.kchunk);
        if (int rc = workspace(ctx, row_blocks * p.ks * kFR * p.tiles_n * kFC * sizeof(float), &ws)) return rc;
        p.part = (float*)ws;
        hipLaunchKernelGGL(vec ? mlp2_split<true> : mlp2_split<false>, dim3((unsigned)(tiles * p.ks)), dim3(256), 0,
                           ctx->stream, p);
        if (int rc = check_launch("mlp2_split")) return rc;
        return ok();
    }
    // For K beyond one staged chunk, K ranges of at least kTilesMinK that
    // bring the grid to about one workgroup per CU (measured, 64 rows, 256
    // hidden: K 784 is fastest whole, 8.2 against 8.5 us with four ranges;
    // K 1500 and 4096 split four ways, 10.9 -> 9.1 and 17.9 -> 10.6 us)
    int ks = K1 <= (size_t)kFKC ? 1 : (int)std::max<size_t>(1, std::min<size_t>(kMaxSplit, 256 / tiles));
    ks = std::max(1, std::min(ks, kMaxSplit));
    while (ks > 1 && K1 < (size_t)ks * kTilesMinK) --ks;
    p.kchunk = (int)((K1 + ks - 1) / ks + 3) / 4 * 4;
    p.ks = (int)((K1 + p.kchunk - 1) / p.kchunk);
    const size_t ybytes = ((size_t)p.tiles_n * M * N2 * sizeof(float) + 255) & ~(size_t)255;
    const size_t hbytes = p.ks > 1 ? tiles * p.ks * kFR * kFC * sizeof(float) : 0;
    if (p.ks > 1)
        if (int rc = counters(ctx, row_blocks + tiles, &p.counters)) return rc;
    if (int rc = workspace(ctx, ybytes + hbytes, &ws)) return rc;
    p.part = (float*)ws;
    p.hpart = p.ks > 1 ? (float*)((char*)ws + ybytes) : nullptr;
    // the group size that leaves the fewest empty blocks in a wave's last
    // group (empty blocks still cost their loads: at K 784, 13 blocks per
    // wave, groups of 13 measured 7.63 against 7.84 us with groups of 16)
    const int per_wave = ((p.kchunk + kKB - 1) / kKB + 3) / 4;  // most blocks of a wave
    int group = kGroup;
    for (int cand : {kGroup, 13, 8}) {
        auto waste = [&](int g) { return (per_wave + g - 1) / g * g - per_wave; };
        if (waste(cand) < waste(group)) group = cand;
    }
    auto kernel = group == 13 ? (vec ? mlp2_tiles<true, 13> : mlp2_tiles<false, 13>)
                  : group == 8 ? (vec ? mlp2_tiles<true, 8> : mlp2_tiles<false, 8>)
                               : (vec ? mlp2_tiles<true, kGroup> : mlp2_tiles<false, kGroup>);
    hipLaunchKernelGGL(kernel, dim3((unsigned)(tiles * p.ks)), dim3(256), 0, ctx->stream, p);
    if (int rc = check_launch("mlp2_tiles")) return rc;
    return ok();
}
