// Fused scaled-dot-product attention, fp32, on the gfx950 matrix cores.
//
// Semantics: bleeding/v11A1/src/math/lancius_kernels.c:278-332 (kernel_attention):
// for each query row i and head h, s_j = (q_i . k_j) * scale, keys j > i get
// -1e9 when causal (:307), online softmax with running max m and sum l
// (:309-319), out = o / l (:322-327).  Tensors are [batch, S, H, D] row-major;
// the reference is batch = 1, causal, scale = 1/sqrt(D) (:284, :293).
// Skipping key blocks that lie entirely above the diagonal is exactly the
// reference's masking: exp(-1e9 - m) is 0 and the correction factor is 1.
//
// Fast kernel (D = 32, 64, 96, 128), "transposed" formulation so that every
// softmax statistic is lane-local:
//   S^T[key][q] = K . Q^T    MFMA A = K tile (LDS), B = Q^T (registers)
//   O^T[d][q]  += V^T . P^T  MFMA A = V^T (LDS),    B = P^T (the S^T registers)
// With v_mfma_f32_32x32x2_f32, lane l holds query l%32 in both accumulators,
// so the row max / sum need one swap with lane l^32 and the O rescale is a
// per-lane multiply.  The P^T accumulator is fed back as the B operand without
// any data movement: step s of the PV product uses register s, whose key index
// 8*(s/4) + 4*(l/32) + s%4 is matched by the V^T operand address.
// The score tile never leaves registers.  Each workgroup (4 waves) owns 128
// queries of one (batch, head); K/V blocks of 64 keys (32 for D > 64) are
// double-buffered in LDS and shared by the 4 waves.  Q is pre-scaled by
// scale*log2(e) so the exponentials are exp2.
#include <math.h>

#include <algorithm>

#include "common.hpp"
#include "kernels.hpp"

namespace lancius {
namespace {

struct AttnParams {
    float* O[LANCIUS_HIP_MAX_GROUP];
    const float* Q[LANCIUS_HIP_MAX_GROUP];
    const float* K[LANCIUS_HIP_MAX_GROUP];
    const float* V[LANCIUS_HIP_MAX_GROUP];
    int batch;  // batches per group entry
    int S, H, D;   // queries per sequence, query heads, head dim
    int Skv, Hkv;  // keys per sequence, K/V heads (query head h reads K/V head h / (H / Hkv))
    int causal;    // query i sees keys j <= i + (Skv - S)
    float qscale;  // scale * log2(e)
    int q_tiles;
    int pair_tiles;  // causal grid small enough to be resident at once (see attention_mfma)
    int Z;         // count * batch independent problems
};

constexpr int kBQ = 128;   // queries per workgroup (32 per wave)

// 2^x as the one v_exp_f32.  exp2f adds a range fix-up (compare, select,
// add, select, ldexp: five more instructions) that only changes results
// below 2^-126; the softmax exponents here are <= 0 and a probability under
// 2^-126 does not move a sum that is >= 1.
__device__ __forceinline__ float exp2_raw(float x) { return __builtin_amdgcn_exp2f(x); }

// D = head dim (a multiple of 32, at most 128); BKV = keys per LDS block
// (64 for D <= 64, 32 above, so the K/V blocks of two workgroups fit a
// CU's LDS).  KS = key split: with KS = 2 the workgroup has 8 waves, and
// each 32-query block is owned by two waves, one taking its even key
// blocks and one its odd ones (each step stages one block for each); at
// the end the odd-block waves hand their (O, m, l) to the even-block waves
// through LDS, which merge them in that fixed order.  That puts four waves on a SIMD instead of two
// (at most 128 registers each), each with half the key blocks.  KS = 1:
// 4 waves, every key block.  BQ = queries per workgroup (128, or 64 for
// grids too small to fill the CUs with 128-query tiles).  The staged keys are double-buffered in LDS, or
// with SINGLE held in one buffer (K and V each refilled once every wave is
// done with them: two more barriers a step, half the LDS, so three 4-wave
// workgroups fit a CU).
template <int D, int BKV, int KS, int BQ = kBQ, bool SINGLE = false>
__global__ void __launch_bounds__(BQ / 32 * KS * 64, SINGLE ? 3 : 2 * KS) attention_mfma(const AttnParams p) {
    static_assert(D % 32 == 0 && D <= 128 && BKV % 32 == 0, "tile shape");
    static_assert(KS == 1 || KS == 2, "key split");
    constexpr int NQB = BQ / 32;         // 32-query blocks of the workgroup
    constexpr int NT = NQB * KS * 64;
    constexpr int LDK = D + 1;  // K rows padded: lanes read 32 different keys at one d
    // V rows: lanes read 32 consecutive d of one key, the two lane halves
    // keys 4 rows apart; D + 8 puts those 32 banks apart (64 banks).
    constexpr int LDV = D + 8;
    constexpr int QSTEPS = D / 2;        // K.Q^T MFMA steps (2 d each)
    constexpr int DB = D / 32;           // O^T d-blocks
    constexpr int SB = BKV / 32;         // S^T key blocks
    constexpr int KB = KS * BKV;         // keys staged per step
    constexpr int NKV = KB * D / (4 * NT);  // float4 of each K/V step per thread
    static_assert(NKV * 4 * NT == KB * D, "staging covers the step");
    constexpr int NBUF = SINGLE ? 1 : 2;
    constexpr int K_FLOATS = NBUF * KB * LDK, V_FLOATS = NBUF * KB * LDV;
    constexpr int PER = 16 * DB + 2;  // a lane's hand-off: O^T registers, m, l
    constexpr int RED_FLOATS = KS > 1 ? NQB * PER * 64 : 0;
    constexpr int SMEM = K_FLOATS + V_FLOATS > RED_FLOATS ? K_FLOATS + V_FLOATS : RED_FLOATS;
    static_assert(K_FLOATS % 4 == 0, "V rows 16-byte aligned");
    __shared__ __attribute__((aligned(16))) float smem[SMEM];
    float(*Ks)[KB][LDK] = reinterpret_cast<float(*)[KB][LDK]>(smem);
    float(*Vs)[KB][LDV] = reinterpret_cast<float(*)[KB][LDV]>(smem + K_FLOATS);

    // 1-D task order, query-tile major: consecutive ids (which the hardware
    // deals round-robin to the 8 XCDs) are different (batch, head) problems of
    // the same query tile.  Every XCD therefore gets the same mix of causal
    // tile lengths (longest first) and always the same (batch, head) subset,
    // whose K/V stay in its L2.
    const int hz = p.H * p.Z;
    const int task = (int)blockIdx.x;
    const int t_rank = task / hz;
    const int rem = task - t_rank * hz;
    const int z = rem / p.H;
    const int h = rem - z * p.H;
    const int g = z / p.batch, b = z % p.batch;
    // Causal order: longest tiles first.  When every workgroup is resident at
    // once (p.pair_tiles: two or three per CU), ranks T/2.. run the shortest tiles
    // first instead, so the workgroup that shares a CU with the k-th longest
    // tile gets the k-th shortest one (tile T-1-k with tile k).
    const int half_t = p.q_tiles / 2;
    const int qt = !p.causal                        ? t_rank
                   : (p.pair_tiles && t_rank >= p.q_tiles - half_t) ? t_rank - (p.q_tiles - half_t)
                                                                      : p.q_tiles - 1 - t_rank;
    // The short tile of a resident causal pair waits about 3.4 us (127 x 64
    // clocks at 2.4 GHz) before its first loads, so the long tiles, which
    // bound the launch, get the HBM to themselves for their Q and first K/V
    // blocks: S=512 causal 48.7 / 49.8 -> 47.9 / 47.4 us, B4 S=1024 causal
    // 85.1 / 84.7 -> 82.8 / 82.8 us (one box, builds alternated; half and
    // twice the wait measured no better).
    if constexpr (KS == 2 && BQ == kBQ)
        if (p.causal && p.pair_tiles && t_rank >= p.q_tiles - half_t) __builtin_amdgcn_s_sleep(127);
    const int S = p.S, H = p.H, Skv = p.Skv;
    const int off = Skv - S;  // causal offset of the query rows into the key sequence
    const int hk = h / (H / p.Hkv);
    const size_t row_stride = (size_t)H * D;
    const size_t kv_stride = (size_t)p.Hkv * D;
    const size_t base = ((size_t)b * S * H + h) * D;
    const size_t kv_base = ((size_t)b * Skv * p.Hkv + hk) * D;
    const float* __restrict__ Qg = p.Q[g] + base;
    const float* __restrict__ Kg = p.K[g] + kv_base;
    const float* __restrict__ Vg = p.V[g] + kv_base;
    float* __restrict__ Og = p.O[g] + base;

    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    // KS = 2: wave w < NQB takes the even key blocks of query block w, wave
    // w + NQB the odd key blocks of query block NQB - 1 - w.  The hardware
    // puts waves w and w + 4 of a workgroup on the same SIMD (measured on
    // MI355X from the HW_ID register), so with 128 queries each SIMD gets
    // half of a short and half of a long query block of a causal tile, and
    // the four SIMDs of the CU finish together.
    const int kh = wave / NQB;                      // key parity
    const int wq = kh ? 2 * NQB - 1 - wave : wave;  // query block of the wave
    const int lq = lane & 31, lk = lane >> 5;
    const int q0 = qt * BQ;
    const int qw0 = q0 + wq * 32;     // first query of this wave
    const int q = qw0 + lq;           // this lane's query
    const bool q_valid = q < S;

    // Q^T operand: step s uses d = s + (D/2)*(l/32); the K operand uses the same d.
    float qf[QSTEPS];
    if (q_valid) {
        const f32x4* src = (const f32x4*)(Qg + (size_t)q * row_stride + QSTEPS * lk);
#pragma unroll
        for (int i = 0; i < QSTEPS / 4; ++i) {
            const f32x4 v = src[i];
            qf[4 * i + 0] = v.x * p.qscale;
            qf[4 * i + 1] = v.y * p.qscale;
            qf[4 * i + 2] = v.z * p.qscale;
            qf[4 * i + 3] = v.w * p.qscale;
        }
    } else {
#pragma unroll
        for (int i = 0; i < QSTEPS; ++i) qf[i] = 0.0f;
    }

    // Key range of this workgroup, in blocks of BKV and steps of KS blocks.
    const int kv_end = p.causal ? max(0, min(Skv, q0 + BQ + off)) : Skv;
    const int nblocks = (kv_end + BKV - 1) / BKV;
    const int nsteps = (nblocks + KS - 1) / KS;

    // K/V global -> register staging: KB keys x D floats per tensor, as
    // buffer loads (the sequence's K and V rows, under 2 GiB: the host
    // checks) whose keys past Skv use a past-the-end offset and read 0; a
    // guarded plain load would be a branch per load.
    constexpr int kOut = 0x7ffffff0;
    const int kv_bytes = ((Skv - 1) * (int)kv_stride + D) * (int)sizeof(float);
    const __amdgpu_buffer_rsrc_t kbuf =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(Kg), 0, kv_bytes, kBufferRsrcWord3);
    const __amdgpu_buffer_rsrc_t vbuf =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(Vg), 0, kv_bytes, kBufferRsrcWord3);
    f32x4 kreg[NKV], vreg[NKV];
    // SINGLE: K and V staged in separate halves of the step (K loaded at the
    // step's start and stored once every wave has formed its scores, V
    // loaded then and stored at the step's end), so only one tensor's
    // registers are live at a time
    auto load_one = [&](const __amdgpu_buffer_rsrc_t& buf, f32x4* reg, int k0) {
#pragma unroll
        for (int i = 0; i < NKV; ++i) {
            const int idx = tid + NT * i;
            const int key = idx / (D / 4), dq = idx % (D / 4);
            const int gk = k0 + key;
            const int off = pick(gk < Skv, (gk * (int)kv_stride + 4 * dq) * (int)sizeof(float), kOut);
            reg[i] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(buf, off, 0, 0));
        }
        __builtin_amdgcn_sched_barrier(0);
    };
    auto store_k = [&](int buf) {
#pragma unroll
        for (int i = 0; i < NKV; ++i) {
            const int idx = tid + NT * i;
            const int key = idx / (D / 4), dq = idx % (D / 4);
            float* kd = &Ks[buf][key][4 * dq];
            kd[0] = kreg[i].x;
            kd[1] = kreg[i].y;
            kd[2] = kreg[i].z;
            kd[3] = kreg[i].w;
        }
    };
    auto store_v = [&](int buf) {
#pragma unroll
        for (int i = 0; i < NKV; ++i) {
            const int idx = tid + NT * i;
            const int key = idx / (D / 4), dq = idx % (D / 4);
            *(f32x4*)&Vs[buf][key][4 * dq] = kreg[i];
        }
    };
    auto load_kv = [&](int k0) {
#pragma unroll
        for (int i = 0; i < NKV; ++i) {
            const int idx = tid + NT * i;
            const int key = idx / (D / 4), dq = idx % (D / 4);
            const int gk = k0 + key;
            const int off = pick(gk < Skv, (gk * (int)kv_stride + 4 * dq) * (int)sizeof(float), kOut);
            kreg[i] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(kbuf, off, 0, 0));
            vreg[i] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(vbuf, off, 0, 0));
        }
        // the loads leave before the block's MFMAs (the scheduler would
        // otherwise move them down to the LDS stores they feed)
        __builtin_amdgcn_sched_barrier(0);
    };
    auto store_kv = [&](int buf) {
#pragma unroll
        for (int i = 0; i < NKV; ++i) {
            const int idx = tid + NT * i;
            const int key = idx / (D / 4), dq = idx % (D / 4);
            float* kd = &Ks[buf][key][4 * dq];
            kd[0] = kreg[i].x;
            kd[1] = kreg[i].y;
            kd[2] = kreg[i].z;
            kd[3] = kreg[i].w;
            *(f32x4*)&Vs[buf][key][4 * dq] = vreg[i];
        }
    };

    f32x16 o_acc[DB];  // O^T, d-block db holds d = 32*db .. 32*db + 31
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) o_acc[db][r] = 0.0f;
    float m_run = -1e30f;  // running max (log2 domain); finite so exp2 never sees inf - inf
    float l_part = 0.0f;   // this lane's share of the running sum

    if (nsteps > 0) {
        load_kv(0);
        store_kv(0);
    }
    __syncthreads();

    for (int st = 0; st < nsteps; ++st) {
        const int cur = SINGLE ? 0 : st & 1;
        const bool more = st + 1 < nsteps;
        if constexpr (SINGLE) {
            if (more) load_one(kbuf, kreg, (st + 1) * KB);
        } else {
            if (more) load_kv((st + 1) * KB);
        }
        const int blk = st * KS + kh;  // this wave's block
        const int kb = blk * BKV;
        const int kl = kh * BKV;       // its first row in the staged keys

        // Wave-uniform skip of blocks past the keys or entirely above this
        // wave's diagonal.
        const bool active = blk < nblocks && (!p.causal || kb <= qw0 + 31 + off);
        f32x16 s_acc[SB];
        if (active) {
#pragma unroll
            for (int sb = 0; sb < SB; ++sb)
#pragma unroll
                for (int r = 0; r < 16; ++r) s_acc[sb][r] = 0.0f;
#pragma unroll
            for (int s = 0; s < QSTEPS; ++s) {
                const int d = s + QSTEPS * lk;
#pragma unroll
                for (int sb = 0; sb < SB; ++sb)
                    s_acc[sb] = __builtin_amdgcn_mfma_f32_32x32x2f32(Ks[cur][kl + 32 * sb + lq][d], qf[s], s_acc[sb],
                                                                     0, 0, 0);
            }
        }
        if constexpr (SINGLE) {
            __syncthreads();  // every wave has read the staged K
            if (more) {
                store_k(0);
                load_one(vbuf, kreg, (st + 1) * KB);
            }
        }
        if (active) {
            // Register r of lane l holds key kb + 32*sb + 8*(r/4) + 4*(l/32) + r%4.
            const bool need_mask = (p.causal && kb + BKV - 1 > qw0 + off) || (kb + BKV > Skv);
            if (need_mask) {
                // the lane's last visible key, relative to its first in the block
                const int lim = min(Skv - 1, p.causal ? q + off : Skv - 1) - (kb + 4 * lk);
#pragma unroll
                for (int sb = 0; sb < SB; ++sb)
#pragma unroll
                    for (int r = 0; r < 16; ++r)
                        if (32 * sb + 8 * (r >> 2) + (r & 3) > lim) s_acc[sb][r] = -INFINITY;
            }
            float mx = -INFINITY;
#pragma unroll
            for (int sb = 0; sb < SB; ++sb)
#pragma unroll
                for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s_acc[sb][r]);
            mx = fmaxf(mx, __shfl_xor(mx, 32));
            const float m_new = fmaxf(m_run, mx);
            // The running sums are rescaled only when some lane's maximum
            // grew: otherwise every lane's factor is 2^0 = 1 and skipping
            // the multiplies changes no bit (after the first blocks of a
            // row the maximum rarely moves).
            float corr = 1.0f;
            if (__builtin_amdgcn_ballot_w64(m_new > m_run) != 0) {
                corr = exp2_raw(m_run - m_new);
#pragma unroll
                for (int db = 0; db < DB; ++db)
#pragma unroll
                    for (int r = 0; r < 16; ++r) o_acc[db][r] *= corr;
            }
            m_run = m_new;
            float psum = 0.0f;
#pragma unroll
            for (int sb = 0; sb < SB; ++sb)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const float pv = exp2_raw(s_acc[sb][r] - m_new);
                    s_acc[sb][r] = pv;
                    psum += pv;
                }
            l_part = l_part * corr + psum;
            // O^T += V^T . P^T over the BKV keys of this block.
#pragma unroll
            for (int sb = 0; sb < SB; ++sb)
#pragma unroll
                for (int s = 0; s < 16; ++s) {
                    const int key = 32 * sb + 8 * (s >> 2) + 4 * lk + (s & 3);
#pragma unroll
                    for (int db = 0; db < DB; ++db)
                        o_acc[db] = __builtin_amdgcn_mfma_f32_32x32x2f32(Vs[cur][kl + key][32 * db + lq],
                                                                         s_acc[sb][s], o_acc[db], 0, 0, 0);
                }
        }
        if constexpr (SINGLE) {
            if (more) {
                __syncthreads();  // every wave has read the staged V
                store_v(0);
            }
        } else {
            if (more) store_kv(cur ^ 1);
        }
        __syncthreads();
    }

    if constexpr (KS > 1) {
        // Waves of the odd blocks hand their O^T, m and l to the waves of the
        // even blocks (same queries, same lanes), which merge them:
        // m = max(m0, m1), O = O0 2^(m0 - m) + O1 2^(m1 - m), l likewise.
        // The loop's last barrier has retired every read of the staged keys.
        float* red = smem + wq * PER * 64 + lane;  // [wq][PER][64 lanes]
        if (kh == 1) {
#pragma unroll
            for (int db = 0; db < DB; ++db)
#pragma unroll
                for (int r = 0; r < 16; ++r) red[(16 * db + r) * 64] = o_acc[db][r];
            red[16 * DB * 64] = m_run;
            red[(16 * DB + 1) * 64] = l_part;
        }
        __syncthreads();
        if (kh == 1) return;
        const float m1 = red[16 * DB * 64], l1 = red[(16 * DB + 1) * 64];
        const float m = fmaxf(m_run, m1);
        const float c0 = exp2f(m_run - m), c1 = exp2f(m1 - m);
        l_part = l_part * c0 + l1 * c1;
#pragma unroll
        for (int db = 0; db < DB; ++db)
#pragma unroll
            for (int r = 0; r < 16; ++r) o_acc[db][r] = o_acc[db][r] * c0 + red[(16 * db + r) * 64] * c1;
    }

    const float l_tot = l_part + __shfl_xor(l_part, 32);
    if (!q_valid) return;
    const float inv_l = 1.0f / l_tot;
    float* dst = Og + (size_t)q * row_stride;
    // O^T register r of lane l: d = 32*db + 8*(r/4) + 4*(l/32) + r%4.
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            f32x4 o;
            o.x = o_acc[db][4 * j + 0] * inv_l;
            o.y = o_acc[db][4 * j + 1] * inv_l;
            o.z = o_acc[db][4 * j + 2] * inv_l;
            o.w = o_acc[db][4 * j + 3] * inv_l;
            *(f32x4*)(dst + 32 * db + 8 * j + 4 * lk) = o;
        }
}

// Head dims the MFMA kernel does not take (not a multiple of 32, or above
// 128) and operands that are not 16-byte aligned: one thread per (query
// row, head), the reference's online loop in fp32.  Up to DMAX values the
// output row is accumulated in registers and written once; beyond that
// (DMAX = 0) the output row in memory is the accumulator.
template <int DMAX>
__global__ void __launch_bounds__(256) attention_rowwise(const AttnParams p) {
    const size_t rows = (size_t)p.S * p.H;
    const size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= rows) return;
    const int z = blockIdx.z;
    const int g = z / p.batch, b = z % p.batch;
    const int i = (int)(t / p.H), h = (int)(t % p.H);
    const int D = p.D;
    const size_t rs = (size_t)p.H * D;
    const size_t rkv = (size_t)p.Hkv * D;
    const size_t base = (size_t)b * p.S * rs + (size_t)h * D;
    const size_t kv_base = (size_t)b * p.Skv * rkv + (size_t)(h / (p.H / p.Hkv)) * D;
    const float* q = p.Q[g] + base + (size_t)i * rs;
    const float* K = p.K[g] + kv_base;
    const float* V = p.V[g] + kv_base;
    float* o = p.O[g] + base + (size_t)i * rs;
    float m = -1e30f, l = 0.0f;
    const int jend = p.causal ? min(p.Skv, max(0, i + 1 + p.Skv - p.S)) : p.Skv;
    if constexpr (DMAX > 0) {
        float acc[DMAX];
#pragma unroll
        for (int d = 0; d < DMAX; ++d) acc[d] = 0.0f;
        for (int j = 0; j < jend; ++j) {
            const float* k = K + (size_t)j * rkv;
            float s = 0.0f;
            for (int d = 0; d < D; ++d) s += q[d] * k[d];
            s *= p.qscale;
            const float m_new = fmaxf(m, s);
            const float c = exp2f(m - m_new);
            const float pj = exp2f(s - m_new);
            l = l * c + pj;
            const float* v = V + (size_t)j * rkv;
#pragma unroll
            for (int d = 0; d < DMAX; ++d)
                if (d < D) acc[d] = acc[d] * c + pj * v[d];
            m = m_new;
        }
        const float inv = l > 0.0f ? 1.0f / l : 0.0f;
#pragma unroll
        for (int d = 0; d < DMAX; ++d)
            if (d < D) o[d] = acc[d] * inv;
    } else {
        for (int d = 0; d < D; ++d) o[d] = 0.0f;
        for (int j = 0; j < jend; ++j) {
            const float* k = K + (size_t)j * rkv;
            float s = 0.0f;
            for (int d = 0; d < D; ++d) s += q[d] * k[d];
            s *= p.qscale;
            const float m_new = fmaxf(m, s);
            const float c = exp2f(m - m_new);
            const float pj = exp2f(s - m_new);
            l = l * c + pj;
            const float* v = V + (size_t)j * rkv;
            for (int d = 0; d < D; ++d) o[d] = o[d] * c + pj * v[d];
            m = m_new;
        }
        const float inv = l > 0.0f ? 1.0f / l : 0.0f;
        for (int d = 0; d < D; ++d) o[d] *= inv;
    }
}

// ---- decode: one query token per sequence against a K/V cache --------------
//
// HBM-bound: every cached key and value is read once, so the kernel streams
// K and V straight from HBM into registers and keeps the VALU work under the
// read time.
//  * workgroup (sequence b, K/V head hk, split s, head chunk c) owns keys
//    [s*chunk, min((s+1)*chunk, len_b)) and query heads c*GT .. c*GT+GT-1 of
//    the G = Hq/Hkv heads that share hk (one K/V read serves the chunk);
//  * 16 lanes own one key row: lane l16 holds NV of its D values (float4
//    pieces d = 4*l16 + 64*j when D % 4 == 0 and the pointers are 16-byte
//    aligned, else d = l16 + 16*i), so a key row is one coalesced 256/512-byte
//    read; a wave runs 4 such key streams, the workgroup 16;
//  * each stream takes UNR keys per step (stream t reads keys base + 16u + t),
//    with the next step's rows loading into a second register buffer, forms
//    the scores with a DPP sum over its 16 lanes and keeps its own online
//    softmax (m, l, o) per head in the log2 domain;
//  * the 16 streams merge in a fixed order (xor butterfly over the 4 streams
//    of a wave, then the 4 waves in order through LDS), so results do not
//    depend on timing; one split writes the normalised output directly; with
//    more, each split writes its (o, m, l) partial through the point of
//    coherence and the workgroup that arrives last at its (sequence, K/V
//    head, head chunk) counter merges the splits in split order (one launch:
//    a separate merge kernel cost 8.6 us of launch and latency, the hand-off
//    about 2 us at the end of the last ranges).
// kernel_attention_kv_cache (lancius_kernels.c:338-379) is batch = 1,
// Hq = Hkv, no mask, scale 1/sqrt(D).
struct DecodeParams {
    float* out;             // [B][Hq][D]
    const float* q;         // [B][Hq][D]
    const float* k;         // [B][Skv][Hkv][D]
    const float* v;
    const int32_t* lens;    // per-sequence cache length (<= Skv) or null
    float* part;            // [B*Hkv][splits][G][D + 2]
    unsigned* counters;     // one arrival counter per (sequence, K/V head, head chunk), zero between launches
    int B, Skv, Hq, Hkv, D, G;
    int splits, chunk, hchunks;
    float qscale;           // softmax scale * log2(e)
};

constexpr int kDecMaxD = 128;

constexpr int kDecOut = 0x7ffffff0;  // a byte offset past the end of any operand: the load returns 0

// This lane's NV values of the row at byte offset `row` of buffer r; values
// past D come from a past-the-end offset (0) instead of a branch around the
// load.
template <int NV, bool VEC>
__device__ __forceinline__ void load_piece(__amdgpu_buffer_rsrc_t r, int row, int l16, int D, float (&x)[NV]) {
    if constexpr (VEC) {
#pragma unroll
        for (int j = 0; j < NV / 4; ++j) {
            const int d = 4 * l16 + 64 * j;
            const f32x4 t = __builtin_bit_cast(
                f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, pick(d < D, row + 4 * d, kDecOut), 0, 0));
            x[4 * j] = t.x;
            x[4 * j + 1] = t.y;
            x[4 * j + 2] = t.z;
            x[4 * j + 3] = t.w;
        }
    } else {
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int d = l16 + 16 * i;
            x[i] = __builtin_bit_cast(float,
                                      __builtin_amdgcn_raw_buffer_load_b32(r, pick(d < D, row + 4 * d, kDecOut), 0, 0));
        }
    }
}

// Sum over the 16 lanes of a row with DPP moves (xor 1, xor 2 in the quad,
// then half-row and row mirrors, which pair each lane with one of the other
// half once the halves are uniform); every lane of the row gets the same sum.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, false));
}

__device__ __forceinline__ float row_sum16(float x) {
    x += dpp_mov<0xB1>(x);   // quad_perm [1,0,3,2]
    x += dpp_mov<0x4E>(x);   // quad_perm [2,3,0,1]
    x += dpp_mov<0x141>(x);  // row_half_mirror
    x += dpp_mov<0x140>(x);  // row_mirror
    return x;
}

template <int NV, bool VEC>
__device__ __forceinline__ int piece_d(int l16, int i) {
    if constexpr (VEC) return 4 * l16 + 64 * (i / 4) + (i & 3);
    else return l16 + 16 * i;
}

// (m, l, o) <- merge of itself and (m2, l2, o2); m = -inf means empty.
template <int NV>
__device__ __forceinline__ void merge_state(float& m, float& l, float (&o)[NV], float m2, float l2,
                                            const float (&o2)[NV]) {
    const float mn = fmaxf(m, m2);
    const float a = m > -INFINITY ? exp2f(m - mn) : 0.0f;
    const float c = m2 > -INFINITY ? exp2f(m2 - mn) : 0.0f;
    l = l * a + l2 * c;
#pragma unroll
    for (int i = 0; i < NV; ++i) o[i] = o[i] * a + o2[i] * c;
    m = mn;
}

template <int NV, bool VEC, int GT, int UNR>
__global__ void __launch_bounds__(256) attention_decode(const DecodeParams p) {
    __shared__ float red[4][GT][kDecMaxD + 2];
    __shared__ int s_flag;
    // XCD-aware order: consecutive workgroups go to different XCDs, so logical
    // ids are dealt out in contiguous runs per XCD (the head chunks of one
    // key range then share that XCD's L2).
    const int n = gridDim.x, id = blockIdx.x;
    const int full = n & ~7;
    const int lid = id < full ? (id & 7) * (full >> 3) + (id >> 3) : id;
    const int hc = lid % p.hchunks;
    const int rest = lid / p.hchunks;
    const int split = rest % p.splits;
    const int bh = rest / p.splits;
    const int b = bh / p.Hkv, hk = bh - b * p.Hkv;
    const int D = p.D, G = p.G;
    const int len = p.lens ? min(max(p.lens[b], 0), p.Skv) : p.Skv;
    const int k0 = split * p.chunk, k1 = min(len, k0 + p.chunk);
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int l16 = lane & 15, stream = wave * 4 + (lane >> 4);
    const int kv_row = p.Hkv * D;
    // K and V rows of this key range as buffers (the host keeps a range
    // under 1 GiB); key k is at byte (k - k0) * kv_row * 4
    const size_t kv0 = ((size_t)b * p.Skv + k0) * kv_row + (size_t)hk * D;
    const int kv_bytes = ((max(k1 - k0, 1) - 1) * kv_row + D) * (int)sizeof(float);
    const __amdgpu_buffer_rsrc_t kr_buf =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(p.k + kv0), 0, kv_bytes, kBufferRsrcWord3);
    const __amdgpu_buffer_rsrc_t vr_buf =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(p.v + kv0), 0, kv_bytes, kBufferRsrcWord3);
    const int h0 = hc * GT;
    const __amdgpu_buffer_rsrc_t q_buf = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(p.q + ((size_t)b * p.Hq + (size_t)hk * G + h0) * D), 0,
        min(GT, G - h0) * D * (int)sizeof(float), kBufferRsrcWord3);

    float qv[GT][NV], o[GT][NV], m[GT], l[GT];
#pragma unroll
    for (int h = 0; h < GT; ++h) {
        if (h0 + h < G) {
            load_piece<NV, VEC>(q_buf, h * D * (int)sizeof(float), l16, D, qv[h]);
        } else {
#pragma unroll
            for (int i = 0; i < NV; ++i) qv[h][i] = 0.0f;
        }
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            qv[h][i] *= p.qscale;
            o[h][i] = 0.0f;
        }
        m[h] = -INFINITY;
        l[h] = 0.0f;
    }

    // keys past the range re-read the last row (no branch, so every load
    // stays ahead of the arithmetic) and are masked
    auto fetch = [&](int base, float (&kr)[UNR][NV], float (&vr)[UNR][NV], bool (&valid)[UNR]) {
#pragma unroll
        for (int u = 0; u < UNR; ++u) {
            const int key = base + 16 * u + stream;
            valid[u] = key < k1;
            const int row = ((valid[u] ? key : k1 - 1) - k0) * kv_row * (int)sizeof(float);
            load_piece<NV, VEC>(kr_buf, row, l16, D, kr[u]);
            load_piece<NV, VEC>(vr_buf, row, l16, D, vr[u]);
        }
    };
    auto consume = [&](const float (&kr)[UNR][NV], const float (&vr)[UNR][NV], const bool (&valid)[UNR]) {
#pragma unroll
        for (int h = 0; h < GT; ++h) {
            float sc[UNR];
            float mx = -INFINITY;
#pragma unroll
            for (int u = 0; u < UNR; ++u) {
                float acc = 0.0f;
#pragma unroll
                for (int i = 0; i < NV; ++i) acc += qv[h][i] * kr[u][i];
                acc = row_sum16(acc);
                sc[u] = valid[u] ? acc : -INFINITY;
                mx = fmaxf(mx, sc[u]);
            }
            // branch-free: while the stream has seen no key, m = mn = -inf,
            // corr = 0 and every p = 0, so (o, l) stay 0.  The exponents are
            // <= 0, so the bare v_exp_f32 serves (see exp2_raw): decode
            // B16 x 4096 keys 105.9 -> 104.7 us, same results at the tested
            // shapes
            const float mn = fmaxf(m[h], mx);
            const float corr = m[h] > -INFINITY ? exp2_raw(m[h] - mn) : 0.0f;
            float ps = 0.0f;
#pragma unroll
            for (int i = 0; i < NV; ++i) o[h][i] *= corr;
#pragma unroll
            for (int u = 0; u < UNR; ++u) {
                const float pu = valid[u] ? exp2_raw(sc[u] - mn) : 0.0f;
                ps += pu;
#pragma unroll
                for (int i = 0; i < NV; ++i) o[h][i] += pu * vr[u][i];
            }
            l[h] = l[h] * corr + ps;
            m[h] = mn;
        }
    };
    // two register buffers: the next step's rows are in flight while the
    // current step's arithmetic runs
    float ka[UNR][NV], va[UNR][NV], kn[UNR][NV], vn[UNR][NV];
    bool oka[UNR], okn[UNR];
    constexpr int kStep = 16 * UNR;
    int base = k0;
    if (base < k1) fetch(base, ka, va, oka);
    while (base < k1) {
        if (base + kStep < k1) fetch(base + kStep, kn, vn, okn);
        consume(ka, va, oka);
        base += kStep;
        if (base >= k1) break;
        if (base + kStep < k1) fetch(base + kStep, ka, va, oka);
        consume(kn, vn, okn);
        base += kStep;
    }

    // merge the 4 streams of each wave, then the 4 waves in order
#pragma unroll
    for (int h = 0; h < GT; ++h) {
#pragma unroll
        for (int off = 16; off <= 32; off <<= 1) {
            float o2[NV];
#pragma unroll
            for (int i = 0; i < NV; ++i) o2[i] = __shfl_xor(o[h][i], off);
            const float m2 = __shfl_xor(m[h], off), l2 = __shfl_xor(l[h], off);
            merge_state<NV>(m[h], l[h], o[h], m2, l2, o2);
        }
        if (lane < 16) {
#pragma unroll
            for (int i = 0; i < NV; ++i) {
                const int d = piece_d<NV, VEC>(l16, i);
                if (d < D) red[wave][h][d] = o[h][i];
            }
            if (lane == 0) {
                red[wave][h][kDecMaxD] = m[h];
                red[wave][h][kDecMaxD + 1] = l[h];
            }
        }
    }
    __syncthreads();
    const int nh = min(GT, G - h0);
    const size_t part_floats = (size_t)p.B * p.Hkv * p.splits * G * (D + 2);
    const __amdgpu_buffer_rsrc_t part = coherent_buffer(p.part, p.splits > 1 ? part_floats * sizeof(float) : 0);
    for (int idx = tid; idx < nh * D; idx += 256) {
        const int h = idx / D, d = idx - (idx / D) * D;
        float mm = -INFINITY;
#pragma unroll
        for (int w = 0; w < 4; ++w) mm = fmaxf(mm, red[w][h][kDecMaxD]);
        float ll = 0.0f, oo = 0.0f;
        if (mm > -INFINITY) {
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                const float mw = red[w][h][kDecMaxD];
                const float a = mw > -INFINITY ? exp2f(mw - mm) : 0.0f;
                ll += red[w][h][kDecMaxD + 1] * a;
                oo += red[w][h][d] * a;
            }
        }
        const int hq = hk * G + h0 + h;
        if (p.splits == 1) {
            p.out[((size_t)b * p.Hq + hq) * D + d] = ll > 0.0f ? oo / ll : 0.0f;
        } else {
            const int pr = (int)((((size_t)bh * p.splits + split) * G + h0 + h) * (D + 2));
            store_coherent(part, (pr + d) * (int)sizeof(float), oo);
            if (d == 0) {
                store_coherent(part, (pr + D) * (int)sizeof(float), mm);
                store_coherent(part, (pr + D + 1) * (int)sizeof(float), ll);
            }
        }
    }
    if (p.splits == 1) return;
    unsigned* ctr = p.counters + (size_t)bh * p.hchunks + hc;
    if (!arrive_last(ctr, (unsigned)p.splits, &s_flag)) return;
    reset_arrival(ctr);
    // out = sum_s o_s 2^(m_s - m) / sum_s l_s 2^(m_s - m), m = max_s m_s, the
    // splits in order; a sequence with no keys gets zeros
    const int sstride = G * (D + 2);
    for (int idx = tid; idx < nh * D; idx += 256) {
        const int h = idx / D, d = idx - (idx / D) * D;
        const int base = (int)((((size_t)bh * p.splits) * G + h0 + h) * (D + 2));
        float m = -INFINITY;
        for (int sp = 0; sp < p.splits; ++sp)
            m = fmaxf(m, load_coherent(part, (base + sp * sstride + D) * (int)sizeof(float)));
        float l = 0.0f, acc = 0.0f;
        for (int sp = 0; sp < p.splits; ++sp) {
            const float ms = load_coherent(part, (base + sp * sstride + D) * (int)sizeof(float));
            if (ms > -INFINITY) {
                const float w = exp2f(ms - m);
                l += load_coherent(part, (base + sp * sstride + D + 1) * (int)sizeof(float)) * w;
                acc += load_coherent(part, (base + sp * sstride + d) * (int)sizeof(float)) * w;
            }
        }
        const float inv = l > 0.0f ? 1.0f / l : 0.0f;
        p.out[((size_t)b * p.Hq + hk * G + h0 + h) * D + d] = acc * inv;
    }
}

template <int NV, bool VEC>
void launch_decode(const DecodeParams& p, unsigned grid, hipStream_t stream, int gt) {
    switch (gt) {
        case 1: hipLaunchKernelGGL((attention_decode<NV, VEC, 1, 4>), dim3(grid), dim3(256), 0, stream, p); break;
        case 2: hipLaunchKernelGGL((attention_decode<NV, VEC, 2, 4>), dim3(grid), dim3(256), 0, stream, p); break;
        case 4: hipLaunchKernelGGL((attention_decode<NV, VEC, 4, 4>), dim3(grid), dim3(256), 0, stream, p); break;
        default: hipLaunchKernelGGL((attention_decode<NV, VEC, 8, 2>), dim3(grid), dim3(256), 0, stream, p); break;
    }
}

bool aligned16(const void* ptr) { return ((uintptr_t)ptr & 15u) == 0; }

int attention_dispatch(lancius_hip_ctx* ctx, size_t count, float* const* O, const float* const* Q,
                       const float* const* K, const float* const* V, size_t batch, size_t S, size_t H, size_t D,
                       int causal, float scale, size_t Skv = 0, size_t Hkv = 0) {
    if (Skv == 0) Skv = S;
    if (Hkv == 0) Hkv = H;
    LANCIUS_REQUIRE(ctx && O && Q && K && V, LANCIUS_HIP_ERR_NULL_PTR, "attention: NULL argument");
    LANCIUS_REQUIRE(count >= 1 && count <= LANCIUS_HIP_MAX_GROUP, LANCIUS_HIP_ERR_SHAPE,
                    "attention: group count %zu", count);
    LANCIUS_REQUIRE(batch >= 1 && S >= 1 && H >= 1 && D >= 1, LANCIUS_HIP_ERR_SHAPE,
                    "attention: empty shape batch=%zu S=%zu H=%zu D=%zu", batch, S, H, D);
    LANCIUS_REQUIRE(S < (1u << 24) && Skv < (1u << 24) && H < 65536 && D <= 4096 && count * batch < 65536,
                    LANCIUS_HIP_ERR_SHAPE, "attention: shape too large");
    LANCIUS_REQUIRE(Hkv >= 1 && H % Hkv == 0, LANCIUS_HIP_ERR_SHAPE,
                    "attention: %zu query heads do not group over %zu K/V heads", H, Hkv);
    LANCIUS_REQUIRE(!causal || Skv >= S, LANCIUS_HIP_ERR_SHAPE,
                    "attention: causal with %zu keys for %zu queries", Skv, S);
    if (int rc = bind_device(ctx)) return rc;
    AttnParams p{};
    bool vec = true;
    for (size_t g = 0; g < count; ++g) {
        LANCIUS_REQUIRE(O[g] && Q[g] && K[g] && V[g], LANCIUS_HIP_ERR_NULL_PTR, "attention: NULL operand %zu", g);
        p.O[g] = O[g];
        p.Q[g] = Q[g];
        p.K[g] = K[g];
        p.V[g] = V[g];
        vec = vec && aligned16(O[g]) && aligned16(Q[g]) && aligned16(K[g]) && aligned16(V[g]);
    }
    p.batch = (int)batch;
    p.S = (int)S;
    p.H = (int)H;
    p.D = (int)D;
    p.Skv = (int)Skv;
    p.Hkv = (int)Hkv;
    p.causal = causal ? 1 : 0;
    p.qscale = scale * 1.4426950408889634f;  // log2(e)
    const unsigned z = (unsigned)(count * batch);
    p.Z = (int)z;
    // the MFMA kernel addresses a sequence's K and V rows with 32-bit buffer offsets
    if (vec && D % 32 == 0 && D <= 128 && Skv * Hkv * D * sizeof(float) < ((size_t)1 << 31) - 64) {
        // D = 64 grids of at most three 64-query tiles per CU: 4-wave
        // workgroups with one LDS buffer, three resident per CU, where the
        // 128-query grid leaves CUs idle or half-loaded.  Measured against
        // the 128-query kernel (one box, builds alternated), causal: B1 H16
        // S=512 39.3 -> 26.3 us, B2 H8 S=256 21.9 -> 15.5 us, B8 H16 S=256
        // 22.9 -> 18.7 us, S=384 37.5 -> 33.5 us, B4 H16 S=768 69.5 ->
        // 56.5 us; non-causal: B1 H16 S=512 41.2 -> 26.3 us, S=1024 76 ->
        // 48 us, B4 H16 S=768 108.5 -> 86.6 us.  Non-causal grids whose
        // 128-query tiles give every CU the same count keep them (B2 S=1024
        // 77.4 -> 80, B1 S=2048 147.5 -> 153 us, B8 S=256 even).  At four
        // tiles per CU (B8 S=512, B4 S=1024) it does not fit (three
        // workgroups a CU by registers).
        {
            const size_t cus = (size_t)cu_count(ctx);
            const size_t qt64 = (S + 63) / 64, t64 = qt64 * H * z;
            const size_t t128 = (S + kBQ - 1) / kBQ * H * z;
            if (D == 64 && t64 <= 3 * cus && (causal || t128 % cus != 0)) {
                p.q_tiles = (int)qt64;
                p.pair_tiles = causal ? 1 : 0;
                hipLaunchKernelGGL((attention_mfma<64, 32, 2, 64, true>), dim3((unsigned)t64), dim3(256), 0, ctx->stream, p);
                if (int rc = check_launch("attention_mfma")) return rc;
                return ok();
            }
        }
        p.q_tiles = (int)((S + kBQ - 1) / kBQ);
        const size_t tasks = (size_t)p.q_tiles * H * z;
        LANCIUS_REQUIRE(tasks < kMaxGridX, LANCIUS_HIP_ERR_SHAPE, "attention: too many tiles");
        p.pair_tiles = causal && tasks <= 2 * (size_t)cu_count(ctx);
        const dim3 grid((unsigned)tasks);
        // D = 64 runs the key split (KS = 2, 32-key blocks, four waves a
        // SIMD), measured against one wave per query block (64-key blocks,
        // two waves a SIMD): B8 H16 S512 causal 55.7 -> 50.9 us, S2048
        // causal 0.611 -> 0.585 ms, non-causal 1.136 -> 1.113 ms, B4 S1024
        // causal 94.1 -> 89.2 us.  At D = 32 it measured slower (S2048
        // causal 0.328 -> 0.337 ms); D = 96 and 128 do not fit four waves'
        // registers.
        switch (D) {
            case 32: hipLaunchKernelGGL((attention_mfma<32, 64, 1>), grid, dim3(256), 0, ctx->stream, p); break;
            case 64: hipLaunchKernelGGL((attention_mfma<64, 32, 2>), grid, dim3(512), 0, ctx->stream, p); break;
            case 96: hipLaunchKernelGGL((attention_mfma<96, 32, 1>), grid, dim3(256), 0, ctx->stream, p); break;
            default: hipLaunchKernelGGL((attention_mfma<128, 32, 1>), grid, dim3(256), 0, ctx->stream, p); break;
        }
        if (int rc = check_launch("attention_mfma")) return rc;
    } else {
        const dim3 grid(ceil_div(S * H, 256), 1, z);
        if (D <= 32)
            hipLaunchKernelGGL(attention_rowwise<32>, grid, dim3(256), 0, ctx->stream, p);
        else if (D <= 128)
            hipLaunchKernelGGL(attention_rowwise<128>, grid, dim3(256), 0, ctx->stream, p);
        else
            hipLaunchKernelGGL(attention_rowwise<0>, grid, dim3(256), 0, ctx->stream, p);
        if (int rc = check_launch("attention_rowwise")) return rc;
    }
    return ok();
}

}  // namespace
}  // namespace lancius

using namespace lancius;

extern "C" {

int lancius_hip_attention_f32(lancius_hip_ctx* ctx, float* out, const float* q, const float* k, const float* v,
                              size_t batch, size_t S, size_t H, size_t D, int causal, float scale) {
    float* o1[1] = {out};
    const float* q1[1] = {q};
    const float* k1[1] = {k};
    const float* v1[1] = {v};
    return attention_dispatch(ctx, 1, o1, q1, k1, v1, batch, S, H, D, causal, scale);
}

int lancius_hip_attention_grouped_f32(lancius_hip_ctx* ctx, size_t count, float* const* out, const float* const* q,
                                      const float* const* k, const float* const* v, size_t S, size_t H, size_t D,
                                      int causal, float scale) {
    return attention_dispatch(ctx, count, out, q, k, v, 1, S, H, D, causal, scale);
}

int lancius_hip_attention_gqa_f32(lancius_hip_ctx* ctx, float* out, const float* q, const float* k, const float* v,
                                  size_t batch, size_t S_q, size_t S_kv, size_t H_q, size_t H_kv, size_t D,
                                  int causal, float scale) {
    LANCIUS_REQUIRE(S_kv >= 1 && H_kv >= 1, LANCIUS_HIP_ERR_SHAPE, "attention_gqa: S_kv=%zu H_kv=%zu", S_kv, H_kv);
    float* o1[1] = {out};
    const float* q1[1] = {q};
    const float* k1[1] = {k};
    const float* v1[1] = {v};
    return attention_dispatch(ctx, 1, o1, q1, k1, v1, batch, S_q, H_q, D, causal, scale, S_kv, H_kv);
}

int lancius_hip_attention_decode_f32(lancius_hip_ctx* ctx, float* out, const float* q, const float* k_cache,
                                     const float* v_cache, const int32_t* kv_lens, size_t batch, size_t S_kv,
                                     size_t H_q, size_t H_kv, size_t D, float scale) {
    LANCIUS_REQUIRE(ctx && out && q && k_cache && v_cache, LANCIUS_HIP_ERR_NULL_PTR, "attention_decode: NULL argument");
    LANCIUS_REQUIRE(batch >= 1 && H_q >= 1 && H_kv >= 1 && D >= 1 && H_q % H_kv == 0, LANCIUS_HIP_ERR_SHAPE,
                    "attention_decode: batch=%zu H_q=%zu H_kv=%zu D=%zu", batch, H_q, H_kv, D);
    LANCIUS_REQUIRE(D <= kDecMaxD && S_kv >= 1 && S_kv < (1u << 30) && H_q < 65536, LANCIUS_HIP_ERR_SHAPE,
                    "attention_decode: D=%zu (<= %d), S_kv=%zu or H_q=%zu unsupported", D, kDecMaxD, S_kv, H_q);
    if (int rc = bind_device(ctx)) return rc;
    DecodeParams p{};
    p.out = out;
    p.q = q;
    p.k = k_cache;
    p.v = v_cache;
    p.lens = kv_lens;
    p.B = (int)batch;
    p.Skv = (int)S_kv;
    p.Hq = (int)H_q;
    p.Hkv = (int)H_kv;
    p.D = (int)D;
    p.G = (int)(H_q / H_kv);
    p.qscale = scale * 1.4426950408889634f;  // log2(e)
    const int gt = p.G <= 1 ? 1 : p.G <= 2 ? 2 : p.G <= 4 ? 4 : 8;
    const size_t hchunks = ((size_t)p.G + gt - 1) / gt;
    // about 2 workgroups per CU in all (longer key ranges beat more
    // workgroups here), each split >= 256 keys
    const size_t seqs = batch * H_kv;
    const size_t tasks = seqs * hchunks;
    size_t splits = std::max<size_t>(1, std::min<size_t>((512 + tasks - 1) / tasks, (S_kv + 255) / 256));
    // a key range's K and V rows are addressed with 32-bit buffer offsets:
    // at most 1 GiB per range
    const size_t max_chunk = std::max<size_t>(1, ((size_t)1 << 30) / (H_kv * D * sizeof(float)));
    splits = std::max(splits, (S_kv + max_chunk - 1) / max_chunk);
    const size_t chunk = (S_kv + splits - 1) / splits;
    splits = (S_kv + chunk - 1) / chunk;
    LANCIUS_REQUIRE(tasks * splits < kMaxGridX, LANCIUS_HIP_ERR_SHAPE, "attention_decode: too many heads");
    p.splits = (int)splits;
    p.chunk = (int)chunk;
    p.hchunks = (int)hchunks;
    if (splits > 1) {
        const size_t part_bytes = seqs * splits * p.G * (D + 2) * sizeof(float);
        LANCIUS_REQUIRE(part_bytes < ((size_t)1 << 31), LANCIUS_HIP_ERR_SHAPE,
                        "attention_decode: %zu bytes of split partials (32-bit offsets)", part_bytes);
        void* ws = nullptr;
        if (int rc = workspace(ctx, part_bytes, &ws)) return rc;
        p.part = (float*)ws;
        if (int rc = counters(ctx, tasks, &p.counters)) return rc;
    }
    const bool vec = D % 4 == 0 && aligned16(q) && aligned16(k_cache) && aligned16(v_cache);
    const unsigned grid = (unsigned)(tasks * splits);
    if (vec && D > 64) launch_decode<8, true>(p, grid, ctx->stream, gt);
    else if (vec) launch_decode<4, true>(p, grid, ctx->stream, gt);
    else if (D > 64) launch_decode<8, false>(p, grid, ctx->stream, gt);
    else launch_decode<4, false>(p, grid, ctx->stream, gt);
    if (int rc = check_launch("attention_decode")) return rc;
    return ok();
}

}  // extern "C"
