// Memory-bound row and elementwise kernels: LayerNorm, softmax(+argmax),
// GELU, ReLU, ADD, SUB, MUL, BROADCAST, fill, copy, and the row ops of the
// training graphs (RELU_BWD, SOFTMAX_BWD, CROSS_ENTROPY and its gradient).
//
// Row kernels use one wave64 per row and keep the row in registers, so a row
// is read from HBM once and written once; reductions are wave shuffles
// (no LDS, no barriers).  Elementwise kernels use float4 accesses and a
// grid-stride loop sized to the device.
#include "common.hpp"
#include "kernels.hpp"

namespace lancius {
namespace {

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off);
    return v;
}

// The same sum without LDS traffic: DPP moves inside each row of 16 lanes
// (xor 1 and xor 2 in the quad, the half-row and row mirrors) leave every
// lane with its row's sum, and the four row sums are read from lanes 0, 16,
// 32 and 48 and added in that order, so every lane gets the same value.
template <int CTRL>
__device__ __forceinline__ float dpp_f(float x) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xF, 0xF, false));
}

__device__ __forceinline__ float wave_sum_dpp(float v) {
    v += dpp_f<0xB1>(v);   // quad_perm [1,0,3,2]
    v += dpp_f<0x4E>(v);   // quad_perm [2,3,0,1]
    v += dpp_f<0x141>(v);  // row_half_mirror
    v += dpp_f<0x140>(v);  // row_mirror
    const int b = __builtin_bit_cast(int, v);
    const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 0));
    const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 16));
    const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 32));
    const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 48));
    return (r0 + r1) + (r2 + r3);
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
    return v;
}

constexpr int kRowThreads = 256;  // 4 rows per workgroup
constexpr int kRowsPerBlock = kRowThreads / 64;

// Rows held in registers: lane owns float4 pieces at columns 4*lane + 256*i
// (i < NV) of a row of `cols` <= 256*NV columns, cols % 4 == 0 and 16-byte
// aligned; pieces past the row are not loaded and are left out of every
// statistic.
template <int NV>
__device__ __forceinline__ void load_row_f4(const float* __restrict__ x, int cols, int lane, f32x4 (&v)[NV]) {
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int c0 = 4 * lane + 256 * i;
        v[i] = c0 < cols ? *(const f32x4*)(x + c0) : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }
}

// LayerNorm with the row in registers.  Statistics follow
// bleeding/v11A1/src/math/lancius_kernels.c:217-236: mean, then the biased
// variance of (x - mean), then (x - mean) * inv_std * g + b.
// Member blockIdx.y of a group of LayerNorms of one shape.
struct LnGroup {
    float* out[LANCIUS_HIP_MAX_GROUP];
    const float* in[LANCIUS_HIP_MAX_GROUP];
    const float* gamma[LANCIUS_HIP_MAX_GROUP];
    const float* beta[LANCIUS_HIP_MAX_GROUP];
};

// Gamma (and beta) of rows wider than 1024 columns: the workgroup copies them
// to LDS with the rows' own loads (one float4 piece per lane and register
// slot, as the rows are held), so that no global load follows an output
// store (a wave's loads and stores complete in order: such a load would wait
// for the stores before it).  Up to 1024 columns they stay in registers.
template <int NV>
__device__ __forceinline__ void stage_rows_param(f32x4* dst, const float* __restrict__ src, int H, bool full) {
#pragma unroll
    for (int k = 0; k < NV / 4; ++k) {
        const int piece = threadIdx.x + kRowThreads * k;  // lane + 64 i of the register layout
        dst[piece] = full || 4 * piece < H ? *(const f32x4*)(src + 4 * piece) : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }
}

template <int NV>
__global__ void __launch_bounds__(kRowThreads) layernorm_regs(const LnGroup grp, int rows, int H, float eps) {
    constexpr bool PRE = NV <= 4;  // gamma and beta in registers, else in LDS
    constexpr int NP = PRE ? NV : 1, NS = PRE ? 1 : 64 * NV;
    __shared__ f32x4 gs[NS], bs[NS];
    const int row = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    float* __restrict__ out = grp.out[blockIdx.y];
    const float* __restrict__ gamma = grp.gamma[blockIdx.y];
    const float* __restrict__ beta = grp.beta[blockIdx.y];
    const bool full = H == 256 * NV;
    if constexpr (!PRE) {
        stage_rows_param<NV>(gs, gamma, H, full);
        stage_rows_param<NV>(bs, beta, H, full);
    }
    // Up to 4 pieces a lane, gamma and beta are requested with the row,
    // before the first wait: loaded between the output stores, each would
    // wait for the stores before it.  Pieces past the row are zero and skipped.
    f32x4 v[NV], g[NP], b[NP];
    const float* x = grp.in[blockIdx.y] + (size_t)min(row, rows - 1) * H;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int c0 = 4 * lane + 256 * i;
        const bool in = full || c0 < H;
        v[i] = in ? *(const f32x4*)(x + c0) : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        if constexpr (PRE) {
            g[i] = in ? *(const f32x4*)(gamma + c0) : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            b[i] = in ? *(const f32x4*)(beta + c0) : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        }
    }
    if constexpr (!PRE) __syncthreads();
    if (row >= rows) return;
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < NV; ++i) s += (v[i].x + v[i].y) + (v[i].z + v[i].w);
    const float mean = wave_sum_dpp(s) / (float)H;
    float q = 0.0f;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        if (full || 4 * lane + 256 * i < H) {
            const float a = v[i].x - mean, bb = v[i].y - mean, c = v[i].z - mean, d = v[i].w - mean;
            q += (a * a + bb * bb) + (c * c + d * d);
        }
    }
    const float var = wave_sum_dpp(q) / (float)H;
    const float inv_std = 1.0f / sqrtf(var + eps);
    float* y = out + (size_t)row * H;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int c0 = 4 * lane + 256 * i;
        if (!full && c0 >= H) continue;
        f32x4 gi, bi;
        if constexpr (PRE) {
            gi = g[i];
            bi = b[i];
        } else {
            gi = gs[lane + 64 * i];
            bi = bs[lane + 64 * i];
        }
        f32x4 o;
        o.x = (v[i].x - mean) * inv_std * gi.x + bi.x;
        o.y = (v[i].y - mean) * inv_std * gi.y + bi.y;
        o.z = (v[i].z - mean) * inv_std * gi.z + bi.z;
        o.w = (v[i].w - mean) * inv_std * gi.w + bi.w;
        *(f32x4*)(y + c0) = o;
    }
}

// Smallest register-row width (float4 pieces per lane) for `cols`, 0 if the
// row does not fit 16 pieces or is not float4-shaped.
int regs_width(size_t cols, bool aligned) {
    if (!aligned || cols % 4 != 0 || cols > 4096) return 0;
    for (int nv = 1; nv <= 16; nv *= 2)
        if (cols <= (size_t)256 * nv) return nv;
    return 0;
}

// Any hidden size: three passes over the row (re-reads hit L2).
__global__ void __launch_bounds__(kRowThreads) layernorm_any(float* __restrict__ out, const float* __restrict__ in,
                                                             const float* __restrict__ gamma,
                                                             const float* __restrict__ beta, int rows, int hidden,
                                                             float eps) {
    const int row = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= rows) return;
    const float* x = in + (size_t)row * hidden;
    float s = 0.0f;
    for (int c = lane; c < hidden; c += 64) s += x[c];
    const float mean = wave_sum(s) / (float)hidden;
    float q = 0.0f;
    for (int c = lane; c < hidden; c += 64) {
        const float d = x[c] - mean;
        q += d * d;
    }
    const float var = wave_sum(q) / (float)hidden;
    const float inv_std = 1.0f / sqrtf(var + eps);
    float* y = out + (size_t)row * hidden;
    for (int c = lane; c < hidden; c += 64) y[c] = (x[c] - mean) * inv_std * gamma[c] + beta[c];
}

// Row softmax (lancius_scheduler.c:284-294): max, exp(x - max), sum, divide.
// argmax: first index of the largest probability, scanning with strict '>'
// from -1e9 like the callers (B/examples/train_mnist.c:206-209); ties are
// resolved to the smaller index.
__global__ void __launch_bounds__(kRowThreads) softmax_rows(float* __restrict__ probs, int32_t* __restrict__ argmax,
                                                            const float* __restrict__ in, int rows, int cols) {
    const int row = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= rows) return;
    const float* x = in + (size_t)row * cols;
    float* y = probs + (size_t)row * cols;
    float m = -INFINITY;
    for (int c = lane; c < cols; c += 64) m = fmaxf(m, x[c]);
    m = wave_max(m);
    float s = 0.0f;
    for (int c = lane; c < cols; c += 64) s += expf(x[c] - m);
    s = wave_sum(s);
    const float inv = 1.0f / s;
    float best = -1e9f;
    int best_i = 0x7fffffff;
    for (int c = lane; c < cols; c += 64) {
        const float pv = expf(x[c] - m) / s;
        y[c] = pv;
        if (pv > best) {
            best = pv;
            best_i = c;
        }
    }
    (void)inv;
    if (argmax) {
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) {
            const float ob = __shfl_xor(best, off);
            const int oi = __shfl_xor(best_i, off);
            if (ob > best || (ob == best && oi < best_i)) {
                best = ob;
                best_i = oi;
            }
        }
        if (lane == 0) argmax[row] = best_i == 0x7fffffff ? 0 : best_i;
    }
}


// softmax_rows with the row in registers: one read of x, exp once per element.
template <int NV>
__global__ void __launch_bounds__(kRowThreads) softmax_regs(float* __restrict__ probs, int32_t* __restrict__ argmax,
                                                            const float* __restrict__ in, int rows, int cols) {
    const int row = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= rows) return;
    f32x4 v[NV];
    load_row_f4<NV>(in + (size_t)row * cols, cols, lane, v);
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < NV; ++i)
        if (4 * lane + 256 * i < cols) m = fmaxf(m, fmaxf(fmaxf(v[i].x, v[i].y), fmaxf(v[i].z, v[i].w)));
    m = wave_max(m);
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        if (4 * lane + 256 * i < cols) {
            v[i].x = expf(v[i].x - m);
            v[i].y = expf(v[i].y - m);
            v[i].z = expf(v[i].z - m);
            v[i].w = expf(v[i].w - m);
            s += v[i].x;
            s += v[i].y;
            s += v[i].z;
            s += v[i].w;
        }
    }
    s = wave_sum(s);
    float best = -1e9f;
    int best_i = 0x7fffffff;
    float* y = probs + (size_t)row * cols;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int c0 = 4 * lane + 256 * i;
        if (c0 >= cols) continue;
        f32x4 pv;
        pv.x = v[i].x / s;
        pv.y = v[i].y / s;
        pv.z = v[i].z / s;
        pv.w = v[i].w / s;
        *(f32x4*)(y + c0) = pv;
        if (pv.x > best) { best = pv.x; best_i = c0; }
        if (pv.y > best) { best = pv.y; best_i = c0 + 1; }
        if (pv.z > best) { best = pv.z; best_i = c0 + 2; }
        if (pv.w > best) { best = pv.w; best_i = c0 + 3; }
    }
    if (argmax) {
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) {
            const float ob = __shfl_xor(best, off);
            const int oi = __shfl_xor(best_i, off);
            if (ob > best || (ob == best && oi < best_i)) {
                best = ob;
                best_i = oi;
            }
        }
        if (lane == 0) argmax[row] = best_i == 0x7fffffff ? 0 : best_i;
    }
}

// SOFTMAX_BWD (lancius_scheduler.c:295-304): out = y * (dy - sum_c dy*y).
__global__ void __launch_bounds__(kRowThreads) softmax_bwd_rows(float* __restrict__ out, const float* __restrict__ dy,
                                                                const float* __restrict__ y, int rows, int cols) {
    const int row = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= rows) return;
    const size_t base = (size_t)row * cols;
    float dot = 0.0f;
    for (int c = lane; c < cols; c += 64) dot += dy[base + c] * y[base + c];
    dot = wave_sum(dot);
    for (int c = lane; c < cols; c += 64) out[base + c] = y[base + c] * (dy[base + c] - dot);
}

// Row max and sum of exp(x - max) of one row, for one wave.
__device__ __forceinline__ void row_lse_parts(const float* __restrict__ x, int cols, int lane, float& m, float& s) {
    m = -INFINITY;
    for (int c = lane; c < cols; c += 64) m = fmaxf(m, x[c]);
    m = wave_max(m);
    s = 0.0f;
    for (int c = lane; c < cols; c += 64) s += expf(x[c] - m);
    s = wave_sum(s);
}

// CROSS_ENTROPY, first pass (lancius_scheduler.c:68-83): per row,
// sum over the entries with y == 1 of (x - logsumexp(x)), in fp64.
__global__ void __launch_bounds__(kRowThreads) cross_entropy_rows(double* __restrict__ row_terms,
                                                                  const float* __restrict__ x,
                                                                  const float* __restrict__ y, int rows, int cols) {
    const int row = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= rows) return;
    const float* xr = x + (size_t)row * cols;
    const float* yr = y + (size_t)row * cols;
    float m, s;
    row_lse_parts(xr, cols, lane, m, s);
    const double lse = (double)logf(s) + (double)m;
    double t = 0.0;
    for (int c = lane; c < cols; c += 64)
        if (yr[c] == 1.0f) t += (double)xr[c] - lse;
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) t += __shfl_xor(t, off);
    if (lane == 0) row_terms[row] = t;
}

// Up to 4096 rows: one workgroup does both passes (each wave takes rows
// w, w+4, ...), so the loss is one launch.
__global__ void __launch_bounds__(kRowThreads) cross_entropy_small(float* __restrict__ out, const float* __restrict__ x,
                                                                   const float* __restrict__ y, int rows, int cols) {
    __shared__ double part[kRowsPerBlock];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    double acc = 0.0;  // this wave's rows, in row order
    for (int row = wave; row < rows; row += kRowsPerBlock) {
        const float* xr = x + (size_t)row * cols;
        const float* yr = y + (size_t)row * cols;
        float m, s;
        row_lse_parts(xr, cols, lane, m, s);
        const double lse = (double)logf(s) + (double)m;
        double t = 0.0;
        for (int c = lane; c < cols; c += 64)
            if (yr[c] == 1.0f) t += (double)xr[c] - lse;
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) t += __shfl_xor(t, off);
        acc += t;
    }
    if (lane == 0) part[wave] = acc;
    __syncthreads();
    if (threadIdx.x == 0) {
        double total = 0.0;
        for (int w = 0; w < kRowsPerBlock; ++w) total += part[w];
        out[0] = (float)fabs(-total / (double)rows);
    }
}

// Second pass: out[0] = |-(sum of row terms) / rows| (:84-85), summed by one
// workgroup in a fixed order.
__global__ void __launch_bounds__(256) cross_entropy_finish(float* __restrict__ out,
                                                            const double* __restrict__ row_terms, int rows) {
    __shared__ double part[256];
    double t = 0.0;
    for (int r = threadIdx.x; r < rows; r += 256) t += row_terms[r];
    part[threadIdx.x] = t;
    __syncthreads();
    for (int w = 128; w >= 1; w >>= 1) {
        if ((int)threadIdx.x < w) part[threadIdx.x] += part[threadIdx.x + w];
        __syncthreads();
    }
    if (threadIdx.x == 0) out[0] = (float)fabs(-part[0] / (double)rows);
}

// CROSS_ENTROPY_BWD (lancius_scheduler.c:89-104):
// out = (exp(x - max) / sum - y) * g[0] / rows.
__global__ void __launch_bounds__(kRowThreads) cross_entropy_bwd_rows(float* __restrict__ out,
                                                                      const float* __restrict__ x,
                                                                      const float* __restrict__ y,
                                                                      const float* __restrict__ g, int rows,
                                                                      int cols) {
    const int row = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= rows) return;
    const size_t base = (size_t)row * cols;
    float m, s;
    row_lse_parts(x + base, cols, lane, m, s);
    const float scale = (float)((double)g[0] / (double)rows);
    for (int c = lane; c < cols; c += 64) out[base + c] = (expf(x[base + c] - m) / s - y[base + c]) * scale;
}

// RMSNorm (lancius_kernels.c:381-396): out = x * (1 / sqrt(mean(x^2) + eps)) * gamma.
__global__ void __launch_bounds__(kRowThreads) rmsnorm_rows(float* __restrict__ out, const float* __restrict__ in,
                                                            const float* __restrict__ gamma, int rows, int hidden,
                                                            float eps) {
    const int row = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= rows) return;
    const float* x = in + (size_t)row * hidden;
    float q = 0.0f;
    for (int c = lane; c < hidden; c += 64) q += x[c] * x[c];
    q = wave_sum(q);
    const float inv = 1.0f / sqrtf(q / (float)hidden + eps);
    float* y = out + (size_t)row * hidden;
    for (int c = lane; c < hidden; c += 64) y[c] = (x[c] * inv) * gamma[c];
}

template <int NV>
__global__ void __launch_bounds__(kRowThreads) rmsnorm_regs(float* __restrict__ out, const float* __restrict__ in,
                                                            const float* __restrict__ gamma, int rows, int hidden,
                                                            float eps) {
    // gamma as in layernorm_regs: with the row in registers up to 4 pieces a
    // lane, else staged in LDS with the row loads; pieces past the row are zero
    constexpr bool PRE = NV <= 4;
    constexpr int NP = PRE ? NV : 1, NS = PRE ? 1 : 64 * NV;
    __shared__ f32x4 gs[NS];
    const int row = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const bool full = hidden == 256 * NV;
    if constexpr (!PRE) stage_rows_param<NV>(gs, gamma, hidden, full);
    const float* x = in + (size_t)min(row, rows - 1) * hidden;
    f32x4 v[NV], g[NP];
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int c0 = 4 * lane + 256 * i;
        const bool inside = full || c0 < hidden;
        v[i] = inside ? *(const f32x4*)(x + c0) : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        if constexpr (PRE) g[i] = inside ? *(const f32x4*)(gamma + c0) : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }
    if constexpr (!PRE) __syncthreads();
    if (row >= rows) return;
    float q = 0.0f;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        q += v[i].x * v[i].x;
        q += v[i].y * v[i].y;
        q += v[i].z * v[i].z;
        q += v[i].w * v[i].w;
    }
    q = wave_sum_dpp(q);
    const float inv = 1.0f / sqrtf(q / (float)hidden + eps);
    float* y = out + (size_t)row * hidden;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int c0 = 4 * lane + 256 * i;
        if (!full && c0 >= hidden) continue;
        f32x4 gi;
        if constexpr (PRE)
            gi = g[i];
        else
            gi = gs[lane + 64 * i];
        f32x4 o;
        o.x = (v[i].x * inv) * gi.x;
        o.y = (v[i].y * inv) * gi.y;
        o.z = (v[i].z * inv) * gi.z;
        o.w = (v[i].w * inv) * gi.w;
        *(f32x4*)(y + c0) = o;
    }
}

// SwiGLU (lancius_kernels.c:398-405): out = g / (1 + exp(-g)) * up.
__global__ void __launch_bounds__(256) swiglu_kernel(float* __restrict__ out, const float* __restrict__ gate,
                                                     const float* __restrict__ up, size_t n) {
    const size_t step = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += step) {
        const float g = gate[i];
        out[i] = g / (1.0f + expf(-g)) * up[i];
    }
}

// RoPE (lancius_kernels.c:248-272): pair (d, d+1) of every head at position
// s + pos_offset turns by angle pos / 10000^(d / head_dim).  The angle and its
// sine / cosine are evaluated in fp64 (positions reach thousands of radians,
// where fp32 argument reduction would lose four digits), once per (sequence
// position, pair) and applied to every head of `count` consecutive
// [batch, S, H, head_dim] tensors.
__global__ void __launch_bounds__(256) rope_kernel(float* __restrict__ out, const float* __restrict__ in, int count,
                                                   int batch, int S, int H, int hd, int pos_offset) {
    const int half = hd / 2;
    const size_t pairs = (size_t)S * half;  // (s, pair) units; heads, batch and tensors inside
    const size_t step = (size_t)gridDim.x * blockDim.x;
    const size_t tensor = (size_t)batch * S * H * hd;
    for (size_t u = (size_t)blockIdx.x * blockDim.x + threadIdx.x; u < pairs; u += step) {
        const int s = (int)(u / half), d = 2 * (int)(u - (u / half) * half);
        const double freq = 1.0 / pow(10000.0, (double)d / (double)hd);
        const double angle = (double)(s + pos_offset) * freq;
        const float c = (float)cos(angle), sn = (float)sin(angle);
        for (int t = 0; t < count; ++t)
            for (int b = 0; b < batch; ++b)
                for (int h = 0; h < H; ++h) {
                    const size_t idx = (size_t)t * tensor + (((size_t)b * S + s) * H + h) * hd + d;
                    const float x0 = in[idx], x1 = in[idx + 1];
                    out[idx] = x0 * c - x1 * sn;
                    out[idx + 1] = x0 * sn + x1 * c;
                }
    }
}

// ---- elementwise --------------------------------------------------------

enum EwOp : int { kAdd = 0, kRelu = 1, kGelu = 2, kCopy = 3, kSub = 4, kMul = 5, kReluBwd = 6, kTanh = 7 };

constexpr bool binary_op(int op) { return op == kAdd || op == kSub || op == kMul || op == kReluBwd; }

template <int OP>
__device__ __forceinline__ float ew(float a, float b) {
    if constexpr (OP == kAdd) return a + b;
    if constexpr (OP == kSub) return a - b;
    if constexpr (OP == kMul) return a * b;
    // RELU_BWD (lancius_scheduler.c:279-283): a = incoming gradient, b = the
    // forward input; NaN in b gives 0 like the reference's '>' test.
    if constexpr (OP == kReluBwd) return b > 0.0f ? a : 0.0f;
    if constexpr (OP == kRelu) return relu_ref(a);
    if constexpr (OP == kGelu) return gelu_ref(a);
    if constexpr (OP == kTanh) return tanhf(a);
    return a;
}

template <int OP>
__global__ void __launch_bounds__(256) elementwise_vec(float* __restrict__ out, const float* __restrict__ a,
                                                       const float* __restrict__ b, size_t n4) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += stride) {
        const f32x4 x = ((const f32x4*)a)[i];
        const f32x4 y = binary_op(OP) ? ((const f32x4*)b)[i] : x;
        f32x4 o;
        o.x = ew<OP>(x.x, y.x);
        o.y = ew<OP>(x.y, y.y);
        o.z = ew<OP>(x.z, y.z);
        o.w = ew<OP>(x.w, y.w);
        ((f32x4*)out)[i] = o;
    }
}

template <int OP>
__global__ void __launch_bounds__(256) elementwise_scalar(float* __restrict__ out, const float* __restrict__ a,
                                                          const float* __restrict__ b, size_t begin, size_t n) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = begin + (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
        out[i] = ew<OP>(a[i], binary_op(OP) ? b[i] : 0.0f);
}

__global__ void __launch_bounds__(256) broadcast_rows(float* __restrict__ out, const float* __restrict__ row,
                                                      size_t rows, size_t cols, size_t cols_in) {
    const size_t n = rows * cols;
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
        out[i] = cols_in == 1 ? row[0] : row[i % cols];
}

// out[r][c] = act(a[r][c] + bias[c]); float4 along the row when cols % 4 == 0
// and the pointers are 16-byte aligned (vec).
__global__ void __launch_bounds__(256) bias_act_rows(float* __restrict__ out, const float* __restrict__ a,
                                                     const float* __restrict__ bias, size_t rows, size_t cols,
                                                     int act, int vec) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    if (vec) {
        const size_t c4 = cols / 4, n4 = rows * c4;
        for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += stride) {
            const f32x4 x = ((const f32x4*)a)[i], b = ((const f32x4*)bias)[i % c4];
            f32x4 o;
            o.x = apply_act(x.x + b.x, act);
            o.y = apply_act(x.y + b.y, act);
            o.z = apply_act(x.z + b.z, act);
            o.w = apply_act(x.w + b.w, act);
            ((f32x4*)out)[i] = o;
        }
        return;
    }
    const size_t n = rows * cols;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
        out[i] = apply_act(a[i] + bias[i % cols], act);
}

__global__ void __launch_bounds__(256) fill_kernel(float* __restrict__ out, float value, size_t n) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) out[i] = value;
}

unsigned int ew_grid(size_t work) {
    // 256 CUs x 8 workgroups of 256 threads covers the device; more only adds
    // scheduling overhead for a grid-stride loop.
    const size_t cap = 2048;
    size_t g = (work + 255) / 256;
    if (g < 1) g = 1;
    return (unsigned int)(g < cap ? g : cap);
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

template <int OP>
int run_elementwise(lancius_hip_ctx* ctx, float* out, const float* a, const float* b, size_t n, const char* name) {
    LANCIUS_REQUIRE(ctx && out && a && (!binary_op(OP) || b), LANCIUS_HIP_ERR_NULL_PTR, "%s: NULL argument", name);
    if (n == 0) return ok();
    if (int rc = bind_device(ctx)) return rc;
    const bool vec = aligned16(out) && aligned16(a) && (!binary_op(OP) || aligned16(b));
    size_t done = 0;
    if (vec && n >= 4) {
        const size_t n4 = n / 4;
        hipLaunchKernelGGL(elementwise_vec<OP>, dim3(ew_grid(n4)), dim3(256), 0, ctx->stream, out, a, b, n4);
        if (int rc = check_launch(name)) return rc;
        done = n4 * 4;
    }
    if (done < n) {
        hipLaunchKernelGGL(elementwise_scalar<OP>, dim3(ew_grid(n - done)), dim3(256), 0, ctx->stream, out, a, b,
                           done, n);
        if (int rc = check_launch(name)) return rc;
    }
    return ok();
}

}  // namespace
}  // namespace lancius

using namespace lancius;

extern "C" {

int lancius_hip_layernorm_grouped_f32(lancius_hip_ctx* ctx, size_t count, float* const* out, const float* const* in,
                                      const float* const* gamma, const float* const* beta, size_t rows, size_t hidden,
                                      float eps) {
    LANCIUS_REQUIRE(ctx && out && in && gamma && beta, LANCIUS_HIP_ERR_NULL_PTR, "layernorm: NULL argument");
    LANCIUS_REQUIRE(count >= 1 && count <= LANCIUS_HIP_MAX_GROUP, LANCIUS_HIP_ERR_SHAPE, "layernorm: group count %zu",
                    count);
    LANCIUS_REQUIRE(hidden > 0 && hidden < (1u << 30) && rows < (1u << 30), LANCIUS_HIP_ERR_SHAPE,
                    "layernorm: rows=%zu hidden=%zu", rows, hidden);
    LnGroup grp{};
    bool aligned = true;
    for (size_t g = 0; g < count; ++g) {
        LANCIUS_REQUIRE(out[g] && in[g] && gamma[g] && beta[g], LANCIUS_HIP_ERR_NULL_PTR,
                        "layernorm: NULL operand in group %zu", g);
        grp.out[g] = out[g];
        grp.in[g] = in[g];
        grp.gamma[g] = gamma[g];
        grp.beta[g] = beta[g];
        aligned = aligned && aligned16(out[g]) && aligned16(in[g]) && aligned16(gamma[g]) && aligned16(beta[g]);
    }
    if (rows == 0) return ok();
    if (int rc = bind_device(ctx)) return rc;
    const dim3 grid(ceil_div(rows, kRowsPerBlock), (unsigned)count), block(kRowThreads);
    const int r = (int)rows, h = (int)hidden;
    switch (regs_width(hidden, aligned)) {
        case 1: hipLaunchKernelGGL(layernorm_regs<1>, grid, block, 0, ctx->stream, grp, r, h, eps); break;
        case 2: hipLaunchKernelGGL(layernorm_regs<2>, grid, block, 0, ctx->stream, grp, r, h, eps); break;
        case 4: hipLaunchKernelGGL(layernorm_regs<4>, grid, block, 0, ctx->stream, grp, r, h, eps); break;
        case 8: hipLaunchKernelGGL(layernorm_regs<8>, grid, block, 0, ctx->stream, grp, r, h, eps); break;
        case 16: hipLaunchKernelGGL(layernorm_regs<16>, grid, block, 0, ctx->stream, grp, r, h, eps); break;
        default:  // rows that are not float4-shaped: one three-pass launch per member
            for (size_t g = 0; g < count; ++g) {
                hipLaunchKernelGGL(layernorm_any, dim3(grid.x), block, 0, ctx->stream, out[g], in[g], gamma[g], beta[g],
                                   r, h, eps);
                if (int rc = check_launch("layernorm")) return rc;
            }
    }
    if (int rc = check_launch("layernorm")) return rc;
    return ok();
}

int lancius_hip_layernorm_f32(lancius_hip_ctx* ctx, float* out, const float* in, const float* gamma,
                              const float* beta, size_t rows, size_t hidden, float eps) {
    return lancius_hip_layernorm_grouped_f32(ctx, 1, &out, &in, &gamma, &beta, rows, hidden, eps);
}

int lancius_hip_softmax_f32(lancius_hip_ctx* ctx, float* probs, int32_t* argmax, const float* in, size_t rows,
                            size_t cols) {
    LANCIUS_REQUIRE(ctx && probs && in, LANCIUS_HIP_ERR_NULL_PTR, "softmax: NULL argument");
    LANCIUS_REQUIRE(cols > 0 && cols < (1u << 30) && rows < (1u << 30), LANCIUS_HIP_ERR_SHAPE,
                    "softmax: rows=%zu cols=%zu", rows, cols);
    if (rows == 0) return ok();
    if (int rc = bind_device(ctx)) return rc;
    const dim3 grid(ceil_div(rows, kRowsPerBlock)), block(kRowThreads);
    const int r = (int)rows, c = (int)cols;
    switch (regs_width(cols, aligned16(probs) && aligned16(in))) {
        case 1: hipLaunchKernelGGL(softmax_regs<1>, grid, block, 0, ctx->stream, probs, argmax, in, r, c); break;
        case 2: hipLaunchKernelGGL(softmax_regs<2>, grid, block, 0, ctx->stream, probs, argmax, in, r, c); break;
        case 4: hipLaunchKernelGGL(softmax_regs<4>, grid, block, 0, ctx->stream, probs, argmax, in, r, c); break;
        case 8: hipLaunchKernelGGL(softmax_regs<8>, grid, block, 0, ctx->stream, probs, argmax, in, r, c); break;
        case 16: hipLaunchKernelGGL(softmax_regs<16>, grid, block, 0, ctx->stream, probs, argmax, in, r, c); break;
        default: hipLaunchKernelGGL(softmax_rows, grid, block, 0, ctx->stream, probs, argmax, in, r, c);
    }
    if (int rc = check_launch("softmax")) return rc;
    return ok();
}

int lancius_hip_add_f32(lancius_hip_ctx* ctx, float* out, const float* a, const float* b, size_t n) {
    return run_elementwise<kAdd>(ctx, out, a, b, n, "add");
}

int lancius_hip_tanh_f32(lancius_hip_ctx* ctx, float* out, const float* a, size_t n) {
    return run_elementwise<kTanh>(ctx, out, a, nullptr, n, "tanh");
}

int lancius_hip_bias_act_f32(lancius_hip_ctx* ctx, float* out, const float* a, const float* bias, size_t rows,
                             size_t cols, int act) {
    LANCIUS_REQUIRE(ctx && out && a && bias, LANCIUS_HIP_ERR_NULL_PTR, "bias_act: NULL argument");
    LANCIUS_REQUIRE(act >= LANCIUS_HIP_ACT_NONE && act <= LANCIUS_HIP_ACT_TANH, LANCIUS_HIP_ERR_UNSUPPORTED,
                    "bias_act: activation %d", act);
    LANCIUS_REQUIRE(cols == 0 || rows <= ((size_t)1 << 40) / cols, LANCIUS_HIP_ERR_SHAPE, "bias_act: %zu x %zu",
                    rows, cols);
    if (rows == 0 || cols == 0) return ok();
    if (int rc = bind_device(ctx)) return rc;
    const int vec = cols % 4 == 0 && aligned16(out) && aligned16(a) && aligned16(bias);
    hipLaunchKernelGGL(bias_act_rows, dim3(ew_grid(rows * cols / (vec ? 4 : 1))), dim3(256), 0, ctx->stream, out, a,
                       bias, rows, cols, act, vec);
    return check_launch("bias_act");
}

int lancius_hip_relu_f32(lancius_hip_ctx* ctx, float* out, const float* a, size_t n) {
    return run_elementwise<kRelu>(ctx, out, a, nullptr, n, "relu");
}

int lancius_hip_gelu_f32(lancius_hip_ctx* ctx, float* out, const float* a, size_t n) {
    return run_elementwise<kGelu>(ctx, out, a, nullptr, n, "gelu");
}

int lancius_hip_copy_f32(lancius_hip_ctx* ctx, float* out, const float* in, size_t n) {
    return run_elementwise<kCopy>(ctx, out, in, nullptr, n, "copy");
}

int lancius_hip_rmsnorm_f32(lancius_hip_ctx* ctx, float* out, const float* in, const float* gamma, size_t rows,
                            size_t hidden, float eps) {
    LANCIUS_REQUIRE(ctx && out && in && gamma, LANCIUS_HIP_ERR_NULL_PTR, "rmsnorm: NULL argument");
    LANCIUS_REQUIRE(hidden > 0 && hidden < (1u << 30) && rows < (1u << 30), LANCIUS_HIP_ERR_SHAPE,
                    "rmsnorm: rows=%zu hidden=%zu", rows, hidden);
    if (rows == 0) return ok();
    if (int rc = bind_device(ctx)) return rc;
    const dim3 grid(ceil_div(rows, kRowsPerBlock)), block(kRowThreads);
    const int r = (int)rows, h = (int)hidden;
    switch (regs_width(hidden, aligned16(out) && aligned16(in) && aligned16(gamma))) {
        case 1: hipLaunchKernelGGL(rmsnorm_regs<1>, grid, block, 0, ctx->stream, out, in, gamma, r, h, eps); break;
        case 2: hipLaunchKernelGGL(rmsnorm_regs<2>, grid, block, 0, ctx->stream, out, in, gamma, r, h, eps); break;
        case 4: hipLaunchKernelGGL(rmsnorm_regs<4>, grid, block, 0, ctx->stream, out, in, gamma, r, h, eps); break;
        case 8: hipLaunchKernelGGL(rmsnorm_regs<8>, grid, block, 0, ctx->stream, out, in, gamma, r, h, eps); break;
        case 16: hipLaunchKernelGGL(rmsnorm_regs<16>, grid, block, 0, ctx->stream, out, in, gamma, r, h, eps); break;
        default: hipLaunchKernelGGL(rmsnorm_rows, grid, block, 0, ctx->stream, out, in, gamma, r, h, eps);
    }
    return check_launch("rmsnorm");
}

int lancius_hip_swiglu_f32(lancius_hip_ctx* ctx, float* out, const float* gate, const float* up, size_t n) {
    LANCIUS_REQUIRE(ctx && out && gate && up, LANCIUS_HIP_ERR_NULL_PTR, "swiglu: NULL argument");
    if (n == 0) return ok();
    if (int rc = bind_device(ctx)) return rc;
    hipLaunchKernelGGL(swiglu_kernel, dim3(ew_grid(n)), dim3(256), 0, ctx->stream, out, gate, up, n);
    return check_launch("swiglu");
}

int lancius_hip_rope_f32(lancius_hip_ctx* ctx, float* out, const float* in, size_t count, size_t batch, size_t S,
                         size_t H, size_t head_dim, int pos_offset) {
    LANCIUS_REQUIRE(ctx && out && in, LANCIUS_HIP_ERR_NULL_PTR, "rope: NULL argument");
    LANCIUS_REQUIRE(head_dim % 2 == 0 && count * batch * S * H * head_dim < ((size_t)1 << 40) && S < (1u << 30),
                    LANCIUS_HIP_ERR_SHAPE, "rope: head_dim %zu must be even", head_dim);
    if (count * batch * S * H * head_dim == 0) return ok();
    if (int rc = bind_device(ctx)) return rc;
    hipLaunchKernelGGL(rope_kernel, dim3(ew_grid(S * head_dim / 2)), dim3(256), 0, ctx->stream, out, in, (int)count,
                       (int)batch, (int)S, (int)H, (int)head_dim, pos_offset);
    return check_launch("rope");
}

int lancius_hip_sub_f32(lancius_hip_ctx* ctx, float* out, const float* a, const float* b, size_t n) {
    return run_elementwise<kSub>(ctx, out, a, b, n, "sub");
}

int lancius_hip_mul_f32(lancius_hip_ctx* ctx, float* out, const float* a, const float* b, size_t n) {
    return run_elementwise<kMul>(ctx, out, a, b, n, "mul");
}

int lancius_hip_relu_bwd_f32(lancius_hip_ctx* ctx, float* out, const float* grad, const float* fwd, size_t n) {
    return run_elementwise<kReluBwd>(ctx, out, grad, fwd, n, "relu_bwd");
}

int lancius_hip_softmax_bwd_f32(lancius_hip_ctx* ctx, float* out, const float* dy, const float* y, size_t rows,
                                size_t cols) {
    LANCIUS_REQUIRE(ctx && out && dy && y, LANCIUS_HIP_ERR_NULL_PTR, "softmax_bwd: NULL argument");
    LANCIUS_REQUIRE(cols < (1u << 30) && rows < (1u << 30), LANCIUS_HIP_ERR_SHAPE, "softmax_bwd: rows=%zu cols=%zu",
                    rows, cols);
    if (rows == 0 || cols == 0) return ok();
    if (int rc = bind_device(ctx)) return rc;
    hipLaunchKernelGGL(softmax_bwd_rows, dim3(ceil_div(rows, kRowsPerBlock)), dim3(kRowThreads), 0, ctx->stream, out,
                       dy, y, (int)rows, (int)cols);
    return check_launch("softmax_bwd");
}

int lancius_hip_cross_entropy_f32(lancius_hip_ctx* ctx, float* out, const float* x, const float* y, size_t rows,
                                  size_t cols) {
    LANCIUS_REQUIRE(ctx && out && x && y, LANCIUS_HIP_ERR_NULL_PTR, "cross_entropy: NULL argument");
    LANCIUS_REQUIRE(rows > 0 && cols > 0 && cols < (1u << 30) && rows < (1u << 30), LANCIUS_HIP_ERR_SHAPE,
                    "cross_entropy: rows=%zu cols=%zu", rows, cols);
    if (int rc = bind_device(ctx)) return rc;
    if (rows <= 4096) {
        hipLaunchKernelGGL(cross_entropy_small, dim3(1), dim3(kRowThreads), 0, ctx->stream, out, x, y, (int)rows,
                           (int)cols);
        return check_launch("cross_entropy_small");
    }
    void* ws = nullptr;
    if (int rc = workspace(ctx, rows * sizeof(double), &ws)) return rc;
    hipLaunchKernelGGL(cross_entropy_rows, dim3(ceil_div(rows, kRowsPerBlock)), dim3(kRowThreads), 0, ctx->stream,
                       (double*)ws, x, y, (int)rows, (int)cols);
    if (int rc = check_launch("cross_entropy_rows")) return rc;
    hipLaunchKernelGGL(cross_entropy_finish, dim3(1), dim3(256), 0, ctx->stream, out, (const double*)ws, (int)rows);
    return check_launch("cross_entropy_finish");
}

int lancius_hip_cross_entropy_bwd_f32(lancius_hip_ctx* ctx, float* out, const float* x, const float* y,
                                      const float* g, size_t rows, size_t cols) {
    LANCIUS_REQUIRE(ctx && out && x && y && g, LANCIUS_HIP_ERR_NULL_PTR, "cross_entropy_bwd: NULL argument");
    LANCIUS_REQUIRE(cols < (1u << 30) && rows < (1u << 30), LANCIUS_HIP_ERR_SHAPE,
                    "cross_entropy_bwd: rows=%zu cols=%zu", rows, cols);
    if (rows == 0 || cols == 0) return ok();
    if (int rc = bind_device(ctx)) return rc;
    hipLaunchKernelGGL(cross_entropy_bwd_rows, dim3(ceil_div(rows, kRowsPerBlock)), dim3(kRowThreads), 0,
                       ctx->stream, out, x, y, g, (int)rows, (int)cols);
    return check_launch("cross_entropy_bwd");
}

int lancius_hip_broadcast_f32(lancius_hip_ctx* ctx, float* out, const float* row, size_t rows, size_t cols,
                              size_t cols_in) {
    LANCIUS_REQUIRE(ctx && out && row, LANCIUS_HIP_ERR_NULL_PTR, "broadcast: NULL argument");
    LANCIUS_REQUIRE(cols_in == 1 || cols_in >= cols, LANCIUS_HIP_ERR_SHAPE,
                    "broadcast: input has %zu values for %zu columns", cols_in, cols);
    if (rows * cols == 0) return ok();
    if (int rc = bind_device(ctx)) return rc;
    hipLaunchKernelGGL(broadcast_rows, dim3(ew_grid(rows * cols)), dim3(256), 0, ctx->stream, out, row, rows, cols,
                       cols_in);
    if (int rc = check_launch("broadcast")) return rc;
    return ok();
}

int lancius_hip_fill_f32(lancius_hip_ctx* ctx, float* out, float value, size_t n) {
    LANCIUS_REQUIRE(ctx && out, LANCIUS_HIP_ERR_NULL_PTR, "fill: NULL argument");
    if (n == 0) return ok();
    if (int rc = bind_device(ctx)) return rc;
    hipLaunchKernelGGL(fill_kernel, dim3(ew_grid(n)), dim3(256), 0, ctx->stream, out, value, n);
    if (int rc = check_launch("fill")) return rc;
    return ok();
}

}  // extern "C"
