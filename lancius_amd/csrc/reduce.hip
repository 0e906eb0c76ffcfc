// Reductions and the 2-D transpose of the scheduler dispatch
// (bleeding/v11A1/src/runtime/lancius_scheduler.c:246-267): TRANSPOSE, SUM,
// SUM_AXIS0, SUM_AXIS1.  All HBM-bound.
//
// Sums accumulate in fp64 (the reference's accumulator type) and store fp32.
// Every element goes to a partial chosen from the shape alone and partials
// are combined in a fixed order, so results are bit-identical from run to
// run; no atomics.
#include <algorithm>

#include "common.hpp"
#include "kernels.hpp"

namespace lancius {
namespace {

constexpr int kThreads = 256;

__device__ __forceinline__ double block_sum(double v, double* part) {
    part[threadIdx.x] = v;
    __syncthreads();
    for (int w = kThreads / 2; w >= 1; w >>= 1) {
        if ((int)threadIdx.x < w) part[threadIdx.x] += part[threadIdx.x + w];
        __syncthreads();
    }
    return part[0];
}

// SUM, first stage: workgroup b sums the float4 groups b*256+t, then every
// gridDim*256-th after it (fixed by n and the grid), plus the n % 4 tail in
// workgroup 0.
__global__ void __launch_bounds__(kThreads) sum_partials(double* __restrict__ partial, const float* __restrict__ in,
                                                         size_t n, int vec) {
    __shared__ double part[kThreads];
    const size_t stride = (size_t)gridDim.x * kThreads;
    double t = 0.0;
    if (vec) {
        const size_t n4 = n / 4;
        for (size_t i = (size_t)blockIdx.x * kThreads + threadIdx.x; i < n4; i += stride) {
            const f32x4 v = ((const f32x4*)in)[i];
            t += ((double)v.x + (double)v.y) + ((double)v.z + (double)v.w);
        }
        if (blockIdx.x == 0 && threadIdx.x < n - 4 * n4) t += (double)in[4 * n4 + threadIdx.x];
    } else {
        for (size_t i = (size_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += stride) t += (double)in[i];
    }
    const double s = block_sum(t, part);
    if (threadIdx.x == 0) partial[blockIdx.x] = s;
}

__global__ void __launch_bounds__(kThreads) sum_finish(float* __restrict__ out, const double* __restrict__ partial,
                                                       int count) {
    __shared__ double part[kThreads];
    double t = 0.0;
    for (int i = threadIdx.x; i < count; i += kThreads) t += partial[i];
    const double s = block_sum(t, part);
    if (threadIdx.x == 0) out[0] = (float)s;
}

// SUM_AXIS0 over rows [r0, r1) of split blockIdx.y: one column per thread,
// consecutive threads on consecutive columns (coalesced rows).
__global__ void __launch_bounds__(kThreads) sum_axis0_split(float* __restrict__ out, double* __restrict__ partial,
                                                            const float* __restrict__ in, size_t rows, size_t cols,
                                                            size_t rchunk) {
    const size_t c = (size_t)blockIdx.x * kThreads + threadIdx.x;
    if (c >= cols) return;
    const size_t r0 = (size_t)blockIdx.y * rchunk;
    const size_t r1 = std::min(rows, r0 + rchunk);
    double t = 0.0;
    for (size_t r = r0; r < r1; ++r) t += (double)in[r * cols + c];
    if (gridDim.y == 1)
        out[c] = (float)t;
    else
        partial[(size_t)blockIdx.y * cols + c] = t;
}

__global__ void __launch_bounds__(kThreads) sum_axis0_finish(float* __restrict__ out,
                                                             const double* __restrict__ partial, size_t cols,
                                                             int splits) {
    const size_t c = (size_t)blockIdx.x * kThreads + threadIdx.x;
    if (c >= cols) return;
    double t = 0.0;
    for (int s = 0; s < splits; ++s) t += partial[(size_t)s * cols + c];
    out[c] = (float)t;
}

// SUM_AXIS1: one wave per row, lanes strided over the columns, fp64 wave sum.
__global__ void __launch_bounds__(kThreads) sum_axis1_rows(float* __restrict__ out, const float* __restrict__ in,
                                                           size_t rows, size_t cols) {
    const size_t row = (size_t)blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= rows) return;
    const float* x = in + row * cols;
    double t = 0.0;
    for (size_t c = lane; c < cols; c += 64) t += (double)x[c];
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) t += __shfl_xor(t, off);
    if (lane == 0) out[row] = (float)t;
}

// TRANSPOSE through a 64x65 LDS tile: reads and writes are both 64-float
// row segments.  Tiles are numbered along columns of the input first.
__global__ void __launch_bounds__(kThreads) transpose_tiles(float* __restrict__ out, const float* __restrict__ in,
                                                            size_t rows, size_t cols, size_t tiles_c) {
    __shared__ float t[64][65];
    const size_t tile = blockIdx.x;
    const size_t r0 = (tile / tiles_c) * 64, c0 = (tile % tiles_c) * 64;
    const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const size_t r = r0 + ty + 4 * i, c = c0 + tx;
        if (r < rows && c < cols) t[ty + 4 * i][tx] = in[r * cols + c];
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const size_t c = c0 + ty + 4 * i, r = r0 + tx;  // out row c, column r
        if (r < rows && c < cols) out[c * rows + r] = t[tx][ty + 4 * i];
    }
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

}  // namespace
}  // namespace lancius

using namespace lancius;

extern "C" {

int lancius_hip_sum_f32(lancius_hip_ctx* ctx, float* out, const float* in, size_t n) {
    LANCIUS_REQUIRE(ctx && out && in, LANCIUS_HIP_ERR_NULL_PTR, "sum: NULL argument");
    if (int rc = bind_device(ctx)) return rc;
    // Enough workgroups to stream from every CU, each with >= 4096 values.
    const size_t blocks = std::max<size_t>(1, std::min<size_t>(1024, (n + 4095) / 4096));
    void* ws = nullptr;
    if (int rc = workspace(ctx, blocks * sizeof(double), &ws)) return rc;
    hipLaunchKernelGGL(sum_partials, dim3((unsigned)blocks), dim3(kThreads), 0, ctx->stream, (double*)ws, in, n,
                       (int)aligned16(in));
    if (int rc = check_launch("sum_partials")) return rc;
    hipLaunchKernelGGL(sum_finish, dim3(1), dim3(kThreads), 0, ctx->stream, out, (const double*)ws, (int)blocks);
    return check_launch("sum_finish");
}

int lancius_hip_sum_axis0_f32(lancius_hip_ctx* ctx, float* out, const float* in, size_t rows, size_t cols) {
    LANCIUS_REQUIRE(ctx && out && in, LANCIUS_HIP_ERR_NULL_PTR, "sum_axis0: NULL argument");
    if (cols == 0) return ok();
    if (int rc = bind_device(ctx)) return rc;
    const size_t col_blocks = (cols + kThreads - 1) / kThreads;
    LANCIUS_REQUIRE(col_blocks < kMaxGridX, LANCIUS_HIP_ERR_SHAPE, "sum_axis0: %zu columns", cols);
    // Row splits: ~1024 workgroups in all, each over >= 16 rows; none below
    // 512 rows, where one pass is latency-bound anyway and a second launch
    // would cost more than it saves.
    size_t splits = rows <= 512 ? 1 : std::max<size_t>(1, std::min<size_t>((rows + 15) / 16, 1024 / col_blocks));
    splits = std::min<size_t>(splits, 65535);
    const size_t rchunk = rows ? (rows + splits - 1) / splits : 1;
    splits = rows ? (rows + rchunk - 1) / rchunk : 1;
    double* ws = nullptr;
    if (splits > 1)
        if (int rc = workspace(ctx, splits * cols * sizeof(double), (void**)&ws)) return rc;
    hipLaunchKernelGGL(sum_axis0_split, dim3((unsigned)col_blocks, (unsigned)splits), dim3(kThreads), 0, ctx->stream,
                       out, ws, in, rows, cols, rchunk);
    if (int rc = check_launch("sum_axis0_split")) return rc;
    if (splits > 1) {
        hipLaunchKernelGGL(sum_axis0_finish, dim3((unsigned)col_blocks), dim3(kThreads), 0, ctx->stream, out,
                           (const double*)ws, cols, (int)splits);
        if (int rc = check_launch("sum_axis0_finish")) return rc;
    }
    return ok();
}

int lancius_hip_sum_axis1_f32(lancius_hip_ctx* ctx, float* out, const float* in, size_t rows, size_t cols) {
    LANCIUS_REQUIRE(ctx && out && in, LANCIUS_HIP_ERR_NULL_PTR, "sum_axis1: NULL argument");
    if (rows == 0) return ok();
    if (int rc = bind_device(ctx)) return rc;
    const size_t blocks = (rows + 3) / 4;
    LANCIUS_REQUIRE(blocks < kMaxGridX, LANCIUS_HIP_ERR_SHAPE, "sum_axis1: %zu rows", rows);
    hipLaunchKernelGGL(sum_axis1_rows, dim3((unsigned)blocks), dim3(kThreads), 0, ctx->stream, out, in, rows, cols);
    return check_launch("sum_axis1");
}

int lancius_hip_transpose_f32(lancius_hip_ctx* ctx, float* out, const float* in, size_t rows, size_t cols) {
    LANCIUS_REQUIRE(ctx && out && in, LANCIUS_HIP_ERR_NULL_PTR, "transpose: NULL argument");
    if (rows == 0 || cols == 0) return ok();
    if (int rc = bind_device(ctx)) return rc;
    const size_t tr = (rows + 63) / 64, tc = (cols + 63) / 64;
    LANCIUS_REQUIRE(tr * tc < kMaxGridX, LANCIUS_HIP_ERR_SHAPE, "transpose: %zu x %zu", rows, cols);
    hipLaunchKernelGGL(transpose_tiles, dim3((unsigned)(tr * tc)), dim3(kThreads), 0, ctx->stream, out, in, rows, cols,
                       tc);
    return check_launch("transpose");
}

}  // extern "C"
