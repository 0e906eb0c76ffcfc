// MAXPOOL2D and MAXPOOL2D_BWD of the vision router
// (bleeding/v11A1/src/runtime/lancius_vision_ops.c:82-112 and :149-190).
//
// Forward: K x K window, no padding, the running maximum starts at -1e9 and
// takes a value only when strictly greater (so NaN never wins and a window
// with nothing above -1e9 yields -1e9).
//
// Backward: the reference scatters each dy value onto the first maximum of
// its window (row-major scan), or onto plane position (0,0) when no value
// beats -1e9 (its max_ih = max_iw = 0 start).  Here the scatter is turned
// into gathers, so no two threads write one element and the order of
// additions is fixed: each input element other than (0,0) takes the dy of the
// windows that cover it and chose it, in (ho, wo) order, and per plane one
// workgroup sums the dy of every window whose winner is (0,0).
#include <algorithm>

#include "common.hpp"

namespace lancius {
namespace {

constexpr int kThreads = 256;
constexpr float kStart = -1e9f;

__device__ __forceinline__ int window_argmax(const float* __restrict__ plane, int W, int ho, int wo, int K,
                                             int stride, float& best) {
    best = kStart;
    int at = 0;  // (0,0) of the plane when nothing beats the start value
    for (int kh = 0; kh < K; ++kh)
        for (int kw = 0; kw < K; ++kw) {
            const int ih = ho * stride + kh, iw = wo * stride + kw;
            const float v = plane[ih * W + iw];
            if (v > best) {
                best = v;
                at = ih * W + iw;
            }
        }
    return at;
}

__global__ void __launch_bounds__(kThreads) maxpool_fwd(float* __restrict__ out, const float* __restrict__ in,
                                                        size_t total, int H, int W, int Ho, int Wo, int K,
                                                        int stride) {
    const size_t step = (size_t)gridDim.x * kThreads;
    for (size_t o = (size_t)blockIdx.x * kThreads + threadIdx.x; o < total; o += step) {
        const size_t plane = o / ((size_t)Ho * Wo);
        const int pix = (int)(o - plane * Ho * Wo);
        const int ho = pix / Wo, wo = pix - (pix / Wo) * Wo;
        float best;
        (void)window_argmax(in + plane * H * W, W, ho, wo, K, stride, best);
        out[o] = best;
    }
}

// One launch: workgroups [0, planes) each sum, for their plane, the dy of the
// windows whose winner is (0,0); the others give every other input element
// the dy of the windows that cover it and choose it, in (ho, wo) order.
// Winners are recomputed from x (K*K reads per covering window, L2-resident)
// instead of being stored.
__global__ void __launch_bounds__(kThreads) maxpool_bwd_fused(float* __restrict__ dx, const float* __restrict__ dy,
                                                              const float* __restrict__ x, size_t planes, int H,
                                                              int W, int Ho, int Wo, int K, int stride) {
    const int HW = H * W, HoWo = Ho * Wo;
    if (blockIdx.x < planes) {
        __shared__ float part[kThreads];
        const size_t plane = blockIdx.x;
        const float* xp = x + plane * HW;
        const float* gp = dy + plane * HoWo;
        float g = 0.0f;
        for (int o = threadIdx.x; o < HoWo; o += kThreads) {
            float best;
            if (window_argmax(xp, W, o / Wo, o - (o / Wo) * Wo, K, stride, best) == 0) g += gp[o];
        }
        part[threadIdx.x] = g;
        __syncthreads();
        for (int w = kThreads / 2; w >= 1; w >>= 1) {
            if ((int)threadIdx.x < w) part[threadIdx.x] += part[threadIdx.x + w];
            __syncthreads();
        }
        if (threadIdx.x == 0) dx[plane * HW] = part[0];
        return;
    }
    const size_t total = planes * HW;
    const size_t step = (size_t)(gridDim.x - planes) * kThreads;
    for (size_t i = (size_t)(blockIdx.x - planes) * kThreads + threadIdx.x; i < total; i += step) {
        const size_t plane = i / HW;
        const int pos = (int)(i - plane * HW);
        if (pos == 0) continue;  // the plane's first workgroup writes it
        const int ih = pos / W, iw = pos - (pos / W) * W;
        // windows ho with ho*stride <= ih <= ho*stride + K - 1
        const int ho_lo = ih >= K ? (ih - K) / stride + 1 : 0;
        const int ho_hi = min(Ho - 1, ih / stride);
        const int wo_lo = iw >= K ? (iw - K) / stride + 1 : 0;
        const int wo_hi = min(Wo - 1, iw / stride);
        const float* xp = x + plane * HW;
        const float* gp = dy + plane * HoWo;
        float g = 0.0f;
        for (int ho = ho_lo; ho <= ho_hi; ++ho)
            for (int wo = wo_lo; wo <= wo_hi; ++wo) {
                float best;
                if (window_argmax(xp, W, ho, wo, K, stride, best) == pos) g += gp[ho * Wo + wo];
            }
        dx[i] = g;
    }
}

unsigned grid_for(size_t work) { return (unsigned)std::max<size_t>(1, std::min<size_t>((work + 255) / 256, 8192)); }

}  // namespace
}  // namespace lancius

using namespace lancius;

extern "C" {

int lancius_hip_maxpool2d_f32(lancius_hip_ctx* ctx, float* out, const float* in, size_t N, size_t C, size_t H,
                              size_t W, size_t K, size_t stride) {
    LANCIUS_REQUIRE(ctx && out && in, LANCIUS_HIP_ERR_NULL_PTR, "maxpool2d: NULL argument");
    LANCIUS_REQUIRE(K >= 1 && stride >= 1 && H >= K && W >= K, LANCIUS_HIP_ERR_SHAPE,
                    "maxpool2d: spatial dimensions underflow (H=%zu W=%zu K=%zu)", H, W, K);
    LANCIUS_REQUIRE(H * W < (1u << 30), LANCIUS_HIP_ERR_SHAPE, "maxpool2d: plane too large");
    const size_t Ho = (H - K) / stride + 1, Wo = (W - K) / stride + 1;
    const size_t total = N * C * Ho * Wo;
    if (total == 0) return ok();
    if (int rc = bind_device(ctx)) return rc;
    hipLaunchKernelGGL(maxpool_fwd, dim3(grid_for(total)), dim3(kThreads), 0, ctx->stream, out, in, total, (int)H,
                       (int)W, (int)Ho, (int)Wo, (int)K, (int)stride);
    return check_launch("maxpool2d");
}

int lancius_hip_maxpool2d_bwd_f32(lancius_hip_ctx* ctx, float* dx, const float* dy, const float* x, size_t N,
                                  size_t C, size_t H, size_t W, size_t H_out, size_t W_out, size_t K, size_t stride) {
    LANCIUS_REQUIRE(ctx && dx && dy && x, LANCIUS_HIP_ERR_NULL_PTR, "maxpool2d_bwd: NULL argument");
    LANCIUS_REQUIRE(K >= 1 && stride >= 1 && H * W < (1u << 30) && H_out * W_out < (1u << 30), LANCIUS_HIP_ERR_SHAPE,
                    "maxpool2d_bwd: bad shape");
    // Every window must lie inside the input plane (the reference reads it
    // unchecked).
    LANCIUS_REQUIRE(H_out == 0 || W_out == 0 || ((H_out - 1) * stride + K <= H && (W_out - 1) * stride + K <= W),
                    LANCIUS_HIP_ERR_SHAPE, "maxpool2d_bwd: %zu x %zu windows of %zu exceed the %zu x %zu input",
                    H_out, W_out, K, H, W);
    const size_t planes = N * C;
    if (planes == 0 || H * W == 0) return ok();
    LANCIUS_REQUIRE(planes < kMaxGridX, LANCIUS_HIP_ERR_SHAPE, "maxpool2d_bwd: %zu planes", planes);
    if (int rc = bind_device(ctx)) return rc;
    const size_t total = planes * H * W;
    const size_t gather = std::max<size_t>(1, std::min<size_t>((total + 255) / 256, 8192));
    LANCIUS_REQUIRE(planes + gather < kMaxGridX, LANCIUS_HIP_ERR_SHAPE, "maxpool2d_bwd: %zu planes", planes);
    hipLaunchKernelGGL(maxpool_bwd_fused, dim3((unsigned)(planes + gather)), dim3(kThreads), 0, ctx->stream, dx, dy,
                       x, planes, (int)H, (int)W, (int)H_out, (int)W_out, (int)K, (int)stride);
    return check_launch("maxpool2d_bwd");
}

}  // extern "C"
