// Device ceilings for roofline reporting: the sustained fp32 MFMA rate and
// the HBM copy and read bandwidths of this GPU (lancius_hip_peak_probe).
#include "common.hpp"
#include "kernels.hpp"

namespace lancius {
namespace {

constexpr int kChains = 8;  // independent accumulators per wave

// Every wave issues `iters` rounds of kChains independent
// v_mfma_f32_32x32x2_f32.  The accumulators carry from round to round, so
// nothing folds; the A/B operands stay fixed, so no VALU instruction sits
// between the MFMAs (changing them every round - a VALU write of an MFMA
// source each round - measured 135 TFLOP/s against 144-154 without).
__global__ void __launch_bounds__(256) mfma_rate(float* out, int iters) {
    f32x16 acc[kChains];
#pragma unroll
    for (int c = 0; c < kChains; ++c)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[c][r] = 0.0f;
    float a = 1.0f + 1e-7f * threadIdx.x, b = 1.0f - 1e-7f * blockIdx.x;
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int c = 0; c < kChains; ++c) acc[c] = __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, acc[c], 0, 0, 0);
    }
    float s = 0.0f;
#pragma unroll
    for (int c = 0; c < kChains; ++c)
#pragma unroll
        for (int r = 0; r < 16; ++r) s += acc[c][r];
    if (s == 1234.5f) out[blockIdx.x * blockDim.x + threadIdx.x] = s;  // keeps the loop alive
}

// Streaming probes: every workgroup walks its own contiguous chunk of
// per_wg float4s with kInFlight loads in flight per thread (per_wg is a
// multiple of kInFlight * 256).  Measured on MI355X this pattern beats a
// grid-stride walk (1 GiB read 6.1 against 5.0 TB/s; the grid-stride copy
// with 4 loads in flight read 4.4 TB/s).
constexpr int kInFlight = 8;

__global__ void __launch_bounds__(256) copy_f4(f32x4* __restrict__ dst, const f32x4* __restrict__ src,
                                               size_t per_wg) {
    const size_t base = (size_t)blockIdx.x * per_wg + threadIdx.x;
    for (size_t i = 0; i < per_wg; i += kInFlight * 256) {
        f32x4 v[kInFlight];
#pragma unroll
        for (int u = 0; u < kInFlight; ++u) v[u] = src[base + i + u * 256];
#pragma unroll
        for (int u = 0; u < kInFlight; ++u) __builtin_nontemporal_store(v[u], dst + base + i + u * 256);
    }
}

// Read-only stream; one float per thread is stored so the loads stay live.
__global__ void __launch_bounds__(256) read_f4(float* __restrict__ out, const f32x4* __restrict__ src,
                                               size_t per_wg) {
    const size_t base = (size_t)blockIdx.x * per_wg + threadIdx.x;
    f32x4 a = {0.f, 0.f, 0.f, 0.f};
    for (size_t i = 0; i < per_wg; i += kInFlight * 256) {
        f32x4 v[kInFlight];
#pragma unroll
        for (int u = 0; u < kInFlight; ++u) v[u] = src[base + i + u * 256];
#pragma unroll
        for (int u = 0; u < kInFlight; ++u) a += v[u];
    }
    out[(size_t)blockIdx.x * 256 + threadIdx.x] = a.x + a.y + a.z + a.w;
}

}  // namespace
}  // namespace lancius

using namespace lancius;

extern "C" int lancius_hip_peak_probe(lancius_hip_ctx* ctx, int which, double* result) {
    LANCIUS_REQUIRE(ctx && result, LANCIUS_HIP_ERR_NULL_PTR, "peak_probe: NULL argument");
    LANCIUS_REQUIRE(which >= 0 && which <= 2, LANCIUS_HIP_ERR_UNSUPPORTED, "peak_probe: which=%d", which);
    if (int rc = bind_device(ctx)) return rc;
    hipDeviceProp_t prop;
    LANCIUS_HIP_TRY(hipGetDeviceProperties(&prop, ctx->device), "hipGetDeviceProperties");
    hipEvent_t e0, e1;
    LANCIUS_HIP_TRY(hipEventCreate(&e0), "hipEventCreate");
    LANCIUS_HIP_TRY(hipEventCreate(&e1), "hipEventCreate");
    int rc = 0;
    float ms = 0.0f;
    if (which == 0) {
        // 8 waves per CU (2 per SIMD) keep every MFMA pipe busy.
        const int blocks = prop.multiProcessorCount * 2;
        const int iters = 4096;
        float* out = nullptr;
        hipError_t e = hipMalloc(&out, (size_t)blocks * 256 * sizeof(float));
        if (e == hipSuccess) {
            // The clock settles over the first milliseconds of MFMA load: one
            // untimed launch, then the fastest of three timed ones.
            hipLaunchKernelGGL(mfma_rate, dim3(blocks), dim3(256), 0, ctx->stream, out, iters);
            for (int rep = 0; rep < 3 && e == hipSuccess; ++rep) {
                float t = 0.0f;
                (void)hipEventRecord(e0, ctx->stream);
                hipLaunchKernelGGL(mfma_rate, dim3(blocks), dim3(256), 0, ctx->stream, out, iters);
                (void)hipEventRecord(e1, ctx->stream);
                e = hipEventSynchronize(e1);
                if (e == hipSuccess) e = hipEventElapsedTime(&t, e0, e1);
                if (e == hipSuccess && (rep == 0 || t < ms)) ms = t;
            }
            (void)hipFree(out);
        }
        if (e != hipSuccess) rc = from_hip(e, "mfma probe");
        const double flops = (double)blocks * 4 /*waves*/ * iters * kChains * 32.0 * 32.0 * 2.0 * 2.0;
        if (!rc) *result = flops / (ms * 1e-3) / 1e12;
    } else {
        // 1 GiB, four times the 256 MB last-level cache: HBM, not cache, bandwidth
        const size_t bytes = (size_t)1 << 30;
        const unsigned blocks = 2048;
        const size_t per_wg = bytes / 16 / blocks;  // 32768 float4s, a multiple of kInFlight * 256
        void *a = nullptr, *b = nullptr;
        hipError_t e = hipMalloc(&a, bytes);
        if (e == hipSuccess) e = hipMalloc(&b, which == 1 ? bytes : (size_t)blocks * 256 * sizeof(float));
        if (e == hipSuccess) e = hipMemsetAsync(a, 0, bytes, ctx->stream);
        auto launch = [&] {
            if (which == 1)
                hipLaunchKernelGGL(copy_f4, dim3(blocks), dim3(256), 0, ctx->stream, (f32x4*)b, (const f32x4*)a,
                                   per_wg);
            else
                hipLaunchKernelGGL(read_f4, dim3(blocks), dim3(256), 0, ctx->stream, (float*)b, (const f32x4*)a,
                                   per_wg);
        };
        if (e == hipSuccess) {
            launch();
            launch();
            (void)hipEventRecord(e0, ctx->stream);
            for (int r = 0; r < 5; ++r) launch();
            (void)hipEventRecord(e1, ctx->stream);
            e = hipEventSynchronize(e1);
            if (e == hipSuccess) e = hipEventElapsedTime(&ms, e0, e1);
        }
        if (a) (void)hipFree(a);
        if (b) (void)hipFree(b);
        if (e != hipSuccess) rc = from_hip(e, which == 1 ? "copy probe" : "read probe");
        if (!rc) *result = 5.0 * (which == 1 ? 2.0 : 1.0) * (double)bytes / (ms * 1e-3) / 1e9;
    }
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    return rc ? rc : ok();
}
