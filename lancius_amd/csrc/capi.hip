// Context, memory, timing and error entry points of liblancius_hip, plus the
// host-pointer bridge kernel_matmul_f32 declared by the reference
// (bleeding/v11A1/include/lancius/lancius_kernels.h:55).
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <mutex>

#include "common.hpp"

namespace lancius {

static thread_local int t_status = 0;
static thread_local char t_message[512] = "success";

int set_error(int code, const char* fmt, ...) {
    t_status = code;
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(t_message, sizeof(t_message), fmt, ap);
    va_end(ap);
    return code;
}

int ok() {
    t_status = 0;
    return 0;
}

int from_hip(hipError_t e, const char* what) {
    // HIP keeps the failure as the thread's pending "last error"; reset it so
    // the launch check of the next, unrelated call (hipGetLastError after
    // <<<>>>) does not report it again.
    (void)hipGetLastError();
    int code = (e == hipErrorOutOfMemory || e == hipErrorMemoryAllocation) ? LANCIUS_HIP_ERR_OOM
                                                                           : LANCIUS_HIP_ERR_INTERNAL;
    return set_error(code, "%s: %s", what, hipGetErrorString(e));
}

int check_launch(const char* kernel) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return from_hip(e, kernel);
    return 0;
}

int cu_count(lancius_hip_ctx* ctx) {
    if (ctx->cus <= 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, ctx->device) != hipSuccess || n <= 0)
            n = 256;  // MI355X
        ctx->cus = n;
    }
    return ctx->cus;
}

int workspace(lancius_hip_ctx* ctx, size_t bytes, void** out) {
    *out = nullptr;
    if (bytes <= ctx->workspace_bytes && ctx->workspace) {
        *out = ctx->workspace;
        return 0;
    }
    LANCIUS_REQUIRE(!ctx->capturing, LANCIUS_HIP_ERR_UNSUPPORTED,
                    "workspace of %zu bytes needed during graph capture: run the launches once before capturing",
                    bytes);
    if (ctx->workspace) {
        LANCIUS_HIP_TRY(hipStreamSynchronize(ctx->stream), "workspace sync");
        LANCIUS_HIP_TRY(hipFree(ctx->workspace), "workspace free");
        ctx->workspace = nullptr;
        ctx->workspace_bytes = 0;
    }
    const size_t want = (bytes + ((size_t)1 << 20) - 1) & ~(((size_t)1 << 20) - 1);
    LANCIUS_HIP_TRY(hipMalloc(&ctx->workspace, want), "workspace hipMalloc");
    ctx->workspace_bytes = want;
    *out = ctx->workspace;
    return 0;
}

__global__ void zero_u32(unsigned* p, size_t n) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        p[i] = 0u;
}

int counters(lancius_hip_ctx* ctx, size_t n, unsigned** out) {
    *out = nullptr;
    if (n <= ctx->counters_n && ctx->counters) {
        *out = ctx->counters;
        return 0;
    }
    LANCIUS_REQUIRE(!ctx->capturing, LANCIUS_HIP_ERR_UNSUPPORTED, "counters needed during graph capture");
    if (ctx->counters) {
        LANCIUS_HIP_TRY(hipStreamSynchronize(ctx->stream), "counters sync");
        LANCIUS_HIP_TRY(hipFree(ctx->counters), "counters free");
        ctx->counters = nullptr;
        ctx->counters_n = 0;
    }
    const size_t want = (n + 4095) & ~(size_t)4095;
    LANCIUS_HIP_TRY(hipMalloc((void**)&ctx->counters, want * sizeof(unsigned)), "counters hipMalloc");
    hipLaunchKernelGGL(zero_u32, dim3(64), dim3(256), 0, ctx->stream, ctx->counters, want);
    if (int rc = check_launch("zero_u32")) return rc;
    ctx->counters_n = want;
    *out = ctx->counters;
    return 0;
}

int bind_device(lancius_hip_ctx* ctx) {
    // A failure of a HIP call whose status was ignored (cleanup paths) must
    // not surface in this call's launch checks.
    (void)hipGetLastError();
    int cur = -1;
    LANCIUS_HIP_TRY(hipGetDevice(&cur), "hipGetDevice");
    if (cur != ctx->device) LANCIUS_HIP_TRY(hipSetDevice(ctx->device), "hipSetDevice");
    return 0;
}

}  // namespace lancius

using namespace lancius;

extern "C" {

const char* lancius_hip_last_error(void) { return t_message; }
int lancius_hip_last_status(void) { return t_status; }

int lancius_hip_device_count(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) {
        (void)hipGetLastError();
        return 0;
    }
    return n;
}

int lancius_hip_ctx_create(int device, void* stream, lancius_hip_ctx** out) {
    LANCIUS_REQUIRE(out != nullptr, LANCIUS_HIP_ERR_NULL_PTR, "ctx_create: out is NULL");
    *out = nullptr;
    int n = 0;
    LANCIUS_HIP_TRY(hipGetDeviceCount(&n), "hipGetDeviceCount");
    LANCIUS_REQUIRE(device >= 0 && device < n, LANCIUS_HIP_ERR_SHAPE, "ctx_create: device %d of %d", device, n);
    LANCIUS_HIP_TRY(hipSetDevice(device), "hipSetDevice");
    lancius_hip_ctx* c = (lancius_hip_ctx*)calloc(1, sizeof(lancius_hip_ctx));
    LANCIUS_REQUIRE(c != nullptr, LANCIUS_HIP_ERR_OOM, "ctx_create: host allocation failed");
    c->device = device;
    c->stream = (hipStream_t)stream;
    hipError_t e = hipEventCreate(&c->ev_start);
    if (e == hipSuccess) e = hipEventCreate(&c->ev_stop);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&c->ev_order, hipEventDisableTiming);
    if (e != hipSuccess) {
        free(c);
        return from_hip(e, "hipEventCreate");
    }
    if (int rc = noalloc_scratch_init(c)) {
        (void)hipEventDestroy(c->ev_start);
        (void)hipEventDestroy(c->ev_stop);
        (void)hipEventDestroy(c->ev_order);
        free(c);
        return rc;
    }
    *out = c;
    return ok();
}

int lancius_hip_ctx_create_own_stream(int device, lancius_hip_ctx** out) {
    LANCIUS_REQUIRE(out != nullptr, LANCIUS_HIP_ERR_NULL_PTR, "ctx_create_own_stream: out is NULL");
    *out = nullptr;
    int n = 0;
    LANCIUS_HIP_TRY(hipGetDeviceCount(&n), "hipGetDeviceCount");
    LANCIUS_REQUIRE(device >= 0 && device < n, LANCIUS_HIP_ERR_SHAPE, "ctx_create: device %d of %d", device, n);
    LANCIUS_HIP_TRY(hipSetDevice(device), "hipSetDevice");
    hipStream_t s = nullptr;
    LANCIUS_HIP_TRY(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "hipStreamCreateWithFlags");
    if (int rc = lancius_hip_ctx_create(device, (void*)s, out)) {
        (void)hipStreamDestroy(s);
        return rc;
    }
    (*out)->owns_stream = 1;
    return ok();
}

void lancius_hip_ctx_destroy(lancius_hip_ctx* ctx) {
    if (!ctx) return;
    (void)bind_device(ctx);
    (void)hipStreamSynchronize(ctx->stream);
    if (ctx->workspace) (void)hipFree(ctx->workspace);
    if (ctx->counters) (void)hipFree(ctx->counters);
    for (int s = 0; s < 3; ++s) {
        if (ctx->host_stage[s]) (void)hipHostFree(ctx->host_stage[s]);
        if (ctx->stage_done[s]) (void)hipEventDestroy(ctx->stage_done[s]);
    }
    (void)hipEventDestroy(ctx->ev_start);
    (void)hipEventDestroy(ctx->ev_stop);
    (void)hipEventDestroy(ctx->ev_order);
    if (ctx->owns_stream) (void)hipStreamDestroy(ctx->stream);
    free(ctx);
}

int lancius_hip_ctx_device(const lancius_hip_ctx* ctx) { return ctx ? ctx->device : -1; }

void* lancius_hip_ctx_stream(const lancius_hip_ctx* ctx) { return ctx ? (void*)ctx->stream : nullptr; }

int lancius_hip_stream_wait(lancius_hip_ctx* waiter, lancius_hip_ctx* signaler) {
    LANCIUS_REQUIRE(waiter && signaler, LANCIUS_HIP_ERR_NULL_PTR, "stream_wait: NULL context");
    if (waiter->stream == signaler->stream) return ok();
    if (int rc = bind_device(signaler)) return rc;
    LANCIUS_HIP_TRY(hipEventRecord(signaler->ev_order, signaler->stream), "hipEventRecord");
    LANCIUS_HIP_TRY(hipStreamWaitEvent(waiter->stream, signaler->ev_order, 0), "hipStreamWaitEvent");
    return ok();
}

int lancius_hip_capture_begin(lancius_hip_ctx* ctx) {
    LANCIUS_REQUIRE(ctx, LANCIUS_HIP_ERR_NULL_PTR, "capture_begin: NULL context");
    LANCIUS_REQUIRE(ctx->stream != nullptr, LANCIUS_HIP_ERR_UNSUPPORTED,
                    "capture_begin: the null stream cannot be captured (use lancius_hip_ctx_create_own_stream)");
    LANCIUS_REQUIRE(!ctx->capturing, LANCIUS_HIP_ERR_UNSUPPORTED, "capture_begin: already capturing");
    if (int rc = bind_device(ctx)) return rc;
    LANCIUS_HIP_TRY(hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
    ctx->capturing = 1;
    return ok();
}

int lancius_hip_capture_end(lancius_hip_ctx* ctx, lancius_hip_graph** out) {
    LANCIUS_REQUIRE(ctx && out, LANCIUS_HIP_ERR_NULL_PTR, "capture_end: NULL argument");
    LANCIUS_REQUIRE(ctx->capturing, LANCIUS_HIP_ERR_UNSUPPORTED, "capture_end without capture_begin");
    *out = nullptr;
    ctx->capturing = 0;
    hipGraph_t graph = nullptr;
    LANCIUS_HIP_TRY(hipStreamEndCapture(ctx->stream, &graph), "hipStreamEndCapture");
    lancius_hip_graph* g = (lancius_hip_graph*)calloc(1, sizeof(lancius_hip_graph));
    if (!g) {
        (void)hipGraphDestroy(graph);
        return set_error(LANCIUS_HIP_ERR_OOM, "capture_end: host allocation failed");
    }
    g->graph = graph;
    hipError_t e = hipGraphInstantiate(&g->exec, graph, nullptr, nullptr, 0);
    if (e != hipSuccess) {
        (void)hipGraphDestroy(graph);
        free(g);
        return from_hip(e, "hipGraphInstantiate");
    }
    *out = g;
    return ok();
}

int lancius_hip_graph_launch(lancius_hip_graph* graph, lancius_hip_ctx* ctx) {
    LANCIUS_REQUIRE(graph && ctx, LANCIUS_HIP_ERR_NULL_PTR, "graph_launch: NULL argument");
    if (int rc = bind_device(ctx)) return rc;
    LANCIUS_HIP_TRY(hipGraphLaunch(graph->exec, ctx->stream), "hipGraphLaunch");
    return ok();
}

void lancius_hip_graph_destroy(lancius_hip_graph* graph) {
    if (!graph) return;
    (void)hipGraphExecDestroy(graph->exec);
    (void)hipGraphDestroy(graph->graph);
    free(graph);
}

int lancius_hip_malloc(lancius_hip_ctx* ctx, void** device_ptr, size_t bytes) {
    LANCIUS_REQUIRE(ctx && device_ptr, LANCIUS_HIP_ERR_NULL_PTR, "malloc: NULL argument");
    *device_ptr = nullptr;
    if (int rc = bind_device(ctx)) return rc;
    LANCIUS_HIP_TRY(hipMalloc(device_ptr, bytes ? bytes : 1), "hipMalloc");
    return ok();
}

int lancius_hip_free(lancius_hip_ctx* ctx, void* device_ptr) {
    LANCIUS_REQUIRE(ctx, LANCIUS_HIP_ERR_NULL_PTR, "free: NULL context");
    if (!device_ptr) return ok();
    if (int rc = bind_device(ctx)) return rc;
    LANCIUS_HIP_TRY(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
    LANCIUS_HIP_TRY(hipFree(device_ptr), "hipFree");
    return ok();
}

int lancius_hip_upload(lancius_hip_ctx* ctx, void* device_dst, const void* host_src, size_t bytes) {
    LANCIUS_REQUIRE(ctx && device_dst && host_src, LANCIUS_HIP_ERR_NULL_PTR, "upload: NULL argument");
    if (int rc = bind_device(ctx)) return rc;
    LANCIUS_HIP_TRY(hipMemcpyAsync(device_dst, host_src, bytes, hipMemcpyHostToDevice, ctx->stream), "upload");
    LANCIUS_HIP_TRY(hipStreamSynchronize(ctx->stream), "upload sync");
    return ok();
}

int lancius_hip_download(lancius_hip_ctx* ctx, void* host_dst, const void* device_src, size_t bytes) {
    LANCIUS_REQUIRE(ctx && host_dst && device_src, LANCIUS_HIP_ERR_NULL_PTR, "download: NULL argument");
    if (int rc = bind_device(ctx)) return rc;
    LANCIUS_HIP_TRY(hipMemcpyAsync(host_dst, device_src, bytes, hipMemcpyDeviceToHost, ctx->stream), "download");
    LANCIUS_HIP_TRY(hipStreamSynchronize(ctx->stream), "download sync");
    return ok();
}

int lancius_hip_synchronize(lancius_hip_ctx* ctx) {
    LANCIUS_REQUIRE(ctx, LANCIUS_HIP_ERR_NULL_PTR, "synchronize: NULL context");
    if (int rc = bind_device(ctx)) return rc;
    LANCIUS_HIP_TRY(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
    return ok();
}

int lancius_hip_timer_start(lancius_hip_ctx* ctx) {
    LANCIUS_REQUIRE(ctx, LANCIUS_HIP_ERR_NULL_PTR, "timer_start: NULL context");
    if (int rc = bind_device(ctx)) return rc;
    LANCIUS_HIP_TRY(hipEventRecord(ctx->ev_start, ctx->stream), "hipEventRecord");
    ctx->timer_armed = 1;
    return ok();
}

int lancius_hip_timer_stop(lancius_hip_ctx* ctx, float* elapsed_ms) {
    LANCIUS_REQUIRE(ctx && elapsed_ms, LANCIUS_HIP_ERR_NULL_PTR, "timer_stop: NULL argument");
    LANCIUS_REQUIRE(ctx->timer_armed, LANCIUS_HIP_ERR_UNSUPPORTED, "timer_stop without timer_start");
    if (int rc = bind_device(ctx)) return rc;
    LANCIUS_HIP_TRY(hipEventRecord(ctx->ev_stop, ctx->stream), "hipEventRecord");
    LANCIUS_HIP_TRY(hipEventSynchronize(ctx->ev_stop), "hipEventSynchronize");
    LANCIUS_HIP_TRY(hipEventElapsedTime(elapsed_ms, ctx->ev_start, ctx->ev_stop), "hipEventElapsedTime");
    ctx->timer_armed = 0;
    return ok();
}

// ---- reference-ABI bridge: host pointers in, host pointers out ----------

static std::mutex g_bridge_mu;
static lancius_hip_ctx* g_bridge_ctx = nullptr;
static void* g_bridge_buf = nullptr;
static size_t g_bridge_cap = 0;

void kernel_matmul_f32(float* out, const float* a, const float* b, size_t M, size_t K, size_t N) {
    if (!out || !a || !b) {
        set_error(LANCIUS_HIP_ERR_NULL_PTR, "kernel_matmul_f32: NULL argument");
        return;
    }
    std::lock_guard<std::mutex> lock(g_bridge_mu);
    if (!g_bridge_ctx && lancius_hip_ctx_create(0, nullptr, &g_bridge_ctx) != 0) return;
    const size_t ea = M * K, eb = K * N, ec = M * N;
    const size_t bytes = (ea + eb + ec) * sizeof(float) + 3 * 256;
    if (bytes > g_bridge_cap) {
        if (g_bridge_buf) lancius_hip_free(g_bridge_ctx, g_bridge_buf);
        g_bridge_buf = nullptr;
        g_bridge_cap = 0;
        if (lancius_hip_malloc(g_bridge_ctx, &g_bridge_buf, bytes) != 0) return;
        g_bridge_cap = bytes;
    }
    auto align = [](size_t x) { return (x + 255) & ~(size_t)255; };
    char* base = (char*)g_bridge_buf;
    float* dA = (float*)base;
    float* dB = (float*)(base + align(ea * sizeof(float)));
    float* dC = (float*)(base + align(ea * sizeof(float)) + align(eb * sizeof(float)));
    if (lancius_hip_upload(g_bridge_ctx, dA, a, ea * sizeof(float)) != 0) return;
    if (lancius_hip_upload(g_bridge_ctx, dB, b, eb * sizeof(float)) != 0) return;
    if (lancius_hip_gemm_f32(g_bridge_ctx, dC, dA, dB, M, K, N, nullptr, LANCIUS_HIP_ACT_NONE, nullptr) != 0) return;
    (void)lancius_hip_download(g_bridge_ctx, out, dC, ec * sizeof(float));
}

}  // extern "C"
