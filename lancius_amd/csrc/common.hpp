// Internal helpers shared by the HIP translation units of liblancius_hip.
// Nothing here is visible through the public C headers.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "lancius_hip.h"

struct lancius_hip_ctx {
    int device;
    hipStream_t stream;
    hipEvent_t ev_start;
    hipEvent_t ev_stop;
    int timer_armed;
    void* workspace;        // split-K partials, transposed conv weights
    size_t workspace_bytes;
    unsigned* counters;     // arrival counters of split reductions, kept at zero between calls
    size_t counters_n;
    int owns_stream;        // stream created by lancius_hip_ctx_create_own_stream
    int capturing;          // between lancius_hip_capture_begin and _end
    hipEvent_t ev_order;    // lancius_hip_stream_wait
    void* host_stage[3];    // pinned staging of lancius_hip_upload_file, kept until destroy
    hipEvent_t stage_done[3];
    int cus;                // compute units of the device (0 until first asked)
};

struct lancius_hip_graph {
    hipGraph_t graph;
    hipGraphExec_t exec;
};

namespace lancius {

// Records a failure in the thread-local status/message and returns the code.
int set_error(int code, const char* fmt, ...);
// Clears the thread-local status and returns 0.
int ok();
// Maps a HIP error to a status (OOM -> -1, everything else -> -10).
int from_hip(hipError_t e, const char* what);

// Checks a kernel launch: reads hipGetLastError() after <<<>>>.
int check_launch(const char* kernel);

// Makes `ctx->device` current for the calling thread.
int bind_device(lancius_hip_ctx* ctx);

// Device scratch owned by the context, grown with hipMalloc on demand and
// kept until the context is destroyed.  Calls on one context are ordered by
// its stream, so one buffer serves every kernel of the context.
int workspace(lancius_hip_ctx* ctx, size_t bytes, void** out);

// Compute units of the context's device (cached in the context).
int cu_count(lancius_hip_ctx* ctx);

// At least n zero-initialised arrival counters (see counters in the context);
// every kernel that increments a counter returns it to zero before exiting.
int counters(lancius_hip_ctx* ctx, size_t n, unsigned** out);

// Device address of lancius_hip_gemm_f32_noalloc's scratch on the
// context's device (current), resolved and its counters cleared once per
// device; called by lancius_hip_ctx_create.
int noalloc_scratch_init(lancius_hip_ctx* ctx);

static inline unsigned int ceil_div(size_t a, size_t b) { return (unsigned int)((a + b - 1) / b); }

// Largest grid dimension we launch in x (hardware limit is 2^32-1 work-items).
constexpr size_t kMaxGridX = (size_t)1 << 30;

}  // namespace lancius

#define LANCIUS_REQUIRE(cond, code, ...)                                  \
    do {                                                                  \
        if (!(cond)) return ::lancius::set_error((code), __VA_ARGS__);    \
    } while (0)

#define LANCIUS_HIP_TRY(expr, what)                                       \
    do {                                                                  \
        hipError_t _e = (expr);                                           \
        if (_e != hipSuccess) return ::lancius::from_hip(_e, (what));     \
    } while (0)
