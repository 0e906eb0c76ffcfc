// Model-file tensors to HBM: the file is read with pread into three pinned
// host pieces in turn (kept in the context); each filled piece is copied to
// the device asynchronously on the context's stream while the host reads the
// next, and fp64 or int8 pieces are converted to fp32 by a kernel on the
// device from a staging slot of the context workspace.  An event per piece
// keeps the host from refilling a piece whose copy has not finished.
#include <errno.h>
#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>

#include "common.hpp"

namespace lancius {
namespace {

constexpr size_t kPiece = (size_t)16 << 20;  // bytes per staging buffer

// f64 -> f32, round to nearest (the conversion instruction's default mode).
__global__ void __launch_bounds__(256) f64_to_f32(float* __restrict__ dst, const double* __restrict__ src, size_t n) {
    const size_t step = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += step) dst[i] = (float)src[i];
}

// int8 -> f32: (float)((double)q * scale).
__global__ void __launch_bounds__(256) i8_to_f32(float* __restrict__ dst, const int8_t* __restrict__ src, double scale,
                                                 size_t n) {
    const size_t step = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += step)
        dst[i] = (float)((double)src[i] * scale);
}

size_t file_elem_bytes(int dt) { return dt == LANCIUS_HIP_FILE_I8 ? 1 : dt == LANCIUS_HIP_FILE_F32 ? 4 : 8; }

int read_fully(int fd, void* dst, size_t bytes, uint64_t offset) {
    char* p = (char*)dst;
    while (bytes) {
        const ssize_t got = pread(fd, p, bytes, (off_t)offset);
        if (got < 0 && errno == EINTR) continue;
        if (got <= 0) return -1;
        p += got;
        bytes -= (size_t)got;
        offset += (uint64_t)got;
    }
    return 0;
}

constexpr int kStages = 3;

// Waits for every staging piece still in flight (on an error path the
// copies enqueued so far must finish before the caller reuses anything).
struct Drain {
    lancius_hip_ctx* ctx;
    bool enqueued = false;
    int fd = -1;
    ~Drain() {
        if (enqueued) (void)hipStreamSynchronize(ctx->stream);
        if (fd >= 0) close(fd);
    }
};

}  // namespace
}  // namespace lancius

using namespace lancius;

extern "C" int lancius_hip_upload_file(lancius_hip_ctx* ctx, const char* path, size_t count,
                                       const lancius_hip_file_tensor* tensors) {
    LANCIUS_REQUIRE(ctx && path && (count == 0 || tensors), LANCIUS_HIP_ERR_NULL_PTR, "upload_file: NULL argument");
    LANCIUS_REQUIRE(!ctx->capturing, LANCIUS_HIP_ERR_UNSUPPORTED, "upload_file: the context is capturing a graph");
    Drain st{ctx};
    st.fd = open(path, O_RDONLY | O_CLOEXEC);
    LANCIUS_REQUIRE(st.fd >= 0, LANCIUS_HIP_ERR_UNSUPPORTED, "upload_file: cannot open %s", path);
    struct stat sb;
    LANCIUS_REQUIRE(fstat(st.fd, &sb) == 0, LANCIUS_HIP_ERR_UNSUPPORTED, "upload_file: cannot stat %s", path);
    const uint64_t file_size = (uint64_t)sb.st_size;
    bool convert = false;
    for (size_t t = 0; t < count; ++t) {
        const lancius_hip_file_tensor& x = tensors[t];
        LANCIUS_REQUIRE(x.dst || x.elements == 0, LANCIUS_HIP_ERR_NULL_PTR, "upload_file: tensor %zu has no destination",
                        t);
        const bool same = (x.dst_dtype == LANCIUS_HIP_FILE_F32 && x.file_dtype == LANCIUS_HIP_FILE_F32) ||
                          (x.dst_dtype == LANCIUS_HIP_FILE_I8 && x.file_dtype == LANCIUS_HIP_FILE_I8);
        const bool conv = x.dst_dtype == LANCIUS_HIP_FILE_F32 &&
                          (x.file_dtype == LANCIUS_HIP_FILE_F64 || x.file_dtype == LANCIUS_HIP_FILE_I8);
        LANCIUS_REQUIRE(same || conv, LANCIUS_HIP_ERR_DTYPE, "upload_file: tensor %zu: file dtype %d to device dtype %d",
                        t, x.file_dtype, x.dst_dtype);
        convert = convert || conv;
        const uint64_t bytes = x.elements * file_elem_bytes(x.file_dtype);
        LANCIUS_REQUIRE(x.elements < ((uint64_t)1 << 40) && x.file_offset <= file_size &&
                            bytes <= file_size - x.file_offset,
                        LANCIUS_HIP_ERR_SHAPE, "upload_file: tensor %zu (%llu bytes at %llu) beyond the file (%llu bytes)",
                        t, (unsigned long long)bytes, (unsigned long long)x.file_offset,
                        (unsigned long long)file_size);
    }
    if (int rc = bind_device(ctx)) return rc;
    // pinned pieces and their events live in the context (allocated once)
    for (int s = 0; s < kStages; ++s) {
        if (!ctx->host_stage[s])
            LANCIUS_HIP_TRY(hipHostMalloc(&ctx->host_stage[s], kPiece, hipHostMallocDefault), "hipHostMalloc(staging)");
        if (!ctx->stage_done[s])
            LANCIUS_HIP_TRY(hipEventCreateWithFlags(&ctx->stage_done[s], hipEventDisableTiming), "hipEventCreate");
    }
    char* dev_stage = nullptr;  // conversions read their piece from the context workspace
    if (convert) {
        void* ws = nullptr;
        if (int rc = workspace(ctx, kStages * kPiece, &ws)) return rc;
        dev_stage = (char*)ws;
    }
    int slot = 0;
    bool used[kStages] = {false, false, false};
    for (size_t t = 0; t < count; ++t) {
        const lancius_hip_file_tensor& x = tensors[t];
        const size_t eb = file_elem_bytes(x.file_dtype);
        const size_t per_piece = kPiece / eb;  // whole elements per piece
        for (uint64_t e0 = 0; e0 < x.elements; e0 += per_piece) {
            const size_t n = (size_t)std::min<uint64_t>(per_piece, x.elements - e0);
            const size_t bytes = n * eb;
            if (used[slot]) LANCIUS_HIP_TRY(hipEventSynchronize(ctx->stage_done[slot]), "hipEventSynchronize(staging)");
            void* host = ctx->host_stage[slot];
            LANCIUS_REQUIRE(read_fully(st.fd, host, bytes, x.file_offset + e0 * eb) == 0,
                            LANCIUS_HIP_ERR_UNSUPPORTED, "upload_file: read of %s failed", path);
            st.enqueued = true;
            if (x.dst_dtype == x.file_dtype) {
                char* dst = (char*)x.dst + e0 * eb;
                LANCIUS_HIP_TRY(hipMemcpyAsync(dst, host, bytes, hipMemcpyHostToDevice, ctx->stream),
                                "hipMemcpyAsync(upload_file)");
            } else {
                char* stage = dev_stage + (size_t)slot * kPiece;
                LANCIUS_HIP_TRY(hipMemcpyAsync(stage, host, bytes, hipMemcpyHostToDevice, ctx->stream),
                                "hipMemcpyAsync(upload_file)");
                float* dst = (float*)x.dst + e0;
                const unsigned grid = (unsigned)std::min<size_t>(4096, (n + 255) / 256);
                if (x.file_dtype == LANCIUS_HIP_FILE_F64)
                    hipLaunchKernelGGL(f64_to_f32, dim3(grid), dim3(256), 0, ctx->stream, dst,
                                       (const double*)stage, n);
                else
                    hipLaunchKernelGGL(i8_to_f32, dim3(grid), dim3(256), 0, ctx->stream, dst,
                                       (const int8_t*)stage, x.scale, n);
                if (int rc = check_launch("upload_file convert")) return rc;
            }
            LANCIUS_HIP_TRY(hipEventRecord(ctx->stage_done[slot], ctx->stream), "hipEventRecord(staging)");
            used[slot] = true;
            slot = (slot + 1) % kStages;
        }
    }
    LANCIUS_HIP_TRY(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize(upload_file)");
    st.enqueued = false;
    return ok();
}
