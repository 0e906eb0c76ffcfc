// Device-side building blocks shared by the kernels: MFMA vector types,
// epilogue math and the workgroup -> tile mapping.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

namespace lancius {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

// MI355X: 256 CUs in 8 XCDs.  Consecutive workgroup ids are dealt round-robin
// to the XCDs, so id i runs on XCD i % 8.  Renumbering so that each XCD owns
// one contiguous range of tiles keeps tiles that share operands in the same
// 4 MB L2.
constexpr int kNumXcd = 8;

__device__ __forceinline__ uint32_t xcd_contiguous_id(uint32_t id, uint32_t count) {
    if (count % kNumXcd != 0) return id;
    return (id % kNumXcd) * (count / kNumXcd) + id / kNumXcd;
}

// Grouped raster: walks `group_m` tile-rows column by column, so that a run of
// consecutive ids reuses a few A row-panels and B column-panels.
__device__ __forceinline__ void grouped_tile(uint32_t id, uint32_t tiles_m, uint32_t tiles_n, uint32_t group_m,
                                             uint32_t& tm, uint32_t& tn) {
    const uint32_t per_group = group_m * tiles_n;
    const uint32_t g = id / per_group;
    const uint32_t first_m = g * group_m;
    const uint32_t gm = min(tiles_m - first_m, group_m);
    const uint32_t in_group = id - g * per_group;
    tm = first_m + in_group % gm;
    tn = in_group / gm;
}

// ---- passing data between workgroups of one launch -------------------------
// The 8 XCDs each have their own L2, and an agent-scope release/acquire
// fence writes back and invalidates an XCD's whole L2 (measured 4x slower
// than a second launch).  Data handed from one workgroup to another instead
// goes through the point of coherence: stored and loaded with the
// device-scope cache policy (sc1: stores written through, loads missing in
// L2), the storing wave waits for its stores to complete (vmcnt 0) before the
// arrival counter's atomic add, and workgroup-scope fences order the rest.
// The workgroup that arrives last (counter == expected - 1) resets the
// counter, so counters are zero between launches.

// s_waitcnt operand that waits for vmcnt 0 and leaves expcnt / lgkmcnt alone.
constexpr int kWaitVmcnt0 = (0x7 << 4) | (0xf << 8);
// Cache-policy operand of the raw buffer load/store builtins on gfx950: sc1,
// device scope (the access is coherent across the XCDs' L2 caches).
constexpr int kCachePolicySc1 = 16;
// Fourth word of a raw buffer resource on gfx9 (32-bit data format).
constexpr int kBufferRsrcWord3 = 0x00020000;
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

// Raw buffer over `bytes` bytes at `base` (bytes < 2^31).
// c ? a : b without a branch.  hipcc tends to turn a select between a
// computed load offset and a constant (the past-the-end offset of a buffer
// load) into an exec-mask branch around the computation, once per load.
__device__ __forceinline__ int pick(bool c, int a, int b) {
    const int m = -(int)c;
    return (a & m) | (b & ~m);
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t coherent_buffer(const void* base, size_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)bytes, kBufferRsrcWord3);
}
__device__ __forceinline__ void store_coherent(__amdgpu_buffer_rsrc_t buf, int byte_off, float v) {
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, v), buf, byte_off, 0, kCachePolicySc1);
}
__device__ __forceinline__ void store_coherent4(__amdgpu_buffer_rsrc_t buf, int byte_off, f32x4 v) {
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), buf, byte_off, 0, kCachePolicySc1);
}
__device__ __forceinline__ float load_coherent(__amdgpu_buffer_rsrc_t buf, int byte_off) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(buf, byte_off, 0, kCachePolicySc1));
}
__device__ __forceinline__ f32x4 load_coherent4(__amdgpu_buffer_rsrc_t buf, int byte_off) {
    return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(buf, byte_off, 0, kCachePolicySc1));
}

// Called by every thread of the workgroup after its coherent stores: true in
// the workgroup that arrives last of `expected` at `*ctr` (which it then owns
// and must reset with reset_arrival once done reading).  s_flag is a
// __shared__ int of the caller.
__device__ __forceinline__ bool arrive_last(unsigned* ctr, unsigned expected, int* s_flag) {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
    __syncthreads();
    if (threadIdx.x == 0)
        *s_flag = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == expected - 1;
    __syncthreads();
    const bool last = *s_flag != 0;
    if (last) {
        __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    }
    return last;
}
__device__ __forceinline__ void reset_arrival(unsigned* ctr) {
    if (threadIdx.x == 0) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Activation codes match LANCIUS_HIP_ACT_* in lancius_hip.h.
enum : int { kActNone = 0, kActRelu = 1, kActGelu = 2, kActTanh = 3 };

// max(x, 0) written as the reference's comparison (NaN maps to 0):
// bleeding/v11A1/src/runtime/lancius_scheduler.c:307.
__device__ __forceinline__ float relu_ref(float x) { return x > 0.0f ? x : 0.0f; }

// tanh-approximation GELU with the +-100 input clamp of
// bleeding/v11A1/src/math/lancius_kernels.c:238-246 (NaN passes through),
// evaluated as 0.5 x (1 + tanh u) = x / (1 + e^(-2u)): one v_exp_f32 and
// one v_rcp_f32 (a few ulp) instead of tanhf's sequence, and no
// cancellation in 1 + tanh u for negative u.  At the clamp, e^(-2u) is 0
// (x = 100 gives 100) or +inf (x = -100 gives -0, as 0.5 x (1 + tanh u)).
__device__ __forceinline__ float gelu_ref(float x) {
    x = x > 100.0f ? 100.0f : x;
    x = x < -100.0f ? -100.0f : x;
    const float k0 = 0.7978845608028654f;  // sqrt(2/pi)
    const float u = k0 * (x + 0.044715f * x * x * x);
    const float e = __builtin_amdgcn_exp2f(-2.8853900817779268f * u);  // e^(-2u) = 2^(-2u log2 e)
    return x * __builtin_amdgcn_rcpf(1.0f + e);
}

__device__ __forceinline__ float apply_act(float x, int act) {
    if (act == kActRelu) return relu_ref(x);
    if (act == kActGelu) return gelu_ref(x);
    if (act == kActTanh) return tanhf(x);
    return x;
}

template <int ACT>
__device__ __forceinline__ float act_fixed(float x) {
    if constexpr (ACT == kActRelu) return relu_ref(x);
    if constexpr (ACT == kActGelu) return gelu_ref(x);
    if constexpr (ACT == kActTanh) return tanhf(x);
    return x;
}

// Calls f(std::integral_constant<int, ACT>) for the activation code act.  A
// fully unrolled epilogue written against the constant holds one
// activation's code per element instead of all four: with hundreds of
// outputs per lane the four-way version is tens of thousands of
// instructions, and fetching them costs more than the stores.
template <typename F>
__device__ __forceinline__ void with_act(int act, F&& f) {
    switch (act) {
        case kActRelu: f(std::integral_constant<int, kActRelu>{}); break;
        case kActGelu: f(std::integral_constant<int, kActGelu>{}); break;
        case kActTanh: f(std::integral_constant<int, kActTanh>{}); break;
        default: f(std::integral_constant<int, kActNone>{}); break;
    }
}

}  // namespace lancius
