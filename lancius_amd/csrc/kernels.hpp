// Device-side building blocks shared by the kernels: MFMA vector types,
// epilogue math and the workgroup -> tile mapping.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

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

// Activation codes match LANCIUS_HIP_ACT_* in lancius_hip.h.
enum : int { kActNone = 0, kActRelu = 1, kActGelu = 2, kActTanh = 3 };

// max(x, 0) written as the reference's comparison (NaN maps to 0):
// bleeding/v11A1/src/runtime/lancius_scheduler.c:307.
__device__ __forceinline__ float relu_ref(float x) { return x > 0.0f ? x : 0.0f; }

// tanh-approximation GELU with the +-100 input clamp of
// bleeding/v11A1/src/math/lancius_kernels.c:238-246 (NaN passes through).
__device__ __forceinline__ float gelu_ref(float x) {
    x = x > 100.0f ? 100.0f : x;
    x = x < -100.0f ? -100.0f : x;
    const float k0 = 0.7978845608028654f;  // sqrt(2/pi)
    const float u = k0 * (x + 0.044715f * x * x * x);
    return 0.5f * x * (1.0f + tanhf(u));
}

__device__ __forceinline__ float apply_act(float x, int act) {
    if (act == kActRelu) return relu_ref(x);
    if (act == kActGelu) return gelu_ref(x);
    if (act == kActTanh) return tanhf(x);
    return x;
}

}  // namespace lancius
