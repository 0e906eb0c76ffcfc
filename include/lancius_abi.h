/*
 * lancius_abi.h - binary-compatible declarations of the Lancius graph types
 * that the MI355X backend reads.
 *
 * The device executor (lancius_hip_graph.h) consumes graphs, schedules and
 * memory plans built by Lancius's own C host code, so the structures below
 * must have exactly the field order, types and enum values of the reference:
 *
 *   lancius_dtype, lancius_memory_owner,
 *   lancius_runtime_state ...... bleeding/v11A1/include/lancius/lancius_types.h:9-60
 *   lancius_opcode ............. bleeding/v11A1/include/lancius/lancius_ir.h:16-29
 *   lancius_node, lancius_graph  bleeding/v11A1/include/lancius/lancius_ir.h:31-62
 *   lancius_node_elements/_bytes bleeding/v11A1/include/lancius/lancius_ir.h:64-78
 *   lancius_wave, lancius_schedule
 *                                bleeding/v11A1/include/lancius/lancius_scheduler.h:10-12
 *   lancius_memory_plan ........ bleeding/v11A1/include/lancius/lancius_memory_planner.h:13-17
 *
 * Every block is skipped when the reference header that defines the same
 * type was included first (its include guard is tested), so a translation
 * unit may include the reference headers and then this one.  The layout is
 * checked field by field against the reference headers by the test suite.
 *
 * Pure C11; no HIP or C++ types.
 */
#ifndef LANCIUS_AMD_ABI_H
#define LANCIUS_AMD_ABI_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#ifndef LANCIUS_TYPES_H
#define LANCIUS_TYPES_H
typedef enum {
    LANCIUS_DTYPE_FP64 = 0,
    LANCIUS_DTYPE_INT8 = 1,
    LANCIUS_DTYPE_FP32 = 2,
    LANCIUS_DTYPE_INT32 = 3
} lancius_dtype;

static inline size_t lancius_dtype_size(lancius_dtype dtype) {
    return dtype == LANCIUS_DTYPE_FP32  ? 4u
         : dtype == LANCIUS_DTYPE_INT8  ? 1u
         : dtype == LANCIUS_DTYPE_INT32 ? 4u
         : 8u;
}

typedef enum {
    LANCIUS_MEMORY_EXTERNAL = 0,
    LANCIUS_MEMORY_ARENA = 1,
    LANCIUS_MEMORY_POOL = 2,
    LANCIUS_MEMORY_OWNED_HEAP = 3
} lancius_memory_owner;

typedef struct lancius_runtime_state {
    void* buffer;
    int8_t* buffer_int8;
    lancius_dtype dtype;
    double scale;
    lancius_memory_owner owner;
    lancius_memory_owner buffer_owner;
    lancius_memory_owner int8_owner;
    size_t offset;
    uint32_t flags;
} lancius_runtime_state;
#endif /* LANCIUS_TYPES_H */

#ifndef Lancius_LANCIUS_IR_H
#define Lancius_LANCIUS_IR_H
/* Opcode numbers are part of the ABI (and of the .lancius file format). */
typedef enum {
    LANCIUS_OP_NOP = 0,
    LANCIUS_OP_INPUT = 1,
    LANCIUS_OP_CONST = 2,
    LANCIUS_OP_ADD = 3,
    LANCIUS_OP_SUB = 4,
    LANCIUS_OP_MUL = 5,
    LANCIUS_OP_MATMUL = 6,
    LANCIUS_OP_RELU = 7,
    LANCIUS_OP_SOFTMAX = 8,
    LANCIUS_OP_SUM = 9,
    LANCIUS_OP_BROADCAST = 10,
    LANCIUS_OP_TRANSPOSE = 11,
    LANCIUS_OP_RELU_BWD = 12,
    LANCIUS_OP_SOFTMAX_BWD = 13,
    LANCIUS_OP_SUM_AXIS0 = 14,
    LANCIUS_OP_SUM_AXIS1 = 15,
    LANCIUS_OP_CONV2D = 16,
    LANCIUS_OP_MAXPOOL2D = 17,
    LANCIUS_OP_FLATTEN = 18,
    LANCIUS_OP_CONV2D_RELU_FUSED = 19,
    LANCIUS_OP_CROSS_ENTROPY = 20,
    LANCIUS_OP_CROSS_ENTROPY_BWD = 21,
    LANCIUS_OP_PERMUTE = 22,
    LANCIUS_OP_MATMUL_BATCHED = 23,
    LANCIUS_OP_CONV2D_BWD = 24,
    LANCIUS_OP_CONV2D_BWD_W = 25,
    LANCIUS_OP_MAXPOOL2D_BWD = 26,
    LANCIUS_OP_RESHAPE = 27,
    LANCIUS_OP_EMBEDDING = 28,
    LANCIUS_OP_LAYERNORM = 29,
    LANCIUS_OP_GELU = 30,
    LANCIUS_OP_ROPE = 31,
    LANCIUS_OP_ATTENTION = 32,
    LANCIUS_OP_KV_CACHE_READ = 33,
    LANCIUS_OP_KV_CACHE_WRITE = 34,
    LANCIUS_OP_RMSNORM = 35,
    LANCIUS_OP_SWIGLU = 36,
    LANCIUS_OP_GQA = 37
} lancius_opcode;

typedef struct lancius_arena lancius_arena;

typedef struct lancius_node {
    uint32_t id;
    lancius_opcode op;
    size_t shape[4];
    uint8_t ndim;
    uint32_t kernel_h, kernel_w, stride, pad;
    uint32_t axes[4];
    const struct lancius_node** inputs;
    uint32_t input_count;
    double attr_val;
    double* runtime_data;        /* host fp64 buffer of the CPU executor */
    lancius_dtype dtype;
    double scale;
    int8_t* runtime_data_int8;
    lancius_runtime_state* rt;
    uint8_t is_view;
    size_t strides[4];
    const struct lancius_node* view_source;
} lancius_node;

typedef struct lancius_graph {
    lancius_arena* arena;
    lancius_node** nodes;
    uint32_t node_count, node_cap, next_id;
    lancius_runtime_state* rt_states;
    size_t rt_cap;
} lancius_graph;

static inline size_t lancius_node_elements(const lancius_node* n) {
    size_t e = 1;
    for (uint8_t d = 0; d < n->ndim; d++) e *= n->shape[d];
    return e;
}

static inline size_t lancius_node_bytes(const lancius_node* n) {
    return n ? lancius_node_elements(n) * lancius_dtype_size(n->dtype) : 0;
}
#endif /* Lancius_LANCIUS_IR_H */

#ifndef Lancius_LANCIUS_SCHEDULER_H
#define Lancius_LANCIUS_SCHEDULER_H
typedef struct { lancius_node** nodes; uint32_t node_count; } lancius_wave;
struct lancius_memory_plan;
typedef struct {
    lancius_wave* waves;
    uint32_t wave_count;
    struct lancius_memory_plan* plan;
    void* static_pool;
} lancius_schedule;
#endif /* Lancius_LANCIUS_SCHEDULER_H */

#ifndef LANCIUS_MEMORY_PLANNER_H
#define LANCIUS_MEMORY_PLANNER_H
typedef struct lancius_memory_plan {
    size_t peak_memory;   /* bytes of the flat buffer */
    size_t* offsets;      /* [graph->next_id] byte offset of each pooled node */
    uint8_t* is_pooled;   /* [graph->next_id] 1 when offsets[id] is valid */
} lancius_memory_plan;
#endif /* LANCIUS_MEMORY_PLANNER_H */

/* Where each INPUT tensor's bytes sit in a .lancius model file: filled by
 * lancius_graph_load_mapped (liblancius_graph), read by
 * lancius_device_upload_weights (liblancius_hip).  No reference counterpart. */
#ifndef LANCIUS_AMD_WEIGHT_MAP_H
#define LANCIUS_AMD_WEIGHT_MAP_H
typedef struct {
    const lancius_node* node; /* INPUT node of the loaded graph */
    uint64_t file_offset;     /* first byte of the tensor in the file */
    uint64_t elements;        /* lancius_node_elements(node) */
    lancius_dtype file_dtype; /* encoding in the file: FP64, FP32 or INT8 */
    double scale;             /* int8 scale (also in node->scale) */
} lancius_weight_ref;

typedef struct {
    uint32_t format;          /* 9, 10, or 2 */
    uint32_t count;           /* entries of refs */
    lancius_weight_ref* refs; /* malloc'd; lancius_weight_map_free */
    uint64_t file_bytes;
    uint32_t crc32;           /* v2: the verified header checksum; else 0 */
} lancius_weight_map;
#endif /* LANCIUS_AMD_WEIGHT_MAP_H */

#ifdef __cplusplus
}
#endif

#endif /* LANCIUS_AMD_ABI_H */
