/*
 * lancius_hip_graph.h - device executor: runs a Lancius graph, scheduled by
 * lancius_ir_schedule and planned by lancius_build_memory_plan, on one MI355X
 * with every intermediate in a single hipMalloc'd HBM arena.
 *
 * It replaces the host executors lancius_schedule_execute / _parallel /
 * _static (bleeding/v11A1/src/runtime/lancius_scheduler.c:311-520) and their
 * dispatch execute_node_math (:61-309) for the ops of the device path:
 * INPUT, CONST, NOP, MATMUL, ADD, BROADCAST, RELU, GELU, SOFTMAX, LAYERNORM,
 * ATTENTION, CONV2D, CONV2D_RELU_FUSED, RESHAPE, FLATTEN; the training ops
 * SUB, MUL, RELU_BWD, TRANSPOSE, SUM, SUM_AXIS0, SUM_AXIS1, SOFTMAX_BWD,
 * CROSS_ENTROPY, CROSS_ENTROPY_BWD, CONV2D_BWD, CONV2D_BWD_W, MAXPOOL2D,
 * MAXPOOL2D_BWD; and RMSNORM, SWIGLU, GQA, ROPE.  MATMUL and conv nodes whose
 * weight operand is an int8 INPUT (dtype INT8 or an int8 copy bound) run on
 * the int8 kernels.
 *
 * Compilation turns the waves into a launch list:
 *  - MATMUL -> ADD(BROADCAST bias) -> RELU|GELU -> ADD(residual) chains whose
 *    intermediates have one consumer become one GEMM with a fused epilogue;
 *  - RESHAPE / FLATTEN become aliases of their input (no copy);
 *  - a TRANSPOSE whose only consumer is a MATMUL is folded into it (the GEMM
 *    reads that operand transposed);
 *  - launches of one wave with the same shape are merged into one grouped
 *    launch (the branches of a batch);
 *  - a small-batch GEMM -> GEMM [-> SOFTMAX] chain (M <= 64 rows, <= 64
 *    outputs) becomes one lancius_hip_mlp2_f32 call (two kernels).
 * Buffer lifetimes are recomputed over that launch list.  The caller's plan
 * offsets are used unchanged (buffer = arena + plan->offsets[id]) when they
 * keep every pair of simultaneously live buffers apart; otherwise the program
 * re-plans with the same first-fit linear scan and reports it (info.replanned).
 * INPUT and CONST tensors, which no plan covers (lancius_memory_planner.c:60),
 * live in a second region of the same allocation.
 *
 * ATTENTION keeps the reference meaning (causal, scale 1/sqrt(D)); a node with
 * axes[0] == 1 runs the non-causal variant (axes survive save/load,
 * lancius_serialize.c:181).
 *
 * Pure C.  All calls return 0 or a negative LANCIUS_HIP_ERR_* code.
 */
#ifndef LANCIUS_HIP_GRAPH_H
#define LANCIUS_HIP_GRAPH_H

#include "lancius_abi.h"
#include "lancius_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct lancius_device_program lancius_device_program;

/* Flags of lancius_device_program_create. */
#define LANCIUS_DEVICE_NO_FUSION 0x1u /* one launch per node, no grouping */
#define LANCIUS_DEVICE_KEEP_ALL  0x2u /* every node keeps its own buffer (readable after run) */
#define LANCIUS_DEVICE_NO_GROUP  0x4u /* fuse epilogues but do not merge branches */
#define LANCIUS_DEVICE_NO_CHAIN 0x10u /* keep a small GEMM -> GEMM -> SOFTMAX chain as separate
                                         launches (default: one lancius_hip_mlp2_f32 call) */
#define LANCIUS_DEVICE_GRAPH     0x8u /* first run: eager + capture into a HIP graph; later runs
                                         replay it on the context's stream (on a null-stream
                                         context: on a private stream, ordered after and before
                                         the null stream by events) */

typedef struct {
    size_t arena_bytes;    /* the one device allocation */
    size_t plan_bytes;     /* region addressed by plan offsets */
    size_t input_bytes;    /* INPUT / CONST / argmax region */
    uint32_t launches;     /* kernel launches per lancius_device_run */
    uint32_t fused_nodes;  /* nodes folded into another node's launch */
    uint32_t aliased_nodes;/* RESHAPE / FLATTEN nodes served by their input's buffer */
    uint32_t replanned;    /* 1 when the caller's plan could not be used as is */
    uint32_t used_caller_plan; /* 1 when buffers sit at the caller's plan offsets */
} lancius_device_program_info;

/* `plan` may be NULL (the program plans its own arena).  The graph, schedule
 * and plan are only read during this call. */
LANCIUS_HIP_EXPORT int lancius_device_program_create(lancius_hip_ctx* ctx, const lancius_graph* g,
                                                     const lancius_schedule* sched,
                                                     const lancius_memory_plan* plan, uint32_t flags,
                                                     lancius_device_program** out);
LANCIUS_HIP_EXPORT void lancius_device_program_destroy(lancius_device_program* prog);
LANCIUS_HIP_EXPORT int lancius_device_program_info_get(const lancius_device_program* prog,
                                                       lancius_device_program_info* info);

/* Copy a host tensor into an INPUT node's device buffer; host_dtype is
 * LANCIUS_DTYPE_FP64 (converted) or LANCIUS_DTYPE_FP32. */
LANCIUS_HIP_EXPORT int lancius_device_upload(lancius_device_program* prog, const lancius_node* n,
                                             const void* host, lancius_dtype host_dtype);
/* Copy a node's device buffer to the host.  Valid for INPUT/CONST nodes,
 * graph sinks, and every node when built with LANCIUS_DEVICE_KEEP_ALL. */
LANCIUS_HIP_EXPORT int lancius_device_download(lancius_device_program* prog, const lancius_node* n, void* host,
                                               lancius_dtype host_dtype);
/* argmax (int32 per row, first maximum) of a SOFTMAX node's output. */
LANCIUS_HIP_EXPORT int lancius_device_download_argmax(lancius_device_program* prog, const lancius_node* n,
                                                      int32_t* host);
/* Every tensor of `map` (from lancius_graph_load_mapped on `path`, for the
 * graph this program was built from) streamed from the file straight into
 * its INPUT buffer in the arena with lancius_hip_upload_file: fp64 and fp32
 * tensors land as fp32, int8 tensors as int8 when the program keeps the node
 * int8 (a weight operand) and dequantized to fp32 otherwise.  Returns when
 * the data is in place.  No reference counterpart (the reference reads
 * weights into host fp64 buffers, lancius_serialize.c:221-240). */
LANCIUS_HIP_EXPORT int lancius_device_upload_weights(lancius_device_program* prog, const char* path,
                                                     const lancius_weight_map* map);
/* Device address of a node's buffer (NULL for fused intermediates).  The
 * caller may write through it between runs.  A weight the program keeps a
 * packed copy of (an int8 MATMUL weight, a conv filter with C_in % 16 == 0)
 * is re-packed at the start of every run once its address has been handed
 * out, so writes through the pointer reach every later run (a few
 * microseconds per weight and run). */
LANCIUS_HIP_EXPORT void* lancius_device_buffer(lancius_device_program* prog, const lancius_node* n);

/* Enqueue one forward pass on the context's stream (asynchronous). */
LANCIUS_HIP_EXPORT int lancius_device_run(lancius_device_program* prog);

/* Drop-in for lancius_schedule_execute: builds a program for `schedule`
 * (using schedule->plan when attached), uploads every INPUT node's host fp64
 * runtime_data, runs, waits, and writes every sink's result into its
 * runtime_data as fp64 (malloc'd and marked LANCIUS_MEMORY_OWNED_HEAP when
 * it was NULL).  CONST nodes are filled with attr_val on the device. */
LANCIUS_HIP_EXPORT int lancius_schedule_execute_device(lancius_schedule* schedule, lancius_graph* g,
                                                       lancius_hip_ctx* ctx);

#ifdef __cplusplus
}
#endif

#endif /* LANCIUS_HIP_GRAPH_H */
