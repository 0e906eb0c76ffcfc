/*
 * lancius_graph.h - the C host side of the Lancius graph path, rebuilt for the
 * MI355X backend: graph IR builders, wave scheduler, linear-scan memory planner
 * and the Conv+ReLU fusion pass (library liblancius_graph).
 *
 * Names, signatures, struct layouts (lancius_abi.h) and results follow the
 * reference so that a program written against the reference headers builds
 * graphs with either library:
 *   builders ............ bleeding/v11A1/src/ir/lancius_ir.c:72-299
 *   lancius_ir_schedule . bleeding/v11A1/src/runtime/lancius_scheduler.c:12-59
 *   planner ............. bleeding/v11A1/src/runtime/lancius_memory_planner.c:33-182
 *   fusion .............. bleeding/v11A1/src/compiler/lancius_optimizer.c:15-41
 *   arena ............... bleeding/v11A1/src/core/lancius_arena.c:30-100
 *   errors .............. bleeding/v11A1/src/core/lancius_error.c:5-34
 *
 * One deliberate difference: the reference planner never stores the offset it
 * assigns into its active-interval list (lancius_memory_planner.c:140,167), so
 * every block it frees re-enters the free list at offset 0 and later tensors
 * can overlap live ones.  lancius_build_memory_plan here runs the same
 * first-fit / LIFO / no-coalescing / sink-pinning scan with the offset kept,
 * which gives identical offsets whenever the reference's are overlap-free.
 */
#ifndef LANCIUS_AMD_GRAPH_H
#define LANCIUS_AMD_GRAPH_H

#include "lancius_abi.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ---- errors (lancius_error.h:6-18) ---- */
#ifndef LANCIUS_ERROR_H
#define LANCIUS_ERROR_H
typedef enum {
    LANCIUS_ERROR_OK = 0,
    LANCIUS_ERROR_OOM = -1,
    LANCIUS_ERROR_NULL_PTR = -2,
    LANCIUS_ERROR_SHAPE_MISMATCH = -3,
    LANCIUS_ERROR_UNSUPPORTED_OP = -4,
    LANCIUS_ERROR_UNSUPPORTED_DTYPE = -5,
    LANCIUS_ERROR_INVALID_MODEL = -6,
    LANCIUS_ERROR_VERSION_MISMATCH = -7,
    LANCIUS_ERROR_IO = -8,
    LANCIUS_ERROR_OVERFLOW = -9,
    LANCIUS_ERROR_INTERNAL = -10
} lancius_error;
void lancius_set_error(lancius_error err);
lancius_error lancius_get_error(void);
void lancius_clear_error(void);
const char* lancius_error_string(lancius_error err);
#endif

/* ---- host bump arena (lancius_arena.h:12-15) ---- */
lancius_arena* lancius_arena_create(size_t block_size);
void* lancius_arena_alloc(lancius_arena* arena, size_t size, size_t alignment);
void lancius_arena_reset(lancius_arena* arena);
void lancius_arena_destroy(lancius_arena* arena);

/* ---- graph IR (lancius_ir.h:80-123, the ops on the device path) ---- */
lancius_graph* lancius_graph_create(void);
void lancius_graph_destroy(lancius_graph* g);

lancius_node* lancius_input(lancius_graph* g, size_t r, size_t c);
lancius_node* lancius_input_4d(lancius_graph* g, size_t n, size_t c, size_t h, size_t w);
lancius_node* lancius_const(lancius_graph* g, double val, size_t r, size_t c);
lancius_node* lancius_add(lancius_graph* g, const lancius_node* a, const lancius_node* b);
lancius_node* lancius_matmul(lancius_graph* g, const lancius_node* a, const lancius_node* b);
lancius_node* lancius_relu(lancius_graph* g, const lancius_node* a);
lancius_node* lancius_softmax(lancius_graph* g, const lancius_node* a);
lancius_node* lancius_broadcast(lancius_graph* g, const lancius_node* a, size_t r, size_t c);
lancius_node* lancius_conv2d(lancius_graph* g, const lancius_node* in, const lancius_node* w, uint32_t stride,
                             uint32_t pad);
lancius_node* lancius_flatten(lancius_graph* g, const lancius_node* in);
lancius_node* lancius_reshape(lancius_graph* g, const lancius_node* in, uint8_t ndim, size_t s0, size_t s1, size_t s2,
                              size_t s3);
lancius_node* lancius_attention(lancius_graph* g, const lancius_node* q, const lancius_node* k, const lancius_node* v);
lancius_node* lancius_layernorm(lancius_graph* g, const lancius_node* in, const lancius_node* gamma,
                                const lancius_node* beta);
lancius_node* lancius_gelu(lancius_graph* g, const lancius_node* in);

/* Builders of the training graph (lancius_ir.c:92-97,164-177,207-241,263-280,300-368). */
lancius_node* lancius_sub(lancius_graph* g, const lancius_node* a, const lancius_node* b);
lancius_node* lancius_mul(lancius_graph* g, const lancius_node* a, const lancius_node* b);
lancius_node* lancius_sum(lancius_graph* g, const lancius_node* a);
lancius_node* lancius_transpose(lancius_graph* g, const lancius_node* a);
lancius_node* lancius_relu_bwd(lancius_graph* g, const lancius_node* grad, const lancius_node* fwd_a);
lancius_node* lancius_softmax_bwd(lancius_graph* g, const lancius_node* grad, const lancius_node* fwd_y);
lancius_node* lancius_sum_axis0(lancius_graph* g, const lancius_node* a);
lancius_node* lancius_sum_axis1(lancius_graph* g, const lancius_node* a);
lancius_node* lancius_broadcast_4d(lancius_graph* g, const lancius_node* a, size_t n, size_t c, size_t h, size_t w);
lancius_node* lancius_maxpool2d(lancius_graph* g, const lancius_node* in, uint32_t kernel, uint32_t stride);
lancius_node* lancius_cross_entropy(lancius_graph* g, const lancius_node* logits, const lancius_node* targets);
lancius_node* lancius_cross_entropy_bwd(lancius_graph* g, const lancius_node* logits, const lancius_node* targets,
                                        const lancius_node* grad_out);
lancius_node* lancius_conv2d_bwd(lancius_graph* g, const lancius_node* grad, const lancius_node* fwd_in,
                                 const lancius_node* fwd_w, uint32_t stride, uint32_t pad);
lancius_node* lancius_conv2d_bwd_w(lancius_graph* g, const lancius_node* grad, const lancius_node* fwd_in,
                                   uint32_t k_h, uint32_t k_w, uint32_t stride, uint32_t pad);
lancius_node* lancius_maxpool2d_bwd(lancius_graph* g, const lancius_node* grad, const lancius_node* fwd_in,
                                    uint32_t kernel, uint32_t stride);
/* Decode-side blocks (lancius_ir.c:370-401). */
lancius_node* lancius_rmsnorm(lancius_graph* g, const lancius_node* in, const lancius_node* gamma);
lancius_node* lancius_swiglu(lancius_graph* g, const lancius_node* gate, const lancius_node* up);
lancius_node* lancius_gqa(lancius_graph* g, const lancius_node* q, const lancius_node* k, const lancius_node* v,
                          uint32_t n_heads_q, uint32_t n_heads_kv);
/* Built for autodiff; neither executor runs them (no reference branch either). */
lancius_node* lancius_permute(lancius_graph* g, const lancius_node* in, uint32_t a0, uint32_t a1, uint32_t a2,
                              uint32_t a3);
lancius_node* lancius_matmul_batched(lancius_graph* g, const lancius_node* a, const lancius_node* b);

/* ---- reverse-mode autodiff (lancius_autodiff.h:8-17) ----
 * Copies the forward graph into a new graph and appends the vector-Jacobian
 * products of every node back to `loss_node`; grad_nodes[id] (for the ids of
 * the FORWARD graph, max_id of them) is the gradient node of that forward
 * node in the new graph, or NULL.  Same construction, node order and result
 * as lancius_autodiff.c:44-207. */
#ifndef Lancius_LANCIUS_AUTODIFF_H
#define Lancius_LANCIUS_AUTODIFF_H
typedef struct {
    lancius_graph* graph;
    lancius_node* loss_node;
    lancius_node** grad_nodes;
    uint32_t max_id;
} lancius_training_graph;
lancius_training_graph* lancius_ir_autodiff(lancius_graph* fwd_g, lancius_node* loss_node);
void lancius_training_graph_destroy(lancius_training_graph* tg);
#endif

/* Per-tensor int8 quantization of conv filters (lancius_quantize.c:6-33,
 * declared at lancius_ir.h:118): every 4-D INPUT with bound fp64 data gets
 * runtime_data_int8, scale and dtype INT8 (graph-owned int8 copy). */
void lancius_quantize_graph(lancius_graph* g);

/* Conv2D + ReLU fusion pass (lancius_optimizer.c:15-41). */
void lancius_optimize_fusion(lancius_graph* g);

/* ---- scheduler (lancius_scheduler.h:14-29) ---- */
lancius_schedule* lancius_ir_schedule(lancius_graph* g);
void lancius_schedule_destroy(lancius_schedule* schedule);
void lancius_schedule_attach_pool(lancius_schedule* schedule, void* flat_buffer, struct lancius_memory_plan* plan);
size_t lancius_schedule_peak_memory(lancius_schedule* schedule);

/* ---- memory planner (lancius_memory_planner.h:20-23) ---- */
lancius_memory_plan* lancius_build_memory_plan(lancius_schedule* sched, lancius_graph* g);
void lancius_memory_plan_destroy(lancius_memory_plan* plan);

/* Sets the dtype of every node (e.g. LANCIUS_DTYPE_FP32 before planning the
 * device arena; the reference sizes plan blocks by dtype, lancius_ir.h:75-78),
 * except int8 weights (INPUT nodes of dtype INT8, quantized or loaded as int8,
 * and nodes holding int8 data).  No reference counterpart. */
void lancius_graph_set_dtype(lancius_graph* g, lancius_dtype dtype);

/* ---- .lancius model files (lancius_serialize.c:13-259, lancius_model_format.h) ----
 *
 * Three layouts are read, told apart by their contents:
 *   v10  magic 0x21434E41, node_count, then per node: id u32, op u32, ndim u8,
 *        shape 4 x u64, input_count u32, input ids u32[], attr_val f64,
 *        kernel_h/kernel_w/stride/pad u32[4], axes u32[4], is_view u8
 *        [+ strides 4 x u64, view source id u32], has_weights u8
 *        [+ dtype u8, scale f64, elements x (i8 when dtype INT8, else f64)];
 *        what lancius_graph_save writes (lancius_serialize.c:13-63);
 *   v9   the same records without the is_view byte (stable/v9S, whose
 *        shipped models the reference's v10+ loader cannot read);
 *   v2   the 48-byte header declared in lancius_model_format.h:75-92 (magic
 *        0x32434E41, version 2, CRC-32 of every byte after the header), the
 *        v10 records with each tensor's payload replaced by (elements u64,
 *        offset u64) into a weight block at weight_block_offset (4096-aligned,
 *        every tensor 256-aligned), tensors stored as i8, f32 or f64.
 * The v9/v10 choice is the layout whose records parse and build and end
 * exactly at the end of the file (v10 first); failing that, the first layout
 * whose records parse and build.
 *
 * Nodes are rebuilt with the builders, like lancius_graph_load does, for every
 * op with a builder (the reference loader's subset plus BROADCAST, TRANSPOSE,
 * GELU, the backward ops, SUM_AXIS0/1, PERMUTE, MATMUL_BATCHED, RMSNORM,
 * SWIGLU, GQA); ROPE, EMBEDDING and KV_CACHE_READ/WRITE keep the recorded
 * shape and inputs; NOP and unknown ops are skipped with a warning, as in the
 * reference, and a node that reads a skipped one fails the load.  Stored
 * shapes of built ops are ignored (the builders derive them), as in the
 * reference; kernel_h/kernel_w/stride/pad, axes, attr_val and the view fields
 * are restored.  Any malformed, truncated or out-of-range field fails the load
 * with NULL and LANCIUS_ERROR_INVALID_MODEL (LANCIUS_ERROR_IO when the file
 * cannot be read); limits as in the reference: 1e6 nodes, 16 inputs, 1e8
 * elements per tensor, ids below node_count + 1000. */

/* INPUT weights land in malloc'd fp64 runtime_data (int8 in
 * runtime_data_int8), owned by the graph and freed by lancius_graph_destroy
 * (the reference's graph keeps them until the process ends). */
lancius_graph* lancius_graph_load(const char* path);
/* v10 records, byte for byte what lancius_serialize.c:13-63 writes.  Weights
 * are written for INPUT nodes with data: int8 when dtype is INT8 and an int8
 * copy exists, else fp64.  Sets LANCIUS_ERROR_IO when the file cannot be
 * written. */
void lancius_graph_save(lancius_graph* g, const char* path);

/* v2 container (no reference counterpart: the header is declared there but
 * nothing writes or reads it).  weight_dtype LANCIUS_DTYPE_FP64 stores the
 * fp64 data exactly, LANCIUS_DTYPE_FP32 rounds it to fp32 (half the bytes,
 * the device's own format); int8 tensors stay int8.  Returns 0 or a
 * lancius_error. */
#define LANCIUS_MODEL_MAGIC_V1 0x21434E41u
#define LANCIUS_MODEL_MAGIC_V2 0x32434E41u
#define LANCIUS_MODEL_HEADER_SIZE_V2 48u
#define LANCIUS_MODEL_FLAG_LITTLE_ENDIAN (1u << 0)
#define LANCIUS_MODEL_FLAG_STATIC_GRAPH (1u << 1)
int lancius_graph_save_v2(const lancius_graph* g, const char* path, lancius_dtype weight_dtype);

/* lancius_weight_ref / lancius_weight_map (lancius_abi.h): where each INPUT
 * tensor's bytes sit in a model file, for loaders that move them straight to
 * the device (lancius_device_upload_weights) instead of through host fp64
 * copies. */
/* lancius_graph_load without host weight copies: INPUT nodes with stored data
 * get their dtype and scale but no runtime_data; `map` lists the tensors. */
lancius_graph* lancius_graph_load_mapped(const char* path, lancius_weight_map* map);
void lancius_weight_map_free(lancius_weight_map* map);

/* CRC-32 (IEEE 802.3, reflected polynomial 0xEDB88320, the zlib crc32) of
 * len bytes continuing from crc (0 to start). */
uint32_t lancius_crc32(uint32_t crc, const void* data, size_t len);

#ifdef __cplusplus
}
#endif

#endif /* LANCIUS_AMD_GRAPH_H */
