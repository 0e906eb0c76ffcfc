/*
 * lancius_basis.h - the BASIS interfaces the backend keeps, in pure C.
 *
 * 1. The BASIS memory API, declared by the reference and implemented
 *    nowhere there (include/basis/core/memory.h:14-29).  liblancius_hip.so
 *    implements it on HBM: an arena or pool hands out DEVICE pointers of the
 *    GPU that was current when it was created.
 * 2. The BASIS static graph IR (include/basis/stage6_ir/graph.h:7-39,
 *    src/basis/stage6_ir/graph.c), which has builders and no executor in
 *    the reference.  liblancius_graph.so provides the builders under the same
 *    names and layouts; liblancius_hip.so adds a device executor
 *    (lancius_basis_program_*), which only reads the structs, so it runs
 *    graphs built by either library.
 *
 * The type declarations sit behind the reference headers' own include
 * guards, so this header may be included before or after them.
 */
#ifndef LANCIUS_BASIS_H
#define LANCIUS_BASIS_H

#include <stddef.h>
#include <stdint.h>

#include "lancius_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

#if defined(_WIN32)
#define LANCIUS_BASIS_EXPORT __declspec(dllexport)
#else
#define LANCIUS_BASIS_EXPORT __attribute__((visibility("default")))
#endif

/* ---- memory: arena and pool (include/basis/core/memory.h:7-29) -------- */

#ifndef BASIS_V7_MEMORY_H
#define BASIS_V7_MEMORY_H
typedef struct basis_arena basis_arena;
typedef struct basis_pool basis_pool;
#endif

/* An arena of HBM blocks on the current device.  basis_arena_alloc bumps a
 * pointer in the current block (alignment: a power of two, 0 means 256) and
 * moves to the next block, or hipMalloc's a new one of
 * max(default_block_size, size + alignment) bytes, when it does not fit.
 * basis_arena_reset rewinds every block in O(1) and keeps them; destroy
 * frees them.  NULL on failure (message in lancius_hip_last_error()).
 * Not thread-safe: one arena per thread or external locking. */
LANCIUS_BASIS_EXPORT basis_arena* basis_arena_create(size_t default_block_size);
LANCIUS_BASIS_EXPORT void* basis_arena_alloc(basis_arena* arena, size_t size, size_t alignment);
LANCIUS_BASIS_EXPORT void basis_arena_reset(basis_arena* arena);
LANCIUS_BASIS_EXPORT void basis_arena_destroy(basis_arena* arena);

/* A pool of fixed-size HBM objects (object_size rounded up to 256 bytes)
 * carved from chunks of objects_per_chunk objects.  The free list lives in
 * host memory: alloc pops it (a new chunk when it is empty) and free pushes
 * to it, host operations only, after a scan over the pool's chunks that
 * checks the pointer; freeing NULL, a pointer the pool did not hand out or
 * an object twice is ignored. */
LANCIUS_BASIS_EXPORT basis_pool* basis_pool_create(size_t object_size, size_t objects_per_chunk);
LANCIUS_BASIS_EXPORT void* basis_pool_alloc(basis_pool* pool);
LANCIUS_BASIS_EXPORT void basis_pool_free(basis_pool* pool, void* ptr);
LANCIUS_BASIS_EXPORT void basis_pool_destroy(basis_pool* pool);

/* Bytes of HBM the arena / pool holds (diagnostics and tests). */
LANCIUS_BASIS_EXPORT size_t lancius_basis_arena_capacity(const basis_arena* arena);
LANCIUS_BASIS_EXPORT size_t lancius_basis_pool_capacity(const basis_pool* pool);

/* ---- static graph IR (include/basis/stage6_ir/graph.h:7-39) ------------- */

#ifndef BASIS_STAGE6_IR_GRAPH_H
#define BASIS_STAGE6_IR_GRAPH_H
typedef enum {
    BASIS_OP_INPUT,
    BASIS_OP_MATMUL,
    BASIS_OP_ADD,
    BASIS_OP_RELU,
    BASIS_OP_TANH,
    BASIS_OP_BROADCAST_ADD
} basis_op_type;

typedef struct basis_node {
    int id;
    basis_op_type op;
    int input_ids[2];
    size_t rows;
    size_t cols;
    char* name;
} basis_node;

typedef struct basis_graph {
    basis_node* nodes;
    size_t node_count;
    size_t node_cap;
} basis_graph;

/* Builders (liblancius_graph.so).  Nodes live in one array that grows by
 * realloc, so a basis_node* stays valid only until the next builder call
 * that adds a node; ids are stable.  Shape errors print to stderr and
 * return NULL (graph.c:39-70). */
basis_graph* basis_graph_new(void);
basis_node* basis_graph_input(basis_graph* g, const char* name, size_t r, size_t c);
basis_node* basis_graph_matmul(basis_graph* g, basis_node* a, basis_node* b);
basis_node* basis_graph_add(basis_graph* g, basis_node* a, basis_node* b);
basis_node* basis_graph_broadcast_add(basis_graph* g, basis_node* a, basis_node* bias);
basis_node* basis_graph_relu(basis_graph* g, basis_node* a);
basis_node* basis_graph_tanh(basis_graph* g, basis_node* a);
void basis_graph_print(basis_graph* g);
void basis_graph_free(basis_graph* g);
#endif

/* ---- device executor for BASIS graphs (liblancius_hip.so) --------------- */

/* Every node is an fp32 [rows x cols] row-major tensor.  Semantics:
 * MATMUL = a . b, ADD = a + b, BROADCAST_ADD = a + bias[0, c] per row,
 * RELU = max(x, 0) (NaN -> 0), TANH = tanh(x).
 *
 * create compiles the graph in node-id order: a MATMUL whose result has one
 * consumer absorbs a following BROADCAST_ADD, then RELU or TANH, then an
 * ADD with an earlier tensor, into the GEMM's epilogue (that order only),
 * and a BROADCAST_ADD absorbs a following RELU or TANH; the rest run as
 * elementwise kernels.  Every node that is not absorbed gets its buffer in
 * one HBM basis_arena sized for the whole graph; absorbed nodes have none
 * (flags LANCIUS_BASIS_KEEP_ALL keeps every node).  The graph must stay
 * alive and unchanged while the program exists.
 *
 * upload / download copy host fp32 data of exactly rows*cols elements
 * (count) to an INPUT node / from any node that has a buffer; run launches
 * the graph on the context's stream. */
typedef struct lancius_basis_program lancius_basis_program;

#define LANCIUS_BASIS_KEEP_ALL 0x1u

LANCIUS_BASIS_EXPORT int lancius_basis_program_create(lancius_hip_ctx* ctx, const basis_graph* g, unsigned flags,
                                                      lancius_basis_program** out);
LANCIUS_BASIS_EXPORT int lancius_basis_program_upload(lancius_basis_program* p, int node_id, const float* host,
                                                      size_t count);
LANCIUS_BASIS_EXPORT int lancius_basis_program_run(lancius_basis_program* p);
LANCIUS_BASIS_EXPORT int lancius_basis_program_download(lancius_basis_program* p, int node_id, float* host,
                                                        size_t count);
/* Device address of a node's buffer, or NULL when the node was absorbed. */
LANCIUS_BASIS_EXPORT float* lancius_basis_program_buffer(lancius_basis_program* p, int node_id);
/* Kernel launches per run and bytes of the program's HBM arena. */
LANCIUS_BASIS_EXPORT int lancius_basis_program_info(const lancius_basis_program* p, size_t* launches,
                                                    size_t* arena_bytes);
LANCIUS_BASIS_EXPORT void lancius_basis_program_destroy(lancius_basis_program* p);

#ifdef __cplusplus
}
#endif

#endif /* LANCIUS_BASIS_H */
