/*
 * Graph IR of the host library: error state, bump arena, graph and node
 * builders for the ops on the device path.
 *
 * Shapes and input wiring follow bleeding/v11A1/src/ir/lancius_ir.c (cited per
 * builder); node storage lives in the graph's arena so node addresses are
 * stable for the life of the graph.
 */
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "lancius_graph.h"
#include "graph_internal.h"

/* ---- error state: thread-local code (lancius_error.c:5-34) ---------------- */

static _Thread_local lancius_error t_error = LANCIUS_ERROR_OK;

void lancius_set_error(lancius_error err) { t_error = err; }
lancius_error lancius_get_error(void) { return t_error; }
void lancius_clear_error(void) { t_error = LANCIUS_ERROR_OK; }

const char* lancius_error_string(lancius_error err) {
    switch (err) {
        case LANCIUS_ERROR_OK: return "success";
        case LANCIUS_ERROR_OOM: return "out of memory";
        case LANCIUS_ERROR_NULL_PTR: return "null pointer";
        case LANCIUS_ERROR_SHAPE_MISMATCH: return "shape mismatch";
        case LANCIUS_ERROR_UNSUPPORTED_OP: return "unsupported op";
        case LANCIUS_ERROR_UNSUPPORTED_DTYPE: return "unsupported dtype";
        case LANCIUS_ERROR_INVALID_MODEL: return "invalid model";
        case LANCIUS_ERROR_VERSION_MISMATCH: return "version mismatch";
        case LANCIUS_ERROR_IO: return "io error";
        case LANCIUS_ERROR_OVERFLOW: return "overflow";
        case LANCIUS_ERROR_INTERNAL: return "internal error";
        default: return "unknown error";
    }
}

/* ---- bump arena ------------------------------------------------------------
 * Chained blocks, allocations rounded to 32 bytes and aligned to a power of
 * two (32 by default), O(1) reset that keeps the first block
 * (lancius_arena.c:39-89). */

typedef struct arena_block {
    struct arena_block* next;
    size_t size, used;
    unsigned char* mem;
} arena_block;

struct lancius_arena {
    arena_block* head;
    arena_block* tail;
    size_t block_size;
};

static arena_block* arena_block_new(size_t size) {
    arena_block* b = (arena_block*)malloc(sizeof(arena_block));
    if (!b) return NULL;
    b->mem = (unsigned char*)malloc(size);
    if (!b->mem) {
        free(b);
        return NULL;
    }
    b->next = NULL;
    b->size = size;
    b->used = 0;
    return b;
}

lancius_arena* lancius_arena_create(size_t block_size) {
    lancius_arena* a = (lancius_arena*)calloc(1, sizeof(lancius_arena));
    if (!a) return NULL;
    a->block_size = block_size ? block_size : ((size_t)16 << 20);
    a->head = a->tail = arena_block_new(a->block_size);
    if (!a->head) {
        free(a);
        return NULL;
    }
    return a;
}

void* lancius_arena_alloc(lancius_arena* a, size_t size, size_t alignment) {
    if (!a) return NULL;
    if (alignment == 0) alignment = 32;
    if (alignment & (alignment - 1)) return NULL;
    if (size == 0) size = 1;
    if (size > SIZE_MAX - 64 - alignment) return NULL; /* rounding below must not wrap */
    size = (size + 31) & ~(size_t)31;
    arena_block* b = a->tail;
    uintptr_t at = (uintptr_t)(b->mem + b->used);
    size_t pad = (size_t)(((at + alignment - 1) & ~(uintptr_t)(alignment - 1)) - at);
    if (pad + size > b->size - b->used) {
        size_t want = size + alignment;
        arena_block* nb = arena_block_new(want > a->block_size ? want : a->block_size);
        if (!nb) return NULL;
        b->next = nb;
        a->tail = b = nb;
        at = (uintptr_t)b->mem;
        pad = (size_t)(((at + alignment - 1) & ~(uintptr_t)(alignment - 1)) - at);
    }
    b->used += pad + size;
    return (void*)(at + pad);
}

void lancius_arena_reset(lancius_arena* a) {
    if (!a) return;
    arena_block* b = a->head->next;
    while (b) {
        arena_block* n = b->next;
        free(b->mem);
        free(b);
        b = n;
    }
    a->head->next = NULL;
    a->head->used = 0;
    a->tail = a->head;
}

void lancius_arena_destroy(lancius_arena* a) {
    if (!a) return;
    arena_block* b = a->head;
    while (b) {
        arena_block* n = b->next;
        free(b->mem);
        free(b);
        b = n;
    }
    free(a);
}

/* ---- graph ------------------------------------------------------------------ */

lancius_graph* lancius_graph_create(void) {
    lancius_graph* g = (lancius_graph*)calloc(1, sizeof(lancius_graph));
    if (!g) {
        lancius_set_error(LANCIUS_ERROR_OOM);
        return NULL;
    }
    g->arena = lancius_arena_create(1 << 20);
    g->node_cap = 256;
    g->nodes = (lancius_node**)malloc(sizeof(lancius_node*) * g->node_cap);
    if (!g->arena || !g->nodes) {
        lancius_arena_destroy(g->arena);
        free(g->nodes);
        free(g);
        lancius_set_error(LANCIUS_ERROR_OOM);
        return NULL;
    }
    return g;
}

void lancius_graph_destroy(lancius_graph* g) {
    if (!g) return;
    /* int8 copies made by lancius_quantize_graph or lancius_graph_load, and
     * fp64 weights read by lancius_graph_load, belong to the graph */
    for (uint32_t i = 0; i < g->node_count; i++) {
        lancius_node* n = g->nodes[i];
        if (n->rt && n->rt->int8_owner == LANCIUS_MEMORY_OWNED_HEAP && n->runtime_data_int8) {
            free(n->runtime_data_int8);
            n->runtime_data_int8 = NULL;
            n->rt->buffer_int8 = NULL;
        }
        if (n->rt && (n->rt->flags & LANCIUS_RT_FLAG_LOADED) && n->runtime_data) {
            free(n->runtime_data);
            n->runtime_data = NULL;
            n->rt->buffer = NULL;
        }
    }
    free(g->nodes);
    free(g->rt_states);
    lancius_arena_destroy(g->arena);
    free(g);
}

void lancius_graph_set_dtype(lancius_graph* g, lancius_dtype dtype) {
    if (!g) return;
    for (uint32_t i = 0; i < g->node_count; i++) {
        lancius_node* n = g->nodes[i];
        /* quantized or int8-loaded weights stay int8 */
        if (n->dtype == LANCIUS_DTYPE_INT8 && (n->runtime_data_int8 || n->op == LANCIUS_OP_INPUT)) continue;
        n->dtype = dtype;
        if (n->rt) n->rt->dtype = dtype;
    }
}

/* lancius_quantize.c:6-33: every 4-D INPUT with bound fp64 data (a conv
 * filter) gets a per-tensor int8 copy, scale = max|w| / 127 (1e-8 when all
 * zero), q = (int8) round(w / scale), and dtype INT8, which routes its convs
 * to the int8 kernels.  The int8 buffer is owned by the graph. */
void lancius_quantize_graph(lancius_graph* g) {
    if (!g) return;
    int count = 0;
    for (uint32_t i = 0; i < g->node_count; i++) {
        lancius_node* n = g->nodes[i];
        if (n->op != LANCIUS_OP_INPUT || !n->runtime_data || n->ndim != 4) continue;
        size_t e = 1;
        for (uint8_t d = 0; d < n->ndim; d++) e *= n->shape[d];
        double m = 0.0;
        for (size_t j = 0; j < e; j++) {
            const double a = fabs(n->runtime_data[j]);
            if (a > m) m = a;
        }
        const double scale = m > 0.0 ? m / 127.0 : 1e-8;
        int8_t* q = (int8_t*)malloc(e ? e : 1);
        if (!q) {
            lancius_set_error(LANCIUS_ERROR_OOM);
            return;
        }
        for (size_t j = 0; j < e; j++) q[j] = (int8_t)round(n->runtime_data[j] / scale);
        if (n->rt && n->rt->int8_owner == LANCIUS_MEMORY_OWNED_HEAP) free(n->runtime_data_int8);
        n->runtime_data_int8 = q;
        n->scale = scale;
        n->dtype = LANCIUS_DTYPE_INT8;
        if (n->rt) {
            n->rt->buffer_int8 = q;
            n->rt->int8_owner = LANCIUS_MEMORY_OWNED_HEAP;
            n->rt->scale = scale;
            n->rt->dtype = LANCIUS_DTYPE_INT8;
        }
        count++;
    }
    printf("[LANCIUS QUANTIZER] %d weight tensors to int8\n", count);
}

/* A node with its input array and runtime-state record, all in the arena. */
static lancius_node* new_node(lancius_graph* g, lancius_opcode op, uint8_t ndim, uint32_t n_in) {
    if (!g) return NULL;
    if (g->node_count == g->node_cap) {
        uint32_t cap = g->node_cap * 2;
        lancius_node** grown = (lancius_node**)realloc(g->nodes, sizeof(lancius_node*) * cap);
        if (!grown) {
            lancius_set_error(LANCIUS_ERROR_OOM);
            return NULL;
        }
        g->nodes = grown;
        g->node_cap = cap;
    }
    lancius_node* n = (lancius_node*)lancius_arena_alloc(g->arena, sizeof(lancius_node), 8);
    lancius_runtime_state* rt = (lancius_runtime_state*)lancius_arena_alloc(g->arena, sizeof(*rt), 8);
    const lancius_node** ins = NULL;
    if (n_in) ins = (const lancius_node**)lancius_arena_alloc(g->arena, sizeof(lancius_node*) * n_in, 8);
    if (!n || !rt || (n_in && !ins)) {
        lancius_set_error(LANCIUS_ERROR_OOM);
        return NULL;
    }
    memset(n, 0, sizeof(*n));
    memset(rt, 0, sizeof(*rt));
    rt->dtype = LANCIUS_DTYPE_FP64;
    rt->scale = 1.0;
    n->id = g->next_id++;
    n->op = op;
    n->ndim = ndim;
    n->input_count = n_in;
    n->inputs = ins;
    n->rt = rt;
    n->dtype = LANCIUS_DTYPE_FP64;
    g->nodes[g->node_count++] = n;
    return n;
}

lancius_node* lancius__raw_node(lancius_graph* g, lancius_opcode op, uint8_t ndim, uint32_t n_in) {
    return new_node(g, op, ndim, n_in);
}

static void copy_shape(lancius_node* n, const lancius_node* from) {
    for (uint8_t d = 0; d < from->ndim && d < 4; d++) n->shape[d] = from->shape[d];
}

/* lancius_ir.c:145-148 */
lancius_node* lancius_input(lancius_graph* g, size_t r, size_t c) {
    lancius_node* n = new_node(g, LANCIUS_OP_INPUT, 2, 0);
    if (n) {
        n->shape[0] = r;
        n->shape[1] = c;
    }
    return n;
}

/* lancius_ir.c:149-152 */
lancius_node* lancius_input_4d(lancius_graph* g, size_t nn, size_t c, size_t h, size_t w) {
    lancius_node* n = new_node(g, LANCIUS_OP_INPUT, 4, 0);
    if (n) {
        n->shape[0] = nn;
        n->shape[1] = c;
        n->shape[2] = h;
        n->shape[3] = w;
    }
    return n;
}

/* lancius_ir.c:153-156: value filled in by the executor from attr_val. */
lancius_node* lancius_const(lancius_graph* g, double val, size_t r, size_t c) {
    lancius_node* n = new_node(g, LANCIUS_OP_CONST, 2, 0);
    if (n) {
        n->shape[0] = r;
        n->shape[1] = c;
        n->attr_val = val;
    }
    return n;
}

/* lancius_ir.c:157-163: shape of `a`, no shape check (a bias must come through
 * a BROADCAST node). */
lancius_node* lancius_add(lancius_graph* g, const lancius_node* a, const lancius_node* b) {
    if (!a || !b) {
        lancius_set_error(LANCIUS_ERROR_NULL_PTR);
        return NULL;
    }
    lancius_node* n = new_node(g, LANCIUS_OP_ADD, a->ndim, 2);
    if (n) {
        copy_shape(n, a);
        n->inputs[0] = a;
        n->inputs[1] = b;
    }
    return n;
}

/* lancius_ir.c:178-196: uses the last two dims of each operand; 2-D result. */
lancius_node* lancius_matmul(lancius_graph* g, const lancius_node* a, const lancius_node* b) {
    if (!a || !b || a->ndim < 2 || b->ndim < 2) {
        lancius_set_error(LANCIUS_ERROR_SHAPE_MISMATCH);
        return NULL;
    }
    const size_t ar = a->shape[a->ndim - 2], ac = a->shape[a->ndim - 1];
    const size_t br = b->shape[b->ndim - 2], bc = b->shape[b->ndim - 1];
    if (ac != br) {
        fprintf(stderr, "[LANCIUS IR] MATMUL mismatch: [%zux%zu] x [%zux%zu]\n", ar, ac, br, bc);
        lancius_set_error(LANCIUS_ERROR_SHAPE_MISMATCH);
        return NULL;
    }
    lancius_node* n = new_node(g, LANCIUS_OP_MATMUL, 2, 2);
    if (n) {
        n->shape[0] = ar;
        n->shape[1] = bc;
        n->inputs[0] = a;
        n->inputs[1] = b;
    }
    return n;
}

static lancius_node* unary(lancius_graph* g, lancius_opcode op, const lancius_node* a) {
    if (!a) {
        lancius_set_error(LANCIUS_ERROR_NULL_PTR);
        return NULL;
    }
    lancius_node* n = new_node(g, op, a->ndim, 1);
    if (n) {
        copy_shape(n, a);
        n->inputs[0] = a;
    }
    return n;
}

/* lancius_ir.c:197-201 */
lancius_node* lancius_relu(lancius_graph* g, const lancius_node* a) { return unary(g, LANCIUS_OP_RELU, a); }

/* lancius_ir.c:202-206: 2-D only. */
lancius_node* lancius_softmax(lancius_graph* g, const lancius_node* a) {
    if (!a || a->ndim != 2) {
        lancius_set_error(LANCIUS_ERROR_SHAPE_MISMATCH);
        return NULL;
    }
    return unary(g, LANCIUS_OP_SOFTMAX, a);
}

/* lancius_ir.c:212-216 */
lancius_node* lancius_broadcast(lancius_graph* g, const lancius_node* a, size_t r, size_t c) {
    if (!a) {
        lancius_set_error(LANCIUS_ERROR_NULL_PTR);
        return NULL;
    }
    lancius_node* n = new_node(g, LANCIUS_OP_BROADCAST, 2, 1);
    if (n) {
        n->shape[0] = r;
        n->shape[1] = c;
        n->inputs[0] = a;
    }
    return n;
}

/* lancius_ir.c:243-261: NCHW input, OIHW weights, output [N, C_out, H_out, W_out]. */
lancius_node* lancius_conv2d(lancius_graph* g, const lancius_node* in, const lancius_node* w, uint32_t stride,
                             uint32_t pad) {
    if (!in || !w || in->ndim != 4 || w->ndim != 4 || stride == 0) {
        lancius_set_error(LANCIUS_ERROR_SHAPE_MISMATCH);
        return NULL;
    }
    const size_t N = in->shape[0], C_in = in->shape[1], H = in->shape[2], W = in->shape[3];
    const size_t C_out = w->shape[0], K_h = w->shape[2], K_w = w->shape[3];
    if (C_in != w->shape[1] || H + 2 * (size_t)pad < K_h || W + 2 * (size_t)pad < K_w) {
        fprintf(stderr, "[LANCIUS IR] CONV2D shape mismatch\n");
        lancius_set_error(LANCIUS_ERROR_SHAPE_MISMATCH);
        return NULL;
    }
    lancius_node* n = new_node(g, LANCIUS_OP_CONV2D, 4, 2);
    if (n) {
        n->shape[0] = N;
        n->shape[1] = C_out;
        n->shape[2] = (H + 2 * (size_t)pad - K_h) / stride + 1;
        n->shape[3] = (W + 2 * (size_t)pad - K_w) / stride + 1;
        n->kernel_h = (uint32_t)K_h;
        n->kernel_w = (uint32_t)K_w;
        n->stride = stride;
        n->pad = pad;
        n->inputs[0] = in;
        n->inputs[1] = w;
    }
    return n;
}

/* lancius_ir.c:281-288 */
lancius_node* lancius_flatten(lancius_graph* g, const lancius_node* in) {
    if (!in || in->ndim != 4) {
        lancius_set_error(LANCIUS_ERROR_SHAPE_MISMATCH);
        return NULL;
    }
    lancius_node* n = new_node(g, LANCIUS_OP_FLATTEN, 2, 1);
    if (n) {
        n->shape[0] = in->shape[0];
        n->shape[1] = in->shape[1] * in->shape[2] * in->shape[3];
        n->inputs[0] = in;
    }
    return n;
}

/* lancius_ir.c:291-299: the executor copies the first elems(out) values. */
lancius_node* lancius_reshape(lancius_graph* g, const lancius_node* in, uint8_t ndim, size_t s0, size_t s1, size_t s2,
                              size_t s3) {
    if (!in || ndim == 0 || ndim > 4) {
        lancius_set_error(LANCIUS_ERROR_SHAPE_MISMATCH);
        return NULL;
    }
    lancius_node* n = new_node(g, LANCIUS_OP_RESHAPE, ndim, 1);
    if (n) {
        const size_t s[4] = {s0, s1, s2, s3};
        for (uint8_t d = 0; d < ndim; d++) n->shape[d] = s[d];
        n->inputs[0] = in;
    }
    return n;
}

/* lancius_ir.c:72-77: output takes q's 3-D shape [S, H, D]. */
lancius_node* lancius_attention(lancius_graph* g, const lancius_node* q, const lancius_node* k,
                                const lancius_node* v) {
    if (!q || !k || !v) {
        lancius_set_error(LANCIUS_ERROR_NULL_PTR);
        return NULL;
    }
    lancius_node* n = new_node(g, LANCIUS_OP_ATTENTION, 3, 3);
    if (n) {
        n->shape[0] = q->shape[0];
        n->shape[1] = q->shape[1];
        n->shape[2] = q->shape[2];
        n->inputs[0] = q;
        n->inputs[1] = k;
        n->inputs[2] = v;
    }
    return n;
}

/* lancius_ir.c:78-83 */
lancius_node* lancius_layernorm(lancius_graph* g, const lancius_node* in, const lancius_node* gamma,
                                const lancius_node* beta) {
    if (!in || !gamma || !beta) {
        lancius_set_error(LANCIUS_ERROR_NULL_PTR);
        return NULL;
    }
    lancius_node* n = new_node(g, LANCIUS_OP_LAYERNORM, in->ndim, 3);
    if (n) {
        copy_shape(n, in);
        n->inputs[0] = in;
        n->inputs[1] = gamma;
        n->inputs[2] = beta;
    }
    return n;
}

/* lancius_ir.c:84-89 */
lancius_node* lancius_gelu(lancius_graph* g, const lancius_node* in) { return unary(g, LANCIUS_OP_GELU, in); }

/* ---- builders of the training graph ----------------------------------------- */

/* Two inputs, the shape of `a` (lancius_ir.c:164-177: SUB and MUL, like ADD,
 * do no shape check). */
static lancius_node* binary(lancius_graph* g, lancius_opcode op, const lancius_node* a, const lancius_node* b) {
    if (!a || !b) {
        lancius_set_error(LANCIUS_ERROR_NULL_PTR);
        return NULL;
    }
    lancius_node* n = new_node(g, op, a->ndim, 2);
    if (n) {
        copy_shape(n, a);
        n->inputs[0] = a;
        n->inputs[1] = b;
    }
    return n;
}

/* lancius_ir.c:164-170 */
lancius_node* lancius_sub(lancius_graph* g, const lancius_node* a, const lancius_node* b) {
    return binary(g, LANCIUS_OP_SUB, a, b);
}

/* lancius_ir.c:171-177 */
lancius_node* lancius_mul(lancius_graph* g, const lancius_node* a, const lancius_node* b) {
    return binary(g, LANCIUS_OP_MUL, a, b);
}

/* lancius_ir.c:222-226: shape of the gradient. */
lancius_node* lancius_relu_bwd(lancius_graph* g, const lancius_node* grad, const lancius_node* fwd_a) {
    return binary(g, LANCIUS_OP_RELU_BWD, grad, fwd_a);
}

/* lancius_ir.c:227-231 */
lancius_node* lancius_softmax_bwd(lancius_graph* g, const lancius_node* grad, const lancius_node* fwd_y) {
    return binary(g, LANCIUS_OP_SOFTMAX_BWD, grad, fwd_y);
}

/* A 2-D node of `rows` x `cols` with one input. */
static lancius_node* shaped1(lancius_graph* g, lancius_opcode op, const lancius_node* a, size_t rows, size_t cols) {
    lancius_node* n = new_node(g, op, 2, 1);
    if (n) {
        n->shape[0] = rows;
        n->shape[1] = cols;
        n->inputs[0] = a;
    }
    return n;
}

/* lancius_ir.c:207-211: [1,1] over every element of the input. */
lancius_node* lancius_sum(lancius_graph* g, const lancius_node* a) {
    if (!a) {
        lancius_set_error(LANCIUS_ERROR_NULL_PTR);
        return NULL;
    }
    return shaped1(g, LANCIUS_OP_SUM, a, 1, 1);
}

/* lancius_ir.c:217-221: 2-D only. */
lancius_node* lancius_transpose(lancius_graph* g, const lancius_node* a) {
    if (!a || a->ndim != 2) {
        lancius_set_error(LANCIUS_ERROR_SHAPE_MISMATCH);
        return NULL;
    }
    return shaped1(g, LANCIUS_OP_TRANSPOSE, a, a->shape[1], a->shape[0]);
}

/* lancius_ir.c:232-236 */
lancius_node* lancius_sum_axis0(lancius_graph* g, const lancius_node* a) {
    if (!a || a->ndim != 2) {
        lancius_set_error(LANCIUS_ERROR_SHAPE_MISMATCH);
        return NULL;
    }
    return shaped1(g, LANCIUS_OP_SUM_AXIS0, a, 1, a->shape[1]);
}

/* lancius_ir.c:237-241 */
lancius_node* lancius_sum_axis1(lancius_graph* g, const lancius_node* a) {
    if (!a || a->ndim != 2) {
        lancius_set_error(LANCIUS_ERROR_SHAPE_MISMATCH);
        return NULL;
    }
    return shaped1(g, LANCIUS_OP_SUM_AXIS1, a, a->shape[0], 1);
}

/* lancius_ir.c:92-97: a 4-D BROADCAST (the executor fills it from a scalar). */
lancius_node* lancius_broadcast_4d(lancius_graph* g, const lancius_node* a, size_t nn, size_t c, size_t h, size_t w) {
    if (!a) {
        lancius_set_error(LANCIUS_ERROR_NULL_PTR);
        return NULL;
    }
    lancius_node* n = new_node(g, LANCIUS_OP_BROADCAST, 4, 1);
    if (n) {
        n->shape[0] = nn;
        n->shape[1] = c;
        n->shape[2] = h;
        n->shape[3] = w;
        n->inputs[0] = a;
    }
    return n;
}

/* lancius_ir.c:263-280: no padding, square window. */
lancius_node* lancius_maxpool2d(lancius_graph* g, const lancius_node* in, uint32_t kernel, uint32_t stride) {
    if (!in || in->ndim != 4 || kernel == 0 || stride == 0 || in->shape[2] < kernel || in->shape[3] < kernel) {
        lancius_set_error(LANCIUS_ERROR_SHAPE_MISMATCH);
        return NULL;
    }
    lancius_node* n = new_node(g, LANCIUS_OP_MAXPOOL2D, 4, 1);
    if (n) {
        n->shape[0] = in->shape[0];
        n->shape[1] = in->shape[1];
        n->shape[2] = (in->shape[2] - kernel) / stride + 1;
        n->shape[3] = (in->shape[3] - kernel) / stride + 1;
        n->kernel_h = kernel;
        n->kernel_w = kernel;
        n->stride = stride;
        n->inputs[0] = in;
    }
    return n;
}

/* lancius_ir.c:337-343: scalar loss of logits against same-shape targets. */
lancius_node* lancius_cross_entropy(lancius_graph* g, const lancius_node* logits, const lancius_node* targets) {
    if (!logits || !targets || logits->ndim != 2 || targets->ndim != 2 || logits->shape[0] != targets->shape[0] ||
        logits->shape[1] != targets->shape[1]) {
        lancius_set_error(LANCIUS_ERROR_SHAPE_MISMATCH);
        return NULL;
    }
    lancius_node* n = new_node(g, LANCIUS_OP_CROSS_ENTROPY, 2, 2);
    if (n) {
        n->shape[0] = 1;
        n->shape[1] = 1;
        n->inputs[0] = logits;
        n->inputs[1] = targets;
    }
    return n;
}

/* lancius_ir.c:344-350: shape of the logits; inputs logits, targets, scalar
 * upstream gradient. */
lancius_node* lancius_cross_entropy_bwd(lancius_graph* g, const lancius_node* logits, const lancius_node* targets,
                                        const lancius_node* grad_out) {
    if (!logits || !targets || !grad_out) {
        lancius_set_error(LANCIUS_ERROR_NULL_PTR);
        return NULL;
    }
    lancius_node* n = new_node(g, LANCIUS_OP_CROSS_ENTROPY_BWD, logits->ndim, 3);
    if (n) {
        copy_shape(n, logits);
        n->inputs[0] = logits;
        n->inputs[1] = targets;
        n->inputs[2] = grad_out;
    }
    return n;
}

/* lancius_ir.c:351-359: shape of the forward input; inputs grad, fwd_in, fwd_w. */
lancius_node* lancius_conv2d_bwd(lancius_graph* g, const lancius_node* grad, const lancius_node* fwd_in,
                                 const lancius_node* fwd_w, uint32_t stride, uint32_t pad) {
    if (!grad || !fwd_in || !fwd_w) {
        lancius_set_error(LANCIUS_ERROR_NULL_PTR);
        return NULL;
    }
    lancius_node* n = new_node(g, LANCIUS_OP_CONV2D_BWD, 4, 3);
    if (n) {
        for (int d = 0; d < 4; d++) n->shape[d] = fwd_in->shape[d];
        n->stride = stride;
        n->pad = pad;
        n->inputs[0] = grad;
        n->inputs[1] = fwd_in;
        n->inputs[2] = fwd_w;
    }
    return n;
}

/* lancius_ir.c:300-313: [C_out (grad channels), C_in (fwd_in channels), k_h, k_w]. */
lancius_node* lancius_conv2d_bwd_w(lancius_graph* g, const lancius_node* grad, const lancius_node* fwd_in,
                                   uint32_t k_h, uint32_t k_w, uint32_t stride, uint32_t pad) {
    if (!grad || !fwd_in) {
        lancius_set_error(LANCIUS_ERROR_NULL_PTR);
        return NULL;
    }
    lancius_node* n = new_node(g, LANCIUS_OP_CONV2D_BWD_W, 4, 2);
    if (n) {
        n->shape[0] = grad->shape[1];
        n->shape[1] = fwd_in->shape[1];
        n->shape[2] = k_h;
        n->shape[3] = k_w;
        n->kernel_h = k_h;
        n->kernel_w = k_w;
        n->stride = stride;
        n->pad = pad;
        n->inputs[0] = grad;
        n->inputs[1] = fwd_in;
    }
    return n;
}

/* lancius_ir.c:360-368: shape of the forward input; inputs grad, fwd_in. */
lancius_node* lancius_maxpool2d_bwd(lancius_graph* g, const lancius_node* grad, const lancius_node* fwd_in,
                                    uint32_t kernel, uint32_t stride) {
    if (!grad || !fwd_in) {
        lancius_set_error(LANCIUS_ERROR_NULL_PTR);
        return NULL;
    }
    lancius_node* n = new_node(g, LANCIUS_OP_MAXPOOL2D_BWD, 4, 2);
    if (n) {
        for (int d = 0; d < 4; d++) n->shape[d] = fwd_in->shape[d];
        n->kernel_h = kernel;
        n->kernel_w = kernel;
        n->stride = stride;
        n->inputs[0] = grad;
        n->inputs[1] = fwd_in;
    }
    return n;
}

/* lancius_ir.c:315-325: 4-D axis permutation (no executor runs it). */
lancius_node* lancius_permute(lancius_graph* g, const lancius_node* in, uint32_t a0, uint32_t a1, uint32_t a2,
                              uint32_t a3) {
    if (!in || in->ndim != 4 || a0 > 3 || a1 > 3 || a2 > 3 || a3 > 3) {
        lancius_set_error(LANCIUS_ERROR_SHAPE_MISMATCH);
        return NULL;
    }
    lancius_node* n = new_node(g, LANCIUS_OP_PERMUTE, 4, 1);
    if (n) {
        const uint32_t ax[4] = {a0, a1, a2, a3};
        for (int d = 0; d < 4; d++) {
            n->axes[d] = ax[d];
            n->shape[d] = in->shape[ax[d]];
        }
        n->inputs[0] = in;
    }
    return n;
}

/* lancius_ir.c:326-336: [B,M,K] x [B,K,N] -> [B,M,N] (no executor runs it). */
lancius_node* lancius_matmul_batched(lancius_graph* g, const lancius_node* a, const lancius_node* b) {
    if (!a || !b || a->ndim != 3 || b->ndim != 3 || a->shape[0] != b->shape[0] || a->shape[2] != b->shape[1]) {
        lancius_set_error(LANCIUS_ERROR_SHAPE_MISMATCH);
        return NULL;
    }
    lancius_node* n = new_node(g, LANCIUS_OP_MATMUL_BATCHED, 3, 2);
    if (n) {
        n->shape[0] = a->shape[0];
        n->shape[1] = a->shape[1];
        n->shape[2] = b->shape[2];
        n->inputs[0] = a;
        n->inputs[1] = b;
    }
    return n;
}

/* lancius_ir.c:370-378 */
lancius_node* lancius_rmsnorm(lancius_graph* g, const lancius_node* in, const lancius_node* gamma) {
    return binary(g, LANCIUS_OP_RMSNORM, in, gamma);
}

/* lancius_ir.c:380-388 */
lancius_node* lancius_swiglu(lancius_graph* g, const lancius_node* gate, const lancius_node* up) {
    return binary(g, LANCIUS_OP_SWIGLU, gate, up);
}

/* lancius_ir.c:390-401: shape of q, head counts in kernel_h / kernel_w. */
lancius_node* lancius_gqa(lancius_graph* g, const lancius_node* q, const lancius_node* k, const lancius_node* v,
                          uint32_t n_heads_q, uint32_t n_heads_kv) {
    if (!q || !k || !v) {
        lancius_set_error(LANCIUS_ERROR_NULL_PTR);
        return NULL;
    }
    lancius_node* n = new_node(g, LANCIUS_OP_GQA, q->ndim, 3);
    if (n) {
        copy_shape(n, q);
        n->kernel_h = n_heads_q;
        n->kernel_w = n_heads_kv;
        n->inputs[0] = q;
        n->inputs[1] = k;
        n->inputs[2] = v;
    }
    return n;
}
