/*
 * Device executor for BASIS static graphs (include/basis/stage6_ir/graph.h:
 * INPUT, MATMUL, ADD, RELU, TANH, BROADCAST_ADD; the reference has builders
 * and no executor, src/basis/stage6_ir/graph.c).
 *
 * Compiled once into a list of launches in node-id order (inputs always
 * precede their consumers):
 *  - MATMUL -> BROADCAST_ADD(bias) -> RELU|TANH -> ADD(earlier tensor), each
 *    step taken only while the running result has exactly one consumer,
 *    becomes one lancius_hip_gemm_f32 with that epilogue (bias, activation,
 *    residual: the GEMM's own order);
 *  - two such chains back to back with a small batch (one hidden layer of
 *    an MLP) become one lancius_hip_mlp2_ex_f32 (try_mlp2);
 *  - BROADCAST_ADD -> RELU|TANH becomes one lancius_hip_bias_act_f32;
 *  - ADD, RELU, TANH run elementwise.
 * Nodes that are not absorbed get a 256-byte aligned buffer in one HBM
 * basis_arena created for the program (its first block holds the whole
 * graph).
 */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "lancius_basis.h"
#include "lancius_hip.h"

enum { K_GEMM, K_BIAS_ACT, K_ADD, K_RELU, K_TANH, K_MLP2 };

typedef struct {
    int kind;
    int out;                 /* node whose buffer receives the result */
    int a, b;                /* operand nodes (-1: none) */
    int bias, residual, act; /* GEMM / bias_act epilogue */
    int w2, bias2, act2;     /* second layer of K_MLP2 */
    size_t m, k, n, n2;
} basis_launch;

struct lancius_basis_program {
    lancius_hip_ctx* ctx;
    const basis_graph* g;
    basis_arena* arena;
    size_t arena_bytes;
    float** buf;  /* per node: device buffer or NULL when absorbed */
    basis_launch* launches;
    size_t launch_count;
};

static int fail(int code, const char* what) {
    fprintf(stderr, "[LANCIUS BASIS] invalid graph: %s\n", what);
    return code;
}

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

/* Checks every node's op, inputs (earlier ids) and shapes. */
static int validate(const basis_graph* g) {
    for (size_t i = 0; i < g->node_count; i++) {
        const basis_node* n = &g->nodes[i];
        if (n->id != (int)i) return fail(LANCIUS_HIP_ERR_SHAPE, "node id");
        if (n->rows == 0 || n->cols == 0 || n->rows > ((size_t)1 << 30) || n->cols > ((size_t)1 << 30) ||
            n->rows * n->cols > ((size_t)1 << 36))
            return fail(LANCIUS_HIP_ERR_SHAPE, "node shape");
        const int arity = n->op == BASIS_OP_INPUT ? 0 : (n->op == BASIS_OP_RELU || n->op == BASIS_OP_TANH) ? 1 : 2;
        if (n->op < BASIS_OP_INPUT || n->op > BASIS_OP_BROADCAST_ADD) return fail(LANCIUS_HIP_ERR_UNSUPPORTED, "op");
        for (int j = 0; j < arity; j++)
            if (n->input_ids[j] < 0 || n->input_ids[j] >= (int)i) return fail(LANCIUS_HIP_ERR_SHAPE, "input id");
        const basis_node* a = arity > 0 ? &g->nodes[n->input_ids[0]] : NULL;
        const basis_node* b = arity > 1 ? &g->nodes[n->input_ids[1]] : NULL;
        switch (n->op) {
            case BASIS_OP_MATMUL:
                if (a->cols != b->rows || n->rows != a->rows || n->cols != b->cols)
                    return fail(LANCIUS_HIP_ERR_SHAPE, "matmul");
                break;
            case BASIS_OP_ADD:
                if (a->rows != b->rows || a->cols != b->cols || n->rows != a->rows || n->cols != a->cols)
                    return fail(LANCIUS_HIP_ERR_SHAPE, "add");
                break;
            case BASIS_OP_BROADCAST_ADD:
                if (b->rows != 1 || b->cols != a->cols || n->rows != a->rows || n->cols != a->cols)
                    return fail(LANCIUS_HIP_ERR_SHAPE, "broadcast_add");
                break;
            case BASIS_OP_RELU:
            case BASIS_OP_TANH:
                if (n->rows != a->rows || n->cols != a->cols) return fail(LANCIUS_HIP_ERR_SHAPE, "unary");
                break;
            default:
                break;
        }
    }
    return 0;
}

/* The one consumer of node `id`, or -1 when it has none or several. */
static int sole_consumer(const basis_graph* g, const int* uses, int id) {
    if (uses[id] != 1) return -1;
    for (size_t i = (size_t)id + 1; i < g->node_count; i++) {
        const basis_node* n = &g->nodes[i];
        if (n->op != BASIS_OP_INPUT && (n->input_ids[0] == id || n->input_ids[1] == id)) return (int)i;
    }
    return -1;
}

static int ready_before(const basis_graph* g, int node, int head) {
    return g->nodes[node].op == BASIS_OP_INPUT || node < head;
}

static int act_of(basis_op_type op) {
    return op == BASIS_OP_RELU ? LANCIUS_HIP_ACT_RELU : op == BASIS_OP_TANH ? LANCIUS_HIP_ACT_TANH : -1;
}

/* MATMUL(x, W1) [-> BROADCAST_ADD(b1)] [-> RELU|TANH] -> MATMUL(., W2)
 * [-> BROADCAST_ADD(b2)] [-> RELU|TANH] with single consumers, within
 * lancius_hip_mlp2_ex_f32's limits (M <= 64, N2 <= 64, M*N1 <= 16384,
 * N1*N2 <= 8192, K1*max(M, N1) <= 2^28): one launch instead of two
 * split-K GEMMs with their reduces.  Fills L and marks the chain's inner
 * nodes absorbed; returns 0 when the pattern does not match. */
static int try_mlp2(const basis_graph* g, const int* uses, int head, basis_launch* L, char* absorbed) {
    const basis_node* nd = g->nodes;
    int chain[6], len = 0;
    int t = head, c = sole_consumer(g, uses, t);
    int b1 = -1, act1 = LANCIUS_HIP_ACT_NONE, b2 = -1, act2 = LANCIUS_HIP_ACT_NONE;
    chain[len++] = t;
    if (c >= 0 && nd[c].op == BASIS_OP_BROADCAST_ADD && nd[c].input_ids[0] == t && ready_before(g, nd[c].input_ids[1], head)) {
        b1 = nd[c].input_ids[1];
        chain[len++] = t = c;
        c = sole_consumer(g, uses, t);
    }
    if (c >= 0 && act_of(nd[c].op) >= 0) {
        act1 = act_of(nd[c].op);
        chain[len++] = t = c;
        c = sole_consumer(g, uses, t);
    }
    if (c < 0 || nd[c].op != BASIS_OP_MATMUL || nd[c].input_ids[0] != t || !ready_before(g, nd[c].input_ids[1], head))
        return 0;
    const int mm2 = c;
    chain[len++] = t = c;
    c = sole_consumer(g, uses, t);
    if (c >= 0 && nd[c].op == BASIS_OP_BROADCAST_ADD && nd[c].input_ids[0] == t && ready_before(g, nd[c].input_ids[1], head)) {
        b2 = nd[c].input_ids[1];
        chain[len++] = t = c;
        c = sole_consumer(g, uses, t);
    }
    if (c >= 0 && act_of(nd[c].op) >= 0) {
        act2 = act_of(nd[c].op);
        chain[len++] = t = c;
    }
    const size_t M = nd[head].rows, N1 = nd[head].cols, N2 = nd[mm2].cols, K1 = nd[nd[head].input_ids[0]].cols;
    if (M > 64 || N2 > 64 || M * N1 > 16384 || N1 * N2 > 8192 || K1 * (M > N1 ? M : N1) > ((size_t)1 << 28)) return 0;
    for (int j = 0; j + 1 < len; j++) absorbed[chain[j]] = 1;
    L->kind = K_MLP2;
    L->a = nd[head].input_ids[0];
    L->b = nd[head].input_ids[1];
    L->bias = b1;
    L->act = act1;
    L->w2 = nd[mm2].input_ids[1];
    L->bias2 = b2;
    L->act2 = act2;
    L->m = M;
    L->k = nd[L->a].cols;
    L->n = N1;
    L->n2 = N2;
    L->out = t;
    return 1;
}

int lancius_basis_program_create(lancius_hip_ctx* ctx, const basis_graph* g, unsigned flags,
                                 lancius_basis_program** out) {
    if (!ctx || !g || !out) return LANCIUS_HIP_ERR_NULL_PTR;
    *out = NULL;
    if (g->node_count == 0 || !g->nodes || g->node_count > (1u << 24)) return LANCIUS_HIP_ERR_SHAPE;
    int rc = validate(g);
    if (rc) return rc;
    const size_t nn = g->node_count;
    const int keep_all = (flags & LANCIUS_BASIS_KEEP_ALL) != 0;

    lancius_basis_program* p = (lancius_basis_program*)calloc(1, sizeof(*p));
    int* uses = (int*)calloc(nn, sizeof(int));
    char* absorbed = (char*)calloc(nn, 1); /* value consumed inside a fused launch: no buffer */
    char* done = (char*)calloc(nn, 1);     /* produced by an earlier launch */
    if (p) {
        p->buf = (float**)calloc(nn, sizeof(float*));
        p->launches = (basis_launch*)calloc(nn, sizeof(basis_launch));
    }
    if (!p || !uses || !absorbed || !done || !p->buf || !p->launches) {
        rc = LANCIUS_HIP_ERR_OOM;
        goto fail_out;
    }
    p->ctx = ctx;
    p->g = g;
    for (size_t i = 0; i < nn; i++) {
        const basis_node* n = &g->nodes[i];
        if (n->op == BASIS_OP_INPUT) continue;
        uses[n->input_ids[0]]++;
        if (n->op != BASIS_OP_RELU && n->op != BASIS_OP_TANH) uses[n->input_ids[1]]++;
    }

    for (size_t i = 0; i < nn; i++) {
        const basis_node* n = &g->nodes[i];
        if (n->op == BASIS_OP_INPUT || absorbed[i] || done[i]) continue;
        basis_launch L;
        memset(&L, 0, sizeof(L));
        L.a = n->input_ids[0];
        L.b = n->input_ids[1];
        L.bias = L.residual = -1;
        L.act = LANCIUS_HIP_ACT_NONE;
        int tail = (int)i; /* the node whose value the launch produces */
        if (n->op == BASIS_OP_MATMUL && !keep_all && try_mlp2(g, uses, (int)i, &L, absorbed)) {
            tail = L.out;
        } else if (n->op == BASIS_OP_MATMUL) {
            L.kind = K_GEMM;
            L.m = n->rows;
            L.k = g->nodes[L.a].cols;
            L.n = n->cols;
            /* bias and residual must exist when the GEMM runs: INPUTs, or
             * nodes before the MATMUL (their launches come first) */
            int c = keep_all ? -1 : sole_consumer(g, uses, tail);
            if (c >= 0 && g->nodes[c].op == BASIS_OP_BROADCAST_ADD && g->nodes[c].input_ids[0] == tail &&
                ready_before(g, g->nodes[c].input_ids[1], (int)i)) {
                L.bias = g->nodes[c].input_ids[1];
                absorbed[tail] = 1;
                tail = c;
                c = sole_consumer(g, uses, tail);
            }
            if (c >= 0 && act_of(g->nodes[c].op) >= 0) {
                L.act = act_of(g->nodes[c].op);
                absorbed[tail] = 1;
                tail = c;
                c = sole_consumer(g, uses, tail);
            }
            if (c >= 0 && g->nodes[c].op == BASIS_OP_ADD) {
                const int other = g->nodes[c].input_ids[0] == tail ? g->nodes[c].input_ids[1] : g->nodes[c].input_ids[0];
                if (other != tail && ready_before(g, other, (int)i)) {
                    L.residual = other;
                    absorbed[tail] = 1;
                    tail = c;
                }
            }
        } else if (n->op == BASIS_OP_BROADCAST_ADD) {
            L.kind = K_BIAS_ACT;
            L.bias = L.b;
            L.m = n->rows;
            L.n = n->cols;
            const int c = keep_all ? -1 : sole_consumer(g, uses, tail);
            if (c >= 0 && act_of(g->nodes[c].op) >= 0) {
                L.act = act_of(g->nodes[c].op);
                absorbed[tail] = 1;
                tail = c;
            }
        } else if (n->op == BASIS_OP_ADD) {
            L.kind = K_ADD;
        } else {
            L.kind = n->op == BASIS_OP_RELU ? K_RELU : K_TANH;
        }
        L.out = tail;
        done[tail] = 1;
        p->launches[p->launch_count++] = L;
    }

    /* one arena block sized for every node that keeps a buffer */
    size_t total = 0;
    for (size_t i = 0; i < nn; i++)
        if (!absorbed[i]) total += align256(g->nodes[i].rows * g->nodes[i].cols * sizeof(float));
    p->arena = basis_arena_create(total);
    if (!p->arena) {
        rc = LANCIUS_HIP_ERR_OOM;
        goto fail_out;
    }
    p->arena_bytes = lancius_basis_arena_capacity(p->arena);
    for (size_t i = 0; i < nn; i++) {
        if (absorbed[i]) continue;
        p->buf[i] = (float*)basis_arena_alloc(p->arena, g->nodes[i].rows * g->nodes[i].cols * sizeof(float), 256);
        if (!p->buf[i]) {
            rc = LANCIUS_HIP_ERR_OOM;
            goto fail_out;
        }
    }
    free(uses);
    free(absorbed);
    free(done);
    *out = p;
    return 0;

fail_out:
    free(uses);
    free(absorbed);
    free(done);
    lancius_basis_program_destroy(p);
    return rc;
}

int lancius_basis_program_run(lancius_basis_program* p) {
    if (!p) return LANCIUS_HIP_ERR_NULL_PTR;
    const basis_graph* g = p->g;
    for (size_t i = 0; i < p->launch_count; i++) {
        const basis_launch* L = &p->launches[i];
        float* out = p->buf[L->out];
        const basis_node* o = &g->nodes[L->out];
        int rc = 0;
        switch (L->kind) {
            case K_GEMM:
                rc = lancius_hip_gemm_f32(p->ctx, out, p->buf[L->a], p->buf[L->b], L->m, L->k, L->n,
                                          L->bias >= 0 ? p->buf[L->bias] : NULL, L->act,
                                          L->residual >= 0 ? p->buf[L->residual] : NULL);
                break;
            case K_BIAS_ACT:
                rc = lancius_hip_bias_act_f32(p->ctx, out, p->buf[L->a], p->buf[L->bias], L->m, L->n, L->act);
                break;
            case K_MLP2:
                rc = lancius_hip_mlp2_ex_f32(p->ctx, out, NULL, p->buf[L->a], p->buf[L->b],
                                             L->bias >= 0 ? p->buf[L->bias] : NULL, L->act, p->buf[L->w2],
                                             L->bias2 >= 0 ? p->buf[L->bias2] : NULL, L->act2, L->m, L->k, L->n,
                                             L->n2, 0);
                break;
            case K_ADD:
                rc = lancius_hip_add_f32(p->ctx, out, p->buf[L->a], p->buf[L->b], o->rows * o->cols);
                break;
            case K_RELU:
                rc = lancius_hip_relu_f32(p->ctx, out, p->buf[L->a], o->rows * o->cols);
                break;
            default:
                rc = lancius_hip_tanh_f32(p->ctx, out, p->buf[L->a], o->rows * o->cols);
                break;
        }
        if (rc) return rc;
    }
    return 0;
}

static int node_buffer(lancius_basis_program* p, int node_id, size_t count, float** buf) {
    if (!p) return LANCIUS_HIP_ERR_NULL_PTR;
    if (node_id < 0 || (size_t)node_id >= p->g->node_count) return LANCIUS_HIP_ERR_SHAPE;
    const basis_node* n = &p->g->nodes[node_id];
    if (count != n->rows * n->cols) return LANCIUS_HIP_ERR_SHAPE;
    if (!p->buf[node_id]) return LANCIUS_HIP_ERR_UNSUPPORTED; /* absorbed into a fused launch */
    *buf = p->buf[node_id];
    return 0;
}

int lancius_basis_program_upload(lancius_basis_program* p, int node_id, const float* host, size_t count) {
    float* buf = NULL;
    if (!host) return LANCIUS_HIP_ERR_NULL_PTR;
    int rc = node_buffer(p, node_id, count, &buf);
    if (rc) return rc;
    if (p->g->nodes[node_id].op != BASIS_OP_INPUT) return LANCIUS_HIP_ERR_UNSUPPORTED;
    return lancius_hip_upload(p->ctx, buf, host, count * sizeof(float));
}

int lancius_basis_program_download(lancius_basis_program* p, int node_id, float* host, size_t count) {
    float* buf = NULL;
    if (!host) return LANCIUS_HIP_ERR_NULL_PTR;
    int rc = node_buffer(p, node_id, count, &buf);
    if (rc) return rc;
    return lancius_hip_download(p->ctx, host, buf, count * sizeof(float));
}

float* lancius_basis_program_buffer(lancius_basis_program* p, int node_id) {
    if (!p || node_id < 0 || (size_t)node_id >= p->g->node_count) return NULL;
    return p->buf[node_id];
}

int lancius_basis_program_info(const lancius_basis_program* p, size_t* launches, size_t* arena_bytes) {
    if (!p) return LANCIUS_HIP_ERR_NULL_PTR;
    if (launches) *launches = p->launch_count;
    if (arena_bytes) *arena_bytes = p->arena_bytes;
    return 0;
}

void lancius_basis_program_destroy(lancius_basis_program* p) {
    if (!p) return;
    basis_arena_destroy(p->arena);
    free(p->buf);
    free(p->launches);
    free(p);
}
