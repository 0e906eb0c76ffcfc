/*
 * Device executor: compiles a scheduled Lancius graph into a launch list over
 * one HBM arena and replays it through the lancius_hip_* C ABI.
 * Replaces bleeding/v11A1/src/runtime/lancius_scheduler.c:61-520 (dispatch
 * and executors) for the ops of the device path; see lancius_hip_graph.h.
 */
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "lancius_hip_graph.h"

#define NONE UINT32_MAX
#define MAXG LANCIUS_HIP_MAX_GROUP
#define ALIGN_DEV 256u

typedef enum {
    L_GEMM, L_CONV, L_ATTN, L_LN, L_SOFTMAX, L_ADD, L_RELU, L_GELU, L_BCAST,
    L_SUB, L_MUL, L_RELU_BWD, L_TRANSPOSE, L_SUM, L_SUM0, L_SUM1, L_SOFTMAX_BWD, L_CE, L_CE_BWD,
    L_CONV_BWD_IN, L_CONV_BWD_W, L_POOL, L_POOL_BWD, L_RMSNORM, L_SWIGLU, L_GQA, L_ROPE, L_MLP2
} lkind;

enum { ROLE_NONE = 0, ROLE_INPUT, ROLE_CONST, ROLE_POOLED, ROLE_ALIAS, ROLE_FUSED };
enum { PACK_NONE = 0, PACK_I8, PACK_CONV };
enum { PACK_FRESH = 0, PACK_STALE = 1, PACK_EXPOSED = 2 };

typedef struct {
    uint32_t out;   /* node id written */
    uint32_t in[6]; /* node ids read (alias roots), NONE when unused */
} member_t;

typedef struct {
    lkind kind;
    uint32_t wave, order;
    uint32_t count;
    member_t m[MAXG];
    size_t d[12];
    int act, causal, has_bias, has_res;
    int ta, tb; /* GEMM operands read transposed (an absorbed TRANSPOSE) */
    int i8;     /* GEMM / conv with an int8 weight operand */
    double scale_w; /* its per-tensor scale, taken from the node at create time */
} launch_t;

struct lancius_device_program {
    lancius_hip_ctx* ctx;        /* caller's context: arena, copies, ordering */
    lancius_hip_ctx* exec;       /* context the launches go to (ctx, or the private one) */
    lancius_hip_ctx* private_ctx;/* LANCIUS_DEVICE_GRAPH: context the graph is captured on */
    lancius_hip_graph* graph;    /* captured launch list */
    int cross_stream;            /* private_ctx has its own stream, ordered by events */
    uint32_t n_ids;
    char* arena;
    char** ptr;
    size_t* bytes;
    uint8_t* role;
    uint8_t* is_i8;  /* by id: INPUT holding int8 weights (1 byte per element) */
    /* by id: a weight's copy in the layout its kernel reads, what it is, its
     * dimensions, and whether it must be re-packed before the next run
     * (PACK_STALE after an upload; PACK_EXPOSED once lancius_device_buffer
     * handed out the weight's address, through which the caller may write
     * at any time: re-packed before every run from then on):
     *   PACK_I8:   an int8 GEMM B [K, N] (lancius_hip_i8_pack_weight);
     *   PACK_CONV: an fp32 conv filter OIHW [C_out, C_in, K_h, K_w]
     *              (lancius_hip_conv2d_pack_weight) */
    char** packed;
    uint8_t* packed_kind;
    size_t* packed_dims; /* 4 per id */
    uint8_t* packed_stale;
    uint8_t* readable;
    int32_t** argmax;
    size_t* rows;
    launch_t* launches;
    uint32_t n_launches;
    lancius_device_program_info info;
};

static size_t elems(const lancius_node* n) {
    size_t e = 1;
    for (uint8_t d = 0; d < n->ndim; d++) e *= n->shape[d];
    return e;
}

static size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

/* An int8 weight: dtype INT8 (lancius_quantize.c:26, tested by
 * lancius_vision_ops.c:14) or an int8 copy bound (lancius_scheduler.c:192). */
static int int8_input(const lancius_node* n) {
    return n && n->op == LANCIUS_OP_INPUT && (n->dtype == LANCIUS_DTYPE_INT8 || n->runtime_data_int8 != NULL);
}

static int fail(int code, const char* what) {
    fprintf(stderr, "[LANCIUS DEVICE] %s\n", what);
    return code;
}

/* ---- compile-time scratch ---------------------------------------------------- */

typedef struct {
    const lancius_graph* g;
    const lancius_node** node;  /* by id */
    uint32_t* wave;             /* by id */
    uint32_t* order;            /* by id: index inside its wave */
    uint32_t* consumers;        /* by id */
    uint32_t* sole;             /* by id: the consumer when consumers == 1 */
    uint32_t* root;             /* by id: buffer owner through RESHAPE/FLATTEN */
    uint8_t* absorbed;          /* by id: folded into a later node's GEMM */
    uint32_t* chain_head;       /* by id of a chain's final node: its MATMUL */
    uint32_t* chain_bias;       /* by final node: bias source (root) */
    uint32_t* chain_res;        /* by final node: residual (root) */
    int* chain_act;             /* by final node */
    uint32_t* mm_src;           /* by 2*MATMUL id + operand: untransposed source root, NONE if none */
    const uint8_t* i8;          /* by id: int8 weight input (the program's is_i8) */
} cstate;

static void cstate_free(cstate* c) {
    free(c->node);
    free(c->wave);
    free(c->order);
    free(c->consumers);
    free(c->sole);
    free(c->root);
    free(c->absorbed);
    free(c->chain_head);
    free(c->chain_bias);
    free(c->chain_res);
    free(c->chain_act);
    free(c->mm_src);
}

static const lancius_node* other_operand(const lancius_node* add, uint32_t cur) {
    if (add->input_count != 2 || !add->inputs[0] || !add->inputs[1]) return NULL;
    if (add->inputs[0]->id == cur) return add->inputs[1];
    if (add->inputs[1]->id == cur) return add->inputs[0];
    return NULL;
}

/* A 2-D TRANSPOSE whose only consumer is this MATMUL becomes a transposed
 * read of its input inside the GEMM (no launch, no buffer). */
static void absorb_transposes(cstate* c, const lancius_node* mm) {
    if (c->i8[mm->inputs[1]->id]) return; /* the int8 GEMM reads plain operands */
    for (int j = 0; j < 2; j++) {
        const lancius_node* t = mm->inputs[j];
        if (!t || t->op != LANCIUS_OP_TRANSPOSE || c->consumers[t->id] != 1 || t->ndim != 2 || !t->inputs ||
            !t->inputs[0])
            continue;
        const lancius_node* src = t->inputs[0];
        if (src->ndim != 2 || src->shape[0] != t->shape[1] || src->shape[1] != t->shape[0]) continue;
        c->absorbed[t->id] = 1;
        c->mm_src[2 * mm->id + j] = c->root[src->id];
    }
}

/* MATMUL -> ADD(BROADCAST row) -> RELU|GELU -> ADD(residual), each link only
 * when the intermediate has exactly one consumer; epilogue order matches the
 * node order: ((acc + bias) -> act) + residual. */
static void fuse_gemm_chain(cstate* c, const lancius_node* mm) {
    const size_t M = mm->inputs[0]->shape[0], N = mm->inputs[1]->shape[1];
    uint32_t cur = mm->id;
    uint32_t bias = NONE, res = NONE;
    int act = LANCIUS_HIP_ACT_NONE;
    /* bias */
    if (c->consumers[cur] == 1) {
        const lancius_node* add = c->node[c->sole[cur]];
        const lancius_node* o = add ? other_operand(add, cur) : NULL;
        if (add && add->op == LANCIUS_OP_ADD && o && o->op == LANCIUS_OP_BROADCAST && c->consumers[o->id] == 1 &&
            o->ndim == 2 && o->shape[0] == M && o->shape[1] == N && elems(add) == M * N && o->inputs[0] &&
            elems(o->inputs[0]) >= N && elems(o->inputs[0]) != 1) {
            bias = c->root[o->inputs[0]->id];
            c->absorbed[cur] = 1;
            c->absorbed[o->id] = 1;
            cur = add->id;
        }
    }
    /* activation */
    if (c->consumers[cur] == 1) {
        const lancius_node* a = c->node[c->sole[cur]];
        if (a && (a->op == LANCIUS_OP_RELU || a->op == LANCIUS_OP_GELU) && elems(a) == M * N) {
            act = a->op == LANCIUS_OP_RELU ? LANCIUS_HIP_ACT_RELU : LANCIUS_HIP_ACT_GELU;
            c->absorbed[cur] = 1;
            cur = a->id;
        }
    }
    /* residual */
    if (c->consumers[cur] == 1) {
        const lancius_node* add = c->node[c->sole[cur]];
        const lancius_node* o = add ? other_operand(add, cur) : NULL;
        if (add && add->op == LANCIUS_OP_ADD && o && elems(add) == M * N && elems(o) >= M * N) {
            res = c->root[o->id];
            c->absorbed[cur] = 1;
            cur = add->id;
        }
    }
    if (cur != mm->id) {
        c->chain_head[cur] = mm->id;
        c->chain_bias[cur] = bias;
        c->chain_res[cur] = res;
        c->chain_act[cur] = act;
    }
}

static int supported(lancius_opcode op) {
    switch (op) {
        case LANCIUS_OP_NOP:
        case LANCIUS_OP_INPUT:
        case LANCIUS_OP_CONST:
        case LANCIUS_OP_MATMUL:
        case LANCIUS_OP_ADD:
        case LANCIUS_OP_BROADCAST:
        case LANCIUS_OP_RELU:
        case LANCIUS_OP_GELU:
        case LANCIUS_OP_SOFTMAX:
        case LANCIUS_OP_LAYERNORM:
        case LANCIUS_OP_ATTENTION:
        case LANCIUS_OP_CONV2D:
        case LANCIUS_OP_CONV2D_RELU_FUSED:
        case LANCIUS_OP_RESHAPE:
        case LANCIUS_OP_FLATTEN:
        case LANCIUS_OP_SUB:
        case LANCIUS_OP_MUL:
        case LANCIUS_OP_RELU_BWD:
        case LANCIUS_OP_TRANSPOSE:
        case LANCIUS_OP_SUM:
        case LANCIUS_OP_SUM_AXIS0:
        case LANCIUS_OP_SUM_AXIS1:
        case LANCIUS_OP_SOFTMAX_BWD:
        case LANCIUS_OP_CROSS_ENTROPY:
        case LANCIUS_OP_CROSS_ENTROPY_BWD:
        case LANCIUS_OP_CONV2D_BWD:
        case LANCIUS_OP_CONV2D_BWD_W:
        case LANCIUS_OP_MAXPOOL2D:
        case LANCIUS_OP_MAXPOOL2D_BWD:
        case LANCIUS_OP_RMSNORM:
        case LANCIUS_OP_SWIGLU:
        case LANCIUS_OP_GQA:
        case LANCIUS_OP_ROPE:
            return 1;
        default:
            return 0;
    }
}

#define IN(n, j) ((n)->inputs[j] ? c->root[(n)->inputs[j]->id] : NONE)

/* Builds the launch for final node `n`; checks the operand sizes the
 * reference kernels would read. */
static int make_launch(cstate* c, const lancius_node* n, launch_t* L) {
    memset(L, 0, sizeof(*L));
    L->wave = c->wave[n->id];
    L->order = c->order[n->id];
    L->count = 1;
    member_t* m = &L->m[0];
    m->out = n->id;
    for (int j = 0; j < 6; j++) m->in[j] = NONE;
    for (uint32_t j = 0; j < n->input_count; j++)
        if (!n->inputs[j]) return fail(LANCIUS_HIP_ERR_NULL_PTR, "node with a NULL input");
    const size_t e = elems(n);
    const uint32_t head = c->chain_head[n->id];
    if (head != NONE || n->op == LANCIUS_OP_MATMUL) {
        const lancius_node* mm = head != NONE ? c->node[head] : n;
        const lancius_node* a = mm->inputs[0];
        const lancius_node* b = mm->inputs[1];
        const size_t M = a->shape[0], K = a->shape[1], N = b->shape[1];
        if (M * N > e || elems(a) < M * K || elems(b) < K * N || !M || !K || !N)
            return fail(LANCIUS_HIP_ERR_SHAPE, "MATMUL operand shapes");
        L->kind = L_GEMM;
        L->d[0] = M;
        L->d[1] = K;
        L->d[2] = N;
        const uint32_t sa = c->mm_src[2 * mm->id], sb = c->mm_src[2 * mm->id + 1];
        L->ta = sa != NONE;
        L->tb = sb != NONE;
        m->in[0] = L->ta ? sa : c->root[a->id];
        m->in[1] = L->tb ? sb : c->root[b->id];
        if (head != NONE) {
            m->in[2] = c->chain_bias[n->id];
            m->in[3] = c->chain_res[n->id];
            L->act = c->chain_act[n->id];
        }
        L->has_bias = m->in[2] != NONE;
        L->has_res = m->in[3] != NONE;
        if (c->i8[b->id]) {
            L->i8 = 1;
            L->scale_w = b->scale;
        }
        return 0;
    }
    switch (n->op) {
        case LANCIUS_OP_ADD:
            if (elems(n->inputs[0]) < e || elems(n->inputs[1]) < e) return fail(LANCIUS_HIP_ERR_SHAPE, "ADD sizes");
            L->kind = L_ADD;
            L->d[0] = e;
            m->in[0] = IN(n, 0);
            m->in[1] = IN(n, 1);
            return 0;
        case LANCIUS_OP_RELU:
        case LANCIUS_OP_GELU:
            if (elems(n->inputs[0]) < e) return fail(LANCIUS_HIP_ERR_SHAPE, "unary sizes");
            L->kind = n->op == LANCIUS_OP_RELU ? L_RELU : L_GELU;
            L->d[0] = e;
            m->in[0] = IN(n, 0);
            return 0;
        case LANCIUS_OP_BROADCAST: {
            const size_t in_e = elems(n->inputs[0]);
            L->kind = L_BCAST;
            if (in_e == 1) { /* scalar: every element (lancius_scheduler.c:271-273) */
                L->d[0] = e;
                L->d[1] = 1;
                L->d[2] = 1;
            } else { /* rows x cols of the 2-D view (:275-276) */
                if (n->ndim < 2 || in_e < n->shape[1]) return fail(LANCIUS_HIP_ERR_SHAPE, "BROADCAST sizes");
                L->d[0] = n->shape[0];
                L->d[1] = n->shape[1];
                L->d[2] = in_e;
            }
            m->in[0] = IN(n, 0);
            return 0;
        }
        case LANCIUS_OP_SOFTMAX:
            if (n->ndim != 2 || elems(n->inputs[0]) < e) return fail(LANCIUS_HIP_ERR_SHAPE, "SOFTMAX sizes");
            L->kind = L_SOFTMAX;
            L->d[0] = n->shape[0];
            L->d[1] = n->shape[1];
            m->in[0] = IN(n, 0);
            return 0;
        case LANCIUS_OP_LAYERNORM: {
            /* rows = shape[0], hidden = shape[1] (lancius_scheduler.c:114) */
            const size_t rows = n->shape[0], hid = n->ndim > 1 ? n->shape[1] : 1;
            if (elems(n->inputs[0]) < rows * hid || elems(n->inputs[1]) < hid || elems(n->inputs[2]) < hid)
                return fail(LANCIUS_HIP_ERR_SHAPE, "LAYERNORM sizes");
            L->kind = L_LN;
            L->d[0] = rows;
            L->d[1] = hid;
            m->in[0] = IN(n, 0);
            m->in[1] = IN(n, 1);
            m->in[2] = IN(n, 2);
            return 0;
        }
        case LANCIUS_OP_ATTENTION: {
            const size_t S = n->shape[0], H = n->shape[1], D = n->shape[2];
            const size_t need = S * H * D;
            if (n->ndim != 3 || !need || elems(n->inputs[0]) < need || elems(n->inputs[1]) < need ||
                elems(n->inputs[2]) < need)
                return fail(LANCIUS_HIP_ERR_SHAPE, "ATTENTION sizes");
            L->kind = L_ATTN;
            L->d[0] = S;
            L->d[1] = H;
            L->d[2] = D;
            L->causal = n->axes[0] != 1;
            m->in[0] = IN(n, 0);
            m->in[1] = IN(n, 1);
            m->in[2] = IN(n, 2);
            return 0;
        }
        case LANCIUS_OP_CONV2D:
        case LANCIUS_OP_CONV2D_RELU_FUSED: {
            const lancius_node* x = n->inputs[0];
            const lancius_node* w = n->inputs[1];
            if (x->ndim != 4 || w->ndim != 4 || w->shape[1] != x->shape[1] || n->stride == 0 ||
                x->shape[2] + 2 * (size_t)n->pad < w->shape[2] || x->shape[3] + 2 * (size_t)n->pad < w->shape[3])
                return fail(LANCIUS_HIP_ERR_SHAPE, "CONV2D shapes");
            const size_t Ho = (x->shape[2] + 2 * (size_t)n->pad - w->shape[2]) / n->stride + 1;
            const size_t Wo = (x->shape[3] + 2 * (size_t)n->pad - w->shape[3]) / n->stride + 1;
            if (x->shape[0] * w->shape[0] * Ho * Wo > e) return fail(LANCIUS_HIP_ERR_SHAPE, "CONV2D output size");
            L->kind = L_CONV;
            L->d[0] = x->shape[0];
            L->d[1] = x->shape[1];
            L->d[2] = x->shape[2];
            L->d[3] = x->shape[3];
            L->d[4] = w->shape[0];
            L->d[5] = w->shape[2];
            L->d[6] = w->shape[3];
            L->d[7] = n->stride;
            L->d[8] = n->pad;
            L->act = n->op == LANCIUS_OP_CONV2D_RELU_FUSED ? LANCIUS_HIP_ACT_RELU : LANCIUS_HIP_ACT_NONE;
            m->in[0] = IN(n, 0);
            m->in[1] = IN(n, 1);
            if (w->dtype == LANCIUS_DTYPE_INT8 && c->i8[w->id]) { /* lancius_vision_ops.c:14-16 */
                L->i8 = 1;
                L->scale_w = w->scale;
            }
            return 0;
        }
        case LANCIUS_OP_SUB:
        case LANCIUS_OP_MUL:
        case LANCIUS_OP_RELU_BWD:
            /* elementwise over the node's elements (lancius_scheduler.c:236-245,279-283) */
            if (elems(n->inputs[0]) < e || elems(n->inputs[1]) < e) return fail(LANCIUS_HIP_ERR_SHAPE, "binary sizes");
            L->kind = n->op == LANCIUS_OP_SUB ? L_SUB : n->op == LANCIUS_OP_MUL ? L_MUL : L_RELU_BWD;
            L->d[0] = e;
            m->in[0] = IN(n, 0);
            m->in[1] = IN(n, 1);
            return 0;
        case LANCIUS_OP_TRANSPOSE:
        case LANCIUS_OP_SUM_AXIS0:
        case LANCIUS_OP_SUM_AXIS1: {
            /* rows x cols of the input's first two dims (:246-267) */
            const lancius_node* a = n->inputs[0];
            const size_t R = a->shape[0], Cc = a->ndim > 1 ? a->shape[1] : 1;
            const size_t need = n->op == LANCIUS_OP_TRANSPOSE ? R * Cc : n->op == LANCIUS_OP_SUM_AXIS0 ? Cc : R;
            if (elems(a) < R * Cc || e < need) return fail(LANCIUS_HIP_ERR_SHAPE, "TRANSPOSE/SUM_AXIS sizes");
            L->kind = n->op == LANCIUS_OP_TRANSPOSE ? L_TRANSPOSE : n->op == LANCIUS_OP_SUM_AXIS0 ? L_SUM0 : L_SUM1;
            L->d[0] = R;
            L->d[1] = Cc;
            m->in[0] = IN(n, 0);
            return 0;
        }
        case LANCIUS_OP_SUM:
            if (e < 1) return fail(LANCIUS_HIP_ERR_SHAPE, "SUM output");
            L->kind = L_SUM;
            L->d[0] = elems(n->inputs[0]);
            m->in[0] = IN(n, 0);
            return 0;
        case LANCIUS_OP_SOFTMAX_BWD:
            if (n->ndim != 2 || elems(n->inputs[0]) < e || elems(n->inputs[1]) < e)
                return fail(LANCIUS_HIP_ERR_SHAPE, "SOFTMAX_BWD sizes");
            L->kind = L_SOFTMAX_BWD;
            L->d[0] = n->shape[0];
            L->d[1] = n->shape[1];
            m->in[0] = IN(n, 0);
            m->in[1] = IN(n, 1);
            return 0;
        case LANCIUS_OP_CROSS_ENTROPY: {
            /* rows x cols of the logits (:70) */
            const lancius_node* x = n->inputs[0];
            const size_t R = x->shape[0], Cc = x->ndim > 1 ? x->shape[1] : 1;
            if (!R || !Cc || e < 1 || elems(x) < R * Cc || elems(n->inputs[1]) < R * Cc)
                return fail(LANCIUS_HIP_ERR_SHAPE, "CROSS_ENTROPY sizes");
            L->kind = L_CE;
            L->d[0] = R;
            L->d[1] = Cc;
            m->in[0] = IN(n, 0);
            m->in[1] = IN(n, 1);
            return 0;
        }
        case LANCIUS_OP_CROSS_ENTROPY_BWD: {
            /* rows x cols of the node (:92) */
            const size_t R = n->shape[0], Cc = n->ndim > 1 ? n->shape[1] : 1;
            if (elems(n->inputs[0]) < R * Cc || elems(n->inputs[1]) < R * Cc || elems(n->inputs[2]) < 1 ||
                e < R * Cc)
                return fail(LANCIUS_HIP_ERR_SHAPE, "CROSS_ENTROPY_BWD sizes");
            L->kind = L_CE_BWD;
            L->d[0] = R;
            L->d[1] = Cc;
            m->in[0] = IN(n, 0);
            m->in[1] = IN(n, 1);
            m->in[2] = IN(n, 2);
            return 0;
        }
        case LANCIUS_OP_CONV2D_BWD:
        case LANCIUS_OP_CONV2D_BWD_W: {
            /* CONV2D_BWD: inputs grad, fwd_in, fwd_w; filter from fwd_w
             * (lancius_vision_ops.c:126-137).  CONV2D_BWD_W: inputs grad,
             * fwd_in; C_out and filter from the node (:138-148). */
            const lancius_node* g = n->inputs[0];
            const lancius_node* x = n->inputs[1];
            const int bwd_in = n->op == LANCIUS_OP_CONV2D_BWD;
            const lancius_node* w = bwd_in ? n->inputs[2] : NULL;
            if (g->ndim != 4 || x->ndim != 4 || (bwd_in && w->ndim != 4) || n->ndim != 4 || n->stride == 0)
                return fail(LANCIUS_HIP_ERR_SHAPE, "CONV2D backward ranks");
            const size_t N = x->shape[0], Ci = x->shape[1], H = x->shape[2], W = x->shape[3];
            const size_t Co = bwd_in ? w->shape[0] : n->shape[0];
            const size_t Kh = bwd_in ? w->shape[2] : n->shape[2], Kw = bwd_in ? w->shape[3] : n->shape[3];
            const size_t Ho = g->shape[2], Wo = g->shape[3];
            if (!Kh || !Kw) return fail(LANCIUS_HIP_ERR_SHAPE, "CONV2D backward filter");
            /* every (ho, wo) tap the reference visits lies in [-pad, H + pad) */
            if (elems(g) < N * Co * Ho * Wo || (bwd_in && (w->shape[1] != Ci || elems(w) < Co * Ci * Kh * Kw)) ||
                (!bwd_in && n->shape[1] != Ci) || elems(x) < N * Ci * H * W ||
                e < (bwd_in ? N * Ci * H * W : Co * Ci * Kh * Kw))
                return fail(LANCIUS_HIP_ERR_SHAPE, "CONV2D backward sizes");
            L->kind = bwd_in ? L_CONV_BWD_IN : L_CONV_BWD_W;
            const size_t d[11] = {N, Ci, H, W, Co, Ho, Wo, Kh, Kw, n->stride, n->pad};
            memcpy(L->d, d, sizeof(d));
            m->in[0] = IN(n, 0);
            m->in[1] = bwd_in ? IN(n, 2) : IN(n, 1);
            return 0;
        }
        case LANCIUS_OP_MAXPOOL2D:
        case LANCIUS_OP_MAXPOOL2D_BWD: {
            /* K = kernel_h (lancius_vision_ops.c:87,155); BWD: inputs grad,
             * fwd_in, windows from grad's spatial size (:156) */
            const int bwd = n->op == LANCIUS_OP_MAXPOOL2D_BWD;
            const lancius_node* x = n->inputs[bwd ? 1 : 0];
            const size_t K = n->kernel_h, st = n->stride;
            if (x->ndim != 4 || !K || !st || x->shape[2] < K || x->shape[3] < K)
                return fail(LANCIUS_HIP_ERR_SHAPE, "MAXPOOL2D shape");
            const size_t N = x->shape[0], Cc = x->shape[1], H = x->shape[2], W = x->shape[3];
            size_t Ho = (H - K) / st + 1, Wo = (W - K) / st + 1;
            if (bwd) {
                const lancius_node* g = n->inputs[0];
                if (g->ndim != 4) return fail(LANCIUS_HIP_ERR_SHAPE, "MAXPOOL2D_BWD grad rank");
                if (g->shape[2] > Ho || g->shape[3] > Wo || elems(g) < N * Cc * g->shape[2] * g->shape[3])
                    return fail(LANCIUS_HIP_ERR_SHAPE, "MAXPOOL2D_BWD grad windows");
                Ho = g->shape[2];
                Wo = g->shape[3];
            }
            if (elems(x) < N * Cc * H * W || e < (bwd ? N * Cc * H * W : N * Cc * Ho * Wo))
                return fail(LANCIUS_HIP_ERR_SHAPE, "MAXPOOL2D sizes");
            L->kind = bwd ? L_POOL_BWD : L_POOL;
            const size_t d[8] = {N, Cc, H, W, Ho, Wo, K, st};
            memcpy(L->d, d, sizeof(d));
            m->in[0] = IN(n, 0);
            if (bwd) m->in[1] = IN(n, 1);
            return 0;
        }
        case LANCIUS_OP_RMSNORM: { /* lancius_scheduler.c:134-139: rows shape[0], hidden shape[1] */
            const size_t rows = n->shape[0], hid = n->ndim > 1 ? n->shape[1] : 1;
            if (elems(n->inputs[0]) < rows * hid || elems(n->inputs[1]) < hid || e < rows * hid)
                return fail(LANCIUS_HIP_ERR_SHAPE, "RMSNORM sizes");
            L->kind = L_RMSNORM;
            L->d[0] = rows;
            L->d[1] = hid;
            m->in[0] = IN(n, 0);
            m->in[1] = IN(n, 1);
            return 0;
        }
        case LANCIUS_OP_SWIGLU: /* :140-145 */
            if (elems(n->inputs[0]) < e || elems(n->inputs[1]) < e) return fail(LANCIUS_HIP_ERR_SHAPE, "SWIGLU sizes");
            L->kind = L_SWIGLU;
            L->d[0] = e;
            m->in[0] = IN(n, 0);
            m->in[1] = IN(n, 1);
            return 0;
        case LANCIUS_OP_GQA: { /* :146-152: S shape[0], Hq kernel_h, Hkv kernel_w, D shape[2] */
            const size_t S = n->shape[0], Hq = n->kernel_h, Hkv = n->kernel_w, D = n->ndim > 2 ? n->shape[2] : 0;
            if (n->ndim != 3 || !S || !D || !Hkv || Hq % Hkv || elems(n->inputs[0]) < S * Hq * D ||
                elems(n->inputs[1]) < S * Hkv * D || elems(n->inputs[2]) < S * Hkv * D || e < S * Hq * D)
                return fail(LANCIUS_HIP_ERR_SHAPE, "GQA sizes");
            L->kind = L_GQA;
            L->d[0] = S;
            L->d[1] = Hq;
            L->d[2] = Hkv;
            L->d[3] = D;
            m->in[0] = IN(n, 0);
            m->in[1] = IN(n, 1);
            m->in[2] = IN(n, 2);
            return 0;
        }
        case LANCIUS_OP_ROPE: { /* :153-165: [S, H, 2 hd]: q then k halves */
            const size_t S = n->shape[0], H = n->ndim > 1 ? n->shape[1] : 0, hd2 = n->ndim > 2 ? n->shape[2] : 0;
            if (n->ndim != 3 || hd2 % 2 || hd2 % 4 || elems(n->inputs[0]) < S * H * hd2 || e < S * H * hd2)
                return fail(LANCIUS_HIP_ERR_SHAPE, "ROPE sizes (shape[2] = 2 x an even head dim)");
            L->kind = L_ROPE;
            L->d[0] = S;
            L->d[1] = H;
            L->d[2] = hd2 / 2;
            m->in[0] = IN(n, 0);
            return 0;
        }
        default:
            return fail(LANCIUS_HIP_ERR_UNSUPPORTED, "op outside the device path");
    }
}

static int same_group(const launch_t* a, const launch_t* b) {
    if (a->kind != b->kind || a->wave != b->wave || a->count >= MAXG || a->i8 || b->i8) return 0;
    if (a->kind == L_GEMM)
        return a->d[0] == b->d[0] && a->d[1] == b->d[1] && a->d[2] == b->d[2] && a->act == b->act &&
               a->has_bias == b->has_bias && a->has_res == b->has_res && a->ta == b->ta && a->tb == b->tb;
    if (a->kind == L_ATTN)
        return a->d[0] == b->d[0] && a->d[1] == b->d[1] && a->d[2] == b->d[2] && a->causal == b->causal;
    if (a->kind == L_LN) return a->d[0] == b->d[0] && a->d[1] == b->d[1];
    return 0;
}

static int cmp_launch(const void* x, const void* y) {
    const launch_t* a = (const launch_t*)x;
    const launch_t* b = (const launch_t*)y;
    if (a->wave != b->wave) return a->wave < b->wave ? -1 : 1;
    if (a->order != b->order) return a->order < b->order ? -1 : 1;
    return 0;
}

/* ---- planning over the launch list --------------------------------------------- */

typedef struct {
    uint32_t id, birth, death;
    size_t size, offset;
} ivl_t;

typedef struct fblk {
    size_t off, size;
    struct fblk* next;
} fblk;

/* First fit over a LIFO free list, no coalescing, blocks split from the front
 * (the scan of lancius_memory_planner.c:117-168 with each interval's offset
 * kept).  Returns the region size, or SIZE_MAX on allocation failure. */
static size_t first_fit(ivl_t* iv, uint32_t n) {
    ivl_t** active = (ivl_t**)malloc(sizeof(ivl_t*) * (n ? n : 1));
    fblk* fl = (fblk*)malloc(sizeof(fblk));
    if (!active || !fl) {
        free(active);
        free(fl);
        return SIZE_MAX;
    }
    fl->off = 0;
    fl->size = SIZE_MAX;
    fl->next = NULL;
    size_t peak = 0;
    uint32_t na = 0;
    size_t result = 0;
    for (uint32_t i = 0; i < n; i++) {
        ivl_t* cur = &iv[i];
        uint32_t keep = 0;
        for (uint32_t a = 0; a < na; a++) {
            if (active[a]->death < cur->birth) {
                fblk* b = (fblk*)malloc(sizeof(fblk));
                if (!b) {
                    result = SIZE_MAX;
                    goto done;
                }
                b->off = active[a]->offset;
                b->size = active[a]->size;
                b->next = fl;
                fl = b;
            } else {
                active[keep++] = active[a];
            }
        }
        na = keep;
        fblk *prev = NULL, *b = fl;
        while (b && b->size < cur->size) {
            prev = b;
            b = b->next;
        }
        if (!b) {
            result = SIZE_MAX;
            goto done;
        }
        cur->offset = b->off;
        if (b->size > cur->size) {
            b->off += cur->size;
            b->size -= cur->size;
        } else {
            if (prev) prev->next = b->next;
            else fl = b->next;
            free(b);
        }
        if (cur->offset + cur->size > peak) peak = cur->offset + cur->size;
        active[na++] = cur;
    }
    result = peak;
done:
    while (fl) {
        fblk* nx = fl->next;
        free(fl);
        fl = nx;
    }
    free(active);
    return result;
}

static int caller_plan_fits(const lancius_memory_plan* plan, const ivl_t* iv, uint32_t n, uint32_t n_ids,
                            size_t* region) {
    size_t top = 0;
    for (uint32_t i = 0; i < n; i++) {
        if (iv[i].id >= n_ids || !plan->is_pooled[iv[i].id]) return 0;
        const size_t off = plan->offsets[iv[i].id];
        if (off > SIZE_MAX - iv[i].size) return 0;
        if (off + iv[i].size > top) top = off + iv[i].size;
    }
    for (uint32_t i = 0; i < n; i++) {
        const size_t ai = plan->offsets[iv[i].id], bi = ai + iv[i].size;
        for (uint32_t j = i + 1; j < n; j++) {
            if (iv[i].birth > iv[j].death || iv[j].birth > iv[i].death) continue; /* not live together */
            const size_t aj = plan->offsets[iv[j].id], bj = aj + iv[j].size;
            if (ai < bj && aj < bi) return 0;
        }
    }
    *region = top;
    return 1;
}

static int cmp_ivl_birth(const void* x, const void* y) {
    const ivl_t* a = (const ivl_t*)x;
    const ivl_t* b = (const ivl_t*)y;
    if (a->birth != b->birth) return a->birth < b->birth ? -1 : 1;
    return 0;
}

/* ---- program ------------------------------------------------------------------------ */

void lancius_device_program_destroy(lancius_device_program* p) {
    if (!p) return;
    if (p->graph) lancius_hip_graph_destroy(p->graph);
    if (p->private_ctx) lancius_hip_ctx_destroy(p->private_ctx);
    if (p->arena) lancius_hip_free(p->ctx, p->arena);
    if (p->packed)
        for (uint32_t i = 0; i < p->n_ids; i++)
            if (p->packed[i]) lancius_hip_free(p->ctx, p->packed[i]);
    free(p->packed);
    free(p->packed_kind);
    free(p->packed_dims);
    free(p->packed_stale);
    free(p->ptr);
    free(p->bytes);
    free(p->role);
    free(p->is_i8);
    free(p->readable);
    free(p->argmax);
    free(p->rows);
    free(p->launches);
    free(p);
}

int lancius_device_program_info_get(const lancius_device_program* p, lancius_device_program_info* info) {
    if (!p || !info) return LANCIUS_HIP_ERR_NULL_PTR;
    *info = p->info;
    return 0;
}

#define CALLOC(ptr, n) ((ptr) = calloc((n) ? (n) : 1, sizeof(*(ptr))))

/* GEMM(+bias, act) -> GEMM(+bias) [-> SOFTMAX] on adjacent launches, the
 * hidden and logit tensors each read once by the next launch, small enough
 * for lancius_hip_mlp2_f32 (M <= 64, N2 <= 64, M*N1 <= 16384,
 * N1*N2 <= 8192, K1*max(M, N1) <= 2^28): one launch instead of up to three
 * dependent ones. */
/* Launches read tensors through their buffer owner (RESHAPE/FLATTEN
 * aliases resolved), so a node with one direct consumer can still be read
 * by several launches: h -> FLATTEN -> {GEMM, RELU}.  The buffer of `r` may
 * only be fused away when exactly one operand slot of the whole launch list
 * reads it, that slot is in launch `reader`, and no alias of `r` is a sink
 * (a caller may download sinks). */
static int sole_reader(const lancius_device_program* p, const cstate* c, uint32_t nl, uint32_t r,
                       uint32_t reader) {
    uint32_t reads = 0;
    for (uint32_t s = 0; s < nl; s++) {
        const launch_t* L = &p->launches[s];
        for (uint32_t k = 0; k < L->count; k++)
            for (int j = 0; j < 6; j++)
                if (L->m[k].in[j] == r) {
                    if (s != reader) return 0;
                    reads++;
                }
    }
    if (reads != 1) return 0;
    for (uint32_t i = 0; i < c->g->node_count; i++) {
        const lancius_node* n = c->g->nodes[i];
        if (n->id != r && c->root[n->id] == r && c->consumers[n->id] == 0) return 0;
    }
    return 1;
}

static uint32_t fuse_mlp2(lancius_device_program* p, const cstate* c, uint32_t nl) {
    for (uint32_t s = 0; s + 1 < nl; s++) {
        launch_t* A = &p->launches[s];
        launch_t* B = &p->launches[s + 1];
        if (A->kind != L_GEMM || B->kind != L_GEMM || A->count != 1 || B->count != 1) continue;
        if (A->ta || A->tb || A->i8 || A->has_res || B->ta || B->tb || B->i8 || B->has_res || B->act) continue;
        const uint32_t h = A->m[0].out, y = B->m[0].out;
        if (B->m[0].in[0] != h || B->m[0].in[1] == h || c->consumers[h] != 1 || !sole_reader(p, c, nl, h, s + 1))
            continue;
        const size_t M = A->d[0], K1 = A->d[1], N1 = A->d[2], N2 = B->d[2];
        if (B->d[0] != M || B->d[1] != N1 || M > 64 || N2 > 64 || M * N1 > 16384 || N1 * N2 > 8192 ||
            K1 * (M > N1 ? M : N1) > ((size_t)1 << 28))
            continue;
        int sm = 0;
        if (s + 2 < nl) {
            const launch_t* S = &p->launches[s + 2];
            sm = S->kind == L_SOFTMAX && S->count == 1 && S->m[0].in[0] == y && c->consumers[y] == 1 &&
                 S->d[0] == M && S->d[1] == N2 && sole_reader(p, c, nl, y, s + 2);
        }
        launch_t F = *A;
        F.kind = L_MLP2;
        F.m[0].out = sm ? p->launches[s + 2].m[0].out : y;
        F.m[0].in[3] = B->m[0].in[1]; /* W2 */
        F.m[0].in[4] = B->m[0].in[2]; /* b2 */
        F.d[0] = M;
        F.d[1] = K1;
        F.d[2] = N1;
        F.d[3] = N2;
        F.d[4] = (size_t)sm;
        p->role[h] = ROLE_FUSED;
        p->info.fused_nodes++;
        if (sm) {
            p->role[y] = ROLE_FUSED;
            p->info.fused_nodes++;
        }
        const uint32_t drop = sm ? 2 : 1;
        p->launches[s] = F;
        for (uint32_t k = s + 1; k + drop < nl; k++) p->launches[k] = p->launches[k + drop];
        nl -= drop;
    }
    return nl;
}

int lancius_device_program_create(lancius_hip_ctx* ctx, const lancius_graph* g, const lancius_schedule* sched,
                                  const lancius_memory_plan* plan, uint32_t flags, lancius_device_program** out) {
    if (!ctx || !g || !sched || !out) return LANCIUS_HIP_ERR_NULL_PTR;
    *out = NULL;
    if (flags & LANCIUS_DEVICE_KEEP_ALL) flags |= LANCIUS_DEVICE_NO_FUSION;
    const uint32_t ids = g->next_id;
    int rc = 0;
    cstate c;
    memset(&c, 0, sizeof(c));
    c.g = g;
    lancius_device_program* p = (lancius_device_program*)calloc(1, sizeof(*p));
    ivl_t* iv = NULL;
    uint32_t* birth = NULL;
    uint32_t* last = NULL;
    uint8_t* pinned = NULL;
    float* fillbuf = NULL;
    if (!p) return LANCIUS_HIP_ERR_OOM;
    p->ctx = ctx;
    p->exec = ctx;
    p->n_ids = ids;
    const size_t ids2 = 2 * (size_t)ids, ids4 = 4 * (size_t)ids;
    if (!CALLOC(c.node, ids) || !CALLOC(c.wave, ids) || !CALLOC(c.order, ids) || !CALLOC(c.consumers, ids) ||
        !CALLOC(c.sole, ids) || !CALLOC(c.root, ids) || !CALLOC(c.absorbed, ids) || !CALLOC(c.chain_head, ids) ||
        !CALLOC(c.chain_bias, ids) || !CALLOC(c.chain_res, ids) || !CALLOC(c.chain_act, ids) ||
        !CALLOC(c.mm_src, ids2) ||
        !CALLOC(p->ptr, ids) || !CALLOC(p->bytes, ids) || !CALLOC(p->role, ids) || !CALLOC(p->readable, ids) ||
        !CALLOC(p->is_i8, ids) || !CALLOC(p->packed, ids) || !CALLOC(p->packed_kind, ids) ||
        !CALLOC(p->packed_dims, ids4) || !CALLOC(p->packed_stale, ids) ||
        !CALLOC(p->argmax, ids) || !CALLOC(p->rows, ids) || !CALLOC(birth, ids) || !CALLOC(last, ids) ||
        !CALLOC(pinned, ids)) {
        rc = LANCIUS_HIP_ERR_OOM;
        goto out;
    }
    for (uint32_t i = 0; i < ids; i++) {
        c.wave[i] = NONE;
        c.chain_head[i] = NONE;
        c.mm_src[2 * i] = c.mm_src[2 * i + 1] = NONE;
        c.root[i] = i;
        birth[i] = NONE;
    }
    for (uint32_t i = 0; i < g->node_count; i++) {
        const lancius_node* n = g->nodes[i];
        if (n->id >= ids) {
            rc = fail(LANCIUS_HIP_ERR_SHAPE, "node id beyond graph next_id");
            goto out;
        }
        c.node[n->id] = n;
        p->is_i8[n->id] = (uint8_t)int8_input(n);
        if (!supported(n->op)) {
            fprintf(stderr, "[LANCIUS DEVICE] op %d (node %u) is not on the device path\n", (int)n->op, n->id);
            rc = LANCIUS_HIP_ERR_UNSUPPORTED;
            goto out;
        }
        for (uint32_t j = 0; j < n->input_count; j++) {
            if (!n->inputs[j]) continue;
            const uint32_t in = n->inputs[j]->id;
            if (in >= ids) {
                rc = fail(LANCIUS_HIP_ERR_SHAPE, "input id beyond graph next_id");
                goto out;
            }
            c.consumers[in]++;
            c.sole[in] = n->id;
        }
    }
    /* An int8 INPUT stays int8 only when every consumer reads it as the weight
     * operand of a MATMUL or conv; one used as an activation (the reference's
     * quantizer also converts 4-D images) is fed in fp32 and quantized by the
     * kernel that reads it, which gives the same int8 values. */
    for (uint32_t i = 0; i < g->node_count; i++) {
        const lancius_node* n = g->nodes[i];
        for (uint32_t j = 0; j < n->input_count; j++) {
            if (!n->inputs[j] || !p->is_i8[n->inputs[j]->id]) continue;
            const int weight_slot = j == 1 && (n->op == LANCIUS_OP_MATMUL || n->op == LANCIUS_OP_CONV2D ||
                                               n->op == LANCIUS_OP_CONV2D_RELU_FUSED);
            if (!weight_slot) p->is_i8[n->inputs[j]->id] = 0;
        }
    }
    for (uint32_t i = 0; i < g->node_count; i++) {
        const lancius_node* n = g->nodes[i];
        p->bytes[n->id] = elems(n) * (p->is_i8[n->id] ? 1 : sizeof(float));
    }
    c.i8 = p->is_i8;
    uint32_t scheduled = 0;
    for (uint32_t w = 0; w < sched->wave_count; w++)
        for (uint32_t i = 0; i < sched->waves[w].node_count; i++) {
            const lancius_node* n = sched->waves[w].nodes[i];
            if (n->id >= ids || c.node[n->id] != n) {
                rc = fail(LANCIUS_HIP_ERR_SHAPE, "schedule holds a node of another graph");
                goto out;
            }
            c.wave[n->id] = w;
            c.order[n->id] = i;
            scheduled++;
        }
    if (scheduled != g->node_count) {
        rc = fail(LANCIUS_HIP_ERR_SHAPE, "schedule does not cover the graph (cycle?)");
        goto out;
    }

    /* roles and aliases, in wave order so an alias's input is resolved first */
    for (uint32_t w = 0; w < sched->wave_count; w++)
        for (uint32_t i = 0; i < sched->waves[w].node_count; i++) {
            const lancius_node* n = sched->waves[w].nodes[i];
            if (n->op == LANCIUS_OP_INPUT) {
                p->role[n->id] = ROLE_INPUT;
            } else if (n->op == LANCIUS_OP_CONST) {
                p->role[n->id] = ROLE_CONST;
            } else if (n->op == LANCIUS_OP_NOP) {
                p->role[n->id] = ROLE_NONE;
            } else if (n->op == LANCIUS_OP_RESHAPE || n->op == LANCIUS_OP_FLATTEN) {
                if (!n->inputs || !n->inputs[0]) {
                    rc = fail(LANCIUS_HIP_ERR_NULL_PTR, "RESHAPE without input");
                    goto out;
                }
                const uint32_t r = c.root[n->inputs[0]->id];
                if (elems(n) > elems(c.node[r])) {
                    rc = fail(LANCIUS_HIP_ERR_SHAPE, "RESHAPE larger than its input");
                    goto out;
                }
                c.root[n->id] = r;
                p->role[n->id] = ROLE_ALIAS;
            }
        }

    if (!(flags & LANCIUS_DEVICE_NO_FUSION))
        for (uint32_t w = 0; w < sched->wave_count; w++)
            for (uint32_t i = 0; i < sched->waves[w].node_count; i++) {
                const lancius_node* n = sched->waves[w].nodes[i];
                if (n->op == LANCIUS_OP_MATMUL && !c.absorbed[n->id] && n->inputs && n->inputs[0] && n->inputs[1]) {
                    absorb_transposes(&c, n);
                    fuse_gemm_chain(&c, n);
                }
            }

    /* launches, one per final node, sorted by (wave, position) */
    p->launches = (launch_t*)calloc(g->node_count ? g->node_count : 1, sizeof(launch_t));
    if (!p->launches) {
        rc = LANCIUS_HIP_ERR_OOM;
        goto out;
    }
    uint32_t nl = 0;
    for (uint32_t i = 0; i < g->node_count; i++) {
        const lancius_node* n = g->nodes[i];
        const uint8_t role = p->role[n->id];
        if (role == ROLE_INPUT || role == ROLE_CONST || role == ROLE_ALIAS || n->op == LANCIUS_OP_NOP) continue;
        if (c.absorbed[n->id]) {
            p->role[n->id] = ROLE_FUSED;
            p->info.fused_nodes++;
            continue;
        }
        if ((rc = make_launch(&c, n, &p->launches[nl]))) goto out;
        p->role[n->id] = ROLE_POOLED;
        nl++;
    }
    qsort(p->launches, nl, sizeof(launch_t), cmp_launch);
    /* merge branches of one wave */
    if (!(flags & (LANCIUS_DEVICE_NO_FUSION | LANCIUS_DEVICE_NO_GROUP))) {
        uint32_t k = 0;
        for (uint32_t i = 0; i < nl; i++) {
            int merged = 0;
            for (uint32_t j = k; j-- > 0;) {
                if (p->launches[j].wave != p->launches[i].wave) break;
                if (same_group(&p->launches[j], &p->launches[i])) {
                    p->launches[j].m[p->launches[j].count++] = p->launches[i].m[0];
                    merged = 1;
                    break;
                }
            }
            if (!merged) p->launches[k++] = p->launches[i];
        }
        nl = k;
    }
    if (!(flags & (LANCIUS_DEVICE_NO_FUSION | LANCIUS_DEVICE_KEEP_ALL | LANCIUS_DEVICE_NO_CHAIN)))
        nl = fuse_mlp2(p, &c, nl);
    p->n_launches = nl;
    p->info.launches = nl;

    /* lifetimes over launch steps */
    for (uint32_t s = 0; s < nl; s++) {
        const launch_t* L = &p->launches[s];
        for (uint32_t k = 0; k < L->count; k++) {
            birth[L->m[k].out] = s;
            if (last[L->m[k].out] < s) last[L->m[k].out] = s;
            for (int j = 0; j < 6; j++) {
                const uint32_t r = L->m[k].in[j];
                if (r != NONE && last[r] < s) last[r] = s;
            }
        }
    }
    for (uint32_t i = 0; i < g->node_count; i++) {
        const lancius_node* n = g->nodes[i];
        if (p->role[n->id] == ROLE_ALIAS) p->info.aliased_nodes++;
        const int sink = c.consumers[n->id] == 0 && n->op != LANCIUS_OP_NOP;
        if (sink || (flags & LANCIUS_DEVICE_KEEP_ALL)) {
            pinned[c.root[n->id]] = 1;
            p->readable[n->id] = p->role[n->id] != ROLE_FUSED && p->role[n->id] != ROLE_NONE;
        }
        if (p->role[n->id] == ROLE_INPUT || p->role[n->id] == ROLE_CONST) p->readable[n->id] = 1;
    }
    iv = (ivl_t*)calloc(nl * MAXG + 1, sizeof(ivl_t));
    if (!iv) {
        rc = LANCIUS_HIP_ERR_OOM;
        goto out;
    }
    uint32_t niv = 0;
    for (uint32_t i = 0; i < g->node_count; i++) { /* graph order, then stable by birth */
        const uint32_t id = g->nodes[i]->id;
        if (p->role[id] != ROLE_POOLED) continue;
        iv[niv].id = id;
        iv[niv].birth = birth[id];
        iv[niv].death = pinned[id] ? UINT32_MAX - 1 : last[id];
        iv[niv].size = align_up(p->bytes[id] ? p->bytes[id] : 1, 32);
        niv++;
    }
    /* insertion sort keeps graph order among equal births */
    for (uint32_t i = 1; i < niv; i++) {
        ivl_t key = iv[i];
        uint32_t j = i;
        while (j > 0 && cmp_ivl_birth(&iv[j - 1], &key) > 0) {
            iv[j] = iv[j - 1];
            j--;
        }
        iv[j] = key;
    }
    size_t region = 0;
    if (plan && plan->offsets && plan->is_pooled && caller_plan_fits(plan, iv, niv, ids, &region)) {
        for (uint32_t i = 0; i < niv; i++) iv[i].offset = plan->offsets[iv[i].id];
        p->info.used_caller_plan = 1;
    } else {
        p->info.replanned = plan != NULL;
        region = first_fit(iv, niv);
        if (region == SIZE_MAX) {
            rc = LANCIUS_HIP_ERR_OOM;
            goto out;
        }
    }
    const size_t plan_bytes = align_up(region, ALIGN_DEV);
    size_t in_bytes = 0;
    size_t* in_off = (size_t*)calloc(ids ? ids : 1, sizeof(size_t));
    size_t* am_off = (size_t*)calloc(ids ? ids : 1, sizeof(size_t));
    if (!in_off || !am_off) {
        free(in_off);
        free(am_off);
        rc = LANCIUS_HIP_ERR_OOM;
        goto out;
    }
    for (uint32_t i = 0; i < g->node_count; i++) {
        const lancius_node* n = g->nodes[i];
        if (p->role[n->id] == ROLE_INPUT || p->role[n->id] == ROLE_CONST) {
            in_off[n->id] = in_bytes;
            in_bytes += align_up(p->bytes[n->id] ? p->bytes[n->id] : 1, ALIGN_DEV);
        }
        if (n->op == LANCIUS_OP_SOFTMAX && p->role[n->id] == ROLE_POOLED) {
            am_off[n->id] = in_bytes;
            p->rows[n->id] = n->shape[0];
            in_bytes += align_up(n->shape[0] * sizeof(int32_t) + 1, ALIGN_DEV);
        }
    }
    p->info.plan_bytes = plan_bytes;
    p->info.input_bytes = in_bytes;
    p->info.arena_bytes = plan_bytes + in_bytes;
    void* arena = NULL;
    rc = lancius_hip_malloc(ctx, &arena, p->info.arena_bytes ? p->info.arena_bytes : ALIGN_DEV);
    if (rc) {
        free(in_off);
        free(am_off);
        goto out;
    }
    p->arena = (char*)arena;
    for (uint32_t i = 0; i < niv; i++) p->ptr[iv[i].id] = p->arena + iv[i].offset;
    for (uint32_t i = 0; i < g->node_count; i++) {
        const lancius_node* n = g->nodes[i];
        if (p->role[n->id] == ROLE_INPUT || p->role[n->id] == ROLE_CONST) p->ptr[n->id] = p->arena + plan_bytes + in_off[n->id];
        if (p->rows[n->id]) p->argmax[n->id] = (int32_t*)(p->arena + plan_bytes + am_off[n->id]);
    }
    for (uint32_t i = 0; i < g->node_count; i++) {
        const lancius_node* n = g->nodes[i];
        if (p->role[n->id] == ROLE_ALIAS) p->ptr[n->id] = p->ptr[c.root[n->id]];
    }
    free(in_off);
    free(am_off);
    /* CONST nodes are filled once; the region is never reused */
    for (uint32_t i = 0; i < g->node_count; i++) {
        const lancius_node* n = g->nodes[i];
        if (p->role[n->id] != ROLE_CONST) continue;
        rc = lancius_hip_fill_f32(ctx, (float*)p->ptr[n->id], (float)n->attr_val, elems(n));
        if (rc) goto out;
    }
    /* one packed copy per int8 GEMM weight, and per fp32 conv filter that
     * the caller or a CONST fills (not one a launch computes), filled by the
     * first run */
    for (uint32_t i = 0; i < p->n_launches && !rc; i++) {
        const launch_t* L = &p->launches[i];
        const uint32_t w = L->m[0].in[1];
        /* only these two launch kinds read a weight in slot 1; other kinds
         * may leave it NONE */
        if ((L->kind != L_GEMM && L->kind != L_CONV) || w == NONE || p->packed[w]) continue;
        size_t* d = p->packed_dims + 4 * (size_t)w;
        size_t bytes = 0;
        if (L->kind == L_GEMM && L->i8) {
            p->packed_kind[w] = PACK_I8;
            d[0] = L->d[1];
            d[1] = L->d[2];
            bytes = lancius_hip_i8_packed_bytes(d[0], d[1]);
        } else if (L->kind == L_CONV && !L->i8 && L->d[1] % 16 == 0 && L->d[4] % 4 == 0 &&
                   L->d[1] * L->d[2] * L->d[3] * sizeof(float) < LANCIUS_HIP_CONV_PACKED_MAX_BYTES &&
                   L->d[4] * L->d[1] * L->d[5] * L->d[6] * sizeof(float) < LANCIUS_HIP_CONV_PACKED_MAX_BYTES &&
                   (p->role[w] == ROLE_INPUT || p->role[w] == ROLE_CONST)) {
            p->packed_kind[w] = PACK_CONV;
            d[0] = L->d[4];
            d[1] = L->d[1];
            d[2] = L->d[5];
            d[3] = L->d[6];
            bytes = lancius_hip_conv2d_packed_bytes(d[0], d[1], d[2], d[3]);
        } else {
            continue;
        }
        void* buf = NULL;
        rc = lancius_hip_malloc(ctx, &buf, bytes);
        p->packed[w] = (char*)buf;
        p->packed_stale[w] = PACK_STALE;
    }
    if (rc) goto out;
    rc = lancius_hip_synchronize(ctx);
    if (!rc && (flags & LANCIUS_DEVICE_GRAPH)) {
        /* A private context keeps the workspace the graph captures away from
         * the caller's other launches (which may grow and free theirs).  It
         * shares the caller's stream; the null stream cannot be captured, so
         * there it gets a stream of its own, ordered against the caller's by
         * events. */
        void* stream = lancius_hip_ctx_stream(ctx);
        const int dev = lancius_hip_ctx_device(ctx);
        p->cross_stream = stream == NULL;
        rc = stream ? lancius_hip_ctx_create(dev, stream, &p->private_ctx)
                    : lancius_hip_ctx_create_own_stream(dev, &p->private_ctx);
        if (!rc) p->exec = p->private_ctx;
    }

out:
    free(fillbuf);
    free(iv);
    free(birth);
    free(last);
    free(pinned);
    cstate_free(&c);
    if (rc) {
        lancius_device_program_destroy(p);
        return rc;
    }
    *out = p;
    return 0;
}

/* ---- run ---------------------------------------------------------------------------- */

#define P(id) ((id) == NONE ? NULL : (float*)prog->ptr[(id)])

static int run_launch(lancius_device_program* prog, const launch_t* L) {
    lancius_hip_ctx* ctx = prog->exec;
    const member_t* m = &L->m[0];
    switch (L->kind) {
        case L_GEMM: {
            if (L->i8)
                return lancius_hip_gemm_i8p_f32(ctx, P(m->out), P(m->in[0]), (const int8_t*)prog->packed[m->in[1]],
                                                L->scale_w, L->d[0], L->d[1], L->d[2], P(m->in[2]), L->act,
                                                P(m->in[3]));
            float* C[MAXG];
            const float *A[MAXG], *B[MAXG], *bias[MAXG], *res[MAXG];
            for (uint32_t k = 0; k < L->count; k++) {
                C[k] = P(L->m[k].out);
                A[k] = P(L->m[k].in[0]);
                B[k] = P(L->m[k].in[1]);
                bias[k] = P(L->m[k].in[2]);
                res[k] = P(L->m[k].in[3]);
            }
            return lancius_hip_gemm_grouped_ex_f32(ctx, L->count, C, A, B, L->d[0], L->d[1], L->d[2], L->ta, L->tb,
                                                   bias, L->act, res);
        }
        case L_ATTN: {
            float* O[MAXG];
            const float *Q[MAXG], *K[MAXG], *V[MAXG];
            for (uint32_t k = 0; k < L->count; k++) {
                O[k] = P(L->m[k].out);
                Q[k] = P(L->m[k].in[0]);
                K[k] = P(L->m[k].in[1]);
                V[k] = P(L->m[k].in[2]);
            }
            return lancius_hip_attention_grouped_f32(ctx, L->count, O, Q, K, V, L->d[0], L->d[1], L->d[2], L->causal,
                                                     (float)(1.0 / sqrt((double)L->d[2])));
        }
        case L_CONV:
            if (L->i8)
                return lancius_hip_conv2d_i8_f32(ctx, P(m->out), P(m->in[0]), (const int8_t*)prog->ptr[m->in[1]],
                                                 L->scale_w, NULL, L->d[0], L->d[1], L->d[2], L->d[3], L->d[4],
                                                 L->d[5], L->d[6], L->d[7], L->d[8], L->act);
            if (prog->packed[m->in[1]])
                return lancius_hip_conv2d_packed_f32(ctx, P(m->out), P(m->in[0]), (const float*)prog->packed[m->in[1]],
                                                     NULL, L->d[0], L->d[1], L->d[2], L->d[3], L->d[4], L->d[5],
                                                     L->d[6], L->d[7], L->d[8], L->act);
            return lancius_hip_conv2d_f32(ctx, P(m->out), P(m->in[0]), P(m->in[1]), NULL, L->d[0], L->d[1], L->d[2],
                                          L->d[3], L->d[4], L->d[5], L->d[6], L->d[7], L->d[8], L->act);
        case L_LN: {
            float* O[MAXG];
            const float *X[MAXG], *G[MAXG], *Bt[MAXG];
            for (uint32_t k = 0; k < L->count; k++) {
                O[k] = P(L->m[k].out);
                X[k] = P(L->m[k].in[0]);
                G[k] = P(L->m[k].in[1]);
                Bt[k] = P(L->m[k].in[2]);
            }
            return lancius_hip_layernorm_grouped_f32(ctx, L->count, O, X, G, Bt, L->d[0], L->d[1], 1e-5f);
        }
        case L_SOFTMAX:
            return lancius_hip_softmax_f32(ctx, P(m->out), prog->argmax[m->out], P(m->in[0]), L->d[0], L->d[1]);
        case L_ADD:
            return lancius_hip_add_f32(ctx, P(m->out), P(m->in[0]), P(m->in[1]), L->d[0]);
        case L_RELU:
            return lancius_hip_relu_f32(ctx, P(m->out), P(m->in[0]), L->d[0]);
        case L_GELU:
            return lancius_hip_gelu_f32(ctx, P(m->out), P(m->in[0]), L->d[0]);
        case L_BCAST:
            return lancius_hip_broadcast_f32(ctx, P(m->out), P(m->in[0]), L->d[0], L->d[1], L->d[2]);
        case L_SUB:
            return lancius_hip_sub_f32(ctx, P(m->out), P(m->in[0]), P(m->in[1]), L->d[0]);
        case L_MUL:
            return lancius_hip_mul_f32(ctx, P(m->out), P(m->in[0]), P(m->in[1]), L->d[0]);
        case L_RELU_BWD:
            return lancius_hip_relu_bwd_f32(ctx, P(m->out), P(m->in[0]), P(m->in[1]), L->d[0]);
        case L_TRANSPOSE:
            return lancius_hip_transpose_f32(ctx, P(m->out), P(m->in[0]), L->d[0], L->d[1]);
        case L_SUM:
            return lancius_hip_sum_f32(ctx, P(m->out), P(m->in[0]), L->d[0]);
        case L_SUM0:
            return lancius_hip_sum_axis0_f32(ctx, P(m->out), P(m->in[0]), L->d[0], L->d[1]);
        case L_SUM1:
            return lancius_hip_sum_axis1_f32(ctx, P(m->out), P(m->in[0]), L->d[0], L->d[1]);
        case L_SOFTMAX_BWD:
            return lancius_hip_softmax_bwd_f32(ctx, P(m->out), P(m->in[0]), P(m->in[1]), L->d[0], L->d[1]);
        case L_CE:
            return lancius_hip_cross_entropy_f32(ctx, P(m->out), P(m->in[0]), P(m->in[1]), L->d[0], L->d[1]);
        case L_CE_BWD:
            return lancius_hip_cross_entropy_bwd_f32(ctx, P(m->out), P(m->in[0]), P(m->in[1]), P(m->in[2]), L->d[0],
                                                     L->d[1]);
        case L_CONV_BWD_IN:
            return lancius_hip_conv2d_bwd_input_f32(ctx, P(m->out), P(m->in[0]), P(m->in[1]), L->d[0], L->d[1],
                                                    L->d[2], L->d[3], L->d[4], L->d[5], L->d[6], L->d[7], L->d[8],
                                                    L->d[9], L->d[10]);
        case L_CONV_BWD_W:
            return lancius_hip_conv2d_bwd_weight_f32(ctx, P(m->out), P(m->in[0]), P(m->in[1]), L->d[0], L->d[1],
                                                     L->d[2], L->d[3], L->d[4], L->d[5], L->d[6], L->d[7], L->d[8],
                                                     L->d[9], L->d[10]);
        case L_POOL:
            return lancius_hip_maxpool2d_f32(ctx, P(m->out), P(m->in[0]), L->d[0], L->d[1], L->d[2], L->d[3],
                                             L->d[6], L->d[7]);
        case L_RMSNORM:
            return lancius_hip_rmsnorm_f32(ctx, P(m->out), P(m->in[0]), P(m->in[1]), L->d[0], L->d[1], 1e-5f);
        case L_SWIGLU:
            return lancius_hip_swiglu_f32(ctx, P(m->out), P(m->in[0]), P(m->in[1]), L->d[0]);
        case L_GQA:
            return lancius_hip_attention_gqa_f32(ctx, P(m->out), P(m->in[0]), P(m->in[1]), P(m->in[2]), 1, L->d[0],
                                                 L->d[0], L->d[1], L->d[2], L->d[3], 1,
                                                 (float)(1.0 / sqrt((double)L->d[3])));
        case L_ROPE:
            return lancius_hip_rope_f32(ctx, P(m->out), P(m->in[0]), 2, 1, L->d[0], L->d[1], L->d[2], 0);
        case L_MLP2:
            return lancius_hip_mlp2_f32(ctx, P(m->out), L->d[4] ? prog->argmax[m->out] : NULL, P(m->in[0]),
                                        P(m->in[1]), P(m->in[2]), L->act, P(m->in[3]), P(m->in[4]), L->d[0], L->d[1],
                                        L->d[2], L->d[3], (int)L->d[4]);
        case L_POOL_BWD:
            return lancius_hip_maxpool2d_bwd_f32(ctx, P(m->out), P(m->in[0]), P(m->in[1]), L->d[0], L->d[1],
                                                 L->d[2], L->d[3], L->d[4], L->d[5], L->d[6], L->d[7]);
    }
    return LANCIUS_HIP_ERR_INTERNAL;
}

static int run_all(lancius_device_program* prog) {
    for (uint32_t s = 0; s < prog->n_launches; s++) {
        const int rc = run_launch(prog, &prog->launches[s]);
        if (rc) return rc;
    }
    return 0;
}

/* Re-lay every packed weight that changed since it was last packed, or
 * whose address the caller holds, on the caller's stream (after its
 * uploads, before the launches). */
static int repack_stale(lancius_device_program* prog) {
    for (uint32_t i = 0; i < prog->n_ids; i++) {
        if (!prog->packed_stale[i]) continue;
        const size_t* d = prog->packed_dims + 4 * (size_t)i;
        const int rc = prog->packed_kind[i] == PACK_I8
                           ? lancius_hip_i8_pack_weight(prog->ctx, (int8_t*)prog->packed[i],
                                                        (const int8_t*)prog->ptr[i], d[0], d[1])
                           : lancius_hip_conv2d_pack_weight(prog->ctx, (float*)prog->packed[i],
                                                            (const float*)prog->ptr[i], d[0], d[1], d[2], d[3]);
        if (rc) return rc;
        if (prog->packed_stale[i] == PACK_STALE) prog->packed_stale[i] = PACK_FRESH;
    }
    return 0;
}

int lancius_device_run(lancius_device_program* prog) {
    if (!prog) return LANCIUS_HIP_ERR_NULL_PTR;
    const int rc_pack = repack_stale(prog);
    if (rc_pack) return rc_pack;
    if (!prog->private_ctx) return run_all(prog);
    /* graph mode.  On a stream of its own, the replay starts after the
     * caller's work and the caller's stream continues after it. */
    int rc = prog->cross_stream ? lancius_hip_stream_wait(prog->private_ctx, prog->ctx) : 0;
    if (rc) return rc;
    if (prog->graph) {
        rc = lancius_hip_graph_launch(prog->graph, prog->exec);
    } else {
        /* eager pass (allocates workspaces, produces this run's results), then
         * record the same launches */
        rc = run_all(prog);
        if (!rc) rc = lancius_hip_capture_begin(prog->exec);
        if (!rc) {
            const int rc_run = run_all(prog);
            lancius_hip_graph* g = NULL;
            const int rc_end = lancius_hip_capture_end(prog->exec, &g);
            rc = rc_run ? rc_run : rc_end;
            if (!rc) prog->graph = g;
            else if (g) lancius_hip_graph_destroy(g);
        }
    }
    const int rc2 = prog->cross_stream ? lancius_hip_stream_wait(prog->ctx, prog->private_ctx) : 0;
    return rc ? rc : rc2;
}

void* lancius_device_buffer(lancius_device_program* prog, const lancius_node* n) {
    if (!prog || !n || n->id >= prog->n_ids) return NULL;
    if (prog->packed[n->id]) prog->packed_stale[n->id] = PACK_EXPOSED; /* the caller may write through it */
    return prog->ptr[n->id];
}

int lancius_device_upload(lancius_device_program* prog, const lancius_node* n, const void* host,
                          lancius_dtype host_dtype) {
    if (!prog || !n || !host) return LANCIUS_HIP_ERR_NULL_PTR;
    if (n->id >= prog->n_ids || (prog->role[n->id] != ROLE_INPUT && prog->role[n->id] != ROLE_CONST))
        return LANCIUS_HIP_ERR_UNSUPPORTED;
    const size_t e = elems(n);
    if (prog->packed[n->id] && prog->packed_stale[n->id] != PACK_EXPOSED)
        prog->packed_stale[n->id] = PACK_STALE; /* re-packed by the next run */
    if (prog->is_i8[n->id]) { /* int8 weights take their int8 bytes */
        if (host_dtype != LANCIUS_DTYPE_INT8) return LANCIUS_HIP_ERR_DTYPE;
        return lancius_hip_upload(prog->ctx, prog->ptr[n->id], host, e);
    }
    if (host_dtype == LANCIUS_DTYPE_FP32) return lancius_hip_upload(prog->ctx, prog->ptr[n->id], host, e * 4);
    if (host_dtype != LANCIUS_DTYPE_FP64) return LANCIUS_HIP_ERR_DTYPE;
    float* tmp = (float*)malloc(e * sizeof(float) + 1);
    if (!tmp) return LANCIUS_HIP_ERR_OOM;
    const double* src = (const double*)host;
    for (size_t k = 0; k < e; k++) tmp[k] = (float)src[k];
    const int rc = lancius_hip_upload(prog->ctx, prog->ptr[n->id], tmp, e * 4);
    free(tmp);
    return rc;
}

int lancius_device_upload_weights(lancius_device_program* prog, const char* path, const lancius_weight_map* map) {
    if (!prog || !path || !map || (map->count && !map->refs)) return LANCIUS_HIP_ERR_NULL_PTR;
    lancius_hip_file_tensor* t = (lancius_hip_file_tensor*)calloc(map->count + 1, sizeof(*t));
    if (!t) return LANCIUS_HIP_ERR_OOM;
    int rc = 0;
    for (uint32_t i = 0; i < map->count && !rc; i++) {
        const lancius_weight_ref* r = &map->refs[i];
        const lancius_node* n = r->node;
        if (!n || n->id >= prog->n_ids || prog->role[n->id] != ROLE_INPUT || !prog->ptr[n->id]) {
            rc = fail(LANCIUS_HIP_ERR_UNSUPPORTED, "weight map entry is not an INPUT of this program");
        } else if (r->elements != elems(n)) {
            rc = fail(LANCIUS_HIP_ERR_SHAPE, "weight map entry size differs from its node");
        } else if (r->file_dtype != LANCIUS_DTYPE_FP64 && r->file_dtype != LANCIUS_DTYPE_FP32 &&
                   r->file_dtype != LANCIUS_DTYPE_INT8) {
            rc = fail(LANCIUS_HIP_ERR_DTYPE, "weight map entry dtype");
        } else if (prog->is_i8[n->id] && r->file_dtype != LANCIUS_DTYPE_INT8) {
            rc = fail(LANCIUS_HIP_ERR_DTYPE, "int8 weight stored as floating point");
        } else {
            t[i].dst = prog->ptr[n->id];
            if (prog->packed[n->id] && prog->packed_stale[n->id] != PACK_EXPOSED)
                prog->packed_stale[n->id] = PACK_STALE;
            t[i].dst_dtype = prog->is_i8[n->id] ? LANCIUS_HIP_FILE_I8 : LANCIUS_HIP_FILE_F32;
            t[i].file_dtype = r->file_dtype == LANCIUS_DTYPE_INT8   ? LANCIUS_HIP_FILE_I8
                              : r->file_dtype == LANCIUS_DTYPE_FP32 ? LANCIUS_HIP_FILE_F32
                                                                    : LANCIUS_HIP_FILE_F64;
            t[i].file_offset = r->file_offset;
            t[i].elements = r->elements;
            t[i].scale = r->scale;
        }
    }
    if (!rc) rc = lancius_hip_upload_file(prog->ctx, path, map->count, t);
    free(t);
    return rc;
}

int lancius_device_download(lancius_device_program* prog, const lancius_node* n, void* host,
                            lancius_dtype host_dtype) {
    if (!prog || !n || !host) return LANCIUS_HIP_ERR_NULL_PTR;
    if (n->id >= prog->n_ids || !prog->readable[n->id] || !prog->ptr[n->id]) return LANCIUS_HIP_ERR_UNSUPPORTED;
    const size_t e = elems(n);
    if (prog->is_i8[n->id])
        return host_dtype == LANCIUS_DTYPE_INT8 ? lancius_hip_download(prog->ctx, host, prog->ptr[n->id], e)
                                                : LANCIUS_HIP_ERR_DTYPE;
    if (host_dtype == LANCIUS_DTYPE_FP32) return lancius_hip_download(prog->ctx, host, prog->ptr[n->id], e * 4);
    if (host_dtype != LANCIUS_DTYPE_FP64) return LANCIUS_HIP_ERR_DTYPE;
    float* tmp = (float*)malloc(e * sizeof(float) + 1);
    if (!tmp) return LANCIUS_HIP_ERR_OOM;
    int rc = lancius_hip_download(prog->ctx, tmp, prog->ptr[n->id], e * 4);
    if (!rc) {
        double* dst = (double*)host;
        for (size_t k = 0; k < e; k++) dst[k] = (double)tmp[k];
    }
    free(tmp);
    return rc;
}

int lancius_device_download_argmax(lancius_device_program* prog, const lancius_node* n, int32_t* host) {
    if (!prog || !n || !host) return LANCIUS_HIP_ERR_NULL_PTR;
    if (n->id >= prog->n_ids || !prog->argmax[n->id]) return LANCIUS_HIP_ERR_UNSUPPORTED;
    return lancius_hip_download(prog->ctx, host, prog->argmax[n->id], prog->rows[n->id] * sizeof(int32_t));
}

int lancius_schedule_execute_device(lancius_schedule* schedule, lancius_graph* g, lancius_hip_ctx* ctx) {
    if (!schedule || !g || !ctx) return LANCIUS_HIP_ERR_NULL_PTR;
    lancius_device_program* prog = NULL;
    int rc = lancius_device_program_create(ctx, g, schedule, schedule->plan, 0, &prog);
    if (rc) return rc;
    for (uint32_t i = 0; i < g->node_count && !rc; i++) {
        lancius_node* n = g->nodes[i];
        if (n->op == LANCIUS_OP_INPUT) {
            if (prog->is_i8[n->id])
                rc = n->runtime_data_int8 ? lancius_device_upload(prog, n, n->runtime_data_int8, LANCIUS_DTYPE_INT8)
                                          : fail(LANCIUS_HIP_ERR_NULL_PTR, "int8 INPUT node without runtime_data_int8");
            else if (!n->runtime_data) rc = fail(LANCIUS_HIP_ERR_NULL_PTR, "INPUT node without runtime_data");
            else rc = lancius_device_upload(prog, n, n->runtime_data, LANCIUS_DTYPE_FP64);
        }
    }
    if (!rc) rc = lancius_device_run(prog);
    if (!rc) rc = lancius_hip_synchronize(ctx);
    for (uint32_t i = 0; i < g->node_count && !rc; i++) {
        lancius_node* n = g->nodes[i];
        if (n->op == LANCIUS_OP_INPUT || n->op == LANCIUS_OP_CONST || !prog->readable[n->id]) continue;
        if (!n->runtime_data) {
            n->runtime_data = (double*)malloc(elems(n) * sizeof(double) + 1);
            if (!n->runtime_data) {
                rc = LANCIUS_HIP_ERR_OOM;
                break;
            }
            if (n->rt) {
                n->rt->buffer = n->runtime_data;
                n->rt->owner = LANCIUS_MEMORY_OWNED_HEAP;
                n->rt->buffer_owner = LANCIUS_MEMORY_OWNED_HEAP;
            }
        }
        rc = lancius_device_download(prog, n, n->runtime_data, LANCIUS_DTYPE_FP64);
    }
    lancius_device_program_destroy(prog);
    return rc;
}
