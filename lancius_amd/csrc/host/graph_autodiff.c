/*
 * Reverse-mode autodiff over the graph IR: the training graph of a forward
 * graph and a scalar loss node.
 *
 * The construction follows bleeding/v11A1/src/math/lancius_autodiff.c:44-207
 * step for step, because a training graph is only interchangeable with the
 * reference's (same node ids, same waves, same planner input) when the same
 * builders run in the same order:
 *   1. the forward nodes are re-created in order in a new graph (INPUT nodes
 *      keep their bound data; NOP nodes are dropped; a fused Conv+ReLU keeps
 *      its opcode);
 *   2. the loss gets the seed gradient CONST 1.0 [1,1];
 *   3. the forward nodes are visited in reverse and each pushes the
 *      vector-Jacobian product of its op to its inputs; a gradient whose
 *      shape differs from its target is reduced or broadcast to it, and
 *      several gradients of one node are summed with ADD nodes.
 */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "lancius_graph.h"

typedef struct {
    lancius_graph* g;       /* the training graph */
    lancius_node** full;    /* forward id -> its copy in g */
    lancius_node** grad;    /* forward id -> accumulated gradient node */
} ad_state;

static int same_shape(const lancius_node* a, const lancius_node* b) {
    if (a->ndim != b->ndim) return 0;
    for (uint8_t d = 0; d < a->ndim; d++)
        if (a->shape[d] != b->shape[d]) return 0;
    return 1;
}

static int is_scalar2(const lancius_node* n) { return n->shape[0] == 1 && n->shape[1] == 1; }

/* Adds gradient `dg` to forward node `id` (lancius_autodiff.c:7-42): equal
 * shapes add directly; a 2-D mismatch is first reconciled by BROADCAST of a
 * scalar, SUM to a scalar, SUM_AXIS0 to a row or SUM_AXIS1 to a column. */
static void push_grad(ad_state* s, uint32_t id, lancius_node* dg) {
    if (!dg) return;
    const lancius_node* target = s->full[id];
    if (!target) return;
    if (!same_shape(dg, target) && dg->ndim == 2 && target->ndim == 2) {
        if (is_scalar2(dg) && !is_scalar2(target))
            dg = lancius_broadcast(s->g, dg, target->shape[0], target->shape[1]);
        else if (!is_scalar2(dg) && is_scalar2(target))
            dg = lancius_sum(s->g, dg);
        else if (dg->shape[0] > 1 && dg->shape[1] == target->shape[1] && target->shape[0] == 1)
            dg = lancius_sum_axis0(s->g, dg);
        else if (dg->shape[1] > 1 && dg->shape[0] == target->shape[0] && target->shape[1] == 1)
            dg = lancius_sum_axis1(s->g, dg);
    }
    s->grad[id] = s->grad[id] ? lancius_add(s->g, s->grad[id], dg) : dg;
}

/* The fused Conv+ReLU node is re-created with its own opcode (the builders
 * only make CONV2D), same shape and attributes (lancius_autodiff.c:78-101). */
static lancius_node* copy_fused_conv(lancius_graph* g, const lancius_node* old, const lancius_node* x,
                                     const lancius_node* w) {
    if (!x || !w) return NULL;
    lancius_node* n = lancius_conv2d(g, x, w, old->stride, old->pad);
    if (!n) return NULL;
    n->op = LANCIUS_OP_CONV2D_RELU_FUSED;
    for (int d = 0; d < 4; d++) n->shape[d] = old->shape[d];
    n->kernel_h = old->kernel_h;
    n->kernel_w = old->kernel_w;
    n->runtime_data = old->runtime_data;
    if (n->rt) n->rt->buffer = old->runtime_data;
    return n;
}

/* Step 1 for one node (lancius_autodiff.c:53-104). */
static lancius_node* copy_forward(ad_state* s, const lancius_node* old) {
    const lancius_node* a = old->input_count > 0 && old->inputs[0] ? s->full[old->inputs[0]->id] : NULL;
    const lancius_node* b = old->input_count > 1 && old->inputs[1] ? s->full[old->inputs[1]->id] : NULL;
    lancius_graph* g = s->g;
    lancius_node* n = NULL;
    switch (old->op) {
        case LANCIUS_OP_INPUT:
            n = old->ndim == 4 ? lancius_input_4d(g, old->shape[0], old->shape[1], old->shape[2], old->shape[3])
                               : lancius_input(g, old->shape[0], old->shape[1]);
            if (n) {
                n->runtime_data = old->runtime_data;
                if (n->rt) n->rt->buffer = old->runtime_data;
            }
            return n;
        case LANCIUS_OP_CONST: return lancius_const(g, old->attr_val, old->shape[0], old->shape[1]);
        case LANCIUS_OP_ADD: return lancius_add(g, a, b);
        case LANCIUS_OP_SUB: return lancius_sub(g, a, b);
        case LANCIUS_OP_MUL: return lancius_mul(g, a, b);
        case LANCIUS_OP_MATMUL: return lancius_matmul(g, a, b);
        case LANCIUS_OP_RELU: return lancius_relu(g, a);
        case LANCIUS_OP_TRANSPOSE: return lancius_transpose(g, a);
        case LANCIUS_OP_SUM: return lancius_sum(g, a);
        case LANCIUS_OP_BROADCAST: return lancius_broadcast(g, a, old->shape[0], old->shape[1]);
        case LANCIUS_OP_SOFTMAX: return lancius_softmax(g, a);
        case LANCIUS_OP_CROSS_ENTROPY: return lancius_cross_entropy(g, a, b);
        case LANCIUS_OP_PERMUTE:
            return lancius_permute(g, a, old->axes[0], old->axes[1], old->axes[2], old->axes[3]);
        case LANCIUS_OP_MATMUL_BATCHED: return lancius_matmul_batched(g, a, b);
        case LANCIUS_OP_CONV2D: return lancius_conv2d(g, a, b, old->stride, old->pad);
        case LANCIUS_OP_MAXPOOL2D: return lancius_maxpool2d(g, a, old->kernel_h, old->stride);
        case LANCIUS_OP_FLATTEN: return lancius_flatten(g, a);
        case LANCIUS_OP_RESHAPE:
            return lancius_reshape(g, a, old->ndim, old->shape[0], old->shape[1], old->shape[2], old->shape[3]);
        case LANCIUS_OP_NOP: return NULL;
        case LANCIUS_OP_CONV2D_RELU_FUSED: return copy_fused_conv(g, old, a, b);
        default:
            fprintf(stderr, "[LANCIUS AUTODIFF] op %d has no gradient rule\n", (int)old->op);
            return NULL;
    }
}

/* Step 3 for one node (lancius_autodiff.c:113-197).  Returns -1 for an op
 * whose backward pass the reference refuses (RMSNORM, SWIGLU, GQA). */
static int backward(ad_state* s, const lancius_node* f, lancius_node* dy) {
    lancius_graph* g = s->g;
    const uint32_t i0 = f->input_count > 0 ? f->inputs[0]->id : 0;
    const uint32_t i1 = f->input_count > 1 ? f->inputs[1]->id : 0;
    lancius_node* A = f->input_count > 0 ? s->full[i0] : NULL;
    lancius_node* B = f->input_count > 1 ? s->full[i1] : NULL;
    switch (f->op) {
        case LANCIUS_OP_ADD:
            push_grad(s, i0, dy);
            push_grad(s, i1, dy);
            break;
        case LANCIUS_OP_SUB: {
            push_grad(s, i0, dy);
            lancius_node* neg = lancius_const(g, -1.0, dy->shape[0], dy->shape[1]);
            push_grad(s, i1, lancius_mul(g, dy, neg));
            break;
        }
        case LANCIUS_OP_MUL: {
            /* a scalar upstream gradient is broadcast to each operand first */
            lancius_node* dA = dy;
            lancius_node* dB = dy;
            if (dA->ndim == 2 && is_scalar2(dA) && A && (A->shape[0] > 1 || A->shape[1] > 1))
                dA = lancius_broadcast(g, dA, A->shape[0], A->shape[1]);
            if (dB->ndim == 2 && is_scalar2(dB) && B && (B->shape[0] > 1 || B->shape[1] > 1))
                dB = lancius_broadcast(g, dB, B->shape[0], B->shape[1]);
            push_grad(s, i0, lancius_mul(g, dA, B));
            push_grad(s, i1, lancius_mul(g, dB, A));
            break;
        }
        case LANCIUS_OP_RMSNORM:
        case LANCIUS_OP_SWIGLU:
        case LANCIUS_OP_GQA:
            fprintf(stderr, "[LANCIUS AUTODIFF] no backward pass for op %d\n", (int)f->op);
            return -1;
        case LANCIUS_OP_MATMUL: {
            /* dA = dY . B^T, dB = A^T . dY */
            lancius_node* bt = lancius_transpose(g, B);
            push_grad(s, i0, lancius_matmul(g, dy, bt));
            lancius_node* at = lancius_transpose(g, A);
            push_grad(s, i1, lancius_matmul(g, at, dy));
            break;
        }
        case LANCIUS_OP_RELU: push_grad(s, i0, lancius_relu_bwd(g, dy, A)); break;
        case LANCIUS_OP_SUM:
            if (A && A->ndim == 4 && dy->ndim == 2 && is_scalar2(dy))
                push_grad(s, i0, lancius_broadcast_4d(g, dy, A->shape[0], A->shape[1], A->shape[2], A->shape[3]));
            else
                push_grad(s, i0, dy);
            break;
        case LANCIUS_OP_BROADCAST: push_grad(s, i0, dy); break;
        case LANCIUS_OP_TRANSPOSE: push_grad(s, i0, lancius_transpose(g, dy)); break;
        case LANCIUS_OP_MATMUL_BATCHED:
            push_grad(s, i0, dy);
            push_grad(s, i1, dy);
            break;
        case LANCIUS_OP_PERMUTE: {
            uint32_t inv[4] = {0, 0, 0, 0};
            for (uint32_t d = 0; d < 4; d++) inv[f->axes[d] & 3u] = d;
            push_grad(s, i0, lancius_permute(g, dy, inv[0], inv[1], inv[2], inv[3]));
            break;
        }
        case LANCIUS_OP_CROSS_ENTROPY: push_grad(s, i0, lancius_cross_entropy_bwd(g, A, B, dy)); break;
        case LANCIUS_OP_SOFTMAX: push_grad(s, i0, lancius_softmax_bwd(g, dy, s->full[f->id])); break;
        case LANCIUS_OP_FLATTEN:
            if (A) push_grad(s, i0, lancius_reshape(g, dy, A->ndim, A->shape[0], A->shape[1], A->shape[2], A->shape[3]));
            break;
        case LANCIUS_OP_MAXPOOL2D: push_grad(s, i0, lancius_maxpool2d_bwd(g, dy, A, f->kernel_h, f->stride)); break;
        case LANCIUS_OP_CONV2D:
        case LANCIUS_OP_CONV2D_RELU_FUSED: {
            lancius_node* d = dy;
            if (f->op == LANCIUS_OP_CONV2D_RELU_FUSED) d = lancius_relu_bwd(g, dy, s->full[f->id]);
            push_grad(s, i0, lancius_conv2d_bwd(g, d, A, B, f->stride, f->pad));
            push_grad(s, i1, lancius_conv2d_bwd_w(g, d, A, f->kernel_h, f->kernel_w, f->stride, f->pad));
            break;
        }
        default: break; /* no rule: the gradient stops here, as in the reference */
    }
    return 0;
}

lancius_training_graph* lancius_ir_autodiff(lancius_graph* fwd_g, lancius_node* loss_node) {
    if (!fwd_g || !loss_node) {
        lancius_set_error(LANCIUS_ERROR_NULL_PTR);
        return NULL;
    }
    const uint32_t ids = fwd_g->next_id;
    lancius_training_graph* tg = (lancius_training_graph*)calloc(1, sizeof(*tg));
    ad_state s;
    s.g = lancius_graph_create();
    s.full = (lancius_node**)calloc(ids ? ids : 1, sizeof(lancius_node*));
    s.grad = (lancius_node**)calloc(ids ? ids : 1, sizeof(lancius_node*));
    lancius_node** out_grads = (lancius_node**)calloc(ids ? ids : 1, sizeof(lancius_node*));
    if (!tg || !s.g || !s.full || !s.grad || !out_grads) {
        lancius_set_error(LANCIUS_ERROR_OOM);
        goto fail;
    }
    for (uint32_t i = 0; i < fwd_g->node_count; i++) {
        const lancius_node* old = fwd_g->nodes[i];
        s.full[old->id] = copy_forward(&s, old);
    }
    s.grad[loss_node->id] = lancius_const(s.g, 1.0, 1, 1);
    for (int64_t i = (int64_t)fwd_g->node_count - 1; i >= 0; i--) {
        const lancius_node* f = fwd_g->nodes[i];
        lancius_node* dy = s.grad[f->id];
        if (!dy || f->op == LANCIUS_OP_INPUT || f->op == LANCIUS_OP_CONST || f->op == LANCIUS_OP_NOP) continue;
        if (backward(&s, f, dy)) goto fail;
    }
    memcpy(out_grads, s.grad, sizeof(lancius_node*) * ids);
    tg->graph = s.g;
    tg->loss_node = s.full[loss_node->id];
    tg->grad_nodes = out_grads;
    tg->max_id = ids;
    free(s.full);
    free(s.grad);
    return tg;
fail:
    free(out_grads);
    free(s.full);
    free(s.grad);
    if (s.g) lancius_graph_destroy(s.g);
    free(tg);
    return NULL;
}

void lancius_training_graph_destroy(lancius_training_graph* tg) {
    if (!tg) return;
    free(tg->grad_nodes);
    lancius_graph_destroy(tg->graph);
    free(tg);
}
