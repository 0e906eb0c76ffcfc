/*
 * The BASIS static graph IR builders (reference
 * include/basis/stage6_ir/graph.h:7-39, src/basis/stage6_ir/graph.c:35-135):
 * same names, struct layouts and shape rules, so a program written against
 * the reference header builds the same node array.
 *
 * Nodes live in one array grown by doubling (16 first), so ids are stable and
 * a returned basis_node* is valid until the next builder call that adds a
 * node, as in the reference.  Unlike the reference, a NULL graph or operand,
 * or a failed allocation, returns NULL instead of dereferencing it.
 */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "lancius_basis.h"

static basis_node* push_node(basis_graph* g, basis_op_type op, size_t rows, size_t cols, const char* name) {
    if (!g) return NULL;
    if (g->node_count == g->node_cap) {
        const size_t cap = g->node_cap ? 2 * g->node_cap : 16;
        basis_node* grown = (basis_node*)realloc(g->nodes, cap * sizeof(basis_node));
        if (!grown) return NULL;
        g->nodes = grown;
        g->node_cap = cap;
    }
    char* copy = NULL;
    if (name) {
        const size_t len = strlen(name) + 1;
        copy = (char*)malloc(len);
        if (!copy) return NULL;
        memcpy(copy, name, len);
    }
    basis_node* n = &g->nodes[g->node_count];
    n->id = (int)g->node_count;
    n->op = op;
    n->input_ids[0] = n->input_ids[1] = -1;
    n->rows = rows;
    n->cols = cols;
    n->name = copy;
    g->node_count++;
    return n;
}

/* The operands may be pointers into g->nodes that the push moves: read
 * their ids and shapes before it. */
static basis_node* unary(basis_graph* g, basis_op_type op, const basis_node* a) {
    if (!a) return NULL;
    const int ia = a->id;
    basis_node* n = push_node(g, op, a->rows, a->cols, NULL);
    if (n) n->input_ids[0] = ia;
    return n;
}

static basis_node* binary(basis_graph* g, basis_op_type op, const basis_node* a, const basis_node* b, size_t rows,
                          size_t cols) {
    const int ia = a->id, ib = b->id;
    basis_node* n = push_node(g, op, rows, cols, NULL);
    if (n) {
        n->input_ids[0] = ia;
        n->input_ids[1] = ib;
    }
    return n;
}

basis_graph* basis_graph_new(void) { return (basis_graph*)calloc(1, sizeof(basis_graph)); }

basis_node* basis_graph_input(basis_graph* g, const char* name, size_t r, size_t c) {
    return push_node(g, BASIS_OP_INPUT, r, c, name);
}

/* a [m x k] . b [k x n] -> [m x n] (graph.c:39-48). */
basis_node* basis_graph_matmul(basis_graph* g, basis_node* a, basis_node* b) {
    if (!a || !b) return NULL;
    if (a->cols != b->rows) {
        fprintf(stderr, "[BASIS IR] matmul: [%zu x %zu] . [%zu x %zu] inner dimensions differ\n", a->rows, a->cols,
                b->rows, b->cols);
        return NULL;
    }
    return binary(g, BASIS_OP_MATMUL, a, b, a->rows, b->cols);
}

/* Same shapes (graph.c:50-59). */
basis_node* basis_graph_add(basis_graph* g, basis_node* a, basis_node* b) {
    if (!a || !b) return NULL;
    if (a->rows != b->rows || a->cols != b->cols) {
        fprintf(stderr, "[BASIS IR] add: [%zu x %zu] + [%zu x %zu] shapes differ\n", a->rows, a->cols, b->rows,
                b->cols);
        return NULL;
    }
    return binary(g, BASIS_OP_ADD, a, b, a->rows, a->cols);
}

/* bias must be [1 x a.cols] (graph.c:61-70). */
basis_node* basis_graph_broadcast_add(basis_graph* g, basis_node* a, basis_node* bias) {
    if (!a || !bias) return NULL;
    if (bias->rows != 1 || bias->cols != a->cols) {
        fprintf(stderr, "[BASIS IR] broadcast_add: bias [%zu x %zu] is not [1 x %zu]\n", bias->rows, bias->cols,
                a->cols);
        return NULL;
    }
    return binary(g, BASIS_OP_BROADCAST_ADD, a, bias, a->rows, a->cols);
}

basis_node* basis_graph_relu(basis_graph* g, basis_node* a) { return unary(g, BASIS_OP_RELU, a); }

basis_node* basis_graph_tanh(basis_graph* g, basis_node* a) { return unary(g, BASIS_OP_TANH, a); }

static const char* op_name(basis_op_type op) {
    switch (op) {
        case BASIS_OP_INPUT: return "INPUT";
        case BASIS_OP_MATMUL: return "MATMUL";
        case BASIS_OP_ADD: return "ADD";
        case BASIS_OP_BROADCAST_ADD: return "BROADCAST_ADD";
        case BASIS_OP_RELU: return "RELU";
        case BASIS_OP_TANH: return "TANH";
    }
    return "UNKNOWN";
}

/* One line per node in the reference's layout (graph.c:98-115), so tools
 * that read the dump see the same text. */
void basis_graph_print(basis_graph* g) {
    if (!g) return;
    printf("=== BASIS Static Graph IR ===\n");
    for (size_t i = 0; i < g->node_count; i++) {
        const basis_node* n = &g->nodes[i];
        printf("Node %2d | %-15s | Shape: [%3zu x %3zu] | Inputs: ", n->id, op_name(n->op), n->rows, n->cols);
        if (n->op == BASIS_OP_INPUT)
            printf("None (Name: \"%s\")", n->name ? n->name : "(null)");
        else
            printf("[%d, %d]", n->input_ids[0], n->input_ids[1]);
        printf("\n");
    }
    printf("=============================\n");
}

void basis_graph_free(basis_graph* g) {
    if (!g) return;
    for (size_t i = 0; i < g->node_count; i++) free(g->nodes[i].name);
    free(g->nodes);
    free(g);
}
