/*
 * Wave scheduler, linear-scan memory planner and Conv2D+ReLU fusion of the
 * host library.
 */
#include <stdbool.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "lancius_graph.h"

/* ---- scheduler ----------------------------------------------------------------
 * Levelization as in bleeding/v11A1/src/runtime/lancius_scheduler.c:12-59: a
 * wave holds every not-yet-scheduled node whose inputs are all scheduled, in
 * g->nodes order; nodes without inputs form wave 0.  A graph with a cycle
 * stops with the waves found so far and a FATAL line on stderr (:33-36). */

lancius_schedule* lancius_ir_schedule(lancius_graph* g) {
    if (!g || g->node_count == 0) return NULL;
    const uint32_t n = g->node_count;
    lancius_schedule* s = (lancius_schedule*)calloc(1, sizeof(lancius_schedule));
    uint8_t* done = (uint8_t*)calloc(g->next_id ? g->next_id : 1, 1);
    uint32_t* ready = (uint32_t*)malloc(sizeof(uint32_t) * n);
    uint32_t cap = 16;
    if (s) s->waves = (lancius_wave*)malloc(sizeof(lancius_wave) * cap);
    if (!s || !done || !ready || !s->waves) {
        if (s) free(s->waves);
        free(s);
        free(done);
        free(ready);
        lancius_set_error(LANCIUS_ERROR_OOM);
        return NULL;
    }
    uint32_t scheduled = 0;
    while (scheduled < n) {
        uint32_t cnt = 0;
        for (uint32_t i = 0; i < n; i++) {
            const lancius_node* nd = g->nodes[i];
            if (done[nd->id]) continue;
            bool ok = true;
            for (uint32_t j = 0; j < nd->input_count; j++) {
                const lancius_node* in = nd->inputs[j];
                if (in && !done[in->id]) {
                    ok = false;
                    break;
                }
            }
            if (ok) ready[cnt++] = i;
        }
        if (cnt == 0) {
            fprintf(stderr, "[SCHEDULER FATAL] Cycle or disconnect! Processed %u / %u\n", scheduled, n);
            break;
        }
        if (s->wave_count == cap) {
            cap *= 2;
            lancius_wave* grown = (lancius_wave*)realloc(s->waves, sizeof(lancius_wave) * cap);
            if (!grown) break;
            s->waves = grown;
        }
        lancius_wave* w = &s->waves[s->wave_count++];
        w->node_count = cnt;
        w->nodes = (lancius_node**)malloc(sizeof(lancius_node*) * cnt);
        for (uint32_t k = 0; k < cnt; k++) {
            w->nodes[k] = g->nodes[ready[k]];
            done[g->nodes[ready[k]]->id] = 1;
        }
        scheduled += cnt;
    }
    free(done);
    free(ready);
    return s;
}

void lancius_schedule_destroy(lancius_schedule* s) {
    if (!s) return;
    for (uint32_t w = 0; w < s->wave_count; w++) free(s->waves[w].nodes);
    free(s->waves);
    free(s);
}

void lancius_schedule_attach_pool(lancius_schedule* s, void* flat_buffer, struct lancius_memory_plan* plan) {
    if (!s) return;
    s->static_pool = flat_buffer;
    s->plan = plan;
}

/* lancius_scheduler.c:428-443: the largest per-wave sum of non-INPUT/CONST
 * node bytes. */
size_t lancius_schedule_peak_memory(lancius_schedule* s) {
    if (!s) return 0;
    size_t peak = 0;
    for (uint32_t w = 0; w < s->wave_count; w++) {
        size_t sum = 0;
        for (uint32_t i = 0; i < s->waves[w].node_count; i++) {
            const lancius_node* nd = s->waves[w].nodes[i];
            if (nd->op != LANCIUS_OP_INPUT && nd->op != LANCIUS_OP_CONST) sum += lancius_node_bytes(nd);
        }
        if (sum > peak) peak = sum;
    }
    return peak;
}

/* ---- memory planner ------------------------------------------------------------
 * bleeding/v11A1/src/runtime/lancius_memory_planner.c:33-182:
 *  1. every node that is not INPUT/CONST is born in its wave; an input dies in
 *     the last wave that reads it;
 *  2. a node nobody reads (a sink) lives to the end (death = wave_count);
 *  3. intervals in g->nodes order, stably sorted by birth wave;
 *  4. linear scan: before each allocation, intervals that died in an earlier
 *     wave return their block to the FRONT of a free list (LIFO, no
 *     coalescing); the first block large enough is used and split from its
 *     front.  Block sizes are node bytes rounded up to 32.
 * The offset of each allocation is kept with its interval, so the blocks that
 * return to the free list are the ones the tensors occupied. */

typedef struct {
    uint32_t id, birth, death;
    size_t size, offset;
} interval_t;

typedef struct free_blk {
    size_t offset, size;
    struct free_blk* next;
} free_blk;

static size_t round32(size_t x) { return (x + 31) & ~(size_t)31; }

lancius_memory_plan* lancius_build_memory_plan(lancius_schedule* sched, lancius_graph* g) {
    if (!sched || !g || sched->wave_count == 0) return NULL;
    const uint32_t ids = g->next_id;
    uint32_t* birth = (uint32_t*)malloc(sizeof(uint32_t) * ids);
    uint32_t* death = (uint32_t*)calloc(ids, sizeof(uint32_t));
    uint8_t* read = (uint8_t*)calloc(ids, 1);
    interval_t* iv = (interval_t*)calloc(g->node_count ? g->node_count : 1, sizeof(interval_t));
    interval_t* active = (interval_t*)calloc(g->node_count ? g->node_count : 1, sizeof(interval_t));
    lancius_memory_plan* plan = (lancius_memory_plan*)calloc(1, sizeof(lancius_memory_plan));
    if (plan) {
        plan->offsets = (size_t*)calloc(ids ? ids : 1, sizeof(size_t));
        plan->is_pooled = (uint8_t*)calloc(ids ? ids : 1, 1);
    }
    free_blk* fl = (free_blk*)malloc(sizeof(free_blk));
    if (!birth || !death || !read || !iv || !active || !plan || !plan->offsets || !plan->is_pooled || !fl) {
        free(birth);
        free(death);
        free(read);
        free(iv);
        free(active);
        free(fl);
        lancius_memory_plan_destroy(plan);
        lancius_set_error(LANCIUS_ERROR_OOM);
        return NULL;
    }
    for (uint32_t i = 0; i < ids; i++) birth[i] = UINT32_MAX;
    for (uint32_t i = 0; i < g->node_count; i++) {
        const lancius_node* nd = g->nodes[i];
        for (uint32_t j = 0; j < nd->input_count; j++)
            if (nd->inputs[j]) read[nd->inputs[j]->id] = 1;
    }
    for (uint32_t w = 0; w < sched->wave_count; w++) {
        for (uint32_t i = 0; i < sched->waves[w].node_count; i++) {
            const lancius_node* nd = sched->waves[w].nodes[i];
            if (nd->op != LANCIUS_OP_INPUT && nd->op != LANCIUS_OP_CONST) birth[nd->id] = w;
            for (uint32_t j = 0; j < nd->input_count; j++) {
                if (!nd->inputs[j]) continue;
                const uint32_t in = nd->inputs[j]->id;
                if (birth[in] != UINT32_MAX && w > death[in]) death[in] = w;
            }
        }
    }
    uint32_t count = 0;
    for (uint32_t i = 0; i < g->node_count; i++) {
        const lancius_node* nd = g->nodes[i];
        if (birth[nd->id] == UINT32_MAX) continue;
        interval_t* t = &iv[count++];
        t->id = nd->id;
        t->birth = birth[nd->id];
        t->death = death[nd->id] > t->birth ? death[nd->id] : t->birth;
        if (!read[nd->id]) t->death = sched->wave_count;
        t->size = round32(lancius_node_bytes(nd));
    }
    /* stable insertion sort by birth */
    for (uint32_t i = 1; i < count; i++) {
        interval_t key = iv[i];
        uint32_t j = i;
        while (j > 0 && iv[j - 1].birth > key.birth) {
            iv[j] = iv[j - 1];
            j--;
        }
        iv[j] = key;
    }

    fl->offset = 0;
    fl->size = SIZE_MAX;
    fl->next = NULL;
    size_t peak = 0;
    uint32_t nactive = 0;
    for (uint32_t i = 0; i < count; i++) {
        interval_t* cur = &iv[i];
        uint32_t keep = 0;
        for (uint32_t a = 0; a < nactive; a++) {
            if (active[a].death < cur->birth) {
                free_blk* fb = (free_blk*)malloc(sizeof(free_blk));
                if (!fb) continue; /* the block is lost to reuse; the plan stays valid */
                fb->offset = active[a].offset;
                fb->size = active[a].size;
                fb->next = fl;
                fl = fb;
            } else {
                active[keep++] = active[a];
            }
        }
        nactive = keep;
        free_blk* prev = NULL;
        free_blk* b = fl;
        while (b && b->size < cur->size) {
            prev = b;
            b = b->next;
        }
        if (b) {
            cur->offset = b->offset;
            if (b->size > cur->size) {
                b->offset += cur->size;
                b->size -= cur->size;
            } else {
                if (prev) prev->next = b->next;
                else fl = b->next;
                free(b);
            }
        } else {
            cur->offset = peak;
        }
        if (cur->offset + cur->size > peak) peak = cur->offset + cur->size;
        plan->offsets[cur->id] = cur->offset;
        plan->is_pooled[cur->id] = 1;
        active[nactive++] = *cur;
    }
    plan->peak_memory = peak;
    while (fl) {
        free_blk* n = fl->next;
        free(fl);
        fl = n;
    }
    free(birth);
    free(death);
    free(read);
    free(iv);
    free(active);
    return plan;
}

void lancius_memory_plan_destroy(lancius_memory_plan* plan) {
    if (!plan) return;
    free(plan->offsets);
    free(plan->is_pooled);
    free(plan);
}

/* ---- Conv2D + ReLU fusion ------------------------------------------------------
 * bleeding/v11A1/src/compiler/lancius_optimizer.c:15-41: walking the nodes
 * backwards, a RELU whose input is a CONV2D with exactly one consumer becomes
 * CONV2D_RELU_FUSED with the conv's inputs, geometry and shape; the conv turns
 * into a NOP with no inputs (it keeps its id and still receives a plan block). */

static int consumers(const lancius_graph* g, const lancius_node* target) {
    int c = 0;
    for (uint32_t i = 0; i < g->node_count; i++)
        for (uint32_t j = 0; j < g->nodes[i]->input_count; j++)
            if (g->nodes[i]->inputs[j] == target) c++;
    return c;
}

void lancius_optimize_fusion(lancius_graph* g) {
    if (!g) return;
    int fused = 0;
    for (int i = (int)g->node_count - 1; i >= 0; i--) {
        lancius_node* n = g->nodes[i];
        if (n->op != LANCIUS_OP_RELU || n->input_count == 0 || !n->inputs[0]) continue;
        lancius_node* conv = (lancius_node*)n->inputs[0];
        if (conv->op != LANCIUS_OP_CONV2D || consumers(g, conv) != 1) continue;
        n->op = LANCIUS_OP_CONV2D_RELU_FUSED;
        n->inputs = conv->inputs;
        n->input_count = 2;
        n->kernel_h = conv->kernel_h;
        n->kernel_w = conv->kernel_w;
        n->stride = conv->stride;
        n->pad = conv->pad;
        for (int d = 0; d < 4; d++) n->shape[d] = conv->shape[d];
        n->ndim = 4;
        conv->op = LANCIUS_OP_NOP;
        conv->input_count = 0;
        conv->inputs = NULL;
        fused++;
    }
    printf("[LANCIUS OPTIMIZER] Fused %d Conv2D+ReLU patterns.\n", fused);
}
