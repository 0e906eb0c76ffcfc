/*
 * drop_in.c - a reference program changed as INTEGRATION.md section 2
 * describes: graphs built with the reference's builders
 * (bleeding/v11A1/src/ir/lancius_ir.c), scheduled by its lancius_ir_schedule
 * (src/runtime/lancius_scheduler.c:12-59), planned in fp32 by its
 * lancius_build_memory_plan (src/runtime/lancius_memory_planner.c:33-182)
 * and attached with lancius_schedule_attach_pool (:416-420), then executed by
 * lancius_schedule_execute_device instead of lancius_schedule_execute (:311).
 *
 * Each graph is built twice with the same seeded inputs: once run by the
 * reference's CPU executor with a scratch arena, once by the device.  Every
 * sink must agree to max|y - y_ref| / max|y_ref| <= 1e-4 * max(1, sqrt(K)/32),
 * K the longest reduction.  Prints "ok <graph> ..." per graph; exit 0 only
 * when all agree.
 *
 * Test infrastructure: compiled by oracle/Makefile against the reference
 * headers, linked with oracle/_ref/liblancius_ref.so and
 * lancius_amd/liblancius_hip.so.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <lancius.h>                       /* reference headers, unchanged */
#include "lancius/lancius_memory_planner.h"
#include "lancius_hip_graph.h"             /* after the reference headers */

#define MAXN 64

typedef struct {
    lancius_graph* g;
    lancius_node* in[MAXN];
    double mean[MAXN], std[MAXN]; /* of each INPUT's seeded values */
    int n_in;
    lancius_node* out[8];
    int n_out;
} built;

/* SplitMix64 -> uniform (0,1) -> Box-Muller normal, widened from fp32 so the
 * device (which stores fp32) and the CPU see identical values. */
static uint64_t sm_state;
static uint64_t splitmix64(void) {
    uint64_t z = (sm_state += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
static double uniform01(void) { return ((double)(splitmix64() >> 11) + 0.5) / 9007199254740992.0; }
static double normal01(void) {
    const double u = uniform01(), v = uniform01();
    return sqrt(-2.0 * log(u)) * cos(6.283185307179586 * v);
}

static lancius_node* add_input(built* b, lancius_node* n, double mean, double std) {
    b->in[b->n_in] = n;
    b->mean[b->n_in] = mean;
    b->std[b->n_in] = std;
    b->n_in++;
    return n;
}

static lancius_node* inp(built* b, size_t r, size_t c, double mean, double std) {
    return add_input(b, lancius_input(b->g, r, c), mean, std);
}

static lancius_node* linear(lancius_graph* g, lancius_node* x, lancius_node* w, lancius_node* bias, size_t rows,
                            size_t cols) {
    return lancius_add(g, lancius_matmul(g, x, w), lancius_broadcast(g, bias, rows, cols));
}

/* BASELINE configs[0]: 64x784 -> 256 (ReLU) -> 10, softmax. */
static void build_mlp(built* b) {
    memset(b, 0, sizeof(*b));
    b->g = lancius_graph_create();
    lancius_node *x = inp(b, 64, 784, 0, 1), *w1 = inp(b, 784, 256, 0, 0.02), *b1 = inp(b, 1, 256, 0, 0.02),
                 *w2 = inp(b, 256, 10, 0, 0.02), *b2 = inp(b, 1, 10, 0, 0.02);
    lancius_node* h = lancius_relu(b->g, linear(b->g, x, w1, b1, 64, 256));
    b->out[b->n_out++] = lancius_softmax(b->g, linear(b->g, h, w2, b2, 64, 10));
}

/* conv 3x3 stride 1 pad 1 -> RELU, fused by the reference's pass. */
static void build_conv(built* b) {
    memset(b, 0, sizeof(*b));
    b->g = lancius_graph_create();
    lancius_node* x = add_input(b, lancius_input_4d(b->g, 2, 3, 8, 8), 0, 1);
    lancius_node* w = add_input(b, lancius_input_4d(b->g, 4, 3, 3, 3), 0, sqrt(2.0 / 27.0)); /* He */
    b->out[b->n_out++] = lancius_relu(b->g, lancius_conv2d(b->g, x, w, 1, 1));
    lancius_optimize_fusion(b->g);
}

/* Pre-norm transformer block, two sequences sharing the weights (the
 * BASELINE configs[4] recipe at S=32, d=64, H=4, F=256). */
static void build_block(built* b) {
    enum { S = 32, d = 64, H = 4, F = 256, D = d / H, BATCH = 2 };
    memset(b, 0, sizeof(*b));
    b->g = lancius_graph_create();
    lancius_graph* g = b->g;
    const double p = 0.02; /* weights and biases ~ N(0, 0.02), LayerNorm gains ~ 1 + N(0, 0.02) */
    lancius_node *g1 = inp(b, 1, d, 1, p), *be1 = inp(b, 1, d, 0, p), *wq = inp(b, d, d, 0, p),
                 *bq = inp(b, 1, d, 0, p), *wk = inp(b, d, d, 0, p), *bk = inp(b, 1, d, 0, p), *wv = inp(b, d, d, 0, p),
                 *bv = inp(b, 1, d, 0, p), *wo = inp(b, d, d, 0, p), *bo = inp(b, 1, d, 0, p), *g2 = inp(b, 1, d, 1, p),
                 *be2 = inp(b, 1, d, 0, p), *w1 = inp(b, d, F, 0, p), *bf1 = inp(b, 1, F, 0, p),
                 *w2 = inp(b, F, d, 0, p), *bf2 = inp(b, 1, d, 0, p);
    for (int s = 0; s < BATCH; s++) {
        lancius_node* x = inp(b, S, d, 0, 1);
        lancius_node* ln1 = lancius_layernorm(g, x, g1, be1);
        lancius_node* q = lancius_reshape(g, linear(g, ln1, wq, bq, S, d), 3, S, H, D, 0);
        lancius_node* k = lancius_reshape(g, linear(g, ln1, wk, bk, S, d), 3, S, H, D, 0);
        lancius_node* v = lancius_reshape(g, linear(g, ln1, wv, bv, S, d), 3, S, H, D, 0);
        lancius_node* att = lancius_reshape(g, lancius_attention(g, q, k, v), 2, S, d, 0, 0);
        lancius_node* x1 = lancius_add(g, linear(g, att, wo, bo, S, d), x);
        lancius_node* ln2 = lancius_layernorm(g, x1, g2, be2);
        lancius_node* f1 = lancius_gelu(g, linear(g, ln2, w1, bf1, S, F));
        b->out[b->n_out++] = lancius_add(g, linear(g, f1, w2, bf2, S, d), x1);
    }
}

/* Seeded values of every INPUT, mean + std * N(0,1) rounded to fp32 (the
 * device stores fp32; both runs see the same numbers). */
static double** make_inputs(const built* b, uint64_t seed) {
    double** v = (double**)calloc((size_t)b->n_in, sizeof(double*));
    sm_state = seed;
    for (int i = 0; i < b->n_in; i++) {
        const size_t e = lancius_node_elements(b->in[i]);
        v[i] = (double*)malloc(e * sizeof(double));
        for (size_t k = 0; k < e; k++) v[i][k] = (double)(float)(b->mean[i] + b->std[i] * normal01());
    }
    return v;
}

static int compare(const char* name, const built* cpu, const built* dev, size_t K) {
    const double tol = 1e-4 * (sqrt((double)K) / 32.0 > 1.0 ? sqrt((double)K) / 32.0 : 1.0);
    double worst = 0.0;
    for (int o = 0; o < cpu->n_out; o++) {
        const lancius_node* a = cpu->out[o];
        const lancius_node* b = dev->out[o];
        if (!a->runtime_data || !b->runtime_data) {
            printf("FAIL %s: sink %d has no runtime_data\n", name, o);
            return 1;
        }
        double num = 0.0, den = 0.0;
        const size_t e = lancius_node_elements(a);
        for (size_t k = 0; k < e; k++) {
            const double diff = fabs(b->runtime_data[k] - a->runtime_data[k]);
            if (!(diff <= num)) num = diff; /* NaN propagates as a failure */
            if (fabs(a->runtime_data[k]) > den) den = fabs(a->runtime_data[k]);
        }
        const double err = den > 0.0 ? num / den : num;
        if (!(err <= worst)) worst = err;
    }
    if (!(worst <= tol)) {
        printf("FAIL %s: normwise error %.3e > %.1e\n", name, worst, tol);
        return 1;
    }
    printf("ok %s: %d sink(s), normwise error %.3e (tol %.1e)\n", name, cpu->n_out, worst, tol);
    return 0;
}

static int run_one(const char* name, void (*build)(built*), uint64_t seed, size_t K, lancius_hip_ctx* ctx) {
    built cpu, dev;
    build(&cpu);
    build(&dev);
    double** vin = make_inputs(&cpu, seed);
    for (int i = 0; i < cpu.n_in; i++) {
        cpu.in[i]->runtime_data = vin[i];
        dev.in[i]->runtime_data = vin[i];
    }
    /* the reference CPU path */
    lancius_schedule* s_cpu = lancius_ir_schedule(cpu.g);
    lancius_arena* scratch = lancius_arena_create(64u << 20);
    lancius_schedule_execute(s_cpu, scratch);

    /* the device path, exactly as INTEGRATION.md section 2 */
    lancius_schedule* s = lancius_ir_schedule(dev.g);
    for (uint32_t i = 0; i < dev.g->node_count; i++) dev.g->nodes[i]->dtype = LANCIUS_DTYPE_FP32;
    lancius_memory_plan* plan = lancius_build_memory_plan(s, dev.g);
    for (uint32_t i = 0; i < dev.g->node_count; i++) dev.g->nodes[i]->dtype = LANCIUS_DTYPE_FP64;
    lancius_schedule_attach_pool(s, NULL, plan);
    const int rc = lancius_schedule_execute_device(s, dev.g, ctx);
    int bad = 0;
    if (rc != 0) {
        printf("FAIL %s: lancius_schedule_execute_device returned %d (%s)\n", name, rc, lancius_hip_last_error());
        bad = 1;
    } else {
        bad = compare(name, &cpu, &dev, K);
    }
    for (int o = 0; o < dev.n_out; o++) { /* sinks the device executor malloc'd */
        free(dev.out[o]->runtime_data);
        dev.out[o]->runtime_data = NULL;
    }
    for (int i = 0; i < cpu.n_in; i++) {
        cpu.in[i]->runtime_data = NULL;
        dev.in[i]->runtime_data = NULL;
        free(vin[i]);
    }
    free(vin);
    lancius_schedule_attach_pool(s, NULL, NULL);
    lancius_memory_plan_destroy(plan);
    lancius_schedule_destroy(s);
    lancius_schedule_destroy(s_cpu);
    lancius_arena_destroy(scratch);
    lancius_graph_destroy(dev.g);
    lancius_graph_destroy(cpu.g);
    return bad;
}

int main(void) {
    lancius_hip_ctx* ctx = NULL;
    if (lancius_hip_ctx_create(0, NULL, &ctx) != 0) {
        printf("FAIL: lancius_hip_ctx_create: %s\n", lancius_hip_last_error());
        return 2;
    }
    int bad = 0;
    bad |= run_one("mlp", build_mlp, 42, 784, ctx);
    bad |= run_one("conv", build_conv, 43, 27, ctx);
    bad |= run_one("block", build_block, 44, 256, ctx);
    lancius_hip_ctx_destroy(ctx);
    return bad;
}
