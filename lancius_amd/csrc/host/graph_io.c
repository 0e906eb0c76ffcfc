/*
 * graph_io.c - .lancius model files for the host graph library.
 *
 *   lancius_graph_load / lancius_graph_save .. bleeding/v11A1/src/core/lancius_serialize.c:13-259
 *   v9 record layout (no is_view byte) ....... stable/v9S/src/core/lancius_serialize.c
 *   v2 header, magic, flags, dtypes .......... bleeding/v11A1/include/lancius/lancius_model_format.h:7-92
 *
 * The file is memory-mapped and read through a bounds-checked cursor; every
 * count, id, rank, dtype and payload extent is checked before it is used, so
 * a malformed or truncated file fails the load instead of reading past the
 * mapping.  The layouts and the rules for telling them apart are described
 * with the declarations in lancius_graph.h.
 */
#define _GNU_SOURCE
#include <fcntl.h>
#include <pthread.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include "graph_internal.h"

#define MAX_NODES 1000000u   /* lancius_serialize.c:73 */
#define MAX_INPUTS 16u       /* :92 */
#define ID_SLACK 1000u       /* map_size = node_count + 1000, :77 */
#define MAX_ELEMS 100000000u /* :217 */
#define V2_BLOCK_ALIGN 4096u
#define V2_TENSOR_ALIGN 256u

enum { LAYOUT_V9 = 9, LAYOUT_V10 = 10, LAYOUT_V2 = 2 };

/* ---- CRC-32 -------------------------------------------------------------------
 * Reflected polynomial 0xEDB88320, initial value and final xor 0xFFFFFFFF
 * (IEEE 802.3 / zlib).  Eight tables, eight bytes per step ("slicing by 8",
 * Kounavis and Berry, Intel 2005). */
static uint32_t crc_tab[8][256];

__attribute__((constructor)) static void crc_init(void) {
    for (uint32_t i = 0; i < 256; i++) {
        uint32_t c = i;
        for (int k = 0; k < 8; k++) c = (c & 1u) ? (c >> 1) ^ 0xEDB88320u : c >> 1;
        crc_tab[0][i] = c;
    }
    for (uint32_t i = 0; i < 256; i++)
        for (int t = 1; t < 8; t++) crc_tab[t][i] = (crc_tab[t - 1][i] >> 8) ^ crc_tab[0][crc_tab[t - 1][i] & 0xFFu];
}

static uint32_t crc32_serial(uint32_t crc, const void* data, size_t len) {
    const uint8_t* p = (const uint8_t*)data;
    crc = ~crc;
    while (len >= 8) {
        const uint32_t lo = crc ^ ((uint32_t)p[0] | (uint32_t)p[1] << 8 | (uint32_t)p[2] << 16 | (uint32_t)p[3] << 24);
        const uint32_t hi = (uint32_t)p[4] | (uint32_t)p[5] << 8 | (uint32_t)p[6] << 16 | (uint32_t)p[7] << 24;
        crc = crc_tab[7][lo & 0xFFu] ^ crc_tab[6][(lo >> 8) & 0xFFu] ^ crc_tab[5][(lo >> 16) & 0xFFu] ^
              crc_tab[4][lo >> 24] ^ crc_tab[3][hi & 0xFFu] ^ crc_tab[2][(hi >> 8) & 0xFFu] ^
              crc_tab[1][(hi >> 16) & 0xFFu] ^ crc_tab[0][hi >> 24];
        p += 8;
        len -= 8;
    }
    while (len--) crc = crc_tab[0][(crc ^ *p++) & 0xFFu] ^ (crc >> 8);
    return ~crc;
}

/* Polynomials over GF(2) modulo P in the reflected representation of the
 * table above: bit k holds the coefficient of x^(31-k), so 1u << 31 is 1 and
 * multiplying by x is a right shift that folds bit 0 (x^32) back in as the
 * low terms of P. */
static uint32_t gf2_mulmod(uint32_t a, uint32_t b) {
    uint32_t prod = 0;
    for (uint32_t m = 1u << 31; m; m >>= 1) {
        if (a & m) prod ^= b;
        b = (b & 1u) ? (b >> 1) ^ 0xEDB88320u : b >> 1;
    }
    return prod;
}

/* x^(8 n) mod P by squaring: x^(2^j) for every set bit j of 8n. */
static uint32_t x_pow_8n(uint64_t n) {
    uint32_t result = 1u << 31, sq = 1u << 30; /* 1 and x */
    for (uint64_t e = n << 3; e; e >>= 1) {
        if (e & 1u) result = gf2_mulmod(result, sq);
        sq = gf2_mulmod(sq, sq);
    }
    return result;
}

/* CRC of A followed by B from crc(A), crc(B) and |B|: the bits of A move
 * 8|B| places further from the end, i.e. crc(A) * x^(8|B|) mod P, and the
 * pre/post-conditioning terms cancel (the combination used by zlib's
 * crc32_combine, M. Adler). */
static uint32_t crc32_combine_(uint32_t crc_a, uint32_t crc_b, uint64_t len_b) {
    return gf2_mulmod(x_pow_8n(len_b), crc_a) ^ crc_b;
}

typedef struct {
    const uint8_t* p;
    size_t len;
    uint32_t crc;
} crc_job;

static void* crc_worker(void* arg) {
    crc_job* j = (crc_job*)arg;
    j->crc = crc32_serial(0, j->p, j->len);
    return NULL;
}

/* Large buffers are split over up to 16 threads (each chunk's CRC from 0)
 * and the chunk CRCs combined in order; the result equals the serial CRC. */
uint32_t lancius_crc32(uint32_t crc, const void* data, size_t len) {
    enum { MAX_JOBS = 16 };
    const size_t min_chunk = (size_t)4 << 20;
    long cpus = sysconf(_SC_NPROCESSORS_ONLN);
    size_t jobs = len / min_chunk;
    if (jobs > MAX_JOBS) jobs = MAX_JOBS;
    if (cpus > 0 && jobs > (size_t)cpus) jobs = (size_t)cpus;
    if (jobs < 2) return crc32_serial(crc, data, len);
    crc_job job[MAX_JOBS];
    pthread_t tid[MAX_JOBS];
    int started[MAX_JOBS] = {0};
    const uint8_t* p = (const uint8_t*)data;
    const size_t chunk = len / jobs;
    for (size_t i = 0; i < jobs; i++) {
        job[i].p = p + i * chunk;
        job[i].len = i + 1 == jobs ? len - i * chunk : chunk;
        started[i] = i > 0 && pthread_create(&tid[i], NULL, crc_worker, &job[i]) == 0;
    }
    for (size_t i = 0; i < jobs; i++)
        if (!started[i]) crc_worker(&job[i]); /* the calling thread takes chunk 0 and any thread that failed */
    for (size_t i = 0; i < jobs; i++) {
        if (started[i]) pthread_join(tid[i], NULL);
        crc = crc32_combine_(crc, job[i].crc, job[i].len);
    }
    return crc;
}

/* ---- reading ------------------------------------------------------------------ */

typedef struct {
    const uint8_t* base;
    size_t size;
    size_t off;
} cursor;

static int get(cursor* c, void* dst, size_t k) {
    if (k > c->size - c->off) return -1;
    memcpy(dst, c->base + c->off, k);
    c->off += k;
    return 0;
}

static int skip(cursor* c, uint64_t k) {
    if (k > (uint64_t)(c->size - c->off)) return -1;
    c->off += (size_t)k;
    return 0;
}

typedef struct {
    uint32_t id, op, input_count;
    uint8_t ndim;
    uint64_t shape[4];
    uint32_t in_ids[MAX_INPUTS];
    double attr;
    uint32_t meta[4], axes[4];
    uint8_t is_view;
    uint64_t strides[4];
    uint32_t view_src;
    uint8_t has_w;
} record;

/* One node record up to and including has_weights (lancius_serialize.c:84-136). */
static int read_record(cursor* c, int layout, uint32_t map_size, record* r) {
    if (get(c, &r->id, 4) || r->id >= map_size) return -1;
    if (get(c, &r->op, 4) || get(c, &r->ndim, 1) || get(c, r->shape, 32) || get(c, &r->input_count, 4)) return -1;
    if (r->ndim > 4 || r->input_count > MAX_INPUTS || get(c, r->in_ids, 4 * (size_t)r->input_count)) return -1;
    for (uint32_t j = 0; j < r->input_count; j++)
        if (r->in_ids[j] >= map_size) return -1;
    if (get(c, &r->attr, 8) || get(c, r->meta, 16) || get(c, r->axes, 16)) return -1;
    r->is_view = 0;
    r->view_src = UINT32_MAX;
    memset(r->strides, 0, sizeof(r->strides));
    if (layout != LAYOUT_V9) {
        if (get(c, &r->is_view, 1) || r->is_view > 1) return -1;
        if (r->is_view && (get(c, r->strides, 32) || get(c, &r->view_src, 4))) return -1;
    }
    if (get(c, &r->has_w, 1) || r->has_w > 1) return -1;
    return 0;
}

/* Rebuild a node with the builder for its op (lancius_serialize.c:143-182).
 * Returns NULL with *skipped = 1 for NOP and unknown ops, NULL with
 * *skipped = 0 when an input it reads is missing or the builder refuses. */
static lancius_node* build(lancius_graph* g, const record* r, lancius_node* const* id_map, int* skipped) {
    const lancius_node* in[MAX_INPUTS];
    for (uint32_t j = 0; j < r->input_count; j++) in[j] = id_map[r->in_ids[j]];
    *skipped = 0;
#define NEED(k)                                                              \
    do {                                                                     \
        if (r->input_count < (k)) return NULL;                               \
        for (uint32_t j_ = 0; j_ < (k); j_++)                                \
            if (!in[j_]) return NULL;                                        \
    } while (0)
    const uint64_t* s = r->shape;
    const uint32_t* m = r->meta;
    lancius_node* n = NULL;
    switch ((lancius_opcode)r->op) {
        case LANCIUS_OP_INPUT:
            return r->ndim == 4 ? lancius_input_4d(g, s[0], s[1], s[2], s[3]) : lancius_input(g, s[0], s[1]);
        case LANCIUS_OP_CONST: return lancius_const(g, r->attr, s[0], s[1]);
        case LANCIUS_OP_ADD: NEED(2); return lancius_add(g, in[0], in[1]);
        case LANCIUS_OP_SUB: NEED(2); return lancius_sub(g, in[0], in[1]);
        case LANCIUS_OP_MUL: NEED(2); return lancius_mul(g, in[0], in[1]);
        case LANCIUS_OP_MATMUL: NEED(2); return lancius_matmul(g, in[0], in[1]);
        case LANCIUS_OP_RELU: NEED(1); return lancius_relu(g, in[0]);
        case LANCIUS_OP_SOFTMAX: NEED(1); return lancius_softmax(g, in[0]);
        case LANCIUS_OP_SUM: NEED(1); return lancius_sum(g, in[0]);
        case LANCIUS_OP_BROADCAST:
            NEED(1);
            return r->ndim == 4 ? lancius_broadcast_4d(g, in[0], s[0], s[1], s[2], s[3])
                                : lancius_broadcast(g, in[0], s[0], s[1]);
        case LANCIUS_OP_TRANSPOSE: NEED(1); return lancius_transpose(g, in[0]);
        case LANCIUS_OP_RELU_BWD: NEED(2); return lancius_relu_bwd(g, in[0], in[1]);
        case LANCIUS_OP_SOFTMAX_BWD: NEED(2); return lancius_softmax_bwd(g, in[0], in[1]);
        case LANCIUS_OP_SUM_AXIS0: NEED(1); return lancius_sum_axis0(g, in[0]);
        case LANCIUS_OP_SUM_AXIS1: NEED(1); return lancius_sum_axis1(g, in[0]);
        case LANCIUS_OP_CONV2D: NEED(2); return lancius_conv2d(g, in[0], in[1], m[2], m[3]);
        case LANCIUS_OP_CONV2D_RELU_FUSED:
            NEED(2);
            n = lancius_conv2d(g, in[0], in[1], m[2], m[3]);
            if (n) n->op = LANCIUS_OP_CONV2D_RELU_FUSED;
            return n;
        case LANCIUS_OP_MAXPOOL2D: NEED(1); return lancius_maxpool2d(g, in[0], m[0], m[2]);
        case LANCIUS_OP_FLATTEN: NEED(1); return lancius_flatten(g, in[0]);
        case LANCIUS_OP_RESHAPE: NEED(1); return lancius_reshape(g, in[0], r->ndim, s[0], s[1], s[2], s[3]);
        case LANCIUS_OP_CROSS_ENTROPY: NEED(2); return lancius_cross_entropy(g, in[0], in[1]);
        case LANCIUS_OP_CROSS_ENTROPY_BWD: NEED(3); return lancius_cross_entropy_bwd(g, in[0], in[1], in[2]);
        case LANCIUS_OP_PERMUTE:
            NEED(1);
            return lancius_permute(g, in[0], r->axes[0], r->axes[1], r->axes[2], r->axes[3]);
        case LANCIUS_OP_MATMUL_BATCHED: NEED(2); return lancius_matmul_batched(g, in[0], in[1]);
        case LANCIUS_OP_CONV2D_BWD: NEED(3); return lancius_conv2d_bwd(g, in[0], in[1], in[2], m[2], m[3]);
        case LANCIUS_OP_CONV2D_BWD_W: NEED(2); return lancius_conv2d_bwd_w(g, in[0], in[1], m[0], m[1], m[2], m[3]);
        case LANCIUS_OP_MAXPOOL2D_BWD: NEED(2); return lancius_maxpool2d_bwd(g, in[0], in[1], m[0], m[2]);
        case LANCIUS_OP_LAYERNORM: NEED(3); return lancius_layernorm(g, in[0], in[1], in[2]);
        case LANCIUS_OP_GELU: NEED(1); return lancius_gelu(g, in[0]);
        case LANCIUS_OP_ATTENTION: NEED(3); return lancius_attention(g, in[0], in[1], in[2]);
        case LANCIUS_OP_RMSNORM: NEED(2); return lancius_rmsnorm(g, in[0], in[1]);
        case LANCIUS_OP_SWIGLU: NEED(2); return lancius_swiglu(g, in[0], in[1]);
        case LANCIUS_OP_GQA: NEED(3); return lancius_gqa(g, in[0], in[1], in[2], m[0], m[1]);
        case LANCIUS_OP_ROPE:
        case LANCIUS_OP_EMBEDDING:
        case LANCIUS_OP_KV_CACHE_READ:
        case LANCIUS_OP_KV_CACHE_WRITE:
            /* no builder: the recorded shape and inputs */
            NEED(r->input_count);
            n = lancius__raw_node(g, (lancius_opcode)r->op, r->ndim, r->input_count);
            if (n) {
                for (uint8_t d = 0; d < r->ndim; d++) n->shape[d] = (size_t)s[d];
                for (uint32_t j = 0; j < r->input_count; j++) n->inputs[j] = in[j];
            }
            return n;
        default:
            *skipped = 1;
            return NULL;
    }
#undef NEED
}

typedef struct {
    lancius_weight_ref* refs;
    uint32_t count, cap;
} ref_list;

static int push_ref(ref_list* l, lancius_weight_ref ref) {
    if (l->count == l->cap) {
        const uint32_t cap = l->cap ? 2 * l->cap : 16;
        lancius_weight_ref* grown = (lancius_weight_ref*)realloc(l->refs, cap * sizeof(*grown));
        if (!grown) return -1;
        l->refs = grown;
        l->cap = cap;
    }
    l->refs[l->count++] = ref;
    return 0;
}

typedef struct {
    lancius_graph* g;
    ref_list refs;
    uint32_t skipped, first_skipped_op;
    uint32_t tensors; /* weighted records */
    int exact; /* the records end exactly where the layout says they must */
    int oom;
} attempt;

static void attempt_drop(attempt* a) {
    lancius_graph_destroy(a->g);
    free(a->refs.refs);
    memset(a, 0, sizeof(*a));
}

static size_t enc_size(lancius_dtype enc) { return enc == LANCIUS_DTYPE_INT8 ? 1 : enc == LANCIUS_DTYPE_FP32 ? 4 : 8; }

/* A node's element count must be representable: the product of its dims,
 * formed with overflow checks, at most 2^40 (so byte counts of any dtype
 * stay far inside size_t).  A crafted shape such as [2^32, 2^32], recorded
 * or derived by a builder from such inputs, would otherwise wrap to a small
 * count that passes every later size check. */
#define MAX_NODE_ELEMS ((uint64_t)1 << 40)
static int shape_ok(const lancius_node* n) {
    uint64_t e = 1;
    if (n->ndim > 4) return 0;
    for (uint8_t d = 0; d < n->ndim; d++)
        if (__builtin_mul_overflow(e, (uint64_t)n->shape[d], &e)) return 0;
    return e <= MAX_NODE_ELEMS;
}

/* Payload of a weighted node: host copy (lazy == 0) or a map entry. */
static int take_weights(attempt* a, lancius_node* n, lancius_dtype node_dtype, double scale, lancius_dtype enc,
                        const uint8_t* src, uint64_t file_offset, uint64_t e, int lazy) {
    n->dtype = node_dtype;
    n->scale = scale;
    if (n->rt) {
        n->rt->dtype = node_dtype;
        n->rt->scale = scale;
    }
    if (lazy) {
        const lancius_weight_ref ref = {n, file_offset, e, enc, scale};
        if (push_ref(&a->refs, ref)) return a->oom = 1, -1;
        return 0;
    }
    if (enc == LANCIUS_DTYPE_INT8) {
        int8_t* q = (int8_t*)malloc(e ? (size_t)e : 1);
        if (!q) return a->oom = 1, -1;
        memcpy(q, src, (size_t)e);
        n->runtime_data_int8 = q;
        if (n->rt) {
            n->rt->buffer_int8 = q;
            n->rt->int8_owner = LANCIUS_MEMORY_OWNED_HEAP;
        }
        return 0;
    }
    double* d = (double*)malloc(e ? (size_t)e * sizeof(double) : sizeof(double));
    if (!d) return a->oom = 1, -1;
    if (enc == LANCIUS_DTYPE_FP64) {
        memcpy(d, src, (size_t)e * sizeof(double));
    } else {
        for (uint64_t k = 0; k < e; k++) {
            float f;
            memcpy(&f, src + 4 * k, 4);
            d[k] = (double)f;
        }
    }
    n->runtime_data = d;
    if (n->rt) {
        n->rt->buffer = d;
        n->rt->buffer_owner = LANCIUS_MEMORY_OWNED_HEAP;
        n->rt->owner = LANCIUS_MEMORY_OWNED_HEAP;
        n->rt->flags |= LANCIUS_RT_FLAG_LOADED;
    }
    return 0;
}

/* Records of one layout in file bytes [rec_begin, rec_end); v2 payloads lie
 * in [wblock, file_size).  0 on success (a->g holds the graph). */
static int parse_records(const uint8_t* base, size_t file_size, size_t rec_begin, size_t rec_end, int layout,
                         uint32_t node_count, uint64_t wblock, int lazy, attempt* a) {
    cursor c = {base, rec_end, rec_begin};
    memset(a, 0, sizeof(*a));
    const uint32_t map_size = node_count + ID_SLACK;
    lancius_node** id_map = (lancius_node**)calloc(map_size, sizeof(lancius_node*));
    a->g = lancius_graph_create();
    if (!id_map || !a->g) {
        a->oom = 1;
        goto bad;
    }
    for (uint32_t i = 0; i < node_count; i++) {
        record r;
        if (read_record(&c, layout, map_size, &r)) goto bad;
        int skipped = 0;
        lancius_node* n = build(a->g, &r, id_map, &skipped);
        if (!n && !skipped) goto bad;
        if (n && !shape_ok(n)) goto bad;
        if (n) {
            n->kernel_h = r.meta[0];
            n->kernel_w = r.meta[1];
            n->stride = r.meta[2];
            n->pad = r.meta[3];
            memcpy(n->axes, r.axes, sizeof(n->axes));
            n->attr_val = r.attr;
            if (r.is_view) {
                n->is_view = 1;
                for (int d = 0; d < 4; d++) n->strides[d] = (size_t)r.strides[d];
                if (r.view_src < map_size) n->view_source = id_map[r.view_src];
            }
            id_map[r.id] = n;
        } else {
            if (!a->skipped) a->first_skipped_op = r.op;
            a->skipped++;
        }
        if (!r.has_w) continue;
        if (!n) goto bad; /* the payload of a skipped node cannot be sized */
        uint8_t dt;
        double scale;
        if (get(&c, &dt, 1) || dt > LANCIUS_DTYPE_INT32 || get(&c, &scale, 8)) goto bad;
        const uint64_t e = lancius_node_elements(n);
        if (e > MAX_ELEMS) goto bad;
        lancius_dtype enc;
        uint64_t off;
        if (layout == LAYOUT_V2) {
            uint8_t ev;
            uint64_t fe, fo;
            if (get(&c, &ev, 1) || get(&c, &fe, 8) || get(&c, &fo, 8) || fe != e) goto bad;
            if (ev != LANCIUS_DTYPE_FP64 && ev != LANCIUS_DTYPE_FP32 && ev != LANCIUS_DTYPE_INT8) goto bad;
            enc = (lancius_dtype)ev;
            const uint64_t bytes = e * enc_size(enc);
            if (wblock > file_size || fo > file_size - wblock || bytes > file_size - wblock - fo) goto bad;
            off = wblock + fo;
        } else {
            /* lancius_serialize.c:233-240: int8 bytes for INT8, else fp64 */
            enc = dt == LANCIUS_DTYPE_INT8 ? LANCIUS_DTYPE_INT8 : LANCIUS_DTYPE_FP64;
            off = c.off;
            if (skip(&c, e * enc_size(enc))) goto bad;
        }
        if (take_weights(a, n, (lancius_dtype)dt, scale, enc, base + off, off, e, lazy)) goto bad;
        a->tensors++;
    }
    if (layout == LAYOUT_V2) {
        /* records end inside the record section; the rest up to the weight
         * block is zero padding */
        a->exact = c.off <= wblock;
        for (size_t k = c.off; a->exact && k < wblock; k++) a->exact = base[k] == 0;
        if (!a->exact) goto bad;
    } else {
        a->exact = c.off == c.size;
    }
    free(id_map);
    return 0;
bad:
    free(id_map);
    lancius_graph_destroy(a->g);
    a->g = NULL;
    free(a->refs.refs);
    a->refs.refs = NULL;
    a->refs.count = a->refs.cap = 0;
    return -1;
}

typedef struct {
    const uint8_t* base;
    size_t size;
    void* map;
} mapped_file;

static int map_file(const char* path, mapped_file* f) {
    memset(f, 0, sizeof(*f));
    const int fd = open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) return -1;
    struct stat st;
    if (fstat(fd, &st) || !S_ISREG(st.st_mode)) {
        close(fd);
        return -1;
    }
    f->size = (size_t)st.st_size;
    if (f->size) {
        f->map = mmap(NULL, f->size, PROT_READ, MAP_PRIVATE, fd, 0);
        if (f->map == MAP_FAILED) {
            f->map = NULL;
            close(fd);
            return -1;
        }
        f->base = (const uint8_t*)f->map;
    }
    close(fd);
    return 0;
}

static void unmap_file(mapped_file* f) {
    if (f->map) munmap(f->map, f->size);
    memset(f, 0, sizeof(*f));
}

static lancius_graph* invalid(const char* path, const char* why) {
    fprintf(stderr, "[SERIAL FATAL] %s: %s\n", path ? path : "(null)", why);
    lancius_set_error(LANCIUS_ERROR_INVALID_MODEL);
    return NULL;
}

static lancius_graph* load_any(const char* path, lancius_weight_map* map, int lazy) {
    if (map) memset(map, 0, sizeof(*map));
    if (!path) {
        lancius_set_error(LANCIUS_ERROR_NULL_PTR);
        return NULL;
    }
    mapped_file f;
    if (map_file(path, &f)) {
        lancius_set_error(LANCIUS_ERROR_IO);
        return NULL;
    }
    cursor c = {f.base, f.size, 0};
    uint32_t magic = 0, node_count = 0, crc = 0;
    attempt a;
    memset(&a, 0, sizeof(a));
    int layout = 0;
    lancius_graph* result = NULL;
    if (get(&c, &magic, 4)) {
        result = invalid(path, "truncated header");
        goto out;
    }
    if (magic == LANCIUS_MODEL_MAGIC_V2) {
        uint32_t h[8], reserved1;
        uint64_t wblock;
        c.off = 0;
        if (get(&c, h, sizeof(h)) || get(&c, &wblock, 8) || get(&c, &crc, 4) || get(&c, &reserved1, 4)) {
            result = invalid(path, "truncated v2 header");
            goto out;
        }
        /* h: magic, version, flags, node_count, tensor_count, attribute_count,
         * header_size, reserved0 */
        if (h[1] != 2u || h[6] != LANCIUS_MODEL_HEADER_SIZE_V2 || !(h[2] & LANCIUS_MODEL_FLAG_LITTLE_ENDIAN) ||
            h[3] > MAX_NODES || wblock < LANCIUS_MODEL_HEADER_SIZE_V2 || wblock > f.size) {
            result = invalid(path, "v2 header fields out of range");
            goto out;
        }
        if (lancius_crc32(0, f.base + LANCIUS_MODEL_HEADER_SIZE_V2, f.size - LANCIUS_MODEL_HEADER_SIZE_V2) != crc) {
            result = invalid(path, "v2 checksum mismatch");
            goto out;
        }
        node_count = h[3];
        if (parse_records(f.base, f.size, LANCIUS_MODEL_HEADER_SIZE_V2, (size_t)wblock, LAYOUT_V2, node_count, wblock,
                          lazy, &a) == 0) {
            if (a.tensors == h[4]) layout = LAYOUT_V2;
            else attempt_drop(&a);
        }
        if (!layout) {
            if (a.oom) lancius_set_error(LANCIUS_ERROR_OOM);
            else result = invalid(path, "malformed v2 records");
            goto out;
        }
    } else if (magic == LANCIUS_MODEL_MAGIC_V1) {
        if (get(&c, &node_count, 4)) {
            result = invalid(path, "truncated node count");
            goto out;
        }
        if (node_count > MAX_NODES) {
            result = invalid(path, "node count exceeds sanity limit");
            goto out;
        }
        attempt v10, v9;
        const int ok10 = parse_records(f.base, f.size, 8, f.size, LAYOUT_V10, node_count, 0, lazy, &v10) == 0;
        if (ok10 && v10.exact) {
            a = v10;
            layout = LAYOUT_V10;
        } else {
            const int ok9 = parse_records(f.base, f.size, 8, f.size, LAYOUT_V9, node_count, 0, lazy, &v9) == 0;
            if (ok9 && (v9.exact || !ok10)) {
                if (ok10) attempt_drop(&v10);
                a = v9;
                layout = LAYOUT_V9;
            } else if (ok10) {
                if (ok9) attempt_drop(&v9);
                a = v10;
                layout = LAYOUT_V10;
            } else if (v10.oom || v9.oom) {
                lancius_set_error(LANCIUS_ERROR_OOM);
                goto out;
            }
        }
        if (!layout) {
            result = invalid(path, "malformed or truncated .lancius file");
            goto out;
        }
    } else {
        result = invalid(path, "bad magic");
        goto out;
    }
    if (a.skipped)
        fprintf(stderr, "[LANCIUS SERIAL WARN] %s: skipped %u node(s) of unknown op (first: op %u)\n", path,
                a.skipped, a.first_skipped_op);
    if (map) {
        map->format = (uint32_t)layout;
        map->count = a.refs.count;
        map->refs = a.refs.refs;
        map->file_bytes = f.size;
        map->crc32 = layout == LAYOUT_V2 ? crc : 0;
        a.refs.refs = NULL;
    }
    free(a.refs.refs);
    result = a.g;
    printf("[LANCIUS SERIAL] Loaded %u nodes (layout v%d) from %s\n", node_count, layout, path);
out:
    unmap_file(&f);
    return result;
}

lancius_graph* lancius_graph_load(const char* path) { return load_any(path, NULL, 0); }

lancius_graph* lancius_graph_load_mapped(const char* path, lancius_weight_map* map) {
    if (!map) {
        lancius_set_error(LANCIUS_ERROR_NULL_PTR);
        return NULL;
    }
    return load_any(path, map, 1);
}

void lancius_weight_map_free(lancius_weight_map* map) {
    if (!map) return;
    free(map->refs);
    memset(map, 0, sizeof(*map));
}

/* ---- writing ------------------------------------------------------------------ */

typedef struct {
    FILE* f;
    uint32_t crc;
    int crc_on;
    int err;
    uint64_t pos;
} writer;

static void put(writer* w, const void* p, size_t k) {
    if (w->err || !k) return;
    if (fwrite(p, 1, k, w->f) != k) {
        w->err = 1;
        return;
    }
    if (w->crc_on) w->crc = lancius_crc32(w->crc, p, k);
    w->pos += k;
}

static void put_zeros(writer* w, uint64_t k) {
    static const uint8_t zeros[4096];
    while (k) {
        const size_t step = k < sizeof(zeros) ? (size_t)k : sizeof(zeros);
        put(w, zeros, step);
        k -= step;
    }
}

/* The record fields both layouts share, through has_weights
 * (lancius_serialize.c:23-43). */
static void put_record_head(writer* w, const lancius_node* n, uint8_t has_w) {
    const uint32_t id = n->id, op = (uint32_t)n->op, ic = n->input_count;
    put(w, &id, 4);
    put(w, &op, 4);
    put(w, &n->ndim, 1);
    for (int d = 0; d < 4; d++) {
        const uint64_t s = n->shape[d];
        put(w, &s, 8);
    }
    put(w, &ic, 4);
    for (uint32_t j = 0; j < ic; j++) {
        const uint32_t in = n->inputs[j] ? n->inputs[j]->id : UINT32_MAX;
        put(w, &in, 4);
    }
    put(w, &n->attr_val, 8);
    const uint32_t meta[4] = {n->kernel_h, n->kernel_w, n->stride, n->pad};
    put(w, meta, 16);
    put(w, n->axes, 16);
    const uint8_t view = n->is_view ? 1 : 0;
    put(w, &view, 1);
    if (view) {
        for (int d = 0; d < 4; d++) {
            const uint64_t s = n->strides[d];
            put(w, &s, 8);
        }
        const uint32_t src = n->view_source ? n->view_source->id : UINT32_MAX;
        put(w, &src, 4);
    }
    put(w, &has_w, 1);
}

/* Node dtype as written (lancius_serialize.c:48-51: invalid -> FP64) and the
 * payload encoding: int8 when the node is INT8 and has int8 data or has only
 * int8 data, else fp64. */
static void weight_kind(const lancius_node* n, uint8_t* dtype, lancius_dtype* enc) {
    uint8_t dt = (uint8_t)n->dtype;
    if (dt > LANCIUS_DTYPE_INT32) dt = LANCIUS_DTYPE_FP64;
    int i8 = dt == LANCIUS_DTYPE_INT8 && n->runtime_data_int8;
    if (!n->runtime_data) i8 = 1;
    if (dt == LANCIUS_DTYPE_INT8 && !i8) dt = LANCIUS_DTYPE_FP64;
    if (i8) dt = LANCIUS_DTYPE_INT8;
    *dtype = dt;
    *enc = i8 ? LANCIUS_DTYPE_INT8 : LANCIUS_DTYPE_FP64;
}

static int has_weights(const lancius_node* n) {
    return n->op == LANCIUS_OP_INPUT && (n->runtime_data || n->runtime_data_int8);
}

void lancius_graph_save(lancius_graph* g, const char* path) {
    if (!g || !path) {
        lancius_set_error(LANCIUS_ERROR_NULL_PTR);
        return;
    }
    for (uint32_t i = 0; i < g->node_count; i++)
        if (has_weights(g->nodes[i]) && lancius_node_elements(g->nodes[i]) > MAX_ELEMS) {
            fprintf(stderr, "[SERIAL FATAL] Tensor size exceeds sanity limit.\n");
            lancius_set_error(LANCIUS_ERROR_OVERFLOW);
            return;
        }
    writer w = {fopen(path, "wb"), 0, 0, 0, 0};
    if (!w.f) {
        lancius_set_error(LANCIUS_ERROR_IO);
        return;
    }
    const uint32_t magic = LANCIUS_MODEL_MAGIC_V1, count = g->node_count;
    put(&w, &magic, 4);
    put(&w, &count, 4);
    for (uint32_t i = 0; i < g->node_count; i++) {
        const lancius_node* n = g->nodes[i];
        const uint8_t hw = (uint8_t)has_weights(n);
        put_record_head(&w, n, hw);
        if (!hw) continue;
        uint8_t dt;
        lancius_dtype enc;
        weight_kind(n, &dt, &enc);
        put(&w, &dt, 1);
        put(&w, &n->scale, 8);
        const size_t e = lancius_node_elements(n);
        if (enc == LANCIUS_DTYPE_INT8) put(&w, n->runtime_data_int8, e);
        else put(&w, n->runtime_data, e * sizeof(double));
    }
    if (fclose(w.f) || w.err) lancius_set_error(LANCIUS_ERROR_IO);
    else printf("[LANCIUS SERIAL] Saved %u nodes to %s\n", g->node_count, path);
}

static uint64_t align_to(uint64_t x, uint64_t a) { return (x + a - 1) / a * a; }

int lancius_graph_save_v2(const lancius_graph* g, const char* path, lancius_dtype weight_dtype) {
    if (!g || !path) return LANCIUS_ERROR_NULL_PTR;
    if (weight_dtype != LANCIUS_DTYPE_FP64 && weight_dtype != LANCIUS_DTYPE_FP32)
        return LANCIUS_ERROR_UNSUPPORTED_DTYPE;
    /* pass 1: record bytes and the weight block layout */
    uint64_t rec_bytes = 0, wbytes = 0;
    uint32_t tensors = 0;
    for (uint32_t i = 0; i < g->node_count; i++) {
        const lancius_node* n = g->nodes[i];
        rec_bytes += 4 + 4 + 1 + 32 + 4 + 4ull * n->input_count + 8 + 16 + 16 + 1 + (n->is_view ? 36 : 0) + 1;
        if (!has_weights(n)) continue;
        const uint64_t e = lancius_node_elements(n);
        if (e > MAX_ELEMS) return LANCIUS_ERROR_OVERFLOW;
        uint8_t dt;
        lancius_dtype enc;
        weight_kind(n, &dt, &enc);
        if (enc != LANCIUS_DTYPE_INT8) enc = weight_dtype;
        rec_bytes += 1 + 8 + 1 + 8 + 8;
        wbytes = align_to(wbytes, V2_TENSOR_ALIGN) + e * enc_size(enc);
        tensors++;
    }
    const uint64_t wblock = align_to(LANCIUS_MODEL_HEADER_SIZE_V2 + rec_bytes, V2_BLOCK_ALIGN);
    writer w = {fopen(path, "wb"), 0, 0, 0, 0};
    if (!w.f) return LANCIUS_ERROR_IO;
    put_zeros(&w, LANCIUS_MODEL_HEADER_SIZE_V2); /* header written last */
    w.crc_on = 1;
    uint64_t woff = 0;
    for (uint32_t i = 0; i < g->node_count; i++) {
        const lancius_node* n = g->nodes[i];
        const uint8_t hw = (uint8_t)has_weights(n);
        put_record_head(&w, n, hw);
        if (!hw) continue;
        uint8_t dt;
        lancius_dtype enc;
        weight_kind(n, &dt, &enc);
        if (enc != LANCIUS_DTYPE_INT8) enc = weight_dtype;
        const uint8_t ev = (uint8_t)enc;
        const uint64_t e = lancius_node_elements(n);
        woff = align_to(woff, V2_TENSOR_ALIGN);
        put(&w, &dt, 1);
        put(&w, &n->scale, 8);
        put(&w, &ev, 1);
        put(&w, &e, 8);
        put(&w, &woff, 8);
        woff += e * enc_size(enc);
    }
    put_zeros(&w, wblock - w.pos);
    woff = 0;
    for (uint32_t i = 0; i < g->node_count && !w.err; i++) {
        const lancius_node* n = g->nodes[i];
        if (!has_weights(n)) continue;
        uint8_t dt;
        lancius_dtype enc;
        weight_kind(n, &dt, &enc);
        if (enc != LANCIUS_DTYPE_INT8) enc = weight_dtype;
        const uint64_t e = lancius_node_elements(n);
        const uint64_t at = align_to(woff, V2_TENSOR_ALIGN);
        put_zeros(&w, at - woff);
        if (enc == LANCIUS_DTYPE_INT8) {
            put(&w, n->runtime_data_int8, (size_t)e);
        } else if (enc == LANCIUS_DTYPE_FP64) {
            put(&w, n->runtime_data, (size_t)e * sizeof(double));
        } else {
            float buf[4096];
            for (uint64_t k = 0; k < e; k += 4096) {
                const size_t m = (size_t)(e - k < 4096 ? e - k : 4096);
                for (size_t j = 0; j < m; j++) buf[j] = (float)n->runtime_data[k + j];
                put(&w, buf, m * sizeof(float));
            }
        }
        woff = at + e * enc_size(enc);
    }
    (void)wbytes;
    /* header: magic, version, flags, node_count, tensor_count,
     * attribute_count (one attribute block per record), header_size,
     * reserved0, weight_block_offset, checksum_crc32, reserved1 */
    const uint32_t head[7] = {LANCIUS_MODEL_MAGIC_V2, 2u,
                              LANCIUS_MODEL_FLAG_LITTLE_ENDIAN | LANCIUS_MODEL_FLAG_STATIC_GRAPH,
                              g->node_count, tensors, g->node_count, LANCIUS_MODEL_HEADER_SIZE_V2};
    const uint32_t reserved0 = 0, reserved1 = 0;
    w.crc_on = 0;
    if (!w.err && fseek(w.f, 0, SEEK_SET)) w.err = 1;
    put(&w, head, sizeof(head));
    put(&w, &reserved0, 4);
    put(&w, &wblock, 8);
    put(&w, &w.crc, 4);
    put(&w, &reserved1, 4);
    const int bad = fclose(w.f) || w.err;
    if (bad) {
        remove(path);
        return LANCIUS_ERROR_IO;
    }
    return LANCIUS_ERROR_OK;
}
