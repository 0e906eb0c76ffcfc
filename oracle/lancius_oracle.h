/*
 * lancius_oracle.h - TEST INFRASTRUCTURE ONLY.
 *
 * fp64 CPU restatement of the reference Lancius hot path, used by tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg as the checker.
 * Nothing in the product (lancius_amd/, include/) links, loads or calls it.
 *
 * Every function follows the reference's loop order and fp64 accumulation
 * (citations per function in lancius_oracle.c; paths relative to the
 * reference root, B/ = bleeding/v11A1/).  How each function is pinned:
 *   oracle_matmul_rows    golden vectors of the compiled reference graph
 *                         MATMUL; closed forms (ones, identity, audit_ffi
 *                         [4,4,4,4,5,5,5,5]); NaN/Inf propagation
 *   oracle_conv2d         golden vectors of kernel_conv2d_fwd/_relu_fwd;
 *                         conv == im2col . GEMM; constant-input closed form
 *   oracle_attention      golden vectors of kernel_attention (causal);
 *                         naive softmax(QK^T)V (S9/examples/audit_flash_attention.c:9-49);
 *                         V constant => out constant; S = 1 => out = v0;
 *                         non-causal: textbook formula (no reference kernel)
 *   oracle_layernorm/gelu/softmax/argmax/add/relu/broadcast
 *                         golden vectors + closed forms (constant row => beta,
 *                         GELU(0) = 0 and the +-100 clamp, uniform softmax)
 *   oracle_sub/mul/relu_bwd/transpose/sum/sum_axis0/sum_axis1/softmax_bwd/
 *   cross_entropy/cross_entropy_bwd/maxpool2d/maxpool2d_bwd
 *                         golden vectors of the compiled reference scheduler
 *                         and vision router; closed forms (transpose twice =
 *                         identity, sums against numpy, softmax_bwd against
 *                         the Jacobian product, CE against numpy logsumexp,
 *                         CE gradient against finite differences)
 *   oracle_conv2d_bwd_input/_weight
 *                         golden vectors of kernel_conv2d_bwd_in/_w; adjoint
 *                         identities <conv(x,w), g> = <x, bwd_in(g,w)> =
 *                         <w, bwd_w(g,x)>; finite differences
 *   oracle_rmsnorm/swiglu/rope/attention_gqa/attention_decode
 *                         golden vectors of kernel_rmsnorm, kernel_swiglu,
 *                         kernel_rope, kernel_gqa, kernel_attention_kv_cache
 *                         and of the RMSNORM/SWIGLU/GQA/ROPE scheduler
 *                         branches; closed forms (rope is a rotation:
 *                         norms kept, inverse at -pos; GQA with Hkv = Hq is
 *                         oracle_attention; decode = last row of causal
 *                         attention over the cache)
 *   oracle_quantize_i8/matmul_i8/conv2d_i8
 *                         golden vectors of the compiled reference's int8
 *                         MATMUL branch and int8 conv route; int32 sums
 *                         equal to exact integer products (numpy int64);
 *                         quantization bounds |q| <= 127, q = round(x/s)
 *   oracle_schedule_execute
 *                         golden sink values of reference graph runs,
 *                         including autodiff training graphs
 */
#ifndef LANCIUS_ORACLE_H
#define LANCIUS_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#include "lancius_abi.h"

#ifdef __cplusplus
extern "C" {
#endif

/* OpenMP team size of the parallel oracle loops (n > 0). */
void oracle_set_threads(int n);

/* Rows [r0, r1) of out[M,N] = a[M,K] . b[K,N] (IKJ, fp64). */
void oracle_matmul_rows(double* out, const double* a, const double* b, size_t M, size_t K, size_t N, size_t r0,
                        size_t r1);

/* Images [n0, n1) of the NCHW conv; relu != 0 clamps on store. */
void oracle_conv2d(double* out, const double* in, const double* w, size_t N, size_t C_in, size_t H, size_t W,
                   size_t C_out, size_t K_h, size_t K_w, size_t stride, size_t pad, int relu, size_t n0, size_t n1);

/* Batches [b0, b1) and query rows [i0, i1) of attention over [batch,S,H,D]. */
void oracle_attention(double* out, const double* q, const double* k, const double* v, size_t batch, size_t S,
                      size_t H, size_t D, int causal, double scale, size_t b0, size_t b1, size_t i0, size_t i1);

void oracle_layernorm(double* out, const double* in, const double* gamma, const double* beta, size_t rows,
                      size_t hidden, double eps);
void oracle_gelu(double* out, const double* in, size_t n);
void oracle_softmax(double* out, const double* in, size_t rows, size_t cols);
void oracle_argmax(int32_t* idx, const double* in, size_t rows, size_t cols);
void oracle_add(double* out, const double* a, const double* b, size_t n);
void oracle_relu(double* out, const double* a, size_t n);
void oracle_broadcast(double* out, const double* a, size_t a_elems, size_t rows, size_t cols);

/* The rest of the scheduler dispatch (B/src/runtime/lancius_scheduler.c:68-104,
 * 236-304; B/src/math/lancius_kernels.c:62-136; B/src/runtime/lancius_vision_ops.c:82-190). */
void oracle_sub(double* out, const double* a, const double* b, size_t n);
void oracle_mul(double* out, const double* a, const double* b, size_t n);
void oracle_relu_bwd(double* out, const double* grad, const double* fwd, size_t n);
void oracle_transpose(double* out, const double* a, size_t rows, size_t cols);
void oracle_sum(double* out, const double* a, size_t n);
void oracle_sum_axis0(double* out, const double* a, size_t rows, size_t cols);
void oracle_sum_axis1(double* out, const double* a, size_t rows, size_t cols);
void oracle_softmax_bwd(double* out, const double* dy, const double* y, size_t rows, size_t cols);
void oracle_cross_entropy(double* out, const double* x, const double* y, size_t rows, size_t cols);
void oracle_cross_entropy_bwd(double* out, const double* x, const double* y, const double* g, size_t rows,
                              size_t cols);
void oracle_conv2d_bwd_input(double* dx, const double* dy, const double* w, size_t N, size_t C_in, size_t H,
                             size_t W, size_t C_out, size_t Ho, size_t Wo, size_t K_h, size_t K_w, size_t stride,
                             size_t pad);
void oracle_conv2d_bwd_weight(double* dw, const double* dy, const double* x, size_t N, size_t C_in, size_t H,
                              size_t W, size_t C_out, size_t Ho, size_t Wo, size_t K_h, size_t K_w, size_t stride,
                              size_t pad);
void oracle_maxpool2d(double* out, const double* in, size_t N, size_t C, size_t H, size_t W, size_t K,
                      size_t stride);
void oracle_maxpool2d_bwd(double* dx, const double* dy, const double* x, size_t N, size_t C, size_t H, size_t W,
                          size_t Ho, size_t Wo, size_t K, size_t stride);

/* Decode-side attention family (B/src/math/lancius_kernels.c:248-272, 338-448). */
void oracle_rmsnorm(double* out, const double* in, const double* gamma, size_t rows, size_t hidden, double eps);
void oracle_swiglu(double* out, const double* gate, const double* up, size_t n);
void oracle_rope(double* out, const double* in, size_t count, size_t batch, size_t S, size_t H, size_t hd,
                 int pos_offset);
void oracle_attention_gqa(double* out, const double* q, const double* k, const double* v, size_t batch, size_t Sq,
                          size_t Skv, size_t Hq, size_t Hkv, size_t D, int causal, double scale);
void oracle_attention_decode(double* out, const double* q, const double* k, const double* v, const int32_t* lens,
                             size_t batch, size_t Skv, size_t Hq, size_t Hkv, size_t D, double scale);

/* The int8 path (B/src/runtime/lancius_scheduler.c:195-220,
 * B/src/math/lancius_kernels.c:177-210, B/src/runtime/lancius_vision_ops.c:16-57,
 * B/src/compiler/lancius_quantize.c:6-33).  0, or -1 on allocation failure. */
double oracle_quantize_i8(int8_t* q, const double* x, size_t n);
int oracle_matmul_i8(double* out, const double* a, const int8_t* b, double scale_b, size_t M, size_t K, size_t N);
int oracle_conv2d_i8(double* out, const double* in, const int8_t* w, double scale_w, size_t N, size_t C_in, size_t H,
                     size_t W, size_t C_out, size_t K_h, size_t K_w, size_t stride, size_t pad, int relu);

/* fp64 CPU execution of a scheduled graph, node by node in wave order, the
 * way the reference's scratch-arena executor does it
 * (B/src/runtime/lancius_scheduler.c:311-362).  Nodes whose runtime_data is
 * NULL get a fresh malloc'd buffer (released by oracle_release_buffers);
 * INPUT nodes must already be bound.  Returns 0, or -4 for an op outside
 * the device path, -1 on allocation failure. */
int oracle_schedule_execute(lancius_schedule* s, int num_threads);
void oracle_release_buffers(lancius_graph* g);

#ifdef __cplusplus
}
#endif

#endif
