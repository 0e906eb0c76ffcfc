/*
 * lancius_hip.h - C ABI of the MI355X (gfx950) kernel backend for Lancius.
 *
 * Pure C.  Every pointer named "device" is an address in GPU memory (HBM);
 * buffers are owned by the caller.  Every entry point returns an int status:
 * 0 on success or a negative code with the values of the reference error
 * model (bleeding/v11A1/include/lancius/lancius_error.h:6-18):
 *   -1 out of memory, -2 null pointer, -3 shape mismatch / bad size,
 *   -4 unsupported op, -10 internal (any other HIP failure).
 * A thread-local message for the last failure is available from
 * lancius_hip_last_error().  No entry point aborts the process.
 *
 * Kernel launches are asynchronous on the stream of the context; two
 * contexts on different streams may be used from different host threads
 * concurrently (the reference runs nodes of one wave from a pthread pool,
 * bleeding/v11A1/src/runtime/lancius_scheduler.c:405-411).
 */
#ifndef LANCIUS_HIP_H
#define LANCIUS_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#if defined(_WIN32)
#define LANCIUS_HIP_EXPORT __declspec(dllexport)
#else
#define LANCIUS_HIP_EXPORT __attribute__((visibility("default")))
#endif

/* Status codes; same numbers as lancius_error (lancius_error.h:6-18). */
#define LANCIUS_HIP_OK                 0
#define LANCIUS_HIP_ERR_OOM           (-1)
#define LANCIUS_HIP_ERR_NULL_PTR      (-2)
#define LANCIUS_HIP_ERR_SHAPE         (-3)
#define LANCIUS_HIP_ERR_UNSUPPORTED   (-4)
#define LANCIUS_HIP_ERR_DTYPE         (-5)
#define LANCIUS_HIP_ERR_INTERNAL      (-10)

/* Epilogue activation of the GEMM / conv kernels. */
#define LANCIUS_HIP_ACT_NONE 0
#define LANCIUS_HIP_ACT_RELU 1   /* max(x, 0): lancius_scheduler.c:305-308       */
#define LANCIUS_HIP_ACT_GELU 2   /* tanh GELU with +-100 clamp: lancius_kernels.c:238-246 */
#define LANCIUS_HIP_ACT_TANH 3   /* tanh(x): BASIS_OP_TANH (include/basis/stage6_ir/graph.h:12) */

typedef struct lancius_hip_ctx lancius_hip_ctx;

/* ---- context, memory, timing --------------------------------------- */

/* Creates a context on `device`.  `stream` is a hipStream_t passed as an
 * opaque pointer; NULL selects the device's null stream. */
LANCIUS_HIP_EXPORT int lancius_hip_ctx_create(int device, void* stream, lancius_hip_ctx** out);
LANCIUS_HIP_EXPORT void lancius_hip_ctx_destroy(lancius_hip_ctx* ctx);
LANCIUS_HIP_EXPORT const char* lancius_hip_last_error(void);
/* Number of GPUs visible to HIP (0 when none; never fails). */
LANCIUS_HIP_EXPORT int lancius_hip_device_count(void);

LANCIUS_HIP_EXPORT int lancius_hip_malloc(lancius_hip_ctx* ctx, void** device_ptr, size_t bytes);
LANCIUS_HIP_EXPORT int lancius_hip_free(lancius_hip_ctx* ctx, void* device_ptr);
/* Synchronous copies (they wait for the context's stream). */
LANCIUS_HIP_EXPORT int lancius_hip_upload(lancius_hip_ctx* ctx, void* device_dst, const void* host_src, size_t bytes);
LANCIUS_HIP_EXPORT int lancius_hip_download(lancius_hip_ctx* ctx, void* host_dst, const void* device_src, size_t bytes);
LANCIUS_HIP_EXPORT int lancius_hip_synchronize(lancius_hip_ctx* ctx);

/* HIP events on the context's stream: start, then stop returns the
 * elapsed milliseconds between the two records (waits for the stop). */
LANCIUS_HIP_EXPORT int lancius_hip_timer_start(lancius_hip_ctx* ctx);
LANCIUS_HIP_EXPORT int lancius_hip_timer_stop(lancius_hip_ctx* ctx, float* elapsed_ms);

/* ---- kernels (device pointers, fp32, row-major) --------------------- */

/* C[M,N] = epilogue(A[M,K] . B[K,N]).
 * Epilogue order: y = acc + bias[n] (bias may be NULL); y = act(y) with act
 * any LANCIUS_HIP_ACT_*; y = y + residual[m,n] (residual may be NULL; it
 * may alias C).  Replaces the MATMUL branch (lancius_scheduler.c:222-234)
 * plus the BROADCAST/ADD/RELU/GELU nodes that follow it in a graph (and the
 * BASIS graph's BROADCAST_ADD/RELU/TANH/ADD, include/lancius_basis.h). */
LANCIUS_HIP_EXPORT int lancius_hip_gemm_f32(lancius_hip_ctx* ctx, float* C, const float* A, const float* B,
                                            size_t M, size_t K, size_t N,
                                            const float* bias, int act, const float* residual);

/* No counterpart in the reference.  For callers that cannot allocate device
 * memory (code under HIP graph capture, serving loops or harnesses that
 * forbid hipMalloc): lancius_hip_gemm_f32 with its split-K partial sums in a
 * fixed scratch array of LANCIUS_HIP_NOALLOC_SCRATCH_BYTES inside the
 * library, one per GPU, held until the process ends; it never grows the
 * context workspace and calls no hipMalloc or hipFree.  Same kernels and same
 * split choice as lancius_hip_gemm_f32, hence the same bits.  A shape whose
 * partial sums would exceed the scratch returns -3 before anything is
 * launched.  Every call on one GPU shares that GPU's scratch: calls that
 * overlap on one GPU (two streams or two host threads) race, so order them. */
#define LANCIUS_HIP_NOALLOC_SCRATCH_BYTES ((size_t)32 << 20)
LANCIUS_HIP_EXPORT int lancius_hip_gemm_f32_noalloc(lancius_hip_ctx* ctx, float* C, const float* A, const float* B,
                                                    size_t M, size_t K, size_t N,
                                                    const float* bias, int act, const float* residual);

/* `count` independent GEMMs of one shape in a single launch (the branches of
 * one scheduler wave).  Every array is a host array of `count` device
 * pointers; B[g] and bias[g] may repeat; bias and residual may be NULL (the
 * array) or hold NULLs.  count <= LANCIUS_HIP_MAX_GROUP. */
#define LANCIUS_HIP_MAX_GROUP 16
LANCIUS_HIP_EXPORT int lancius_hip_gemm_grouped_f32(lancius_hip_ctx* ctx, size_t count,
                                                    float* const* C, const float* const* A, const float* const* B,
                                                    size_t M, size_t K, size_t N,
                                                    const float* const* bias, int act, const float* const* residual);

/* The same with transposed operands: trans_a != 0 reads A as stored
 * [K][M] (element (m,k) at A[k*M + m]); trans_b != 0 reads B as stored
 * [N][K] (element (k,n) at B[n*K + k]).  A TRANSPOSE node feeding a
 * MATMUL (the autodiff products dX = dY . W^T and dW = X^T . dY,
 * lancius_autodiff.c:149-153) runs as one of these, with no transposed copy. */
LANCIUS_HIP_EXPORT int lancius_hip_gemm_ex_f32(lancius_hip_ctx* ctx, float* C, const float* A, const float* B,
                                               size_t M, size_t K, size_t N, int trans_a, int trans_b,
                                               const float* bias, int act, const float* residual);
LANCIUS_HIP_EXPORT int lancius_hip_gemm_grouped_ex_f32(lancius_hip_ctx* ctx, size_t count,
                                                       float* const* C, const float* const* A,
                                                       const float* const* B, size_t M, size_t K, size_t N,
                                                       int trans_a, int trans_b, const float* const* bias, int act,
                                                       const float* const* residual);

/* out[N,C_out,H_out,W_out] = act(conv(in[N,C_in,H,W], w[C_out,C_in,K_h,K_w]) + bias[C_out]).
 * Cross-correlation with zero padding, H_out = (H + 2 pad - K_h)/stride + 1
 * (lancius_kernels.c:28-60, ReLU variant :140-173).  bias may be NULL;
 * act is LANCIUS_HIP_ACT_NONE or LANCIUS_HIP_ACT_RELU. */
LANCIUS_HIP_EXPORT int lancius_hip_conv2d_f32(lancius_hip_ctx* ctx, float* out, const float* in, const float* w,
                                              const float* bias,
                                              size_t N, size_t C_in, size_t H, size_t W,
                                              size_t C_out, size_t K_h, size_t K_w,
                                              size_t stride, size_t pad, int act);
/* The same conv split in two for a weight used many times (an inference
 * graph's constant filters): the reference reads w in OIHW inside its loops
 * (lancius_kernels.c:147-165); the device kernels read the filter per
 * output channel with taps outer and input channels inner, and
 * lancius_hip_conv2d_f32 re-lays w into that order on every call.
 * lancius_hip_conv2d_pack_weight does it once into `packed`
 * (lancius_hip_conv2d_packed_bytes(...) bytes), and
 * lancius_hip_conv2d_packed_f32 takes the packed copy in place of w; results
 * are bit-identical to lancius_hip_conv2d_f32.  Both require C_in % 16 == 0
 * and C_out % 4 == 0, and the packed conv also one image (C_in * H * W
 * floats) and the filter each under LANCIUS_HIP_CONV_PACKED_MAX_BYTES
 * (else -3); other convs read OIHW directly and have nothing to pack.  The
 * device executor keeps one packed copy per such filter and re-packs it
 * after an upload. */
#define LANCIUS_HIP_CONV_PACKED_MAX_BYTES ((size_t)2147483584u) /* 2^31 - 64 */
LANCIUS_HIP_EXPORT size_t lancius_hip_conv2d_packed_bytes(size_t C_out, size_t C_in, size_t K_h, size_t K_w);
LANCIUS_HIP_EXPORT int lancius_hip_conv2d_pack_weight(lancius_hip_ctx* ctx, float* packed, const float* w,
                                                      size_t C_out, size_t C_in, size_t K_h, size_t K_w);
LANCIUS_HIP_EXPORT int lancius_hip_conv2d_packed_f32(lancius_hip_ctx* ctx, float* out, const float* in,
                                                     const float* packed, const float* bias, size_t N, size_t C_in,
                                                     size_t H, size_t W, size_t C_out, size_t K_h, size_t K_w,
                                                     size_t stride, size_t pad, int act);

/* Scaled-dot-product attention over [batch, S, H, D] row-major tensors
 * (row (b,i,h) starts at ((b*S + i)*H + h)*D).  causal != 0 masks keys
 * j > i exactly as lancius_kernels.c:307; scale multiplies q.k
 * (the reference uses 1/sqrt(D), :284).  batch = 1, causal = 1,
 * scale = 1/sqrt(D) is the reference kernel_attention (:278-332). */
LANCIUS_HIP_EXPORT int lancius_hip_attention_f32(lancius_hip_ctx* ctx, float* out,
                                                 const float* q, const float* k, const float* v,
                                                 size_t batch, size_t S, size_t H, size_t D,
                                                 int causal, float scale);

/* Same, for `count` independent [S,H,D] problems given by host arrays of
 * device pointers (count <= LANCIUS_HIP_MAX_GROUP). */
LANCIUS_HIP_EXPORT int lancius_hip_attention_grouped_f32(lancius_hip_ctx* ctx, size_t count, float* const* out,
                                                         const float* const* q, const float* const* k,
                                                         const float* const* v,
                                                         size_t S, size_t H, size_t D, int causal, float scale);

/* Row LayerNorm: two-pass mean and biased variance, then
 * (x - mean) * (1/sqrt(var + eps)) * gamma + beta (lancius_kernels.c:217-236). */
LANCIUS_HIP_EXPORT int lancius_hip_layernorm_f32(lancius_hip_ctx* ctx, float* out, const float* in,
                                                 const float* gamma, const float* beta,
                                                 size_t rows, size_t hidden, float eps);
/* `count` independent LayerNorms of one shape in one launch (the device
 * executor's launch for the LAYERNORM nodes of one scheduler wave, which
 * the reference runs one by one, lancius_scheduler.c:109-115); each member
 * has its own out, in, gamma and beta (count <= LANCIUS_HIP_MAX_GROUP).
 * Results equal lancius_hip_layernorm_f32's member by member. */
LANCIUS_HIP_EXPORT int lancius_hip_layernorm_grouped_f32(lancius_hip_ctx* ctx, size_t count, float* const* out,
                                                         const float* const* in, const float* const* gamma,
                                                         const float* const* beta, size_t rows, size_t hidden,
                                                         float eps);

/* Row softmax (max-subtracted, lancius_scheduler.c:284-294).  When argmax
 * is not NULL it receives int32 per row: the index of the first maximum of
 * the output probabilities, the strict '>' scan from -1e9 that the callers
 * run over a softmax output (B/examples/train_mnist.c:206-209,
 * B/examples/run_edge.c:82-88). */
LANCIUS_HIP_EXPORT int lancius_hip_softmax_f32(lancius_hip_ctx* ctx, float* probs, int32_t* argmax,
                                               const float* in, size_t rows, size_t cols);

/* Elementwise ops (lancius_scheduler.c:169-189, 268-278, 305-308;
 * lancius_kernels.c:238-246). */
LANCIUS_HIP_EXPORT int lancius_hip_add_f32(lancius_hip_ctx* ctx, float* out, const float* a, const float* b, size_t n);
LANCIUS_HIP_EXPORT int lancius_hip_relu_f32(lancius_hip_ctx* ctx, float* out, const float* a, size_t n);
LANCIUS_HIP_EXPORT int lancius_hip_gelu_f32(lancius_hip_ctx* ctx, float* out, const float* a, size_t n);
/* out = tanh(a) over n elements (BASIS_OP_TANH). */
LANCIUS_HIP_EXPORT int lancius_hip_tanh_f32(lancius_hip_ctx* ctx, float* out, const float* a, size_t n);
/* out[r,c] = act(a[r,c] + bias[c]) for a rows x cols matrix: BASIS_OP_BROADCAST_ADD
 * with the activation of a following RELU / TANH (act: LANCIUS_HIP_ACT_*). */
LANCIUS_HIP_EXPORT int lancius_hip_bias_act_f32(lancius_hip_ctx* ctx, float* out, const float* a, const float* bias,
                                                size_t rows, size_t cols, int act);
/* out[r,c] = row[c] for r < rows (row has `cols` values); with cols_in == 1
 * every element is row[0] (the scalar branch, lancius_scheduler.c:271-273). */
LANCIUS_HIP_EXPORT int lancius_hip_broadcast_f32(lancius_hip_ctx* ctx, float* out, const float* row,
                                                 size_t rows, size_t cols, size_t cols_in);
LANCIUS_HIP_EXPORT int lancius_hip_fill_f32(lancius_hip_ctx* ctx, float* out, float value, size_t n);
LANCIUS_HIP_EXPORT int lancius_hip_copy_f32(lancius_hip_ctx* ctx, float* out, const float* in, size_t n);

/* ---- the rest of the scheduler dispatch: training and reduction ops ---- */

/* out = a - b, out = a * b over n elements (lancius_scheduler.c:236-245). */
LANCIUS_HIP_EXPORT int lancius_hip_sub_f32(lancius_hip_ctx* ctx, float* out, const float* a, const float* b, size_t n);
LANCIUS_HIP_EXPORT int lancius_hip_mul_f32(lancius_hip_ctx* ctx, float* out, const float* a, const float* b, size_t n);
/* out = fwd > 0 ? grad : 0 (RELU_BWD, lancius_scheduler.c:279-283). */
LANCIUS_HIP_EXPORT int lancius_hip_relu_bwd_f32(lancius_hip_ctx* ctx, float* out, const float* grad,
                                                const float* fwd, size_t n);
/* out[c,r] = in[r,c] for an R x C input (TRANSPOSE, lancius_scheduler.c:246-250). */
LANCIUS_HIP_EXPORT int lancius_hip_transpose_f32(lancius_hip_ctx* ctx, float* out, const float* in,
                                                 size_t rows, size_t cols);
/* Sums with fp64 accumulation in a fixed order (bit-identical from run to
 * run), stored as fp32:
 *   sum:       out[0] = sum of n values (SUM, :251-256);
 *   sum_axis0: out[c] = sum over rows of in[r,c] (SUM_AXIS0, :257-262);
 *   sum_axis1: out[r] = sum over columns of in[r,c] (SUM_AXIS1, :263-267). */
LANCIUS_HIP_EXPORT int lancius_hip_sum_f32(lancius_hip_ctx* ctx, float* out, const float* in, size_t n);
LANCIUS_HIP_EXPORT int lancius_hip_sum_axis0_f32(lancius_hip_ctx* ctx, float* out, const float* in,
                                                 size_t rows, size_t cols);
LANCIUS_HIP_EXPORT int lancius_hip_sum_axis1_f32(lancius_hip_ctx* ctx, float* out, const float* in,
                                                 size_t rows, size_t cols);
/* out[r,c] = y[r,c] * (dy[r,c] - sum_c dy[r,c] y[r,c]) (SOFTMAX_BWD, :295-304). */
LANCIUS_HIP_EXPORT int lancius_hip_softmax_bwd_f32(lancius_hip_ctx* ctx, float* out, const float* dy,
                                                   const float* y, size_t rows, size_t cols);
/* Mean cross-entropy of row logits x against targets y (entries equal to
 * 1.0 select the class), returned as |loss| in out[0]
 * (CROSS_ENTROPY, lancius_scheduler.c:68-87, including the fabs of :85). */
LANCIUS_HIP_EXPORT int lancius_hip_cross_entropy_f32(lancius_hip_ctx* ctx, float* out, const float* x,
                                                     const float* y, size_t rows, size_t cols);
/* out[r,c] = (softmax(x)[r,c] - y[r,c]) * g[0] / rows, g a device scalar
 * (CROSS_ENTROPY_BWD, :89-104). */
LANCIUS_HIP_EXPORT int lancius_hip_cross_entropy_bwd_f32(lancius_hip_ctx* ctx, float* out, const float* x,
                                                         const float* y, const float* g, size_t rows, size_t cols);
/* Input gradient of conv2d: dx[N,C_in,H,W] = sum over (co,kh,kw) of
 * dy[N,C_out,H_out,W_out] * w[C_out,C_in,K_h,K_w] at ho*stride - pad + kh = h
 * (kernel_conv2d_bwd_in, lancius_kernels.c:62-91). */
LANCIUS_HIP_EXPORT int lancius_hip_conv2d_bwd_input_f32(lancius_hip_ctx* ctx, float* dx, const float* dy,
                                                        const float* w, size_t N, size_t C_in, size_t H, size_t W,
                                                        size_t C_out, size_t H_out, size_t W_out,
                                                        size_t K_h, size_t K_w, size_t stride, size_t pad);
/* Weight gradient of conv2d: dw[C_out,C_in,K_h,K_w] = sum over (n,ho,wo) of
 * dy[n,co,ho,wo] * x[n,ci,ho*stride-pad+kh,wo*stride-pad+kw]
 * (kernel_conv2d_bwd_w, lancius_kernels.c:93-136). */
LANCIUS_HIP_EXPORT int lancius_hip_conv2d_bwd_weight_f32(lancius_hip_ctx* ctx, float* dw, const float* dy,
                                                         const float* x, size_t N, size_t C_in, size_t H, size_t W,
                                                         size_t C_out, size_t H_out, size_t W_out,
                                                         size_t K_h, size_t K_w, size_t stride, size_t pad);
/* Max pooling, K x K window, no padding, H_out = (H - K)/stride + 1; the
 * running maximum starts at -1e9 with a strict '>' (MAXPOOL2D,
 * lancius_vision_ops.c:82-112). */
LANCIUS_HIP_EXPORT int lancius_hip_maxpool2d_f32(lancius_hip_ctx* ctx, float* out, const float* in, size_t N,
                                                 size_t C, size_t H, size_t W, size_t K, size_t stride);
/* Its gradient: each dy value goes to the first maximum of its window
 * (position (0,0) of the plane when no value exceeds -1e9), contributions
 * summed (MAXPOOL2D_BWD, lancius_vision_ops.c:149-190).  H_out, W_out are
 * dy's spatial size. */
LANCIUS_HIP_EXPORT int lancius_hip_maxpool2d_bwd_f32(lancius_hip_ctx* ctx, float* dx, const float* dy,
                                                     const float* x, size_t N, size_t C, size_t H, size_t W,
                                                     size_t H_out, size_t W_out, size_t K, size_t stride);

/* ---- decode-side attention family ----------------------------------- */

/* Attention with grouped K/V heads and a key sequence that may be longer
 * than the query sequence: q/out [batch, S_q, H_q, D], k/v [batch, S_kv,
 * H_kv, D]; query head h reads K/V head h / (H_q / H_kv); causal lets query
 * i see keys j <= i + (S_kv - S_q) (masked with the reference's -1e9
 * semantics, lancius_kernels.c:307,428).  S_kv == S_q, causal, scale
 * 1/sqrt(D) is kernel_gqa (lancius_kernels.c:407-448; the GQA node,
 * lancius_scheduler.c:146-152); S_kv > S_q is the prefill-with-history case
 * the reference's q-length-only loop cannot express. */
LANCIUS_HIP_EXPORT int lancius_hip_attention_gqa_f32(lancius_hip_ctx* ctx, float* out, const float* q,
                                                     const float* k, const float* v, size_t batch, size_t S_q,
                                                     size_t S_kv, size_t H_q, size_t H_kv, size_t D, int causal,
                                                     float scale);
/* One new query token per sequence against its K/V cache:
 * q/out [batch, H_q, D], k_cache/v_cache [batch, S_kv, H_kv, D]; sequence b
 * uses keys [0, kv_lens[b]) (kv_lens NULL: all S_kv).  No mask (every cached
 * key precedes the query).  batch 1, H_q == H_kv, scale 1/sqrt(D) is
 * kernel_attention_kv_cache (lancius_kernels.c:338-379).  D <= 128,
 * H_q / H_kv <= 64.  Split-KV: partials in the context workspace, combined
 * in a fixed order. */
LANCIUS_HIP_EXPORT int lancius_hip_attention_decode_f32(lancius_hip_ctx* ctx, float* out, const float* q,
                                                        const float* k_cache, const float* v_cache,
                                                        const int32_t* kv_lens, size_t batch, size_t S_kv,
                                                        size_t H_q, size_t H_kv, size_t D, float scale);
/* out = x * (1/sqrt(mean(x^2) + eps)) * gamma per row (kernel_rmsnorm,
 * lancius_kernels.c:381-396; the RMSNORM node uses eps 1e-5). */
LANCIUS_HIP_EXPORT int lancius_hip_rmsnorm_f32(lancius_hip_ctx* ctx, float* out, const float* in, const float* gamma,
                                               size_t rows, size_t hidden, float eps);
/* out = gate / (1 + exp(-gate)) * up (kernel_swiglu, lancius_kernels.c:398-405). */
LANCIUS_HIP_EXPORT int lancius_hip_swiglu_f32(lancius_hip_ctx* ctx, float* out, const float* gate, const float* up,
                                              size_t n);
/* Rotary embedding of `count` consecutive [batch, S, H, head_dim] tensors
 * (kernel_rope, lancius_kernels.c:248-272): pair (d, d+1) at position
 * s + pos_offset rotates by (s + pos_offset) / 10000^(d / head_dim).  The
 * ROPE node (lancius_scheduler.c:153-165) is count 2 (its q and k halves),
 * batch 1, head_dim = shape[2] / 2, pos_offset 0.  out may equal in. */
LANCIUS_HIP_EXPORT int lancius_hip_rope_f32(lancius_hip_ctx* ctx, float* out, const float* in, size_t count,
                                            size_t batch, size_t S, size_t H, size_t head_dim, int pos_offset);

/* ---- the int8 path (v_mfma_i32_32x32x32_i8) -------------------------- */

/* Per-tensor symmetric quantization, the reference's formula
 * (lancius_scheduler.c:199-204, lancius_vision_ops.c:28-36,
 * lancius_quantize.c:14-25): scale = max|x| / 127 (1e-8 for an all-zero
 * tensor), q[i] = (int8) round(x[i] / scale) in fp64, round half away from
 * zero.  `scale` is a DEVICE pointer to one double. */
LANCIUS_HIP_EXPORT int lancius_hip_quantize_i8(lancius_hip_ctx* ctx, int8_t* q, double* scale, const float* x,
                                               size_t n);
/* C[M,N] = epilogue((double) sum_k qa[m,k] * B[k,n] * scale_a * scale_b) with
 * qa the dynamic per-tensor quantization of the fp32 A and B an int8 [K,N]
 * matrix of scale scale_b: the int8 MATMUL branch
 * (lancius_scheduler.c:195-220); int32 accumulation, exact.  Epilogue as
 * lancius_hip_gemm_f32 (bias, act, residual; all may be NULL / NONE). */
LANCIUS_HIP_EXPORT int lancius_hip_gemm_i8_f32(lancius_hip_ctx* ctx, float* C, const float* A, const int8_t* B,
                                               double scale_b, size_t M, size_t K, size_t N,
                                               const float* bias, int act, const float* residual);
/* The same product split in two for a weight used many times: the reference
 * walks b_int8 [K,N] column by column inside the product
 * (lancius_scheduler.c:210-215); the device re-lays it once into the
 * k-contiguous layout its int8 matrix cores read (B^T [N, Kp], k zero-padded
 * to a multiple of 128: lancius_hip_i8_packed_bytes(K, N) bytes), and
 * lancius_hip_gemm_i8p_f32 takes that packed copy in place of B.  Results are
 * bit-identical to lancius_hip_gemm_i8_f32.  The device executor keeps one
 * packed copy per int8 weight and re-packs it after an upload. */
LANCIUS_HIP_EXPORT size_t lancius_hip_i8_packed_bytes(size_t K, size_t N);
LANCIUS_HIP_EXPORT int lancius_hip_i8_pack_weight(lancius_hip_ctx* ctx, int8_t* packed, const int8_t* B, size_t K,
                                                  size_t N);
LANCIUS_HIP_EXPORT int lancius_hip_gemm_i8p_f32(lancius_hip_ctx* ctx, float* C, const float* A,
                                                const int8_t* packed, double scale_b, size_t M, size_t K, size_t N,
                                                const float* bias, int act, const float* residual);
/* conv2d with int8 OIHW weights of scale scale_w and the fp32 NCHW input
 * quantized per tensor on the fly: kernel_conv2d_int8_fwd
 * (lancius_kernels.c:177-210) as routed by lancius_vision_ops.c:16-57;
 * act = LANCIUS_HIP_ACT_RELU is the fused Conv+ReLU (:49-54).  bias may be
 * NULL (the reference has none). */
LANCIUS_HIP_EXPORT int lancius_hip_conv2d_i8_f32(lancius_hip_ctx* ctx, float* out, const float* in, const int8_t* w,
                                                 double scale_w, const float* bias,
                                                 size_t N, size_t C_in, size_t H, size_t W,
                                                 size_t C_out, size_t K_h, size_t K_w,
                                                 size_t stride, size_t pad, int act);

/* ---- streams and HIP graphs ------------------------------------------ */

/* A context on a new non-blocking stream of default priority, owned by the
 * context (destroyed with it). */
LANCIUS_HIP_EXPORT int lancius_hip_ctx_create_own_stream(int device, lancius_hip_ctx** out);
/* Device index of a context (-1 for NULL). */
LANCIUS_HIP_EXPORT int lancius_hip_ctx_device(const lancius_hip_ctx* ctx);
/* The hipStream_t a context enqueues on (NULL: the null stream). */
LANCIUS_HIP_EXPORT void* lancius_hip_ctx_stream(const lancius_hip_ctx* ctx);
/* Work enqueued on `waiter` after this call starts only after everything
 * enqueued on `signaler` before it (an event recorded and waited). */
LANCIUS_HIP_EXPORT int lancius_hip_stream_wait(lancius_hip_ctx* waiter, lancius_hip_ctx* signaler);

typedef struct lancius_hip_graph lancius_hip_graph;
/* Record every launch enqueued on ctx between begin and end into a graph
 * instead of running it (ctx must own a stream: the null stream cannot be
 * captured).  Launches that allocate (first use of a workspace) must have
 * run once before capture. */
LANCIUS_HIP_EXPORT int lancius_hip_capture_begin(lancius_hip_ctx* ctx);
LANCIUS_HIP_EXPORT int lancius_hip_capture_end(lancius_hip_ctx* ctx, lancius_hip_graph** out);
LANCIUS_HIP_EXPORT int lancius_hip_graph_launch(lancius_hip_graph* graph, lancius_hip_ctx* ctx);
LANCIUS_HIP_EXPORT void lancius_hip_graph_destroy(lancius_hip_graph* graph);

/* ---- fused small-batch MLP ------------------------------------------- */

/* out = softmax(act1(x . W1 + b1) . W2 + b2) row by row (softmax != 0, with
 * the first-maximum argmax when argmax != NULL), or the logits y when
 * softmax == 0, in one launch (workgroups own 16x16 tiles of the hidden
 * layer over the whole K1 and hand their share of the second layer to the
 * last-arriving workgroup of each 16-row block): the MATMUL -> BROADCAST+ADD
 * -> RELU|GELU|TANH -> MATMUL -> BROADCAST+ADD -> SOFTMAX chain of
 * lancius_scheduler.c:169-233, 284-308 for small batches, whose unfused form
 * (five launches) is bound by its launch count.  x [M][K1], W1 [K1][N1],
 * W2 [N1][N2], out [M][N2]; b1, b2 may be NULL.  Limits: M <= 64, N2 <= 64,
 * M*N1 <= 16384, N1*N2 <= 8192, K1*max(M, N1) <= 2^28 (else -3).  Results
 * equal the unfused
 * launches up to fp32 summation order; repeated calls give identical bits.
 * Uses the context's workspace and arrival counters, so calls on one context
 * are ordered by its stream. */
LANCIUS_HIP_EXPORT int lancius_hip_mlp2_f32(lancius_hip_ctx* ctx, float* out, int32_t* argmax, const float* x,
                                            const float* w1, const float* b1, int act1, const float* w2,
                                            const float* b2, size_t M, size_t K1, size_t N1, size_t N2, int softmax);
/* The same with an activation on the second layer too: y = act2(h . W2 +
 * b2) before the softmax or the store (the BASIS graph's MATMUL ->
 * BROADCAST_ADD -> RELU|TANH -> MATMUL -> BROADCAST_ADD -> RELU|TANH). */
LANCIUS_HIP_EXPORT int lancius_hip_mlp2_ex_f32(lancius_hip_ctx* ctx, float* out, int32_t* argmax, const float* x,
                                               const float* w1, const float* b1, int act1, const float* w2,
                                               const float* b2, int act2, size_t M, size_t K1, size_t N1, size_t N2,
                                               int softmax);

/* ---- model-file tensors to HBM -------------------------------------- */

/* Element codes of lancius_hip_file_tensor (the lancius_dtype numbers,
 * bleeding/v11A1/include/lancius/lancius_types.h:9-14). */
#define LANCIUS_HIP_FILE_F64 0
#define LANCIUS_HIP_FILE_I8  1
#define LANCIUS_HIP_FILE_F32 2

/* One tensor stored in a file: `elements` values of `file_dtype` starting at
 * byte `file_offset`, to land in device memory `dst` as `dst_dtype`:
 *   F64 -> F32  rounded to nearest on the device;
 *   F32 -> F32, I8 -> I8  copied;
 *   I8  -> F32  dequantized, (float)(q * scale) with the product in fp64. */
typedef struct {
    void* dst;
    int dst_dtype;
    int file_dtype;
    uint64_t file_offset;
    uint64_t elements;
    double scale;
} lancius_hip_file_tensor;

/* Streams the tensors from `path` straight into device memory: the file is
 * read in 16 MiB pieces into two pinned host buffers, each piece is copied
 * to the device while the next is read, and conversions run on the device
 * (no host fp64/fp32 copy of a tensor is made).  Returns when every tensor
 * is in place.  Checks every extent against the file size first.  No
 * reference counterpart: the reference reads weights into host fp64 buffers
 * (lancius_serialize.c:221-240). */
LANCIUS_HIP_EXPORT int lancius_hip_upload_file(lancius_hip_ctx* ctx, const char* path, size_t count,
                                               const lancius_hip_file_tensor* tensors);

/* ---- diagnostics ---------------------------------------------------- */

/* Measured ceilings of this device, for roofline reporting:
 *   which = 0: fp32 matrix rate, TFLOP/s (independent back-to-back
 *              v_mfma_f32_32x32x2_f32 on every SIMD, no memory traffic);
 *   which = 1: HBM copy bandwidth, GB/s (float4 copy of 1 GiB into another
 *              1 GiB, bytes read + written);
 *   which = 2: HBM read bandwidth, GB/s (float4 reads of 1 GiB).
 * Allocates and frees its own buffers; takes a few hundred milliseconds. */
LANCIUS_HIP_EXPORT int lancius_hip_peak_probe(lancius_hip_ctx* ctx, int which, double* result);

/* ---- reference-ABI bridge ------------------------------------------- */

/* The fp32 matmul that the reference declares but never defines
 * (bleeding/v11A1/include/lancius/lancius_kernels.h:55).  HOST pointers,
 * row-major out[M,N] = a[M,K] . b[K,N]; stages through the device of a
 * process-wide default context (device 0, null stream) and returns when
 * `out` holds the result.  Failures are reported by
 * lancius_hip_last_status() (void return, as declared by the reference). */
LANCIUS_HIP_EXPORT void kernel_matmul_f32(float* out, const float* a, const float* b, size_t M, size_t K, size_t N);
LANCIUS_HIP_EXPORT int lancius_hip_last_status(void);

#ifdef __cplusplus
}
#endif

#endif /* LANCIUS_HIP_H */
