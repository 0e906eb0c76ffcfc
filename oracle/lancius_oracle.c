/*
 * lancius_oracle.c - TEST INFRASTRUCTURE ONLY (see lancius_oracle.h).
 *
 * fp64 CPU restatement of the reference hot path.  Paths are relative to the
 * reference root; B/ = bleeding/v11A1/.  Loop order and accumulation follow
 * the cited reference code so the results agree with the compiled reference
 * to rounding (the golden fixtures check this).
 */
#include "lancius_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

#define ORACLE_OWNED (1u << 8) /* rt->flags bit: buffer malloc'd by this executor */

void oracle_set_threads(int n) {
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
#else
    (void)n;
#endif
}

/* B/src/runtime/lancius_scheduler.c:222-234: zero the output, then for each
 * row r and k, out[r, :] += a[r, k] * b[k, :] (single-threaded in the
 * reference; rows are independent, so splitting rows over threads gives the
 * same numbers). */
void oracle_matmul_rows(double* out, const double* a, const double* b, size_t M, size_t K, size_t N, size_t r0,
                        size_t r1) {
    if (r1 > M) r1 = M;
#pragma omp parallel for schedule(static)
    for (long long rr = (long long)r0; rr < (long long)r1; rr++) {
        const size_t r = (size_t)rr;
        double* o = out + r * N;
        memset(o, 0, N * sizeof(double));
        for (size_t k = 0; k < K; k++) {
            const double av = a[r * K + k];
            const double* br = b + k * N;
            for (size_t c = 0; c < N; c++) o[c] += av * br[c];
        }
    }
}

/* B/src/math/lancius_kernels.c:28-60 (and the ReLU variant :140-173): direct
 * cross-correlation, taps outside the image skipped (:156-158), ReLU applied
 * on store (:168).  Parallel over (image, output channel) like the reference
 * (:147). */
void oracle_conv2d(double* out, const double* in, const double* w, size_t N, size_t C_in, size_t H, size_t W,
                   size_t C_out, size_t K_h, size_t K_w, size_t stride, size_t pad, int relu, size_t n0, size_t n1) {
    const size_t Ho = (H + 2 * pad - K_h) / stride + 1;
    const size_t Wo = (W + 2 * pad - K_w) / stride + 1;
    if (n1 > N) n1 = N;
#pragma omp parallel for collapse(2) schedule(static)
    for (long long ni = (long long)n0; ni < (long long)n1; ni++) {
        for (long long co = 0; co < (long long)C_out; co++) {
            for (size_t ho = 0; ho < Ho; ho++) {
                for (size_t wo = 0; wo < Wo; wo++) {
                    double sum = 0.0;
                    for (size_t ci = 0; ci < C_in; ci++) {
                        for (size_t kh = 0; kh < K_h; kh++) {
                            for (size_t kw = 0; kw < K_w; kw++) {
                                const long ih = (long)(ho * stride) - (long)pad + (long)kh;
                                const long iw = (long)(wo * stride) - (long)pad + (long)kw;
                                if (ih >= 0 && ih < (long)H && iw >= 0 && iw < (long)W) {
                                    sum += in[(size_t)ni * (C_in * H * W) + ci * (H * W) + (size_t)ih * W + (size_t)iw] *
                                           w[(size_t)co * (C_in * K_h * K_w) + ci * (K_h * K_w) + kh * K_w + kw];
                                }
                            }
                        }
                    }
                    out[(size_t)ni * (C_out * Ho * Wo) + (size_t)co * (Ho * Wo) + ho * Wo + wo] =
                        relu ? (sum > 0.0 ? sum : 0.0) : sum;
                }
            }
        }
    }
}

/* B/src/math/lancius_kernels.c:278-332 with a batch loop and a causal switch:
 * for each (i, h): m = -1e9, l = 0, o = 0; for every key j, s = (q.k)*scale,
 * causal keys j > i get s = -1e9 (:307); m' = max(m, s), c = exp(m - m'),
 * p = exp(s - m'), l = l*c + p, o = o*c + p*v (:309-319); out = o / l.
 * Masked keys are still visited, as in the reference. */
void oracle_attention(double* out, const double* q, const double* k, const double* v, size_t batch, size_t S,
                      size_t H, size_t D, int causal, double scale, size_t b0, size_t b1, size_t i0, size_t i1) {
    if (b1 > batch) b1 = batch;
    if (i1 > S) i1 = S;
#pragma omp parallel
    {
        double* o = (double*)calloc(D ? D : 1, sizeof(double));
#pragma omp for collapse(3) schedule(static)
        for (long long b = (long long)b0; b < (long long)b1; b++) {
            for (long long ii = (long long)i0; ii < (long long)i1; ii++) {
                for (long long h = 0; h < (long long)H; h++) {
                    const size_t i = (size_t)ii;
                    const size_t base = (size_t)b * S * H * D;
                    const double* qr = q + base + i * H * D + (size_t)h * D;
                    double m = -1e9, l = 0.0;
                    memset(o, 0, D * sizeof(double));
                    for (size_t j = 0; j < S; j++) {
                        const double* kr = k + base + j * H * D + (size_t)h * D;
                        const double* vr = v + base + j * H * D + (size_t)h * D;
                        double s = 0.0;
                        for (size_t d = 0; d < D; d++) s += qr[d] * kr[d];
                        s *= scale;
                        if (causal && j > i) s = -1e9;
                        const double mn = s > m ? s : m;
                        const double c = exp(m - mn);
                        const double p = exp(s - mn);
                        l = l * c + p;
                        for (size_t d = 0; d < D; d++) o[d] = o[d] * c + p * vr[d];
                        m = mn;
                    }
                    double* orow = out + base + i * H * D + (size_t)h * D;
                    const double inv = 1.0 / l;
                    for (size_t d = 0; d < D; d++) orow[d] = o[d] * inv;
                }
            }
        }
        free(o);
    }
}

/* B/src/math/lancius_kernels.c:217-236: mean, biased variance of (x - mean),
 * y = (x - mean) * (1/sqrt(var + eps)) * gamma + beta. */
void oracle_layernorm(double* out, const double* in, const double* gamma, const double* beta, size_t rows,
                      size_t hidden, double eps) {
    for (size_t r = 0; r < rows; r++) {
        const double* x = in + r * hidden;
        double* y = out + r * hidden;
        double mean = 0.0;
        for (size_t i = 0; i < hidden; i++) mean += x[i];
        mean /= (double)hidden;
        double var = 0.0;
        for (size_t i = 0; i < hidden; i++) var += (x[i] - mean) * (x[i] - mean);
        var /= (double)hidden;
        const double inv_std = 1.0 / sqrt(var + eps);
        for (size_t i = 0; i < hidden; i++) y[i] = (x[i] - mean) * inv_std * gamma[i] + beta[i];
    }
}

/* B/src/math/lancius_kernels.c:238-246: clamp to [-100, 100], then the tanh
 * approximation 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))). */
void oracle_gelu(double* out, const double* in, size_t n) {
    const double k0 = 0.7978845608028654;
    for (size_t i = 0; i < n; i++) {
        double x = in[i];
        if (x > 100.0) x = 100.0;
        if (x < -100.0) x = -100.0;
        out[i] = 0.5 * x * (1.0 + tanh(k0 * (x + 0.044715 * x * x * x)));
    }
}

/* B/src/runtime/lancius_scheduler.c:284-294. */
void oracle_softmax(double* out, const double* in, size_t rows, size_t cols) {
    for (size_t r = 0; r < rows; r++) {
        const double* a = in + r * cols;
        double* y = out + r * cols;
        double mx = a[0];
        for (size_t c = 1; c < cols; c++)
            if (a[c] > mx) mx = a[c];
        double sum = 0.0;
        for (size_t c = 0; c < cols; c++) {
            y[c] = exp(a[c] - mx);
            sum += y[c];
        }
        for (size_t c = 0; c < cols; c++) y[c] /= sum;
    }
}

/* B/examples/train_mnist.c:206-209: pred = 0, best = -1e9, strict '>'. */
void oracle_argmax(int32_t* idx, const double* in, size_t rows, size_t cols) {
    for (size_t r = 0; r < rows; r++) {
        int32_t pred = 0;
        double best = -1e9;
        for (size_t c = 0; c < cols; c++)
            if (in[r * cols + c] > best) {
                best = in[r * cols + c];
                pred = (int32_t)c;
            }
        idx[r] = pred;
    }
}

/* B/src/runtime/lancius_scheduler.c:188 */
void oracle_add(double* out, const double* a, const double* b, size_t n) {
    for (size_t k = 0; k < n; k++) out[k] = a[k] + b[k];
}

/* B/src/runtime/lancius_scheduler.c:307 (NaN maps to 0) */
void oracle_relu(double* out, const double* a, size_t n) {
    for (size_t k = 0; k < n; k++) out[k] = a[k] > 0.0 ? a[k] : 0.0;
}

/* B/src/runtime/lancius_scheduler.c:268-278 */
void oracle_broadcast(double* out, const double* a, size_t a_elems, size_t rows, size_t cols) {
    if (a_elems == 1) {
        for (size_t k = 0; k < rows * cols; k++) out[k] = a[0];
    } else {
        for (size_t r = 0; r < rows; r++)
            for (size_t c = 0; c < cols; c++) out[r * cols + c] = a[c];
    }
}

/* ---- the rest of the scheduler dispatch (training and reduction ops) ---------- */

/* B/src/runtime/lancius_scheduler.c:241-245 */
void oracle_sub(double* out, const double* a, const double* b, size_t n) {
    for (size_t k = 0; k < n; k++) out[k] = a[k] - b[k];
}

/* B/src/runtime/lancius_scheduler.c:236-240 */
void oracle_mul(double* out, const double* a, const double* b, size_t n) {
    for (size_t k = 0; k < n; k++) out[k] = a[k] * b[k];
}

/* B/src/runtime/lancius_scheduler.c:279-283: the forward input decides. */
void oracle_relu_bwd(double* out, const double* grad, const double* fwd, size_t n) {
    for (size_t k = 0; k < n; k++) out[k] = fwd[k] > 0.0 ? grad[k] : 0.0;
}

/* B/src/runtime/lancius_scheduler.c:246-250 */
void oracle_transpose(double* out, const double* a, size_t rows, size_t cols) {
    for (size_t r = 0; r < rows; r++)
        for (size_t c = 0; c < cols; c++) out[c * rows + r] = a[r * cols + c];
}

/* B/src/runtime/lancius_scheduler.c:251-256 */
void oracle_sum(double* out, const double* a, size_t n) {
    double s = 0.0;
    for (size_t k = 0; k < n; k++) s += a[k];
    out[0] = s;
}

/* B/src/runtime/lancius_scheduler.c:257-262 */
void oracle_sum_axis0(double* out, const double* a, size_t rows, size_t cols) {
    for (size_t c = 0; c < cols; c++) out[c] = 0.0;
    for (size_t r = 0; r < rows; r++)
        for (size_t c = 0; c < cols; c++) out[c] += a[r * cols + c];
}

/* B/src/runtime/lancius_scheduler.c:263-267 */
void oracle_sum_axis1(double* out, const double* a, size_t rows, size_t cols) {
    for (size_t r = 0; r < rows; r++) {
        double s = 0.0;
        for (size_t c = 0; c < cols; c++) s += a[r * cols + c];
        out[r] = s;
    }
}

/* B/src/runtime/lancius_scheduler.c:295-304 */
void oracle_softmax_bwd(double* out, const double* dy, const double* y, size_t rows, size_t cols) {
    for (size_t r = 0; r < rows; r++) {
        double dot = 0.0;
        for (size_t c = 0; c < cols; c++) dot += dy[r * cols + c] * y[r * cols + c];
        for (size_t c = 0; c < cols; c++) out[r * cols + c] = y[r * cols + c] * (dy[r * cols + c] - dot);
    }
}

/* Row maximum (first element, then strict '>') and sum of exp(x - max), as
 * B/src/runtime/lancius_scheduler.c:74-77 and :95-98 compute them. */
static void row_max_sumexp(const double* x, size_t cols, double* mx, double* se) {
    double m = x[0];
    for (size_t c = 1; c < cols; c++)
        if (x[c] > m) m = x[c];
    double s = 0.0;
    for (size_t c = 0; c < cols; c++) s += exp(x[c] - m);
    *mx = m;
    *se = s;
}

/* B/src/runtime/lancius_scheduler.c:68-87 (the fabs of :85 included) */
void oracle_cross_entropy(double* out, const double* x, const double* y, size_t rows, size_t cols) {
    double total = 0.0;
    for (size_t r = 0; r < rows; r++) {
        double m, se;
        row_max_sumexp(x + r * cols, cols, &m, &se);
        const double lse = log(se) + m;
        for (size_t c = 0; c < cols; c++)
            if (y[r * cols + c] == 1.0) total -= x[r * cols + c] - lse;
    }
    out[0] = fabs(total / (double)rows);
}

/* B/src/runtime/lancius_scheduler.c:89-104 */
void oracle_cross_entropy_bwd(double* out, const double* x, const double* y, const double* g, size_t rows,
                              size_t cols) {
    const double scale = g[0] / (double)rows;
    for (size_t r = 0; r < rows; r++) {
        double m, se;
        row_max_sumexp(x + r * cols, cols, &m, &se);
        for (size_t c = 0; c < cols; c++)
            out[r * cols + c] = (exp(x[r * cols + c] - m) / se - y[r * cols + c]) * scale;
    }
}

/* B/src/math/lancius_kernels.c:62-91: scatter of every dy value through
 * the filter taps that produced it. */
void oracle_conv2d_bwd_input(double* dx, const double* dy, const double* w, size_t N, size_t C_in, size_t H,
                             size_t W, size_t C_out, size_t Ho, size_t Wo, size_t K_h, size_t K_w, size_t stride,
                             size_t pad) {
    memset(dx, 0, N * C_in * H * W * sizeof(double));
#pragma omp parallel for schedule(static)
    for (size_t n = 0; n < N; n++)
        for (size_t co = 0; co < C_out; co++)
            for (size_t ho = 0; ho < Ho; ho++)
                for (size_t wo = 0; wo < Wo; wo++) {
                    const double g = dy[((n * C_out + co) * Ho + ho) * Wo + wo];
                    for (size_t ci = 0; ci < C_in; ci++)
                        for (size_t kh = 0; kh < K_h; kh++)
                            for (size_t kw = 0; kw < K_w; kw++) {
                                const long ih = (long)(ho * stride) - (long)pad + (long)kh;
                                const long iw = (long)(wo * stride) - (long)pad + (long)kw;
                                if (ih < 0 || ih >= (long)H || iw < 0 || iw >= (long)W) continue;
                                dx[((n * C_in + ci) * H + (size_t)ih) * W + (size_t)iw] +=
                                    g * w[((co * C_in + ci) * K_h + kh) * K_w + kw];
                            }
                }
}

/* B/src/math/lancius_kernels.c:93-136, one accumulator (the reference's
 * per-thread partials are summed in thread order; the terms are the same). */
void oracle_conv2d_bwd_weight(double* dw, const double* dy, const double* x, size_t N, size_t C_in, size_t H,
                              size_t W, size_t C_out, size_t Ho, size_t Wo, size_t K_h, size_t K_w, size_t stride,
                              size_t pad) {
    memset(dw, 0, C_out * C_in * K_h * K_w * sizeof(double));
#pragma omp parallel for schedule(static)
    for (size_t co = 0; co < C_out; co++)
        for (size_t n = 0; n < N; n++)
            for (size_t ho = 0; ho < Ho; ho++)
                for (size_t wo = 0; wo < Wo; wo++) {
                    const double g = dy[((n * C_out + co) * Ho + ho) * Wo + wo];
                    for (size_t ci = 0; ci < C_in; ci++)
                        for (size_t kh = 0; kh < K_h; kh++)
                            for (size_t kw = 0; kw < K_w; kw++) {
                                const long ih = (long)(ho * stride) - (long)pad + (long)kh;
                                const long iw = (long)(wo * stride) - (long)pad + (long)kw;
                                if (ih < 0 || ih >= (long)H || iw < 0 || iw >= (long)W) continue;
                                dw[((co * C_in + ci) * K_h + kh) * K_w + kw] +=
                                    g * x[((n * C_in + ci) * H + (size_t)ih) * W + (size_t)iw];
                            }
                }
}

/* B/src/runtime/lancius_vision_ops.c:82-112 */
void oracle_maxpool2d(double* out, const double* in, size_t N, size_t C, size_t H, size_t W, size_t K,
                      size_t stride) {
    const size_t Ho = (H - K) / stride + 1, Wo = (W - K) / stride + 1;
    for (size_t p = 0; p < N * C; p++)
        for (size_t ho = 0; ho < Ho; ho++)
            for (size_t wo = 0; wo < Wo; wo++) {
                double m = -1e9;
                for (size_t kh = 0; kh < K; kh++)
                    for (size_t kw = 0; kw < K; kw++) {
                        const double v = in[(p * H + ho * stride + kh) * W + wo * stride + kw];
                        if (v > m) m = v;
                    }
                out[(p * Ho + ho) * Wo + wo] = m;
            }
}

/* B/src/runtime/lancius_vision_ops.c:149-190: each dy value is added at the
 * first maximum of its window, (0,0) of the plane when none beats -1e9. */
void oracle_maxpool2d_bwd(double* dx, const double* dy, const double* x, size_t N, size_t C, size_t H, size_t W,
                          size_t Ho, size_t Wo, size_t K, size_t stride) {
    memset(dx, 0, N * C * H * W * sizeof(double));
    for (size_t p = 0; p < N * C; p++)
        for (size_t ho = 0; ho < Ho; ho++)
            for (size_t wo = 0; wo < Wo; wo++) {
                double m = -1e9;
                size_t at_h = 0, at_w = 0;
                for (size_t kh = 0; kh < K; kh++)
                    for (size_t kw = 0; kw < K; kw++) {
                        const size_t ih = ho * stride + kh, iw = wo * stride + kw;
                        if (x[(p * H + ih) * W + iw] > m) {
                            m = x[(p * H + ih) * W + iw];
                            at_h = ih;
                            at_w = iw;
                        }
                    }
                dx[(p * H + at_h) * W + at_w] += dy[(p * Ho + ho) * Wo + wo];
            }
}

/* ---- decode-side attention family ------------------------------------------------ */

/* B/src/math/lancius_kernels.c:381-396 */
void oracle_rmsnorm(double* out, const double* in, const double* gamma, size_t rows, size_t hidden, double eps) {
    for (size_t i = 0; i < rows; i++) {
        const double* x = in + i * hidden;
        double sq = 0.0;
        for (size_t j = 0; j < hidden; j++) sq += x[j] * x[j];
        const double inv = 1.0 / sqrt(sq / (double)hidden + eps);
        for (size_t j = 0; j < hidden; j++) out[i * hidden + j] = (x[j] * inv) * gamma[j];
    }
}

/* B/src/math/lancius_kernels.c:398-405 */
void oracle_swiglu(double* out, const double* gate, const double* up, size_t n) {
    for (size_t i = 0; i < n; i++) out[i] = gate[i] / (1.0 + exp(-gate[i])) * up[i];
}

/* B/src/math/lancius_kernels.c:248-272 applied to `count` consecutive
 * [batch, S, H, hd] tensors (in place when out == in). */
void oracle_rope(double* out, const double* in, size_t count, size_t batch, size_t S, size_t H, size_t hd,
                 int pos_offset) {
    const size_t tensor = batch * S * H * hd;
    if (out != in) memcpy(out, in, count * tensor * sizeof(double));
    for (size_t t = 0; t < count; t++)
        for (size_t b = 0; b < batch; b++)
            for (size_t s = 0; s < S; s++) {
                const int pos = (int)s + pos_offset;
                for (size_t h = 0; h < H; h++)
                    for (size_t d = 0; d < hd; d += 2) {
                        const double freq = 1.0 / pow(10000.0, (double)d / (double)hd);
                        const double angle = pos * freq;
                        const double c = cos(angle), sn = sin(angle);
                        double* x = out + t * tensor + ((b * S + s) * H + h) * hd + d;
                        const double x0 = x[0], x1 = x[1];
                        x[0] = x0 * c - x1 * sn;
                        x[1] = x0 * sn + x1 * c;
                    }
            }
}

/* B/src/math/lancius_kernels.c:407-448 (kernel_gqa: causal, -1e9 masking,
 * online softmax), generalised to a batch and to S_kv >= S_q keys, query i
 * seeing keys j <= i + (S_kv - S_q) when causal.  S_kv == S_q, batch 1,
 * causal, scale 1/sqrt(D) is the reference kernel. */
void oracle_attention_gqa(double* out, const double* q, const double* k, const double* v, size_t batch, size_t Sq,
                          size_t Skv, size_t Hq, size_t Hkv, size_t D, int causal, double scale) {
    const size_t group = Hq / Hkv;
    const long off = (long)Skv - (long)Sq;
#pragma omp parallel for collapse(2) schedule(static)
    for (size_t b = 0; b < batch; b++)
        for (size_t i = 0; i < Sq; i++) {
            double* o = (double*)calloc(D, sizeof(double));
            for (size_t hq = 0; hq < Hq; hq++) {
                const size_t hk = hq / group;
                const double* qr = q + ((b * Sq + i) * Hq + hq) * D;
                double m = -1e9, l = 0.0;
                for (size_t d = 0; d < D; d++) o[d] = 0.0;
                for (size_t j = 0; j < Skv; j++) {
                    const double* kr = k + ((b * Skv + j) * Hkv + hk) * D;
                    const double* vr = v + ((b * Skv + j) * Hkv + hk) * D;
                    double s = 0.0;
                    for (size_t d = 0; d < D; d++) s += qr[d] * kr[d];
                    s *= scale;
                    if (causal && (long)j > (long)i + off) s = -1e9;
                    const double m_new = s > m ? s : m;
                    const double corr = exp(m - m_new), pj = exp(s - m_new);
                    l = l * corr + pj;
                    for (size_t d = 0; d < D; d++) o[d] = o[d] * corr + pj * vr[d];
                    m = m_new;
                }
                double* orow = out + ((b * Sq + i) * Hq + hq) * D;
                for (size_t d = 0; d < D; d++) orow[d] = o[d] / l;
            }
            free(o);
        }
}

/* B/src/math/lancius_kernels.c:338-379 (kernel_attention_kv_cache: scores
 * against every cached key, max from -1e9, softmax, weighted V), for a batch
 * of sequences with their own cache lengths (lens NULL: all S_kv) and K/V
 * heads shared by groups of query heads.  A sequence with no keys gives 0. */
void oracle_attention_decode(double* out, const double* q, const double* k, const double* v, const int32_t* lens,
                             size_t batch, size_t Skv, size_t Hq, size_t Hkv, size_t D, double scale) {
    const size_t group = Hq / Hkv;
    double* sc = (double*)malloc((Skv ? Skv : 1) * sizeof(double));
    for (size_t b = 0; b < batch; b++) {
        const size_t len = lens ? (size_t)(lens[b] < 0 ? 0 : (lens[b] > (int32_t)Skv ? (int32_t)Skv : lens[b])) : Skv;
        for (size_t h = 0; h < Hq; h++) {
            const size_t hk = h / group;
            const double* qr = q + (b * Hq + h) * D;
            double* orow = out + (b * Hq + h) * D;
            for (size_t d = 0; d < D; d++) orow[d] = 0.0;
            if (len == 0) continue;
            double mx = -1e9;
            for (size_t j = 0; j < len; j++) {
                const double* kr = k + ((b * Skv + j) * Hkv + hk) * D;
                double s = 0.0;
                for (size_t d = 0; d < D; d++) s += qr[d] * kr[d];
                sc[j] = s * scale;
                if (sc[j] > mx) mx = sc[j];
            }
            double se = 0.0;
            for (size_t j = 0; j < len; j++) {
                sc[j] = exp(sc[j] - mx);
                se += sc[j];
            }
            for (size_t j = 0; j < len; j++) sc[j] /= se;
            for (size_t d = 0; d < D; d++) {
                double s = 0.0;
                for (size_t j = 0; j < len; j++) s += sc[j] * v[((b * Skv + j) * Hkv + hk) * D + d];
                orow[d] = s;
            }
        }
    }
    free(sc);
}

/* ---- the int8 path --------------------------------------------------------------- */

/* Per-tensor quantization: B/src/runtime/lancius_scheduler.c:199-204 (MATMUL
 * activation), B/src/runtime/lancius_vision_ops.c:28-36 (conv activation),
 * B/src/compiler/lancius_quantize.c:14-25 (conv filters).  Returns the scale. */
double oracle_quantize_i8(int8_t* q, const double* x, size_t n) {
    double m = 0.0;
    for (size_t i = 0; i < n; i++) {
        const double a = fabs(x[i]);
        if (a > m) m = a;
    }
    const double scale = m > 0.0 ? m / 127.0 : 1e-8;
    for (size_t i = 0; i < n; i++) q[i] = (int8_t)round(x[i] / scale);
    return scale;
}

/* B/src/runtime/lancius_scheduler.c:195-220: quantized A times int8 B,
 * int32 sums scaled by scale_a * scale_b. */
int oracle_matmul_i8(double* out, const double* a, const int8_t* b, double scale_b, size_t M, size_t K, size_t N) {
    int8_t* qa = (int8_t*)malloc(M * K ? M * K : 1);
    if (!qa) return -1;
    const double scale = oracle_quantize_i8(qa, a, M * K) * scale_b;
    for (size_t r = 0; r < M; r++)
        for (size_t c = 0; c < N; c++) {
            int32_t s = 0;
            for (size_t k = 0; k < K; k++) s += (int32_t)qa[r * K + k] * (int32_t)b[k * N + c];
            out[r * N + c] = (double)s * scale;
        }
    free(qa);
    return 0;
}

/* B/src/math/lancius_kernels.c:177-210 on the activation quantized as
 * B/src/runtime/lancius_vision_ops.c:28-36 does, then the fused ReLU of :49-54. */
int oracle_conv2d_i8(double* out, const double* in, const int8_t* w, double scale_w, size_t N, size_t C_in, size_t H,
                     size_t W, size_t C_out, size_t K_h, size_t K_w, size_t stride, size_t pad, int relu) {
    const size_t n_in = N * C_in * H * W;
    int8_t* q = (int8_t*)malloc(n_in ? n_in : 1);
    if (!q) return -1;
    const double scale = oracle_quantize_i8(q, in, n_in) * scale_w;
    const size_t Ho = (H + 2 * pad - K_h) / stride + 1, Wo = (W + 2 * pad - K_w) / stride + 1;
#pragma omp parallel for collapse(2) schedule(static)
    for (size_t n = 0; n < N; n++)
        for (size_t co = 0; co < C_out; co++)
            for (size_t ho = 0; ho < Ho; ho++)
                for (size_t wo = 0; wo < Wo; wo++) {
                    int32_t s = 0;
                    for (size_t ci = 0; ci < C_in; ci++)
                        for (size_t kh = 0; kh < K_h; kh++)
                            for (size_t kw = 0; kw < K_w; kw++) {
                                const long ih = (long)(ho * stride) - (long)pad + (long)kh;
                                const long iw = (long)(wo * stride) - (long)pad + (long)kw;
                                if (ih < 0 || ih >= (long)H || iw < 0 || iw >= (long)W) continue;
                                s += (int32_t)q[((n * C_in + ci) * H + (size_t)ih) * W + (size_t)iw] *
                                     (int32_t)w[((co * C_in + ci) * K_h + kh) * K_w + kw];
                            }
                    double v = (double)s * scale;
                    if (relu && v < 0.0) v = 0.0;
                    out[((n * C_out + co) * Ho + ho) * Wo + wo] = v;
                }
    free(q);
    return 0;
}

/* ---- fp64 graph executor ------------------------------------------------------ */

static size_t elems_of(const lancius_node* n) {
    size_t e = 1;
    for (uint8_t d = 0; d < n->ndim; d++) e *= n->shape[d];
    return e;
}

static int ensure_buffer(lancius_node* n) {
    if (n->runtime_data) return 0;
    const size_t e = elems_of(n);
    n->runtime_data = (double*)calloc(e ? e : 1, sizeof(double));
    if (!n->runtime_data) return -1;
    if (n->rt) {
        n->rt->buffer = n->runtime_data;
        n->rt->flags |= ORACLE_OWNED;
    }
    return 0;
}

/* One node, the branches of B/src/runtime/lancius_scheduler.c:61-309 and
 * B/src/runtime/lancius_vision_ops.c:60-190 that the device path covers. */
static int run_node(lancius_node* n) {
    double* y = n->runtime_data;
    const size_t e = elems_of(n);
    const lancius_node* const* in = (const lancius_node* const*)n->inputs;
    switch (n->op) {
        case LANCIUS_OP_ADD:
            oracle_add(y, in[0]->runtime_data, in[1]->runtime_data, e);
            return 0;
        case LANCIUS_OP_MATMUL: {
            const size_t M = in[0]->shape[0], K = in[0]->shape[1], N = in[1]->shape[1];
            if (M * N > e) return -3;
            if (in[1]->runtime_data_int8) /* the int8 branch (lancius_scheduler.c:195) */
                return oracle_matmul_i8(y, in[0]->runtime_data, in[1]->runtime_data_int8, in[1]->scale, M, K, N);
            oracle_matmul_rows(y, in[0]->runtime_data, in[1]->runtime_data, M, K, N, 0, M);
            return 0;
        }
        case LANCIUS_OP_RELU:
            oracle_relu(y, in[0]->runtime_data, e);
            return 0;
        case LANCIUS_OP_GELU:
            oracle_gelu(y, in[0]->runtime_data, e);
            return 0;
        case LANCIUS_OP_SOFTMAX:
            oracle_softmax(y, in[0]->runtime_data, n->shape[0], n->shape[1]);
            return 0;
        case LANCIUS_OP_BROADCAST:
            oracle_broadcast(y, in[0]->runtime_data, elems_of(in[0]), n->shape[0], n->shape[1]);
            return 0;
        case LANCIUS_OP_LAYERNORM:
            oracle_layernorm(y, in[0]->runtime_data, in[1]->runtime_data, in[2]->runtime_data, n->shape[0],
                             n->shape[1], 1e-5);
            return 0;
        case LANCIUS_OP_ATTENTION: {
            const size_t S = n->shape[0], H = n->shape[1], D = n->shape[2];
            const int causal = n->axes[0] != 1; /* axes[0] == 1 selects the non-causal variant */
            oracle_attention(y, in[0]->runtime_data, in[1]->runtime_data, in[2]->runtime_data, 1, S, H, D, causal,
                             1.0 / sqrt((double)D), 0, 1, 0, S);
            return 0;
        }
        case LANCIUS_OP_CONV2D:
        case LANCIUS_OP_CONV2D_RELU_FUSED: {
            const lancius_node* x = in[0];
            const lancius_node* w = in[1];
            if (w->dtype == LANCIUS_DTYPE_INT8) /* lancius_vision_ops.c:14-16 */
                return oracle_conv2d_i8(y, x->runtime_data, w->runtime_data_int8, w->scale, x->shape[0], x->shape[1],
                                        x->shape[2], x->shape[3], w->shape[0], w->shape[2], w->shape[3], n->stride,
                                        n->pad, n->op == LANCIUS_OP_CONV2D_RELU_FUSED);
            oracle_conv2d(y, x->runtime_data, w->runtime_data, x->shape[0], x->shape[1], x->shape[2], x->shape[3],
                          w->shape[0], w->shape[2], w->shape[3], n->stride, n->pad,
                          n->op == LANCIUS_OP_CONV2D_RELU_FUSED, 0, x->shape[0]);
            return 0;
        }
        case LANCIUS_OP_RESHAPE:
        case LANCIUS_OP_FLATTEN:
            memcpy(y, in[0]->runtime_data, e * sizeof(double));
            return 0;
        case LANCIUS_OP_SUB:
            oracle_sub(y, in[0]->runtime_data, in[1]->runtime_data, e);
            return 0;
        case LANCIUS_OP_RMSNORM: /* lancius_scheduler.c:134-139 */
            oracle_rmsnorm(y, in[0]->runtime_data, in[1]->runtime_data, n->shape[0], n->shape[1], 1e-5);
            return 0;
        case LANCIUS_OP_SWIGLU: /* :140-145 */
            oracle_swiglu(y, in[0]->runtime_data, in[1]->runtime_data, e);
            return 0;
        case LANCIUS_OP_GQA: /* :146-152: S = shape[0], Hq = kernel_h, Hkv = kernel_w, D = shape[2] */
            if (n->kernel_w == 0 || n->kernel_h % n->kernel_w) return -3;
            oracle_attention_gqa(y, in[0]->runtime_data, in[1]->runtime_data, in[2]->runtime_data, 1, n->shape[0],
                                 n->shape[0], n->kernel_h, n->kernel_w, n->shape[2], 1,
                                 1.0 / sqrt((double)n->shape[2]));
            return 0;
        case LANCIUS_OP_ROPE: /* :153-165: copy, then q = first half, k = second half */
            oracle_rope(y, in[0]->runtime_data, 2, 1, n->shape[0], n->shape[1], n->shape[2] / 2, 0);
            return 0;
        case LANCIUS_OP_MUL:
            oracle_mul(y, in[0]->runtime_data, in[1]->runtime_data, e);
            return 0;
        case LANCIUS_OP_RELU_BWD:
            oracle_relu_bwd(y, in[0]->runtime_data, in[1]->runtime_data, e);
            return 0;
        case LANCIUS_OP_TRANSPOSE:
            oracle_transpose(y, in[0]->runtime_data, in[0]->shape[0], in[0]->shape[1]);
            return 0;
        case LANCIUS_OP_SUM:
            oracle_sum(y, in[0]->runtime_data, elems_of(in[0]));
            return 0;
        case LANCIUS_OP_SUM_AXIS0:
            oracle_sum_axis0(y, in[0]->runtime_data, in[0]->shape[0], in[0]->shape[1]);
            return 0;
        case LANCIUS_OP_SUM_AXIS1:
            oracle_sum_axis1(y, in[0]->runtime_data, in[0]->shape[0], in[0]->shape[1]);
            return 0;
        case LANCIUS_OP_SOFTMAX_BWD:
            oracle_softmax_bwd(y, in[0]->runtime_data, in[1]->runtime_data, n->shape[0], n->shape[1]);
            return 0;
        case LANCIUS_OP_CROSS_ENTROPY:
            oracle_cross_entropy(y, in[0]->runtime_data, in[1]->runtime_data, in[0]->shape[0], in[0]->shape[1]);
            return 0;
        case LANCIUS_OP_CROSS_ENTROPY_BWD:
            oracle_cross_entropy_bwd(y, in[0]->runtime_data, in[1]->runtime_data, in[2]->runtime_data, n->shape[0],
                                     n->shape[1]);
            return 0;
        case LANCIUS_OP_CONV2D_BWD: { /* inputs: grad, fwd_in, fwd_w (vision_ops.c:126-137) */
            const lancius_node *g = in[0], *x = in[1], *w = in[2];
            oracle_conv2d_bwd_input(y, g->runtime_data, w->runtime_data, x->shape[0], x->shape[1], x->shape[2],
                                    x->shape[3], w->shape[0], g->shape[2], g->shape[3], w->shape[2], w->shape[3],
                                    n->stride, n->pad);
            return 0;
        }
        case LANCIUS_OP_CONV2D_BWD_W: { /* inputs: grad, fwd_in (vision_ops.c:138-148) */
            const lancius_node *g = in[0], *x = in[1];
            oracle_conv2d_bwd_weight(y, g->runtime_data, x->runtime_data, x->shape[0], x->shape[1], x->shape[2],
                                     x->shape[3], n->shape[0], g->shape[2], g->shape[3], n->shape[2], n->shape[3],
                                     n->stride, n->pad);
            return 0;
        }
        case LANCIUS_OP_MAXPOOL2D: {
            const lancius_node* x = in[0];
            oracle_maxpool2d(y, x->runtime_data, x->shape[0], x->shape[1], x->shape[2], x->shape[3], n->kernel_h,
                             n->stride);
            return 0;
        }
        case LANCIUS_OP_MAXPOOL2D_BWD: {
            const lancius_node *g = in[0], *x = in[1];
            oracle_maxpool2d_bwd(y, g->runtime_data, x->runtime_data, x->shape[0], x->shape[1], x->shape[2],
                                 x->shape[3], g->shape[2], g->shape[3], n->kernel_h, n->stride);
            return 0;
        }
        default:
            return -4;
    }
}

int oracle_schedule_execute(lancius_schedule* s, int num_threads) {
    if (!s) return -2;
#ifdef _OPENMP
    if (num_threads > 0) omp_set_num_threads(num_threads);
#else
    (void)num_threads;
#endif
    for (uint32_t w = 0; w < s->wave_count; w++) {
        for (uint32_t i = 0; i < s->waves[w].node_count; i++) {
            lancius_node* n = s->waves[w].nodes[i];
            if (n->op == LANCIUS_OP_INPUT || n->op == LANCIUS_OP_NOP) continue;
            if (n->op == LANCIUS_OP_CONST) {
                if (!n->runtime_data) {
                    if (ensure_buffer(n)) return -1;
                    const size_t e = elems_of(n);
                    for (size_t k = 0; k < e; k++) n->runtime_data[k] = n->attr_val;
                }
                continue;
            }
            for (uint32_t j = 0; j < n->input_count; j++)
                if (!n->inputs[j] || !n->inputs[j]->runtime_data) return -2;
            if (ensure_buffer(n)) return -1;
            const int rc = run_node(n);
            if (rc) return rc;
        }
    }
    return 0;
}

void oracle_release_buffers(lancius_graph* g) {
    if (!g) return;
    for (uint32_t i = 0; i < g->node_count; i++) {
        lancius_node* n = g->nodes[i];
        if (n->rt && (n->rt->flags & ORACLE_OWNED)) {
            free(n->runtime_data);
            n->runtime_data = NULL;
            n->rt->buffer = NULL;
            n->rt->flags &= ~ORACLE_OWNED;
        }
    }
}
