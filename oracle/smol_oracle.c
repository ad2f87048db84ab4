/*
 * smol_oracle.c - CPU oracle for the attention path and the decoders' bf16
 * projections. TEST INFRASTRUCTURE ONLY.
 *
 * This file restates, in plain C, the reference's CPU attention, RoPE and
 * RoPE-table arithmetic so that the HIP path can be checked against it on the
 * same inputs. Only the tests, the smoke check and the CPU-baseline leg of the
 * bench may load it; the product library never links or calls it.
 *
 * What each function follows (reference files, tmzt/smol-genius):
 *   orc_dot / orc_scale / orc_axpy / orc_scale_add
 *       common/kernels/vecops_avx.c:13-156 (AVX-512 accumulation order:
 *       4 x 16-lane accumulators over 64-wide blocks, then 16-wide blocks,
 *       a halving tree over the 16 lanes, then a scalar tail) and
 *       vecops_generic.c:7-23 (sequential order, ORC_VEC_GENERIC).
 *   orc_causal_attention            attention.c:79-170
 *   orc_bidirectional_attention     attention.c:32-77
 *   orc_sliding_window_attention    attention.c:176-273
 *   orc_causal_attention_softcap    attention.c:281-368
 *   orc_sliding_window_attention_softcap  attention.c:370-462
 *   orc_rope_inv_freq               common/decoder/qkn_decoder.c:261-274
 *   orc_fill_rope_table             common/decoder/qkn_decoder.c:276-311
 *   orc_compute_rope_neox / _interleaved   rope.c:27-66
 *   orc_apply_rope_neox             rope.c:99-164
 *   orc_apply_rope_interleaved      rope.c:68-93
 *   orc_bf16_attention_softcap      common/decoder/qkn_bf16_decoder.c:120-229
 *       (two-pass softmax, truncating bf16 output, optional window/softcap)
 *   orc_bf16_rms_norm_per_head      common/decoder/qkn_bf16_decoder.c:73-91
 *   orc_bf16_apply_rope_interleaved common/decoder/qkn_bf16_decoder.c:264-283
 *       (truncating bf16 after each step, with a stated operation order)
 *   orc_rms_norm_per_head           common/kernels/rmsnorm.c:78-140
 *       (AVX-512 order: 16-lane fused multiply-add accumulators over the
 *       16-wide blocks, a halving tree, then a scalar tail)
 *   orc_linear_bf16                 common/kernels/matmul.c:70-97 (smol_linear's
 *       loops) on the exactly widened bf16 weights (matmul.c:101-106, 196-205),
 *       as smol_linear_bf16 / smol_linear_nobias_bf16 / smol_matmul_t_bf16 run
 *       them for seq_len > 1 (matmul.c:336-358, 419-429)
 *   orc_bf16_linear_nobias          common/decoder/qkn_bf16_decoder.c:99-117
 *   orc_bf16_rms_norm / orc_bf16_geglu / orc_bf16_add_inplace
 *                                   common/decoder/qkn_bf16_decoder.c:51-71, 235-251, 255-258
 *   orc_rms_norm                    common/kernels/rmsnorm.c:17-75 (the AVX-512 order
 *       of orc_rms_norm_per_head with the whole row as one head)
 *   orc_swiglu / orc_geglu          common/kernels/activation.c:55-88, 104-125
 *
 * Parity pins (see tests/test_oracle_*.py): golden vectors written by the
 * compiled reference (oracle/_ref), closed forms (one visible key, identical
 * keys, scale 0, empty rows), a float64 brute-force softmax, and RoPE identities.
 *
 * Threading: heads are split over a fork-join set of pthreads exactly as
 * attention.c:140-151 splits them (chunk = ceil(H / threads)); the arithmetic
 * per (head, row) does not depend on the thread count.
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define ORC_LANES 16

/* ---------------------------------------------------------------- vecops */

static int orc_vec_generic = 0; /* 1 = vecops_generic.c order */

void orc_set_vec_generic(int on) { orc_vec_generic = on ? 1 : 0; }

static float lane_tree_sum(const float *v) {
    /* halving tree 16 -> 8 -> 4 -> 2 -> 1, as a 512-bit horizontal add does */
    float t8[8], t4[4], t2[2];
    for (int i = 0; i < 8; i++) t8[i] = v[i] + v[i + 8];
    for (int i = 0; i < 4; i++) t4[i] = t8[i] + t8[i + 4];
    for (int i = 0; i < 2; i++) t2[i] = t4[i] + t4[i + 2];
    return t2[0] + t2[1];
}

static float orc_dot(const float *a, const float *b, int n) {
    if (orc_vec_generic) {
        float s = 0.0f;
        for (int i = 0; i < n; i++) s += a[i] * b[i];
        return s;
    }
    float acc[4][ORC_LANES];
    memset(acc, 0, sizeof(acc));
    int i = 0;
    for (; i + 64 <= n; i += 64)
        for (int q = 0; q < 4; q++)
            for (int l = 0; l < ORC_LANES; l++)
                acc[q][l] = fmaf(a[i + 16 * q + l], b[i + 16 * q + l], acc[q][l]);
    float s16[ORC_LANES];
    for (int l = 0; l < ORC_LANES; l++)
        s16[l] = (acc[0][l] + acc[1][l]) + (acc[2][l] + acc[3][l]);
    for (; i + 16 <= n; i += 16)
        for (int l = 0; l < ORC_LANES; l++) s16[l] = fmaf(a[i + l], b[i + l], s16[l]);
    float s = lane_tree_sum(s16);
    for (; i < n; i++) s += a[i] * b[i];
    return s;
}

/* dst *= scale */
static void orc_scale(float *dst, float scale, int n) {
    for (int i = 0; i < n; i++) dst[i] *= scale;
}

/* dst += alpha * src; the vector body is a fused multiply-add */
static void orc_axpy(float *dst, const float *src, float alpha, int n) {
    if (orc_vec_generic) {
        for (int i = 0; i < n; i++) dst[i] += alpha * src[i];
        return;
    }
    int body = n - (n % 16);
    for (int i = 0; i < body; i++) dst[i] = fmaf(src[i], alpha, dst[i]);
    for (int i = body; i < n; i++) dst[i] += alpha * src[i];
}

/* dst = dst * correction + src; the vector body is a fused multiply-add */
static void orc_scale_add(float *dst, const float *src, float correction, int n) {
    if (orc_vec_generic) {
        for (int i = 0; i < n; i++) dst[i] = dst[i] * correction + src[i];
        return;
    }
    int body = n - (n % 16);
    for (int i = 0; i < body; i++) dst[i] = fmaf(dst[i], correction, src[i]);
    for (int i = body; i < n; i++) dst[i] = dst[i] * correction + src[i];
}

/* ------------------------------------------------------- fork-join threads */

static int orc_threads = 1;

void orc_set_threads(int n) { orc_threads = n < 1 ? 1 : (n > 64 ? 64 : n); }
int orc_get_threads(void) { return orc_threads; }

typedef void (*orc_fn)(int tid, int nt, void *arg);
typedef struct { orc_fn fn; void *arg; int tid, nt; } orc_job;

static void *orc_trampoline(void *p) {
    orc_job *j = (orc_job *)p;
    j->fn(j->tid, j->nt, j->arg);
    return NULL;
}

static void orc_parallel_for(orc_fn fn, void *arg) {
    int nt = orc_threads;
    if (nt <= 1) { fn(0, 1, arg); return; }
    pthread_t th[64];
    orc_job jobs[64];
    for (int t = 1; t < nt; t++) {
        jobs[t] = (orc_job){fn, arg, t, nt};
        pthread_create(&th[t], NULL, orc_trampoline, &jobs[t]);
    }
    fn(0, nt, arg);
    for (int t = 1; t < nt; t++) pthread_join(th[t], NULL);
}

/* ------------------------------------------------------------- attention */

/* One row of online softmax over keys [k_begin, k_end), as in
 * attention.c:98-123. K/V rows are kv_stride floats apart. With use_cap the
 * score becomes cap * tanhf(score * (1 / cap)) for any cap, as in
 * attention.c:284-308 (a negative cap is the same as |cap|); cap == 0 is
 * restated as a zero score, which is what the reference computes for every
 * nonzero score (0 * tanhf(+-inf)). */
static void orc_row(float *o, const float *q, const float *K, const float *V,
                    int k_begin, int k_end, int kv_stride, int hd, float scale,
                    int use_cap, float cap) {
    float m = -1e30f, l = 0.0f;
    for (int d = 0; d < hd; d++) o[d] = 0.0f;
    float inv_cap = cap != 0.0f ? 1.0f / cap : 0.0f;
    for (int j = k_begin; j < k_end; j++) {
        const float *k = K + (size_t)j * kv_stride;
        const float *v = V + (size_t)j * kv_stride;
        float s = orc_dot(q, k, hd) * scale;
        if (use_cap) s = cap != 0.0f ? cap * tanhf(s * inv_cap) : 0.0f;
        if (s > m) {
            float c = expf(m - s);
            l = l * c + 1.0f;
            orc_scale_add(o, v, c, hd);
            m = s;
        } else {
            float w = expf(s - m);
            l += w;
            orc_axpy(o, v, w, hd);
        }
    }
    if (l > 0.0f) orc_scale(o, 1.0f / l, hd);
}

typedef struct {
    float *out; const float *Q, *K, *V;
    int seq_q, seq_k, n_heads, n_kv_heads, hd;
    float scale, cap;
    int q_offset, window;
    int use_window, use_cap; /* the sliding-window / softcap variants */
} orc_causal_task;

static void orc_causal_worker(int tid, int nt, void *arg) {
    orc_causal_task *t = (orc_causal_task *)arg;
    int chunk = (t->n_heads + nt - 1) / nt;
    int h0 = tid * chunk, h1 = h0 + chunk;
    if (h1 > t->n_heads) h1 = t->n_heads;
    int per_kv = t->n_heads / t->n_kv_heads;
    int qh = t->n_heads * t->hd, kvh = t->n_kv_heads * t->hd;
    for (int h = h0; h < h1; h++) {
        int g = h / per_kv;
        for (int i = 0; i < t->seq_q; i++) {
            int gp = t->q_offset + i;
            int k_end = gp + 1;
            if (k_end > t->seq_k) k_end = t->seq_k;
            /* attention.c:190-192: the window starts at gp - window + 1 once
             * gp >= window, for any window_size (<= 0 leaves no key) */
            int k_begin = 0;
            if (t->use_window && gp >= t->window) k_begin = gp - t->window + 1;
            orc_row(t->out + (size_t)i * qh + (size_t)h * t->hd,
                    t->Q + (size_t)i * qh + (size_t)h * t->hd,
                    t->K + (size_t)g * t->hd, t->V + (size_t)g * t->hd,
                    k_begin, k_end, kvh, t->hd, t->scale, t->use_cap, t->cap);
        }
    }
}

static void orc_causal_common(float *out, const float *Q, const float *K, const float *V,
                              int seq_q, int seq_k, int n_heads, int n_kv_heads, int hd,
                              float scale, int q_offset, int use_window, int window,
                              int use_cap, float cap) {
    orc_causal_task t = {out, Q, K, V, seq_q, seq_k, n_heads, n_kv_heads, hd,
                         scale, cap, q_offset, window, use_window, use_cap};
    /* attention.c:156 threads only when n_heads >= 2 and the call is not tiny */
    if (orc_threads > 1 && n_heads >= 2 && (seq_q >= 2 || seq_k >= 128))
        orc_parallel_for(orc_causal_worker, &t);
    else
        orc_causal_worker(0, 1, &t);
}

void orc_causal_attention(float *out, const float *Q, const float *K, const float *V,
                          int seq_q, int seq_k, int n_heads, int n_kv_heads, int hd,
                          float scale, int q_offset) {
    orc_causal_common(out, Q, K, V, seq_q, seq_k, n_heads, n_kv_heads, hd, scale,
                      q_offset, 0, 0, 0, 0.0f);
}

void orc_sliding_window_attention(float *out, const float *Q, const float *K,
                                  const float *V, int seq_q, int seq_k, int n_heads,
                                  int n_kv_heads, int hd, float scale, int q_offset,
                                  int window) {
    orc_causal_common(out, Q, K, V, seq_q, seq_k, n_heads, n_kv_heads, hd, scale,
                      q_offset, 1, window, 0, 0.0f);
}

void orc_causal_attention_softcap(float *out, const float *Q, const float *K,
                                  const float *V, int seq_q, int seq_k, int n_heads,
                                  int n_kv_heads, int hd, float scale, int q_offset,
                                  float cap) {
    orc_causal_common(out, Q, K, V, seq_q, seq_k, n_heads, n_kv_heads, hd, scale,
                      q_offset, 0, 0, 1, cap);
}

void orc_sliding_window_attention_softcap(float *out, const float *Q, const float *K,
                                          const float *V, int seq_q, int seq_k,
                                          int n_heads, int n_kv_heads, int hd,
                                          float scale, int q_offset, int window,
                                          float cap) {
    orc_causal_common(out, Q, K, V, seq_q, seq_k, n_heads, n_kv_heads, hd, scale,
                      q_offset, 1, window, 1, cap);
}

/* attention.c:32-77: heads x windows x rows, single-threaded in the reference;
 * `seq` is unused there as well. */
void orc_bidirectional_attention(float *out, const float *Q, const float *K,
                                 const float *V, int seq, int n_heads, int hd,
                                 float scale, const int *window_starts, int n_windows) {
    (void)seq;
    int hidden = n_heads * hd;
    for (int h = 0; h < n_heads; h++)
        for (int w = 0; w < n_windows; w++) {
            int ws = window_starts[w], we = window_starts[w + 1];
            for (int i = ws; i < we; i++)
                orc_row(out + (size_t)i * hidden + (size_t)h * hd,
                        Q + (size_t)i * hidden + (size_t)h * hd,
                        K + (size_t)h * hd, V + (size_t)h * hd, ws, we, hidden, hd,
                        scale, 0, 0.0f);
        }
}

/* ------------------------------------------------------------------ RoPE */

/* qkn_decoder.c:269-271 */
void orc_rope_inv_freq(float *inv, int hd, float theta) {
    for (int d = 0; d < hd / 2; d++)
        inv[d] = 1.0f / powf(theta, (float)(2 * d) / (float)hd);
}

/* qkn_decoder.c:292-308: rows [pos0, pos0 + n_pos) of the cos/sin table,
 * duplicated to (d, half + d) for NeoX or (2d, 2d + 1) for interleaved. */
void orc_fill_rope_table(float *cos_out, float *sin_out, int pos0, int n_pos, int hd,
                         float theta, int interleaved) {
    int half = hd / 2;
    float *inv = (float *)malloc(sizeof(float) * (size_t)(half > 0 ? half : 1));
    orc_rope_inv_freq(inv, hd, theta);
    for (int r = 0; r < n_pos; r++) {
        float p = (float)(pos0 + r);
        float *cr = cos_out + (size_t)r * hd, *sr = sin_out + (size_t)r * hd;
        for (int d = 0; d < half; d++) {
            float a = p * inv[d];
            float c = cosf(a), s = sinf(a);
            if (interleaved) { cr[2 * d] = c; cr[2 * d + 1] = c; sr[2 * d] = s; sr[2 * d + 1] = s; }
            else { cr[d] = c; cr[half + d] = c; sr[d] = s; sr[half + d] = s; }
        }
    }
    free(inv);
}

/* rope.c:27-66 (frequency computed inline per call) */
static void orc_compute_rope(float *cos_out, float *sin_out, const int *positions,
                             int seq, int hd, float theta, int interleaved) {
    int half = hd / 2;
    for (int s = 0; s < seq; s++) {
        float pos = (float)positions[s];
        for (int d = 0; d < half; d++) {
            float freq = 1.0f / powf(theta, (float)(2 * d) / (float)hd);
            float a = pos * freq;
            float c = cosf(a), sn = sinf(a);
            if (interleaved) {
                cos_out[s * hd + 2 * d] = c; cos_out[s * hd + 2 * d + 1] = c;
                sin_out[s * hd + 2 * d] = sn; sin_out[s * hd + 2 * d + 1] = sn;
            } else {
                cos_out[s * hd + d] = c; cos_out[s * hd + half + d] = c;
                sin_out[s * hd + d] = sn; sin_out[s * hd + half + d] = sn;
            }
        }
    }
}

void orc_compute_rope_neox(float *c, float *s, const int *pos, int seq, int hd, float theta) {
    orc_compute_rope(c, s, pos, seq, hd, theta, 0);
}

void orc_compute_rope_interleaved(float *c, float *s, const int *pos, int seq, int hd,
                                  float theta) {
    orc_compute_rope(c, s, pos, seq, hd, theta, 1);
}

/* rope.c:99-164: x1*c - x2*s and x2*c + x1*s, the vector body as
 * fmsub(x1, c, x2*s) / fmadd(x2, c, x1*s) */
void orc_apply_rope_neox(float *x, const float *cos_vals, const float *sin_vals, int seq,
                         int n_heads, int hd) {
    int half = hd / 2, hidden = n_heads * hd;
    for (int s = 0; s < seq; s++) {
        const float *c = cos_vals + (size_t)s * hd, *sn = sin_vals + (size_t)s * hd;
        for (int h = 0; h < n_heads; h++) {
            float *v = x + (size_t)s * hidden + (size_t)h * hd;
            int body = orc_vec_generic ? 0 : half - (half % 16);
            for (int d = 0; d < body; d++) {
                float x1 = v[d], x2 = v[half + d];
                v[d] = fmaf(x1, c[d], -(x2 * sn[d]));
                v[half + d] = fmaf(x2, c[d], x1 * sn[d]);
            }
            for (int d = body; d < half; d++) {
                float x1 = v[d], x2 = v[half + d];
                v[d] = x1 * c[d] + (-x2) * sn[d];
                v[half + d] = x2 * c[half + d] + x1 * sn[half + d];
            }
        }
    }
}

/* rope.c:68-93 */
void orc_apply_rope_interleaved(float *x, const float *cos_vals, const float *sin_vals,
                                int seq, int n_heads, int hd) {
    int half = hd / 2, hidden = n_heads * hd;
    for (int s = 0; s < seq; s++) {
        const float *c = cos_vals + (size_t)s * hd, *sn = sin_vals + (size_t)s * hd;
        for (int h = 0; h < n_heads; h++) {
            float *v = x + (size_t)s * hidden + (size_t)h * hd;
            for (int d = 0; d < half; d++) {
                float x0 = v[2 * d], x1 = v[2 * d + 1];
                v[2 * d] = x0 * c[2 * d] - x1 * sn[2 * d];
                v[2 * d + 1] = x1 * c[2 * d + 1] + x0 * sn[2 * d + 1];
            }
        }
    }
}

/* ------------------------------------------------------- per-head RMSNorm */

/* rmsnorm.c:78-140: each head_dim segment of x [seq][n_heads * hd] becomes
 * x * w / sqrt(mean(x^2) + eps), in place. The sum of squares follows the
 * AVX-512 body (86-94): 16 lane accumulators updated by fused multiply-adds
 * over the 16-wide blocks, the halving-tree reduction, then the tail added
 * element by element; the 16-wide blocks scale as (x * w) * r (119-121), the
 * tail as x * r * w (123). ORC_VEC_GENERIC follows the scalar branch
 * (107-112, 134-136): a sequential sum and x * r * w throughout. */
void orc_rms_norm_per_head(float *x, const float *w, int seq, int n_heads, int hd, float eps) {
    int hidden = n_heads * hd;
    for (int s = 0; s < seq; s++) {
        for (int h = 0; h < n_heads; h++) {
            float *v = x + (size_t)s * hidden + (size_t)h * hd;
            int body = orc_vec_generic ? 0 : hd - (hd % ORC_LANES);
            float ss;
            if (body > 0) {
                float acc[ORC_LANES] = {0};
                for (int d = 0; d < body; d += ORC_LANES)
                    for (int i = 0; i < ORC_LANES; i++) acc[i] = fmaf(v[d + i], v[d + i], acc[i]);
                ss = lane_tree_sum(acc);
            } else {
                ss = 0.0f;
            }
            for (int d = body; d < hd; d++) ss += v[d] * v[d];
            float r = 1.0f / sqrtf(ss / hd + eps);
            for (int d = 0; d < body; d++) v[d] = (v[d] * w[d]) * r;
            for (int d = body; d < hd; d++) v[d] = v[d] * r * w[d];
        }
    }
}

/* ------------------------------------------------------------ bf16 helpers */

static inline float orc_bf16_to_f32(uint16_t b) {
    uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static inline uint16_t orc_f32_to_bf16_trunc(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return (uint16_t)(u >> 16);
}

void orc_bf16_widen(float *dst, const uint16_t *src, size_t n) {
    for (size_t i = 0; i < n; i++) dst[i] = orc_bf16_to_f32(src[i]);
}

/* qkn_bf16_decoder.c:73-91 (bf16_rms_norm_per_head), in place on bf16 rows
 * x [seq][n_heads * hd], with the operation order that the GPU path fixes:
 * ss = fmaf(v, v, ss) element by element from 0, r = 1 / sqrtf(ss / hd +
 * eps) (each step correctly rounded), v' = trunc((v * r) * w[d]).
 * (The reference's clang -O3 -ffast-math build may reassociate the sum and
 * use a reciprocal square root estimate, so its own bits depend on the build;
 * this is the order written in its source with the multiply-add fused.) */
void orc_bf16_rms_norm_per_head(uint16_t *x, const float *w, int seq, int n_heads, int hd, float eps) {
    for (size_t r = 0; r < (size_t)seq * n_heads; r++) {
        uint16_t *v = x + r * hd;
        float ss = 0.0f;
        for (int d = 0; d < hd; d++) {
            float a = orc_bf16_to_f32(v[d]);
            ss = fmaf(a, a, ss);
        }
        float ri = 1.0f / sqrtf(ss / (float)hd + eps);
        for (int d = 0; d < hd; d++) {
            float a = orc_bf16_to_f32(v[d]) * ri;
            v[d] = orc_f32_to_bf16_trunc(a * w[d]);
        }
    }
}

/* qkn_bf16_decoder.c:264-283 (bf16_apply_rope_interleaved), in place on
 * bf16 rows x [seq][n_heads * hd]; row s uses cos_t / sin_t row s. Pair
 * (2i, 2i + 1) with c = cos[2i], s = sin[2i]:
 *   x0' = trunc(fmaf(x0, c, -(x1 * s))), x1' = trunc(fmaf(x1, c, x0 * s))
 * (the source's x0*c - x1*s and x1*c + x0*s with the first product fused,
 * as a contracting compiler emits them). */
void orc_bf16_apply_rope_interleaved(uint16_t *x, const float *cos_t, const float *sin_t, int seq,
                                     int n_heads, int hd) {
    int half = hd / 2;
    for (int s = 0; s < seq; s++) {
        const float *cr = cos_t + (size_t)s * hd, *sr = sin_t + (size_t)s * hd;
        for (int h = 0; h < n_heads; h++) {
            uint16_t *v = x + ((size_t)s * n_heads + h) * hd;
            for (int i = 0; i < half; i++) {
                float x0 = orc_bf16_to_f32(v[2 * i]), x1 = orc_bf16_to_f32(v[2 * i + 1]);
                float c = cr[2 * i], sn = sr[2 * i];
                float p1 = x1 * sn, p0 = x0 * sn;
                v[2 * i] = orc_f32_to_bf16_trunc(fmaf(x0, c, -p1));
                v[2 * i + 1] = orc_f32_to_bf16_trunc(fmaf(x1, c, p0));
            }
        }
    }
}

/* qkn_bf16_decoder.c:120-229: scores into a buffer, max, expf, sum, weighted
 * sum, bf16 output by truncation; window <= 0 means full causal, cap <= 0 no
 * softcap. */
void orc_bf16_attention_softcap(uint16_t *out, const uint16_t *q, const uint16_t *k,
                                const uint16_t *v, int seq_q, int seq_k, int n_heads,
                                int n_kv_heads, int hd, float scale, int q_offset,
                                int window, float cap) {
    int per_kv = n_heads / n_kv_heads, qh = n_heads * hd, kvh = n_kv_heads * hd;
    float inv_cap = cap > 0.0f ? 1.0f / cap : 0.0f;
    float *scores = (float *)malloc(sizeof(float) * (size_t)(seq_k > 0 ? seq_k : 1));
    for (int h = 0; h < n_heads; h++) {
        int g = h / per_kv;
        for (int i = 0; i < seq_q; i++) {
            const uint16_t *qr = q + (size_t)i * qh + (size_t)h * hd;
            uint16_t *orow = out + (size_t)i * qh + (size_t)h * hd;
            int gp = q_offset + i, k_end = gp + 1;
            if (k_end > seq_k) k_end = seq_k;
            int k_start = 0;
            if (window > 0 && gp >= window) k_start = gp - window + 1;
            int nk = k_end - k_start;
            float m = -1e30f;
            for (int j = k_start; j < k_end; j++) {
                const uint16_t *kr = k + (size_t)j * kvh + (size_t)g * hd;
                float dot = 0.0f;
                for (int d = 0; d < hd; d++) dot += orc_bf16_to_f32(qr[d]) * orc_bf16_to_f32(kr[d]);
                float s = dot * scale;
                if (cap > 0.0f) s = cap * tanhf(s * inv_cap);
                scores[j - k_start] = s;
                if (s > m) m = s;
            }
            float sum = 0.0f;
            for (int j = 0; j < nk; j++) { scores[j] = expf(scores[j] - m); sum += scores[j]; }
            float inv = 1.0f / sum;
            for (int d = 0; d < hd; d++) {
                float val = 0.0f;
                for (int j = 0; j < nk; j++)
                    val += scores[j] * inv *
                           orc_bf16_to_f32(v[(size_t)(k_start + j) * kvh + (size_t)g * hd + d]);
                orow[d] = orc_f32_to_bf16_trunc(val);
            }
        }
    }
    free(scores);
}

/* ---------------------------------------------------------------- linear */

/* matmul.c:70-97 (smol_linear without BLAS) with W widened from bf16 bits:
 * y[s][o] = b[o] (or 0), then + x[s][i] * W[o][i] for i ascending, every
 * product and sum rounded to fp32 (this file is built without contraction).
 * The reference's seq_len == 1 path (bf16_matvec_fused, matmul.c:210-247)
 * adds the same products in its SIMD order; threads there split output rows,
 * which does not change any row's arithmetic. */
void orc_linear_bf16(float *y, const float *x, const uint16_t *W, const float *b, int seq, int in, int out) {
    for (int s = 0; s < seq; s++) {
        const float *xr = x + (size_t)s * in;
        float *yr = y + (size_t)s * out;
        for (int o = 0; o < out; o++) {
            const uint16_t *wr = W + (size_t)o * in;
            float sum = b ? b[o] : 0.0f;
            for (int i = 0; i < in; i++) sum += xr[i] * orc_bf16_to_f32(wr[i]);
            yr[o] = sum;
        }
    }
}

/* qkn_bf16_decoder.c:99-117 (bf16_linear_nobias): bf16 x and W widened,
 * sum from 0 over i ascending in fp32, the result truncated to bf16 */
void orc_bf16_linear_nobias(uint16_t *y, const uint16_t *x, const uint16_t *W, int seq, int in, int out) {
    for (int s = 0; s < seq; s++) {
        const uint16_t *xr = x + (size_t)s * in;
        uint16_t *yr = y + (size_t)s * out;
        for (int o = 0; o < out; o++) {
            const uint16_t *wr = W + (size_t)o * in;
            float sum = 0.0f;
            for (int i = 0; i < in; i++) sum += orc_bf16_to_f32(xr[i]) * orc_bf16_to_f32(wr[i]);
            yr[o] = orc_f32_to_bf16_trunc(sum);
        }
    }
}

/* qkn_bf16_decoder.c:51-71 (bf16_rms_norm) on whole rows: out[s][i] =
 * trunc((x[s][i] * r) * w[i]), r = 1 / sqrtf(ss / dim + eps), with the
 * arithmetic of orc_bf16_rms_norm_per_head (the row as one head). out may
 * equal x. */
void orc_bf16_rms_norm(uint16_t *out, const uint16_t *x, const float *w, int seq, int dim, float eps) {
    if (out != x) memcpy(out, x, (size_t)seq * dim * sizeof(uint16_t));
    orc_bf16_rms_norm_per_head(out, w, seq, 1, dim, eps);
}

/* qkn_bf16_decoder.c:235-251 (bf16_geglu): g = gu[s][2j], u = gu[s][2j + 1]
 * widened from bf16, out[s][j] = trunc(gelu_tanh(g) * u) with the GELU of
 * orc_geglu (0.5 g (1 + tanh(0.7978845608028654 (g + 0.044715 g^3)))). */
void orc_bf16_geglu(uint16_t *out, const uint16_t *gu, int seq, int inter) {
    for (int s = 0; s < seq; s++)
        for (int j = 0; j < inter; j++) {
            float g = orc_bf16_to_f32(gu[(size_t)s * 2 * inter + 2 * j]);
            float u = orc_bf16_to_f32(gu[(size_t)s * 2 * inter + 2 * j + 1]);
            float x3 = g * g * g;
            float inner = 0.7978845608028654f * (g + 0.044715f * x3);
            g = 0.5f * g * (1.0f + tanhf(inner));
            out[(size_t)s * inter + j] = orc_f32_to_bf16_trunc(g * u);
        }
}

/* qkn_bf16_decoder.c:255-258 (bf16_add_inplace): a[i] = trunc(a[i] + b[i]) */
void orc_bf16_add_inplace(uint16_t *a, const uint16_t *b, size_t n) {
    for (size_t i = 0; i < n; i++) a[i] = orc_f32_to_bf16_trunc(orc_bf16_to_f32(a[i]) + orc_bf16_to_f32(b[i]));
}

/* rmsnorm.c:17-75: the same arithmetic as rmsnorm.c:78-140 per head, over
 * the whole row (16-lane fused multiply-add accumulators, a halving tree, a
 * scalar tail; (x * w) * r on the 16-wide body, x * r * w on the tail) */
void orc_rms_norm(float *out, const float *x, const float *w, int seq, int dim, float eps) {
    if (out != x) memcpy(out, x, (size_t)seq * dim * sizeof(float));
    orc_rms_norm_per_head(out, w, seq, 1, dim, eps);
}

/* activation.c:55-88 (SwiGLU) and :104-125 (GeGLU, tanh form) on interleaved
 * (gate, up) pairs: out[s][j] = act(gu[s][2j]) * gu[s][2j + 1] */
void orc_swiglu(float *out, const float *gu, int seq, int inter) {
    for (int s = 0; s < seq; s++)
        for (int j = 0; j < inter; j++) {
            float g = gu[(size_t)s * 2 * inter + 2 * j];
            float u = gu[(size_t)s * 2 * inter + 2 * j + 1];
            g = g / (1.0f + expf(-g));
            out[(size_t)s * inter + j] = g * u;
        }
}

void orc_geglu(float *out, const float *gu, int seq, int inter) {
    for (int s = 0; s < seq; s++)
        for (int j = 0; j < inter; j++) {
            float g = gu[(size_t)s * 2 * inter + 2 * j];
            float u = gu[(size_t)s * 2 * inter + 2 * j + 1];
            float x3 = g * g * g;
            float inner = 0.7978845608028654f * (g + 0.044715f * x3);
            g = 0.5f * g * (1.0f + tanhf(inner));
            out[(size_t)s * inter + j] = g * u;
        }
}
