/*
 * smol_linear.h - the decoders' bf16-weight projections on the GPU
 * (device-resident API; the reference-signature drop-ins are declared in
 * smol_kernels_linear.h). Library: libsmol_attn.so.
 *
 * One call computes, for s < seq and o < out_dim,
 *     y[s][o] = sum_i x[s][i] * W[o][i]  (+ bias[o])
 * which is smol_linear_bf16 / smol_linear_nobias_bf16
 * (common/kernels/matmul.c:336-358) when x and y are fp32, and the bf16
 * decoder's bf16_linear_nobias (common/decoder/qkn_bf16_decoder.c:99-117)
 * when x and y are bf16: fp32 sums, the result rounded to bf16 by
 * truncation.
 *
 * Layouts (all row-major, rows contiguous, device pointers of the context's
 * device): x [seq][in_dim] (fp32 or bf16), W [out_dim][in_dim] bf16,
 * bias [out_dim] fp32 or NULL, y [seq][out_dim] (fp32 or bf16). y must not
 * overlap x or W. Work is enqueued on the context's stream.
 *
 * Numerics: every product and sum is fp32 arithmetic on the exact bf16
 * weights. For seq <= SMOL_LINEAR_GEMV_MAX_SEQ a GEMV kernel reads fp32 x
 * as it is. Longer inputs run on the library's bf16 MFMA kernel: an fp32 x
 * is split as it is staged into x_hi = bf16(x) and x_lo = bf16(x - x_hi),
 * and y = W x_hi + W x_lo with fp32 accumulation, which carries x to about
 * 2^-17 relative. A bf16 x is used as it is. The fused operations of
 * smol_linear_ops_dev (norm, bias, activation, residual) run in the same
 * launch; y is written once.
 *
 * Errors: SMOL_ATTN_OK or a negative SMOL_ATTN_ERR_* status, with the
 * message in smol_attn_last_error().
 */
#ifndef SMOL_LINEAR_H
#define SMOL_LINEAR_H

#include "smol_attn.h"

#ifdef __cplusplus
extern "C" {
#endif

/* inputs of at most this many rows run on the GEMV kernel */
#define SMOL_LINEAR_GEMV_MAX_SEQ 4

/* y = x W^T (+ bias). x_dtype, y_dtype: SMOL_ATTN_F32 or SMOL_ATTN_BF16
 * (a bf16 y is truncated from the fp32 sum). Replaces
 * smol_linear_bf16 / smol_linear_nobias_bf16 (common/kernels/matmul.c:336-358)
 * and bf16_linear_nobias (common/decoder/qkn_bf16_decoder.c:99-117). */
SMOL_ATTN_API int smol_linear_dev(smol_attn_ctx *ctx, void *y, int y_dtype, const void *x, int x_dtype,
                                  const uint16_t *w, const float *bias, int seq, int in_dim, int out_dim);

/* The three projections of one decoder layer from one input:
 * q = x Wq^T [seq][q_dim], k = x Wk^T and v = x Wv^T [seq][kv_dim], without
 * bias. For seq <= SMOL_LINEAR_GEMV_MAX_SEQ the three run as one launch.
 * Replaces smol_linear_nobias_bf16_qkv (common/kernels/matmul.c:308-334)
 * and the three separate projections of qkn_decoder.c:474-476 and
 * qkn_bf16_decoder.c:498-500 / :647-649. */
SMOL_ATTN_API int smol_linear_qkv_dev(smol_attn_ctx *ctx, void *q, void *k, void *v, int y_dtype, const void *x,
                                      int x_dtype, const uint16_t *wq, const uint16_t *wk, const uint16_t *wv,
                                      int seq, int in_dim, int q_dim, int kv_dim);

/* ---- a decoder layer's operations around its projections ----------------
 *
 * The decoders wrap their projections in an RMSNorm of the input, a gated
 * activation of the gate/up product and a residual add
 * (common/decoder/qkn_decoder.c:633-705 for one token, :470-560 for a
 * prefill). smol_linear_ops_dev runs them with the projection; for
 * seq <= SMOL_LINEAR_GEMV_MAX_SEQ all of them happen inside the one GEMV
 * launch (the input row's sum of squares is accumulated by the waves that
 * read it, the activation and the add are applied as each output is
 * written), so a Qwen3 decoder layer's MLP is two launches. */
#define SMOL_LINEAR_ACT_NONE 0
#define SMOL_LINEAR_ACT_SWIGLU 1 /* silu(g) * u = g / (1 + expf(-g)) * u (activation.c:55-88) */
#define SMOL_LINEAR_ACT_GEGLU 2  /* gelu_tanh(g) * u (activation.c:104-125) */

typedef struct {
    /* non-NULL: x is first RMS-normalised with this weight [in_dim]:
     * x'[s][i] = x[s][i] * w[i] / sqrt(mean_i x[s][i]^2 + norm_eps)
     * (smol_rms_norm, common/kernels/rmsnorm.c:17-75) */
    const float *norm_weight;
    float norm_eps;
    /* SMOL_LINEAR_ACT_*: the weight's rows are (gate, up) pairs, row 2j the
     * gate and row 2j + 1 the up projection of unit j (the decoders' fused
     * gate_up weight, qkn_decoder.c:139-152); y [seq][out_dim / 2] gets
     * act(gate) * up (smol_swiglu_multiply / smol_geglu_multiply) */
    int act;
    /* non-NULL: added to the result, y = residual + ...; may equal y (the
     * decoders' smol_add_inplace of the sublayer output into the residual
     * stream, qkn_decoder.c:684-704) */
    const float *residual;
} smol_linear_ops;

/* y = residual + act(norm(x) W^T + bias) with the parts ops selects; ops may
 * be NULL (then this is smol_linear_dev on fp32). x, y, residual fp32
 * [seq][...] on the device; y must not overlap x; in_dim > 0. */
SMOL_ATTN_API int smol_linear_ops_dev(smol_attn_ctx *ctx, float *y, const float *x, const uint16_t *w,
                                      const float *bias, int seq, int in_dim, int out_dim,
                                      const smol_linear_ops *ops);

/* The Q/K/V projections of smol_linear_qkv_dev (fp32) behind the layer's
 * input RMSNorm (norm_weight [in_dim], or NULL for none): one launch for
 * seq <= SMOL_LINEAR_GEMV_MAX_SEQ (qkn_decoder.c:634-639). */
SMOL_ATTN_API int smol_linear_qkv_norm_dev(smol_attn_ctx *ctx, float *q, float *k, float *v, const float *x,
                                           const uint16_t *wq, const uint16_t *wk, const uint16_t *wv, int seq,
                                           int in_dim, int q_dim, int kv_dim, const float *norm_weight,
                                           float norm_eps);

/* out[s][i] = residual[s][i] + (x[s][i] * weight[i]) * (1 / sqrtf(sum_i x[s][i]^2 / dim + eps)),
 * without the residual term when residual is NULL; smol_rms_norm
 * (common/kernels/rmsnorm.c:17-75), plus the smol_add_inplace that follows
 * it in the Gemma 3 post-sublayer norms (qkn_decoder.c:682-686, 701-704).
 * out may equal x or residual. */
SMOL_ATTN_API int smol_rms_norm_dev(smol_attn_ctx *ctx, float *out, const float *x, const float *weight,
                                    const float *residual, int seq, int dim, float eps);

/* ---- the bf16 decoder's row operations ----------------------------------
 *
 * On bf16 arrays [seq][dim] (device pointers, enqueued on the context's
 * stream), every result truncated to bf16 as common/decoder/qkn_bf16_decoder.c
 * does. With bf() the widening of bf16 bits and tr() the truncation:
 *   norm(v, w)[i] = tr((bf(v[i]) * r) * w[i]), r = 1 / sqrtf(sum_i bf(v[i])^2 / dim + eps)
 * The sum of squares runs in a fixed order of its own, so a row can differ
 * from the reference's in the last bit where a product lies on a bf16
 * boundary. */

/* out = norm(x, weight): bf16_rms_norm (qkn_bf16_decoder.c:51-71); out may
 * equal x. */
SMOL_ATTN_API int smol_bf16_rms_norm_dev(smol_attn_ctx *ctx, uint16_t *out, const uint16_t *x, const float *weight,
                                         int seq, int dim, float eps);

/* The step between two sublayers, one launch:
 *   p non-NULL:         x = tr(bf(x) + bf(p_norm ? norm(p, p_norm) : p))
 *   next_norm non-NULL: xn = norm(x, next_norm), of the updated x
 * which is bf16_add_inplace (:255-258), optionally behind a post-sublayer
 * norm and before the next input norm (:551-557, 567-570). p is not
 * modified. xn may equal x only when p is NULL; no other arrays overlap. */
SMOL_ATTN_API int smol_bf16_add_norm_dev(smol_attn_ctx *ctx, uint16_t *x, const uint16_t *p, const float *p_norm,
                                         const float *next_norm, uint16_t *xn, int seq, int dim, float eps);

/* out [seq][inter] = tr(gelu_tanh(bf(g)) * bf(u)) of the interleaved pairs
 * gate_up [seq][2 * inter] (g = row[2j], u = row[2j + 1]): bf16_geglu
 * (:235-251). gate_up 4-byte aligned; out does not overlap it. */
SMOL_ATTN_API int smol_bf16_geglu_dev(smol_attn_ctx *ctx, uint16_t *out, const uint16_t *gate_up, int seq,
                                      int inter);

#ifdef __cplusplus
}
#endif

#endif
