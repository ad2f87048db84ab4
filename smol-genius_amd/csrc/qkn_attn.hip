/*
 * qkn_attn.hip - the reference decoders' attention block on the GPU, keyed by
 * the decoder context's address (include/smol_qkn_attn.h). Host code only:
 * it composes the device API of attn_api.hip.
 *
 * Per call it does what common/decoder/qkn_decoder.c:460-528 (prefill) and
 * :625-677 (one decode step) do between the projections and o_proj, and what
 * common/decoder/qkn_bf16_decoder.c:486-546 / :638-674 do in bf16:
 *   table  = local-theta table if the layer is sliding and a local table
 *            exists (:460-468), else the global one
 *   window = sliding_window if (is_sliding && sliding_window > 0), else none
 *   cap    = attn_logit_softcap if > 0, else none          (:505-528)
 * and the four attention entry points become one device call with those
 * two arguments.
 */
#include <hip/hip_runtime.h>

#include <mutex>
#include <unordered_map>
#include <vector>

#include <math.h>
#include <string.h>

#include "smol_linear.h"
#include "smol_qkn_attn.h"

extern "C" int smol_internal_fail(int code, const char *msg);
extern "C" int smol_launch_to_bf16_trunc(const float *x, uint16_t *y, long long n, hipStream_t st);
/* decode launches under graph capture (attn_api.hip) */
struct smol_graph_dec;
extern "C" int smol_internal_gdec_create(smol_attn_ctx *ctx, int n_heads, int n_kv_heads, int hd, int plan_pos,
                                         smol_graph_dec **out);
extern "C" void smol_internal_gdec_destroy(smol_graph_dec *g);
extern "C" void smol_internal_gdec_capture(smol_attn_ctx *ctx, smol_graph_dec *g);
extern "C" int smol_internal_gdec_step(smol_attn_ctx *ctx, smol_graph_dec *g, int pos, int slot);

extern "C" int smol_internal_norm_rope_bf16_qk(smol_attn_ctx *ctx, const smol_rope_table *rope, uint16_t *q,
                                               const float *q_weight, uint16_t *k, const float *k_weight, float eps,
                                               int pos0, int seq, int n_heads, int n_kv_heads, int head_dim);
extern "C" int smol_internal_linear_bf16_ops(smol_attn_ctx *ctx, uint16_t *y, const void *x, int x_f32_trunc,
                                             const uint16_t *w, int seq, int in_dim, int out_dim, int act,
                                             const uint16_t *res16);
extern "C" int smol_internal_linear_qkv_bf16_norm(smol_attn_ctx *ctx, uint16_t *q, uint16_t *k, uint16_t *v,
                                                  const uint16_t *x, const float *norm_w, float eps,
                                                  const uint16_t *wq, const uint16_t *wk, const uint16_t *wv, int seq,
                                                  int in_dim, int q_dim, int kv_dim);
extern "C" int smol_internal_linear_bf16_addnorm_geglu(smol_attn_ctx *ctx, uint16_t *g, const uint16_t *x,
                                                       const uint16_t *p, uint16_t *x_new, const float *norm_w,
                                                       float eps, const uint16_t *w_gate_up, int seq, int in_dim,
                                                       int out_dim);

namespace {

int qfail(int code, const char *msg) { return smol_internal_fail(code, msg); }

#define QHIP(expr)                                                                          \
    do {                                                                                    \
        hipError_t e_ = (expr);                                                             \
        if (e_ != hipSuccess) return qfail(SMOL_ATTN_ERR_DEVICE, hipGetErrorString(e_));    \
    } while (0)

struct Buf {
    void *p = nullptr;
    size_t cap = 0;
};

struct Binding {
    unsigned long long serial = 0; /* tells a binding from a later one at the same address */
    smol_qkn_attn_config cfg{};
    hipStream_t stream = nullptr;
    smol_attn_ctx *ctx = nullptr;
    smol_kv_cache *kv = nullptr;
    smol_rope_table *rope_global = nullptr, *rope_local = nullptr;
    std::vector<int> sliding;
    std::vector<float *> q_norm, k_norm; /* device [head_dim] or null */
    Buf q, k, v, out32, out16;           /* staging */
    Buf lq, lk, lv, la, lp, lg;          /* a whole layer's activations (smol_qkn_layer_*) */
    Buf lx, lh;                          /* bf16 layer: normed input, GeGLU output */
};

std::mutex g_mu;
std::unordered_map<const void *, Binding *> g_bind;
unsigned long long g_serial = 0;

Binding *find(const void *owner) {
    std::lock_guard<std::mutex> lk(g_mu);
    auto it = g_bind.find(owner);
    return it == g_bind.end() ? nullptr : it->second;
}

/* grows a staging buffer; the binding's stream is drained first, since
 * earlier work on it may still read the old allocation */
int reserve(Binding *b, Buf &buf, size_t bytes) {
    if (bytes <= buf.cap) return 0;
    size_t want = std::max(bytes, buf.cap * 2);
    want = (want + 255) & ~(size_t)255;
    if (buf.p) {
        QHIP(hipStreamSynchronize(b->stream));
        QHIP(hipFree(buf.p));
        buf.p = nullptr;
        buf.cap = 0;
    }
    QHIP(hipMalloc(&buf.p, want));
    buf.cap = want;
    return 0;
}

void release(Binding *b) {
    if (!b) return;
    hipSetDevice(b->cfg.device);
    if (b->stream) hipStreamSynchronize(b->stream);
    for (float *p : b->q_norm)
        if (p) hipFree(p);
    for (float *p : b->k_norm)
        if (p) hipFree(p);
    for (Buf *x : {&b->q, &b->k, &b->v, &b->out32, &b->out16, &b->lq, &b->lk, &b->lv, &b->la, &b->lp, &b->lg, &b->lx, &b->lh})
        if (x->p) hipFree(x->p);
    if (b->kv) smol_kv_cache_destroy(b->kv);
    if (b->rope_global) smol_rope_table_destroy(b->rope_global);
    if (b->rope_local) smol_rope_table_destroy(b->rope_local);
    if (b->ctx) smol_attn_ctx_destroy(b->ctx);
    if (b->stream) hipStreamDestroy(b->stream);
    delete b;
}

bool hd_ok(int hd) { return hd == 64 || hd == 72 || hd == 80 || hd == 96 || hd == 128 || hd == 256; }

/* The whole block for seq_len rows at start_pos (decode: one launch of the
 * direct decode kernel when seq_len == 1 and `decode` is set). */
/* out32 (bf16 bindings on the device): non-NULL receives the fp32 result
 * and the bf16 conversion into attn_out is left to the caller (the layer's
 * o_proj truncates it as it loads it) */
int run_block(Binding *b, int layer, int start_pos, int seq_len, const void *q, const void *k, const void *v,
              void *attn_out, bool decode, bool sync = true, bool own_qk = false, float **out32 = nullptr) {
    const smol_qkn_attn_config &c = b->cfg;
    if (layer < 0 || layer >= c.n_layers) return qfail(SMOL_ATTN_ERR_ARG, "layer out of range");
    if (start_pos < 0 || seq_len <= 0) return qfail(SMOL_ATTN_ERR_ARG, "bad start_pos / seq_len");
    if (!q || !k || !v || !attn_out) return qfail(SMOL_ATTN_ERR_ARG, "NULL q / k / v / attn_out");
    QHIP(hipSetDevice(c.device));
    const int hd = c.head_dim;
    const size_t es = c.bf16 ? 2 : 4;
    const size_t q_elems = (size_t)seq_len * c.n_heads * hd, kv_elems = (size_t)seq_len * c.n_kv_heads * hd;
    const bool sliding = b->sliding[layer] != 0;
    const smol_rope_table *rope = sliding && b->rope_local ? b->rope_local : b->rope_global;
    const int window = sliding && c.sliding_window > 0 ? c.sliding_window : 0;
    const float cap = c.attn_logit_softcap > 0.0f ? c.attn_logit_softcap : 0.0f;
    const float scale = 1.0f / sqrtf((float)hd);
    int rc;

    /* device inputs: the caller's arrays when they are on the device and are
     * only read; staged copies otherwise (the bf16 contract rounds Q and K in
     * place, and the caller's inputs stay unmodified unless they are the
     * layer step's own scratch, own_qk) */
    const void *dq = q, *dk = k, *dv = v;
    const bool copy_qk = !c.on_device || (c.bf16 && !own_qk);
    const hipMemcpyKind kind = c.on_device ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice;
    if (copy_qk) {
        if ((rc = reserve(b, b->q, q_elems * es)) || (rc = reserve(b, b->k, kv_elems * es))) return rc;
        QHIP(hipMemcpyAsync(b->q.p, q, q_elems * es, kind, b->stream));
        QHIP(hipMemcpyAsync(b->k.p, k, kv_elems * es, kind, b->stream));
        dq = b->q.p;
        dk = b->k.p;
    }
    if (!c.on_device) {
        if ((rc = reserve(b, b->v, kv_elems * es))) return rc;
        QHIP(hipMemcpyAsync(b->v.p, v, kv_elems * es, kind, b->stream));
        dv = b->v.p;
    }
    /* the fp32 result: the caller's array when it is a device fp32 array */
    float *out = nullptr;
    if (c.bf16 || !c.on_device) {
        if ((rc = reserve(b, b->out32, q_elems * 4))) return rc;
        out = (float *)b->out32.p;
    } else {
        out = (float *)attn_out;
    }
    const float *qn = b->q_norm[layer], *kn = b->k_norm[layer];
    if (c.bf16) {
        /* per-head norm + rotation rounded by truncation, then the rows go
         * into the cache as their bits (no further rounding: bf16 in) */
        if ((rc = smol_internal_norm_rope_bf16_qk(b->ctx, rope, (uint16_t *)dq, qn, (uint16_t *)dk, kn, c.eps,
                                                  start_pos, seq_len, c.n_heads, c.n_kv_heads, hd)))
            return rc;
        if (decode) {
            const int slot = 0;
            rc = smol_attn_decode(b->ctx, b->kv, layer, nullptr, 1, &slot, &start_pos, dq, dk, dv, SMOL_ATTN_BF16,
                                  c.n_heads, scale, window, cap, out);
        } else {
            rc = smol_attn_prefill(b->ctx, b->kv, layer, 0, nullptr, start_pos, seq_len, dq, dk, dv, SMOL_ATTN_BF16,
                                   c.n_heads, scale, window, cap, out);
        }
        if (rc) return rc;
        if (out32 && c.on_device) {
            *out32 = out;
            return sync ? smol_attn_ctx_synchronize(b->ctx) : SMOL_ATTN_OK;
        }
        uint16_t *o16 = (uint16_t *)attn_out;
        if (!c.on_device) {
            if ((rc = reserve(b, b->out16, q_elems * 2))) return rc;
            o16 = (uint16_t *)b->out16.p;
        }
        if (smol_launch_to_bf16_trunc(out, o16, (long long)q_elems, b->stream))
            return qfail(SMOL_ATTN_ERR_DEVICE, "bf16 output conversion failed");
        if (!c.on_device) QHIP(hipMemcpyAsync(attn_out, o16, q_elems * 2, hipMemcpyDeviceToHost, b->stream));
    } else {
        if (decode) {
            const int slot = 0;
            rc = smol_attn_decode_qknorm(b->ctx, b->kv, layer, rope, 1, &slot, &start_pos, dq, dk, dv, SMOL_ATTN_F32,
                                         c.n_heads, scale, window, cap, qn, kn, c.eps, out);
        } else {
            rc = smol_attn_prefill_qknorm(b->ctx, b->kv, layer, 0, rope, start_pos, seq_len, dq, dk, dv, SMOL_ATTN_F32,
                                          c.n_heads, scale, window, cap, qn, kn, c.eps, out);
        }
        if (rc) return rc;
        if (!c.on_device) QHIP(hipMemcpyAsync(attn_out, out, q_elems * 4, hipMemcpyDeviceToHost, b->stream));
    }
    /* waits; SMOL_ATTN_ERR_RANGE when the prefill's fp16 staging overflowed */
    return sync ? smol_attn_ctx_synchronize(b->ctx) : SMOL_ATTN_OK;
}

/* One decoder layer on the device (qkn_decoder.c:633-705 for one token,
 * :470-560 for a prefill), x [n][dim] the residual stream, updated in place:
 *   q, k, v = (rmsnorm(x, input_norm)) Wq/Wk/Wv^T          one launch (n <= 4)
 *   attention block of the binding                           run_block
 *   Qwen3:   x += attn Wo^T;  g = act(rmsnorm(x, post_attn_norm) Wgu^T)
 *   Gemma 3: x += rmsnorm(attn Wo^T, post_attn_norm);
 *            g = act(rmsnorm(x, pre_ffn_norm) Wgu^T)
 *   x += g Wd^T, or x += rmsnorm(g Wd^T, post_ffn_norm) when that norm exists
 * Nothing waits for the device except the prefill's attention block (its
 * range check). */
int run_layer(Binding *b, int layer, int pos, int n, float *x, const smol_qkn_layer_weights *w, int dim, int inter,
              int act, bool decode) {
    const smol_qkn_attn_config &c = b->cfg;
    if (!c.on_device || c.bf16)
        return qfail(SMOL_ATTN_ERR_ARG, "the device layer step needs a binding with on_device = 1 and bf16 = 0");
    if (layer < 0 || layer >= c.n_layers) return qfail(SMOL_ATTN_ERR_ARG, "layer out of range");
    if (!x || !w || dim <= 0 || inter <= 0 || n <= 0 || pos < 0) return qfail(SMOL_ATTN_ERR_ARG, "bad layer arguments");
    if (act != SMOL_LINEAR_ACT_SWIGLU && act != SMOL_LINEAR_ACT_GEGLU)
        return qfail(SMOL_ATTN_ERR_ARG, "act must be SMOL_LINEAR_ACT_SWIGLU or SMOL_LINEAR_ACT_GEGLU");
    if (!w->input_norm || !w->wq || !w->wk || !w->wv || !w->wo || !w->post_attn_norm || !w->gate_up || !w->down)
        return qfail(SMOL_ATTN_ERR_ARG, "a required layer weight is NULL");
    QHIP(hipSetDevice(c.device));
    const int q_dim = c.n_heads * c.head_dim, kv_dim = c.n_kv_heads * c.head_dim;
    int rc;
    if ((rc = reserve(b, b->lq, (size_t)n * q_dim * 4)) || (rc = reserve(b, b->lk, (size_t)n * kv_dim * 4)) ||
        (rc = reserve(b, b->lv, (size_t)n * kv_dim * 4)) || (rc = reserve(b, b->la, (size_t)n * q_dim * 4)) ||
        (rc = reserve(b, b->lp, (size_t)n * dim * 4)) || (rc = reserve(b, b->lg, (size_t)n * inter * 4)))
        return rc;
    float *q = (float *)b->lq.p, *k = (float *)b->lk.p, *v = (float *)b->lv.p;
    float *attn = (float *)b->la.p, *p = (float *)b->lp.p, *g = (float *)b->lg.p;
    smol_attn_ctx *ctx = b->ctx;
    if ((rc = smol_linear_qkv_norm_dev(ctx, q, k, v, x, w->wq, w->wk, w->wv, n, dim, q_dim, kv_dim, w->input_norm,
                                       c.eps)))
        return rc;
    if ((rc = run_block(b, layer, pos, n, q, k, v, attn, decode, !decode))) return rc;
    smol_linear_ops ops{};
    if (w->pre_ffn_norm) {
        if ((rc = smol_linear_ops_dev(ctx, p, attn, w->wo, nullptr, n, q_dim, dim, nullptr))) return rc;
        if ((rc = smol_rms_norm_dev(ctx, x, p, w->post_attn_norm, x, n, dim, c.eps))) return rc;
        ops.norm_weight = w->pre_ffn_norm;
    } else {
        ops.residual = x;
        if ((rc = smol_linear_ops_dev(ctx, x, attn, w->wo, nullptr, n, q_dim, dim, &ops))) return rc;
        ops.residual = nullptr;
        ops.norm_weight = w->post_attn_norm;
    }
    ops.norm_eps = c.eps;
    ops.act = act;
    if ((rc = smol_linear_ops_dev(ctx, g, x, w->gate_up, nullptr, n, dim, 2 * inter, &ops))) return rc;
    if (w->post_ffn_norm) {
        if ((rc = smol_linear_ops_dev(ctx, p, g, w->down, nullptr, n, inter, dim, nullptr))) return rc;
        return smol_rms_norm_dev(ctx, x, p, w->post_ffn_norm, x, n, dim, c.eps);
    }
    smol_linear_ops res{};
    res.residual = x;
    return smol_linear_ops_dev(ctx, x, g, w->down, nullptr, n, inter, dim, &res);
}

/* One bf16 decoder layer on the device (qkn_bf16_decoder.c:634-697 for one
 * token, :482-571 for a prefill), x [n][dim] bf16, updated in place; every
 * step truncates to bf16:
 *   xn = norm(x, input_norm)                                  k_bf16_rows
 *   q, k, v = xn (Wq, Wk, Wv)^T                               one launch (n <= 4)
 *   attention block of the binding (Q, K rounded in place)    run_block
 *   p = attn Wo^T
 *   x = x + (pre_ffn_norm ? norm(p, post_attn_norm) : p);
 *   xn = norm(x, pre_ffn_norm or post_attn_norm)              k_bf16_rows
 *   g = geglu(xn Wgu^T); f = g Wd^T
 *   x = x + (post_ffn_norm ? norm(f, post_ffn_norm) : f)      k_bf16_rows */
int run_layer_bf16(Binding *b, int layer, int pos, int n, uint16_t *x, const smol_qkn_layer_weights *w, int dim,
                   int inter, bool decode) {
    const smol_qkn_attn_config &c = b->cfg;
    if (!c.on_device || !c.bf16)
        return qfail(SMOL_ATTN_ERR_ARG, "the bf16 device layer step needs a binding with on_device = 1 and bf16 = 1");
    if (layer < 0 || layer >= c.n_layers) return qfail(SMOL_ATTN_ERR_ARG, "layer out of range");
    if (!x || !w || dim <= 0 || inter <= 0 || n <= 0 || pos < 0) return qfail(SMOL_ATTN_ERR_ARG, "bad layer arguments");
    if (!w->input_norm || !w->wq || !w->wk || !w->wv || !w->wo || !w->post_attn_norm || !w->gate_up || !w->down)
        return qfail(SMOL_ATTN_ERR_ARG, "a required layer weight is NULL");
    QHIP(hipSetDevice(c.device));
    const int q_dim = c.n_heads * c.head_dim, kv_dim = c.n_kv_heads * c.head_dim;
    int rc;
    if ((rc = reserve(b, b->lq, (size_t)n * q_dim * 2)) || (rc = reserve(b, b->lk, (size_t)n * kv_dim * 2)) ||
        (rc = reserve(b, b->lv, (size_t)n * kv_dim * 2)) || (rc = reserve(b, b->la, (size_t)n * q_dim * 2)) ||
        (rc = reserve(b, b->lp, (size_t)n * dim * 2)) || (rc = reserve(b, b->lg, (size_t)n * 2 * inter * 2)) ||
        (rc = reserve(b, b->lx, (size_t)n * dim * 2)) || (rc = reserve(b, b->lh, (size_t)n * inter * 2)))
        return rc;
    uint16_t *q = (uint16_t *)b->lq.p, *k = (uint16_t *)b->lk.p, *v = (uint16_t *)b->lv.p;
    uint16_t *attn = (uint16_t *)b->la.p, *p = (uint16_t *)b->lp.p, *gu = (uint16_t *)b->lg.p;
    uint16_t *xn = (uint16_t *)b->lx.p, *g = (uint16_t *)b->lh.p;
    smol_attn_ctx *ctx = b->ctx;
    const int BF = SMOL_ATTN_BF16;
    /* a few rows: the input norm inside the Q/K/V GEMV (the same bits, one launch fewer) */
    rc = n <= SMOL_LINEAR_GEMV_MAX_SEQ ? smol_internal_linear_qkv_bf16_norm(ctx, q, k, v, x, w->input_norm, c.eps, w->wq,
                                                                           w->wk, w->wv, n, dim, q_dim, kv_dim)
                                      : 1;
    if (rc < 0) return rc;
    if (rc == 1) {
        if ((rc = smol_bf16_rms_norm_dev(ctx, xn, x, w->input_norm, n, dim, c.eps))) return rc;
        if ((rc = smol_linear_qkv_dev(ctx, q, k, v, BF, xn, BF, w->wq, w->wk, w->wv, n, dim, q_dim, kv_dim))) return rc;
    }
    /* a few rows (decode): the GEMV launches take the attention output as
     * fp32 and truncate it as they load it, and fold GeGLU into gate_up and
     * the last residual add into down (the same truncations, three launches
     * fewer) */
    const bool few = n <= SMOL_LINEAR_GEMV_MAX_SEQ;
    float *attn32 = nullptr;
    if ((rc = run_block(b, layer, pos, n, q, k, v, attn, decode, !decode, true, few ? &attn32 : nullptr))) return rc;
    if (few && attn32) {
        if ((rc = smol_internal_linear_bf16_ops(ctx, p, attn32, 1, w->wo, n, q_dim, dim, SMOL_LINEAR_ACT_NONE,
                                                nullptr)))
            return rc;
    } else if ((rc = smol_linear_dev(ctx, p, BF, attn, BF, w->wo, nullptr, n, q_dim, dim))) {
        return rc;
    }
    if (few && !w->pre_ffn_norm && !w->post_ffn_norm) {
        /* the residual add and the post-attention norm inside the gate_up
         * GEMV (the same bits; x + p goes to xn, which the down GEMV adds
         * its result to, writing x) */
        rc = smol_internal_linear_bf16_addnorm_geglu(ctx, g, x, p, xn, w->post_attn_norm, c.eps, w->gate_up, n, dim,
                                                     2 * inter);
        if (rc < 0) return rc;
        if (rc == 0)
            return smol_internal_linear_bf16_ops(ctx, x, g, 0, w->down, n, inter, dim, SMOL_LINEAR_ACT_NONE, xn);
    }
    if (w->pre_ffn_norm)
        rc = smol_bf16_add_norm_dev(ctx, x, p, w->post_attn_norm, w->pre_ffn_norm, xn, n, dim, c.eps);
    else
        rc = smol_bf16_add_norm_dev(ctx, x, p, nullptr, w->post_attn_norm, xn, n, dim, c.eps);
    if (rc) return rc;
    if (few) {
        if ((rc = smol_internal_linear_bf16_ops(ctx, g, xn, 0, w->gate_up, n, dim, 2 * inter, SMOL_LINEAR_ACT_GEGLU,
                                                nullptr)))
            return rc;
        if (!w->post_ffn_norm)
            return smol_internal_linear_bf16_ops(ctx, x, g, 0, w->down, n, inter, dim, SMOL_LINEAR_ACT_NONE, x);
    } else {
        if ((rc = smol_linear_dev(ctx, gu, BF, xn, BF, w->gate_up, nullptr, n, dim, 2 * inter))) return rc;
        if ((rc = smol_bf16_geglu_dev(ctx, g, gu, n, inter))) return rc;
    }
    if ((rc = smol_linear_dev(ctx, p, BF, g, BF, w->down, nullptr, n, inter, dim))) return rc;
    return smol_bf16_add_norm_dev(ctx, x, p, w->post_ffn_norm, nullptr, nullptr, n, dim, c.eps);
}

}  // namespace

extern "C" int smol_qkn_layer_forward(const void *owner, int layer, int pos, float *x,
                                      const smol_qkn_layer_weights *w, int dim, int intermediate, int act) {
    Binding *b = find(owner);
    if (!b) return qfail(SMOL_ATTN_ERR_ARG, "owner is not bound");
    return run_layer(b, layer, pos, 1, x, w, dim, intermediate, act, true);
}

extern "C" int smol_qkn_layer_prefill(const void *owner, int layer, int start_pos, int seq_len, float *x,
                                      const smol_qkn_layer_weights *w, int dim, int intermediate, int act) {
    Binding *b = find(owner);
    if (!b) return qfail(SMOL_ATTN_ERR_ARG, "owner is not bound");
    return run_layer(b, layer, start_pos, seq_len, x, w, dim, intermediate, act, false);
}

extern "C" int smol_qkn_layer_forward_bf16(const void *owner, int layer, int pos, uint16_t *x,
                                           const smol_qkn_layer_weights *w, int dim, int intermediate) {
    Binding *b = find(owner);
    if (!b) return qfail(SMOL_ATTN_ERR_ARG, "owner is not bound");
    return run_layer_bf16(b, layer, pos, 1, x, w, dim, intermediate, true);
}

extern "C" int smol_qkn_layer_prefill_bf16(const void *owner, int layer, int start_pos, int seq_len, uint16_t *x,
                                           const smol_qkn_layer_weights *w, int dim, int intermediate) {
    Binding *b = find(owner);
    if (!b) return qfail(SMOL_ATTN_ERR_ARG, "owner is not bound");
    return run_layer_bf16(b, layer, start_pos, seq_len, x, w, dim, intermediate, false);
}

/* ---- one decode step of every layer as a HIP graph ---- */

struct smol_qkn_step_graph {
    const void *owner = nullptr;
    unsigned long long serial = 0;
    smol_graph_dec *gd = nullptr;
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    int max_pos = 0;
    std::vector<const void *> fp; /* what the captured launches were built on */
};

namespace {

/* the binding's buffers and capacities that captured launches point into:
 * if any of them changes, the graph would read freed memory */
std::vector<const void *> fingerprint(const Binding *b) {
    std::vector<const void *> f{b->lq.p, b->lk.p, b->lv.p, b->la.p, b->lp.p, b->lg.p};
    for (float *p : b->q_norm) f.push_back(p);
    for (float *p : b->k_norm) f.push_back(p);
    f.push_back(reinterpret_cast<const void *>((intptr_t)smol_kv_cache_capacity(b->kv)));
    f.push_back(reinterpret_cast<const void *>((intptr_t)smol_rope_table_capacity(b->rope_global)));
    f.push_back(reinterpret_cast<const void *>((intptr_t)smol_rope_table_capacity(b->rope_local)));
    return f;
}

void destroy_graph(smol_qkn_step_graph *g) {
    if (g->exec) hipGraphExecDestroy(g->exec);
    if (g->graph) hipGraphDestroy(g->graph);
    smol_internal_gdec_destroy(g->gd);
    delete g;
}

}  // namespace

extern "C" int smol_qkn_step_graph_create(const void *owner, float *x, const smol_qkn_layer_weights *w, int dim,
                                          int intermediate, int act, int max_pos, smol_qkn_step_graph **out) {
    if (!out) return qfail(SMOL_ATTN_ERR_ARG, "NULL out");
    *out = nullptr;
    Binding *b = find(owner);
    if (!b) return qfail(SMOL_ATTN_ERR_ARG, "owner is not bound");
    const smol_qkn_attn_config &c = b->cfg;
    if (!c.on_device || c.bf16)
        return qfail(SMOL_ATTN_ERR_ARG, "a step graph needs a binding with on_device = 1 and bf16 = 0");
    if (!x || !w || dim <= 0 || intermediate <= 0 || max_pos <= 0) return qfail(SMOL_ATTN_ERR_ARG, "bad step graph arguments");
    if (c.n_layers > 254) return qfail(SMOL_ATTN_ERR_UNSUPPORTED, "a step graph holds at most 254 layers");
    QHIP(hipSetDevice(c.device));
    const int q_dim = c.n_heads * c.head_dim, kv_dim = c.n_kv_heads * c.head_dim;
    int rc;
    /* everything the step touches is sized first: nothing may be allocated
     * while the launches are captured */
    if ((rc = smol_kv_cache_reserve(b->kv, max_pos))) return rc;
    if ((rc = smol_rope_table_ensure(b->rope_global, max_pos))) return rc;
    if (b->rope_local && (rc = smol_rope_table_ensure(b->rope_local, max_pos))) return rc;
    if ((rc = reserve(b, b->lq, (size_t)q_dim * 4)) || (rc = reserve(b, b->lk, (size_t)kv_dim * 4)) ||
        (rc = reserve(b, b->lv, (size_t)kv_dim * 4)) || (rc = reserve(b, b->la, (size_t)q_dim * 4)) ||
        (rc = reserve(b, b->lp, (size_t)dim * 4)) || (rc = reserve(b, b->lg, (size_t)intermediate * 4)))
        return rc;
    auto *g = new smol_qkn_step_graph();
    g->owner = owner;
    g->serial = b->serial;
    g->max_pos = max_pos;
    if ((rc = smol_internal_gdec_create(b->ctx, c.n_heads, c.n_kv_heads, c.head_dim, max_pos - 1, &g->gd))) {
        destroy_graph(g);
        return rc;
    }
    hipError_t e = hipStreamSynchronize(b->stream);
    if (e == hipSuccess) e = hipStreamBeginCapture(b->stream, hipStreamCaptureModeThreadLocal);
    if (e != hipSuccess) {
        destroy_graph(g);
        return qfail(SMOL_ATTN_ERR_DEVICE, hipGetErrorString(e));
    }
    smol_internal_gdec_capture(b->ctx, g->gd);
    for (int l = 0; l < c.n_layers && !rc; l++)
        rc = run_layer(b, l, max_pos - 1, 1, x, &w[l], dim, intermediate, act, true);
    smol_internal_gdec_capture(b->ctx, nullptr);
    e = hipStreamEndCapture(b->stream, &g->graph);
    if (!rc && e == hipSuccess) e = hipGraphInstantiate(&g->exec, g->graph, nullptr, nullptr, 0);
    if (rc || e != hipSuccess) {
        destroy_graph(g);
        return rc ? rc : qfail(SMOL_ATTN_ERR_DEVICE, hipGetErrorString(e));
    }
    g->fp = fingerprint(b);
    *out = g;
    return SMOL_ATTN_OK;
}

extern "C" int smol_qkn_step_graph_launch(smol_qkn_step_graph *g, int pos) {
    if (!g) return qfail(SMOL_ATTN_ERR_ARG, "NULL graph");
    Binding *b = find(g->owner);
    if (!b || b->serial != g->serial) return qfail(SMOL_ATTN_ERR_ARG, "the graph's binding is gone");
    if (pos < 0 || pos >= g->max_pos) return qfail(SMOL_ATTN_ERR_ARG, "pos outside the graph's [0, max_pos)");
    if (fingerprint(b) != g->fp)
        return qfail(SMOL_ATTN_ERR_ARG, "a buffer, cache or table of the binding was reallocated since the capture; "
                                        "create the graph again");
    QHIP(hipSetDevice(b->cfg.device));
    if (int rc = smol_internal_gdec_step(b->ctx, g->gd, pos, 0)) return rc;
    QHIP(hipGraphLaunch(g->exec, b->stream));
    return SMOL_ATTN_OK;
}

extern "C" int smol_qkn_step_graph_destroy(smol_qkn_step_graph *g) {
    if (!g) return SMOL_ATTN_OK;
    Binding *b = find(g->owner);
    if (b && b->serial == g->serial) {
        hipSetDevice(b->cfg.device);
        hipStreamSynchronize(b->stream);
    }
    destroy_graph(g);
    return SMOL_ATTN_OK;
}

extern "C" int smol_qkn_layer_synchronize(const void *owner) {
    Binding *b = find(owner);
    if (!b) return qfail(SMOL_ATTN_ERR_ARG, "owner is not bound");
    return smol_attn_ctx_synchronize(b->ctx);
}

extern "C" void *smol_qkn_attn_stream(const void *owner) {
    Binding *b = find(owner);
    return b ? (void *)b->stream : nullptr;
}

extern "C" int smol_qkn_attn_bind(const void *owner, const smol_qkn_attn_config *cfg) {
    if (!owner || !cfg) return qfail(SMOL_ATTN_ERR_ARG, "NULL owner / config");
    const smol_qkn_attn_config &c = *cfg;
    if (c.n_layers <= 0 || c.n_heads <= 0 || c.n_kv_heads <= 0 || c.n_heads % c.n_kv_heads || !hd_ok(c.head_dim) ||
        c.max_seq <= 0 || !(c.rope_theta > 0.0f) || !(c.eps >= 0.0f))
        return qfail(SMOL_ATTN_ERR_ARG, "bad decoder config");
    if (!c.bf16 && c.rope_type != SMOL_ROPE_NEOX && c.rope_type != SMOL_ROPE_INTERLEAVED)
        return qfail(SMOL_ATTN_ERR_ARG, "rope_type must be SMOL_ROPE_NEOX or SMOL_ROPE_INTERLEAVED");
    const int n_dev = smol_attn_device_count();
    if (n_dev < 0) return n_dev;
    if (c.device < 0 || c.device >= n_dev) return qfail(SMOL_ATTN_ERR_ARG, "device ordinal out of range");
    smol_qkn_attn_unbind(owner);
    Binding *b = new Binding();
    b->cfg = c;
    {
        std::lock_guard<std::mutex> lk(g_mu);
        b->serial = ++g_serial;
    }
    b->sliding.assign(c.n_layers, 0);
    b->q_norm.assign(c.n_layers, nullptr);
    b->k_norm.assign(c.n_layers, nullptr);
    int rc = SMOL_ATTN_OK;
    hipError_t e = hipSetDevice(c.device);
    if (e == hipSuccess) e = hipStreamCreateWithFlags(&b->stream, hipStreamNonBlocking);
    if (e != hipSuccess) rc = qfail(SMOL_ATTN_ERR_DEVICE, hipGetErrorString(e));
    if (!rc) rc = smol_attn_ctx_create(c.device, b->stream, &b->ctx);
    if (!rc) rc = smol_kv_cache_create(b->ctx, c.n_layers, 1, c.n_kv_heads, c.head_dim, c.max_seq, &b->kv);
    /* the bf16 decoder rotates interleaved pairs whatever rope_type says
     * (bf16_apply_rope_interleaved, qkn_bf16_decoder.c:522-523) */
    const int rt = c.bf16 ? SMOL_ROPE_INTERLEAVED : c.rope_type;
    const int rcap = std::max(1024, c.max_seq);
    if (!rc) rc = smol_rope_table_create(b->ctx, c.head_dim, c.rope_theta, rt, rcap, &b->rope_global);
    /* a local table only when its theta differs (qkn_decoder.c:326-337);
     * the bf16 decoder builds one for any local theta > 0 (:368-370), whose
     * rows equal the global ones when the thetas are equal */
    if (!rc && c.rope_local_theta > 0.0f && c.rope_local_theta != c.rope_theta)
        rc = smol_rope_table_create(b->ctx, c.head_dim, c.rope_local_theta, rt, rcap, &b->rope_local);
    if (rc) {
        release(b);
        return rc;
    }
    std::lock_guard<std::mutex> lk(g_mu);
    g_bind[owner] = b;
    return SMOL_ATTN_OK;
}

extern "C" int smol_qkn_attn_set_layer(const void *owner, int layer, int is_sliding, const float *q_norm_weight,
                                       const float *k_norm_weight) {
    Binding *b = find(owner);
    if (!b) return qfail(SMOL_ATTN_ERR_ARG, "owner is not bound");
    if (layer < 0 || layer >= b->cfg.n_layers) return qfail(SMOL_ATTN_ERR_ARG, "layer out of range");
    QHIP(hipSetDevice(b->cfg.device));
    QHIP(hipStreamSynchronize(b->stream));
    b->sliding[layer] = is_sliding ? 1 : 0;
    const size_t bytes = (size_t)b->cfg.head_dim * sizeof(float);
    const float *src[2] = {q_norm_weight, k_norm_weight};
    float **dst[2] = {&b->q_norm[layer], &b->k_norm[layer]};
    for (int i = 0; i < 2; i++) {
        if (!src[i]) {
            if (*dst[i]) QHIP(hipFree(*dst[i]));
            *dst[i] = nullptr;
            continue;
        }
        if (!*dst[i]) QHIP(hipMalloc((void **)dst[i], bytes));
        QHIP(hipMemcpy(*dst[i], src[i], bytes, hipMemcpyHostToDevice));
    }
    return SMOL_ATTN_OK;
}

extern "C" int smol_qkn_attn_prefill(const void *owner, int layer, int start_pos, int seq_len, const void *q,
                                     const void *k, const void *v, void *attn_out) {
    Binding *b = find(owner);
    if (!b) return qfail(SMOL_ATTN_ERR_ARG, "owner is not bound");
    return run_block(b, layer, start_pos, seq_len, q, k, v, attn_out, false);
}

extern "C" int smol_qkn_attn_forward(const void *owner, int layer, int pos, const void *q, const void *k,
                                     const void *v, void *attn_out) {
    Binding *b = find(owner);
    if (!b) return qfail(SMOL_ATTN_ERR_ARG, "owner is not bound");
    return run_block(b, layer, pos, 1, q, k, v, attn_out, true);
}

extern "C" int smol_qkn_attn_read_cache(const void *owner, int layer, int pos0, int n, uint16_t *k_out,
                                        uint16_t *v_out) {
    Binding *b = find(owner);
    if (!b) return qfail(SMOL_ATTN_ERR_ARG, "owner is not bound");
    return smol_kv_cache_read(b->kv, layer, 0, pos0, n, k_out, v_out);
}

extern "C" int smol_qkn_attn_unbind(const void *owner) {
    Binding *b = nullptr;
    {
        std::lock_guard<std::mutex> lk(g_mu);
        auto it = g_bind.find(owner);
        if (it == g_bind.end()) return SMOL_ATTN_OK;
        b = it->second;
        g_bind.erase(it);
    }
    release(b);
    return SMOL_ATTN_OK;
}
