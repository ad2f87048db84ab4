/*
 * smol_qkn_attn.h - the attention block of the reference decoders on the
 * GPU, for a decoder context identified by its address.
 *
 * Per layer, one call replaces the block between the Q/K/V projections and
 * the output projection:
 *   per-head Q/K RMSNorm, the choice of the global- or local-theta RoPE
 *   table, RoPE on Q and the new K rows, the KV-cache write, and the
 *   (is_sliding && sliding_window > 0, attn_logit_softcap > 0) dispatch over
 *   the four attention entry points, with scale 1/sqrtf(head_dim):
 *     qkn_decoder_prefill       common/decoder/qkn_decoder.c:460-528
 *     qkn_decoder_forward       common/decoder/qkn_decoder.c:625-677
 *     qkn_bf16_decoder_prefill  common/decoder/qkn_bf16_decoder.c:486-546
 *     qkn_bf16_decoder_forward  common/decoder/qkn_bf16_decoder.c:638-674
 *
 * The decoder contexts (qkn_ctx_t, qkn_decoder.h:95-144; qkn_bf16_ctx_t,
 * qkn_bf16_decoder.h:22-66) are caller-allocated structs whose layout is
 * ABI: callers calloc them, free() their cache pointers and assign
 * kv_cache_len. The device state (KV cache, RoPE tables, norm weights,
 * staging) therefore lives in a registry keyed by the context pointer
 * (`owner`), and the decoder's own kv_cache_len stays the source of truth:
 * each call takes the position the decoder computed from it (start_pos /
 * pos). A rewind (qwen_asr.c:1609 assigns kv_cache_len) is a smaller
 * position on the next call; qkn_kv_cache_reset (qkn_decoder.h:165-167) and
 * qkn_bf16_kv_cache_reset (qkn_bf16_decoder.c:309-311) only set the length
 * to 0, so they need no device call. The device cache is bf16
 * [layer][kv_head][pos][head_dim], post-RoPE, and grows by doubling.
 *
 * Two rounding contracts, chosen per binding:
 *   bf16 = 0  qkn_decoder.c: fp32 Q/K/V projections in, fp32 attn_out.
 *             Norm and RoPE run in fp32; the new rows are used at fp32 by
 *             the call that appends them and are stored in bf16 (round to
 *             nearest even) for later calls.
 *   bf16 = 1  qkn_bf16_decoder.c: bf16 Q/K/V in, bf16 attn_out rounded by
 *             truncation. Norm and the (always interleaved) rotation round
 *             to bf16 by truncation after each step, as
 *             smol_attn_norm_rope_bf16 states; the rotated K rows and the V
 *             rows are appended as their bf16 bits (a byte copy, :525-531).
 *
 * Errors: every function returns SMOL_ATTN_OK or a negative SMOL_ATTN_ERR_*
 * code and leaves a message in smol_attn_last_error(); the decoders map a
 * failure to their existing silent return (qkn_decoder.c:383-389) or
 * sentinel token (:605-611; 1 in qkn_bf16_decoder.c:626-629). A prefill
 * whose fp16 staging overflowed (a normed, rotated Q or K value times the
 * softmax scale, or a V value, at or beyond 65520 in magnitude) returns
 * SMOL_ATTN_ERR_RANGE; its attn_out is not valid, and the rows it appended
 * to the cache are.
 *
 * Threading: one binding is used by one thread at a time (the decoders'
 * contexts are single-threaded); the registry itself is thread-safe.
 */
#ifndef SMOL_QKN_ATTN_H
#define SMOL_QKN_ATTN_H

#include "smol_attn.h"

#ifdef __cplusplus
extern "C" {
#endif

/* The qkn_config_t fields the attention block reads (qkn_decoder.h:75-93) */
typedef struct {
    int n_layers;             /* dec_layers */
    int n_heads;              /* dec_heads */
    int n_kv_heads;           /* dec_kv_heads */
    int head_dim;             /* dec_head_dim: 64, 72, 80, 96, 128 or 256 */
    float eps;                /* dec_rms_norm_eps (per-head Q/K norm) */
    float rope_theta;         /* dec_rope_theta */
    float rope_local_theta;   /* dec_rope_local_theta: sliding layers rotate with it when it is
                               * > 0 and differs from rope_theta (qkn_decoder.c:326-337) */
    int rope_type;            /* SMOL_ROPE_NEOX or SMOL_ROPE_INTERLEAVED (ignored when bf16 = 1:
                               * the bf16 decoder always rotates interleaved pairs) */
    int sliding_window;       /* > 0: window of the layers marked sliding */
    float attn_logit_softcap; /* > 0: cap * tanh(score / cap) */
    int bf16;                 /* rounding contract, see above */
    int on_device;            /* 1: q, k, v, attn_out are device pointers; 0: host arrays */
    int device;               /* GPU ordinal */
    int max_seq;              /* initial cache positions (>= 1; grows by doubling) */
} smol_qkn_attn_config;

/* Creates the device state of `owner` (or replaces it when owner is already
 * bound). No weights are needed: layers start non-sliding, without norms. */
SMOL_ATTN_API int smol_qkn_attn_bind(const void *owner, const smol_qkn_attn_config *cfg);

/* Layer fields the block reads (qkn_dec_layer_t, qkn_decoder.h:38-67):
 * is_sliding and the per-head norm weights, host fp32 [head_dim] copied to
 * the device (NULL: no norm for Q or K, as a NULL q_norm_weight /
 * k_norm_weight skips it, qkn_decoder.c:487-491). */
SMOL_ATTN_API int smol_qkn_attn_set_layer(const void *owner, int layer, int is_sliding,
                                          const float *q_norm_weight, const float *k_norm_weight);

/* One layer of prefill over positions [start_pos, start_pos + seq_len):
 * q [seq_len][n_heads*hd], k, v [seq_len][n_kv*hd] are the projections
 * (before the per-head norm), attn_out [seq_len][n_heads*hd] receives the
 * attention output. Element types follow the binding's contract (fp32, or
 * bf16 bits as uint16_t). The inputs are not modified. Returns when attn_out
 * is valid. */
SMOL_ATTN_API int smol_qkn_attn_prefill(const void *owner, int layer, int start_pos, int seq_len,
                                        const void *q, const void *k, const void *v,
                                        void *attn_out);

/* One layer of a single-token decode step at position pos (the prefill
 * call with seq_len 1, run as one decode launch). */
SMOL_ATTN_API int smol_qkn_attn_forward(const void *owner, int layer, int pos, const void *q,
                                        const void *k, const void *v, void *attn_out);

/* Reads cache rows [pos0, pos0 + n) of one layer back as bf16 bits
 * [n][n_kv*hd] (host arrays); for tests and for exporting a cache. */
SMOL_ATTN_API int smol_qkn_attn_read_cache(const void *owner, int layer, int pos0, int n,
                                           uint16_t *k_out, uint16_t *v_out);

/* Releases the device state of owner (call before freeing the decoder
 * context). Unbinding an unknown owner is not an error. */
SMOL_ATTN_API int smol_qkn_attn_unbind(const void *owner);

/* ---- the whole decoder layer on the device ------------------------------
 *
 * With the projections on the GPU (smol_linear.h), a binding with
 * on_device = 1 and bf16 = 0 runs a complete layer of qkn_decoder_forward
 * (common/decoder/qkn_decoder.c:633-705) or of qkn_decoder_prefill
 * (:470-560) per call, the residual stream x staying in device memory:
 *
 *   q, k, v  = rmsnorm(x, input_norm) (Wq, Wk, Wv)^T
 *   attn     = the attention block above (per-head norm, RoPE, cache, attention)
 *   Qwen3   (pre_ffn_norm NULL): x += attn Wo^T; h = rmsnorm(x, post_attn_norm)
 *   Gemma 3 (pre_ffn_norm set):  x += rmsnorm(attn Wo^T, post_attn_norm);
 *                                h = rmsnorm(x, pre_ffn_norm)
 *   g        = act(h Wgu^T)     rows of gate_up are (gate j, up j) pairs
 *   x       += g Wd^T, or rmsnorm(g Wd^T, post_ffn_norm) when that is set
 *
 * For one token that is five launches (the norms, the activation and the
 * residual adds are fused into the projections). All pointers are device
 * pointers on the binding's device; the weights are the decoder's own
 * tensors (bf16 [out][in] row-major, fp32 norm weights) copied to the device
 * once by the caller. Calls are enqueued on the binding's stream
 * (smol_qkn_attn_stream) and return without waiting, except the prefill,
 * which waits for its attention block (SMOL_ATTN_ERR_RANGE check).
 * smol_qkn_layer_synchronize waits for the stream. */
typedef struct {
    const float *input_norm;     /* [dim] */
    const uint16_t *wq;          /* [n_heads * head_dim][dim] */
    const uint16_t *wk, *wv;     /* [n_kv_heads * head_dim][dim] */
    const uint16_t *wo;          /* [dim][n_heads * head_dim] */
    const float *post_attn_norm; /* [dim] */
    const float *pre_ffn_norm;   /* [dim] or NULL (Gemma 3 post-sublayer norms when set) */
    const float *post_ffn_norm;  /* [dim] or NULL */
    const uint16_t *gate_up;     /* [2 * intermediate][dim] */
    const uint16_t *down;        /* [dim][intermediate] */
} smol_qkn_layer_weights;

/* act: SMOL_LINEAR_ACT_SWIGLU or SMOL_LINEAR_ACT_GEGLU (qkn_decoder.c:548-551).
 * x [1][dim] at position pos (forward) or [seq_len][dim] from start_pos (prefill). */
SMOL_ATTN_API int smol_qkn_layer_forward(const void *owner, int layer, int pos, float *x,
                                         const smol_qkn_layer_weights *w, int dim, int intermediate, int act);
SMOL_ATTN_API int smol_qkn_layer_prefill(const void *owner, int layer, int start_pos, int seq_len, float *x,
                                         const smol_qkn_layer_weights *w, int dim, int intermediate, int act);

/* The bf16 decoder's whole layer (a binding with on_device = 1 and bf16 = 1):
 * qkn_bf16_decoder_forward's layer loop (qkn_bf16_decoder.c:634-697) for one
 * token at pos, qkn_bf16_decoder_prefill's (:482-571) for seq_len rows from
 * start_pos. x [rows][dim] bf16, updated in place; every step truncates to
 * bf16 (smol_linear.h's bf16 row operations, the bf16 projections and the
 * bf16 attention block above):
 *   xn = norm(x, input_norm); q, k, v = xn (Wq, Wk, Wv)^T
 *   attn = the attention block; p = attn Wo^T
 *   pre_ffn_norm set: x = x + norm(p, post_attn_norm); h = norm(x, pre_ffn_norm)
 *   otherwise:        x = x + p;                         h = norm(x, post_attn_norm)
 *   f = geglu(h Wgu^T) Wd^T, normed by post_ffn_norm when set; x = x + f
 * The FFN is always GeGLU, as in the reference's bf16 decoder. Waiting
 * behaviour as for the fp32 layer calls. */
SMOL_ATTN_API int smol_qkn_layer_forward_bf16(const void *owner, int layer, int pos, uint16_t *x,
                                              const smol_qkn_layer_weights *w, int dim, int intermediate);
SMOL_ATTN_API int smol_qkn_layer_prefill_bf16(const void *owner, int layer, int start_pos, int seq_len, uint16_t *x,
                                              const smol_qkn_layer_weights *w, int dim, int intermediate);
SMOL_ATTN_API int smol_qkn_layer_synchronize(const void *owner);

/* ---- a whole decode step as one HIP graph -------------------------------
 *
 * No counterpart in the reference: qkn_decoder_forward's per-token layer
 * loop issues five device launches per layer through the calls above; a
 * step graph captures the loop over every layer once and replays it, so a
 * token costs two launches (a one-thread kernel that writes the position,
 * then the graph). For a binding with on_device = 1 and bf16 = 0:
 *
 *   create: sizes the cache, the RoPE tables and the layer buffers for
 *           positions [0, max_pos), then captures smol_qkn_layer_forward of
 *           layers 0 .. n_layers - 1 on x [1][dim] (device fp32, the residual
 *           stream) with the weights w[0 .. n_layers - 1]. The decode launches
 *           are planned for a key length of max_pos (a shorter sequence runs
 *           the same workgroups, some of them over no keys) and keep their
 *           split partials and flags in the graph's own device memory.
 *   launch: one decode step at pos (0 <= pos < max_pos), exactly what the
 *           layer loop of smol_qkn_layer_forward calls at pos computes. x, the
 *           weights and the binding's norms must be the captured ones, still
 *           allocated; the call fails (SMOL_ATTN_ERR_ARG) when a layer buffer,
 *           the cache or a RoPE table of the binding was reallocated since
 *           the capture (a longer prefill, for instance): create it again.
 *   destroy: waits for the binding's stream, then frees the graph.
 *
 * Launches are enqueued on the binding's stream and return without waiting;
 * smol_qkn_layer_synchronize waits and reports a merge time-out. One graph is
 * replayed by one thread at a time. */
typedef struct smol_qkn_step_graph smol_qkn_step_graph;
SMOL_ATTN_API int smol_qkn_step_graph_create(const void *owner, float *x, const smol_qkn_layer_weights *w, int dim,
                                             int intermediate, int act, int max_pos, smol_qkn_step_graph **out);
SMOL_ATTN_API int smol_qkn_step_graph_launch(smol_qkn_step_graph *g, int pos);
SMOL_ATTN_API int smol_qkn_step_graph_destroy(smol_qkn_step_graph *g);
/* the binding's stream (a hipStream_t), for ordering the caller's own work */
SMOL_ATTN_API void *smol_qkn_attn_stream(const void *owner);

#ifdef __cplusplus
}
#endif

#endif /* SMOL_QKN_ATTN_H */
