/*
 * smol_attn.h - C ABI of the MI355X (gfx950) attention path for smol-genius.
 *
 * Plain C types only (pointers, ints, floats); no HIP or torch types cross
 * this boundary. Library: libsmol_attn.so (link with -lsmol_attn).
 *
 * Two layers:
 *  1. Device-resident API (this section): a context (device + stream +
 *     workspace), a RoPE table, a bf16 KV cache, and decode / prefill /
 *     bidirectional attention on device pointers, enqueued on the context's
 *     stream. Every call returns an int status (SMOL_ATTN_OK or a negative
 *     code); smol_attn_last_error() describes the last failure of the calling
 *     thread. These replace the attention block of the reference decoders:
 *     RoPE on Q/K + cache append + attention
 *     (common/decoder/qkn_decoder.c:493-528 in qkn_decoder_prefill and
 *      :647-677 in qkn_decoder_forward).
 *  2. Drop-ins with the reference's exact signatures on host fp32 arrays,
 *     declared in smol_kernels_attn.h (common/kernels/smol_kernels.h:109-161).
 *
 * Tensor layouts are the reference's (common/kernels/attention.c:84-104):
 *   Q, out      [tokens][n_heads * head_dim]        row-major
 *   K, V (new)  [tokens][n_kv_heads * head_dim]     row-major
 * head h uses KV head h / (n_heads / n_kv_heads). Outputs are fp32.
 * Supported head_dim: 64, 72, 80, 96, 128, 256.
 *
 * Numerics: the softmax runs in fp32. Prefill and bidirectional calls form
 * QK^T from fp16 hi + lo parts of Q (times scale * log2 e) and of K
 * (Khi.Qhi + Khi.Qlo + Klo.Qhi on the matrix cores, about 21 significant
 * bits; bf16 cache rows and bf16 inputs without RoPE are exact in fp16 and
 * have no lo part), and P.V from fp16 probabilities and fp16 V (bf16 inputs
 * convert exactly). SMOL_OPT_QK_FP16 selects single fp16 Q and K operands
 * instead. A staged value that is not finite or whose magnitude reaches
 * 65520 raises the context's range flag, and the next
 * smol_attn_ctx_synchronize returns SMOL_ATTN_ERR_RANGE (the affected
 * outputs are not valid). Single-token decode has no such limit (its cache
 * operands are bf16, Q is split into bf16 hi + lo, and the new key is scored
 * in fp32). The reference-signature drop-ins rescale their inputs by powers
 * of two and repeat the call when the flag is raised.
 * The KV cache stores post-RoPE K and V in bf16 (round to nearest even).
 * Keys written by a call are used by that same call at fp16 precision.
 *
 * Threading: one context per host thread, as the reference's global thread
 * pool is not re-entrant (common/kernels/threading.c:26-47). Calls on one
 * context are ordered on its stream. Contexts share no host state (each
 * builds its own kernel arguments), so threads with one context each may
 * call concurrently.
 */
#ifndef SMOL_ATTN_H
#define SMOL_ATTN_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SMOL_ATTN_API __attribute__((visibility("default")))

/* status codes */
#define SMOL_ATTN_OK 0
#define SMOL_ATTN_ERR_ARG (-1)
#define SMOL_ATTN_ERR_NOMEM (-2)
#define SMOL_ATTN_ERR_DEVICE (-3)
#define SMOL_ATTN_ERR_UNSUPPORTED (-4)
#define SMOL_ATTN_ERR_NO_GPU (-5)
#define SMOL_ATTN_ERR_RANGE (-6) /* a value left the fp16 staging's range (see Numerics) */
#define SMOL_ATTN_ERR_TIMEOUT (-7) /* a decode split-K merge gave up waiting for its splits; the
                                    * rows it merges are NaN (reported by synchronize) */

/* element type of the Q / K / V inputs */
#define SMOL_ATTN_F32 0
#define SMOL_ATTN_BF16 1

/* RoPE pairing; qkn_rope_type_t in common/decoder/qkn_decoder.h:33-36 */
#define SMOL_ROPE_NONE (-1)
#define SMOL_ROPE_NEOX 0        /* (x[d], x[half + d]): Qwen3 */
#define SMOL_ROPE_INTERLEAVED 1 /* (x[2d], x[2d + 1]): Gemma / PaliGemma */

typedef struct smol_attn_ctx smol_attn_ctx;
typedef struct smol_rope_table smol_rope_table;
typedef struct smol_kv_cache smol_kv_cache;

/* ---- library / context -------------------------------------------------- */

SMOL_ATTN_API const char *smol_attn_version(void);
SMOL_ATTN_API const char *smol_attn_last_error(void);
/* number of visible GPUs, or a negative status when the HIP runtime has none */
SMOL_ATTN_API int smol_attn_device_count(void);

/* stream: a hipStream_t passed as void*; NULL selects the device's null
 * stream. The context never creates or destroys the stream. */
SMOL_ATTN_API int smol_attn_ctx_create(int device, void *stream, smol_attn_ctx **out);
SMOL_ATTN_API int smol_attn_ctx_destroy(smol_attn_ctx *ctx);
/* waits for the context's stream; returns SMOL_ATTN_ERR_TIMEOUT when a
 * decode merge since the last synchronize gave up waiting for its splits,
 * else SMOL_ATTN_ERR_RANGE when a call raised the range flag (both flags are
 * cleared) */
SMOL_ATTN_API int smol_attn_ctx_synchronize(smol_attn_ctx *ctx);
SMOL_ATTN_API void *smol_attn_ctx_stream(smol_attn_ctx *ctx);

/* Kernel timing (no counterpart in the reference, which only has wall-clock
 * perf fields, exports/qwen_asr/qwen_asr.h:147-152): when enabled, every
 * kernel the context launches is bracketed by HIP events on its stream.
 * timing_read synchronizes the stream and returns, per kind
 * (0 = RoPE/cache pre-pass, 1 = attention, 2 = other), the summed kernel
 * milliseconds ms[3] and launch counts count[3] since the last read. */
SMOL_ATTN_API int smol_attn_ctx_set_timing(smol_attn_ctx *ctx, int enable);
SMOL_ATTN_API int smol_attn_ctx_timing_read(smol_attn_ctx *ctx, double *ms, int *count);

/* Options of a context (no counterpart in the reference): switches that pick
 * between equivalent kernels or work splits, for tests and tuning. All are 0
 * by default, which selects by call shape. Results stay within the path's
 * tolerance whatever they are set to, except under SMOL_OPT_FAULT_MERGE,
 * which exists to test the error path. */
#define SMOL_OPT_PREFILL_KERNEL 0 /* 1: k_attn_fb wherever its keys allow, 2: k_attn_fa */
#define SMOL_OPT_FB_LISTS 1       /* -1: one k_attn_fb workgroup per tile (no tile lists) */
#define SMOL_OPT_FB_NT 2          /* 2: two row tiles per k_attn_fb wave */
#define SMOL_OPT_DEC_SLABS 3      /* k_dec: 32-key slabs per workgroup (0: by call size) */
#define SMOL_OPT_DEC_WAVES 4      /* k_dec: 4 or 8 waves per workgroup (0: by shape) */
#define SMOL_OPT_DEC_SPLIT 5      /* k_dec: -1 keeps every (sequence, kv head) in one workgroup */
#define SMOL_OPT_XCD_CHECK 6      /* read only: 1 when workgroup b was seen on XCD b % n_xcc at
                                   * creation (k_dec's split merge needs it), 0 when not (then
                                   * k_dec does not split) */
#define SMOL_OPT_BIDIR_WIN 7      /* bidirectional windows: 0 (or 1) k_attn_win (LDS-resident,
                                   * reads the inputs directly) whenever the windows fit in LDS,
                                   * else the pre-pass and k_attn_fb / k_attn_fa; -1: never */
#define SMOL_OPT_WIN_KSPLIT 8     /* k_attn_win: 1: 128-row tiles over every key; 2: 64-row tiles,
                                   * two key groups (0: 2 when 128-row tiles would leave compute
                                   * units idle) */
#define SMOL_OPT_DEC_SPIN 9       /* k_dec: flag polls before a split-K merger gives up (0: 4194304) */
#define SMOL_OPT_FAULT_MERGE 10   /* fault injection for tests: 1 makes every k_dec merger wait for a
                                   * flag value no split writes, so it gives up after SMOL_OPT_DEC_SPIN
                                   * polls, writes NaN rows and synchronize returns
                                   * SMOL_ATTN_ERR_TIMEOUT; every kernel still ends normally */
#define SMOL_OPT_QK_FP16 11       /* 1: QK^T on single fp16 operands (Q and K each rounded to fp16:
                                   * faster, within the bar for logits up to about sigma 1.4 on
                                   * unit-variance rows); 0: fp16 hi + lo operands, see Numerics */
#define SMOL_OPT_FB_GROUPS 12     /* k_attn_fb: 1: one key group of eight waves over 128-row items (long
                                   * items' keys split over workgroups and merged); 0 or 2: two key
                                   * groups over 64-row items */
#define SMOL_OPT_GEMM_TILE 13     /* k_gemm (projections of more than 4 rows): 0: tile chosen per shape;
                                   * 1, 2, 3: 192 x 192, 128 x 128, 64 x 64 (rows x outputs) */
#define SMOL_OPT_FB_QPREP 14      /* k_attn_fb at head_dim 64 / 128 with precise QK^T and no per-head
                                   * Q norm: 0: each item rotates and scales its own Q rows from the
                                   * inputs; 1: the pre-pass stages them (as for k_attn_fa) */
#define SMOL_OPT_COUNT 15
SMOL_ATTN_API int smol_attn_ctx_set_option(smol_attn_ctx *ctx, int option, int value);
SMOL_ATTN_API int smol_attn_ctx_get_option(smol_attn_ctx *ctx, int option, int *value);

/* ---- RoPE table ----------------------------------------------------------
 * Device fp32 cos/sin rows [capacity][head_dim], built on the host exactly as
 * fill_rope_cache does (common/decoder/qkn_decoder.c:261-311):
 * inv_freq[d] = 1 / powf(theta, 2d / head_dim), angle = (float)pos * inv_freq[d],
 * duplicated to (d, half + d) or (2d, 2d + 1). Capacity starts at >= 1024 and
 * doubles on demand, as there. */
SMOL_ATTN_API int smol_rope_table_create(smol_attn_ctx *ctx, int head_dim, float theta,
                                         int rope_type, int capacity, smol_rope_table **out);
SMOL_ATTN_API int smol_rope_table_ensure(smol_rope_table *rt, int required_pos);
SMOL_ATTN_API int smol_rope_table_capacity(const smol_rope_table *rt);
SMOL_ATTN_API int smol_rope_table_destroy(smol_rope_table *rt);
/* host rows [pos0, pos0 + n_pos) of a table, same formula (no device needed) */
SMOL_ATTN_API void smol_rope_fill_host(float *cos_out, float *sin_out, int pos0, int n_pos,
                                       int head_dim, float theta, int rope_type);

/* ---- KV cache -------------------------------------------------------------
 * Device bf16 cache for n_layers x n_slots sequences (a slot is one sequence,
 * e.g. one of a batch of decode streams). The reference keeps one fp32 cache
 * per decoder context (qkn_ctx_t.kv_cache_k/v, qkn_decoder.h:99-103;
 * kv_cache_init/grow/k_at/v_at, qkn_decoder.c:172-220). As there, the valid
 * length is the caller's: attention calls take explicit positions, so a
 * rewind (qwen_asr.c:1609 assigns kv_cache_len) is just passing a smaller
 * position next time. Capacity grows by doubling with contents kept.
 * Memory is zero-filled at creation and growth. */
SMOL_ATTN_API int smol_kv_cache_create(smol_attn_ctx *ctx, int n_layers, int n_slots,
                                       int n_kv_heads, int head_dim, int max_seq,
                                       smol_kv_cache **out);
SMOL_ATTN_API int smol_kv_cache_destroy(smol_kv_cache *kv);
SMOL_ATTN_API int smol_kv_cache_capacity(const smol_kv_cache *kv);
/* grow (doubling) so that at least required_pos positions fit */
SMOL_ATTN_API int smol_kv_cache_reserve(smol_kv_cache *kv, int required_pos);
/* write already-rotated rows [pos0, pos0 + n) of one layer/slot from
 * [n][n_kv_heads * head_dim] arrays (dtype SMOL_ATTN_F32 or _BF16; host
 * pointers when on_device == 0, else device pointers) */
SMOL_ATTN_API int smol_kv_cache_write(smol_kv_cache *kv, int layer, int slot, int pos0, int n,
                                      const void *k, const void *v, int dtype, int on_device);
/* read rows back as bf16 bits [n][n_kv_heads * head_dim] (host pointers) */
SMOL_ATTN_API int smol_kv_cache_read(smol_kv_cache *kv, int layer, int slot, int pos0, int n,
                                     uint16_t *k_out, uint16_t *v_out);

/* ---- attention on device pointers -----------------------------------------
 * window > 0: sliding window (keys with pos - window < key <= pos,
 * attention.c:176-273); cap > 0: score = cap * tanh(score / cap)
 * (attention.c:281-462). scale is the caller's (1/sqrtf(head_dim) in the
 * reference decoders, qkn_decoder.c:430, 620).
 */

/* Prefill / chunked prefill of one sequence (replaces qkn_decoder.c:493-528):
 * rotates Q [seq_q][n_heads*hd] and the new K [seq_q][n_kv*hd] at positions
 * pos0..pos0+seq_q-1 with `rope` (NULL: no RoPE), appends K/V to the cache at
 * (layer, slot), and writes out [seq_q][n_heads*hd] = causal attention of the
 * new rows over cache positions [0, pos0 + seq_q). pos0 > 0 is chunked
 * prefill on top of an existing prefix. */
SMOL_ATTN_API int smol_attn_prefill(smol_attn_ctx *ctx, smol_kv_cache *kv, int layer, int slot,
                                    const smol_rope_table *rope, int pos0, int seq_q,
                                    const void *q, const void *k_new, const void *v_new,
                                    int dtype, int n_heads, float scale, int window, float cap,
                                    float *out);

/* Batched single-token decode (replaces qkn_decoder.c:647-677): for each of
 * n_seq sequences i, rotates q[i] and k_new[i] at position pos[i], appends
 * K/V at (layer, slots[i], pos[i]) and writes out[i] = attention of q[i] over
 * positions [0, pos[i]] of that slot. slots/pos are host arrays. q, out:
 * [n_seq][n_heads*hd]; k_new, v_new: [n_seq][n_kv*hd]. */
SMOL_ATTN_API int smol_attn_decode(smol_attn_ctx *ctx, smol_kv_cache *kv, int layer,
                                   const smol_rope_table *rope, int n_seq, const int *slots,
                                   const int *pos, const void *q, const void *k_new,
                                   const void *v_new, int dtype, int n_heads, float scale,
                                   int window, float cap, float *out);

/* The two calls above with the per-head Q/K RMSNorm of the reference
 * decoders fused in front of RoPE (qkn_decoder.c:487-491 and :640-644,
 * rmsnorm.c:78-140): each head_dim segment of q and of k_new becomes
 * x * w[d] / sqrt(mean(x^2) + eps) before it is rotated. q_norm / k_norm are
 * device fp32 [head_dim] weights (NULL skips that norm, as a NULL
 * q_norm_weight / k_norm_weight does in the reference); loaders that fold
 * Gemma's 1 + w into the weight (gemma.c:166-169) pass the folded weight. */
SMOL_ATTN_API int smol_attn_prefill_qknorm(smol_attn_ctx *ctx, smol_kv_cache *kv, int layer, int slot,
                                           const smol_rope_table *rope, int pos0, int seq_q,
                                           const void *q, const void *k_new, const void *v_new,
                                           int dtype, int n_heads, float scale, int window, float cap,
                                           const float *q_norm, const float *k_norm, float eps,
                                           float *out);
SMOL_ATTN_API int smol_attn_decode_qknorm(smol_attn_ctx *ctx, smol_kv_cache *kv, int layer,
                                          const smol_rope_table *rope, int n_seq, const int *slots,
                                          const int *pos, const void *q, const void *k_new,
                                          const void *v_new, int dtype, int n_heads, float scale,
                                          int window, float cap, const float *q_norm,
                                          const float *k_norm, float eps, float *out);

/* smol_attn_decode_qknorm for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). No counterpart in the reference. Nothing is allocated: the
 * decode kernel's split partials and flags live in a fixed per-GPU scratch
 * array of SMOL_ATTN_NOALLOC_SCRATCH_BYTES (held by each GPU the library
 * runs on until the process ends), the work list rides in the kernel
 * arguments, the cache and RoPE table do not grow, and kernel timing is not
 * recorded. Limits (SMOL_ATTN_ERR_UNSUPPORTED / _ARG otherwise): n_seq <= 32;
 * every pos[i] below the cache's capacity and the table's (reserve / ensure
 * them beforehand with smol_kv_cache_reserve / smol_rope_table_ensure); a
 * call whose split partials would not fit the scratch runs unsplit, one
 * workgroup per (sequence, KV head). All calls on one GPU share its scratch:
 * calls that overlap in time on one GPU (other streams, other contexts,
 * other threads) race and must be serialised by the caller. Results equal
 * smol_attn_decode_qknorm's whenever both split the same way. */
#define SMOL_ATTN_NOALLOC_SCRATCH_BYTES (16u << 20)
SMOL_ATTN_API int smol_attn_decode_noalloc(smol_attn_ctx *ctx, smol_kv_cache *kv, int layer,
                                           const smol_rope_table *rope, int n_seq, const int *slots,
                                           const int *pos, const void *q, const void *k_new,
                                           const void *v_new, int dtype, int n_heads, float scale,
                                           int window, float cap, const float *q_norm,
                                           const float *k_norm, float eps, float *out);

/* Causal attention on flat device arrays, no cache and no RoPE: the device
 * form of smol_causal_attention (attention.c:153-170). K, V: [seq_k][n_kv*hd]. */
SMOL_ATTN_API int smol_attn_causal(smol_attn_ctx *ctx, const void *q, const void *k,
                                   const void *v, int dtype, int seq_q, int seq_k, int n_heads,
                                   int n_kv_heads, int head_dim, float scale, int q_offset,
                                   int window, float cap, float *out);

/* The attention of the bf16 decoder (common/decoder/qkn_bf16_decoder.c:
 * 120-229, bf16_causal_attention_softcap / bf16_swa_attention_softcap): bf16
 * Q/K/V in, bf16 out rounded by truncation (f32_to_bf16, :30-35); window
 * and cap as in smol_attn_causal. The result is computed in fp32 first
 * (a workspace of seq_q * n_heads * head_dim floats in the context). */
SMOL_ATTN_API int smol_attn_causal_bf16(smol_attn_ctx *ctx, const uint16_t *q, const uint16_t *k,
                                        const uint16_t *v, int seq_q, int seq_k, int n_heads,
                                        int n_kv_heads, int head_dim, float scale, int q_offset,
                                        int window, float cap, uint16_t *out);

/* Windowed bidirectional attention on device arrays: the device form of
 * smol_bidirectional_attention (attention.c:32-77). Q, K, V, out:
 * [seq][n_heads*hd]; window_starts: host array of n_windows + 1 offsets
 * (a batch of independent sequences is one window each). */
SMOL_ATTN_API int smol_attn_bidirectional(smol_attn_ctx *ctx, const void *q, const void *k,
                                          const void *v, int dtype, int seq, int n_heads,
                                          int head_dim, float scale, const int *window_starts,
                                          int n_windows, float *out);

/* In-place RoPE on a device fp32 array [seq][n_heads*hd] whose row s uses
 * table position positions[s] (host array): the device form of
 * smol_apply_rope_{neox,interleaved} (rope.c:68-164). */
SMOL_ATTN_API int smol_attn_apply_rope(smol_attn_ctx *ctx, const smol_rope_table *rope, float *x,
                                       const int *positions, int seq, int n_heads);

/* In place on a device fp32 array x [seq][n_heads*head_dim]: per-head
 * RMSNorm with the device weight [head_dim] (skipped when weight is NULL;
 * the device form of smol_rms_norm_per_head, rmsnorm.c:78-140), then RoPE
 * with row s at table position positions[s] (skipped when rope is NULL;
 * positions is then unused). */
SMOL_ATTN_API int smol_attn_norm_rope(smol_attn_ctx *ctx, const smol_rope_table *rope, float *x,
                                      const float *weight, float eps, const int *positions, int seq,
                                      int n_heads, int head_dim);

/* The bf16 decoder's rounding of Q and the new K rows, in place on a device
 * bf16 array x [seq][n_heads*head_dim] (16-byte aligned, head_dim a multiple
 * of 8): per-head RMSNorm with the device fp32 weight (skipped when NULL),
 * then the interleaved rotation of row s at table position pos0 + s (skipped
 * when rope is NULL; the table must be SMOL_ROPE_INTERLEAVED), each result
 * rounded to bf16 by truncation (bf16_rms_norm_per_head and
 * bf16_apply_rope_interleaved, common/decoder/qkn_bf16_decoder.c:73-91 and
 * :264-283). The order of operations is fixed, so the bits do not depend on
 * the launch: the sum of squares is one fused multiply-add per element in
 * element order, 1/sqrt(ss/head_dim + eps) is correctly rounded, the norm
 * is (x*r)*w, and a pair rotates as fma(x0,c,-(x1*s)), fma(x1,c,x0*s). */
SMOL_ATTN_API int smol_attn_norm_rope_bf16(smol_attn_ctx *ctx, const smol_rope_table *rope, uint16_t *x,
                                           const float *weight, float eps, int pos0, int seq,
                                           int n_heads, int head_dim);

#ifdef __cplusplus
}
#endif

#endif /* SMOL_ATTN_H */
