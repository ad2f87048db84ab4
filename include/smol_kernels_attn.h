/*
 * smol_kernels_attn.h - the reference's attention and RoPE entry points with
 * their exact signatures, implemented on the MI355X by libsmol_attn.so.
 *
 * Each prototype below is the one in the reference's
 * common/kernels/smol_kernels.h (line numbers given); linking libsmol_attn.so
 * in place of common/kernels/{attention,rope}.c (and rmsnorm.c's per-head
 * norm) makes the existing callers
 * (qkn_decoder.c:425-528 / :615-677, siglip.c:126, encoder.c:463, nomic.c:180,
 * smolvlm/decoder.c:340, :454) run on the GPU unchanged.
 *
 * Semantics follow the reference: pointers are caller-owned HOST fp32 arrays,
 * `out` rows are fully overwritten, the call returns when `out` is valid.
 * These functions use a per-thread default context on device 0 and stage the
 * arrays through device memory; the device-resident API in smol_attn.h avoids
 * the copies. The reference returns void and has no error channel: on a
 * device error these functions print the error to stderr and abort(), rather
 * than return unwritten output. The attention functions take any head_dim
 * up to 256 (the kernels' sizes 64, 72, 80, 96, 128, 256 run directly; the
 * others run zero-padded to the next of them) and abort above 256. Inputs
 * beyond the kernels' fp16 staging range are rescaled by powers of two and
 * the call repeated (smol_attn.h, Numerics).
 */
#ifndef SMOL_KERNELS_ATTN_H
#define SMOL_KERNELS_ATTN_H

#ifdef __cplusplus
extern "C" {
#endif

#ifndef SMOL_KERNELS_API
#define SMOL_KERNELS_API __attribute__((visibility("default")))
#endif

/* smol_kernels.h:109-113, attention.c:32-77 */
SMOL_KERNELS_API void smol_bidirectional_attention(float *out, const float *Q, const float *K,
                                                   const float *V, int seq, int n_heads,
                                                   int head_dim, float scale,
                                                   const int *window_starts, int n_windows);

/* smol_kernels.h:115-118, attention.c:153-170 */
SMOL_KERNELS_API void smol_causal_attention(float *out, const float *Q, const float *K,
                                            const float *V, int seq_q, int seq_k, int n_heads,
                                            int n_kv_heads, int head_dim, float scale,
                                            int q_offset);

/* smol_kernels.h:120-124, attention.c:254-273 */
SMOL_KERNELS_API void smol_sliding_window_attention(float *out, const float *Q, const float *K,
                                                    const float *V, int seq_q, int seq_k,
                                                    int n_heads, int n_kv_heads, int head_dim,
                                                    float scale, int q_offset, int window_size);

/* smol_kernels.h:126-131, attention.c:350-368 */
SMOL_KERNELS_API void smol_causal_attention_softcap(float *out, const float *Q, const float *K,
                                                    const float *V, int seq_q, int seq_k,
                                                    int n_heads, int n_kv_heads, int head_dim,
                                                    float scale, int q_offset, float cap);

/* smol_kernels.h:133-138, attention.c:443-462 */
SMOL_KERNELS_API void smol_sliding_window_attention_softcap(float *out, const float *Q,
                                                            const float *K, const float *V,
                                                            int seq_q, int seq_k, int n_heads,
                                                            int n_kv_heads, int head_dim,
                                                            float scale, int q_offset,
                                                            int window_size, float cap);

/* smol_kernels.h:147-149, rope.c:27-45 (table rows; host computation, as in
 * the reference: the tables are built once per position) */
SMOL_KERNELS_API void smol_compute_rope_neox(float *cos_out, float *sin_out,
                                             const int *positions, int seq, int head_dim,
                                             float theta);

/* smol_kernels.h:151-153, rope.c:99-164 */
SMOL_KERNELS_API void smol_apply_rope_neox(float *x, const float *cos_vals,
                                           const float *sin_vals, int seq, int n_heads,
                                           int head_dim);

/* smol_kernels.h:156-158, rope.c:51-66 */
SMOL_KERNELS_API void smol_compute_rope_interleaved(float *cos_out, float *sin_out,
                                                    const int *positions, int seq,
                                                    int head_dim, float theta);

/* smol_kernels.h:159-161, rope.c:68-93 */
SMOL_KERNELS_API void smol_apply_rope_interleaved(float *x, const float *cos_vals,
                                                  const float *sin_vals, int seq, int n_heads,
                                                  int head_dim);

/* smol_kernels.h:86-88, rmsnorm.c:78-140: each head_dim segment of x
 * [seq_len][n_heads*head_dim] becomes x * weight / sqrt(mean(x^2) + eps), in
 * place (the per-head Q/K norm of qkn_decoder.c:487-491) */
SMOL_KERNELS_API void smol_rms_norm_per_head(float *x, const float *weight, int seq_len,
                                             int n_heads, int head_dim, float eps);

#ifdef __cplusplus
}
#endif

#endif /* SMOL_KERNELS_ATTN_H */
