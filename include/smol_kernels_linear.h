/*
 * smol_kernels_linear.h - the reference's bf16-weight projection entry
 * points, same names and signatures (common/kernels/smol_kernels.h:45-63),
 * computed on the GPU. Host arrays in and out, as in the reference:
 *
 *   y[s][o] = sum_i x[s][i] * W[o][i] (+ b[o])      x [seq_len][in_dim],
 *                                                    W [out_dim][in_dim] bf16,
 *                                                    y [seq_len][out_dim]
 *   smol_matmul_t_bf16: C[m][n] = sum_k A[m][k] * B[n][k]
 *
 * Each call copies its inputs to the calling thread's device context
 * (device 0), runs smol_linear_dev / smol_linear_qkv_dev and copies the
 * result back before returning. The weights are uploaded on every call,
 * unless SMOL_BF16_CACHE_MB=<n> is set: then, as the reference's
 * bf16_get_cached_f32 does (common/kernels/matmul.c:136-189), a weight is
 * kept by its (pointer, element count) within n MB, here as a device copy,
 * and later calls with that pointer use the copy without reading the host
 * array again (the caller must not change cached weights in place).
 *
 * The reference functions return void and have no error channel; a GPU
 * failure prints smol_attn_last_error() to stderr and aborts. Calls with
 * seq_len, in_dim or out_dim <= 0 do nothing except that in_dim <= 0 sets
 * y to the bias (or zero), as the reference's loops do.
 */
#ifndef SMOL_KERNELS_LINEAR_H
#define SMOL_KERNELS_LINEAR_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#ifndef SMOL_KERNELS_API
#define SMOL_KERNELS_API __attribute__((visibility("default")))
#endif

/* common/kernels/smol_kernels.h:46-47, matmul.c:348-358 */
SMOL_KERNELS_API void smol_linear_bf16(float *y, const float *x, const uint16_t *W_bf16, const float *b,
                                       int seq_len, int in_dim, int out_dim);

/* common/kernels/smol_kernels.h:50-51, matmul.c:336-346 */
SMOL_KERNELS_API void smol_linear_nobias_bf16(float *y, const float *x, const uint16_t *W_bf16, int seq_len,
                                              int in_dim, int out_dim);

/* common/kernels/smol_kernels.h:55-59, matmul.c:308-334: one token's
 * q [q_dim], k [kv_dim], v [kv_dim] from x [in_dim] */
SMOL_KERNELS_API void smol_linear_nobias_bf16_qkv(float *q, float *k, float *v, const float *x,
                                                  const uint16_t *Wq_bf16, const uint16_t *Wk_bf16,
                                                  const uint16_t *Wv_bf16, int in_dim, int q_dim, int kv_dim);

/* common/kernels/smol_kernels.h:62-63, matmul.c:419-429: C [M][N] = A [M][K] B^T, B [N][K] bf16 */
SMOL_KERNELS_API void smol_matmul_t_bf16(float *C, const float *A, const uint16_t *B_bf16, int M, int K,
                                         int N);

#ifdef __cplusplus
}
#endif

#endif
