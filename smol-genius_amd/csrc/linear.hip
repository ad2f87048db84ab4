/*
 * linear.hip - the decoders' bf16-weight projections on gfx950
 * (include/smol_linear.h, include/smol_kernels_linear.h).
 *
 *   y[s][o] = sum_i x[s][i] W[o][i] (+ b[o])
 *     common/kernels/matmul.c:70-97   smol_linear (the loops the seq > 1 path runs)
 *     common/kernels/matmul.c:210-247 bf16_matvec_fused / _threaded (seq == 1)
 *     common/kernels/matmul.c:250-334 the fused Q/K/V matvec
 *     common/decoder/qkn_bf16_decoder.c:99-117 bf16_linear_nobias (bf16 in, truncated bf16 out)
 *
 * Two device paths:
 *   k_gemv   seq <= SMOL_LINEAR_GEMV_MAX_SEQ (decode). HBM-bound: every
 *            weight byte is read once. A row group is GEMV_R consecutive
 *            output rows (of the joint row space of up to three weight
 *            segments, so Q/K/V is one launch) and `kp` waves that split
 *            in_dim; a workgroup packs `groups` row groups (up to
 *            GEMV_WG_WAVES waves). Lane l of wave w (of kp) reads the 16-byte chunks
 *            w*64 + l + j*64*kp of each of its rows, and the x chunk it
 *            multiplies them with (x stays L1/L2 resident). Every load of a
 *            step is issued before the first FMA. Sums: per-lane fp32, then
 *            a wave all-reduce (cross-row swaps + DPP row rotations), then
 *            the kp waves' totals in a fixed order through LDS.
 *   k_gemm   longer inputs (gemm.hip): bf16 MFMA tiles with the input
 *            RMSNorm, the bias, the gated activation and the residual add
 *            fused; an fp32 x is split into bf16 hi + lo as it is staged
 *            (y = W x_hi + W x_lo, x carried to ~2^-17 relative, the
 *            weights exact).
 */
#include <hip/hip_runtime.h>

#include <limits.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <map>
#include <mutex>
#include <numeric>
#include <tuple>
#include <unordered_map>
#include <vector>

#include "attn_device.h"
#include "smol_kernels_linear.h"
#include "smol_linear.h"

extern "C" int smol_internal_fail(int code, const char *msg);
extern "C" int smol_internal_ctx_device(smol_attn_ctx *ctx);
extern "C" void smol_internal_timing_events(smol_attn_ctx *ctx, int kind, hipEvent_t *a, hipEvent_t *b);
extern "C" smol_attn_ctx *smol_internal_legacy_ctx(const char *fn);
extern "C" int smol_launch_to_bf16_trunc(const float *x, uint16_t *y, long long n, hipStream_t st);
extern "C" int smol_internal_ctx_cus(smol_attn_ctx *ctx);
extern "C" int smol_internal_ctx_option(smol_attn_ctx *ctx, int option);
extern "C" int smol_gemm_tile(int cfg, int *bm, int *bn);
extern "C" int smol_launch_gemm(GemmParams *p, int cfg, bool xbf, bool ybf, hipStream_t st, hipEvent_t e0,
                                hipEvent_t e1);

#define GEMV_R 4      /* output rows per row group (one wave, or kp waves) */
#define GEMV_U 2      /* chunks of 8 elements per lane per step */
#define GEMV_MAX_KP 8 /* waves per row group along in_dim */
#ifndef GEMV_WG_WAVES
#define GEMV_WG_WAVES 4 /* target waves per workgroup: row groups are packed up to it */
#endif
#define GEMV_SEGS 3
#define LIN_TIMING_KIND 2 /* the context's "other" timing kind */

/* one weight of a GEMV launch (host side) */
struct GemvSeg {
    const uint16_t *w;  /* [out][in] bf16 */
    const float *bias;  /* [out] or null */
    void *y;            /* [seq][out] */
    int out;
};

/* the fields the loads depend on first, the epilogue's after them */
struct GemvParams {
    const uint16_t *w[GEMV_SEGS];
    const void *x;           /* [seq][in] */
    int row0[GEMV_SEGS];     /* first row of each segment in the joint row space (INT_MAX: unused) */
    int in;
    int rows;                /* rows of all segments */
    int kp;                  /* waves per row group (split in_dim) */
    int groups;              /* row groups per workgroup (kp * groups <= GEMV_MAX_KP) */
    const float *bias[GEMV_SEGS];
    void *y[GEMV_SEGS];
    int out[GEMV_SEGS];
    /* fused operations (fp32 x and y, one segment) */
    const float *norm_w; /* [in] or null: each x row is RMS-normalised with this weight first */
    float eps;
    int act;             /* SMOL_LINEAR_ACT_*: rows (2j, 2j + 1) are (gate, up), y[s][j] = act(gate) up */
    const float *res;    /* [seq][y columns] or null: added to the result (may equal y) */
    /* the bf16 decoder's operations (bf16 y, one segment, not FUSE; every
     * step truncated as qkn_bf16_decoder.c does): act GEGLU: y[s][j] =
     * geglu(tr(gate), tr(up)) as k_bf16_geglu; res16: y = tr(bf(res16) +
     * bf(tr(sum))) as k_bf16_rows' add (may equal y); x_trunc: an fp32 x is
     * truncated to bf16 as it is loaded */
    const uint16_t *res16;
    int x_trunc;
    /* N16 only: add16 [seq][in] bf16 or null: x is first replaced by
     * tr(bf(x) + bf(add16)) (k_bf16_rows' residual add), and workgroup 0
     * writes that sum to xout16 (or not, when null) */
    const uint16_t *add16;
    uint16_t *xout16;
};

/* ---------------------------------------------------------------- kernels */

/* bf16 bits widened to fp32, and fp32 truncated to bf16 bits */
__device__ __forceinline__ float bfw(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }
__device__ __forceinline__ uint16_t bftr(float v) { return (uint16_t)(__float_as_uint(v) >> 16); }

/* sum over the 64 lanes, the total in every lane */
__device__ __forceinline__ float wave_sum(float v) {
    const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(b[0]) + __uint_as_float(b[1]);
    /* DPP row_ror:8, 4, 2, 1 (rotations within each row of 16 lanes) */
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x128, 0xF, 0xF, false));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x124, 0xF, 0xF, false));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x122, 0xF, 0xF, false));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x121, 0xF, 0xF, false));
    return v;
}

/* segment of joint row `row` (uniform when row is) */
__device__ __forceinline__ int seg_of(const GemvParams &p, int row) {
    return (row >= p.row0[1]) + (row >= p.row0[2]);
}

/* VEC: in % 8 == 0 and 16-byte aligned x / W (every chunk one 16-byte
 * load); otherwise elementwise loads. Loads past a row or past x read
 * zero (buffer range checks), so no branch guards them. */
template <int SEQ, bool XBF, bool YBF, bool VEC, bool FUSE>
__global__ __launch_bounds__(64 * GEMV_MAX_KP) void k_gemv(const GemvParams p) {
    __shared__ float red[GEMV_MAX_KP][GEMV_R * SEQ];
    __shared__ float red_ss[GEMV_MAX_KP][GEMV_R * SEQ];
    /* FUSE with an fp32 x: the fp32 RMSNorm (scale applied to the sums);
     * with a bf16 x (N16): the bf16 decoder's input norm, x replaced by
     * tr((bf(x) * r) * w) as it is loaded (k_bf16_rows' values) */
    constexpr bool N16 = FUSE && XBF, F32N = FUSE && !XBF;
    const GemvParams &h = p;
    const int lane = threadIdx.x & 63;
    const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int kp = h.kp;
    const int wave = wid % kp;  /* position along in_dim */
    const int in = h.in;
    const int row_base = (blockIdx.x * h.groups + wid / kp) * GEMV_R;

    rsrc_t wr[GEMV_R];
#pragma unroll
    for (int r = 0; r < GEMV_R; r++) {
        const int row = row_base + r;
        const int sg = (row >= h.row0[1]) + (row >= h.row0[2]);
        const uint16_t *w = sg == 0 ? h.w[0] : sg == 1 ? h.w[1] : h.w[2];
        const int r0 = sg == 0 ? h.row0[0] : sg == 1 ? h.row0[1] : h.row0[2];
        const bool live = row < h.rows;
        wr[r] = make_rsrc(live ? w + (long long)(row - r0) * in : h.w[0], live ? (long long)in * 2 : 0);
    }
    const rsrc_t xr = make_rsrc(h.x, (long long)SEQ * in * (XBF ? 2 : 4));
    const rsrc_t ar = make_rsrc(N16 && p.add16 ? (const void *)p.add16 : h.x, N16 && p.add16 ? (long long)SEQ * in * 2 : 0);
    /* the norm weight (reads zero when there is none, then unused) */
    const bool norm = FUSE && p.norm_w;
    const rsrc_t gr = make_rsrc(norm ? (const void *)p.norm_w : (const void *)h.w[0], norm ? (long long)in * 4 : 0);
    float ssq[SEQ];
#pragma unroll
    for (int s = 0; s < SEQ; s++) ssq[s] = 0.0f;
    /* N16: r of each input row before the products, in k_bf16_rows' order
     * (the host launches 256 threads: per-thread strided fused
     * multiply-adds, a butterfly over each wave, the four waves in order),
     * so the normalised x has that kernel's bits */
    float r16[SEQ];
    if constexpr (N16) {
        __shared__ float red16[4][SEQ];
        const uint16_t *xb = static_cast<const uint16_t *>(h.x);
        const bool wr_x = p.xout16 && blockIdx.x == 0;
#pragma unroll
        for (int s = 0; s < SEQ; s++) {
            float ss = 0.0f;
            for (int i = threadIdx.x; i < in; i += 256) {
                const long long j = (long long)s * in + i;
                float v = bfw(xb[j]);
                if (p.add16) {
                    const uint16_t t = bftr(v + bfw(p.add16[j]));
                    if (wr_x) p.xout16[j] = t;
                    v = bfw(t);
                }
                ss = fmaf(v, v, ss);
            }
#pragma unroll
            for (int m = 32; m > 0; m >>= 1) ss += __shfl_xor(ss, m, 64);
            if (lane == 0) red16[wid][s] = ss;
        }
        __syncthreads();
#pragma unroll
        for (int s = 0; s < SEQ; s++)
            r16[s] = 1.0f / sqrtf((((red16[0][s] + red16[1][s]) + red16[2][s]) + red16[3][s]) / (float)in + p.eps);
    }

    float acc[GEMV_R][SEQ];
#pragma unroll
    for (int r = 0; r < GEMV_R; r++)
#pragma unroll
        for (int s = 0; s < SEQ; s++) acc[r][s] = 0.0f;

    const int C = (in + 7) >> 3; /* chunks per row */
    const uint32_t xmask = !FUSE && p.x_trunc ? 0xffff0000u : 0xffffffffu;
    const int stride = 64 * kp;
    for (int c0 = wave * 64; c0 < C; c0 += stride * GEMV_U) {
        float wf[GEMV_U][GEMV_R][8];
        float xf[GEMV_U][SEQ][8];
        float gf[GEMV_U][8];
        if constexpr (VEC) {
            uint4 wv[GEMV_U][GEMV_R];
            uint4 xv[GEMV_U][SEQ][XBF ? 1 : 2];
            uint4 av[GEMV_U][SEQ];
            uint4 gv[GEMV_U][2];
#pragma unroll
            for (int u = 0; u < GEMV_U; u++) {
                const int c = c0 + lane + u * stride;
                const bool ok = c < C;
                if constexpr (FUSE) {
                    gv[u][0] = bload(gr, ok ? (unsigned)c * 32u : OOB_OFF, 0);
                    gv[u][1] = bload(gr, ok ? (unsigned)c * 32u + 16u : OOB_OFF, 0);
                }
#pragma unroll
                for (int r = 0; r < GEMV_R; r++) wv[u][r] = bload(wr[r], ok ? (unsigned)c * 16u : OOB_OFF, 0);
#pragma unroll
                for (int s = 0; s < SEQ; s++) {
                    if constexpr (XBF) {
                        xv[u][s][0] = bload(xr, ok ? (unsigned)(s * in + c * 8) * 2u : OOB_OFF, 0);
                        if constexpr (N16) av[u][s] = bload(ar, ok ? (unsigned)(s * in + c * 8) * 2u : OOB_OFF, 0);
                    } else {
                        const unsigned o = (unsigned)(s * in + c * 8) * 4u;
                        xv[u][s][0] = bload(xr, ok ? o : OOB_OFF, 0);
                        xv[u][s][1] = bload(xr, ok ? o + 16u : OOB_OFF, 0);
                    }
                }
            }
            /* keeps every load of the step ahead of the first use: the
             * scheduler would otherwise sink loads below waits to save
             * registers, turning one memory round trip into several */
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int u = 0; u < GEMV_U; u++) {
                if constexpr (FUSE) {
                    const uint32_t t[8] = {gv[u][0].x, gv[u][0].y, gv[u][0].z, gv[u][0].w,
                                           gv[u][1].x, gv[u][1].y, gv[u][1].z, gv[u][1].w};
#pragma unroll
                    for (int e = 0; e < 8; e++) gf[u][e] = __uint_as_float(t[e]);
                }
#pragma unroll
                for (int r = 0; r < GEMV_R; r++) unpack_bf16x8(wv[u][r], wf[u][r]);
#pragma unroll
                for (int s = 0; s < SEQ; s++) {
                    if constexpr (XBF) {
                        unpack_bf16x8(xv[u][s][0], xf[u][s]);
                        if constexpr (N16) {
                            float af[8];
                            unpack_bf16x8(av[u][s], af);
#pragma unroll
                            for (int e = 0; e < 8; e++) xf[u][s][e] = bfw(bftr(xf[u][s][e] + af[e]));
                        }
                    } else {
                        const uint4 a = xv[u][s][0], b = xv[u][s][1];
                        const uint32_t t[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
                        for (int e = 0; e < 8; e++) xf[u][s][e] = __uint_as_float(t[e] & xmask);
                    }
                }
            }
        } else {
#pragma unroll
            for (int u = 0; u < GEMV_U; u++) {
                const int c = c0 + lane + u * stride;
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    const int i = c * 8 + e;
                    const bool ok = c < C && i < in;
                    if constexpr (FUSE)
                        gf[u][e] = __uint_as_float(
                            __builtin_amdgcn_raw_buffer_load_b32(gr, ok ? (unsigned)i * 4u : OOB_OFF, 0, 0));
#pragma unroll
                    for (int r = 0; r < GEMV_R; r++) {
                        const unsigned short h = __builtin_amdgcn_raw_buffer_load_b16(
                            wr[r], ok ? (unsigned)i * 2u : OOB_OFF, 0, 0);
                        wf[u][r][e] = __uint_as_float((uint32_t)h << 16);
                    }
#pragma unroll
                    for (int s = 0; s < SEQ; s++) {
                        if constexpr (XBF) {
                            const unsigned short h = __builtin_amdgcn_raw_buffer_load_b16(
                                xr, ok ? (unsigned)(s * in + i) * 2u : OOB_OFF, 0, 0);
                            xf[u][s][e] = __uint_as_float((uint32_t)h << 16);
                            if constexpr (N16) {
                                const unsigned short ha = __builtin_amdgcn_raw_buffer_load_b16(
                                    ar, ok ? (unsigned)(s * in + i) * 2u : OOB_OFF, 0, 0);
                                xf[u][s][e] = bfw(bftr(xf[u][s][e] + __uint_as_float((uint32_t)ha << 16)));
                            }
                        } else {
                            xf[u][s][e] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
                                xr, ok ? (unsigned)(s * in + i) * 4u : OOB_OFF, 0, 0) & xmask);
                        }
                    }
                }
            }
        }
        if constexpr (N16) {
#pragma unroll
            for (int u = 0; u < GEMV_U; u++)
#pragma unroll
                for (int s = 0; s < SEQ; s++)
#pragma unroll
                    for (int e = 0; e < 8; e++) xf[u][s][e] = bfw(bftr((xf[u][s][e] * r16[s]) * gf[u][e]));
        }
        if constexpr (F32N) {
            /* sum of squares of the raw x, then x * g (rmsnorm.c:17-75 scales after the product) */
#pragma unroll
            for (int u = 0; u < GEMV_U; u++)
#pragma unroll
                for (int s = 0; s < SEQ; s++)
#pragma unroll
                    for (int e = 0; e < 8; e++) {
                        ssq[s] = fmaf(xf[u][s][e], xf[u][s][e], ssq[s]);
                        xf[u][s][e] = norm ? xf[u][s][e] * gf[u][e] : xf[u][s][e];
                    }
        }
#pragma unroll
        for (int u = 0; u < GEMV_U; u++)
#pragma unroll
            for (int r = 0; r < GEMV_R; r++)
#pragma unroll
                for (int s = 0; s < SEQ; s++)
#pragma unroll
                    for (int e = 0; e < 8; e++) acc[r][s] = fmaf(wf[u][r][e], xf[u][s][e], acc[r][s]);
    }

    /* lane i = s * GEMV_R + r ends with the total of (row r, input s) */
    float mine = 0.0f, myss = 0.0f;
#pragma unroll
    for (int r = 0; r < GEMV_R; r++)
#pragma unroll
        for (int s = 0; s < SEQ; s++) {
            const float t = wave_sum(acc[r][s]);
            if (lane == s * GEMV_R + r) mine = t;
        }
    if constexpr (F32N) {
        if (norm) {
#pragma unroll
            for (int s = 0; s < SEQ; s++) {
                const float t = wave_sum(ssq[s]);
                if (lane / GEMV_R == s) myss = t;
            }
        }
    }
    if (kp > 1) {
        if (lane < GEMV_R * SEQ) {
            red[wid][lane] = mine;
            if constexpr (F32N) red_ss[wid][lane] = myss;
        }
        __syncthreads();
        if (wave != 0) return;
        if (lane < GEMV_R * SEQ) {
            mine = 0.0f;
            myss = 0.0f;
            for (int w = 0; w < kp; w++) {
                mine += red[wid + w][lane];
                if constexpr (F32N) myss += red_ss[wid + w][lane];
            }
        }
    }
    if constexpr (F32N) {
        const int r = lane % GEMV_R, s = lane / GEMV_R;
        const int o = row_base + r;
        const bool live = lane < GEMV_R * SEQ && o < p.rows;
        /* selects, not p.y[sg]: a lane-dependent index into the kernel
         * arguments would be lowered through scratch memory */
        const int sg = seg_of(p, o);
        const int r0 = sg == 0 ? p.row0[0] : sg == 1 ? p.row0[1] : p.row0[2];
        const int so = sg == 0 ? p.out[0] : sg == 1 ? p.out[1] : p.out[2];
        const float *bias = sg == 0 ? p.bias[0] : sg == 1 ? p.bias[1] : p.bias[2];
        float *y = static_cast<float *>(sg == 0 ? p.y[0] : sg == 1 ? p.y[1] : p.y[2]);
        float v = mine;
        if (norm) v *= 1.0f / sqrtf(myss / (float)in + p.eps);
        if (live && bias) v += bias[o - r0];
        if (p.act) {
            /* one segment. Lane i holds row r; the up row of gate row r (even)
             * is in lane i + 1 */
            const float up = __shfl_down(v, 1);
            float g = v;
            if (p.act == SMOL_LINEAR_ACT_SWIGLU) {
                g = g / (1.0f + expf(-g));
            } else {
                const float x3 = g * g * g;
                const float inner = 0.7978845608028654f * (g + 0.044715f * x3);
                g = 0.5f * g * (1.0f + tanhf(inner));
            }
            if (live && (r & 1) == 0) {
                const long long j = (long long)s * (so >> 1) + (o >> 1);
                const float val = g * up;
                y[j] = p.res ? p.res[j] + val : val;
            }
        } else if (live) {
            /* the residual belongs to segment 0 */
            const long long j = (long long)s * so + (o - r0);
            y[j] = (sg == 0 && p.res) ? p.res[j] + v : v;
        }
        return;
    }
    if constexpr (YBF) {
        if (p.act) {
            /* bf16 GeGLU (one segment): lane i holds row r, the up row of
             * gate row r (even) is in lane i + 1; both truncated first, then
             * the arithmetic of k_bf16_geglu */
            const int r = lane % GEMV_R, s = lane / GEMV_R;
            const int row = row_base + r;
            const float vt = bfw(bftr(mine + (p.bias[0] && row < p.rows ? p.bias[0][row] : 0.0f)));
            const float u = __shfl_down(vt, 1);
            if (lane < GEMV_R * SEQ && row < p.rows && (r & 1) == 0) {
                const float g = vt;
                const float x3 = __fmul_rn(__fmul_rn(g, g), g);
                const float inner = __fmul_rn(0.7978845608028654f, __fadd_rn(g, __fmul_rn(0.044715f, x3)));
                const float gl = __fmul_rn(__fmul_rn(0.5f, g), __fadd_rn(1.0f, tanhf(inner)));
                static_cast<uint16_t *>(p.y[0])[(long long)s * (p.out[0] >> 1) + (row >> 1)] = bftr(__fmul_rn(gl, u));
            }
            return;
        }
    }
    if (lane < GEMV_R * SEQ) {
        const int r = lane % GEMV_R, s = lane / GEMV_R;
        const int row = row_base + r;
        if (row < p.rows) {
            /* selects, not p.y[sg]: a lane-dependent index into the kernel
             * arguments would be lowered through scratch memory */
            const int sg = seg_of(p, row);
            const int r0 = sg == 0 ? p.row0[0] : sg == 1 ? p.row0[1] : p.row0[2];
            const int out = sg == 0 ? p.out[0] : sg == 1 ? p.out[1] : p.out[2];
            const float *bias = sg == 0 ? p.bias[0] : sg == 1 ? p.bias[1] : p.bias[2];
            void *y = sg == 0 ? p.y[0] : sg == 1 ? p.y[1] : p.y[2];
            const int o = row - r0;
            const float v = mine + (bias ? bias[o] : 0.0f);
            if constexpr (YBF) {
                const long long j = (long long)s * out + o;
                uint16_t t = (uint16_t)(__float_as_uint(v) >> 16);
                if (p.res16) t = bftr(bfw(p.res16[j]) + bfw(t)); /* the residual is segment 0's */
                static_cast<uint16_t *>(y)[j] = t;
            } else
                static_cast<float *>(y)[(long long)s * out + o] = v;
        }
    }
}

/* out[s][i] = (x[s][i] * w[i]) * r_s, r_s = 1 / sqrtf(sum_i x[s][i]^2 / dim + eps)
 * (rmsnorm.c:17-75); one workgroup per row, the sum in a fixed order
 * (per-thread strided partials, then a tree in LDS) */
__global__ __launch_bounds__(256) void k_rmsnorm_rows(float *out, const float *x, const float *w,
                                                      const float *res, int dim, float eps) {
    __shared__ float part[256];
    const float *xr = x + (long long)blockIdx.x * dim;
    float *orow = out + (long long)blockIdx.x * dim;
    float ss = 0.0f;
    for (int i = threadIdx.x; i < dim; i += 256) ss = fmaf(xr[i], xr[i], ss);
    part[threadIdx.x] = ss;
    __syncthreads();
    for (int h = 128; h > 0; h >>= 1) {
        if ((int)threadIdx.x < h) part[threadIdx.x] += part[threadIdx.x + h];
        __syncthreads();
    }
    const float rinv = 1.0f / sqrtf(part[0] / (float)dim + eps);
    const float *rr = res ? res + (long long)blockIdx.x * dim : nullptr;
    for (int i = threadIdx.x; i < dim; i += 256) {
        const float v = (xr[i] * w[i]) * rinv;
        orow[i] = rr ? rr[i] + v : v;
    }
}

/* ---- the bf16 decoder's row operations (common/decoder/qkn_bf16_decoder.c)
 * With bf(b) the bf16 bits b widened and tr(v) the truncation of v to bf16:
 *   nrm(v, w)[i] = tr((bf(v[i]) * r) * w[i]), r = 1 / sqrtf(sum_i bf(v[i])^2 / dim + eps)
 *                                                       (bf16_rms_norm, :51-71)
 *   add(a, b)[i] = tr(bf(a[i]) + bf(b[i]))            (bf16_add_inplace, :255-258)
 *   geglu(g, u)  = tr(0.5 g (1 + tanhf(0.7978845608028654 (g + 0.044715 g^3))) * u)
 *                                                       (bf16_geglu, :235-251)
 * The sums of squares run in a fixed order: per-thread strided fused
 * multiply-adds, a butterfly over the wave, then the four waves in order
 * (bfw / bftr: the widening and the truncation, defined with the GEMV). */

/* the sum of v over the 256 threads, returned to every thread */
__device__ __forceinline__ float block_sum256(float v, float *red) {
#pragma unroll
    for (int m = 32; m > 0; m >>= 1) v += __shfl_xor(v, m, 64);
    __syncthreads(); /* red may still be read by an earlier call */
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return ((red[0] + red[1]) + red[2]) + red[3];
}

/* One workgroup per row s of [seq][dim] bf16 arrays:
 *   p non-NULL:     q = w_post ? nrm(p, w_post) : p;  x = add(x, q)  (x updated)
 *   w_next non-NULL: xn = nrm(x, w_next)               (of the updated x)
 * (the Gemma 3 post-sublayer norm, the residual add and the next sublayer's
 * input norm, qkn_bf16_decoder.c:551-557 and 567-570, in one pass). xn may
 * equal x only when p is NULL; each thread reads back only the elements it
 * wrote itself. */
__global__ __launch_bounds__(256) void k_bf16_rows(uint16_t *x, const uint16_t *p, const float *w_post,
                                                   const float *w_next, uint16_t *xn, int dim, float eps) {
    __shared__ float red[4];
    const long long base = (long long)blockIdx.x * dim;
    uint16_t *xr = x + base;
    float ss = 0.0f;
    if (p) {
        const uint16_t *pr = p + base;
        float rp = 0.0f;
        if (w_post) {
            float sp = 0.0f;
            for (int i = threadIdx.x; i < dim; i += 256) {
                const float v = bfw(pr[i]);
                sp = fmaf(v, v, sp);
            }
            rp = 1.0f / sqrtf(block_sum256(sp, red) / (float)dim + eps);
        }
        for (int i = threadIdx.x; i < dim; i += 256) {
            float q = bfw(pr[i]);
            if (w_post) q = bfw(bftr((q * rp) * w_post[i]));
            const uint16_t xb = bftr(bfw(xr[i]) + q);
            xr[i] = xb;
            const float v = bfw(xb);
            ss = fmaf(v, v, ss);
        }
    } else if (w_next) {
        for (int i = threadIdx.x; i < dim; i += 256) {
            const float v = bfw(xr[i]);
            ss = fmaf(v, v, ss);
        }
    }
    if (!w_next) return;
    const float r = 1.0f / sqrtf(block_sum256(ss, red) / (float)dim + eps);
    uint16_t *nr = xn + base;
    for (int i = threadIdx.x; i < dim; i += 256) nr[i] = bftr((bfw(xr[i]) * r) * w_next[i]);
}

/* out[i] = geglu(bf(gu[2i]), bf(gu[2i + 1])) over n = seq * inter outputs
 * (row s's pair j sits at flat pair s * inter + j); every step rounded as
 * written, no fused multiply-add */
__global__ __launch_bounds__(256) void k_bf16_geglu(uint16_t *out, const uint32_t *gu, long long n) {
    const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    const uint32_t pr = gu[i];
    const float g = __uint_as_float(pr << 16), u = __uint_as_float(pr & 0xffff0000u);
    const float x3 = __fmul_rn(__fmul_rn(g, g), g);
    const float inner = __fmul_rn(0.7978845608028654f, __fadd_rn(g, __fmul_rn(0.044715f, x3)));
    const float gl = __fmul_rn(__fmul_rn(0.5f, g), __fadd_rn(1.0f, tanhf(inner)));
    out[i] = bftr(__fmul_rn(gl, u));
}

/* ------------------------------------------------------------------ host */

namespace {

int lfail(int code, const char *msg) { return smol_internal_fail(code, msg); }

#define LHIP(expr)                                                                          \
    do {                                                                                    \
        hipError_t e_ = (expr);                                                             \
        if (e_ != hipSuccess) return lfail(SMOL_ATTN_ERR_DEVICE, hipGetErrorString(e_));    \
    } while (0)

struct Buf {
    void *p = nullptr;
    size_t cap = 0;
};

/* grows a device buffer (contents not kept); the stream is drained first */
int reserve(Buf &b, size_t bytes, hipStream_t st) {
    if (bytes <= b.cap) return 0;
    size_t want = std::max(bytes, b.cap + b.cap / 2);
    want = (want + 4095) & ~(size_t)4095;
    if (b.p) {
        LHIP(hipStreamSynchronize(st));
        LHIP(hipFree(b.p));
        b.p = nullptr;
        b.cap = 0;
    }
    LHIP(hipMalloc(&b.p, want));
    b.cap = want;
    return 0;
}

int launch_rmsnorm(float *out, const float *x, const float *w, int seq, int dim, float eps, hipStream_t st,
                   const float *res = nullptr) {
    if (seq <= 0 || dim <= 0) return 0;
    hipLaunchKernelGGL(k_rmsnorm_rows, dim3((unsigned)seq), dim3(256), 0, st, out, x, w, res, dim, eps);
    LHIP(hipGetLastError());
    return 0;
}

/* the operations fused into a GEMV launch (fp32 x and y, one weight) */
struct GemvFuse {
    const float *norm_w;
    float eps;
    int act;
    const float *res;
};

template <int SEQ, bool XBF, bool YBF, bool FUSE>
int launch_gemv_v(const GemvParams &p, bool vec, hipStream_t st) {
    const int row_groups = (p.rows + GEMV_R - 1) / GEMV_R;
    const dim3 grid((unsigned)((row_groups + p.groups - 1) / p.groups)), block(64 * p.kp * p.groups);
    if (vec)
        hipLaunchKernelGGL((k_gemv<SEQ, XBF, YBF, true, FUSE>), grid, block, 0, st, p);
    else
        hipLaunchKernelGGL((k_gemv<SEQ, XBF, YBF, false, FUSE>), grid, block, 0, st, p);
    LHIP(hipGetLastError());
    return 0;
}

template <int SEQ>
int launch_gemv_s(const GemvParams &p, bool xbf, bool ybf, bool vec, bool fuse, hipStream_t st) {
    if (fuse)
        return xbf ? launch_gemv_v<SEQ, true, true, true>(p, vec, st) : launch_gemv_v<SEQ, false, false, true>(p, vec, st);
    if (xbf)
        return ybf ? launch_gemv_v<SEQ, true, true, false>(p, vec, st)
                   : launch_gemv_v<SEQ, true, false, false>(p, vec, st);
    return ybf ? launch_gemv_v<SEQ, false, true, false>(p, vec, st)
               : launch_gemv_v<SEQ, false, false, false>(p, vec, st);
}

bool aligned16(const void *p) { return ((uintptr_t)p & 15) == 0; }

/* one GEMV launch over n_seg weight segments (f: fused operations, one
 * segment, fp32 x and y) */
/* the bf16 decoder's operations of a GEMV with a bf16 y (GemvParams) */
struct GemvBf16Ops {
    int act;               /* SMOL_LINEAR_ACT_NONE or _GEGLU */
    const uint16_t *res16; /* or null */
    bool x_trunc;
    const float *norm16 = nullptr; /* bf16 x: the input RMSNorm's weight (k_bf16_rows' values), or null */
    float eps = 0.0f;
    const uint16_t *add16 = nullptr; /* with norm16: x + add16 (truncated) is normalised */
    uint16_t *xout16 = nullptr;      /* with add16: that sum is written here */
};

int run_gemv(smol_attn_ctx *ctx, hipStream_t st, const void *x, bool xbf, bool ybf, int seq, int in, int n_seg,
             const GemvSeg *segs, const GemvFuse *f = nullptr, const GemvBf16Ops *bo = nullptr) {
    GemvParams p{};
    p.x = x;
    p.in = in;
    if (f) {
        p.norm_w = f->norm_w;
        p.eps = f->eps;
        p.act = f->act;
        p.res = f->res;
    } else if (bo) {
        p.act = bo->act;
        p.res16 = bo->res16;
        p.x_trunc = bo->x_trunc ? 1 : 0;
        p.norm_w = bo->norm16;
        p.eps = bo->eps;
        p.add16 = bo->norm16 ? bo->add16 : nullptr;
        p.xout16 = bo->norm16 ? bo->xout16 : nullptr;
    }
    const bool n16 = bo && bo->norm16;
    if (n16 && (!xbf || !ybf)) return 1;
    int rows = 0;
    bool vec = (in % 8) == 0 && aligned16(x) && aligned16(p.norm_w);
    for (int i = 0; i < GEMV_SEGS; i++) {
        if (i < n_seg) {
            p.w[i] = segs[i].w;
            p.bias[i] = segs[i].bias;
            p.y[i] = segs[i].y;
            p.out[i] = segs[i].out;
            p.row0[i] = rows;
            rows += segs[i].out;
            vec = vec && aligned16(segs[i].w);
        } else {
            p.w[i] = segs[0].w;
            p.bias[i] = nullptr;
            p.y[i] = nullptr;
            p.out[i] = 0;
            p.row0[i] = INT_MAX;
        }
    }
    p.rows = rows;
    const int chunks = (in + 7) / 8;
    p.kp = std::max(1, std::min(GEMV_MAX_KP, (chunks + 64 * GEMV_U - 1) / (64 * GEMV_U)));
    p.groups = std::max(1, std::min(GEMV_WG_WAVES / p.kp, (rows + GEMV_R - 1) / GEMV_R));
    if (rows <= 0) return 0;
    if (n16) {
        /* the norm's order needs 256 threads a workgroup */
        if (4 % p.kp != 0) return 1;
        p.groups = 4 / p.kp;
    }
    hipEvent_t e0 = nullptr, e1 = nullptr;
    smol_internal_timing_events(ctx, LIN_TIMING_KIND, &e0, &e1);
    if (e0) LHIP(hipEventRecord(e0, st));
    int rc;
    const bool fuse = f != nullptr || n16;
    switch (seq) {
    case 1: rc = launch_gemv_s<1>(p, xbf, ybf, vec, fuse, st); break;
    case 2: rc = launch_gemv_s<2>(p, xbf, ybf, vec, fuse, st); break;
    case 3: rc = launch_gemv_s<3>(p, xbf, ybf, vec, fuse, st); break;
    default: rc = launch_gemv_s<4>(p, xbf, ybf, vec, fuse, st); break;
    }
    if (rc) return rc;
    if (e1) LHIP(hipEventRecord(e1, st));
    return 0;
}

/* y = x W^T (+ bias) as GEMV launches over blocks of up to
 * SMOL_LINEAR_GEMV_MAX_SEQ rows (in_dim 0, and operands k_gemm's 16-byte
 * staging cannot take) */
int run_gemv_rows(smol_attn_ctx *ctx, hipStream_t st, void *y, bool ybf, const void *x, bool xbf,
                  const uint16_t *w, const float *bias, int seq, int in, int out, const GemvFuse *f = nullptr) {
    const size_t xe = xbf ? 2 : 4, ye = ybf ? 2 : 4;
    const int ycols = f && f->act ? out / 2 : out;
    for (int s0 = 0; s0 < seq; s0 += SMOL_LINEAR_GEMV_MAX_SEQ) {
        const int n = std::min(SMOL_LINEAR_GEMV_MAX_SEQ, seq - s0);
        const GemvSeg sg{w, bias, static_cast<char *>(y) + (size_t)s0 * ycols * ye, out};
        const void *xs = x ? static_cast<const char *>(x) + (size_t)s0 * in * xe : nullptr;
        GemvFuse fb;
        if (f) {
            fb = *f;
            if (fb.res) fb.res += (size_t)s0 * ycols;
        }
        if (int rc = run_gemv(ctx, st, xs, xbf, ybf, n, in, 1, &sg, f ? &fb : nullptr)) return rc;
    }
    return 0;
}

/* k_gemm's tile configurations (gemm.hip): 192 x 192, 128 x 128 and 64 x 64
 * (rows x outputs); one workgroup per compute unit for the first two, two
 * for the last. The time of a launch is about its rounds of workgroups over
 * the device times a round's time; the weights below are the measured time
 * of one round per unit of tile area relative to 192 x 192 (M = 1536,
 * K = 1024, fp32 x: about 41-51, 22-24 and 16-18 us a round; the bf16 x
 * ratios are alike). */
int gemm_cfg(smol_attn_ctx *ctx, int M, int N, int seg_align = 0) {
    static const int per_cu[3] = {1, 1, 2};
    static const float cost[3] = {1.0f, 1.15f, 3.4f};
    const int forced = smol_internal_ctx_option(ctx, SMOL_OPT_GEMM_TILE);
    if (forced >= 1 && forced <= 3) {
        int bm, bn;
        smol_gemm_tile(forced - 1, &bm, &bn);
        return seg_align % bn == 0 ? forced - 1 : -1;
    }
    const int cus = smol_internal_ctx_cus(ctx);
    int best = -1;
    double best_t = 1e300;
    for (int cfg = 0; cfg < 3; cfg++) {
        int bm, bn;
        smol_gemm_tile(cfg, &bm, &bn);
        if (seg_align % bn != 0) continue; /* segment boundaries on tile edges */
        const long long tiles = (long long)((M + bm - 1) / bm) * ((N + bn - 1) / bn);
        const long long slots = (long long)cus * per_cu[cfg];
        const double t = (double)((tiles + slots - 1) / slots) * bm * bn * cost[cfg];
        if (t < best_t) {
            best_t = t;
            best = cfg;
        }
    }
    return best;
}

/* y = res + act(norm(x) W^T + bias) for seq rows on k_gemm; falls back to
 * GEMV launches over blocks of rows where the operands do not suit the
 * tiles' 16-byte staging (in_dim % 8 != 0, unaligned x or W) */
int run_gemm(smol_attn_ctx *ctx, hipStream_t st, void *y, bool ybf, const void *x, bool xbf, const uint16_t *w,
             const float *bias, int seq, int in, int out, const GemvFuse *f = nullptr) {
    if (in % 8 != 0 || !aligned16(x) || !aligned16(w) || (f && f->norm_w && !aligned16(f->norm_w)) ||
        (long long)out * in * 2 > 0x7FFF0000LL || (long long)seq * in * 4 > 0x7FFF0000LL)
        return run_gemv_rows(ctx, st, y, ybf, x, xbf, w, bias, seq, in, out, f);
    GemmParams p{};
    p.w = w;
    p.x = x;
    p.y = y;
    p.bias = bias;
    if (f) {
        p.g = f->norm_w;
        p.eps = f->eps;
        p.act = f->act;
        p.res = f->res;
    }
    p.M = seq;
    p.N = out;
    p.K = in;
    p.rm = 1; /* the launcher chooses the region split */
    hipEvent_t e0 = nullptr, e1 = nullptr;
    smol_internal_timing_events(ctx, LIN_TIMING_KIND, &e0, &e1);
    const int rc = smol_launch_gemm(&p, gemm_cfg(ctx, seq, out), xbf, ybf, st, e0, e1);
    if (rc) return lfail(SMOL_ATTN_ERR_DEVICE, rc == -1 ? "k_gemm: unsupported operands" : "k_gemm launch failed");
    return 0;
}

/* Q, K and V of one x on k_gemm as one launch: the three outputs side by
 * side as column segments of one product (x is staged and split once per
 * row tile instead of three times); 1 when the shapes do not allow it
 * (segment widths not multiples of a tile width, operands the staging
 * cannot take), and the caller runs three products */
int run_gemm_qkv(smol_attn_ctx *ctx, hipStream_t st, void *q, void *k, void *v, bool ybf, const void *x, bool xbf,
                 const uint16_t *wq, const uint16_t *wk, const uint16_t *wv, int seq, int in, int q_dim, int kv_dim,
                 const GemvFuse *f) {
    if (!q_dim || !kv_dim || in % 8 != 0 || !aligned16(x) || !aligned16(wq) || !aligned16(wk) || !aligned16(wv) ||
        (f && f->norm_w && !aligned16(f->norm_w)) || (long long)q_dim * in * 2 > 0x7FFF0000LL ||
        (long long)kv_dim * in * 2 > 0x7FFF0000LL || (long long)seq * in * 4 > 0x7FFF0000LL)
        return 1;
    const int cfg = gemm_cfg(ctx, seq, q_dim + 2 * kv_dim, std::gcd(q_dim, kv_dim));
    if (cfg < 0) return 1;
    GemmParams p{};
    p.w = wq;
    p.x = x;
    p.y = q;
    if (f) {
        p.g = f->norm_w;
        p.eps = f->eps;
    }
    p.M = seq;
    p.N = q_dim + 2 * kv_dim;
    p.K = in;
    p.rm = 1;
    p.nseg = 3;
    p.seg_c[0] = 0;
    p.seg_c[1] = q_dim;
    p.seg_c[2] = q_dim + kv_dim;
    p.seg_c[3] = q_dim + 2 * kv_dim;
    p.seg_w[0] = wq; p.seg_w[1] = wk; p.seg_w[2] = wv;
    p.seg_y[0] = q; p.seg_y[1] = k; p.seg_y[2] = v;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    smol_internal_timing_events(ctx, LIN_TIMING_KIND, &e0, &e1);
    const int rc = smol_launch_gemm(&p, cfg, xbf, ybf, st, e0, e1);
    if (rc) return lfail(SMOL_ATTN_ERR_DEVICE, rc == -1 ? "k_gemm: unsupported operands" : "k_gemm launch failed");
    return 0;
}

int check_dtype(int t) { return t == SMOL_ATTN_F32 || t == SMOL_ATTN_BF16; }

}  // namespace

extern "C" int smol_linear_dev(smol_attn_ctx *ctx, void *y, int y_dtype, const void *x, int x_dtype,
                               const uint16_t *w, const float *bias, int seq, int in_dim, int out_dim) {
    if (!ctx) return lfail(SMOL_ATTN_ERR_ARG, "smol_linear_dev: null context");
    if (!check_dtype(x_dtype) || !check_dtype(y_dtype)) return lfail(SMOL_ATTN_ERR_ARG, "smol_linear_dev: dtype");
    if (seq < 0 || in_dim < 0 || out_dim < 0) return lfail(SMOL_ATTN_ERR_ARG, "smol_linear_dev: negative size");
    if (seq == 0 || out_dim == 0) return SMOL_ATTN_OK;
    if (!y || (in_dim > 0 && (!x || !w))) return lfail(SMOL_ATTN_ERR_ARG, "smol_linear_dev: null pointer");
    if ((long long)seq * in_dim > INT_MAX / 4 || (long long)seq * out_dim > INT_MAX / 4 ||
        (long long)out_dim * in_dim > (1LL << 40))
        return lfail(SMOL_ATTN_ERR_UNSUPPORTED, "smol_linear_dev: sizes beyond the supported range");
    LHIP(hipSetDevice(smol_internal_ctx_device(ctx)));
    hipStream_t st = static_cast<hipStream_t>(smol_attn_ctx_stream(ctx));
    const bool xbf = x_dtype == SMOL_ATTN_BF16, ybf = y_dtype == SMOL_ATTN_BF16;
    if (seq <= SMOL_LINEAR_GEMV_MAX_SEQ || in_dim == 0)
        return run_gemv_rows(ctx, st, y, ybf, x, xbf, w, bias, seq, in_dim, out_dim);
    return run_gemm(ctx, st, y, ybf, x, xbf, w, bias, seq, in_dim, out_dim);
}

/* For the bf16 decoder's layer (qkn_attn.hip), seq <= SMOL_LINEAR_GEMV_MAX_SEQ
 * only: y [seq][out or out / 2] bf16 = the truncating projection of x (bf16,
 * or fp32 truncated to bf16 as it is loaded: x_f32_trunc), then act GEGLU of
 * the (gate, up) pairs (bf16_geglu) or the residual add y = tr(bf(res16) +
 * bf(y)) (bf16_add_inplace; res16 may equal y), in the one GEMV launch. */
extern "C" int smol_internal_linear_bf16_ops(smol_attn_ctx *ctx, uint16_t *y, const void *x, int x_f32_trunc,
                                             const uint16_t *w, int seq, int in_dim, int out_dim, int act,
                                             const uint16_t *res16) {
    if (!ctx || !y || !x || !w || seq <= 0 || seq > SMOL_LINEAR_GEMV_MAX_SEQ || in_dim <= 0 || out_dim <= 0 ||
        (act != SMOL_LINEAR_ACT_NONE && act != SMOL_LINEAR_ACT_GEGLU) || (act && ((out_dim & 1) || res16)))
        return lfail(SMOL_ATTN_ERR_ARG, "smol_internal_linear_bf16_ops: arguments");
    LHIP(hipSetDevice(smol_internal_ctx_device(ctx)));
    hipStream_t st = static_cast<hipStream_t>(smol_attn_ctx_stream(ctx));
    const GemvSeg sg{w, nullptr, y, out_dim};
    const GemvBf16Ops bo{act, res16, x_f32_trunc != 0};
    return run_gemv(ctx, st, x, x_f32_trunc == 0, true, seq, in_dim, 1, &sg, nullptr, &bo);
}

extern "C" int smol_linear_qkv_dev(smol_attn_ctx *ctx, void *q, void *k, void *v, int y_dtype, const void *x,
                                   int x_dtype, const uint16_t *wq, const uint16_t *wk, const uint16_t *wv, int seq,
                                   int in_dim, int q_dim, int kv_dim) {
    if (!ctx) return lfail(SMOL_ATTN_ERR_ARG, "smol_linear_qkv_dev: null context");
    if (!check_dtype(x_dtype) || !check_dtype(y_dtype)) return lfail(SMOL_ATTN_ERR_ARG, "smol_linear_qkv_dev: dtype");
    if (seq < 0 || in_dim < 0 || q_dim < 0 || kv_dim < 0)
        return lfail(SMOL_ATTN_ERR_ARG, "smol_linear_qkv_dev: negative size");
    if (seq > SMOL_LINEAR_GEMV_MAX_SEQ && in_dim > 0 && q_dim > 0 && kv_dim > 0 && q && k && v && x && wq && wk &&
        wv && (long long)seq * in_dim <= INT_MAX / 4 && (long long)seq * (q_dim + 2LL * kv_dim) <= INT_MAX / 4) {
        LHIP(hipSetDevice(smol_internal_ctx_device(ctx)));
        hipStream_t st = static_cast<hipStream_t>(smol_attn_ctx_stream(ctx));
        const int rc = run_gemm_qkv(ctx, st, q, k, v, y_dtype == SMOL_ATTN_BF16, x, x_dtype == SMOL_ATTN_BF16, wq, wk,
                                    wv, seq, in_dim, q_dim, kv_dim, nullptr);
        if (rc <= 0) return rc;
    }
    if (seq > SMOL_LINEAR_GEMV_MAX_SEQ || in_dim == 0) {
        if (int rc = smol_linear_dev(ctx, q, y_dtype, x, x_dtype, wq, nullptr, seq, in_dim, q_dim)) return rc;
        if (int rc = smol_linear_dev(ctx, k, y_dtype, x, x_dtype, wk, nullptr, seq, in_dim, kv_dim)) return rc;
        return smol_linear_dev(ctx, v, y_dtype, x, x_dtype, wv, nullptr, seq, in_dim, kv_dim);
    }
    if (seq == 0 || (q_dim == 0 && kv_dim == 0)) return SMOL_ATTN_OK;
    if (!x || (q_dim && (!q || !wq)) || (kv_dim && (!k || !v || !wk || !wv)))
        return lfail(SMOL_ATTN_ERR_ARG, "smol_linear_qkv_dev: null pointer");
    if ((long long)seq * in_dim > INT_MAX / 4 || (long long)q_dim + 2LL * kv_dim > INT_MAX / 4)
        return lfail(SMOL_ATTN_ERR_UNSUPPORTED, "smol_linear_qkv_dev: sizes beyond the supported range");
    LHIP(hipSetDevice(smol_internal_ctx_device(ctx)));
    hipStream_t st = static_cast<hipStream_t>(smol_attn_ctx_stream(ctx));
    GemvSeg segs[GEMV_SEGS];
    int n = 0;
    if (q_dim) segs[n++] = GemvSeg{wq, nullptr, q, q_dim};
    if (kv_dim) {
        segs[n++] = GemvSeg{wk, nullptr, k, kv_dim};
        segs[n++] = GemvSeg{wv, nullptr, v, kv_dim};
    }
    return run_gemv(ctx, st, x, x_dtype == SMOL_ATTN_BF16, y_dtype == SMOL_ATTN_BF16, seq, in_dim, n, segs);
}

/* The bf16 decoder's input RMSNorm (qkn_bf16_decoder.c:51-71) and its Q/K/V
 * projections for at most SMOL_LINEAR_GEMV_MAX_SEQ rows in one GEMV launch:
 * the normalised row is formed as x is loaded, with the bits k_bf16_rows
 * (smol_bf16_rms_norm_dev) would write, so the outputs equal the two launches'
 * bit for bit. Returns 1, launching nothing, where the shape does not allow
 * it (more rows, an in_dim needing eight waves a row, misaligned operands are
 * still handled; the caller then runs the norm and the projections apart). */
extern "C" int smol_internal_linear_qkv_bf16_norm(smol_attn_ctx *ctx, uint16_t *q, uint16_t *k, uint16_t *v,
                                                  const uint16_t *x, const float *norm_w, float eps,
                                                  const uint16_t *wq, const uint16_t *wk, const uint16_t *wv, int seq,
                                                  int in_dim, int q_dim, int kv_dim) {
    if (!ctx || !q || !k || !v || !x || !norm_w || !wq || !wk || !wv || seq <= 0 ||
        seq > SMOL_LINEAR_GEMV_MAX_SEQ || in_dim <= 0 || q_dim <= 0 || kv_dim <= 0 ||
        (long long)seq * in_dim > INT_MAX / 4 || (long long)q_dim + 2LL * kv_dim > INT_MAX / 4)
        return 1;
    LHIP(hipSetDevice(smol_internal_ctx_device(ctx)));
    hipStream_t st = static_cast<hipStream_t>(smol_attn_ctx_stream(ctx));
    const GemvSeg segs[3] = {GemvSeg{wq, nullptr, q, q_dim}, GemvSeg{wk, nullptr, k, kv_dim},
                             GemvSeg{wv, nullptr, v, kv_dim}};
    GemvBf16Ops bo{SMOL_LINEAR_ACT_NONE, nullptr, false};
    bo.norm16 = norm_w;
    bo.eps = eps;
    return run_gemv(ctx, st, x, true, true, seq, in_dim, 3, segs, nullptr, &bo);
}

/* The bf16 decoder's residual add, post-attention RMSNorm and GeGLU gate_up
 * projection (qkn_bf16_decoder.c:551-557 without the Gemma 3 post-sublayer
 * norm, then :560-563) for at most SMOL_LINEAR_GEMV_MAX_SEQ rows in one GEMV
 * launch: x_new = tr(bf(x) + bf(p)) is written to x_new (x is left as it is:
 * every workgroup reads it), normalised as k_bf16_rows does and multiplied,
 * and g = geglu of the truncated (gate, up) pairs. Returns 1, launching
 * nothing, where the shape does not allow it. */
extern "C" int smol_internal_linear_bf16_addnorm_geglu(smol_attn_ctx *ctx, uint16_t *g, const uint16_t *x,
                                                       const uint16_t *p, uint16_t *x_new, const float *norm_w,
                                                       float eps, const uint16_t *w_gate_up, int seq, int in_dim,
                                                       int out_dim) {
    if (!ctx || !g || !x || !p || !x_new || !norm_w || !w_gate_up || seq <= 0 || seq > SMOL_LINEAR_GEMV_MAX_SEQ ||
        in_dim <= 0 || out_dim <= 0 || (out_dim & 1) || (long long)seq * in_dim > INT_MAX / 4 ||
        (long long)seq * out_dim > INT_MAX / 4)
        return 1;
    LHIP(hipSetDevice(smol_internal_ctx_device(ctx)));
    hipStream_t st = static_cast<hipStream_t>(smol_attn_ctx_stream(ctx));
    const GemvSeg sg{w_gate_up, nullptr, g, out_dim};
    GemvBf16Ops bo{SMOL_LINEAR_ACT_GEGLU, nullptr, false};
    bo.norm16 = norm_w;
    bo.eps = eps;
    bo.add16 = p;
    bo.xout16 = x_new;
    return run_gemv(ctx, st, x, true, true, seq, in_dim, 1, &sg, nullptr, &bo);
}

extern "C" int smol_linear_ops_dev(smol_attn_ctx *ctx, float *y, const float *x, const uint16_t *w,
                                   const float *bias, int seq, int in_dim, int out_dim, const smol_linear_ops *ops) {
    if (!ctx) return lfail(SMOL_ATTN_ERR_ARG, "smol_linear_ops_dev: null context");
    const smol_linear_ops none{};
    if (!ops) ops = &none;
    if (seq < 0 || in_dim <= 0 || out_dim < 0) return lfail(SMOL_ATTN_ERR_ARG, "smol_linear_ops_dev: sizes");
    if (ops->act != SMOL_LINEAR_ACT_NONE && ops->act != SMOL_LINEAR_ACT_SWIGLU && ops->act != SMOL_LINEAR_ACT_GEGLU)
        return lfail(SMOL_ATTN_ERR_ARG, "smol_linear_ops_dev: act");
    if (ops->act && (out_dim & 1)) return lfail(SMOL_ATTN_ERR_ARG, "smol_linear_ops_dev: act needs an even out_dim");
    if (seq == 0 || out_dim == 0) return SMOL_ATTN_OK;
    if (!y || !x || !w) return lfail(SMOL_ATTN_ERR_ARG, "smol_linear_ops_dev: null pointer");
    if (x == y || (ops->residual && ops->residual != y &&
                   !((const char *)ops->residual + (size_t)seq * (ops->act ? out_dim / 2 : out_dim) * 4 <=
                         (const char *)y ||
                     (const char *)y + (size_t)seq * (ops->act ? out_dim / 2 : out_dim) * 4 <=
                         (const char *)ops->residual)))
        return lfail(SMOL_ATTN_ERR_ARG, "smol_linear_ops_dev: y overlaps x, or partly overlaps the residual");
    if ((long long)seq * in_dim > INT_MAX / 4 || (long long)seq * out_dim > INT_MAX / 4 ||
        (long long)out_dim * in_dim > (1LL << 40))
        return lfail(SMOL_ATTN_ERR_UNSUPPORTED, "smol_linear_ops_dev: sizes beyond the supported range");
    LHIP(hipSetDevice(smol_internal_ctx_device(ctx)));
    hipStream_t st = static_cast<hipStream_t>(smol_attn_ctx_stream(ctx));
    const GemvFuse f{ops->norm_weight, ops->norm_eps, ops->act, ops->residual};
    if (seq <= SMOL_LINEAR_GEMV_MAX_SEQ) return run_gemv_rows(ctx, st, y, false, x, false, w, bias, seq, in_dim, out_dim, &f);
    return run_gemm(ctx, st, y, false, x, false, w, bias, seq, in_dim, out_dim, &f);
}

extern "C" int smol_linear_qkv_norm_dev(smol_attn_ctx *ctx, float *q, float *k, float *v, const float *x,
                                        const uint16_t *wq, const uint16_t *wk, const uint16_t *wv, int seq,
                                        int in_dim, int q_dim, int kv_dim, const float *norm_weight,
                                        float norm_eps) {
    if (!norm_weight)
        return smol_linear_qkv_dev(ctx, q, k, v, SMOL_ATTN_F32, x, SMOL_ATTN_F32, wq, wk, wv, seq, in_dim, q_dim,
                                   kv_dim);
    if (!ctx) return lfail(SMOL_ATTN_ERR_ARG, "smol_linear_qkv_norm_dev: null context");
    if (seq < 0 || in_dim <= 0 || q_dim < 0 || kv_dim < 0)
        return lfail(SMOL_ATTN_ERR_ARG, "smol_linear_qkv_norm_dev: sizes");
    if (seq == 0 || (q_dim == 0 && kv_dim == 0)) return SMOL_ATTN_OK;
    if (!x || (q_dim && (!q || !wq)) || (kv_dim && (!k || !v || !wk || !wv)))
        return lfail(SMOL_ATTN_ERR_ARG, "smol_linear_qkv_norm_dev: null pointer");
    if ((long long)seq * in_dim > INT_MAX / 4 || (long long)seq * (q_dim + 2LL * kv_dim) > INT_MAX / 4)
        return lfail(SMOL_ATTN_ERR_UNSUPPORTED, "smol_linear_qkv_norm_dev: sizes beyond the supported range");
    LHIP(hipSetDevice(smol_internal_ctx_device(ctx)));
    hipStream_t st = static_cast<hipStream_t>(smol_attn_ctx_stream(ctx));
    if (seq > SMOL_LINEAR_GEMV_MAX_SEQ) {
        /* the GEMM path: the products normalise their rows from the x they
         * stage (one launch for the three where the shapes allow) */
        const GemvFuse f{norm_weight, norm_eps, SMOL_LINEAR_ACT_NONE, nullptr};
        const int rq = run_gemm_qkv(ctx, st, q, k, v, false, x, false, wq, wk, wv, seq, in_dim, q_dim, kv_dim, &f);
        if (rq <= 0) return rq;
        if (int rc = run_gemm(ctx, st, q, false, x, false, wq, nullptr, seq, in_dim, q_dim, &f)) return rc;
        if (int rc = run_gemm(ctx, st, k, false, x, false, wk, nullptr, seq, in_dim, kv_dim, &f)) return rc;
        return run_gemm(ctx, st, v, false, x, false, wv, nullptr, seq, in_dim, kv_dim, &f);
    }
    GemvSeg segs[GEMV_SEGS];
    int n = 0;
    if (q_dim) segs[n++] = GemvSeg{wq, nullptr, q, q_dim};
    if (kv_dim) {
        segs[n++] = GemvSeg{wk, nullptr, k, kv_dim};
        segs[n++] = GemvSeg{wv, nullptr, v, kv_dim};
    }
    const GemvFuse f{norm_weight, norm_eps, SMOL_LINEAR_ACT_NONE, nullptr};
    return run_gemv(ctx, st, x, false, false, seq, in_dim, n, segs, &f);
}

extern "C" int smol_rms_norm_dev(smol_attn_ctx *ctx, float *out, const float *x, const float *weight,
                                 const float *residual, int seq, int dim, float eps) {
    if (!ctx) return lfail(SMOL_ATTN_ERR_ARG, "smol_rms_norm_dev: null context");
    if (seq < 0 || dim < 0) return lfail(SMOL_ATTN_ERR_ARG, "smol_rms_norm_dev: negative size");
    if (seq == 0 || dim == 0) return SMOL_ATTN_OK;
    if (!out || !x || !weight) return lfail(SMOL_ATTN_ERR_ARG, "smol_rms_norm_dev: null pointer");
    LHIP(hipSetDevice(smol_internal_ctx_device(ctx)));
    hipStream_t st = static_cast<hipStream_t>(smol_attn_ctx_stream(ctx));
    hipEvent_t e0 = nullptr, e1 = nullptr;
    smol_internal_timing_events(ctx, LIN_TIMING_KIND, &e0, &e1);
    if (e0) LHIP(hipEventRecord(e0, st));
    if (int rc = launch_rmsnorm(out, x, weight, seq, dim, eps, st, residual)) return rc;
    if (e1) LHIP(hipEventRecord(e1, st));
    return 0;
}

extern "C" int smol_bf16_add_norm_dev(smol_attn_ctx *ctx, uint16_t *x, const uint16_t *p, const float *p_norm,
                                      const float *next_norm, uint16_t *xn, int seq, int dim, float eps) {
    if (!ctx) return lfail(SMOL_ATTN_ERR_ARG, "smol_bf16_add_norm_dev: null context");
    if (seq < 0 || dim < 0) return lfail(SMOL_ATTN_ERR_ARG, "smol_bf16_add_norm_dev: negative size");
    if (seq == 0 || dim == 0 || (!p && !next_norm)) return SMOL_ATTN_OK;
    if (!x || (next_norm && !xn) || (p_norm && !p)) return lfail(SMOL_ATTN_ERR_ARG, "smol_bf16_add_norm_dev: null pointer");
    const size_t bytes = (size_t)seq * dim * 2;
    auto overlap = [bytes](const void *a, const void *b) {
        return a && b && (const char *)a < (const char *)b + bytes && (const char *)b < (const char *)a + bytes;
    };
    if (overlap(x, p) || (p && overlap(xn, x)) || overlap(xn, p) || (xn && xn != x && overlap(xn, x)))
        return lfail(SMOL_ATTN_ERR_ARG, "smol_bf16_add_norm_dev: overlapping arrays (xn may equal x only without p)");
    LHIP(hipSetDevice(smol_internal_ctx_device(ctx)));
    hipStream_t st = static_cast<hipStream_t>(smol_attn_ctx_stream(ctx));
    hipLaunchKernelGGL(k_bf16_rows, dim3((unsigned)seq), dim3(256), 0, st, x, p, p_norm, next_norm, xn, dim, eps);
    LHIP(hipGetLastError());
    return 0;
}

extern "C" int smol_bf16_rms_norm_dev(smol_attn_ctx *ctx, uint16_t *out, const uint16_t *x, const float *weight,
                                      int seq, int dim, float eps) {
    if (!ctx) return lfail(SMOL_ATTN_ERR_ARG, "smol_bf16_rms_norm_dev: null context");
    if (seq < 0 || dim < 0) return lfail(SMOL_ATTN_ERR_ARG, "smol_bf16_rms_norm_dev: negative size");
    if (seq == 0 || dim == 0) return SMOL_ATTN_OK;
    if (!out || !x || !weight) return lfail(SMOL_ATTN_ERR_ARG, "smol_bf16_rms_norm_dev: null pointer");
    const size_t bytes = (size_t)seq * dim * 2;
    if (out != x && (const char *)out < (const char *)x + bytes && (const char *)x < (const char *)out + bytes)
        return lfail(SMOL_ATTN_ERR_ARG, "smol_bf16_rms_norm_dev: out partly overlaps x");
    LHIP(hipSetDevice(smol_internal_ctx_device(ctx)));
    hipStream_t st = static_cast<hipStream_t>(smol_attn_ctx_stream(ctx));
    /* the kernel reads x through its residual pointer and writes xn; nothing is added */
    hipLaunchKernelGGL(k_bf16_rows, dim3((unsigned)seq), dim3(256), 0, st, const_cast<uint16_t *>(x),
                       (const uint16_t *)nullptr, (const float *)nullptr, weight, out, dim, eps);
    LHIP(hipGetLastError());
    return 0;
}

extern "C" int smol_bf16_geglu_dev(smol_attn_ctx *ctx, uint16_t *out, const uint16_t *gate_up, int seq, int inter) {
    if (!ctx) return lfail(SMOL_ATTN_ERR_ARG, "smol_bf16_geglu_dev: null context");
    if (seq < 0 || inter < 0) return lfail(SMOL_ATTN_ERR_ARG, "smol_bf16_geglu_dev: negative size");
    if (seq == 0 || inter == 0) return SMOL_ATTN_OK;
    if (!out || !gate_up) return lfail(SMOL_ATTN_ERR_ARG, "smol_bf16_geglu_dev: null pointer");
    if ((uintptr_t)gate_up & 3) return lfail(SMOL_ATTN_ERR_ARG, "smol_bf16_geglu_dev: gate_up must be 4-byte aligned");
    const long long n = (long long)seq * inter;
    if ((const char *)out < (const char *)gate_up + n * 4 && (const char *)gate_up < (const char *)out + n * 2)
        return lfail(SMOL_ATTN_ERR_ARG, "smol_bf16_geglu_dev: out overlaps gate_up");
    LHIP(hipSetDevice(smol_internal_ctx_device(ctx)));
    hipStream_t st = static_cast<hipStream_t>(smol_attn_ctx_stream(ctx));
    hipLaunchKernelGGL(k_bf16_geglu, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, out,
                       reinterpret_cast<const uint32_t *>(gate_up), n);
    LHIP(hipGetLastError());
    return 0;
}

/* ------------------------------------------------- reference-signature drop-ins */

namespace {

[[noreturn]] void dropin_abort(const char *fn) {
    fprintf(stderr, "smol_attn: %s failed on the GPU: %s\n", fn, smol_attn_last_error());
    abort();
}

/* device copies of weights kept by (host pointer, elements) when
 * SMOL_BF16_CACHE_MB is set (common/kernels/matmul.c:136-189) */
struct WeightCache {
    bool init = false;
    size_t limit = 0, used = 0;
    std::map<std::pair<const void *, size_t>, void *> map;
};

struct DropIn {
    Buf x, w[3], b, y[3];
    WeightCache cache;
};

thread_local DropIn g_drop;

void upload(const char *fn, smol_attn_ctx *ctx, Buf &b, const void *h, size_t bytes) {
    hipStream_t st = static_cast<hipStream_t>(smol_attn_ctx_stream(ctx));
    if (reserve(b, std::max<size_t>(bytes, 16), st)) dropin_abort(fn);
    if (bytes && hipMemcpyAsync(b.p, h, bytes, hipMemcpyHostToDevice, st) != hipSuccess) dropin_abort(fn);
}

/* device weight for a host weight array */
const uint16_t *weight(const char *fn, smol_attn_ctx *ctx, int slot, const uint16_t *h, size_t n) {
    WeightCache &c = g_drop.cache;
    if (!c.init) {
        c.init = true;
        const char *env = getenv("SMOL_BF16_CACHE_MB");
        if (env && env[0]) {
            char *end = nullptr;
            const unsigned long long mb = strtoull(env, &end, 10);
            if (end != env) c.limit = (size_t)mb << 20;
        }
    }
    const auto key = std::make_pair((const void *)h, n);
    auto it = c.map.find(key);
    if (it != c.map.end()) return static_cast<const uint16_t *>(it->second);
    const size_t bytes = n * 2;
    hipStream_t st = static_cast<hipStream_t>(smol_attn_ctx_stream(ctx));
    if (c.limit && bytes <= c.limit && c.used + bytes <= c.limit) {
        void *d = nullptr;
        if (hipMalloc(&d, std::max<size_t>(bytes, 16)) == hipSuccess) {
            if (bytes && hipMemcpyAsync(d, h, bytes, hipMemcpyHostToDevice, st) != hipSuccess) dropin_abort(fn);
            c.map.emplace(key, d);
            c.used += bytes;
            return static_cast<const uint16_t *>(d);
        }
    }
    upload(fn, ctx, g_drop.w[slot], h, bytes);
    return static_cast<const uint16_t *>(g_drop.w[slot].p);
}

void download(const char *fn, smol_attn_ctx *ctx, void *h, const Buf &b, size_t bytes) {
    hipStream_t st = static_cast<hipStream_t>(smol_attn_ctx_stream(ctx));
    if (bytes && hipMemcpyAsync(h, b.p, bytes, hipMemcpyDeviceToHost, st) != hipSuccess) dropin_abort(fn);
}

void finish(const char *fn, smol_attn_ctx *ctx) {
    if (smol_attn_ctx_synchronize(ctx) != SMOL_ATTN_OK) dropin_abort(fn);
}

void linear_dropin(const char *fn, float *y, const float *x, const uint16_t *W, const float *b, int seq, int in,
                   int out) {
    if (seq <= 0 || out <= 0) return;
    smol_attn_ctx *ctx = smol_internal_legacy_ctx(fn);
    if (in < 0) in = 0;
    const size_t nx = (size_t)seq * in, ny = (size_t)seq * out;
    hipStream_t st = static_cast<hipStream_t>(smol_attn_ctx_stream(ctx));
    if (hipSetDevice(smol_internal_ctx_device(ctx)) != hipSuccess) dropin_abort(fn);
    upload(fn, ctx, g_drop.x, x, nx * 4);
    const uint16_t *wd = in ? weight(fn, ctx, 0, W, (size_t)out * in) : nullptr;
    const float *bd = nullptr;
    if (b) {
        upload(fn, ctx, g_drop.b, b, (size_t)out * 4);
        bd = static_cast<const float *>(g_drop.b.p);
    }
    if (reserve(g_drop.y[0], ny * 4, st)) dropin_abort(fn);
    if (smol_linear_dev(ctx, g_drop.y[0].p, SMOL_ATTN_F32, g_drop.x.p, SMOL_ATTN_F32, wd, bd, seq, in, out))
        dropin_abort(fn);
    download(fn, ctx, y, g_drop.y[0], ny * 4);
    finish(fn, ctx);
}

}  // namespace

extern "C" void smol_linear_bf16(float *y, const float *x, const uint16_t *W_bf16, const float *b, int seq_len,
                                 int in_dim, int out_dim) {
    linear_dropin("smol_linear_bf16", y, x, W_bf16, b, seq_len, in_dim, out_dim);
}

extern "C" void smol_linear_nobias_bf16(float *y, const float *x, const uint16_t *W_bf16, int seq_len, int in_dim,
                                        int out_dim) {
    linear_dropin("smol_linear_nobias_bf16", y, x, W_bf16, nullptr, seq_len, in_dim, out_dim);
}

extern "C" void smol_matmul_t_bf16(float *C, const float *A, const uint16_t *B_bf16, int M, int K, int N) {
    linear_dropin("smol_matmul_t_bf16", C, A, B_bf16, nullptr, M, K, N);
}

extern "C" void smol_linear_nobias_bf16_qkv(float *q, float *k, float *v, const float *x, const uint16_t *Wq_bf16,
                                            const uint16_t *Wk_bf16, const uint16_t *Wv_bf16, int in_dim, int q_dim,
                                            int kv_dim) {
    const char *fn = "smol_linear_nobias_bf16_qkv";
    if (q_dim < 0) q_dim = 0;
    if (kv_dim < 0) kv_dim = 0;
    if (q_dim == 0 && kv_dim == 0) return;
    smol_attn_ctx *ctx = smol_internal_legacy_ctx(fn);
    if (in_dim < 0) in_dim = 0;
    hipStream_t st = static_cast<hipStream_t>(smol_attn_ctx_stream(ctx));
    if (hipSetDevice(smol_internal_ctx_device(ctx)) != hipSuccess) dropin_abort(fn);
    upload(fn, ctx, g_drop.x, x, (size_t)in_dim * 4);
    const uint16_t *wq = nullptr, *wk = nullptr, *wv = nullptr;
    if (in_dim) {
        if (q_dim) wq = weight(fn, ctx, 0, Wq_bf16, (size_t)q_dim * in_dim);
        if (kv_dim) {
            wk = weight(fn, ctx, 1, Wk_bf16, (size_t)kv_dim * in_dim);
            wv = weight(fn, ctx, 2, Wv_bf16, (size_t)kv_dim * in_dim);
        }
    }
    const int dims[3] = {q_dim, kv_dim, kv_dim};
    for (int i = 0; i < 3; i++)
        if (reserve(g_drop.y[i], (size_t)std::max(dims[i], 4) * 4, st)) dropin_abort(fn);
    if (smol_linear_qkv_dev(ctx, g_drop.y[0].p, g_drop.y[1].p, g_drop.y[2].p, SMOL_ATTN_F32, g_drop.x.p,
                            SMOL_ATTN_F32, wq, wk, wv, 1, in_dim, q_dim, kv_dim))
        dropin_abort(fn);
    download(fn, ctx, q, g_drop.y[0], (size_t)q_dim * 4);
    download(fn, ctx, k, g_drop.y[1], (size_t)kv_dim * 4);
    download(fn, ctx, v, g_drop.y[2], (size_t)kv_dim * 4);
    finish(fn, ctx);
}
