/*
 * attn_prep.hip - the pre-pass k_prep (per-head RMSNorm + RoPE + cache append
 * + fp16 staging: common/decoder/qkn_decoder.c:487-503 and :640-652),
 * k_norm_rope (in-place per-head RMSNorm and / or RoPE on fp32) and
 * k_to_bf16_trunc, with their launchers.
 */
#include "attn_device.h"

/* grid (n_blocks, Hkv), 256 threads. A Q block normalises (when a q_norm
 * weight is given), rotates and scales the G heads of its tokens into the Q
 * scratch. A fresh-slab block covers 32 positions of one KV head: old cache
 * rows are copied to the fresh buffers, new rows are normalised and rotated
 * (K), appended to the bf16 cache and written to the fresh buffers,
 * positions past the new rows are zero. Work is done in chunks of 8 elements
 * (16-byte stores); V goes through LDS so that the transposed stores are 8
 * consecutive positions of one column.
 *
 * Built per (head_dim, input type, RoPE pairing, norm) so that a thread's
 * chunks are a fixed, unrolled count whose loads are all issued before any
 * of them is used: one memory round trip per pass instead of one per chunk. */
/* Q rows of one block: token t, head g*G + hg -> scratch row q_row0 + t*G + hg */
template <int HD, bool BF, int RK, bool NORM>
__device__ __forceinline__ void prep_q(const PrepParams &p, const PrepBlock &blk, const PrepBatch &b, int g, int tid,
                                       float *sv) {
    constexpr int DT = BF ? SMOL_IN_BF16 : SMOL_IN_F32;
    constexpr int HDP = (HD + 31) & ~31;     /* Q-scratch row, zero-padded */
    constexpr int CPP = HDP / 8;
    using RC = RopeChunk<HD, BF, RK, NORM>;
    {
        const int G = p.G;
        const int per_tok = G * CPP;
        /* per-head RMSNorm: 1/rms of each of the block's count * G head rows
         * (the host keeps that within the LDS array) */
        float *s_qr = sv;
        if constexpr (NORM) {
            for (int r = tid >> 3; r < blk.count * G; r += 32) {
                const int tl = r / G, hg = r - tl * G;
                const long long row =
                    (long long)(b.q_tok0 + blk.first + tl) * p.q_stride + (long long)(g * G + hg) * HD;
                const float ri = head_rinv8(p.q, DT, row, HD, p.norm_eps, tid & 7);
                if ((tid & 7) == 0) s_qr[r] = ri;
            }
            __syncthreads();
        }
        /* passes of four 8-element chunks per thread (the loop bound is
         * block-uniform: every lane takes part in the partner shuffles) */
        const int total = blk.count * per_tok;
        for (int base = 0; base < total; base += 4 * 256) {
            RC in[4];
            float rinv[4];
            long long qi[4];
            int dd[4];
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const int e = base + tid + 256 * u;
                const int ee = e < total ? e : total - 1;
                const int tl = ee / per_tok, rem = ee - tl * per_tok;
                const int hg = rem / CPP, d0 = (rem - hg * CPP) * 8;
                const int t = blk.first + tl;
                dd[u] = d0;
                rinv[u] = NORM ? s_qr[tl * G + hg] : 1.0f;
                if (HDP == HD || d0 < HD) {
                    const long long row = (long long)(b.q_tok0 + t) * p.q_stride + (long long)(g * G + hg) * HD;
                    in[u].load(p.q, row, d0, p.rope_cos, p.rope_sin, b.q_pos0 + t, p.q_norm);
                }
                qi[u] = e < total ? (long long)g * p.qs_head_stride + (long long)(b.q_row0 + t * G + hg) * HDP + d0 : -1;
            }
#pragma unroll
            for (int u = 0; u < 4; u++) {
                float v[8];
                in[u].finish(v, dd[u], rinv[u]);
                if (HDP != HD && dd[u] >= HD) {
#pragma unroll
                    for (int i = 0; i < 8; i++) v[i] = 0.0f;
                }
                if (qi[u] < 0) continue;
#pragma unroll
                for (int i = 0; i < 8; i++) v[i] *= p.qscale;
                if (p.stage == SMOL_STAGE_QF32) {
                    *reinterpret_cast<float4 *>(p.qs32 + qi[u]) = make_float4(v[0], v[1], v[2], v[3]);
                    *reinterpret_cast<float4 *>(p.qs32 + qi[u] + 4) = make_float4(v[4], v[5], v[6], v[7]);
                } else if (p.qs_lo) {
                    note_h_range(p.range_flag, v);
                    uint4 hi, lo;
                    pack_h8_hilo(v, hi, lo);
                    *reinterpret_cast<uint4 *>(p.qs + qi[u]) = hi;
                    *reinterpret_cast<uint4 *>(p.qs_lo + qi[u]) = lo;
                } else {
                    note_h_range(p.range_flag, v);
                    *reinterpret_cast<uint4 *>(p.qs + qi[u]) = pack_h8(v);
                }
            }
        }
    }
}

/* One 32-position fresh slab of one KV head */
template <int HD, bool BF, int RK, bool NORM>
__device__ __forceinline__ void prep_fresh(const PrepParams &p, const PrepBlock &blk, const PrepBatch &b, int g,
                                           int tid, float *sv, float *s_kr) {
    constexpr int DT = BF ? SMOL_IN_BF16 : SMOL_IN_F32;
    constexpr int CPR = HD / 8;              /* 8-element chunks per head row */
    using RC = RopeChunk<HD, BF, RK, NORM>;
    const int pos_base = b.fresh_pos0 + blk.first * SMOL_SLAB;
    const int frow_base = b.fresh_row0 + blk.first * SMOL_SLAB;
    const bool has_cache = b.slot >= 0 && p.kc != nullptr;
    const long long cbase = has_cache ? (long long)b.slot * p.c_slot_stride + (long long)g * p.cap * HD : 0;
    uint16_t *kc = has_cache ? p.kc + cbase : nullptr;
    uint16_t *vtc = has_cache ? p.vtc + cbase : nullptr;
    _Float16 *kf = p.kf + (long long)g * p.fcap * HD;
    _Float16 *vtf = p.vtf + (long long)g * p.fcap * HD;
    const int new_lo = b.kv_pos0, new_hi = b.kv_pos0 + b.n_kv;
    /* blk.count: 0 the slab's K and V, 1 its K only, 2 its V only (two
     * blocks per slab double the workgroups that keep loads in flight) */
    const bool doK = blk.count != 2, doV = blk.count != 1;

    /* per-head RMSNorm of the new K rows: row r by lanes 8r .. 8r+7 */
    if (NORM && doK) {
        const int r = tid >> 3, pos = pos_base + r;
        if (pos >= new_lo && pos < new_hi) {
            const long long row = (long long)(b.kv_in0 + pos - new_lo) * p.kv_stride + (long long)g * HD;
            const float ri = head_rinv8(p.k, DT, row, HD, p.norm_eps, tid & 7);
            if ((tid & 7) == 0) s_kr[r] = ri;
        }
        __syncthreads();
    }

    /* K rows and the new V rows (into LDS): chunk e = (r, d0), NK per
     * thread. Loads only sit inside the row-kind branches; the values are
     * used after all of them are issued. */
    constexpr int NKC = SMOL_SLAB * CPR;
    constexpr int NK = (NKC + 255) / 256;
    RC kin[NK];
    Raw8<BF> vin[NK];
    uint4 kold[NK];
#pragma unroll
    for (int u = 0; u < NK; u++) {
        const int e = tid + 256 * u;
        const int r = e / CPR, d0 = (e - r * CPR) * 8;
        const int pos = pos_base + r;
        if (NKC % 256 != 0 && e >= NKC) continue;
        if (pos < new_lo) {
            if (has_cache && doK) kold[u] = *reinterpret_cast<const uint4 *>(kc + (long long)pos * HD + d0);
        } else if (pos < new_hi) {
            const long long row = (long long)(b.kv_in0 + pos - new_lo) * p.kv_stride + (long long)g * HD;
            if (doK) kin[u].load(p.k, row, d0, p.rope_cos, p.rope_sin, pos, p.k_norm);
            if (doV) raw_load<BF>(vin[u], p.v, row + d0);
        }
    }
#pragma unroll
    for (int u = 0; u < NK; u++) {
        const int e = tid + 256 * u;
        const int r = e / CPR, d0 = (e - r * CPR) * 8;
        const int pos = pos_base + r;
        const bool valid = NKC % 256 == 0 || e < NKC;
        const bool is_new = valid && pos >= new_lo && pos < new_hi;
        if (doK) {
            float kv[8];
            /* every lane computes the new-row values (the NeoX partner
             * shuffle needs all lanes); rows that are not new discard them */
            kin[u].finish(kv, d0, NORM && is_new ? s_kr[r] : 1.0f);
            if (valid) {
                if (!is_new) {
                    if (pos < new_lo && has_cache) unpack_bf16x8(kold[u], kv);
                    else {
#pragma unroll
                        for (int i = 0; i < 8; i++) kv[i] = 0.0f;
                    }
                }
                if (has_cache && is_new) *reinterpret_cast<uint4 *>(kc + (long long)pos * HD + d0) = pack_bf16x8(kv);
                note_h_range(p.range_flag, kv);
                if (p.kf_lo) {
                    uint4 hi, lo;
                    pack_h8_hilo(kv, hi, lo);
                    const long long fo = (long long)g * p.fcap * HD + (long long)(frow_base + r) * HD + d0;
                    *reinterpret_cast<uint4 *>(kf + (long long)(frow_base + r) * HD + d0) = hi;
                    *reinterpret_cast<uint4 *>(p.kf_lo + fo) = lo;
                } else {
                    *reinterpret_cast<uint4 *>(kf + (long long)(frow_base + r) * HD + d0) = pack_h8(kv);
                }
            }
        }
        if (doV) {
            float vv[8];
            raw_unpack<BF>(vin[u], vv);
            if (valid) {
                if (!is_new) {
#pragma unroll
                    for (int i = 0; i < 8; i++) vv[i] = 0.0f;
                }
#pragma unroll
                for (int i = 0; i < 8; i++) sv[r * 257 + d0 + i] = vv[i];
            }
        }
    }
    if (!doV) return;
    __syncthreads();
    /* V^T (slab-blocked, the slab's 32 positions of column d are contiguous):
     * chunk (d, 8 consecutive positions q0..q0+7) */
    uint16_t *vtc_blk = has_cache ? vtc + (long long)(pos_base / SMOL_SLAB) * SMOL_SLAB * HD : nullptr;
    _Float16 *vtf_blk = vtf + (long long)(frow_base / SMOL_SLAB) * SMOL_SLAB * HD;
    constexpr int NVC = HD * (SMOL_SLAB / 8);
    constexpr int NV = (NVC + 255) / 256;
    /* older cache rows of the slab: whole 16-byte chunks, all loads first */
    uint4 vold[NV];
#pragma unroll
    for (int u = 0; u < NV; u++) {
        const int e = tid + 256 * u;
        const int d = e / (SMOL_SLAB / 8), q0 = (e - d * (SMOL_SLAB / 8)) * 8;
        vold[u] = make_uint4(0, 0, 0, 0);
        if ((NVC % 256 == 0 || e < NVC) && has_cache && pos_base + q0 < new_lo)
            vold[u] = *reinterpret_cast<const uint4 *>(vtc_blk + d * SMOL_SLAB + q0);
    }
#pragma unroll
    for (int u = 0; u < NV; u++) {
        const int e = tid + 256 * u;
        if (NVC % 256 != 0 && e >= NVC) continue;
        const int d = e / (SMOL_SLAB / 8), q0 = (e - d * (SMOL_SLAB / 8)) * 8;
        const int pos = pos_base + q0;
        const int ci = d * SMOL_SLAB + q0;
        float v[8];
        unpack_bf16x8(vold[u], v);
        if (pos + 8 > new_lo) {
#pragma unroll
            for (int i = 0; i < 8; i++)
                if (pos + i >= new_lo) v[i] = sv[(q0 + i) * 257 + d];
            if (has_cache) {
                if (pos >= new_lo && pos + 8 <= new_hi) {
                    *reinterpret_cast<uint4 *>(vtc_blk + ci) = pack_bf16x8(v);
                } else {
                    for (int i = 0; i < 8; i++)
                        if (pos + i >= new_lo && pos + i < new_hi) vtc_blk[ci + i] = f32_to_bf16(v[i]);
                }
            }
        }
        note_h_range(p.range_flag, v);
        *reinterpret_cast<uint4 *>(vtf_blk + ci) = pack_h8(v);
    }
}

/* NORM builds normalise Q when q_norm is given and K when k_norm is given */
template <int HD, bool BF, int RK, bool NORM>
__global__ __launch_bounds__(256) void k_prep(PrepParams p) {
    /* block-uniform indices in scalar registers: the descriptors come through
     * scalar loads */
    const int bi = __builtin_amdgcn_readfirstlane((int)(blockIdx.x / (unsigned)p.Hkv));
    const int g = __builtin_amdgcn_readfirstlane((int)(blockIdx.x % (unsigned)p.Hkv)); /* kv head fastest: XCD-local */
    const PrepBlockB rec = p.blocks[bi];
    const PrepBlock &blk = rec.blk;
    const PrepBatch &b = rec.b;
    __shared__ float sv[SMOL_SLAB * 257];
    __shared__ float s_kr[SMOL_SLAB];
    if (blk.kind == 1) {
        if (NORM && p.q_norm) prep_q<HD, BF, RK, NORM>(p, blk, b, g, threadIdx.x, sv);
        else prep_q<HD, BF, RK, false>(p, blk, b, g, threadIdx.x, sv);
    } else {
        if (NORM && p.k_norm) prep_fresh<HD, BF, RK, NORM>(p, blk, b, g, threadIdx.x, sv, s_kr);
        else prep_fresh<HD, BF, RK, false>(p, blk, b, g, threadIdx.x, sv, s_kr);
    }
}

/* ------------------------------------------------------------- k_norm_rope */

/* In place on x [seq][H][hd] fp32: per-head RMSNorm with weight w [hd]
 * (skipped when w is null; rmsnorm.c:78-140), then RoPE (kind != OFF), row s
 * rotated at table row pos[s] (or s when pos is null). Eight lanes per head
 * row: the sum of squares reads the whole row before any lane writes (the
 * butterfly consumes every load), then lane j handles pairs j, j + 8, ... The rotation
 * is that of rope.c:99-164 (NeoX: fmsub / fmadd with the first-half table
 * entries over the 16-wide vector body, the scalar tail with the second-half
 * entries) and rope.c:68-93 (interleaved). */
__global__ __launch_bounds__(256) void k_norm_rope(float *x, const float *w, float eps, const float *cos_t,
                                                   const float *sin_t, const int *pos, int seq, int H, int hd,
                                                   int kind) {
    const int j = threadIdx.x & 7;
    const int half = hd >> 1;
    const long long rows = (long long)seq * H;
    const long long step = ((long long)gridDim.x * blockDim.x) >> 3;
    for (long long r = ((long long)blockIdx.x * blockDim.x + threadIdx.x) >> 3; r < rows; r += step) {
        float *v = x + r * hd;
        float ri = 1.0f;
        if (w) { /* any head_dim and alignment: element-strided sum of squares */
            float ss = 0.0f;
            for (int d = j; d < hd; d += 8) ss = fmaf(v[d], v[d], ss);
            ss += __shfl_xor(ss, 1, 8);
            ss += __shfl_xor(ss, 2, 8);
            ss += __shfl_xor(ss, 4, 8);
            ri = 1.0f / sqrtf(ss / (float)hd + eps);
        }
        auto nrm = [&](int d) { return w ? (v[d] * w[d]) * ri : v[d]; };
        if (kind == SMOL_ROPE_OFF) {
            for (int d = j; d < hd; d += 8) v[d] = nrm(d);
            continue;
        }
        const long long trow = (long long)(pos ? pos[r / H] : r / H) * hd;
        const float *c = cos_t + trow, *sn = sin_t + trow;
        if (kind == SMOL_ROPE_NEOX_K) {
            const int body = half - (half % 16);
            for (int i = j; i < half; i += 8) {
                const float x1 = nrm(i), x2 = nrm(half + i);
                if (i < body) {
                    v[i] = fmaf(x1, c[i], -(x2 * sn[i]));
                    v[half + i] = fmaf(x2, c[i], x1 * sn[i]);
                } else {
                    v[i] = x1 * c[i] + (-x2) * sn[i];
                    v[half + i] = x2 * c[half + i] + x1 * sn[half + i];
                }
            }
        } else {
            for (int i = j; i < half; i += 8) {
                const float x0 = nrm(2 * i), x1 = nrm(2 * i + 1);
                v[2 * i] = x0 * c[2 * i] - x1 * sn[2 * i];
                v[2 * i + 1] = x1 * c[2 * i + 1] + x0 * sn[2 * i + 1];
            }
        }
    }
}

/* ------------------------------------------------------- k_bf16_norm_rope */

/* Correctly rounded square root of a finite x >= 0: the hardware square
 * root is within one ulp, and the neighbour whose square brackets x is
 * chosen by the sign of the fused residuals x - s'*s (no float lies
 * between the residual threshold and the true midpoint, so the choice is
 * exact). Inputs below 2^-96 are scaled by 2^32 first, out of the range
 * where the hardware flushes. */
__device__ __forceinline__ float sqrt_rn(float x) {
    const bool tiny = x < 0x1.0p-96f;
    const float xs = tiny ? x * 0x1.0p+32f : x;
    float s = __builtin_amdgcn_sqrtf(xs);
    const float dn = __int_as_float(__float_as_int(s) - 1), up = __int_as_float(__float_as_int(s) + 1);
    const float vp = __fmaf_rn(-dn, s, xs), vs = __fmaf_rn(-up, s, xs);
    if (vp <= 0.0f) s = dn;
    if (vs > 0.0f) s = up;
    return tiny ? s * 0x1.0p-16f : s;
}

/* In place on x [seq][H][hd] bf16 (the bf16 decoder's Q or new K rows):
 * per-head RMSNorm with weight w (skipped when w is null), then the
 * interleaved rotation at table row pos0 + s (skipped when cos_t is null),
 * each result rounded to bf16 by truncation: bf16_rms_norm_per_head and
 * bf16_apply_rope_interleaved, common/decoder/qkn_bf16_decoder.c:73-91 and
 * :264-283. The operation order is fixed so that the bits are reproducible:
 *   ss = fma(v[d], v[d], ss) for d = 0, 1, ... (one thread per head row)
 *   r  = 1 / sqrt(ss / hd + eps), every step correctly rounded
 *   v' = trunc((v * r) * w[d])
 *   x0' = trunc(fma(x0, c, -(x1 * s))), x1' = trunc(fma(x1, c, x0 * s))
 * with c, s the table entries of column 2i. hd is a multiple of 8. */
/* rows [0, seq H) of x (weight w) and then rows [0, seq H2) of x2 (weight
 * w2; x2 NULL: none), one thread per head row */
__global__ __launch_bounds__(256) void k_bf16_norm_rope(uint16_t *x, const float *w, uint16_t *x2, const float *w2,
                                                        float eps, const float *cos_t, const float *sin_t, int pos0,
                                                        int seq, int H, int H2, int hd) {
    const long long rows1 = (long long)seq * H, rows = rows1 + (x2 ? (long long)seq * H2 : 0);
    const long long step = (long long)gridDim.x * blockDim.x;
    for (long long rr = (long long)blockIdx.x * blockDim.x + threadIdx.x; rr < rows; rr += step) {
        const bool second = rr >= rows1;
        const long long r = second ? rr - rows1 : rr;
        const int Hr = second ? H2 : H;
        const float *w_r = second ? w2 : w;
        uint4 *row = reinterpret_cast<uint4 *>((second ? x2 : x) + r * hd);
        const int n8 = hd >> 3;
        float ri = 1.0f;
        if (w_r) {
            float ss = 0.0f;
            for (int c8 = 0; c8 < n8; c8++) {
                float v[8];
                unpack_bf16x8(row[c8], v);
#pragma unroll
                for (int i = 0; i < 8; i++) ss = __fmaf_rn(v[i], v[i], ss);
            }
            ri = __fdiv_rn(1.0f, sqrt_rn(__fadd_rn(__fdiv_rn(ss, (float)hd), eps)));
        }
        const float *ct = cos_t ? cos_t + (long long)(pos0 + r / Hr) * hd : nullptr;
        const float *st = cos_t ? sin_t + (long long)(pos0 + r / Hr) * hd : nullptr;
        for (int c8 = 0; c8 < n8; c8++) {
            float v[8];
            unpack_bf16x8(row[c8], v);
            if (w_r) {
#pragma unroll
                for (int i = 0; i < 8; i++) v[i] = __uint_as_float(__float_as_uint(__fmul_rn(__fmul_rn(v[i], ri), w_r[c8 * 8 + i])) & 0xFFFF0000u);
            }
            if (ct) {
#pragma unroll
                for (int i = 0; i < 8; i += 2) {
                    const float c = ct[c8 * 8 + i], s = st[c8 * 8 + i];
                    const float x0 = v[i], x1 = v[i + 1];
                    v[i] = __fmaf_rn(x0, c, -__fmul_rn(x1, s));
                    v[i + 1] = __fmaf_rn(x1, c, __fmul_rn(x0, s));
                }
            }
            uint32_t o[4];
#pragma unroll
            for (int k = 0; k < 4; k++)
                o[k] = (__float_as_uint(v[2 * k]) >> 16) | (__float_as_uint(v[2 * k + 1]) & 0xFFFF0000u);
            row[c8] = make_uint4(o[0], o[1], o[2], o[3]);
        }
    }
}

/* The same operations for one position (a decode step: at most 256 head
 * rows): one workgroup first stages the rows (16-byte loads), both weight
 * vectors and the table row in LDS with coalesced loads (one round of loads
 * instead of a chain of dependent ones per thread), then one thread per row runs
 * k_bf16_norm_rope's operation order on the staged values, so the bits are
 * the same. LDS: the rows (bf16), then w, w2, cos and sin (hd floats each). */
__global__ __launch_bounds__(256) void k_bf16_norm_rope1(uint16_t *x, const float *w, uint16_t *x2, const float *w2,
                                                         float eps, const float *cos_t, const float *sin_t, int pos,
                                                         int H, int H2, int hd) {
    extern __shared__ __attribute__((aligned(16))) unsigned char lds_nr[];
    const int tid = threadIdx.x;
    const int rows1 = H, rows = H + (x2 ? H2 : 0);
    const int c1 = rows1 * hd / 8, ch = rows * hd / 8; /* 16-byte chunks of the rows */
    uint4 *s_rows = reinterpret_cast<uint4 *>(lds_nr);
    float *s_w = reinterpret_cast<float *>(lds_nr + (size_t)rows * hd * 2);
    float *s_w2 = s_w + hd, *s_c = s_w2 + hd, *s_s = s_c + hd;
    for (int e = tid; e < ch; e += blockDim.x)
        s_rows[e] = e < c1 ? reinterpret_cast<const uint4 *>(x)[e] : reinterpret_cast<const uint4 *>(x2)[e - c1];
    for (int e = tid; e < hd; e += blockDim.x) {
        s_w[e] = w ? w[e] : 1.0f;
        s_w2[e] = w2 ? w2[e] : 1.0f;
        if (cos_t) {
            s_c[e] = cos_t[(long long)pos * hd + e];
            s_s[e] = sin_t[(long long)pos * hd + e];
        }
    }
    __syncthreads();
    if (tid >= rows) return;
    const bool second = tid >= rows1;
    const bool norm = second ? w2 != nullptr : w != nullptr;
    const float *w_r = second ? s_w2 : s_w;
    const int n8 = hd >> 3;
    const uint4 *src = s_rows + (size_t)tid * n8;
    uint4 *row = reinterpret_cast<uint4 *>(second ? x2 + (size_t)(tid - rows1) * hd : x + (size_t)tid * hd);
    float ri = 1.0f;
    if (norm) {
        float ss = 0.0f;
        for (int c8 = 0; c8 < n8; c8++) {
            float v[8];
            unpack_bf16x8(src[c8], v);
#pragma unroll
            for (int i = 0; i < 8; i++) ss = __fmaf_rn(v[i], v[i], ss);
        }
        ri = __fdiv_rn(1.0f, sqrt_rn(__fadd_rn(__fdiv_rn(ss, (float)hd), eps)));
    }
    for (int c8 = 0; c8 < n8; c8++) {
        float v[8];
        unpack_bf16x8(src[c8], v);
        if (norm) {
#pragma unroll
            for (int i = 0; i < 8; i++) v[i] = __uint_as_float(__float_as_uint(__fmul_rn(__fmul_rn(v[i], ri), w_r[c8 * 8 + i])) & 0xFFFF0000u);
        }
        if (cos_t) {
#pragma unroll
            for (int i = 0; i < 8; i += 2) {
                const float c = s_c[c8 * 8 + i], sn = s_s[c8 * 8 + i];
                const float x0 = v[i], x1 = v[i + 1];
                v[i] = __fmaf_rn(x0, c, -__fmul_rn(x1, sn));
                v[i + 1] = __fmaf_rn(x1, c, __fmul_rn(x0, sn));
            }
        }
        uint32_t o[4];
#pragma unroll
        for (int k = 0; k < 4; k++)
            o[k] = (__float_as_uint(v[2 * k]) >> 16) | (__float_as_uint(v[2 * k + 1]) & 0xFFFF0000u);
        row[c8] = make_uint4(o[0], o[1], o[2], o[3]);
    }
}

/* x2 / w2 / H2: a second tensor at the same positions (NULL: none), the K
 * rows of the call that normalises and rotates its Q rows in x */
extern "C" int smol_launch_bf16_norm_rope(uint16_t *x, const float *w, uint16_t *x2, const float *w2, int H2,
                                          float eps, const float *cos_t, const float *sin_t, int pos0, int seq, int H,
                                          int hd, hipStream_t st) {
    const long long rows = (long long)seq * H + (x2 ? (long long)seq * H2 : 0);
    if (rows <= 0) return 0;
    const size_t lds1 = (size_t)rows * hd * 2 + 4 * (size_t)hd * 4;
    if (seq == 1 && rows <= 256 && lds1 <= 64 * 1024) {
        hipLaunchKernelGGL(k_bf16_norm_rope1, dim3(1), dim3(256), lds1, st, x, w, x2, w2, eps, cos_t, sin_t, pos0, H,
                           x2 ? H2 : 0, hd);
        return hipGetLastError() == hipSuccess ? 0 : -3;
    }
    const int blocks = (int)std::min<long long>((rows + 255) / 256, 4096);
    hipLaunchKernelGGL(k_bf16_norm_rope, dim3(blocks), dim3(256), 0, st, x, w, x2, w2, eps, cos_t, sin_t, pos0, seq,
                       H, H2, hd);
    return hipGetLastError() == hipSuccess ? 0 : -3;
}

/* ------------------------------------------------------------ k_to_bf16 */

/* y = the upper 16 bits of x (bf16 by truncation, the f32_to_bf16 of
 * common/decoder/qkn_bf16_decoder.c:30-35), 8 elements per thread */
__global__ __launch_bounds__(256) void k_to_bf16_trunc(const float *x, uint16_t *y, long long n) {
    const long long i0 = ((long long)blockIdx.x * blockDim.x + threadIdx.x) * 8;
    if (i0 + 8 <= n) {
        const float4 a = *reinterpret_cast<const float4 *>(x + i0), b = *reinterpret_cast<const float4 *>(x + i0 + 4);
        const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
        uint32_t w[4];
#pragma unroll
        for (int k = 0; k < 4; k++) w[k] = (__float_as_uint(v[2 * k]) >> 16) | (__float_as_uint(v[2 * k + 1]) & 0xFFFF0000u);
        *reinterpret_cast<uint4 *>(y + i0) = make_uint4(w[0], w[1], w[2], w[3]);
    } else {
        for (long long i = i0; i < n; i++) y[i] = (uint16_t)(__float_as_uint(x[i]) >> 16);
    }
}

/* ------------------------------------------------------------ launchers */

extern "C" int smol_launch_to_bf16_trunc(const float *x, uint16_t *y, long long n, hipStream_t st) {
    if (n <= 0) return 0;
    const long long threads = (n + 7) / 8;
    hipLaunchKernelGGL(k_to_bf16_trunc, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, st, x, y, n);
    return hipGetLastError() == hipSuccess ? 0 : -3;
}

extern "C" int smol_launch_norm_rope(float *x, const float *w, float eps, const float *cos_t, const float *sin_t,
                                     const int *pos, int seq, int n_heads, int hd, int kind, hipStream_t st) {
    const long long rows = (long long)seq * n_heads;
    if (rows <= 0) return 0;
    const int blocks = (int)std::min<long long>((rows + 31) / 32, 4096);
    hipLaunchKernelGGL(k_norm_rope, dim3(blocks), dim3(256), 0, st, x, w, eps, cos_t, sin_t, pos, seq, n_heads, hd,
                       kind);
    return hipGetLastError() == hipSuccess ? 0 : -3;
}

template <int HD>
static int launch_prep_hd(const PrepParams *pp, dim3 grid, hipStream_t st, hipEvent_t e0, hipEvent_t e1) {
    /* Q and the new K are rotated together or not at all (the host sets both flags from one table) */
    const int rk = (pp->rope_q && pp->rope_k) ? pp->rope_kind : SMOL_ROPE_OFF;
    /* one input type for Q and the new K/V (the host passes one dtype per call) */
    const bool bf = pp->kv_dtype == SMOL_IN_BF16;
    if (pp->kv_dtype != pp->q_dtype || pp->rope_q != pp->rope_k) return -1;
#define SMOL_PREP(BF, RK)                                                                        \
    do {                                                                                         \
        if (pp->q_norm || pp->k_norm)                                                            \
            hipExtLaunchKernelGGL((k_prep<HD, BF, RK, true>), grid, dim3(256), 0, st, e0, e1, 0, *pp); \
        else hipExtLaunchKernelGGL((k_prep<HD, BF, RK, false>), grid, dim3(256), 0, st, e0, e1, 0, *pp); \
    } while (0)
    if (rk == SMOL_ROPE_OFF) { if (bf) SMOL_PREP(true, SMOL_ROPE_OFF); else SMOL_PREP(false, SMOL_ROPE_OFF); }
    else if (rk == SMOL_ROPE_NEOX_K) { if (bf) SMOL_PREP(true, SMOL_ROPE_NEOX_K); else SMOL_PREP(false, SMOL_ROPE_NEOX_K); }
    else if (rk == SMOL_ROPE_INTERLEAVED_K) {
        if (bf) SMOL_PREP(true, SMOL_ROPE_INTERLEAVED_K); else SMOL_PREP(false, SMOL_ROPE_INTERLEAVED_K);
    } else return -1;
#undef SMOL_PREP
    return hipGetLastError() == hipSuccess ? 0 : -3;
}

/* e0 / e1 (may be null): events recorded around the kernel alone */
extern "C" int smol_launch_prep(const PrepParams *pp, int n_blocks, hipStream_t st, hipEvent_t e0, hipEvent_t e1) {
    if (n_blocks <= 0) return 0;
    const dim3 grid(n_blocks * pp->Hkv);
    switch (pp->hd) {
    case 64: return launch_prep_hd<64>(pp, grid, st, e0, e1);
    case 72: return launch_prep_hd<72>(pp, grid, st, e0, e1);
    case 80: return launch_prep_hd<80>(pp, grid, st, e0, e1);
    case 96: return launch_prep_hd<96>(pp, grid, st, e0, e1);
    case 128: return launch_prep_hd<128>(pp, grid, st, e0, e1);
    case 256: return launch_prep_hd<256>(pp, grid, st, e0, e1);
    default: return -1;
    }
}

