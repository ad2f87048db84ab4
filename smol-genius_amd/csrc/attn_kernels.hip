/*
 * attn_kernels.hip - gfx950 (CDNA4) kernels of the attention path.
 *
 *   k_prep      per-head RMSNorm + RoPE + cache append + fp16 staging, one
 *               pass over the new rows: replaces smol_rms_norm_per_head and
 *               smol_apply_rope_{neox,interleaved} on Q and K and the K/V row
 *               memcpy into the cache (common/decoder/qkn_decoder.c:487-503
 *               and :640-652).
 *   k_norm_rope per-head RMSNorm and / or RoPE in place on an fp32 array.
 *   k_attn_fb   prefill / bidirectional attention whose keys are all new:
 *               fp16 MFMA (v_mfma_f32_16x16x32_f16), one workgroup per
 *               64-row tile, K/V staged into LDS by direct transfers;
 *   k_attn_fa   prefill over an existing cache prefix (and head_dim 256):
 *               the same LDS image, key ranges split across workgroups;
 *   k_attn_dec  decode and short chunks: bf16 MFMA straight on the bf16 cache
 *               with hi/lo-split Q and P;
 *               all compute the causal / sliding-window / softcap /
 *               windowed-bidirectional online softmax of
 *               common/kernels/attention.c:32-462 over the bf16 KV cache plus
 *               the call's fresh fp16 keys; split key ranges end in a
 *               log-sum-exp merge by the group's last workgroup.
 *
 * Numerics: softmax state in fp32 and in log2 units (Q is pre-multiplied by
 * scale * log2 e, so exp(s - m) = exp2(s' - m')). MFMA operands are fp16:
 * bf16 -> fp16 is exact for |x| < 65504, and fp16 keeps 3 more mantissa bits
 * than bf16 for the rotated Q/K and the probabilities P, which is what keeps
 * the result within 2e-3 + 1e-2 |ref| of the fp32 reference on early causal
 * rows (bf16 operands do not).
 */
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "attn_internal.h"

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));

#define LOG2E_F 1.4426950408889634f

/* ------------------------------------------------------------------ helpers */

__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
    return __uint_as_float((uint32_t)b << 16);
}

/* float -> bf16 bits, round to nearest even (inputs are finite) */
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
    uint32_t u = __float_as_uint(f);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

__device__ __forceinline__ h8 bf16x8_to_h8(uint4 w) {
    h8 r;
    const uint32_t a[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
        r[2 * i] = (_Float16)__uint_as_float(a[i] << 16);
        r[2 * i + 1] = (_Float16)__uint_as_float(a[i] & 0xFFFF0000u);
    }
    return r;
}

__device__ __forceinline__ h8 load_h8(const _Float16 *p) {
    uint4 w = *reinterpret_cast<const uint4 *>(p);
    return *reinterpret_cast<h8 *>(&w);
}

__device__ __forceinline__ h8 load_bf16x8(const uint16_t *p) {
    return bf16x8_to_h8(*reinterpret_cast<const uint4 *>(p));
}

__device__ __forceinline__ h8 zero_h8() {
    h8 z;
#pragma unroll
    for (int i = 0; i < 8; i++) z[i] = (_Float16)0.0f;
    return z;
}

__device__ __forceinline__ float load_in(const void *base, int dtype, long long idx) {
    return dtype == SMOL_IN_BF16 ? bf16_to_f32(((const uint16_t *)base)[idx])
                                 : ((const float *)base)[idx];
}

__device__ __forceinline__ int rope_partner(int d, int hd, int kind) {
    if (kind == SMOL_ROPE_NEOX_K) { int half = hd >> 1; return d < half ? d + half : d - half; }
    if (kind == SMOL_ROPE_INTERLEAVED_K) return d ^ 1;
    return d;
}

/* ------------------------------------------------------------------ k_prep */

/* 8 consecutive input elements (fp32 or bf16) as fp32; idx is a multiple of 8 */
__device__ __forceinline__ void load8(const void *base, int dtype, long long idx, float *v) {
    if (dtype == SMOL_IN_BF16) {
        const uint4 w = *reinterpret_cast<const uint4 *>((const uint16_t *)base + idx);
        const uint32_t a[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            v[2 * i] = __uint_as_float(a[i] << 16);
            v[2 * i + 1] = __uint_as_float(a[i] & 0xFFFF0000u);
        }
    } else {
        const float4 x = *reinterpret_cast<const float4 *>((const float *)base + idx);
        const float4 y = *reinterpret_cast<const float4 *>((const float *)base + idx + 4);
        v[0] = x.x; v[1] = x.y; v[2] = x.z; v[3] = x.w;
        v[4] = y.x; v[5] = y.y; v[6] = y.z; v[7] = y.w;
    }
}

__device__ __forceinline__ uint4 pack_bf16x8(const float *v) {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; i++) w[i] = (uint32_t)f32_to_bf16(v[2 * i]) | ((uint32_t)f32_to_bf16(v[2 * i + 1]) << 16);
    return make_uint4(w[0], w[1], w[2], w[3]);
}

__device__ __forceinline__ uint4 pack_h8(const float *v) {
    h8 h;
#pragma unroll
    for (int i = 0; i < 8; i++) h[i] = (_Float16)v[i];
    return *reinterpret_cast<uint4 *>(&h);
}

__device__ __forceinline__ void unpack_bf16x8(uint4 w, float *v) {
    const uint32_t a[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
        v[2 * i] = __uint_as_float(a[i] << 16);
        v[2 * i + 1] = __uint_as_float(a[i] & 0xFFFF0000u);
    }
}

/* 8 consecutive fp32 table entries (16-byte aligned: d0 % 8 == 0) */
__device__ __forceinline__ void tab8(const float *t, float *v) {
    const float4 a = *reinterpret_cast<const float4 *>(t), b = *reinterpret_cast<const float4 *>(t + 4);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}

/* 1 / sqrt(mean(x^2) + eps) of the head row at `base + row` (hd elements,
 * fp32 or bf16), computed by the 8 lanes of an aligned lane group (j = lane
 * & 7): lane j sums the squares of chunks j, j + 8, ... in order, then a
 * butterfly over the 8 lanes, so every lane returns the same value. This is
 * rmsnorm.c:78-113 with another summation order. All 8 lanes must call it. */
__device__ __forceinline__ float head_rinv8(const void *base, int dtype, long long row, int hd, float eps, int j) {
    float ss = 0.0f;
    for (int d0 = j * 8; d0 < hd; d0 += 64) {
        float v[8];
        load8(base, dtype, row + d0, v);
#pragma unroll
        for (int i = 0; i < 8; i++) ss = fmaf(v[i], v[i], ss);
    }
    ss += __shfl_xor(ss, 1, 8);
    ss += __shfl_xor(ss, 2, 8);
    ss += __shfl_xor(ss, 4, 8);
    return 1.0f / sqrtf(ss / (float)hd + eps);
}

/* Rotates the 8 elements [d0, d0+8) of a head vector whose row starts at
 * `base + row` (fp32 or bf16 input), position `pos` of the table. With a
 * norm weight `nw`, each element (and each rotation partner) is first
 * normalised as (x * nw[d]) * rinv, the order of rmsnorm.c:119-121. */
__device__ __forceinline__ void rope8(const void *base, int dtype, long long row, int d0, int hd, int kind,
                                      const float *cos_t, const float *sin_t, long long pos, float *out,
                                      const float *nw = nullptr, float rinv = 1.0f) {
    load8(base, dtype, row + d0, out);
    if (nw) {
#pragma unroll
        for (int i = 0; i < 8; i++) out[i] = (out[i] * nw[d0 + i]) * rinv;
    }
    if (kind == SMOL_ROPE_OFF) return;
    const float *c = cos_t + pos * hd, *s = sin_t + pos * hd;
    float cv[8], sv[8];
    tab8(c + d0, cv);
    tab8(s + d0, sv);
    if (kind == SMOL_ROPE_INTERLEAVED_K) {
#pragma unroll
        for (int i = 0; i < 8; i += 2) {
            const float x0 = out[i], x1 = out[i + 1];
            out[i] = x0 * cv[i] - x1 * sv[i];
            out[i + 1] = x1 * cv[i + 1] + x0 * sv[i + 1];
        }
        return;
    }
    const int half = hd >> 1;
    float pr[8];
    if ((half & 7) == 0) {
        const int p0 = d0 < half ? d0 + half : d0 - half;
        load8(base, dtype, row + p0, pr);
        if (nw) {
#pragma unroll
            for (int i = 0; i < 8; i++) pr[i] = (pr[i] * nw[p0 + i]) * rinv;
        }
    } else {
        /* half not a multiple of 8 (head_dim 72): partners element by element */
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int pd = rope_partner(d0 + i, hd, kind);
            pr[i] = load_in(base, dtype, row + pd);
            if (nw) pr[i] = (pr[i] * nw[pd]) * rinv;
        }
    }
    /* NeoX: x1 c - x2 s for the first half, x2 c + x1 s for the second
     * (rope.c:99-164, fmsub / fmadd) */
#pragma unroll
    for (int i = 0; i < 8; i++)
        out[i] = d0 + i < half ? fmaf(out[i], cv[i], -(pr[i] * sv[i])) : fmaf(out[i], cv[i], pr[i] * sv[i]);
}

/* Raw bits of 8 consecutive input elements (bf16: one 16-byte load, fp32:
 * two), held without use so that a thread's loads can all be in flight. */
template <bool BF> struct Raw8 { uint4 a[BF ? 1 : 2]; };

template <bool BF>
__device__ __forceinline__ void raw_load(Raw8<BF> &r, const void *base, long long idx) {
    if constexpr (BF) {
        r.a[0] = *reinterpret_cast<const uint4 *>((const uint16_t *)base + idx);
    } else {
        r.a[0] = *reinterpret_cast<const uint4 *>((const float *)base + idx);
        r.a[1] = *reinterpret_cast<const uint4 *>((const float *)base + idx + 4);
    }
}

template <bool BF>
__device__ __forceinline__ void raw_unpack(const Raw8<BF> &r, float *v) {
    if constexpr (BF) {
        unpack_bf16x8(r.a[0], v);
    } else {
        v[0] = __uint_as_float(r.a[0].x); v[1] = __uint_as_float(r.a[0].y);
        v[2] = __uint_as_float(r.a[0].z); v[3] = __uint_as_float(r.a[0].w);
        v[4] = __uint_as_float(r.a[1].x); v[5] = __uint_as_float(r.a[1].y);
        v[6] = __uint_as_float(r.a[1].z); v[7] = __uint_as_float(r.a[1].w);
    }
}

/* Operands of the normalised rotation of one 8-element chunk [d0, d0+8) of
 * a head row: load() only issues loads, finish() turns them into the
 * rotated values. NeoX partners (d0 +- hd/2) come from another lane by
 * __shfl_xor when head_dim is 64, 128 or 256 (a row's chunks are then an
 * aligned power-of-two group of consecutive lanes), otherwise from memory
 * (whole chunks when hd/2 is a multiple of 8, element by element for hd 72).
 * With a norm weight each element becomes (x * w[d]) * rinv
 * (rmsnorm.c:119-121), then the rotation of rope.c:99-164 (NeoX) or
 * rope.c:68-93 (interleaved) is applied. */
template <int HD, bool BF, int RK, bool NORM>
struct RopeChunk {
    static constexpr int HALF = HD / 2;
    static constexpr bool NEOX = RK == SMOL_ROPE_NEOX_K;
    static constexpr bool SHFL = NEOX && (HD == 64 || HD == 128 || HD == 256);
    static constexpr bool PCHUNK = NEOX && !SHFL && HALF % 8 == 0;
    static constexpr bool PELEM = NEOX && !SHFL && HALF % 8 != 0;
    Raw8<BF> x, p;
    uint32_t pe[8];
    float4 c0, c1, s0, s1, w0, w1, wp0, wp1;
    float wpe[8];

    __device__ __forceinline__ void load(const void *base, long long row, int d0, const float *cos_t,
                                         const float *sin_t, long long pos, const float *nw) {
        raw_load<BF>(x, base, row + d0);
        const int p0 = d0 < HALF ? d0 + HALF : d0 - HALF;
        if constexpr (PCHUNK) raw_load<BF>(p, base, row + p0);
        if constexpr (PELEM) {
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const int pd = rope_partner(d0 + i, HD, RK);
                pe[i] = BF ? (uint32_t)((const uint16_t *)base)[row + pd] << 16
                           : __float_as_uint(((const float *)base)[row + pd]);
                if constexpr (NORM) wpe[i] = nw[pd];
            }
        }
        if constexpr (RK != SMOL_ROPE_OFF) {
            /* the tables repeat the first half of a NeoX row in the second:
             * chunks of the second half read the first, so only half of each
             * row's cache lines are fetched */
            const int dc = (SHFL || PCHUNK) && d0 >= HALF ? d0 - HALF : d0;
            const float *c = cos_t + pos * HD + dc, *s = sin_t + pos * HD + dc;
            c0 = *reinterpret_cast<const float4 *>(c); c1 = *reinterpret_cast<const float4 *>(c + 4);
            s0 = *reinterpret_cast<const float4 *>(s); s1 = *reinterpret_cast<const float4 *>(s + 4);
        }
        if constexpr (NORM) {
            w0 = make_float4(nw[d0], nw[d0 + 1], nw[d0 + 2], nw[d0 + 3]);
            w1 = make_float4(nw[d0 + 4], nw[d0 + 5], nw[d0 + 6], nw[d0 + 7]);
            if constexpr (PCHUNK) {
                wp0 = make_float4(nw[p0], nw[p0 + 1], nw[p0 + 2], nw[p0 + 3]);
                wp1 = make_float4(nw[p0 + 4], nw[p0 + 5], nw[p0 + 6], nw[p0 + 7]);
            }
        }
    }

    /* out = the normalised, rotated chunk; every lane of the wave must call
     * this together when SHFL (the partner exchange is a lane shuffle) */
    __device__ __forceinline__ void finish(float *out, int d0, float rinv) const {
        raw_unpack<BF>(x, out);
        if constexpr (NORM) {
            const float w[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
            for (int i = 0; i < 8; i++) out[i] = (out[i] * w[i]) * rinv;
        }
        if constexpr (RK == SMOL_ROPE_OFF) return;
        const float cv[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
        const float sv[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
        if constexpr (RK == SMOL_ROPE_INTERLEAVED_K) {
#pragma unroll
            for (int i = 0; i < 8; i += 2) {
                const float x0 = out[i], x1 = out[i + 1];
                out[i] = x0 * cv[i] - x1 * sv[i];
                out[i + 1] = x1 * cv[i + 1] + x0 * sv[i + 1];
            }
            return;
        } else {
            float pr[8];
            if constexpr (SHFL) {
#pragma unroll
                for (int i = 0; i < 8; i++) pr[i] = __shfl_xor(out[i], HALF / 8);
            } else if constexpr (PCHUNK) {
                raw_unpack<BF>(p, pr);
                if constexpr (NORM) {
                    const float w[8] = {wp0.x, wp0.y, wp0.z, wp0.w, wp1.x, wp1.y, wp1.z, wp1.w};
#pragma unroll
                    for (int i = 0; i < 8; i++) pr[i] = (pr[i] * w[i]) * rinv;
                }
            } else {
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    pr[i] = __uint_as_float(pe[i]);
                    if constexpr (NORM) pr[i] = (pr[i] * wpe[i]) * rinv;
                }
            }
            /* NeoX: x1 c - x2 s for the first half, x2 c + x1 s for the
             * second (rope.c:99-164, fmsub / fmadd) */
#pragma unroll
            for (int i = 0; i < 8; i++)
                out[i] = d0 + i < HALF ? fmaf(out[i], cv[i], -(pr[i] * sv[i])) : fmaf(out[i], cv[i], pr[i] * sv[i]);
        }
    }
};

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
                } else {
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

    /* per-head RMSNorm of the new K rows: row r by lanes 8r .. 8r+7 */
    if constexpr (NORM) {
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
            if (has_cache) kold[u] = *reinterpret_cast<const uint4 *>(kc + (long long)pos * HD + d0);
        } else if (pos < new_hi) {
            const long long row = (long long)(b.kv_in0 + pos - new_lo) * p.kv_stride + (long long)g * HD;
            kin[u].load(p.k, row, d0, p.rope_cos, p.rope_sin, pos, p.k_norm);
            raw_load<BF>(vin[u], p.v, row + d0);
        }
    }
#pragma unroll
    for (int u = 0; u < NK; u++) {
        const int e = tid + 256 * u;
        const int r = e / CPR, d0 = (e - r * CPR) * 8;
        const int pos = pos_base + r;
        const bool valid = NKC % 256 == 0 || e < NKC;
        const bool is_new = valid && pos >= new_lo && pos < new_hi;
        float kv[8], vv[8];
        /* every lane computes the new-row values (the NeoX partner shuffle
         * needs all lanes); rows that are not new discard them */
        kin[u].finish(kv, d0, NORM && is_new ? s_kr[r] : 1.0f);
        raw_unpack<BF>(vin[u], vv);
        if (!valid) continue;
        if (!is_new) {
#pragma unroll
            for (int i = 0; i < 8; i++) vv[i] = 0.0f;
            if (pos < new_lo && has_cache) unpack_bf16x8(kold[u], kv);
            else {
#pragma unroll
                for (int i = 0; i < 8; i++) kv[i] = 0.0f;
            }
        }
        if (has_cache && is_new) *reinterpret_cast<uint4 *>(kc + (long long)pos * HD + d0) = pack_bf16x8(kv);
        *reinterpret_cast<uint4 *>(kf + (long long)(frow_base + r) * HD + d0) = pack_h8(kv);
#pragma unroll
        for (int i = 0; i < 8; i++) sv[r * 257 + d0 + i] = vv[i];
    }
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

/* --------------------------------------------------------- shared by kernels */

/* Raw buffer resources: a base address plus a byte range; a load whose
 * VGPR offset (+ immediate) is past the range returns zero, which is how the
 * padded columns of head_dim 72 / 80 / 96 read as zeros. */
typedef __amdgpu_buffer_rsrc_t rsrc_t;
typedef unsigned u4v __attribute__((ext_vector_type(4)));
#define RSRC_WORD3 0x00020000
#define OOB_OFF 0x7FFFFFF0u

__device__ __forceinline__ rsrc_t make_rsrc(const void *ptr, long long bytes) {
    const long long n = bytes < 0x7FFF0000LL ? bytes : 0x7FFF0000LL;
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(ptr), (short)0, (int)n, RSRC_WORD3);
}

__device__ __forceinline__ uint4 bload(rsrc_t r, unsigned voff, unsigned soff) {
    const u4v v = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
    return make_uint4(v[0], v[1], v[2], v[3]);
}

/* Device-coherent (SC1) buffer accesses for the split-K partials. The L2s
 * of the XCDs are not coherent with each other; SC1 stores write through to
 * the device coherence point and SC1 loads read from it, so partials pass
 * between workgroups on different XCDs without an L2 write-back or
 * invalidate (what an agent-scope release / acquire fence would cost). */
#define CPOL_SC1 16
__device__ __forceinline__ void store_f4_sc1(rsrc_t r, unsigned voff, f4 v) {
    __builtin_amdgcn_raw_buffer_store_b128(u4v{__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]),
                                               __float_as_uint(v[3])},
                                           r, voff, 0, CPOL_SC1);
}
__device__ __forceinline__ f4 load_f4_sc1(rsrc_t r, unsigned voff) {
    const u4v v = __builtin_amdgcn_raw_buffer_load_b128(r, voff, 0, CPOL_SC1);
    return f4{__uint_as_float(v[0]), __uint_as_float(v[1]), __uint_as_float(v[2]), __uint_as_float(v[3])};
}
__device__ __forceinline__ void store_f2_sc1(rsrc_t r, unsigned voff, float a, float b) {
    typedef unsigned u2v __attribute__((ext_vector_type(2)));
    __builtin_amdgcn_raw_buffer_store_b64(u2v{__float_as_uint(a), __float_as_uint(b)}, r, voff, 0, CPOL_SC1);
}
__device__ __forceinline__ float2 load_f2_sc1(rsrc_t r, unsigned voff) {
    typedef unsigned u2v __attribute__((ext_vector_type(2)));
    const u2v v = __builtin_amdgcn_raw_buffer_load_b64(r, voff, 0, CPOL_SC1);
    return make_float2(__uint_as_float(v[0]), __uint_as_float(v[1]));
}

/* One 1 KB direct-to-LDS transfer: lane l's 16 bytes land at lds + 16 l.
 * The LDS address travels in M0. GFX9-family parts (gfx950 included) need
 * one wait state between an SALU write of M0 and an LDS-DMA load that reads
 * it; without the s_nop the load can take the previous transfer's M0 and
 * land in the previous 1 KB region, leaving its own region stale. The
 * compiler inserts that nop for LDS-DMA it emits itself but cannot see into
 * inline asm. M0 is a reserved register to the compiler, so listing it below
 * only documents the write: the kernels of this file contain no other M0
 * writer or reader (tests/test_abi.py disassembles the built code object and
 * checks that every M0 write is this sequence). The compiler's own LDS-DMA
 * builtin is not used because its wait insertion drains every transfer
 * (vmcnt(0)) before any LDS read, which would serialise the staging ring. */
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma_1k(rsrc_t r, unsigned voff, unsigned soff, unsigned lds) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds" ::"s"(lds), "v"(voff),
                 "s"(r), "s"(soff)
                 : "memory", "m0");
}
#pragma clang diagnostic pop

#define SK_WAVES 4

/* Reductions over the four lanes c, c+16, c+32, c+48 that hold one softmax
 * row, with the gfx950 cross-row swaps (VALU, no LDS round trip). Each swap
 * hands every lane the pair {x[l], x[l ^ 32]} (resp. l ^ 16), so all four
 * lanes end with the same value. */
__device__ __forceinline__ float row_max4(float v) {
    const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

__device__ __forceinline__ float row_sum4(float v) {
    const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

/* Merge of one split-K group by its last workgroup (all 64*SK_WAVES threads).
 * Only the batch's real rows are read and written. Every thread owns E
 * (row, 4-column) elements, taken EB at a time, and walks the splits U at a
 * time with all EB * U loads in flight (MAXL at most), so the merge costs
 * about (E / EB) * n_split / U memory round trips; when one round covers
 * everything (decode), those loads are issued before the group's (max, sum)
 * pairs are even read, and the two sweeps share one round trip. Each row's
 * max and 1/sum and every split's weight are formed in LDS. The host keeps
 * ROWS * n_split within SK_MERGE_MAX. Resets the group's counter for the
 * next call. */
template <int HD, int ROWS, int MAXL = 16, int TPB = 64 * SK_WAVES>
__device__ __forceinline__ void merge_group(const SkParams &p, const SkItem &it, const SkBatch &b, int item, int g,
                                            int tid, float *s_o) {
    const int G = p.G, Hq = p.Hq;
    const int first = item - it.split;
    const int nsp = it.n_split;
    const int n_valid = min(ROWS, b.n_rows - it.row0);
    float *s_ml = s_o;                       /* [nsp][ROWS][2], then weights [nsp][ROWS] */
    float *s_row = s_o + 2 * SK_MERGE_MAX;   /* per row: max, 1/sum */
    /* the group's items are contiguous: item `first + sp` holds split sp */
    const rsrc_t rml = make_rsrc(p.part_ml + (long long)first * p.Hkv * ROWS * 2, (long long)nsp * p.Hkv * ROWS * 2 * 4);
    const rsrc_t ro = make_rsrc(p.part_o + (long long)first * p.Hkv * ROWS * HD, (long long)nsp * p.Hkv * ROWS * HD * 4);
    constexpr int C4 = HD / 4;
    constexpr int E = (ROWS * C4 + TPB - 1) / (TPB);
    constexpr int EB = E < 8 ? E : 8;
    constexpr int U = MAXL / EB > 16 ? 16 : (MAXL / EB < 1 ? 1 : MAXL / EB);
    const int nel = n_valid * C4;
    const unsigned sp_stride = (unsigned)((long long)p.Hkv * ROWS * HD * 4);
    auto setup = [&](int e0, int (&prow)[EB], int (&pcol)[EB]) __attribute__((always_inline)) {
#pragma unroll
        for (int e = 0; e < EB; e++) {
            const int idx = tid + TPB * (e0 + e);
            const int rr = idx / C4;
            prow[e] = (e0 + e < E && idx < nel) ? rr : -1;
            pcol[e] = (idx - rr * C4) * 4;
        }
    };
    auto issue = [&](int sp0, const int (&prow)[EB], const int (&pcol)[EB], f4 (&v)[U][EB]) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < U; u++) {
            const unsigned so = (unsigned)min(sp0 + u, nsp - 1) * sp_stride;
#pragma unroll
            for (int e = 0; e < EB; e++) {
                v[u][e] = f4{0.f, 0.f, 0.f, 0.f};
                if (prow[e] >= 0 && sp0 + u < nsp)
                    v[u][e] = load_f4_sc1(ro, (unsigned)(((g * ROWS + prow[e]) * HD + pcol[e]) * 4) + so);
            }
        }
    };
    const bool one_round = E <= EB && nsp <= U;
    int prow[EB], pcol[EB];
    f4 v[U][EB];
    setup(0, prow, pcol);
    if (one_round) issue(0, prow, pcol, v);
    for (int e = tid; e < nsp * ROWS; e += TPB) {
        const int sp = e / ROWS, rr = e - sp * ROWS;
        if (rr >= n_valid) continue;
        const long long pr = ((long long)sp * p.Hkv + g) * ROWS + rr;
        const float2 ml = load_f2_sc1(rml, (unsigned)(pr * 8));
        s_ml[2 * e] = ml.x;
        s_ml[2 * e + 1] = ml.y;
    }
    __syncthreads();
    if (tid < n_valid) {
        float M = -INFINITY;
        for (int sp = 0; sp < nsp; sp++) M = fmaxf(M, s_ml[2 * (sp * ROWS + tid)]);
        const float Mu = M == -INFINITY ? 0.0f : M;
        float L = 0.0f;
        for (int sp = 0; sp < nsp; sp++) {
            const int e = sp * ROWS + tid;
            L += __builtin_amdgcn_exp2f(s_ml[2 * e] - Mu) * s_ml[2 * e + 1];
        }
        s_row[2 * tid] = Mu;
        s_row[2 * tid + 1] = L > 0.0f ? 1.0f / L : 0.0f;
    }
    __syncthreads();
    for (int e = tid; e < nsp * ROWS; e += TPB) {
        const int rr = e % ROWS;
        if (rr >= n_valid) continue;
        s_ml[2 * e] = __builtin_amdgcn_exp2f(s_ml[2 * e] - s_row[2 * rr]); /* weight of (split, row) */
    }
    __syncthreads();
    for (int e0 = 0; e0 < E; e0 += EB) {
        if (TPB * e0 >= nel) break;
        if (e0 > 0) setup(e0, prow, pcol);
        f4 acc[EB];
#pragma unroll
        for (int e = 0; e < EB; e++) acc[e] = f4{0.f, 0.f, 0.f, 0.f};
        for (int sp0 = 0; sp0 < nsp; sp0 += U) {
            if (!one_round) issue(sp0, prow, pcol, v);
#pragma unroll
            for (int u = 0; u < U; u++) {
                if (sp0 + u >= nsp) break;
#pragma unroll
                for (int e = 0; e < EB; e++)
                    if (prow[e] >= 0) acc[e] += s_ml[2 * ((sp0 + u) * ROWS + prow[e])] * v[u][e];
            }
        }
#pragma unroll
        for (int e = 0; e < EB; e++) {
            if (prow[e] < 0) continue;
            const int r = it.row0 + prow[e];
            const int qi = r / G, hg = r - qi * G;
            *reinterpret_cast<f4 *>(p.out + ((long long)(b.out_tok0 + qi) * Hq + (g * G + hg)) * HD + pcol[e]) =
                acc[e] * s_row[2 * prow[e] + 1];
        }
    }
    if (tid == 0)
        __hip_atomic_store(p.counters + ((long long)it.group * p.Hkv + g) * SK_COUNTER_STRIDE, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

/* Epilogue of k_attn_dec: combines the NW waves' (max, sum, O) through LDS
 * into wave 0, then either writes the normalised rows (single split) or
 * publishes the partial and lets the group's last workgroup merge. Every
 * row's state lives in lanes c, c+16, c+32, c+48. */
template <int HD, int NT, int MAXL = 16, int NW = SK_WAVES>
__device__ __forceinline__ void finish_item(const SkParams &p, const SkItem &it, const SkBatch &b, int item, int g,
                                            int tid,
                                            float (&m)[NT], float (&l)[NT], f4 (&o)[NT][(HD + 15) / 16], float *s_o,
                                            float *s_m, float *s_l, int *s_last) {
    constexpr int DT = (HD + 15) / 16;
    constexpr int ROWS = NT * 16;
    constexpr int OSTR = DT * 16 + 4;
    const int wave = tid >> 6, lane = tid & 63;
    const int c = lane & 15, j = lane >> 4;
    const int G = p.G, Hq = p.Hq;
#pragma unroll
    for (int nt = 0; nt < NT; nt++) {
        l[nt] = row_sum4(l[nt]);
    }
    if (wave > 0) {
        const int sl = (wave - 1) * ROWS;
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
            const int rr = nt * 16 + c;
            float *so = s_o + (sl + rr) * OSTR;
#pragma unroll
            for (int dt = 0; dt < DT; dt++) *reinterpret_cast<f4 *>(so + 16 * dt + 4 * j) = o[nt][dt];
            if (j == 0) { s_m[sl + rr] = m[nt]; s_l[sl + rr] = l[nt]; }
        }
    }
    __syncthreads();
    if (wave == 0) {
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
            const int rr = nt * 16 + c;
            float M = m[nt];
#pragma unroll
            for (int w = 0; w < NW - 1; w++) M = fmaxf(M, s_m[w * ROWS + rr]);
            const float Mu = M == -INFINITY ? 0.0f : M;
            const float a0 = __builtin_amdgcn_exp2f(m[nt] - Mu);
            float L = l[nt] * a0;
#pragma unroll
            for (int dt = 0; dt < DT; dt++) o[nt][dt] *= a0;
#pragma unroll
            for (int w = 0; w < NW - 1; w++) {
                const float aw = __builtin_amdgcn_exp2f(s_m[w * ROWS + rr] - Mu);
                L += s_l[w * ROWS + rr] * aw;
                const float *so = s_o + (w * ROWS + rr) * OSTR;
#pragma unroll
                for (int dt = 0; dt < DT; dt++) o[nt][dt] += aw * *reinterpret_cast<const f4 *>(so + 16 * dt + 4 * j);
            }
            m[nt] = M;
            l[nt] = L;
        }
    }
    if (it.n_split == 1) {
        if (wave != 0) return;
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
            const int r = it.row0 + nt * 16 + c;
            if (r >= b.n_rows) continue;
            const int qi = r / G, hg = r - qi * G;
            float *orow = p.out + ((long long)(b.out_tok0 + qi) * Hq + (g * G + hg)) * HD;
            const float inv = l[nt] > 0.0f ? 1.0f / l[nt] : 0.0f;
#pragma unroll
            for (int dt = 0; dt < DT; dt++) {
                const int d = 16 * dt + 4 * j;
                if (HD % 16 != 0 && d >= HD) continue;
                *reinterpret_cast<f4 *>(orow + d) = o[nt][dt] * inv;
            }
        }
        return;
    }
    /* Publish the partial with device-coherent stores, wait until they are
     * complete, then count in; the group's last workgroup merges (reading
     * with device-coherent loads). */
    const long long pbase = ((long long)item * p.Hkv + g) * ROWS;
    if (wave == 0) {
        const rsrc_t ro = make_rsrc(p.part_o + pbase * HD, (long long)ROWS * HD * 4);
        const rsrc_t rml = make_rsrc(p.part_ml + pbase * 2, (long long)ROWS * 2 * 4);
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
            const int rr = nt * 16 + c;
            if (it.row0 + rr >= b.n_rows) continue;
#pragma unroll
            for (int dt = 0; dt < DT; dt++) {
                const int d = 16 * dt + 4 * j;
                if (HD % 16 != 0 && d >= HD) continue;
                store_f4_sc1(ro, (unsigned)((rr * HD + d) * 4), o[nt][dt]);
            }
            if (j == 0) store_f2_sc1(rml, (unsigned)(rr * 8), m[nt], l[nt]);
        }
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __builtin_amdgcn_s_waitcnt(0); /* every store above acknowledged */
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        int prev = 0;
        if (lane == 0)
            prev = __hip_atomic_fetch_add(p.counters + ((long long)it.group * p.Hkv + g) * SK_COUNTER_STRIDE, 1, __ATOMIC_RELAXED,
                                          __HIP_MEMORY_SCOPE_AGENT);
        prev = __shfl(prev, 0);
        if (lane == 0) *s_last = prev == it.n_split - 1;
    }
    __syncthreads();
    if (!*s_last) return;
    merge_group<HD, ROWS, MAXL, 64 * NW>(p, it, b, item, g, tid, s_o);
}

/* --------------------------------------------------------------- k_attn_dec */

/*
 * Key-parallel attention for decode and short chunks. Cache slabs run on
 * bf16 MFMA (v_mfma_f32_16x16x32_bf16) with the cache's bf16 bits as the
 * operands as loaded (no conversion); precision comes from splitting the
 * other operand, Q = Qhi + Qlo and P = Phi + Plo (bf16 each, ~16
 * significant bits together):  S = K.Qhi + K.Qlo,  O += V.Phi + V.Plo.
 * The slab holding the keys this call appends comes from the fp16 fresh
 * staging (k_prep): each fp16 fragment is split into bf16 hi + lo (exact) in
 * registers and the product takes three bf16 MFMAs (hi.hi, hi.lo, lo.hi).
 * The four waves of a workgroup stream every fourth 32-key slab of the item
 * with buffer loads into registers (slab offset in an SGPR) and are combined
 * by finish_item. S^T = K.Q^T takes K as the A operand with rows gathered as
 * key(t, m) = 8(m >> 2) + 4t + (m & 3), so a lane's 8 probabilities are 8
 * consecutive keys and O^T += V^T.P^T reads V^T with one 16-byte load per
 * lane; a softmax row lives in lanes c, c+16, c+32, c+48. The running max is
 * a lazy reference: the accumulator is rescaled only when some row's max
 * grows by more than 2^LAZY_T (decided per wave by vote), so p <= 2^LAZY_T.
 */
typedef __bf16 b8 __attribute__((ext_vector_type(8)));
#define LAZY_T 8.0f

__device__ __forceinline__ b8 as_b8(uint4 w) { return *reinterpret_cast<b8 *>(&w); }

__device__ __forceinline__ void split8(const float *x, b8 &hi, b8 &lo) {
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const __bf16 h = (__bf16)x[i];
        hi[i] = h;
        lo[i] = (__bf16)(x[i] - (float)h);
    }
}

template <int HD, int NT, int W, bool ST, int NW = SK_WAVES>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(W, W))) void k_attn_dec(SkParams p) {
    static_assert(!ST || NW == 4, "the staged build's transfers are laid out for four waves");
    constexpr int KS = (HD + 31) / 32;
    constexpr int DT = (HD + 15) / 16;
    constexpr int HDP = KS * 32;
    constexpr int ROWS = NT * 16;
    constexpr int OSTR = DT * 16 + 4;
    constexpr unsigned SLAB_K_BYTES = SMOL_SLAB * HD * 2; /* one slab of K, and one slab-block of V^T */
    /* ST: every slab of the item (at most SMAX) is requested at once into
     * LDS by direct transfers, before Q is read; the waves then take their
     * slabs' fragments from LDS. Otherwise each wave loads its slabs'
     * fragments into registers, one slab ahead. */
    constexpr int KROW = HD <= 128 ? 256 : 512; /* LDS bytes per key row */
    constexpr int K_LDS = SMOL_SLAB * KROW, V_LDS = 16 * DT * 64;
    constexpr int SLAB_LDS = (K_LDS + V_LDS + 4095) / 4096 * 4096;
    constexpr int NDMA = SLAB_LDS / 4096; /* transfers per wave per slab */
    constexpr int SMAX = ST ? (HD > 128 ? 5 : 4) : 0;
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63;
    const int c = lane & 15, j = lane >> 4;
    /* kv head fastest in the block index: consecutive workgroups go to
     * consecutive XCDs, so each XCD's L2 holds the K/V of its own heads */
    const int g = (int)(blockIdx.x % (unsigned)p.Hkv);
    const int item = (int)(blockIdx.x / (unsigned)p.Hkv);
    const SkItemB rec = p.items[item];
    const SkItem &it = rec.it;
    const SkBatch &b = rec.b;
    const int G = p.G;
    /* s_o: the other waves' (o) rows in the combine, the merge's arrays, and
     * (direct decode) the staged Q rows; past the combine's rows, the new
     * value, which wave 0 reads while the other waves fill theirs */
    constexpr int SVN = (NW - 1) * ROWS * OSTR;
    constexpr int SO = SVN + HD > 2 * SK_MERGE_MAX + 128 ? SVN + HD : 2 * SK_MERGE_MAX + 128;
    /* the epilogue's arrays; with ST they reuse the slab area once every
     * wave is done with it */
    constexpr int FIN_BYTES = (SO + 2 * (NW - 1) * ROWS + 1) * 4;
    constexpr int SMEM = SMAX * SLAB_LDS > FIN_BYTES ? SMAX * SLAB_LDS : FIN_BYTES;
    static_assert(SMEM <= 160 * 1024, "LDS");
    __shared__ __attribute__((aligned(1024))) unsigned char smem[SMEM];
    float *s_o = reinterpret_cast<float *>(smem);
    float *s_m = s_o + SO, *s_l = s_m + (NW - 1) * ROWS;
    int *s_last = reinterpret_cast<int *>(s_l + (NW - 1) * ROWS);

    b8 qh[NT][KS], ql[NT][KS];
    int lo[NT], hi[NT];
    float m[NT], l[NT];
    f4 o[NT][DT];
    int lo_max = -(1 << 30), hi_min = 1 << 30; /* over this lane's valid rows */
#pragma unroll
    for (int nt = 0; nt < NT; nt++) {
        const int r = it.row0 + nt * 16 + c;
        const bool valid = r < b.n_rows;
        const int qi = r / G;
        int rl = b.key_lo, rh = b.key_hi;
        if (b.causal) {
            rh = min(rh, b.q_pos0 + qi + 1);
            if (p.window > 0) rl = max(rl, b.q_pos0 + qi - p.window + 1);
        }
        /* rows past the batch are never stored: leave them unmasked */
        lo[nt] = valid ? rl : -(1 << 30);
        hi[nt] = valid ? rh : (1 << 30);
        lo_max = max(lo_max, lo[nt]);
        hi_min = min(hi_min, hi[nt]);
        m[nt] = -INFINITY;
        l[nt] = 0.0f;
#pragma unroll
        for (int dt = 0; dt < DT; dt++) o[nt][dt] = f4{0.f, 0.f, 0.f, 0.f};
    }
    /* Q fragments (after the first slabs' loads are in flight) */
    auto load_q = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
            const int r = it.row0 + nt * 16 + c;
            const bool valid = r < b.n_rows;
            const float *qrow =
                p.qs32 + (long long)g * p.qs_head_stride + (long long)(b.q_row0 + (valid ? r : 0)) * HDP;
#pragma unroll
            for (int ks = 0; ks < KS; ks++) {
                float x[8] = {0, 0, 0, 0, 0, 0, 0, 0};
                if (valid) {
                    const float4 a = *reinterpret_cast<const float4 *>(qrow + 32 * ks + 8 * j);
                    const float4 e = *reinterpret_cast<const float4 *>(qrow + 32 * ks + 8 * j + 4);
                    x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w; x[4] = e.x; x[5] = e.y; x[6] = e.z; x[7] = e.w;
                }
                split8(x, qh[nt][ks], ql[nt][ks]);
            }
        }
    };
    /* p.dec_direct: the WG stages its Q rows, the table row of the position
     * and the norm weights (and, for the batch's last split, the new key and
     * value) through LDS as fp32 with one round of loads issued before the
     * first slab's; every lane then normalises, rotates (the pre-pass's
     * formulas) and scales its Q fragments from LDS. The last split's wave 0
     * scores the new key against every row (s_new) and appends its bf16 K
     * row to the cache; the value joins that wave's softmax state after the
     * slabs (add_new_key). */
    constexpr int QSTR = HD + 4; /* padded LDS row of a staged Q row */
    const bool last_split = it.split == it.n_split - 1;
    const bool owner = p.dec_direct && wave == 0 && last_split;
    const long long cbase = (long long)b.slot * p.c_slot_stride + (long long)g * p.cap * HD;
    float *s_vnew = s_o + SVN;             /* the new value [HD], read after the slabs */
    float *s_q = s_o;                      /* [ROWS][QSTR] */
    float *s_k = s_q + ROWS * QSTR;        /* new key [HD] */
    float *s_cos = s_k + HD, *s_sin = s_cos + HD, *s_wq = s_sin + HD, *s_wk = s_wq + HD;
    static_assert(ROWS * QSTR + 5 * HD <= SVN, "direct decode staging");
    constexpr int C4Q = HD / 4;            /* 4-element chunks per row */
    constexpr int NSTAGE = (ROWS * C4Q + 6 * C4Q + 64 * NW - 1) / (64 * NW);
    const int n_qrows = min(ROWS, b.n_rows - it.row0);
    const bool bf_in = p.q_dtype == SMOL_IN_BF16;
    /* chunk e of the staged list: Q rows, cos, sin, q weights, then (last
     * split) k, v, k weights; its global source and LDS destination */
    auto stage_src = [&](int e, const void *&src, long long &idx, bool &f32, float *&dst) -> bool {
        const int nq = n_qrows * C4Q;
        if (e < nq) {
            const int r = e / C4Q, c0 = (e - r * C4Q) * 4;
            const int rr = it.row0 + r, qi = rr / G, hg = rr - qi * G;
            src = p.q_in; f32 = !bf_in; dst = s_q + r * QSTR + c0;
            idx = (long long)(b.out_tok0 + qi) * p.q_stride + (long long)(g * G + hg) * HD + c0;
            return true;
        }
        e -= nq;
        const int seg = e / C4Q, c0 = (e - seg * C4Q) * 4;
        const long long kvrow = (long long)b.out_tok0 * p.kv_stride + (long long)g * HD;
        switch (seg) {
        case 0: if (p.rope_q_kind == SMOL_ROPE_OFF) return false;
                src = p.rope_cos; f32 = true; idx = (long long)b.q_pos0 * HD + c0; dst = s_cos + c0; return true;
        case 1: if (p.rope_q_kind == SMOL_ROPE_OFF) return false;
                src = p.rope_sin; f32 = true; idx = (long long)b.q_pos0 * HD + c0; dst = s_sin + c0; return true;
        case 2: if (!p.q_norm) return false;
                src = p.q_norm; f32 = true; idx = c0; dst = s_wq + c0; return true;
        case 3: if (!last_split) return false;
                src = p.k_in; f32 = !bf_in; idx = kvrow + c0; dst = s_k + c0; return true;
        case 4: if (!last_split) return false;
                src = p.v_in; f32 = !bf_in; idx = kvrow + c0; dst = s_vnew + c0; return true;
        case 5: if (!last_split || !p.k_norm) return false;
                src = p.k_norm; f32 = true; idx = c0; dst = s_wk + c0; return true;
        default: return false;
        }
    };
    uint4 st_raw[NSTAGE];
    auto stage_issue = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < NSTAGE; u++) {
            const void *src; long long idx; bool f32; float *dst;
            st_raw[u] = make_uint4(0, 0, 0, 0);
            if (stage_src(tid + 64 * NW * u, src, idx, f32, dst)) {
                if (f32) st_raw[u] = *reinterpret_cast<const uint4 *>((const float *)src + idx);
                else {
                    const uint2 h = *reinterpret_cast<const uint2 *>((const uint16_t *)src + idx);
                    st_raw[u] = make_uint4(h.x, h.y, 0, 0);
                }
            }
        }
    };
    auto stage_store = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < NSTAGE; u++) {
            const void *src; long long idx; bool f32; float *dst;
            if (stage_src(tid + 64 * NW * u, src, idx, f32, dst)) {
                float4 v;
                if (f32) v = make_float4(__uint_as_float(st_raw[u].x), __uint_as_float(st_raw[u].y),
                                         __uint_as_float(st_raw[u].z), __uint_as_float(st_raw[u].w));
                else v = make_float4(__uint_as_float(st_raw[u].x << 16), __uint_as_float(st_raw[u].x & 0xFFFF0000u),
                                     __uint_as_float(st_raw[u].y << 16), __uint_as_float(st_raw[u].y & 0xFFFF0000u));
                *reinterpret_cast<float4 *>(dst) = v;
            }
        }
    };
    float s_new[NT];
    /* 8 consecutive fp32 values of LDS (16-byte aligned) */
    auto ld8 = [&](const float *a, float *v) __attribute__((always_inline)) {
        const float4 x = *reinterpret_cast<const float4 *>(a), y = *reinterpret_cast<const float4 *>(a + 4);
        v[0] = x.x; v[1] = x.y; v[2] = x.z; v[3] = x.w; v[4] = y.x; v[5] = y.y; v[6] = y.z; v[7] = y.w;
    };
    /* x[i] of the staged row `row`, normalised with weights w (null: none)
     * and rotated at element d0 + i, as rope8 does */
    auto rot8 = [&](const float *row, int d0, const float *w, float rinv, float *x) __attribute__((always_inline)) {
        constexpr int HALF = HD / 2;
        float v[8];
        ld8(row + d0, v);
        if (w) {
            float wv[8];
            ld8(w + d0, wv);
#pragma unroll
            for (int i = 0; i < 8; i++) v[i] = (v[i] * wv[i]) * rinv;
        }
        const int kind = p.rope_q_kind;
        if (kind == SMOL_ROPE_OFF) {
#pragma unroll
            for (int i = 0; i < 8; i++) x[i] = v[i];
            return;
        }
        float cv[8], sv[8];
        ld8(s_cos + d0, cv);
        ld8(s_sin + d0, sv);
        if (kind == SMOL_ROPE_INTERLEAVED_K) {
#pragma unroll
            for (int i = 0; i < 8; i += 2) {
                const float x0 = v[i], x1 = v[i + 1];
                x[i] = x0 * cv[i] - x1 * sv[i];
                x[i + 1] = x1 * cv[i + 1] + x0 * sv[i + 1];
            }
            return;
        }
        float pr[8];
        if constexpr (HALF % 8 == 0) {
            const int p0 = d0 < HALF ? d0 + HALF : d0 - HALF;
            ld8(row + p0, pr);
            if (w) {
                float wp[8];
                ld8(w + p0, wp);
#pragma unroll
                for (int i = 0; i < 8; i++) pr[i] = (pr[i] * wp[i]) * rinv;
            }
        } else {
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const int d = d0 + i, pd = d < HALF ? d + HALF : d - HALF;
                pr[i] = w ? (row[pd] * w[pd]) * rinv : row[pd];
            }
        }
#pragma unroll
        for (int i = 0; i < 8; i++)
            x[i] = d0 + i < HALF ? fmaf(v[i], cv[i], -(pr[i] * sv[i])) : fmaf(v[i], cv[i], pr[i] * sv[i]);
    };
    auto rinv_of = [&](const float *row) __attribute__((always_inline)) {
        float ss = 0.0f;
#pragma unroll
        for (int ks = 0; ks < KS; ks++) {
            const int d0 = 32 * ks + 8 * j;
            if (HD % 32 == 0 || d0 < HD) {
                float v[8];
                ld8(row + d0, v);
#pragma unroll
                for (int i = 0; i < 8; i++) ss = fmaf(v[i], v[i], ss);
            }
        }
        ss = row_sum4(ss);
        return 1.0f / sqrtf(ss / (float)HD + p.norm_eps);
    };
    auto load_q_direct = [&]() __attribute__((always_inline)) {
        const float krinv = owner && p.k_norm ? rinv_of(s_k) : 1.0f;
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
            const int r = nt * 16 + c;
            const bool valid = it.row0 + r < b.n_rows;
            const float *qrow = s_q + (valid ? r : 0) * QSTR;
            const float qrinv = p.q_norm ? rinv_of(qrow) : 1.0f;
            float sd = 0.0f;
#pragma unroll
            for (int ks = 0; ks < KS; ks++) {
                const int d0 = 32 * ks + 8 * j;
                float x[8] = {0, 0, 0, 0, 0, 0, 0, 0};
                if (HD % 32 == 0 || d0 < HD) {
                    rot8(qrow, d0, p.q_norm ? s_wq : nullptr, qrinv, x);
#pragma unroll
                    for (int i = 0; i < 8; i++) x[i] = valid ? x[i] * p.qscale : 0.0f;
                    if (owner) {
                        float kx[8];
                        rot8(s_k, d0, p.k_norm ? s_wk : nullptr, krinv, kx);
#pragma unroll
                        for (int i = 0; i < 8; i++) sd = fmaf(x[i], kx[i], sd);
                        if (nt == 0 && c == 0)
                            *reinterpret_cast<uint4 *>(const_cast<uint16_t *>(p.kc) + cbase + (long long)b.q_pos0 * HD + d0) =
                                pack_bf16x8(kx); /* the cache itself: writable */
                    }
                }
                split8(x, qh[nt][ks], ql[nt][ks]);
            }
            s_new[nt] = owner ? row_sum4(sd) : 0.0f;
        }
    };
    /* the new key's term in the last split's state (exact max, no laziness),
     * and its bf16 V^T entries in the cache */
    auto add_new_key = [&]() __attribute__((always_inline)) {
        float vv[DT][4];
#pragma unroll
        for (int dt = 0; dt < DT; dt++) {
            const int d = 16 * dt + 4 * j;
#pragma unroll
            for (int i = 0; i < 4; i++) vv[dt][i] = (HD % 16 == 0 || d + i < HD) ? s_vnew[d + i] : 0.0f;
        }
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
            float sc = s_new[nt];
            if (p.cap2 > 0.0f) sc = p.cap2 * tanhf(sc / p.cap2);
            const float m_new = fmaxf(m[nt], sc);
            const float alpha = __builtin_amdgcn_exp2f(m[nt] - m_new);
            const float pn = __builtin_amdgcn_exp2f(sc - m_new);
#pragma unroll
            for (int dt = 0; dt < DT; dt++)
#pragma unroll
                for (int i = 0; i < 4; i++) o[nt][dt][i] = fmaf(pn, vv[dt][i], o[nt][dt][i] * alpha);
            l[nt] = l[nt] * alpha + (j == 0 ? pn : 0.0f); /* l is summed over the row's four lanes later */
            m[nt] = m_new;
        }
        if (c == 0) {
            uint16_t *vt = const_cast<uint16_t *>(p.vtc) + cbase + (long long)(b.q_pos0 / SMOL_SLAB) * SMOL_SLAB * HD +
                           b.q_pos0 % SMOL_SLAB;
#pragma unroll
            for (int dt = 0; dt < DT; dt++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int d = 16 * dt + 4 * j + i;
                    if (HD % 16 == 0 || d < HD) vt[(long long)d * SMOL_SLAB] = f32_to_bf16(vv[dt][i]);
                }
        }
    };
    /* the slab [k0, k0 + 32) needs no masking when it lies inside every row's range */
#pragma unroll
    for (int sh = 1; sh < 16; sh <<= 1) {
        lo_max = max(lo_max, __shfl_xor(lo_max, sh));
        hi_min = min(hi_min, __shfl_xor(hi_min, sh));
    }
    lo_max = __builtin_amdgcn_readfirstlane(lo_max);
    hi_min = __builtin_amdgcn_readfirstlane(hi_min);

    /* buffer resources: the cache region of (slot, head) and the fresh region of head */
    rsrc_t rk_c = make_rsrc(nullptr, 0), rv_c = make_rsrc(nullptr, 0);
    if (b.slot >= 0 && p.kc != nullptr) {
        const long long cb = (long long)b.slot * p.c_slot_stride + (long long)g * p.cap * HD;
        rk_c = make_rsrc(p.kc + cb, (long long)p.cap * HD * 2);
        rv_c = make_rsrc(p.vtc + cb, (long long)p.cap * HD * 2);
    }
    const rsrc_t rk_f = make_rsrc(p.kf + (long long)g * p.fcap * HD, (long long)p.fcap * HD * 2);
    const rsrc_t rv_f = make_rsrc(p.vtf + (long long)g * p.fcap * HD, (long long)p.fcap * HD * 2);
    /* lane-constant byte offsets within a slab */
    const int kt_row = 8 * (c >> 2) + (c & 3);
    unsigned vo_k[2][KS], vo_v[DT];
#pragma unroll
    for (int t = 0; t < 2; t++)
#pragma unroll
        for (int ks = 0; ks < KS; ks++) {
            const int d0 = 32 * ks + 8 * j;
            vo_k[t][ks] = (HD % 32 == 0 || d0 < HD) ? (unsigned)(((kt_row + 4 * t) * HD + d0) * 2) : OOB_OFF;
        }
#pragma unroll
    for (int dt = 0; dt < DT; dt++) {
        const int d = 16 * dt + c;
        vo_v[dt] = (HD % 16 == 0 || d < HD) ? (unsigned)((d * SMOL_SLAB + 8 * j) * 2) : OOB_OFF;
    }

    struct KRaw {
        uint4 k[2][KS];
    };
    struct VRaw {
        uint4 v[DT];
    };
    /* slab k0's resource and slab offset: a uniform choice (SGPRs) */
    auto slab_src = [&](int k0, bool value, rsrc_t &r, unsigned &so) {
        const bool fr = k0 >= b.fresh_pos0;
        const int kr = fr ? k0 + it.fresh_off : k0;
        so = (unsigned)(kr / SMOL_SLAB) * SLAB_K_BYTES;
        r = value ? (fr ? rv_f : rv_c) : (fr ? rk_f : rk_c);
    };
    /* with head_dim a multiple of 32 (resp. 16) every lane's fragment
     * offsets are one lane base plus constants, which ride in the scalar
     * offset instead of occupying a register each */
    const unsigned kbase = (unsigned)((kt_row * HD + 8 * j) * 2);
    const unsigned vbase = (unsigned)((c * SMOL_SLAB + 8 * j) * 2);
    auto issue_k = [&](int k0, KRaw &r) __attribute__((always_inline)) {
        rsrc_t rs;
        unsigned so;
        slab_src(k0, false, rs, so);
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
            for (int ks = 0; ks < KS; ks++)
                r.k[t][ks] = HD % 32 == 0 ? bload(rs, kbase, so + (unsigned)((4 * t * HD + 32 * ks) * 2))
                                          : bload(rs, vo_k[t][ks], so);
    };
    auto issue_v = [&](int k0, VRaw &r) __attribute__((always_inline)) {
        rsrc_t rs;
        unsigned so;
        slab_src(k0, true, rs, so);
#pragma unroll
        for (int dt = 0; dt < DT; dt++)
            r.v[dt] = HD % 16 == 0 ? bload(rs, vbase, so + (unsigned)(16 * dt * SMOL_SLAB * 2)) : bload(rs, vo_v[dt], so);
    };

    auto qk = [&](const KRaw &r, f4 (&sacc)[NT][2], auto fresh_tag) {
        constexpr bool FRESH = decltype(fresh_tag)::value;
#pragma unroll
        for (int nt = 0; nt < NT; nt++)
#pragma unroll
            for (int t = 0; t < 2; t++) {
                f4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int ks = 0; ks < KS; ks++) {
                    if (FRESH) {
                        /* the fresh slab's fp16 K as bf16 hi + lo (exact: 11 significant
                         * bits), K.Q = Khi.Qhi + Khi.Qlo + Klo.Qhi */
                        b8 kh, kl;
                        float kx[8];
                        const h8 k16 = *reinterpret_cast<const h8 *>(&r.k[t][ks]);
#pragma unroll
                        for (int i = 0; i < 8; i++) kx[i] = (float)k16[i];
                        split8(kx, kh, kl);
                        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kh, qh[nt][ks], acc, 0, 0, 0);
                        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kh, ql[nt][ks], acc, 0, 0, 0);
                        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kl, qh[nt][ks], acc, 0, 0, 0);
                    } else {
                        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_b8(r.k[t][ks]), qh[nt][ks], acc, 0, 0, 0);
                        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_b8(r.k[t][ks]), ql[nt][ks], acc, 0, 0, 0);
                    }
                }
                sacc[nt][t] = acc;
            }
    };

    auto smpv = [&](int k0, const f4 (&sacc)[NT][2], const VRaw &r, auto fresh_tag) {
        constexpr bool FRESH = decltype(fresh_tag)::value;
        const bool full = k0 >= lo_max && k0 + SMOL_SLAB <= hi_min;
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
            float sv[8];
#pragma unroll
            for (int t = 0; t < 2; t++)
#pragma unroll
                for (int i = 0; i < 4; i++) sv[4 * t + i] = sacc[nt][t][i];
            if (p.cap2 > 0.0f) {
#pragma unroll
                for (int e = 0; e < 8; e++) sv[e] = p.cap2 * tanhf(sv[e] / p.cap2);
            }
            if (!full) {
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    const int key = k0 + 8 * j + e;
                    sv[e] = (key >= lo[nt] && key < hi[nt]) ? sv[e] : -INFINITY;
                }
            }
            float mx = sv[0];
#pragma unroll
            for (int e = 1; e < 8; e++) mx = fmaxf(mx, sv[e]);
            mx = row_max4(mx);
            const bool need = mx > m[nt] + LAZY_T;
            if (__any(need)) {
                const float m_new = need ? mx : m[nt];
                const float alpha = need ? __builtin_amdgcn_exp2f(m[nt] - m_new) : 1.0f;
#pragma unroll
                for (int dt = 0; dt < DT; dt++) o[nt][dt] *= alpha;
                l[nt] *= alpha;
                m[nt] = m_new;
            }
            const float m_use = m[nt] == -INFINITY ? 0.0f : m[nt];
            float pv[8];
            float ps = 0.0f;
#pragma unroll
            for (int e = 0; e < 8; e++) {
                pv[e] = __builtin_amdgcn_exp2f(sv[e] - m_use);
                ps += pv[e];
            }
            l[nt] += ps;
            b8 ph, pl;
            split8(pv, ph, pl);
            if (FRESH) {
                /* fp16 V^T as bf16 hi + lo: O += Vhi.Phi + Vhi.Plo + Vlo.Phi */
#pragma unroll
                for (int dt = 0; dt < DT; dt++) {
                    b8 vh, vl;
                    float vx[8];
                    const h8 v16 = *reinterpret_cast<const h8 *>(&r.v[dt]);
#pragma unroll
                    for (int i = 0; i < 8; i++) vx[i] = (float)v16[i];
                    split8(vx, vh, vl);
                    o[nt][dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vh, ph, o[nt][dt], 0, 0, 0);
                    o[nt][dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vh, pl, o[nt][dt], 0, 0, 0);
                    o[nt][dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vl, ph, o[nt][dt], 0, 0, 0);
                }
            } else {
#pragma unroll
                for (int dt = 0; dt < DT; dt++) {
                    o[nt][dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_b8(r.v[dt]), ph, o[nt][dt], 0, 0, 0);
                    o[nt][dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_b8(r.v[dt]), pl, o[nt][dt], 0, 0, 0);
                }
            }
        }
    };

    const int step = SMOL_SLAB * NW;
    const int end = it.key_end;
    if constexpr (ST) {
        /* all n <= SMAX slabs of the item into LDS (slab s at s * SLAB_LDS,
         * the image of k_attn_fb: K rows XOR-swizzled, V^T rows of 64 bytes) */
        const int n = min(SMAX, (end - it.key_begin + SMOL_SLAB - 1) / SMOL_SLAB); /* the host plans n <= SMAX */
        unsigned d_off[NDMA];
        bool d_isk[NDMA];
#pragma unroll
        for (int e = 0; e < NDMA; e++) {
            const int q = wave + 4 * e;
            d_isk[e] = q * 1024 < K_LDS;
            if (d_isk[e]) {
                constexpr int RPR = 1024 / KROW, SPR = KROW / 16; /* rows per region, slots per row */
                const int kr = q * RPR + lane / SPR, slot = lane % SPR;
                const int cb = slot ^ ((kr & 3) | (((kr >> 3) & 3) << 2));
                d_off[e] = cb < HD / 8 ? (unsigned)((kr * HD + cb * 8) * 2) : OOB_OFF;
            } else {
                const int d = (q * 1024 - K_LDS) / 64 + (lane >> 2), slot = lane & 3;
                const int jj = slot ^ ((d >> 1) & 3);
                d_off[e] = (d < HD && q * 1024 < K_LDS + V_LDS) ? (unsigned)((d * SMOL_SLAB + jj * 8) * 2) : OOB_OFF;
            }
        }
        const unsigned lds0 = (unsigned)(size_t)smem;
#pragma unroll
        for (int sl = 0; sl < SMAX; sl++) {
            if (sl >= n) break;
            rsrc_t rk, rv;
            unsigned so;
            slab_src(it.key_begin + SMOL_SLAB * sl, false, rk, so);
            slab_src(it.key_begin + SMOL_SLAB * sl, true, rv, so);
#pragma unroll
            for (int e = 0; e < NDMA; e++)
                dma_1k(d_isk[e] ? rk : rv, d_off[e], so,
                       __builtin_amdgcn_readfirstlane(lds0 + sl * SLAB_LDS + (wave + 4 * e) * 1024));
        }
        load_q();
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        const int kt_row = 8 * (c >> 2) + (c & 3);
        unsigned kfo[KS];
#pragma unroll
        for (int ks = 0; ks < KS; ks++) kfo[ks] = (unsigned)(kt_row * KROW + 16 * ((4 * ks + j) ^ c));
        const unsigned vfo = (unsigned)(K_LDS + c * 64 + 16 * (j ^ ((c >> 1) & 3)));
        for (int sl = wave; sl < n; sl += NW) {
            const unsigned char *base = smem + sl * SLAB_LDS;
            const int kk = it.key_begin + SMOL_SLAB * sl;
            KRaw kr;
            VRaw vr;
#pragma unroll
            for (int t = 0; t < 2; t++)
#pragma unroll
                for (int ks = 0; ks < KS; ks++) kr.k[t][ks] = *reinterpret_cast<const uint4 *>(base + kfo[ks] + t * 4 * KROW);
#pragma unroll
            for (int dt = 0; dt < DT; dt++) vr.v[dt] = *reinterpret_cast<const uint4 *>(base + vfo + dt * 1024);
            f4 sacc[NT][2];
            const bool fr = kk >= b.fresh_pos0;
            if (fr) qk(kr, sacc, std::true_type{});
            else qk(kr, sacc, std::false_type{});
            if (fr) smpv(kk, sacc, vr, std::true_type{});
            else smpv(kk, sacc, vr, std::false_type{});
        }
        __syncthreads(); /* the slab area becomes the epilogue's */
    } else {
        /* Each wave streams slabs wave, wave + NW, ... with one K/V
         * register buffer, the next slab requested while the current one is
         * computed and the first one before Q is loaded. The last slab is
         * peeled off the loop, so no load is left in flight for the
         * epilogue's wait, and every wait inside the loop sees the same
         * number of loads in flight. */
        int k0 = it.key_begin + wave * SMOL_SLAB;
        KRaw kr;
        VRaw vr;
        if (p.dec_direct) {
            /* staging loads, the first slab's loads, then the staged values
             * into LDS (waiting for the staging loads only), Q from LDS, and
             * a barrier before the epilogue may reuse the area */
            stage_issue();
            if (k0 < end) {
                issue_k(k0, kr);
                issue_v(k0, vr);
            }
            stage_store();
            __syncthreads();
            load_q_direct();
            __syncthreads();
        }
        if (k0 < end) {
            if (!p.dec_direct) {
                issue_k(k0, kr);
                issue_v(k0, vr);
                load_q();
            }
            auto slab = [&](auto issue_tag) __attribute__((always_inline)) {
                constexpr bool ISSUE = decltype(issue_tag)::value;
                f4 sacc[NT][2];
                const bool fr = k0 >= b.fresh_pos0;
                if (fr) qk(kr, sacc, std::true_type{});
                else qk(kr, sacc, std::false_type{});
                if constexpr (ISSUE) issue_k(k0 + step, kr);
                if (fr) smpv(k0, sacc, vr, std::true_type{});
                else smpv(k0, sacc, vr, std::false_type{});
                if constexpr (ISSUE) issue_v(k0 + step, vr);
            };
            for (; k0 + step < end; k0 += step) slab(std::true_type{});
            slab(std::false_type{});
        } else if (!p.dec_direct) {
            load_q();
        }
    }
    if (owner) add_new_key();

    finish_item<HD, NT, W == 1 ? 64 : 32, NW>(p, it, b, item, g, tid, m, l, o, s_o, s_m, s_l, s_last);
}

/* ---------------------------------------------------------------- k_attn_fa */

/*
 * Prefill, chunked prefill and windowed bidirectional attention with the
 * four waves of a workgroup on different query rows and the K/V slabs shared
 * through LDS. Wave w owns row tiles w*NT .. w*NT+NT-1 of the item's 64*NT
 * rows; all four walk the item's 32-key slabs together.
 *
 * Staging: every thread loads its 1/256 share of a slab (16-byte chunks)
 * into registers a few slabs ahead and stores one slab per step into a ring
 * of four LDS stages (bf16 cache slabs are widened to fp16 on the way, once
 * per workgroup rather than once per wave). One barrier per slab both
 * publishes the next stage and frees the oldest.
 *
 * Per wave the slabs are software-pipelined: S^T = K.Q^T of slab i+1 is
 * formed on the matrix cores while the vector ALU computes the
 * exponentials of slab i.
 *
 * LDS image, XOR-swizzled so that each ds_read_b128 of an MFMA fragment and
 * each staging store is free of bank conflicts. A b128 access is served eight
 * lanes at a time, and the eight must fall in distinct 16-byte columns of a
 * 128-byte line (measured: the V^T image with slot j ^ ((d >> 2) & 3) ran at
 * half the rate of a linear read, with the slot below at the full rate):
 *   K   : 32 key rows of KROW bytes; 16-byte chunk cb of key row r sits in
 *         slot cb ^ f(r), f(r) = (r & 3) | ((r >> 3) & 3) << 2. The A-operand
 *         rows of lane c are r = 8(c>>2) + (c&3) + 4t, for which f(r) = c.
 *   V^T : 16*DT rows of 64 bytes (32 keys); chunk j of row d sits in slot
 *         j ^ ((d >> 1) & 3).
 * Chunks of a K row past head_dim are zero (the stages are cleared once and
 * those slots are never stored), so padded head dims contribute 0 * 0. V^T
 * rows past head_dim only feed output rows that are never written.
 *
 * Softmax, lazy rescale and MFMA layouts as in k_attn_dec; each wave holds
 * whole rows, so no cross-wave combine is needed.
 */
template <int HD>
struct FaGeom {
    static constexpr int KS = (HD + 31) / 32;
    static constexpr int DT = (HD + 15) / 16;
    static constexpr int HDP = KS * 32;
    static constexpr int KROW = HD <= 128 ? 256 : 512;
    static constexpr int K_BYTES = SMOL_SLAB * KROW;
    static constexpr int V_BYTES = 16 * DT * 64;
    static constexpr int STAGE = K_BYTES + V_BYTES;
    static constexpr int CK = SMOL_SLAB * HD / 8; /* 16-byte chunks in a K (or V^T) slab */
    static constexpr int PER = (CK + 255) / 256;  /* K (and V) chunks per thread */
};

template <int HD, int NT, int W>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(W, W))) void k_attn_fa(SkParams p) {
    using Gm = FaGeom<HD>;
    constexpr int KS = Gm::KS, DT = Gm::DT, HDP = Gm::HDP, KROW = Gm::KROW;
    constexpr int STAGE = Gm::STAGE, K_BYTES = Gm::K_BYTES, CK = Gm::CK, PER = Gm::PER;
    constexpr int ROWS = 4 * 16 * NT;
    constexpr unsigned SLAB_BYTES = SMOL_SLAB * HD * 2;
    constexpr int NSTG = 4;                /* LDS stages: slabs i, i+1 read while i+2 is stored */
    constexpr int SETS = W == 1 ? 4 : 2;   /* register sets of staged slabs in flight */
    constexpr int MERGE_BYTES = (2 * SK_MERGE_MAX + 128) * 4;
    constexpr int SMEM = NSTG * STAGE > MERGE_BYTES ? NSTG * STAGE : MERGE_BYTES;
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63;
    const int c = lane & 15, j = lane >> 4;
    const int g = (int)(blockIdx.x % (unsigned)p.Hkv);
    const int item = (int)(blockIdx.x / (unsigned)p.Hkv);
    const SkItemB rec = p.items[item];
    const SkItem &it = rec.it;
    const SkBatch &b = rec.b;
    const int G = p.G;
    __shared__ __attribute__((aligned(16))) unsigned char smem[SMEM];
    __shared__ int s_last;

    for (int e = tid; e < NSTG * STAGE / 16; e += 256) reinterpret_cast<uint4 *>(smem)[e] = make_uint4(0, 0, 0, 0);

    /* this wave's rows: Q fragments, visible key ranges */
    h8 qf[NT][KS];
    int lo[NT], hi[NT];
    float m[NT], l[NT];
    f4 negm[NT];   /* -m (0 while m = -inf): the accumulator input of S = K.Q^T - m */
    float thr[NT]; /* a score above thr (relative to m) calls for a rescale */
    f4 o[NT][DT];
    int lo_max = -(1 << 30), hi_min = 1 << 30;
#pragma unroll
    for (int nt = 0; nt < NT; nt++) {
        const int r = it.row0 + (wave * NT + nt) * 16 + c;
        const bool valid = r < b.n_rows;
        const int qi = r / G;
        int rl = b.key_lo, rh = b.key_hi;
        if (b.causal) {
            rh = min(rh, b.q_pos0 + qi + 1);
            if (p.window > 0) rl = max(rl, b.q_pos0 + qi - p.window + 1);
        }
        lo[nt] = valid ? rl : -(1 << 30);
        hi[nt] = valid ? rh : (1 << 30);
        lo_max = max(lo_max, lo[nt]);
        hi_min = min(hi_min, hi[nt]);
        m[nt] = -INFINITY;
        l[nt] = 0.0f;
        negm[nt] = f4{0.f, 0.f, 0.f, 0.f};
        thr[nt] = -INFINITY;
        if (p.q_direct) {
            /* rotate and scale Q here: row r is query qi of head g*G + hg */
            const int hg = r - qi * G;
            const long long row = (long long)(b.out_tok0 + (valid ? qi : 0)) * p.q_stride + (long long)(g * G + hg) * HD;
#pragma unroll
            for (int ks = 0; ks < KS; ks++) {
                const int d0 = 32 * ks + 8 * j;
                float v[8] = {0, 0, 0, 0, 0, 0, 0, 0};
                if (valid && (HD % 32 == 0 || d0 < HD)) {
                    rope8(p.q_in, p.q_dtype, row, d0, HD, p.rope_q_kind, p.rope_cos, p.rope_sin, b.q_pos0 + qi, v);
#pragma unroll
                    for (int i = 0; i < 8; i++) v[i] *= p.qscale;
                }
#pragma unroll
                for (int i = 0; i < 8; i++) qf[nt][ks][i] = (_Float16)v[i];
            }
        } else {
            const _Float16 *qrow =
                p.qs + (long long)g * p.qs_head_stride + (long long)(b.q_row0 + (valid ? r : 0)) * HDP;
#pragma unroll
            for (int ks = 0; ks < KS; ks++) qf[nt][ks] = valid ? load_h8(qrow + 32 * ks + 8 * j) : zero_h8();
        }
#pragma unroll
        for (int dt = 0; dt < DT; dt++) o[nt][dt] = f4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int sh = 1; sh < 64; sh <<= 1) {
        lo_max = max(lo_max, __shfl_xor(lo_max, sh));
        hi_min = min(hi_min, __shfl_xor(hi_min, sh));
    }
    lo_max = __builtin_amdgcn_readfirstlane(lo_max);
    hi_min = __builtin_amdgcn_readfirstlane(hi_min);

    /* sources: cache region of (slot, head) and fresh region of head */
    rsrc_t rk_c = make_rsrc(nullptr, 0), rv_c = make_rsrc(nullptr, 0);
    if (b.slot >= 0 && p.kc != nullptr) {
        const long long cb = (long long)b.slot * p.c_slot_stride + (long long)g * p.cap * HD;
        rk_c = make_rsrc(p.kc + cb, (long long)p.cap * HD * 2);
        rv_c = make_rsrc(p.vtc + cb, (long long)p.cap * HD * 2);
    }
    const rsrc_t rk_f = make_rsrc(p.kf + (long long)g * p.fcap * HD, (long long)p.fcap * HD * 2);
    const rsrc_t rv_f = make_rsrc(p.vtf + (long long)g * p.fcap * HD, (long long)p.fcap * HD * 2);

    /* this thread's staging chunks: global byte offset within the slab and LDS slot */
    unsigned g_off[PER], lk_off[PER], lv_off[PER];
    bool c_ok[PER];
#pragma unroll
    for (int e = 0; e < PER; e++) {
        const int q = tid + 256 * e;
        c_ok[e] = (CK % 256 == 0) || q < CK;
        const int kr = q / (HD / 8), cb = q - kr * (HD / 8);
        const int f = (kr & 3) | (((kr >> 3) & 3) << 2);
        lk_off[e] = (unsigned)(kr * KROW + 16 * (cb ^ f));
        const int d = q >> 2, jj = q & 3;
        lv_off[e] = (unsigned)(K_BYTES + d * 64 + 16 * (jj ^ ((d >> 1) & 3)));
        g_off[e] = c_ok[e] ? (unsigned)(q * 16) : OOB_OFF;
    }
    /* this lane's fragment addresses within a stage */
    const int kt_row = 8 * (c >> 2) + (c & 3);
    unsigned kfo[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ks++) kfo[ks] = (unsigned)(kt_row * KROW + 16 * ((4 * ks + j) ^ c));
    const unsigned vfo = (unsigned)(K_BYTES + c * 64 + 16 * (j ^ ((c >> 1) & 3)));

    struct Stg {
        uint4 k[PER], v[PER];
        bool bf; /* bf16 cache slab (widen to fp16 when storing) */
    };
    auto issue = [&](int k0, Stg &s) __attribute__((always_inline)) {
        const bool fr = k0 >= b.fresh_pos0;
        const int kr = fr ? k0 + it.fresh_off : k0;
        const unsigned so = (unsigned)(kr / SMOL_SLAB) * SLAB_BYTES;
        const rsrc_t rk = fr ? rk_f : rk_c, rv = fr ? rv_f : rv_c;
#pragma unroll
        for (int e = 0; e < PER; e++) s.k[e] = bload(rk, g_off[e], so);
#pragma unroll
        for (int e = 0; e < PER; e++) s.v[e] = bload(rv, g_off[e], so);
        s.bf = !fr;
    };
    auto store = [&](const Stg &s, int stage) __attribute__((always_inline)) {
        unsigned char *base = smem + stage * STAGE;
#pragma unroll
        for (int e = 0; e < PER; e++) {
            if (!c_ok[e]) continue;
            uint4 kw = s.k[e], vw = s.v[e];
            if (s.bf) {
                const h8 kh = bf16x8_to_h8(kw), vh = bf16x8_to_h8(vw);
                kw = *reinterpret_cast<const uint4 *>(&kh);
                vw = *reinterpret_cast<const uint4 *>(&vh);
            }
            *reinterpret_cast<uint4 *>(base + lk_off[e]) = kw;
            *reinterpret_cast<uint4 *>(base + lv_off[e]) = vw;
        }
    };
    auto lds_h8 = [&](int stage, unsigned off) __attribute__((always_inline)) -> h8 {
        const uint4 w = *reinterpret_cast<const uint4 *>(smem + stage * STAGE + off);
        return *reinterpret_cast<const h8 *>(&w);
    };
    /* S^T - m = K.Q^T - m of the slab in `stage` (raw S with a softcap) */
    const bool capped = p.cap2 > 0.0f;
    auto qk = [&](int stage, f4 (&sacc)[NT][2]) __attribute__((always_inline)) {
#pragma unroll
        for (int t = 0; t < 2; t++) {
            h8 kfr[KS];
#pragma unroll
            for (int ks = 0; ks < KS; ks++) kfr[ks] = lds_h8(stage, kfo[ks] + t * 4 * KROW);
#pragma unroll
            for (int nt = 0; nt < NT; nt++) {
                f4 acc = capped ? f4{0.f, 0.f, 0.f, 0.f} : negm[nt];
#pragma unroll
                for (int ks = 0; ks < KS; ks++)
                    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(kfr[ks], qf[nt][ks], acc, 0, 0, 0);
                sacc[nt][t] = acc;
            }
        }
    };
    /* softmax front: scores relative to the row reference m, softcap and
     * mask applied. m is lazy: while no score exceeds thr (2^8 above m) the
     * common path is one compare per score; otherwise the row max is formed
     * and O, l and m are rescaled */
    auto front = [&](int k0, const f4 (&sacc)[NT][2], float (&sv)[NT][8]) __attribute__((always_inline)) {
        const bool full = k0 >= lo_max && k0 + SMOL_SLAB <= hi_min;
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
#pragma unroll
            for (int t = 0; t < 2; t++)
#pragma unroll
                for (int i = 0; i < 4; i++) sv[nt][4 * t + i] = sacc[nt][t][i];
            if (capped) {
#pragma unroll
                for (int e = 0; e < 8; e++) sv[nt][e] = p.cap2 * tanhf(sv[nt][e] / p.cap2) + negm[nt][0];
            }
            if (!full) {
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    const int key = k0 + 8 * j + e;
                    sv[nt][e] = (key >= lo[nt] && key < hi[nt]) ? sv[nt][e] : -INFINITY;
                }
            }
            bool hit = sv[nt][0] > thr[nt];
#pragma unroll
            for (int e = 1; e < 8; e++) hit |= sv[nt][e] > thr[nt];
            if (__any(hit)) {
                const float mx = row_max4(fmaxf(fmaxf(fmaxf(sv[nt][0], sv[nt][1]), fmaxf(sv[nt][2], sv[nt][3])),
                                                fmaxf(fmaxf(sv[nt][4], sv[nt][5]), fmaxf(sv[nt][6], sv[nt][7]))));
                const bool need = mx > thr[nt];
                const float sh = need ? mx : 0.0f;
                const float m_new = need ? -negm[nt][0] + mx : m[nt];
                const float alpha = need ? __builtin_amdgcn_exp2f(m[nt] - m_new) : 1.0f;
#pragma unroll
                for (int dt = 0; dt < DT; dt++) o[nt][dt] *= alpha;
                l[nt] *= alpha;
                m[nt] = m_new;
                const float mu = m_new == -INFINITY ? 0.0f : m_new;
                negm[nt] = f4{-mu, -mu, -mu, -mu};
                thr[nt] = m_new == -INFINITY ? -INFINITY : LAZY_T;
#pragma unroll
                for (int e = 0; e < 8; e++) sv[nt][e] -= sh;
            }
        }
    };
    /* P = exp2(S - m) as fp16, row sums */
    auto expo = [&](const float (&sv)[NT][8], h8 (&pf)[NT]) __attribute__((always_inline)) {
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
            float pe[8];
#pragma unroll
            for (int e = 0; e < 8; e++) {
                pe[e] = __builtin_amdgcn_exp2f(sv[nt][e]);
                pf[nt][e] = (_Float16)pe[e];
            }
            l[nt] += ((pe[0] + pe[1]) + (pe[2] + pe[3])) + ((pe[4] + pe[5]) + (pe[6] + pe[7]));
        }
    };
    auto pv = [&](int stage, const h8 (&pf)[NT]) __attribute__((always_inline)) {
#pragma unroll
        for (int dt = 0; dt < DT; dt++) {
            const h8 vfr = lds_h8(stage, vfo + dt * 1024);
#pragma unroll
            for (int nt = 0; nt < NT; nt++)
                o[nt][dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vfr, pf[nt], o[nt][dt], 0, 0, 0);
        }
    };

    /* The item's n slabs are walked in a rotated order (slab (i + rot) mod n
     * at step i; the softmax does not depend on the order), so the
     * workgroups of one head, which start together, read different slabs.
     * Slab i sits in LDS stage i % 4 from the barrier that ends step i-2 to
     * the one that ends step i. Step i: softmax front of slab i; then its
     * exponentials alongside S of slab i+1 (MFMA and VALU work of the same
     * wave with no dependence between them); then P.V of slab i; then slab
     * i+2 is stored from its register set, which is refilled with slab
     * i+2+SETS. Loads and stores are issued unconditionally (clamped to the
     * last slab), so the waits are the same on every path. */
    const int kb = it.key_begin, ke = it.key_end;
    __syncthreads(); /* stages cleared */
    if (ke > kb) {
        const int n = (ke - kb + SMOL_SLAB - 1) / SMOL_SLAB;
        const int rot = (int)(((unsigned)item * 7u + (unsigned)g * 3u) % (unsigned)n);
        auto slab_k = [&](int i) __attribute__((always_inline)) {
            int r = (i < n ? i : n - 1) + rot;
            r = r >= n ? r - n : r;
            return kb + SMOL_SLAB * r;
        };
        Stg st[SETS];
#pragma unroll
        for (int q = 0; q < SETS; q++) issue(slab_k(q), st[q]);
        store(st[0], 0);
        issue(slab_k(SETS), st[0]);
        store(st[1], 1);
        issue(slab_k(SETS + 1), st[1]);
        __syncthreads();
        f4 sa[NT][2], sb[NT][2];
        qk(0, sa);
        /* u = i % 4, compile-time in each unrolled step */
        auto step = [&](int i, auto u_tag, f4 (&scur)[NT][2], f4 (&snext)[NT][2]) __attribute__((always_inline)) {
            constexpr int u = decltype(u_tag)::value;
            float sv[NT][8];
            h8 pf[NT];
            front(slab_k(i), scur, sv);
            qk((u + 1) & 3, snext);
            expo(sv, pf);
            pv(u, pf);
            Stg &s2 = st[(u + 2) % SETS];
            store(s2, (u + 2) & 3);
            issue(slab_k(i + 2 + SETS), s2);
            __syncthreads();
        };
        /* whole groups of four steps in a loop with one exit, then the last
         * one to four steps: a loop left from the middle of its body would
         * merge that exit's outstanding loads into the loop head, and the
         * head would wait for them on every pass */
        using P0 = std::integral_constant<int, 0>;
        using P1 = std::integral_constant<int, 1>;
        using P2 = std::integral_constant<int, 2>;
        using P3 = std::integral_constant<int, 3>;
        int i = 0;
        for (; i + 4 < n; i += 4) {
            step(i, P0{}, sa, sb);
            step(i + 1, P1{}, sb, sa);
            step(i + 2, P2{}, sa, sb);
            step(i + 3, P3{}, sb, sa);
        }
        step(i, P0{}, sa, sb);
        if (i + 1 < n) {
            step(i + 1, P1{}, sb, sa);
            if (i + 2 < n) {
                step(i + 2, P2{}, sa, sb);
                if (i + 3 < n) step(i + 3, P3{}, sb, sa);
            }
        }
    }

#pragma unroll
    for (int nt = 0; nt < NT; nt++) l[nt] = row_sum4(l[nt]);
    /* epilogue: each wave's rows are complete over the item's keys */
    if (it.n_split == 1) {
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
            const int r = it.row0 + (wave * NT + nt) * 16 + c;
            if (r >= b.n_rows) continue;
            const int qi = r / G, hg = r - qi * G;
            float *orow = p.out + ((long long)(b.out_tok0 + qi) * p.Hq + (g * G + hg)) * HD;
            const float inv = l[nt] > 0.0f ? 1.0f / l[nt] : 0.0f;
#pragma unroll
            for (int dt = 0; dt < DT; dt++) {
                const int d = 16 * dt + 4 * j;
                if (HD % 16 != 0 && d >= HD) continue;
                *reinterpret_cast<f4 *>(orow + d) = o[nt][dt] * inv;
            }
        }
        return;
    }
    /* split item: publish this wave's rows with device-coherent stores, then
     * the workgroup counts in once; the group's last workgroup merges */
    const long long pbase = ((long long)item * p.Hkv + g) * ROWS;
    {
        const rsrc_t ro = make_rsrc(p.part_o + pbase * HD, (long long)ROWS * HD * 4);
        const rsrc_t rml = make_rsrc(p.part_ml + pbase * 2, (long long)ROWS * 2 * 4);
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
            const int rr = (wave * NT + nt) * 16 + c;
#pragma unroll
            for (int dt = 0; dt < DT; dt++) {
                const int d = 16 * dt + 4 * j;
                if (HD % 16 != 0 && d >= HD) continue;
                store_f4_sc1(ro, (unsigned)((rr * HD + d) * 4), o[nt][dt]);
            }
            if (j == 0) store_f2_sc1(rml, (unsigned)(rr * 8), m[nt], l[nt]);
        }
    }
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __syncthreads(); /* every wave's stores are acknowledged */
    if (tid == 0) {
        const int prev = __hip_atomic_fetch_add(p.counters + ((long long)it.group * p.Hkv + g) * SK_COUNTER_STRIDE, 1, __ATOMIC_RELAXED,
                                                __HIP_MEMORY_SCOPE_AGENT);
        s_last = prev == it.n_split - 1;
    }
    __syncthreads();
    if (!s_last) return;
    merge_group<HD, ROWS>(p, it, b, item, g, tid, reinterpret_cast<float *>(smem));
}

/* ---------------------------------------------------------------- k_attn_fb */

/*
 * Prefill and windowed bidirectional attention over keys that all sit in the
 * fresh fp16 buffers (no cache slabs), for head_dim <= 128. One workgroup
 * owns one 64-row tile and needs no other workgroup: its waves form two
 * groups, the groups take the first and second half of the tile's key slabs,
 * and the two partial softmax states are merged through LDS at the end.
 * Within a group, wave w holds the NT row tiles 16 (w NT + t) .. +15 of the
 * 64-row tile (four waves of one tile, or two waves of two).
 *
 * Staging is direct-to-LDS: each wave issues buffer_load_dwordx4 ... lds for
 * its share of a slab (one 1 KB LDS region per instruction, 16 bytes per
 * lane, the lane's global chunk chosen so the region receives the swizzled
 * image below) into a ring of NSTG stages per group. No registers hold
 * staged data, which leaves room to double-buffer the MFMA fragments: the
 * fragments a step uses were read from LDS during the step before. Offsets
 * past the slab (padding of K rows and V^T rows past head_dim) are out of
 * range of the buffer and arrive as zeros.
 *
 * LDS image of a slab (as in k_attn_fa):
 *   K   : 32 key rows of KROW bytes; 16-byte chunk cb of key row r sits in
 *         slot cb ^ f(r), f(r) = (r & 3) | ((r >> 3) & 3) << 2.
 *   V^T : 16*DT rows of 64 bytes; chunk j of row d sits in slot
 *         j ^ ((d >> 1) & 3).
 * Step i of a group: the softmax front and exponentials of slab i run on
 * the vector ALU next to S = K.Q^T of slab i+1 on the matrix cores, then
 * P.V of slab i, while K of slab i+2 and V^T of slab i+1 are read from LDS;
 * then the transfer of slab i+3 is waited for and one barrier publishes it.
 */
/* WPG waves per key group, each holding NT 16-row tiles of the 64-row item */
template <int HD, int WPG>
struct FbGeom {
    static constexpr int KS = (HD + 31) / 32;
    static constexpr int DT = (HD + 15) / 16;
    static constexpr int HDP = KS * 32;
    static constexpr int KROW = 256;
    static constexpr int K_BYTES = SMOL_SLAB * KROW;
    static constexpr int V_BYTES = 16 * DT * 64;
    static constexpr int STAGE = (K_BYTES + V_BYTES + 1024 * WPG - 1) / (1024 * WPG) * (1024 * WPG);
    static constexpr int NDMA = STAGE / (1024 * WPG); /* DMA instructions per wave per slab */
    static constexpr int NSTG = 2 * 5 * STAGE <= 160 * 1024 ? 5 : 4;
    static constexpr int GROUP_BYTES = NSTG * STAGE;
};

/* NT = 1: four waves per key group (two per SIMD, 512 threads); NT = 2: two
 * waves per key group, each holding two row tiles (one wave per SIMD, 256
 * threads): every K / V^T fragment read from LDS then feeds two MFMAs, which
 * halves the LDS reads per flop. One MFMA pipe per SIMD is kept busy by a
 * single wave (measured: 16x16x32 f16 MFMAs with independent accumulators
 * issue at the same rate from one wave per SIMD as from two). */
template <int HD, int NT>
__global__ __launch_bounds__(NT == 1 ? 512 : 256)
__attribute__((amdgpu_waves_per_eu(NT == 1 ? 2 : 1, NT == 1 ? 2 : 1))) void k_attn_fb(SkParams p) {
    constexpr int WPG = 4 / NT;
    using Gm = FbGeom<HD, WPG>;
    constexpr int KS = Gm::KS, DT = Gm::DT, HDP = Gm::HDP, KROW = Gm::KROW;
    constexpr int K_BYTES = Gm::K_BYTES, STAGE = Gm::STAGE, NDMA = Gm::NDMA, NSTG = Gm::NSTG;
    constexpr int WAITN = (NSTG - 3) * NDMA; /* transfers that may stay outstanding at a step's end */
    constexpr unsigned SLAB_BYTES = SMOL_SLAB * HD * 2;
    static_assert(HD <= 128, "k_attn_fb covers head_dim <= 128");
    static_assert(2 * Gm::GROUP_BYTES <= 160 * 1024, "LDS");
    static_assert(NSTG >= 3, "the step pipeline keeps three slabs resident");
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int grp = wave / WPG, wg = wave % WPG;
    const int g = (int)(blockIdx.x % (unsigned)p.Hkv);
    const int w = (int)(blockIdx.x / (unsigned)p.Hkv);
    __shared__ __attribute__((aligned(1024))) unsigned char smem[2 * Gm::GROUP_BYTES];
    /* item w, then the rest of this workgroup's list (the host's
     * longest-first assignment when the items outnumber the compute units,
     * where a second wave of workgroups would pay its start-up again) */
    int item = w;
    for (;;) {
    /* lane terms are remade per item rather than held in registers across it */
    int lane = tid & 63;
    asm volatile("" : "+v"(lane));
    const int c = lane & 15, j = lane >> 4;
    const FbItem it = p.fb_items[item]; /* the batch's fields included: one round trip */
    const FbItem &b = it;
    const int next = it.next;
    const int G = p.G;
    unsigned char *gbase = smem + grp * Gm::GROUP_BYTES;
    const unsigned lds_group = (unsigned)(size_t)gbase;

    /* this group's slabs: the first or second half of the item's */
    const int n_all = (it.key_end - it.key_begin + SMOL_SLAB - 1) / SMOL_SLAB;
    const int n0 = (n_all + 1) >> 1;
    const int s_first = grp == 0 ? 0 : n0;
    const int n_own = grp == 0 ? n0 : n_all - n0;
    auto slab_k = [&](int i) __attribute__((always_inline)) {
        const int q = n_own > 0 ? s_first + (i < n_own ? i : n_own - 1) : 0;
        return it.key_begin + SMOL_SLAB * q;
    };

    /* DMA geometry: region q = wg + WPG e of a stage; lane offsets within
     * the slab. The first transfers go out before anything else is set up. */
    const rsrc_t rk = make_rsrc(p.kf + (long long)g * p.fcap * HD, (long long)p.fcap * HD * 2);
    const rsrc_t rv = make_rsrc(p.vtf + (long long)g * p.fcap * HD, (long long)p.fcap * HD * 2);
    unsigned d_off[NDMA];
    bool d_isk[NDMA];
#pragma unroll
    for (int e = 0; e < NDMA; e++) {
        const int q = wg + WPG * e;
        d_isk[e] = q * 1024 < K_BYTES;
        if (d_isk[e]) {
            const int kr = q * 4 + (lane >> 4), slot = lane & 15;
            const int cb = slot ^ ((kr & 3) | (((kr >> 3) & 3) << 2));
            d_off[e] = cb < HD / 8 ? (unsigned)((kr * HD + cb * 8) * 2) : OOB_OFF;
        } else {
            const int d = (q * 1024 - K_BYTES) / 64 + (lane >> 2), slot = lane & 3;
            const int jj = slot ^ ((d >> 1) & 3);
            d_off[e] = d < HD ? (unsigned)((d * SMOL_SLAB + jj * 8) * 2) : OOB_OFF;
        }
    }
    auto dma = [&](int k0, int stage) __attribute__((always_inline)) {
        const int kr = k0 + it.fresh_off; /* from the item: the transfers need no batch load */
        const unsigned so = (unsigned)(kr / SMOL_SLAB) * SLAB_BYTES;
#pragma unroll
        for (int e = 0; e < NDMA; e++)
            dma_1k(d_isk[e] ? rk : rv, d_off[e], so,
                   __builtin_amdgcn_readfirstlane(lds_group + stage * STAGE + (wg + WPG * e) * 1024));
    };
#pragma unroll
    for (int q = 0; q < NSTG; q++) dma(slab_k(q), q);

    /* rows of this wave (the same in both groups): tile nt holds rows
     * 16 (wg NT + nt) + c of the item */
    int lo[NT], hi[NT];
    bool valid[NT];
    h8 qf[NT][KS];
    int lo_max = -(1 << 30), hi_min = 1 << 30;
#pragma unroll
    for (int nt = 0; nt < NT; nt++) {
        const int r = it.row0 + (wg * NT + nt) * 16 + c;
        valid[nt] = r < b.n_rows;
        const int qi = r / G;
        int rl = b.key_lo, rh = b.key_hi;
        if (b.causal) {
            rh = min(rh, b.q_pos0 + qi + 1);
            if (p.window > 0) rl = max(rl, b.q_pos0 + qi - p.window + 1);
        }
        lo[nt] = valid[nt] ? rl : -(1 << 30);
        hi[nt] = valid[nt] ? rh : (1 << 30);
        lo_max = max(lo_max, lo[nt]);
        hi_min = min(hi_min, hi[nt]);
        const _Float16 *qrow =
            p.qs + (long long)g * p.qs_head_stride + (long long)(b.q_row0 + (valid[nt] ? r : 0)) * HDP;
#pragma unroll
        for (int ks = 0; ks < KS; ks++) qf[nt][ks] = valid[nt] ? load_h8(qrow + 32 * ks + 8 * j) : zero_h8();
    }
#pragma unroll
    for (int sh = 1; sh < 64; sh <<= 1) {
        lo_max = max(lo_max, __shfl_xor(lo_max, sh));
        hi_min = min(hi_min, __shfl_xor(hi_min, sh));
    }
    lo_max = __builtin_amdgcn_readfirstlane(lo_max);
    hi_min = __builtin_amdgcn_readfirstlane(hi_min);

    float m[NT], l[NT], thr[NT];
    f4 negm[NT];
    f4 o[NT][DT];
    /* the row sums on the matrix cores (one row tile per wave): one more
     * MFMA per step against a fragment of ones (every element of lsum is the
     * row's sum of its fp16 probabilities, the same weights the P.V product
     * uses) instead of seven vector adds */
    constexpr bool MSUM = HD <= 128 && NT == 1;
    f4 lsum[NT];
    h8 ones;
#pragma unroll
    for (int i = 0; i < 8; i++) ones[i] = (_Float16)1.0f;
#pragma unroll
    for (int nt = 0; nt < NT; nt++) {
        m[nt] = -INFINITY;
        l[nt] = 0.0f;
        lsum[nt] = f4{0.f, 0.f, 0.f, 0.f};
        thr[nt] = -INFINITY;
        negm[nt] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int dt = 0; dt < DT; dt++) o[nt][dt] = f4{0.f, 0.f, 0.f, 0.f};
    }

    const int kt_row = 8 * (c >> 2) + (c & 3);
    unsigned kfo[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ks++) kfo[ks] = (unsigned)(kt_row * KROW + 16 * ((4 * ks + j) ^ c));
    const unsigned vfo = (unsigned)(K_BYTES + c * 64 + 16 * (j ^ ((c >> 1) & 3)));
    auto lds_h8 = [&](int stage, unsigned off) __attribute__((always_inline)) -> h8 {
        const uint4 w = *reinterpret_cast<const uint4 *>(gbase + stage * STAGE + off);
        return *reinterpret_cast<const h8 *>(&w);
    };
    const bool capped = p.cap2 > 0.0f;
    auto read_k = [&](int stage, h8 (&kf)[2][KS]) __attribute__((always_inline)) {
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
            for (int ks = 0; ks < KS; ks++) kf[t][ks] = lds_h8(stage, kfo[ks] + t * 4 * KROW);
    };
    auto read_v = [&](int stage, h8 (&vf)[DT]) __attribute__((always_inline)) {
#pragma unroll
        for (int dt = 0; dt < DT; dt++) vf[dt] = lds_h8(stage, vfo + dt * 1024);
    };
    /* S^T - m = K.Q^T - m (raw S with a softcap) */
    auto qk = [&](const h8 (&kf)[2][KS], f4 (&sacc)[NT][2]) __attribute__((always_inline)) {
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
            for (int nt = 0; nt < NT; nt++) {
                f4 acc = capped ? f4{0.f, 0.f, 0.f, 0.f} : negm[nt];
#pragma unroll
                for (int ks = 0; ks < KS; ks++)
                    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf[t][ks], qf[nt][ks], acc, 0, 0, 0);
                sacc[nt][t] = acc;
            }
    };
    /* softmax front, in place on the scores: softcap, mask, lazy rescale as
     * in k_attn_fa (lane (c, j) holds keys 8j + 4t + i of row c in s[t][i]) */
    auto front = [&](int k0, bool act, f4 (&s)[NT][2]) __attribute__((always_inline)) {
        /* a step past the group's own slabs masks every key, so its
         * arithmetic adds nothing and needs no branch of its own */
        const bool full = act && k0 >= lo_max && k0 + SMOL_SLAB <= hi_min;
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
            if (capped) {
#pragma unroll
                for (int t = 0; t < 2; t++)
#pragma unroll
                    for (int i = 0; i < 4; i++) s[nt][t][i] = p.cap2 * tanhf(s[nt][t][i] / p.cap2) + negm[nt][0];
            }
            if (!full) {
#pragma unroll
                for (int t = 0; t < 2; t++)
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const int key = k0 + 8 * j + 4 * t + i;
                        s[nt][t][i] = (act && key >= lo[nt] && key < hi[nt]) ? s[nt][t][i] : -INFINITY;
                    }
            }
            bool hit = false;
#pragma unroll
            for (int t = 0; t < 2; t++)
#pragma unroll
                for (int i = 0; i < 4; i++) hit |= s[nt][t][i] > thr[nt];
            if (__any(hit)) {
                const float mx = row_max4(fmaxf(fmaxf(fmaxf(s[nt][0][0], s[nt][0][1]), fmaxf(s[nt][0][2], s[nt][0][3])),
                                                fmaxf(fmaxf(s[nt][1][0], s[nt][1][1]), fmaxf(s[nt][1][2], s[nt][1][3]))));
                const bool need = mx > thr[nt];
                const float sh = need ? mx : 0.0f;
                const float m_new = need ? -negm[nt][0] + mx : m[nt];
                const float alpha = need ? __builtin_amdgcn_exp2f(m[nt] - m_new) : 1.0f;
#pragma unroll
                for (int dt = 0; dt < DT; dt++) o[nt][dt] *= alpha;
                if constexpr (MSUM) lsum[nt] *= alpha;
                else l[nt] *= alpha;
                m[nt] = m_new;
                const float mu = m_new == -INFINITY ? 0.0f : m_new;
                negm[nt] = f4{-mu, -mu, -mu, -mu};
                thr[nt] = m_new == -INFINITY ? -INFINITY : LAZY_T;
#pragma unroll
                for (int t = 0; t < 2; t++) s[nt][t] -= sh;
            }
        }
    };
    /* P = exp2(S - m) as fp16, row sums */
    auto expo = [&](const f4 (&s)[NT][2], h8 (&pf)[NT]) __attribute__((always_inline)) {
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
            float pe[8];
#pragma unroll
            for (int e = 0; e < 8; e++) {
                pe[e] = __builtin_amdgcn_exp2f(s[nt][e >> 2][e & 3]);
                pf[nt][e] = (_Float16)pe[e];
            }
            if constexpr (!MSUM) l[nt] += ((pe[0] + pe[1]) + (pe[2] + pe[3])) + ((pe[4] + pe[5]) + (pe[6] + pe[7]));
        }
    };
    auto pv = [&](const h8 (&vf)[DT], const h8 (&pf)[NT]) __attribute__((always_inline)) {
#pragma unroll
        for (int dt = 0; dt < DT; dt++)
#pragma unroll
            for (int nt = 0; nt < NT; nt++)
                o[nt][dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf[dt], pf[nt], o[nt][dt], 0, 0, 0);
        if constexpr (MSUM) {
#pragma unroll
            for (int nt = 0; nt < NT; nt++) lsum[nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ones, pf[nt], lsum[nt], 0, 0, 0);
        }
    };

    /* Slab j of this group sits in stage j % NSTG. Its transfer is issued in
     * step j-NSTG (the prologue for j < NSTG) and waited for at the end of
     * step j-3. Step i computes the softmax of slab i, S of slab i+1 and P.V
     * of slab i. The K fragments of slab i+2 and the V^T fragments of slab
     * i+1 are read at the top of step i into the second register set, so
     * step i+1 starts from registers. Every wave issues NDMA transfers per
     * step: waiting until at most (NSTG-3)*NDMA are outstanding completes
     * slab i+3. Steps past the group's own slab count (the second group may
     * have one fewer, or none) keep the reads, transfers and barriers and
     * mask every key. */
    const int steps = n0;
    /* Slabs 0..NSTG-1 were requested (NDMA transfers each), then the Q
     * loads (NT * KS). Vector-memory loads, LDS transfers included, count
     * down vmcnt in the order they were issued, so waiting until WAITN
     * remain completes every transfer but the last WAITN issued: slabs
     * 0..NSTG-3 are in LDS (step 0 reads slabs 0, 1 and 2), and the barrier
     * extends that to every wave's transfers. (A stale 1 KB region on a
     * process's first call was the M0 hazard of dma_1k, fixed there.) */
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(WAITN) : "memory");
    __syncthreads();
    f4 sa[NT][2], sb[NT][2];
    h8 kfa[2][KS], kfb[2][KS], vfa[DT], vfb[DT];
    read_k(0, kfa);
    qk(kfa, sa);
    read_k(1, kfa);
    read_v(0, vfa);
    /* step 0 refills stage 0 with no barrier in between: V^T of slab 0 must
     * be in registers first. A transfer of a slab already in L2 can land
     * before LDS reads queued behind the other waves' reads are served. */
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    int st_k = 2 % NSTG, st_v = 1, st_d = 0; /* stages read in a step, stage refilled */
    auto step = [&](int i, f4 (&scur)[NT][2], f4 (&snext)[NT][2], auto &kcur, auto &knext, auto &vcur, auto &vnext)
        __attribute__((always_inline)) {
        const bool act = i < n_own;
        h8 pf[NT];
        /* the next step's LDS reads and the transfer of slab i+NSTG go out
         * first and proceed during this step's arithmetic, which works from
         * registers filled before the last barrier */
        read_k(st_k, knext);
        read_v(st_v, vnext);
        dma(slab_k(i + NSTG), st_d);
        __builtin_amdgcn_sched_barrier(0);
        front(slab_k(i), act, scur);
        qk(kcur, snext);
        expo(scur, pf);
        pv(vcur, pf);
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"(WAITN) : "memory");
        __syncthreads();
        st_k = st_k + 1 == NSTG ? 0 : st_k + 1;
        st_v = st_v + 1 == NSTG ? 0 : st_v + 1;
        st_d = st_d + 1 == NSTG ? 0 : st_d + 1;
    };
    int i = 0;
    for (; i + 2 <= steps; i += 2) {
        step(i, sa, sb, kfa, kfb, vfa, vfb);
        step(i + 1, sb, sa, kfb, kfa, vfb, vfa);
    }
    if (i < steps) step(i, sa, sb, kfa, kfb, vfa, vfb);
#pragma unroll
    for (int nt = 0; nt < NT; nt++) l[nt] = MSUM ? lsum[nt][0] : row_sum4(l[nt]);

    /* merge: group 1 hands its state to group 0 through LDS (lane-wise: the
     * two waves wg of the groups hold the same rows in the same lanes), one
     * row tile at a time */
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads(); /* every transfer has landed and every stage read is done */
    float *xo = reinterpret_cast<float *>(smem) + (wg * 64 + lane) * (4 * DT + 4);
#pragma unroll
    for (int nt = 0; nt < NT; nt++) {
        if (nt > 0) __syncthreads();
        if (grp == 1) {
#pragma unroll
            for (int dt = 0; dt < DT; dt++) *reinterpret_cast<f4 *>(xo + 4 * dt) = o[nt][dt];
            xo[4 * DT] = m[nt];
            xo[4 * DT + 1] = l[nt];
        }
        __syncthreads();
        if (grp == 1 || !valid[nt]) continue;
        const int r = it.row0 + (wg * NT + nt) * 16 + c;
        const int qi = r / G, hg = r - qi * G;
        const float m1 = xo[4 * DT], l1 = xo[4 * DT + 1];
        const float M = fmaxf(m[nt], m1);
        const float Mu = M == -INFINITY ? 0.0f : M;
        const float w0 = __builtin_amdgcn_exp2f(m[nt] - Mu), w1 = __builtin_amdgcn_exp2f(m1 - Mu);
        const float L = l[nt] * w0 + l1 * w1;
        const float inv = L > 0.0f ? 1.0f / L : 0.0f;
        const float a0 = w0 * inv, a1 = w1 * inv;
        float *orow = p.out + ((long long)(b.out_tok0 + qi) * p.Hq + (g * G + hg)) * HD;
#pragma unroll
        for (int dt = 0; dt < DT; dt++) {
            const int d = 16 * dt + 4 * j;
            if (HD % 16 != 0 && d >= HD) continue;
            const f4 o1 = *reinterpret_cast<const f4 *>(xo + 4 * dt);
            *reinterpret_cast<f4 *>(orow + d) = o[nt][dt] * a0 + o1 * a1;
        }
    }
    if (next < 0) break;
    item = next;
    __syncthreads(); /* the epilogue is done with LDS */
    } /* items */
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
static int launch_prep_hd(const PrepParams *pp, dim3 grid, hipStream_t st) {
    /* Q and the new K are rotated together or not at all (the host sets both flags from one table) */
    const int rk = (pp->rope_q && pp->rope_k) ? pp->rope_kind : SMOL_ROPE_OFF;
    /* one input type for Q and the new K/V (the host passes one dtype per call) */
    const bool bf = pp->kv_dtype == SMOL_IN_BF16;
    if (pp->kv_dtype != pp->q_dtype || pp->rope_q != pp->rope_k) return -1;
#define SMOL_PREP(BF, RK)                                                                        \
    do {                                                                                         \
        if (pp->q_norm || pp->k_norm) hipLaunchKernelGGL((k_prep<HD, BF, RK, true>), grid, dim3(256), 0, st, *pp); \
        else hipLaunchKernelGGL((k_prep<HD, BF, RK, false>), grid, dim3(256), 0, st, *pp);      \
    } while (0)
    if (rk == SMOL_ROPE_OFF) { if (bf) SMOL_PREP(true, SMOL_ROPE_OFF); else SMOL_PREP(false, SMOL_ROPE_OFF); }
    else if (rk == SMOL_ROPE_NEOX_K) { if (bf) SMOL_PREP(true, SMOL_ROPE_NEOX_K); else SMOL_PREP(false, SMOL_ROPE_NEOX_K); }
    else if (rk == SMOL_ROPE_INTERLEAVED_K) {
        if (bf) SMOL_PREP(true, SMOL_ROPE_INTERLEAVED_K); else SMOL_PREP(false, SMOL_ROPE_INTERLEAVED_K);
    } else return -1;
#undef SMOL_PREP
    return hipGetLastError() == hipSuccess ? 0 : -3;
}

extern "C" int smol_launch_prep(const PrepParams *pp, int n_blocks, hipStream_t st) {
    if (n_blocks <= 0) return 0;
    const dim3 grid(n_blocks * pp->Hkv);
    switch (pp->hd) {
    case 64: return launch_prep_hd<64>(pp, grid, st);
    case 72: return launch_prep_hd<72>(pp, grid, st);
    case 80: return launch_prep_hd<80>(pp, grid, st);
    case 96: return launch_prep_hd<96>(pp, grid, st);
    case 128: return launch_prep_hd<128>(pp, grid, st);
    case 256: return launch_prep_hd<256>(pp, grid, st);
    default: return -1;
    }
}

template <int HD, int NT, int W>
static void launch_dec_v(const SkParams *sp, dim3 grid, bool staged, hipStream_t st) {
    if (staged) hipLaunchKernelGGL((k_attn_dec<HD, NT, W, true>), grid, dim3(64 * SK_WAVES), 0, st, *sp);
    else hipLaunchKernelGGL((k_attn_dec<HD, NT, W, false>), grid, dim3(64 * SK_WAVES), 0, st, *sp);
}

template <int HD>
static int launch_dec_hd(const SkParams *sp, int n_items, int nt, int w, int nw, bool staged, hipStream_t st) {
    /* two waves per SIMD only where the registers allow it (one row tile,
     * head_dim <= 128); other requests run at one. nw = 8: eight waves per
     * workgroup (two per SIMD), for items that hold a whole sequence */
    const dim3 grid(n_items * sp->Hkv);
    if (nw == 8) {
        if constexpr (HD <= 128) {
            if (nt != 1 || w != 2 || staged) return -1;
            hipLaunchKernelGGL((k_attn_dec<HD, 1, 2, false, 8>), grid, dim3(64 * 8), 0, st, *sp);
            return hipGetLastError() == hipSuccess ? 0 : -3;
        }
        return -1;
    }
    if (nt == 1 && w == 2 && HD <= 128) launch_dec_v<HD, 1, (HD <= 128 ? 2 : 1)>(sp, grid, staged, st);
    else if (nt == 1) launch_dec_v<HD, 1, 1>(sp, grid, staged, st);
    else if (nt == 2 && HD <= 128) launch_dec_v<HD, (HD <= 128 ? 2 : 1), 1>(sp, grid, staged, st);
    else return -1;
    return hipGetLastError() == hipSuccess ? 0 : -3;
}

/* staged: every slab of an item goes to LDS in one round of direct
 * transfers (items of at most smol_dec_staged_slabs(hd) slabs) */
extern "C" int smol_launch_dec(const SkParams *sp, int hd, int n_items, int nt, int w, int nw, int staged,
                               hipStream_t st) {
    if (n_items <= 0) return 0;
    switch (hd) {
    case 64: return launch_dec_hd<64>(sp, n_items, nt, w, nw, staged != 0, st);
    case 72: return launch_dec_hd<72>(sp, n_items, nt, w, nw, staged != 0, st);
    case 80: return launch_dec_hd<80>(sp, n_items, nt, w, nw, staged != 0, st);
    case 96: return launch_dec_hd<96>(sp, n_items, nt, w, nw, staged != 0, st);
    case 128: return launch_dec_hd<128>(sp, n_items, nt, w, nw, staged != 0, st);
    case 256: return launch_dec_hd<256>(sp, n_items, nt, w, nw, staged != 0, st);
    default: return -1;
    }
}

template <int HD, int NT, int W>
static void launch_fa_v(const SkParams *sp, dim3 grid, hipStream_t st) {
    hipLaunchKernelGGL((k_attn_fa<HD, NT, W>), grid, dim3(256), 0, st, *sp);
}

/* w: waves per SIMD the kernel is built for (2 with fewer staged slabs) */
template <int HD>
static int launch_fa_hd(const SkParams *sp, int n_items, int nt, int w, hipStream_t st) {
    const dim3 grid(n_items * sp->Hkv);
    if (nt == 1 && w == 1) launch_fa_v<HD, 1, 1>(sp, grid, st);
    else if constexpr (HD <= 128) { /* two tiles or two waves per SIMD fit the registers */
        if (nt == 1 && w == 2) launch_fa_v<HD, 1, 2>(sp, grid, st);
        else if (nt == 2 && w == 1) launch_fa_v<HD, 2, 1>(sp, grid, st);
        else if (nt == 2 && w == 2) launch_fa_v<HD, 2, 2>(sp, grid, st);
        else return -1;
    } else return -1;
    return hipGetLastError() == hipSuccess ? 0 : -3;
}

extern "C" int smol_launch_fa(const SkParams *sp, int hd, int n_items, int nt, int w, hipStream_t st) {
    if (n_items <= 0) return 0;
    switch (hd) {
    case 64: return launch_fa_hd<64>(sp, n_items, nt, w, st);
    case 72: return launch_fa_hd<72>(sp, n_items, nt, w, st);
    case 80: return launch_fa_hd<80>(sp, n_items, nt, w, st);
    case 96: return launch_fa_hd<96>(sp, n_items, nt, w, st);
    case 128: return launch_fa_hd<128>(sp, n_items, nt, w, st);
    case 256: return launch_fa_hd<256>(sp, n_items, nt, w, st);
    default: return -1;
    }
}

template <int HD>
static int launch_fb_hd(const SkParams *sp, int n_items, int nt, hipStream_t st) {
    const int n_wg = sp->n_wg > 0 ? sp->n_wg : n_items; /* workgroups per kv head: the heads of the lists */
    if (nt == 1) hipLaunchKernelGGL((k_attn_fb<HD, 1>), dim3(n_wg * sp->Hkv), dim3(512), 0, st, *sp);
    else if (nt == 2) hipLaunchKernelGGL((k_attn_fb<HD, 2>), dim3(n_wg * sp->Hkv), dim3(256), 0, st, *sp);
    else return -1;
    return hipGetLastError() == hipSuccess ? 0 : -3;
}

/* k_attn_fb: one 64-row tile per item, every key in the fresh buffers; nt
 * row tiles per wave (512 threads for nt 1, 256 for nt 2); sp->n_wg
 * workgroups per kv head (0: one per item) each run their list of items */
extern "C" int smol_launch_fb(const SkParams *sp, int hd, int n_items, int nt, hipStream_t st) {
    if (n_items <= 0) return 0;
    switch (hd) {
    case 64: return launch_fb_hd<64>(sp, n_items, nt, st);
    case 72: return launch_fb_hd<72>(sp, n_items, nt, st);
    case 80: return launch_fb_hd<80>(sp, n_items, nt, st);
    case 96: return launch_fb_hd<96>(sp, n_items, nt, st);
    case 128: return launch_fb_hd<128>(sp, n_items, nt, st);
    default: return -1;
    }
}
