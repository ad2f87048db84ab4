/*
 * attn_device.h - device helpers shared by the gfx950 kernels of the attention
 * path (attn_prep.hip, attn_dec.hip, attn_fa.hip, attn_fb.hip): bf16 / fp16
 * conversions, 8-element loads, the RoPE chunk of the pre-pass, raw buffer
 * resources, the direct-to-LDS transfer, and the softmax-row reductions.
 *
 * Numerics: softmax state in fp32 and in log2 units (Q is pre-multiplied by
 * scale * log2 e, so exp(s - m) = exp2(s' - m')). MFMA operands are fp16:
 * bf16 -> fp16 is exact for |x| < 65504, and fp16 keeps 3 more mantissa bits
 * than bf16 for the rotated Q/K and the probabilities P, which is what keeps
 * the result within 2e-3 + 1e-2 |ref| of the fp32 reference on early causal
 * rows (bf16 operands do not).
 */
#ifndef SMOL_ATTN_DEVICE_H
#define SMOL_ATTN_DEVICE_H

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "attn_internal.h"

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef unsigned u4v __attribute__((ext_vector_type(4)));

/* Streaming 16-byte stores for outputs no later work of the same kernel
 * reads (staging, cache rows, attention outputs): non-temporal, so they
 * drain to memory as they are written instead of collecting in L2 for the
 * end-of-kernel write-back. */
__device__ __forceinline__ void st_stream(void *p, uint4 v) {
    __builtin_nontemporal_store(u4v{v.x, v.y, v.z, v.w}, reinterpret_cast<u4v *>(p));
}
__device__ __forceinline__ void st_stream(float *p, f4 v) { __builtin_nontemporal_store(v, reinterpret_cast<f4 *>(p)); }

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


__device__ __forceinline__ int rope_partner(int d, int hd, int kind) {
    if (kind == SMOL_ROPE_NEOX_K) { int half = hd >> 1; return d < half ? d + half : d - half; }
    if (kind == SMOL_ROPE_INTERLEAVED_K) return d ^ 1;
    return d;
}


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

/* The fp16 staging's range: a value that is not finite, or whose magnitude
 * reaches 65520 (which rounds to inf in fp16), raises the context's range
 * flag (read by smol_attn_ctx_synchronize). One plain store by every lane
 * that finds one. */
__device__ __forceinline__ void note_h_range(int *flag, const float *v) {
    bool bad = false;
#pragma unroll
    for (int i = 0; i < 8; i++) bad |= !(fabsf(v[i]) < 65520.0f);
    if (bad && flag) *flag = 1;
}

/* the same test on 8 bf16 values as loaded: |x| >= 65536 (the next bf16
 * above 65280) or not finite */
__device__ __forceinline__ bool bf16x8_out_of_h_range(uint4 w) {
    const uint32_t a[4] = {w.x, w.y, w.z, w.w};
    bool bad = false;
#pragma unroll
    for (int k = 0; k < 4; k++) bad |= (a[k] & 0x7FFFu) >= 0x4780u || ((a[k] >> 16) & 0x7FFFu) >= 0x4780u;
    return bad;
}

__device__ __forceinline__ uint4 pack_h8(const float *v) {
    h8 h;
#pragma unroll
    for (int i = 0; i < 8; i++) h[i] = (_Float16)v[i];
    return *reinterpret_cast<uint4 *>(&h);
}

/* 8 values as fp16 hi + lo: hi = fp16(v) (nearest even), lo = fp16(v - hi).
 * hi + lo carries about 22 significant bits of v (lo's own rounding; v - hi
 * is exact in fp32), so a product on hi / lo operands reproduces an fp32
 * product to about 2^-21 relative. */
__device__ __forceinline__ void pack_h8_hilo(const float *v, uint4 &hi, uint4 &lo) {
    h8 h, l;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        h[i] = (_Float16)v[i];
        l[i] = (_Float16)(v[i] - (float)h[i]);
    }
    hi = *reinterpret_cast<uint4 *>(&h);
    lo = *reinterpret_cast<uint4 *>(&l);
}

__device__ __forceinline__ void unpack_bf16x8(uint4 w, float *v) {
    const uint32_t a[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
        v[2 * i] = __uint_as_float(a[i] << 16);
        v[2 * i + 1] = __uint_as_float(a[i] & 0xFFFF0000u);
    }
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

/* fp16 hi + lo of two floats (the probabilities of the precise P.V):
 * hi = fp16_rne(p), lo = fp16_rne(p - hi). p - hi is exact in fp32 (hi is p
 * rounded to 11 bits), and v_fma_mix_f32 forms it straight from the packed
 * fp16 hi (-1 * hi + p, one rounding of an exact value), which saves the
 * unpacking of hi: per pair two packed conversions and two mixes. Both halves
 * come back packed as the MFMA operand holds them (element e in the low half
 * of dword e / 2). The kernels run with fp16 and fp32 denormals preserved, so
 * a denormal hi is read exactly. */
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void split_h2(float p0, float p1, uint32_t &hi, uint32_t &lo) {
    typedef _Float16 hv2 __attribute__((ext_vector_type(2)));
    typedef float fv2 __attribute__((ext_vector_type(2)));
    hi = __builtin_bit_cast(uint32_t, __builtin_convertvector((fv2){p0, p1}, hv2));
    float l0, l1;
    asm("v_fma_mix_f32 %0, %1, -1.0, %2 op_sel_hi:[1,0,0]" : "=v"(l0) : "v"(hi), "v"(p0));
    asm("v_fma_mix_f32 %0, %1, -1.0, %2 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(l1) : "v"(hi), "v"(p1));
    lo = __builtin_bit_cast(uint32_t, __builtin_convertvector((fv2){l0, l1}, hv2));
}
#pragma clang diagnostic pop

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

#endif
