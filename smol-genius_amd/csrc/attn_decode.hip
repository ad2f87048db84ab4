/*
 * attn_decode.hip - k_dec: decode and short chunks over the bf16 KV cache.
 *
 * This is the attention of common/kernels/attention.c:79-170 for at most 64
 * query rows per (sequence, kv head): the single-token step of
 * qkn_decoder_forward (common/decoder/qkn_decoder.c:641-677, with the RoPE and
 * cache append of :647-652 and the per-head norm of :640-644 fused in) and a
 * short chunked prefill (qkn_decoder.c:487-528) whose new rows k_prep has
 * already rotated and staged.
 *
 * Work split. A group is one (sequence, kv head); its keys are cut into
 * n_split contiguous slab ranges, one workgroup each, and the NW waves of a
 * workgroup take its 32-key slabs in turn (wave w: slabs w, w + NW, ...). A
 * wave requests its first slab before anything else and the next one as
 * soon as the current one's registers are consumed.
 *
 * Products. Cache slabs run v_mfma_f32_16x16x32_bf16 on the cache's bf16 bits
 * as loaded; precision comes from splitting the other operand into bf16 hi +
 * lo (Q = Qhi + Qlo, P = Phi + Plo, about 16 significant bits together):
 *   S^T = K.Q^T with K as the A operand, rows gathered as
 *         key(t, m) = 8 (m >> 2) + 4 t + (m & 3), so a lane's 8 scores are 8
 *         consecutive keys and the P.V product reads V^T with one 16-byte
 *         load per lane;
 *   O^T += V^T.P^T.
 * PACK (at most 8 query rows, the decode case G <= 8): the 16 columns of the
 * B operand hold Qhi of the rows in columns 0..7 and Qlo in 8..15, so one
 * MFMA forms both halves; the two are summed across lanes c and c + 8 with a
 * DPP row rotation (scores: every slab; outputs: once at the end). Without
 * PACK each 16-row tile takes separate hi and lo MFMAs. Fresh fp16 slabs
 * (chunk mode) are split into bf16 hi + lo in registers (exact).
 *
 * Softmax in log2 units with a lazy reference max (rescale only when a row's
 * max grows by more than 2^LAZY_T), as the other kernels.
 *
 * Decode mode (direct): the workgroup stages its Q rows, the table row of
 * the position, the norm weights and (last split) the new K and V rows into
 * LDS, normalises (per-head RMSNorm, rmsnorm.c:78-140 order of operations)
 * and rotates them once per workgroup (rope.c:68-164 arithmetic), and every
 * lane then takes its B fragments from LDS. The last split scores the new
 * key in fp32, appends its bf16 K row and V^T column to the cache, and adds
 * it to its softmax state with an exact max update.
 *
 * Merge without atomics. Each split combines its waves through LDS, stores
 * its partial (m, l, O) with device-coherent stores, waits for them, then
 * stores the call's epoch into its flag. The group's last split (placed by
 * the host after every other split of its XCD, so each split it waits for
 * was dispatched before it) polls the flags and merges. All splits of a
 * group run on one XCD, so flags and partials meet in that XCD's L2. A
 * merger whose flags do not all arrive within DEC_SPIN_LIMIT polls writes
 * NaN rows instead of waiting for ever and raises the context's merge flag,
 * which smol_attn_ctx_synchronize reports as SMOL_ATTN_ERR_TIMEOUT.
 */
#include "attn_device.h"

#include <hip/hip_ext.h>

namespace {

/* DPP row_ror:8: lane c of every 16-lane row receives lane c ^ 8's value */
__device__ __forceinline__ float ror8(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x128, 0xF, 0xF, false));
}

/* The split partials stay in the XCD's L2: every split of a group runs on
 * one XCD, whose L2 is the point of coherence for its compute units (their
 * L1s write through). Plain stores, acknowledged by L2 before the flag is
 * stored, and plain loads after the flag has been seen (the reading compute
 * unit has not touched those lines in this kernel, and its L1 starts the
 * kernel invalidated). The flag itself travels device-coherently (SC1 store,
 * agent-scope poll). */
__device__ __forceinline__ void store_f4_l2(rsrc_t r, unsigned voff, f4 v) {
    __builtin_amdgcn_raw_buffer_store_b128(u4v{__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]),
                                               __float_as_uint(v[3])},
                                           r, voff, 0, 0);
}
__device__ __forceinline__ void store_f2_l2(rsrc_t r, unsigned voff, float a, float b) {
    typedef unsigned u2v __attribute__((ext_vector_type(2)));
    __builtin_amdgcn_raw_buffer_store_b64(u2v{__float_as_uint(a), __float_as_uint(b)}, r, voff, 0, 0);
}
__device__ __forceinline__ f4 load_f4_l2(rsrc_t r, unsigned voff) {
    const u4v v = __builtin_amdgcn_raw_buffer_load_b128(r, voff, 0, 0);
    return f4{__uint_as_float(v[0]), __uint_as_float(v[1]), __uint_as_float(v[2]), __uint_as_float(v[3])};
}
__device__ __forceinline__ float2 load_f2_l2(rsrc_t r, unsigned voff) {
    typedef unsigned u2v __attribute__((ext_vector_type(2)));
    const u2v v = __builtin_amdgcn_raw_buffer_load_b64(r, voff, 0, 0);
    return make_float2(__uint_as_float(v[0]), __uint_as_float(v[1]));
}

/* a flag read for polling: an atomic load is issued on every call */
__device__ __forceinline__ unsigned poll_u32(const unsigned *f) {
    return __hip_atomic_load(f, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int HD>
struct DecGeom {
    static constexpr int KS = (HD + 31) / 32; /* 32-wide d chunks of a K fragment */
    static constexpr int DT = (HD + 15) / 16; /* 16-wide d tiles of the output */
    static constexpr int HDP = KS * 32;
    static constexpr unsigned SLAB_BYTES = SMOL_SLAB * HD * 2;
};

} // namespace

template <int HD, int NT, bool PACK, int NW, bool DIRECT>
__global__ __launch_bounds__(64 * NW) void k_dec(const DecParams p) {
    using Gm = DecGeom<HD>;
    constexpr int KS = Gm::KS, DT = Gm::DT, HDP = Gm::HDP;
    constexpr unsigned SLAB_BYTES = Gm::SLAB_BYTES;
    static_assert(!PACK || NT == 1, "PACK holds at most 8 rows in one tile");
    constexpr int TR = PACK ? 8 : 16 * NT;     /* query rows the kernel holds */
    constexpr int QSTR = HDP + 4;              /* LDS row of a staged / rotated row */
    constexpr int OSTR = DT * 16 + 4;          /* LDS row of a wave's output in the combine */
    constexpr int TPB = 64 * NW;

    const int tid = threadIdx.x;
    const int lane = tid & 63, c = lane & 15, j = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int bid = blockIdx.x;
    /* The item and, in the same round of loads, sequence `lane` in every
     * lane (the item names one of them; its fields are then read from that
     * lane), so the sequence costs no second memory round trip. A sequence
     * index past 63 is loaded after the item. */
    static_assert(sizeof(DecItem) == 8 && sizeof(DecSeq) == 16, "item / sequence records");
    const DecSeq *seqs = p.seqs_dev ? p.seqs_dev : p.seqs;
    const uint2 iw = reinterpret_cast<const uint2 *>(p.n_items <= DEC_ARG_ITEMS ? p.items : p.items_dev)[bid];
    const int4 sl = reinterpret_cast<const int4 *>(seqs)[min(lane, max(p.n_seq - 1, 0))];
    /* both loads are in flight before either is used (the compiler would
     * otherwise issue the second after the test of the first) */
    asm volatile("" ::"v"(iw.x), "v"(iw.y), "v"(sl.x), "v"(sl.y), "v"(sl.z), "v"(sl.w));
    /* the item and its sequence are wave-uniform: keep them in scalar
     * registers (DecItem: seq 16 bits, kvh, rb, split, n_split 8 bits) */
    const int seq = (int)(short)(__builtin_amdgcn_readfirstlane((int)iw.x) & 0xFFFF);
    if (seq < 0) return;
    const int g = (__builtin_amdgcn_readfirstlane((int)iw.x) >> 16) & 0xFF;
    const int rb = (int)((unsigned)__builtin_amdgcn_readfirstlane((int)iw.x) >> 24);
    const int split = __builtin_amdgcn_readfirstlane((int)iw.y) & 0xFF;
    const int n_split = (__builtin_amdgcn_readfirstlane((int)iw.y) >> 8) & 0xFF;
    DecSeq sq;
    if (seq < 64) {
        sq.pos = __builtin_amdgcn_readlane(sl.x, seq);
        sq.slot = __builtin_amdgcn_readlane(sl.y, seq);
        sq.tok0 = __builtin_amdgcn_readlane(sl.z, seq);
        sq.n_q = __builtin_amdgcn_readlane(sl.w, seq);
    } else {
        const DecSeq sq0 = seqs[seq];
        sq.pos = __builtin_amdgcn_readfirstlane(sq0.pos);
        sq.slot = __builtin_amdgcn_readfirstlane(sq0.slot);
        sq.tok0 = __builtin_amdgcn_readfirstlane(sq0.tok0);
        sq.n_q = __builtin_amdgcn_readfirstlane(sq0.n_q);
    }
    /* this launch's flag value (see DecParams::step_dev) */
    const unsigned epoch = p.step_dev ? (__builtin_amdgcn_readfirstlane(*p.step_dev) << 8) + p.epoch : p.epoch;
    const int G = p.G;
    const int r_base = rb * TR;                   /* first row of this row block */
    const int R = min(TR, sq.n_q * G - r_base);   /* its real rows */
    const bool last_split = split == n_split - 1;

    /* the group's slab keys: decode [lo, pos) plus the new key apart; chunk
     * [lo, pos + n_q); lo: the lowest row's window start, slab-aligned */
    const int kend = DIRECT ? sq.pos : sq.pos + sq.n_q;
    const int klo = (p.window > 0 ? max(0, sq.pos - p.window + 1) : 0) & ~(SMOL_SLAB - 1);
    const int n_slabs = kend > klo ? (kend - klo + SMOL_SLAB - 1) / SMOL_SLAB : 0;
    const int per = (n_slabs + n_split - 1) / n_split;
    const int kb = klo + split * per * SMOL_SLAB;
    const int ke = min(kend, kb + per * SMOL_SLAB);

    /* sources: the (slot, head) region of the cache, the head's fresh region */
    const long long cbase = (long long)sq.slot * p.c_slot_stride + (long long)g * p.cap * HD;
    const uint16_t *kc_base = p.kc + cbase, *vc_base = p.vtc + cbase;
    const long long c_bytes = (long long)p.cap * HD * 2;
    const int fresh_pos0 = DIRECT ? (1 << 30) : p.fresh_pos0;
    const _Float16 *kf_base = DIRECT ? nullptr : p.kf + (long long)g * p.fcap * HD;
    const _Float16 *vf_base = DIRECT ? nullptr : p.vtf + (long long)g * p.fcap * HD;
    const long long f_bytes = DIRECT ? 0 : (long long)p.fcap * HD * 2;
    const int kt_row = 8 * (c >> 2) + (c & 3);
    const unsigned kbase = HD % 32 == 0 ? (unsigned)((kt_row * HD + 8 * j) * 2) : 0u;
    const unsigned vbase = HD % 16 == 0 ? (unsigned)((c * SMOL_SLAB + 8 * j) * 2) : 0u;
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
    struct KRaw { uint4 k[2][KS]; };
    struct VRaw { uint4 v[DT]; };
    /* The resource of the slab at key k0: the cache or the fresh staging; a
     * slab at or past ke (a request made ahead of need that turns out to be
     * past the wave's range) gets an empty range, so its loads return zeros
     * without touching memory. Requests are then unconditional, and the
     * compiler's wait counts are the same on every path. */
    auto slab_src = [&](int k0, bool value, rsrc_t &r, unsigned &so) __attribute__((always_inline)) {
        const bool live = k0 < ke;
        const bool fr = !DIRECT && k0 >= fresh_pos0;
        const int kr = fr ? k0 - fresh_pos0 + p.fresh_row0 : k0;
        so = live ? (unsigned)(kr / SMOL_SLAB) * SLAB_BYTES : 0u;
        const void *base = value ? (fr ? (const void *)vf_base : (const void *)vc_base)
                                 : (fr ? (const void *)kf_base : (const void *)kc_base);
        r = make_rsrc(base, live ? (fr ? f_bytes : c_bytes) : 0);
    };
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
    /* chunk mode, a fresh slab: its K's fp16 lo part (zeros without one) */
    auto issue_klo = [&](int k0, KRaw &r) __attribute__((always_inline)) {
        const int kr = k0 - fresh_pos0 + p.fresh_row0;
        const unsigned so = (unsigned)(kr / SMOL_SLAB) * SLAB_BYTES;
        const bool has = !DIRECT && p.kf_lo != nullptr;
        const rsrc_t rs = make_rsrc(has ? p.kf_lo + (long long)g * p.fcap * HD : nullptr, has && k0 < ke ? f_bytes : 0);
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

    /* LDS: staged rows / rotated Q (decode), then the combine and the merge */
    constexpr int ST_ROWS = TR + 1;                               /* Q rows + the new key */
    constexpr int ST_FLOATS = ST_ROWS * QSTR * 2 + 6 * HDP + 2 * TR + 64;
    constexpr int CB_FLOATS = (NW - 1) * TR * OSTR + 2 * (NW - 1) * TR;
    constexpr int MG_FLOATS = 3 * DEC_MAX_SPLIT * TR + TR + TR * OSTR + 4 * TPB;
    constexpr int SM_FLOATS = ST_FLOATS > CB_FLOATS ? (ST_FLOATS > MG_FLOATS ? ST_FLOATS : MG_FLOATS)
                                                    : (CB_FLOATS > MG_FLOATS ? CB_FLOATS : MG_FLOATS);
    static_assert(SM_FLOATS * 4 <= 160 * 1024, "LDS");
    __shared__ __attribute__((aligned(16))) float smem[SM_FLOATS];

    /* ---- Q fragments ---- */
    b8 qf[PACK ? KS : 1];             /* PACK: column c < 8 holds Qhi of row c, c >= 8 Qlo of row c - 8 */
    b8 qh[PACK ? 1 : NT][KS], ql[PACK ? 1 : NT][KS];
    float s_new = 0.0f;               /* decode, last split: this lane's row's score of the new key */
    float *s_raw = smem;                          /* [ST_ROWS][QSTR] staged inputs */
    float *s_rot = smem + ST_ROWS * QSTR;         /* [ST_ROWS][QSTR] normalised, rotated (Q scaled) */
    float *s_cos = s_rot + ST_ROWS * QSTR, *s_sin = s_cos + HDP;
    float *s_wq = s_sin + HDP, *s_wk = s_wq + HDP, *s_vnew = s_wk + HDP;
    float *s_rinv = s_vnew + HDP;                 /* [ST_ROWS] */
    float *s_snew = s_rinv + ST_ROWS + 1;         /* [TR] */
    auto ld8 = [&](const float *a, float *v) __attribute__((always_inline)) {
        const float4 x = *reinterpret_cast<const float4 *>(a), y = *reinterpret_cast<const float4 *>(a + 4);
        v[0] = x.x; v[1] = x.y; v[2] = x.z; v[3] = x.w; v[4] = y.x; v[5] = y.y; v[6] = y.z; v[7] = y.w;
    };
    int k0 = kb + wave * SMOL_SLAB;
    KRaw kr;
    VRaw vr;
    if constexpr (DIRECT) {
        const bool bf_in = p.in_dtype == SMOL_IN_BF16;
        const bool rope = p.rope_kind != SMOL_ROPE_OFF;
        const int n_rows = R + (last_split ? 1 : 0); /* row R: the new key */
        /* 1. Every staging load of the workgroup goes out in one round, then
         * this wave's first slab; the staged values reach LDS as soon as they
         * return (their loads are older than the slab's, and loads return in
         * order). The loads are unconditional: a lane with nothing to fetch
         * reads a valid dummy address and discards it, so no branch splits
         * the round (the compiler would wait for each load in turn). Chunks
         * of 8 elements: one 16-byte load of bf16, two of fp32. */
        constexpr int CH8 = HD / 8;
        constexpr int NQC = (TR * CH8 + TPB - 1) / TPB; /* Q-row chunks per thread */
        static_assert(6 * CH8 <= TPB, "one chunk of the single-row sources per thread");
        const char *dummy = reinterpret_cast<const char *>(p.q_in);
        const unsigned esz = bf_in ? 2u : 4u;
        uint4 qa[NQC], qb[NQC];
#pragma unroll
        for (int u = 0; u < NQC; u++) {
            const int e = tid + TPB * u, r = e / CH8, d0 = (e - r * CH8) * 8;
            const bool ok = r < R;
            const int qi = (r_base + r) / G, hg = (r_base + r) - qi * G;
            const long long idx = (long long)(sq.tok0 + qi) * p.q_stride + (long long)(g * G + hg) * HD + d0;
            const char *a = ok ? reinterpret_cast<const char *>(p.q_in) + idx * esz : dummy;
            qa[u] = *reinterpret_cast<const uint4 *>(a);
            qb[u] = *reinterpret_cast<const uint4 *>(ok && !bf_in ? a + 16 : dummy);
        }
        /* the single-row sources, thread t: source t / CH8, chunk t % CH8:
         * 0 new K, 1 new V (last split), 2 cos, 3 sin (RoPE), 4 q_norm,
         * 5 k_norm (last split) */
        const int sseg = tid / CH8, sd0 = (tid - sseg * CH8) * 8;
        const long long kv_idx = (long long)sq.tok0 * p.kv_stride + (long long)g * HD + sd0;
        const bool s_in = sseg <= 1; /* an input row (bf16 or fp32), else an fp32 table row */
        const void *sbase = sseg == 0 ? p.k_in : sseg == 1 ? p.v_in : sseg == 2 ? (const void *)p.rope_cos
                          : sseg == 3 ? (const void *)p.rope_sin : sseg == 4 ? (const void *)p.q_norm
                                                                             : (const void *)p.k_norm;
        const long long sidx = s_in ? kv_idx : (sseg <= 3 ? (long long)sq.pos * HD + sd0 : (long long)sd0);
        const bool s_ok = sseg <= 1 ? last_split : sseg <= 3 ? rope : sseg == 4 ? p.q_norm != nullptr
                        : sseg == 5 ? (p.k_norm != nullptr && last_split) : false;
        const bool s_f32 = !s_in || !bf_in;
        const char *sa = s_ok ? reinterpret_cast<const char *>(sbase) + sidx * (s_f32 ? 4 : 2) : dummy;
        const uint4 sa0 = *reinterpret_cast<const uint4 *>(sa);
        const uint4 sa1 = *reinterpret_cast<const uint4 *>(s_ok && s_f32 ? sa + 16 : dummy);
        /* Every wave's staging loads are queued before any wave's slab loads
         * (a compute unit returns its waves' data in request order, so a
         * slab requested first would delay the other waves' staging by its
         * whole transfer). The barrier orders only the requests: nothing
         * here waits for their data. */
        __builtin_amdgcn_s_barrier();
        issue_k(k0, kr);
        issue_v(k0, vr);
        auto unpack8 = [&](uint4 a, uint4 b, bool f32, float *v) __attribute__((always_inline)) {
            if (f32) {
                v[0] = __uint_as_float(a.x); v[1] = __uint_as_float(a.y); v[2] = __uint_as_float(a.z);
                v[3] = __uint_as_float(a.w); v[4] = __uint_as_float(b.x); v[5] = __uint_as_float(b.y);
                v[6] = __uint_as_float(b.z); v[7] = __uint_as_float(b.w);
            } else {
                unpack_bf16x8(a, v);
            }
        };
        auto st8 = [&](float *dst, const float *v) __attribute__((always_inline)) {
            *reinterpret_cast<float4 *>(dst) = make_float4(v[0], v[1], v[2], v[3]);
            *reinterpret_cast<float4 *>(dst + 4) = make_float4(v[4], v[5], v[6], v[7]);
        };
#pragma unroll
        for (int u = 0; u < NQC; u++) {
            const int e = tid + TPB * u, r = e / CH8, d0 = (e - r * CH8) * 8;
            if (r < R) {
                float v[8];
                unpack8(qa[u], qb[u], !bf_in, v);
                st8(s_raw + r * QSTR + d0, v);
            }
        }
        if (s_ok) {
            float v[8];
            unpack8(sa0, sa1, s_f32, v);
            float *dst = sseg == 0 ? s_raw + R * QSTR : sseg == 1 ? s_vnew : sseg == 2 ? s_cos
                       : sseg == 3 ? s_sin : sseg == 4 ? s_wq : s_wk;
            st8(dst + sd0, v);
        }
        __syncthreads();
        /* 2. 1 / rms of each row: eight lanes per row, lane j summing the
         * 8-element chunks j, j + 8, ..., then a butterfly */
        const bool nq = p.q_norm != nullptr, nk = p.k_norm != nullptr;
        constexpr int CH = HD / 8; /* 8-element chunks of a row */
        auto row_dot8 = [&](const float *a, const float *b, int jj) __attribute__((always_inline)) {
            float sd = 0.0f;
            /* loops of this staging phase have compile-time trip counts and
             * unroll: a loop here would make the compiler wait for every
             * outstanding load (the first slab's too) before entering it */
#pragma unroll
            for (int ci = 0; ci < (CH + 7) / 8; ci++) {
                const int ch = jj + 8 * ci;
                if (ch >= CH) break;
                float x[8], y[8];
                ld8(a + 8 * ch, x);
                ld8(b + 8 * ch, y);
#pragma unroll
                for (int i = 0; i < 8; i++) sd = fmaf(x[i], y[i], sd);
            }
            sd += __shfl_xor(sd, 1, 8);
            sd += __shfl_xor(sd, 2, 8);
            sd += __shfl_xor(sd, 4, 8);
            return sd;
        };
        if (nq || nk) {
#pragma unroll
            for (int ri = 0; ri < (TR + 1 + TPB / 8 - 1) / (TPB / 8); ri++) {
                const int r0 = ri * (TPB / 8);
                if (r0 >= n_rows) break;
                const int r = min(r0 + (tid >> 3), n_rows - 1);
                const float ss = row_dot8(s_raw + r * QSTR, s_raw + r * QSTR, tid & 7);
                if (r0 + (tid >> 3) < n_rows && (tid & 7) == 0) s_rinv[r] = 1.0f / sqrtf(ss / (float)HD + p.norm_eps);
            }
            __syncthreads();
        }
        /* 3. normalise, rotate (Q also scaled) into s_rot, 8 elements a thread;
         * the new key's bf16 row and its value's V^T column go to the cache
         * (one row block writes them) */
        constexpr int CHP = HDP / 8;
#pragma unroll
        for (int ei = 0; ei < ((TR + 1) * CHP + TPB - 1) / TPB; ei++) {
            const int e = tid + ei * TPB;
            if (e >= n_rows * CHP) break;
            const int r = e / CHP, d0 = (e - r * CHP) * 8;
            const bool is_k = r >= R;
            float y[8] = {0, 0, 0, 0, 0, 0, 0, 0};
            if (d0 < HD) {
                const float *row = s_raw + r * QSTR;
                const float *w = is_k ? (nk ? s_wk : nullptr) : (nq ? s_wq : nullptr);
                const float ri = w ? s_rinv[r] : 1.0f;
                float x[8];
                ld8(row + d0, x);
                if (w) {
                    float wv[8];
                    ld8(w + d0, wv);
#pragma unroll
                    for (int i = 0; i < 8; i++) x[i] = (x[i] * wv[i]) * ri;
                }
                if (!rope) {
#pragma unroll
                    for (int i = 0; i < 8; i++) y[i] = x[i];
                } else {
                    float cv[8], sv[8];
                    ld8(s_cos + d0, cv);
                    ld8(s_sin + d0, sv);
                    if (p.rope_kind == SMOL_ROPE_INTERLEAVED_K) {
#pragma unroll
                        for (int i = 0; i < 8; i += 2) {
                            y[i] = x[i] * cv[i] - x[i + 1] * sv[i];
                            y[i + 1] = x[i + 1] * cv[i + 1] + x[i] * sv[i + 1];
                        }
                    } else {
                        constexpr int HALF = HD / 2;
                        float pr[8];
                        if constexpr (HALF % 8 == 0) {
                            const int p0 = d0 < HALF ? d0 + HALF : d0 - HALF;
                            ld8(row + p0, pr);
                            if (w) {
                                float wp[8];
                                ld8(w + p0, wp);
#pragma unroll
                                for (int i = 0; i < 8; i++) pr[i] = (pr[i] * wp[i]) * ri;
                            }
                        } else {
#pragma unroll
                            for (int i = 0; i < 8; i++) {
                                const int d = d0 + i, pd = d < HALF ? d + HALF : d - HALF;
                                pr[i] = w ? (row[pd] * w[pd]) * ri : row[pd];
                            }
                        }
                        /* NeoX: x1 c - x2 s for the first half, x2 c + x1 s for the
                         * second (rope.c:99-164, fmsub / fmadd) */
#pragma unroll
                        for (int i = 0; i < 8; i++)
                            y[i] = d0 + i < HALF ? fmaf(x[i], cv[i], -(pr[i] * sv[i])) : fmaf(x[i], cv[i], pr[i] * sv[i]);
                    }
                }
                /* the new key's row stays in s_rot (row R): it joins the
                 * cache after the slab loop (this call reads keys [klo, pos)
                 * from the cache and the new one from LDS; a store here
                 * would sit among the slab loads and blur the compiler's
                 * count of them) */
                if (!is_k) {
#pragma unroll
                    for (int i = 0; i < 8; i++) y[i] *= p.qscale;
                }
            }
            *reinterpret_cast<float4 *>(s_rot + r * QSTR + d0) = make_float4(y[0], y[1], y[2], y[3]);
            *reinterpret_cast<float4 *>(s_rot + r * QSTR + d0 + 4) = make_float4(y[4], y[5], y[6], y[7]);
        }
        __syncthreads();
        /* 4. the new key's fp32 score against every row (last split) */
        if (last_split) {
#pragma unroll
            for (int ri = 0; ri < (TR + TPB / 8 - 1) / (TPB / 8); ri++) {
                const int r0 = ri * (TPB / 8);
                if (r0 >= R) break;
                const int r = min(r0 + (tid >> 3), R - 1);
                const float sd = row_dot8(s_rot + r * QSTR, s_rot + R * QSTR, tid & 7);
                if (r0 + (tid >> 3) < R && (tid & 7) == 0) s_snew[r] = sd;
            }
        }
        /* 5. B fragments from the rotated rows */
        if constexpr (PACK) {
            const int r = c & 7;
#pragma unroll
            for (int ks = 0; ks < KS; ks++) {
                b8 hi, lo;
                float v[8] = {0, 0, 0, 0, 0, 0, 0, 0};
                if (r < R) ld8(s_rot + r * QSTR + 32 * ks + 8 * j, v);
                split8(v, hi, lo);
                qf[ks] = c < 8 ? hi : lo;
            }
        } else {
#pragma unroll
            for (int nt = 0; nt < NT; nt++) {
                const int r = nt * 16 + c;
#pragma unroll
                for (int ks = 0; ks < KS; ks++) {
                    float v[8] = {0, 0, 0, 0, 0, 0, 0, 0};
                    if (r < R) ld8(s_rot + r * QSTR + 32 * ks + 8 * j, v);
                    split8(v, qh[nt][ks], ql[nt][ks]);
                }
            }
        }
        __syncthreads(); /* s_snew complete */
        if (last_split && PACK) s_new = (c & 7) < R ? s_snew[c & 7] : 0.0f;
    } else {
        /* chunk mode: Q rows from the fp32 scratch (k_prep rotated and
         * scaled them). All Q loads, then the first slab's, go out before
         * any is used, unconditionally (a lane past the real rows reads row
         * 0 and drops it), so the loop starts with only the slab loads
         * outstanding and the Q latency overlaps the slab's. */
        const float *qbase = p.qs32 + (long long)g * p.qs_head_stride;
        auto qrow = [&](int r) { return qbase + (long long)(sq.tok0 * G + r_base + r) * HDP; };
        constexpr int QT = PACK ? 1 : NT;
        float4 qa[QT][KS], qb[QT][KS];
#pragma unroll
        for (int nt = 0; nt < QT; nt++) {
            const int r = PACK ? (c & 7) : nt * 16 + c;
            const float *row = qrow(r < R ? r : 0);
#pragma unroll
            for (int ks = 0; ks < KS; ks++) {
                qa[nt][ks] = *reinterpret_cast<const float4 *>(row + 32 * ks + 8 * j);
                qb[nt][ks] = *reinterpret_cast<const float4 *>(row + 32 * ks + 8 * j + 4);
            }
        }
        issue_k(k0, kr);
        issue_v(k0, vr);
#pragma unroll
        for (int nt = 0; nt < QT; nt++) {
            const int r = PACK ? (c & 7) : nt * 16 + c;
#pragma unroll
            for (int ks = 0; ks < KS; ks++) {
                const float4 a = qa[nt][ks], e = qb[nt][ks];
                float v[8] = {a.x, a.y, a.z, a.w, e.x, e.y, e.z, e.w};
                if (r >= R) {
#pragma unroll
                    for (int i = 0; i < 8; i++) v[i] = 0.0f;
                }
                if constexpr (PACK) {
                    b8 hi, lo;
                    split8(v, hi, lo);
                    qf[ks] = c < 8 ? hi : lo;
                } else {
                    split8(v, qh[nt][ks], ql[nt][ks]);
                }
            }
        }
    }

    /* ---- row ranges (visible keys of each row this lane holds) ---- */
    constexpr int NR = PACK ? 1 : NT;
    int lo[NR], hi[NR];
    float m[NR], l[NR];
    f4 o[NR][DT];
    int lo_max = -(1 << 30), hi_min = 1 << 30;
#pragma unroll
    for (int nt = 0; nt < NR; nt++) {
        const int r = PACK ? (c & 7) : nt * 16 + c;
        const bool valid = r < R;
        const int qi = (r_base + r) / G;
        int rl = 0, rh = kend;
        if (!DIRECT) rh = min(rh, sq.pos + qi + 1);
        if (p.window > 0) rl = max(0, sq.pos + qi - p.window + 1);
        lo[nt] = valid ? rl : -(1 << 30);
        hi[nt] = valid ? rh : (1 << 30);
        lo_max = max(lo_max, lo[nt]);
        hi_min = min(hi_min, hi[nt]);
        m[nt] = -INFINITY;
        l[nt] = 0.0f;
#pragma unroll
        for (int dt = 0; dt < DT; dt++) o[nt][dt] = f4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int sh = 1; sh < 16; sh <<= 1) {
        lo_max = max(lo_max, __shfl_xor(lo_max, sh));
        hi_min = min(hi_min, __shfl_xor(hi_min, sh));
    }
    lo_max = __builtin_amdgcn_readfirstlane(lo_max);
    hi_min = __builtin_amdgcn_readfirstlane(hi_min);

    /* ---- S^T = K.Q^T of one slab: sacc[nr][t] ---- */
    auto qk = [&](const KRaw &r, const KRaw &rl, f4 (&sacc)[NR][2], auto fresh_tag) __attribute__((always_inline)) {
        constexpr bool FRESH = decltype(fresh_tag)::value;
#pragma unroll
        for (int t = 0; t < 2; t++) {
#pragma unroll
            for (int nt = 0; nt < NR; nt++) {
                f4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int ks = 0; ks < KS; ks++) {
                    /* the fresh slab's K (fp16 hi + fp16 lo, exact in fp32)
                     * as bf16 hi + lo: 16 significant bits */
                    b8 khs, kls;
                    if constexpr (FRESH) {
                        float kx[8];
                        const h8 k16 = *reinterpret_cast<const h8 *>(&r.k[t][ks]);
                        const h8 kl16 = *reinterpret_cast<const h8 *>(&rl.k[t][ks]);
#pragma unroll
                        for (int i = 0; i < 8; i++) kx[i] = (float)k16[i] + (float)kl16[i];
                        split8(kx, khs, kls);
                    }
                    if constexpr (PACK) {
                        if constexpr (FRESH) {
                            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(khs, qf[ks], acc, 0, 0, 0);
                            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kls, qf[ks], acc, 0, 0, 0);
                        } else {
                            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_b8(r.k[t][ks]), qf[ks], acc, 0, 0, 0);
                        }
                    } else {
                        if constexpr (FRESH) {
                            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(khs, qh[nt][ks], acc, 0, 0, 0);
                            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(khs, ql[nt][ks], acc, 0, 0, 0);
                            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kls, qh[nt][ks], acc, 0, 0, 0);
                        } else {
                            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_b8(r.k[t][ks]), qh[nt][ks], acc, 0, 0, 0);
                            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_b8(r.k[t][ks]), ql[nt][ks], acc, 0, 0, 0);
                        }
                    }
                }
                if constexpr (PACK) {
                    /* column c + 8 holds the Qlo half of row c: S = hi + lo in both lanes */
#pragma unroll
                    for (int i = 0; i < 4; i++) acc[i] += ror8(acc[i]);
                }
                sacc[nt][t] = acc;
            }
        }
    };

    /* ---- softmax of one slab and O^T += V^T.P^T ---- */
    auto smpv = [&](int k0, const f4 (&sacc)[NR][2], const VRaw &r, auto fresh_tag) __attribute__((always_inline)) {
        constexpr bool FRESH = decltype(fresh_tag)::value;
        const bool full = k0 >= lo_max && k0 + SMOL_SLAB <= hi_min;
        /* the fresh slab's fp16 V^T fragment dt as bf16 hi + lo (exact) */
        auto vsplit = [&](int dt, b8 &vh, b8 &vl) __attribute__((always_inline)) {
            float vx[8];
            const h8 v16 = *reinterpret_cast<const h8 *>(&r.v[dt]);
#pragma unroll
            for (int i = 0; i < 8; i++) vx[i] = (float)v16[i];
            split8(vx, vh, vl);
        };
#pragma unroll
        for (int nt = 0; nt < NR; nt++) {
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
            if constexpr (PACK) {
                const b8 pf = c < 8 ? ph : pl; /* column c + 8: the lo half of row c */
#pragma unroll
                for (int dt = 0; dt < DT; dt++) {
                    if constexpr (FRESH) {
                        b8 vh, vl;
                        vsplit(dt, vh, vl);
                        o[nt][dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vh, pf, o[nt][dt], 0, 0, 0);
                        o[nt][dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vl, pf, o[nt][dt], 0, 0, 0);
                    } else {
                        o[nt][dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_b8(r.v[dt]), pf, o[nt][dt], 0, 0, 0);
                    }
                }
            } else {
#pragma unroll
                for (int dt = 0; dt < DT; dt++) {
                    if constexpr (FRESH) {
                        b8 vh, vl;
                        vsplit(dt, vh, vl);
                        o[nt][dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vh, ph, o[nt][dt], 0, 0, 0);
                        o[nt][dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vh, pl, o[nt][dt], 0, 0, 0);
                        o[nt][dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vl, ph, o[nt][dt], 0, 0, 0);
                    } else {
                        o[nt][dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_b8(r.v[dt]), ph, o[nt][dt], 0, 0, 0);
                        o[nt][dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_b8(r.v[dt]), pl, o[nt][dt], 0, 0, 0);
                    }
                }
            }
        }
    };

    /* ---- the wave's slabs: slab i's K fragments are replaced by the
     * request of slab i + DEPTH once they are consumed, its V fragments once
     * they are. Requests past the wave's range are empty, so every path
     * issues the same loads and the loop needs no peeled last slab. DEPTH 2
     * (two register sets, alternating) measured slower than 1: the
     * compiler's wait counts at the loop head cover the second set too. ---- */
    const int step = SMOL_SLAB * NW;
    constexpr int DEPTH = 1;
    auto slab = [&](KRaw &kx, VRaw &vx) __attribute__((always_inline)) {
        f4 sacc[NR][2];
        const bool fr = !DIRECT && k0 >= fresh_pos0;
        if (fr) {
            /* the one or two fresh slabs of a chunk load their K lo here,
             * next to use (the cache slabs carry none) */
            KRaw kl;
            issue_klo(k0, kl);
            qk(kx, kl, sacc, std::true_type{});
        } else {
            qk(kx, kx, sacc, std::false_type{});
        }
        issue_k(k0 + DEPTH * step, kx);
        if (fr) smpv(k0, sacc, vx, std::true_type{});
        else smpv(k0, sacc, vx, std::false_type{});
        issue_v(k0 + DEPTH * step, vx);
        k0 += step;
    };
    if constexpr (DEPTH == 2) {
        KRaw kr2;
        VRaw vr2;
        issue_k(k0 + step, kr2);
        issue_v(k0 + step, vr2);
        while (k0 < ke) {
            slab(kr, vr);
            if (k0 >= ke) break;
            slab(kr2, vr2);
        }
    } else {
        while (k0 < ke) slab(kr, vr);
    }

    /* ---- decode: the new key's bf16 K row and V^T column join the cache
     * (row block 0 of the last split; the rows are still in LDS) ---- */
    if constexpr (DIRECT) {
        if (last_split && rb == 0) {
            for (int d0 = tid * 8; d0 < HD; d0 += TPB * 8) {
                float y[8];
                ld8(s_rot + R * QSTR + d0, y);
                uint16_t *kc = const_cast<uint16_t *>(p.kc) + cbase;
                uint16_t *vt = const_cast<uint16_t *>(p.vtc) + cbase +
                               (long long)(sq.pos / SMOL_SLAB) * SMOL_SLAB * HD + sq.pos % SMOL_SLAB;
                *reinterpret_cast<uint4 *>(kc + (long long)sq.pos * HD + d0) = pack_bf16x8(y);
#pragma unroll
                for (int i = 0; i < 8; i++) vt[(long long)(d0 + i) * SMOL_SLAB] = f32_to_bf16(s_vnew[d0 + i]);
            }
        }
    }

    /* ---- decode, last split, wave 0: the new key joins with an exact max ---- */
    if (DIRECT && last_split && wave == 0) {
#pragma unroll
        for (int nt = 0; nt < NR; nt++) {
            const int r = PACK ? (c & 7) : nt * 16 + c;
            float sc = PACK ? s_new : (r < R ? s_snew[r] : 0.0f);
            if (p.cap2 > 0.0f) sc = p.cap2 * tanhf(sc / p.cap2);
            const float m_new = fmaxf(m[nt], sc);
            const float alpha = __builtin_amdgcn_exp2f(m[nt] - m_new);
            const float pn = __builtin_amdgcn_exp2f(sc - m_new);
            /* PACK: the value joins the hi column only (the lo column adds 0) */
            const float pv = (!PACK || c < 8) ? pn : 0.0f;
#pragma unroll
            for (int dt = 0; dt < DT; dt++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int d = 16 * dt + 4 * j + i;
                    const float vv = (HD % 16 == 0 || d < HD) ? s_vnew[d] : 0.0f;
                    o[nt][dt][i] = fmaf(pv, vv, o[nt][dt][i] * alpha);
                }
            l[nt] = l[nt] * alpha + (j == 0 ? pn : 0.0f); /* summed over the row's four lanes below */
            m[nt] = m_new;
        }
    }

    /* ---- combine the waves: row sums, then waves 1.. hand their state to wave 0 ---- */
#pragma unroll
    for (int nt = 0; nt < NR; nt++) {
        l[nt] = row_sum4(l[nt]);
        if constexpr (PACK) {
#pragma unroll
            for (int dt = 0; dt < DT; dt++)
#pragma unroll
                for (int i = 0; i < 4; i++) o[nt][dt][i] += ror8(o[nt][dt][i]); /* hi + lo columns */
        }
    }
    __syncthreads(); /* the staging area (s_vnew, s_snew) is no longer read */
    float *s_o = smem, *s_m = smem + (NW - 1) * TR * OSTR, *s_l = s_m + (NW - 1) * TR;
    if (wave > 0) {
        const int sl = (wave - 1) * TR;
#pragma unroll
        for (int nt = 0; nt < NR; nt++) {
            const int rr = PACK ? c : nt * 16 + c;
            if (PACK && c >= 8) continue;
            float *so = s_o + (sl + rr) * OSTR;
#pragma unroll
            for (int dt = 0; dt < DT; dt++) *reinterpret_cast<f4 *>(so + 16 * dt + 4 * j) = o[nt][dt];
            if (j == 0) { s_m[sl + rr] = m[nt]; s_l[sl + rr] = l[nt]; }
        }
    }
    __syncthreads();
    if (wave == 0) {
#pragma unroll
        for (int nt = 0; nt < NR; nt++) {
            const int rr = PACK ? (c & 7) : nt * 16 + c;
            float M = m[nt];
#pragma unroll
            for (int w = 0; w < NW - 1; w++) M = fmaxf(M, s_m[w * TR + rr]);
            const float Mu = M == -INFINITY ? 0.0f : M;
            const float a0 = __builtin_amdgcn_exp2f(m[nt] - Mu);
            float L = l[nt] * a0;
#pragma unroll
            for (int dt = 0; dt < DT; dt++) o[nt][dt] *= a0;
#pragma unroll
            for (int w = 0; w < NW - 1; w++) {
                const float aw = __builtin_amdgcn_exp2f(s_m[w * TR + rr] - Mu);
                L += s_l[w * TR + rr] * aw;
                const float *so = s_o + (w * TR + rr) * OSTR;
#pragma unroll
                for (int dt = 0; dt < DT; dt++) o[nt][dt] += aw * *reinterpret_cast<const f4 *>(so + 16 * dt + 4 * j);
            }
            m[nt] = M;
            l[nt] = L;
        }
    }
    /* the output row of row r */
    auto out_row = [&](int r) {
        const int qi = (r_base + r) / G, hg = (r_base + r) - qi * G;
        return p.out + ((long long)(sq.tok0 + qi) * p.Hq + (g * G + hg)) * HD;
    };
    if (n_split == 1) {
        if (wave != 0) return;
#pragma unroll
        for (int nt = 0; nt < NR; nt++) {
            const int r = PACK ? c : nt * 16 + c;
            if ((PACK && c >= 8) || r >= R) continue;
            float *orow = out_row(r);
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

    /* ---- publish the partial, then the flag ---- */
    const long long slot0 = (long long)((seq * p.Hkv + g) * p.n_rb + rb) * DEC_MAX_SPLIT;
    const unsigned SLOTB = (unsigned)p.slot_floats * 4;
    const rsrc_t rpart = make_rsrc(p.part + slot0 * p.slot_floats, (long long)DEC_MAX_SPLIT * SLOTB);
    const unsigned my = (unsigned)split * SLOTB;
    const unsigned ML_OFF = (unsigned)(R * HD) * 4, FLAG_OFF = SLOTB - 4;
    if (!last_split) {
        if (wave == 0) {
#pragma unroll
            for (int nt = 0; nt < NR; nt++) {
                const int r = PACK ? c : nt * 16 + c;
                if ((PACK && c >= 8) || r >= R) continue;
#pragma unroll
                for (int dt = 0; dt < DT; dt++) {
                    const int d = 16 * dt + 4 * j;
                    if (HD % 16 != 0 && d >= HD) continue;
                    store_f4_l2(rpart, my + (unsigned)((r * HD + d) * 4), o[nt][dt]);
                }
                if (j == 0) store_f2_l2(rpart, my + ML_OFF + (unsigned)(r * 8), m[nt], l[nt]);
            }
            __atomic_signal_fence(__ATOMIC_SEQ_CST);
            __builtin_amdgcn_s_waitcnt(0); /* every store above acknowledged */
            __atomic_signal_fence(__ATOMIC_SEQ_CST);
            if (lane == 0) __builtin_amdgcn_raw_buffer_store_b32(epoch, rpart, my + FLAG_OFF, 0, CPOL_SC1);
        }
        return;
    }

    /* ---- the last split merges: wait for the others' flags ---- */
    float *s_w = smem;                                  /* [n_split][TR] weights */
    float *s_ml = smem + DEC_MAX_SPLIT * TR;            /* [n_split][TR][2] */
    float *s_row = smem + 3 * DEC_MAX_SPLIT * TR;       /* [TR]: 1 / sum */
    __syncthreads(); /* the combine's LDS is free */
    const int nsp = n_split;
    int ok = 1;
    if (tid < nsp - 1) {
        const unsigned *flag =
            reinterpret_cast<const unsigned *>(p.part + (slot0 + tid) * p.slot_floats + p.slot_floats - 1);
        /* fault_merge: a value no split stores, so the wait runs to its bound */
        const unsigned want = p.fault_merge ? ~epoch : epoch;
        int spins = 0;
        while (poll_u32(flag) != want) {
            if (++spins >= p.spin_limit) { ok = 0; break; }
            __builtin_amdgcn_s_sleep(1);
        }
    }
    ok = __syncthreads_and(ok);
    if (!ok && tid == 0) *p.err_flag = 1; /* synchronize reports it */
    /* Every load of the merge goes out in one round before anything waits
     * on it: the others' (m, l), then their O partials (which do not depend
     * on the weights). Element e (a row's 4 columns) gets tpe threads,
     * thread k of them holding splits k, k + tpe, ...; with more elements
     * than threads a thread takes elements eo, eo + TPB, ... (NBM at most).
     * UM splits per element a round; more splits take further rounds. Each
     * load is unconditional (an out-of-range offset reads zeros). */
    constexpr int C4 = HD / 4;
    constexpr int NBM = (TR * C4 + TPB - 1) / TPB;
    constexpr int UM = (NW > 4 ? 16 : 32) / NBM; /* loads in flight: the registers of one or two waves a SIMD */
    constexpr int NML = (DEC_MAX_SPLIT * TR + TPB - 1) / TPB;
    const int E = R * C4;
    const int tpe = max(1, min(TPB / E, nsp - 1));
    const int per_batch = TPB / tpe;             /* elements per batch */
    const int n_batch = (E + per_batch - 1) / per_batch;
    const int k = tid / per_batch, eo = tid - k * per_batch;
    const int n_u = (nsp - 1 + tpe - 1) / tpe;   /* splits of one element per thread */
    float2 mlv[NML];
#pragma unroll
    for (int i = 0; i < NML; i++) {
        const int e = tid + TPB * i, sp = e / R, r = e - sp * R;
        mlv[i] = load_f2_l2(rpart, e < (nsp - 1) * R ? (unsigned)sp * SLOTB + ML_OFF + (unsigned)(r * 8) : OOB_OFF);
    }
    auto o_off = [&](int bb, int u) -> unsigned {
        const int e = bb * per_batch + eo, sp = k + tpe * u;
        if (k >= tpe || e >= E || u >= n_u || sp >= nsp - 1) return OOB_OFF;
        const int r = e / C4, d = (e - r * C4) * 4;
        return (unsigned)sp * SLOTB + (unsigned)((r * HD + d) * 4);
    };
    f4 v[NBM][UM];
    /* only the round's real splits are requested (n_u is uniform: the
     * branches are scalar); an out-of-range request still costs the address
     * unit its lanes */
    auto load_round = [&](int u0) __attribute__((always_inline)) {
#pragma unroll
        for (int uu = 0; uu < UM; uu++) {
            if (u0 + uu >= n_u) break;
#pragma unroll
            for (int bb = 0; bb < NBM; bb++) v[bb][uu] = load_f4_l2(rpart, o_off(bb, u0 + uu));
        }
    };
    load_round(0);
    /* this split's own state goes into LDS next to the others' */
    if (wave == 0) {
#pragma unroll
        for (int nt = 0; nt < NR; nt++) {
            const int r = PACK ? c : nt * 16 + c;
            if ((PACK && c >= 8) || r >= R) continue;
            if (j == 0) { s_ml[2 * ((nsp - 1) * TR + r)] = m[nt]; s_ml[2 * ((nsp - 1) * TR + r) + 1] = l[nt]; }
        }
    }
#pragma unroll
    for (int i = 0; i < NML; i++) {
        const int e = tid + TPB * i, sp = e / R, r = e - sp * R;
        if (e < (nsp - 1) * R) {
            s_ml[2 * (sp * TR + r)] = mlv[i].x;
            s_ml[2 * (sp * TR + r) + 1] = mlv[i].y;
        }
    }
    __syncthreads();
    if (tid < R) {
        float M = -INFINITY;
        for (int sp = 0; sp < nsp; sp++) M = fmaxf(M, s_ml[2 * (sp * TR + tid)]);
        const float Mu = M == -INFINITY ? 0.0f : M;
        float L = 0.0f;
        for (int sp = 0; sp < nsp; sp++) {
            const float w = __builtin_amdgcn_exp2f(s_ml[2 * (sp * TR + tid)] - Mu);
            s_w[sp * TR + tid] = w;
            L += w * s_ml[2 * (sp * TR + tid) + 1];
        }
        s_row[tid] = L > 0.0f ? 1.0f / L : 0.0f;
    }
    /* O of every row: this split's own part from wave 0's registers (through
     * LDS), the others' from their slots */
    float *s_own = smem + 3 * DEC_MAX_SPLIT * TR + TR; /* [TR][OSTR] */
    if (wave == 0) {
#pragma unroll
        for (int nt = 0; nt < NR; nt++) {
            const int r = PACK ? c : nt * 16 + c;
            if ((PACK && c >= 8) || r >= R) continue;
#pragma unroll
            for (int dt = 0; dt < DT; dt++) *reinterpret_cast<f4 *>(s_own + r * OSTR + 16 * dt + 4 * j) = o[nt][dt];
        }
    }
    __syncthreads();
    /* each thread's splits in increasing order, then the tpe partial sums
     * and this split's own part in a fixed order: the result does not
     * depend on timing */
    f4 acc[NBM];
#pragma unroll
    for (int bb = 0; bb < NBM; bb++) acc[bb] = f4{0.f, 0.f, 0.f, 0.f};
    for (int u0 = 0; u0 < n_u; u0 += UM) {
        if (u0 > 0) load_round(u0);
#pragma unroll
        for (int bb = 0; bb < NBM; bb++) {
            const int e = bb * per_batch + eo, r = e / C4;
#pragma unroll
            for (int uu = 0; uu < UM; uu++) {
                if (u0 + uu >= n_u) break;
                const int sp = k + tpe * (u0 + uu);
                if (k < tpe && e < E && sp < nsp - 1) acc[bb] += s_w[sp * TR + r] * v[bb][uu];
            }
        }
    }
    f4 *s_part = reinterpret_cast<f4 *>(s_own + TR * OSTR); /* [tpe][per_batch] */
#pragma unroll
    for (int bb = 0; bb < NBM; bb++) {
        if (bb >= n_batch) break;
        const int e = bb * per_batch + eo;
        if (k < tpe) s_part[k * per_batch + eo] = acc[bb];
        __syncthreads();
        if (k == 0 && e < E) {
            const int r = e / C4, d = (e - r * C4) * 4;
            f4 res = s_w[(nsp - 1) * TR + r] * *reinterpret_cast<const f4 *>(s_own + r * OSTR + d);
            for (int kk = 0; kk < tpe; kk++) res += s_part[kk * per_batch + eo];
            res *= s_row[r];
            if (!ok) res = f4{NAN, NAN, NAN, NAN};
            *reinterpret_cast<f4 *>(out_row(r) + d) = res;
        }
        __syncthreads();
    }
}

/* ------------------------------------------------------------------ launcher */

template <int HD, int NT, bool PACK, int NW, bool DIRECT>
static int launch_dec_d(const DecParams *dp, hipStream_t st, hipEvent_t ev0, hipEvent_t ev1) {
    if (ev0)
        hipExtLaunchKernelGGL((k_dec<HD, NT, PACK, NW, DIRECT>), dim3(dp->n_items), dim3(64 * NW), 0, st, ev0, ev1, 0, *dp);
    else
        hipLaunchKernelGGL((k_dec<HD, NT, PACK, NW, DIRECT>), dim3(dp->n_items), dim3(64 * NW), 0, st, *dp);
    return hipGetLastError() == hipSuccess ? 0 : -3;
}

template <int HD, int NT, bool PACK, int NW>
static int launch_dec_v(const DecParams *dp, hipStream_t st, hipEvent_t ev0, hipEvent_t ev1) {
    return dp->direct ? launch_dec_d<HD, NT, PACK, NW, true>(dp, st, ev0, ev1)
                      : launch_dec_d<HD, NT, PACK, NW, false>(dp, st, ev0, ev1);
}

/* workgroups of one k_dec build that fit on a compute unit at once */
template <int HD, int NT, bool PACK, int NW>
static int occ_v(bool direct) {
    int n = 0;
    const void *f = direct ? reinterpret_cast<const void *>(&k_dec<HD, NT, PACK, NW, true>)
                           : reinterpret_cast<const void *>(&k_dec<HD, NT, PACK, NW, false>);
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, f, 64 * NW,
                                                     0) != hipSuccess)
        return 1;
    return n > 0 ? n : 1;
}

template <int HD>
static int occ_hd(int rows, int nw, bool d) {
    if (rows <= 8) {
        if constexpr (HD <= 128) {
            if (nw == 8) return occ_v<HD, 1, true, 8>(d);
        }
        return occ_v<HD, 1, true, 4>(d);
    }
    if (rows <= 16 || HD > 128) return occ_v<HD, 1, false, 4>(d);
    if constexpr (HD <= 128) return occ_v<HD, 2, false, 4>(d);
    return 1;
}

extern "C" int smol_decode_occupancy(int hd, int rows, int nw, int direct) {
    const bool d = direct != 0;
    switch (hd) {
    case 64: return occ_hd<64>(rows, nw, d);
    case 72: return occ_hd<72>(rows, nw, d);
    case 80: return occ_hd<80>(rows, nw, d);
    case 96: return occ_hd<96>(rows, nw, d);
    case 128: return occ_hd<128>(rows, nw, d);
    case 256: return occ_hd<256>(rows, nw, d);
    default: return 1;
    }
}

/* rows: query rows per (sequence, kv head); above 8 they run in row blocks
 * of DEC_RB(hd). nw: waves per workgroup (8 only for at most 8 rows and
 * head_dim <= 128, where two waves per SIMD fit the registers) */
template <int HD>
static int launch_dec_hd(const DecParams *dp, int rows, int nw, hipStream_t st, hipEvent_t ev0, hipEvent_t ev1) {
    if (rows <= 8) {
        if constexpr (HD <= 128) {
            if (nw == 8) return launch_dec_v<HD, 1, true, 8>(dp, st, ev0, ev1);
        }
        return launch_dec_v<HD, 1, true, 4>(dp, st, ev0, ev1);
    }
    if (rows <= 16 || HD > 128) return launch_dec_v<HD, 1, false, 4>(dp, st, ev0, ev1);
    if constexpr (HD <= 128) return launch_dec_v<HD, 2, false, 4>(dp, st, ev0, ev1);
    return -1;
}

extern "C" int smol_launch_decode(const DecParams *dp, int hd, int rows, int nw, hipStream_t st, hipEvent_t ev0,
                                  hipEvent_t ev1) {
    if (dp->n_items <= 0) return 0;
    switch (hd) {
    case 64: return launch_dec_hd<64>(dp, rows, nw, st, ev0, ev1);
    case 72: return launch_dec_hd<72>(dp, rows, nw, st, ev0, ev1);
    case 80: return launch_dec_hd<80>(dp, rows, nw, st, ev0, ev1);
    case 96: return launch_dec_hd<96>(dp, rows, nw, st, ev0, ev1);
    case 128: return launch_dec_hd<128>(dp, rows, nw, st, ev0, ev1);
    case 256: return launch_dec_hd<256>(dp, rows, nw, st, ev0, ev1);
    default: return -1;
    }
}

/* ------------------------------------------------------ XCD dispatch check */

/* workgroup b records the XCC id register; the host checks b % n_xcc, the
 * dispatch order k_dec's merge relies on */
__global__ __launch_bounds__(64) void k_xcc_probe(unsigned *out, int n) {
    unsigned x;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(x));
    if (threadIdx.x == 0 && blockIdx.x < (unsigned)n) out[blockIdx.x] = x & 0xFu;
}

extern "C" int smol_launch_xcc_probe(unsigned *out, int n, hipStream_t st) {
    if (n <= 0) return 0;
    hipLaunchKernelGGL(k_xcc_probe, dim3(n), dim3(64), 0, st, out, n);
    return hipGetLastError() == hipSuccess ? 0 : -3;
}
