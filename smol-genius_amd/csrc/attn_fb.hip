/*
 * attn_fb.hip - k_attn_fb: prefill and windowed bidirectional attention over
 * keys that all sit in the fresh fp16 staging.
 */
#include "attn_splitk.h"

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
 * Step i of a group: the softmax of slab i runs on the vector ALU next to
 * P.V of slab i-1 and S = K.Q^T of slab i+1 on the matrix cores (neither
 * depends on the softmax, so the two units work at once), while K of slab
 * i+1 and V^T of slab i are read from LDS; a row whose maximum passes its
 * threshold takes a rare path at the end of the step; then the transfers
 * are waited for where the schedule needs them and one barrier publishes
 * them.
 */
/* WPG waves per key group, each holding NT 16-row tiles of the item.
 * PREC (precise QK^T): a stage holds the K image twice, fp16 hi then fp16 lo
 * (the same layout), then V^T; with two key groups the larger stage leaves
 * room for three stages per group instead of five. ONE: a single key group
 * of eight waves (128-row items), which keeps five stages either way. */
template <int HD, int WPG, bool PREC, bool ONE>
struct FbGeom {
    static constexpr int KS = (HD + 31) / 32;
    static constexpr int DT = (HD + 15) / 16;
    static constexpr int HDP = KS * 32;
    static constexpr int KROW = 256;
    static constexpr int K_BYTES = SMOL_SLAB * KROW;
    static constexpr int KPARTS = PREC ? 2 : 1;
    static constexpr int V_BYTES = 16 * DT * 64;
    static constexpr int STAGE = (KPARTS * K_BYTES + V_BYTES + 1024 * WPG - 1) / (1024 * WPG) * (1024 * WPG);
    static constexpr int NDMA = STAGE / (1024 * WPG); /* DMA instructions per wave per slab */
    static constexpr int GROUPS = ONE ? 1 : 2;
    static constexpr int NSTG = PREC && !ONE ? 3 : (GROUPS * 5 * STAGE <= 160 * 1024 ? 5 : 4);
    static constexpr int GROUP_BYTES = NSTG * STAGE;
};

/* NT = 1: four waves per key group (two per SIMD, 512 threads); NT = 2: two
 * waves per key group, each holding two row tiles (one wave per SIMD, 256
 * threads): every K / V^T fragment read from LDS then feeds two MFMAs, which
 * halves the LDS reads per flop. One MFMA pipe per SIMD is kept busy by a
 * single wave (measured: 16x16x32 f16 MFMAs with independent accumulators
 * issue at the same rate from one wave per SIMD as from two). */
/* The merge of a split item's group by its last workgroup (merge_group of
 * k_attn_fa on the item's fields), not inlined: its registers then do not add
 * to those of the slab loop, which runs at two waves per SIMD. */
template <int HD, int ROWS, int TPB>
__device__ __attribute__((noinline)) void fb_merge(float *part_o, float *part_ml, int *counters, float *out, int Hkv,
                                                   int Hq, int G, FbItem it, int g, int tid, float *s_o) {
    /* the fields merge_group reads (passed by value: the kernel's own
     * argument block stays private to it, so its fields stay uniform) */
    SkParams p;
    memset(&p, 0, sizeof(p));
    p.part_o = part_o; p.part_ml = part_ml; p.counters = counters; p.out = out;
    p.Hkv = Hkv; p.Hq = Hq; p.G = G;
    SkItem si;
    si.batch = 0; si.row0 = it.row0; si.key_begin = it.key_begin; si.key_end = it.key_end;
    si.group = it.group; si.n_split = it.n_split; si.split = it.split; si.fresh_off = it.fresh_off;
    SkBatch sb;
    sb.n_rows = it.n_rows; sb.q_row0 = it.q_row0; sb.out_tok0 = it.out_tok0; sb.q_pos0 = it.q_pos0;
    sb.key_lo = it.key_lo; sb.key_hi = it.key_hi; sb.causal = it.causal;
    sb.fresh_pos0 = 0; sb.fresh_row0 = 0; sb.slot = -1; sb.pad0 = sb.pad1 = 0;
    merge_group<HD, ROWS, 16, TPB>(p, si, sb, it.part, g, tid, s_o);
}

/* The Q fragments of one 16-row tile straight from the inputs (SkParams.q_in):
 * lane (c, j) holds elements d = 32 ks + 8 j + i of its row (Q scratch row
 * `row` = token * G + head in group, at RoPE position `pos`), so the NeoX
 * partner of a first-half element (d + HD / 2) is in the same lane for head_dim
 * 64 and 128. The arithmetic is that of k_prep's Q blocks without a norm:
 * the rotation of rope.c:68-164, the scale, then the split into fp16 hi + lo
 * (calls with a per-head Q norm stage Q in k_prep). */
template <int HD>
__device__ __forceinline__ void q_from_input(const SkParams &p, int row, int pos, int g, int G, int j, bool valid,
                                             h8 (&qf)[(HD + 31) / 32], h8 (&ql)[(HD + 31) / 32]) {
    static_assert(HD == 64 || HD == 128, "partners in the lane");
    constexpr int KS = HD / 32, HALF = HD / 2;
    const int tok = row / G, hg = row - tok * G;
    const long long base = (long long)tok * p.q_stride + (long long)(g * G + hg) * HD;
    const bool bf = p.q_dtype == SMOL_IN_BF16;
    float v[KS][8];
    /* every load of the tile goes out before any is used; the branches
     * (uniform over the launch) leave out the loads a call does not need:
     * the second 16 bytes of a bf16 row part, the tables of the second half
     * under NeoX (they repeat the first) */
    uint4 ra[KS], rb[KS];
    float4 c0[KS], c1[KS], s0[KS], s1[KS];
    const bool rope = p.q_rope_kind != SMOL_ROPE_OFF;
    const bool neox = p.q_rope_kind == SMOL_ROPE_NEOX_K;
    const char *dummy = static_cast<const char *>(p.q_in);
    const float *fdummy = reinterpret_cast<const float *>(dummy);
#pragma unroll
    for (int ks = 0; ks < KS; ks++) {
        const int d0 = 32 * ks + 8 * j;
        const char *a = valid ? static_cast<const char *>(p.q_in) + (base + d0) * (bf ? 2 : 4) : dummy;
        ra[ks] = *reinterpret_cast<const uint4 *>(a);
        rb[ks] = uint4{0u, 0u, 0u, 0u};
        if (!bf) rb[ks] = *reinterpret_cast<const uint4 *>(valid ? a + 16 : dummy);
        c0[ks] = c1[ks] = s0[ks] = s1[ks] = float4{0.f, 0.f, 0.f, 0.f};
        if (rope && !(neox && d0 >= HALF)) {
            const float *cs = valid ? p.rope_cos + (long long)pos * HD + d0 : fdummy;
            const float *sn = valid ? p.rope_sin + (long long)pos * HD + d0 : fdummy;
            c0[ks] = *reinterpret_cast<const float4 *>(cs); c1[ks] = *reinterpret_cast<const float4 *>(cs + 4);
            s0[ks] = *reinterpret_cast<const float4 *>(sn); s1[ks] = *reinterpret_cast<const float4 *>(sn + 4);
        }
    }
#pragma unroll
    for (int ks = 0; ks < KS; ks++) {
        if (bf) {
            unpack_bf16x8(ra[ks], v[ks]);
        } else {
            const uint32_t t[8] = {ra[ks].x, ra[ks].y, ra[ks].z, ra[ks].w, rb[ks].x, rb[ks].y, rb[ks].z, rb[ks].w};
#pragma unroll
            for (int i = 0; i < 8; i++) v[ks][i] = __uint_as_float(t[i]);
        }
    }
    if (p.q_rope_kind == SMOL_ROPE_NEOX_K) {
#pragma unroll
        for (int ks = 0; ks < KS / 2; ks++) {
            const float cv[8] = {c0[ks].x, c0[ks].y, c0[ks].z, c0[ks].w, c1[ks].x, c1[ks].y, c1[ks].z, c1[ks].w};
            const float sv[8] = {s0[ks].x, s0[ks].y, s0[ks].z, s0[ks].w, s1[ks].x, s1[ks].y, s1[ks].z, s1[ks].w};
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const float x1 = v[ks][i], x2 = v[ks + KS / 2][i];
                v[ks][i] = fmaf(x1, cv[i], -(x2 * sv[i]));
                v[ks + KS / 2][i] = fmaf(x2, cv[i], x1 * sv[i]);
            }
        }
    } else if (p.q_rope_kind == SMOL_ROPE_INTERLEAVED_K) {
#pragma unroll
        for (int ks = 0; ks < KS; ks++) {
            const float cv[8] = {c0[ks].x, c0[ks].y, c0[ks].z, c0[ks].w, c1[ks].x, c1[ks].y, c1[ks].z, c1[ks].w};
            const float sv[8] = {s0[ks].x, s0[ks].y, s0[ks].z, s0[ks].w, s1[ks].x, s1[ks].y, s1[ks].z, s1[ks].w};
#pragma unroll
            for (int i = 0; i < 8; i += 2) {
                const float x0 = v[ks][i], x1 = v[ks][i + 1];
                v[ks][i] = x0 * cv[i] - x1 * sv[i];
                v[ks][i + 1] = x1 * cv[i + 1] + x0 * sv[i + 1];
            }
        }
    }
#pragma unroll
    for (int ks = 0; ks < KS; ks++) {
#pragma unroll
        for (int i = 0; i < 8; i++) v[ks][i] = valid ? v[ks][i] * p.qscale : 0.0f;
        note_h_range(p.range_flag, v[ks]);
        uint4 hi, lo;
        pack_h8_hilo(v[ks], hi, lo);
        qf[ks] = *reinterpret_cast<const h8 *>(&hi);
        ql[ks] = *reinterpret_cast<const h8 *>(&lo);
    }
}

/* ONE: the eight waves form a single key group over a 128-row item (each
 * slab is transferred once for all of them), and an item may cover part of
 * its tile's keys (see FbItem), merged across workgroups */
template <int HD, int NT, bool CAP, bool PREC, bool ONE, bool QIN = false>
__global__ __launch_bounds__(NT == 1 ? 512 : 256)
__attribute__((amdgpu_waves_per_eu(NT == 1 ? 2 : 1, NT == 1 ? 2 : 1))) void k_attn_fb(SkParams p) {
    static_assert(!ONE || NT == 1, "one key group: eight waves of one row tile each");
    constexpr int WPG = ONE ? 8 : 4 / NT;
    using Gm = FbGeom<HD, WPG, PREC, ONE>;
    constexpr int KS = Gm::KS, DT = Gm::DT, HDP = Gm::HDP, KROW = Gm::KROW;
    constexpr int K_BYTES = Gm::K_BYTES, STAGE = Gm::STAGE, NDMA = Gm::NDMA, NSTG = Gm::NSTG;
    constexpr unsigned SLAB_BYTES = SMOL_SLAB * HD * 2;
    /* one barrier a step and one-step transfers (three stages) */
    constexpr bool B1 = NSTG == 3;
    constexpr int ROWS = 16 * NT * WPG; /* rows of an item */
    static_assert(HD <= 128, "k_attn_fb covers head_dim <= 128");
    static_assert(Gm::GROUPS * Gm::GROUP_BYTES <= 160 * 1024, "LDS");
    static_assert(NSTG >= 3, "the step pipeline keeps three slabs resident");
    static_assert(!PREC || K_BYTES % (1024 * WPG) == 0, "each DMA instruction of a wave lands in one part");
    static_assert(!ONE || (2 * SK_MERGE_MAX + 2 * ROWS) * 4 <= Gm::GROUP_BYTES, "merge scratch");
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int grp = ONE ? 0 : wave / WPG, wg = wave % WPG;
    const float icap2 = CAP ? 1.0f / p.cap2 : 0.0f;
    const int g = (int)(blockIdx.x % (unsigned)p.Hkv);
    const int w = (int)(blockIdx.x / (unsigned)p.Hkv);
    __shared__ __attribute__((aligned(1024))) unsigned char smem[Gm::GROUPS * Gm::GROUP_BYTES];
    __shared__ int s_last;
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

    /* this group's slabs: the first or second half of the item's (ONE: all) */
    const int n_all = (it.key_end - it.key_begin + SMOL_SLAB - 1) / SMOL_SLAB;
    const int n0 = ONE ? n_all : (n_all + 1) >> 1;
    const int s_first = grp == 0 ? 0 : n0;
    const int n_own = grp == 0 ? n0 : n_all - n0;
    auto slab_k = [&](int i) __attribute__((always_inline)) {
        const int q = n_own > 0 ? s_first + (i < n_own ? i : n_own - 1) : 0;
        return it.key_begin + SMOL_SLAB * q;
    };

    /* DMA geometry: region q = wg + WPG e of a stage; lane offsets within
     * the slab. The first transfers go out before anything else is set up. */
    const rsrc_t rk = make_rsrc(p.kf + (long long)g * p.fcap * HD, (long long)p.fcap * HD * 2);
    const rsrc_t rkl = PREC ? make_rsrc(p.kf_lo + (long long)g * p.fcap * HD, (long long)p.fcap * HD * 2) : rk;
    const rsrc_t rv = make_rsrc(p.vtf + (long long)g * p.fcap * HD, (long long)p.fcap * HD * 2);
    /* region q of a stage: K (hi), with PREC then K lo, then V^T; the part
     * of each of this wave's regions is the same in every wave (the K parts
     * are whole multiples of WPG regions) */
    unsigned d_off[NDMA];
    int d_part[NDMA]; /* 0: K, 1: K lo, 2: V^T */
#pragma unroll
    for (int e = 0; e < NDMA; e++) {
        const int q = wg + WPG * e;
        const int kparts_bytes = Gm::KPARTS * K_BYTES;
        d_part[e] = q * 1024 < K_BYTES ? 0 : q * 1024 < kparts_bytes ? 1 : 2;
        if (d_part[e] < 2) {
            const int qk = d_part[e] == 0 ? q : q - K_BYTES / 1024;
            const int kr = qk * 4 + (lane >> 4), slot = lane & 15;
            const int cb = slot ^ ((kr & 3) | (((kr >> 3) & 3) << 2));
            d_off[e] = cb < HD / 8 ? (unsigned)((kr * HD + cb * 8) * 2) : OOB_OFF;
        } else {
            const int d = (q * 1024 - kparts_bytes) / 64 + (lane >> 2), slot = lane & 3;
            const int jj = slot ^ ((d >> 1) & 3);
            d_off[e] = d < HD ? (unsigned)((d * SMOL_SLAB + jj * 8) * 2) : OOB_OFF;
        }
    }
    auto dma = [&](int k0, int stage) __attribute__((always_inline)) {
        const int kr = k0 + it.fresh_off; /* from the item: the transfers need no batch load */
        const unsigned so = (unsigned)(kr / SMOL_SLAB) * SLAB_BYTES;
#pragma unroll
        for (int e = 0; e < NDMA; e++)
            dma_1k(d_part[e] == 0 ? rk : d_part[e] == 1 ? rkl : rv, d_off[e], so,
                   __builtin_amdgcn_readfirstlane(lds_group + stage * STAGE + (wg + WPG * e) * 1024));
    };
    /* the prologue stages three slabs (three stages: two); the steps bring
     * the rest in pairs (three stages: one a step) */
    constexpr int PRO = B1 ? 2 : 3;
#pragma unroll
    for (int q = 0; q < PRO; q++) dma(slab_k(q), q);

    /* rows of this wave (the same in both groups): tile nt holds rows
     * 16 (wg NT + nt) + c of the item */
    int lo[NT], hi[NT];
    bool valid[NT];
    h8 qf[NT][KS];
    h8 qfl[PREC ? NT : 1][KS]; /* PREC: Q lo */
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
        if constexpr (QIN) {
            q_from_input<HD>(p, b.q_row0 + (valid[nt] ? r : 0), b.q_pos0 + (valid[nt] ? r : 0) / G, g, G, j,
                         valid[nt], qf[nt], qfl[PREC ? nt : 0]);
            continue;
        }
        const long long qoff = (long long)g * p.qs_head_stride + (long long)(b.q_row0 + (valid[nt] ? r : 0)) * HDP;
        const _Float16 *qrow = p.qs + qoff;
#pragma unroll
        for (int ks = 0; ks < KS; ks++) qf[nt][ks] = valid[nt] ? load_h8(qrow + 32 * ks + 8 * j) : zero_h8();
        if constexpr (PREC) {
            const _Float16 *qrl = p.qs_lo + qoff;
#pragma unroll
            for (int ks = 0; ks < KS; ks++) qfl[nt][ks] = valid[nt] ? load_h8(qrl + 32 * ks + 8 * j) : zero_h8();
        }
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
    /* the row sums: without PREC on the matrix cores, one more MFMA per step
     * against a fragment of ones (every element of lsum is the row's sum of
     * its fp16 probabilities, the same weights the P.V product uses); with
     * PREC (P = Phi + Plo, about 22 bits) in fp32 on the vector ALU, each
     * lane summing its own keys (l), reduced over the row's lanes at the end */
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
    const unsigned vfo = (unsigned)(Gm::KPARTS * K_BYTES + c * 64 + 16 * (j ^ ((c >> 1) & 3)));
    auto lds_h8 = [&](int stage, unsigned off) __attribute__((always_inline)) -> h8 {
        const uint4 w = *reinterpret_cast<const uint4 *>(gbase + stage * STAGE + off);
        return *reinterpret_cast<const h8 *>(&w);
    };
    /* K fragments of a slab (hi; PREC reads the lo part inside qk) */
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
    /* S^T = K.Q^T, less the running max m (raw S with a softcap); PREC:
     * Khi.Qhi + Khi.Qlo, then Klo.Qhi (the Klo.Qlo term is below 2^-21 of
     * S): the K lo fragments are read from `stage` into the registers of
     * the hi ones once the hi products are issued, which keeps one slab's
     * fragments live instead of two, and the hi products cover the reads */
    auto qk_hi = [&](const h8 (&kt)[KS], int t, f4 (&sacc)[NT][2]) __attribute__((always_inline)) {
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
            f4 acc = CAP ? f4{0.f, 0.f, 0.f, 0.f} : negm[nt];
#pragma unroll
            for (int ks = 0; ks < KS; ks++) {
                acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(kt[ks], qf[nt][ks], acc, 0, 0, 0);
                if constexpr (PREC) acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(kt[ks], qfl[nt][ks], acc, 0, 0, 0);
            }
            sacc[nt][t] = acc;
        }
    };
    auto qk_lo = [&](const h8 (&kt)[KS], int t, f4 (&sacc)[NT][2]) __attribute__((always_inline)) {
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
            f4 acc = sacc[nt][t];
#pragma unroll
            for (int ks = 0; ks < KS; ks++) acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(kt[ks], qf[nt][ks], acc, 0, 0, 0);
            sacc[nt][t] = acc;
        }
    };
    auto read_klo = [&](int stage, int t, h8 (&kt)[KS]) __attribute__((always_inline)) {
#pragma unroll
        for (int ks = 0; ks < KS; ks++) kt[ks] = lds_h8(stage, kfo[ks] + t * 4 * KROW + K_BYTES);
    };
    /* PREC order: the hi products of key rows t = 0; the lo fragments of t = 0
     * read into their registers while the hi products of t = 1 run; those of
     * t = 1 while the lo products of t = 0 run; then the lo products of t = 1 */
    auto qk = [&](h8 (&kf)[2][KS], int stage, f4 (&sacc)[NT][2]) __attribute__((always_inline)) {
        if constexpr (PREC) {
            /* the barriers pin the LDS reads and MFMAs in this order; vector
             * and scalar ALU work (the softmax) may move across them (mask:
             * VALU | SALU | transcendental) */
            constexpr int ALU = 0x0002 | 0x0004 | 0x0400;
            qk_hi(kf[0], 0, sacc);
            __builtin_amdgcn_sched_barrier(ALU);
            read_klo(stage, 0, kf[0]);
            qk_hi(kf[1], 1, sacc);
            __builtin_amdgcn_sched_barrier(ALU);
            read_klo(stage, 1, kf[1]);
            qk_lo(kf[0], 0, sacc);
            __builtin_amdgcn_sched_barrier(ALU);
            qk_lo(kf[1], 1, sacc);
        } else {
            qk_hi(kf[0], 0, sacc);
            qk_hi(kf[1], 1, sacc);
        }
    };
    /* P fragments: [0] fp16 P (hi), [1] its lo part (PREC) */
    constexpr int NP = PREC ? 2 : 1;
    auto pv = [&](const h8 (&vf)[DT], const h8 (&pf)[NP][NT]) __attribute__((always_inline)) {
#pragma unroll
        for (int dt = 0; dt < DT; dt++)
#pragma unroll
            for (int nt = 0; nt < NT; nt++) {
                o[nt][dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf[dt], pf[0][nt], o[nt][dt], 0, 0, 0);
                if constexpr (PREC) o[nt][dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf[dt], pf[1][nt], o[nt][dt], 0, 0, 0);
            }
        if constexpr (!PREC) {
#pragma unroll
            for (int nt = 0; nt < NT; nt++)
                lsum[nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ones, pf[0][nt], lsum[nt], 0, 0, 0);
        }
    };
    /* P = exp2(S - m) of one row tile as fp16 (PREC: hi + lo, and the fp32
     * sum of the lane's probabilities in psum) */
    auto p_frag = [&](const f4 (&s)[2], float sh, h8 (&pf)[NP][NT], int nt, float &psum) __attribute__((always_inline)) {
        float ps = 0.0f;
        if constexpr (PREC) {
#pragma unroll
            for (int e = 0; e < 8; e += 2) {
                const float p0 = __builtin_amdgcn_exp2f(s[e >> 2][e & 3] - sh);
                const float p1 = __builtin_amdgcn_exp2f(s[(e + 1) >> 2][(e + 1) & 3] - sh);
                uint32_t hi, lo;
                split_h2(p0, p1, hi, lo);
                reinterpret_cast<uint32_t *>(&pf[0][nt])[e >> 1] = hi;
                reinterpret_cast<uint32_t *>(&pf[1][nt])[e >> 1] = lo;
                ps += p0;
                ps += p1;
            }
        } else {
#pragma unroll
            for (int e = 0; e < 8; e++) pf[0][nt][e] = (_Float16)__builtin_amdgcn_exp2f(s[e >> 2][e & 3] - sh);
        }
        psum = ps;
    };
    /* softcap (raw S -> capped S - m), then the mask of a step that is not
     * wholly inside every row's key range: lane (c, j) holds keys
     * 8j + 4t + i of row c in s[t][i] */
    auto prep_s = [&](int k0, bool act, bool masked, f4 (&s)[NT][2]) __attribute__((always_inline)) {
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
            if constexpr (CAP) {
#pragma unroll
                for (int t = 0; t < 2; t++)
#pragma unroll
                    for (int i = 0; i < 4; i++) s[nt][t][i] = p.cap2 * tanhf(s[nt][t][i] * icap2) + negm[nt][0];
            }
            if (masked) {
                /* lo <= key < hi as one unsigned compare; a step past the
                 * group's slabs has an empty range */
                const unsigned span = act ? (unsigned)hi[nt] - (unsigned)lo[nt] : 0u;
                const unsigned rel0 = (unsigned)(k0 + 8 * j) - (unsigned)lo[nt];
#pragma unroll
                for (int t = 0; t < 2; t++)
#pragma unroll
                    for (int i = 0; i < 4; i++)
                        s[nt][t][i] = rel0 + (unsigned)(4 * t + i) < span ? s[nt][t][i] : -INFINITY;
            }
        }
    };
    /* P = exp2(S - m) as fp16, assuming no row's max passes its threshold;
     * returns whether one does (then the rare path below redoes it) */
    auto expo = [&](const f4 (&s)[NT][2], h8 (&pf)[NP][NT], float (&psum)[NT]) __attribute__((always_inline)) -> bool {
        bool hit = false;
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
#pragma unroll
            for (int e = 0; e < 8; e++) hit |= s[nt][e >> 2][e & 3] > thr[nt];
            p_frag(s[nt], 0.0f, pf, nt, psum[nt]);
        }
        /* the probabilities are computed here, next to this step's MFMAs,
         * and not sunk into the branch after it (the rare path redoes them) */
#pragma unroll
        for (int q = 0; q < NP; q++)
#pragma unroll
            for (int nt = 0; nt < NT; nt++) asm volatile("" : "+v"(pf[q][nt]));
        return __any(hit);
    };
    /* Rare path (a row's max passed its threshold): move m to the row max,
     * redo P, and rescale what was accumulated against the old m: O and the
     * row sums (after the P.V of the previous slab, issued earlier in the
     * step) and S of the next slab (computed against the old m). */
    auto rescale = [&](f4 (&s)[NT][2], h8 (&pf)[NP][NT], f4 (&snext)[NT][2], float (&psum)[NT]) __attribute__((always_inline)) {
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
            const float mx = row_max4(fmaxf(fmaxf(fmaxf(s[nt][0][0], s[nt][0][1]), fmaxf(s[nt][0][2], s[nt][0][3])),
                                            fmaxf(fmaxf(s[nt][1][0], s[nt][1][1]), fmaxf(s[nt][1][2], s[nt][1][3]))));
            const bool need = mx > thr[nt];
            const float sh = need ? mx : 0.0f;
            const float m_new = need ? -negm[nt][0] + mx : m[nt];
            const float alpha = need ? __builtin_amdgcn_exp2f(m[nt] - m_new) : 1.0f;
#pragma unroll
            for (int dt = 0; dt < DT; dt++) o[nt][dt] *= alpha;
            lsum[nt] *= alpha;
            l[nt] *= alpha;
            m[nt] = m_new;
            const float mu = m_new == -INFINITY ? 0.0f : m_new;
            negm[nt] = f4{-mu, -mu, -mu, -mu};
            thr[nt] = m_new == -INFINITY ? -INFINITY : LAZY_T;
            p_frag(s[nt], sh, pf, nt, psum[nt]);
            if constexpr (!CAP) {
#pragma unroll
                for (int t = 0; t < 2; t++) snext[nt][t] -= sh;
            }
        }
    };

    /* Slab j of this group sits in stage j % NSTG. Step i reads the K
     * fragments of slab i+1 and the V^T fragments of slab i, and computes
     * P.V of slab i-1 and S of slab i+1 on the matrix cores next to the
     * softmax of slab i on the vector ALU: the MFMAs of a step depend on
     * nothing the step computes, so one wave keeps both units busy. The
     * prologue stages slabs 0..2. Even step s brings slabs s+3 and s+4 into
     * the stages of slabs s-2 and s-1 (step 0: the two unused stages), whose
     * last reads were in steps s-2 and s-1; the odd step after it waits for
     * them (vmcnt(0)) and ends in a barrier, and slab s+3 is first read at
     * the top of step s+2. Every transfer is waited for with vmcnt(0) before
     * a barrier that precedes the first read of its stage, and every read of
     * a stage precedes a barrier that precedes its refill; even steps need
     * no barrier of their own, so the waves of a workgroup drift apart by up
     * to a step. Steps past the group's own slab count (the second group may
     * have one fewer, or none) keep the reads, transfers and barriers and
     * mask every key. */
    /* Three stages (PREC with two key groups): step i brings slab i+2 into
     * the stage of slab i-1, whose last read (its V^T, step i-1) precedes the
     * barrier ending step i-1, and every step ends in a barrier after
     * vmcnt(0), so the slab has landed before step i+1 reads its K. */
    static_assert(B1 || NSTG == 5, "the transfer schedules are built for five stages (or three)");
    const int steps = n0;
    /* Every transfer of the prologue (and Q) has landed before the first
     * barrier. Counted waits (all but the last slabs' transfers) are not used
     * for LDS transfers: on pages touched for the first time they let a
     * barrier pass with earlier transfers' bytes not yet in LDS, so the
     * transfers do not complete in issue order there. */
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    f4 sa[NT][2], sb[NT][2];
    h8 kf[2][KS], vfa[DT], vfb[DT], pfa[NP][NT], pfb[NP][NT];
    read_k(0, kf);
    qk(kf, 0, sa);
#pragma unroll
    for (int dt = 0; dt < DT; dt++) vfa[dt] = zero_h8();
#pragma unroll
    for (int q = 0; q < NP; q++)
#pragma unroll
        for (int nt = 0; nt < NT; nt++) pfa[q][nt] = zero_h8();
    int st_k = 1, st_v = 0; /* stages of slabs i+1 and i */
    auto step = [&](int i, bool odd, f4 (&scur)[NT][2], f4 (&snext)[NT][2], auto &vprev, auto &vnow, auto &pprev,
                    auto &pnow) __attribute__((always_inline)) {
        const int k0 = slab_k(i);
        const bool act = i < n_own;
        const bool full = act && k0 >= lo_max && k0 + SMOL_SLAB <= hi_min;
        read_k(st_k, kf);
        read_v(st_v, vnow);
        /* slab 'steps' (K read in the last step, its S unused) and later ones are not staged */
        if constexpr (B1) {
            if (i + 2 < steps) dma(slab_k(i + 2), (i + 2) % NSTG);
        } else if (!odd) {
            if (i + 3 < steps) dma(slab_k(i + 3), (i + 3) % NSTG);
            if (i + 4 < steps) dma(slab_k(i + 4), (i + 4) % NSTG);
        }
        /* the LDS reads and transfers go out first, then P.V of the
         * previous slab (its fragments are in registers) covers the reads'
         * latency; the compiler would otherwise start the S MFMAs, which
         * wait for this step's K fragments (measured 4% on the C2 shape) */
        __builtin_amdgcn_sched_barrier(0);
        pv(vprev, pprev);
        __builtin_amdgcn_sched_barrier(0);
        prep_s(k0, act, !full, scur);
        float psum[NT];
        const bool hit = expo(scur, pnow, psum);
        qk(kf, st_k, snext);
        if (hit) rescale(scur, pnow, snext, psum);
        if constexpr (PREC) {
#pragma unroll
            for (int nt = 0; nt < NT; nt++) l[nt] += psum[nt];
        }
        /* only odd steps end in a barrier: it publishes the pair issued by
         * the step before, and the even step after it refills the stages of
         * slabs i-1 and i, whose last reads (steps i-1 and i) it orders
         * (three stages: every step, for its one slab) */
        if (B1 || odd) {
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            __syncthreads();
        }
        st_k = st_k + 1 == NSTG ? 0 : st_k + 1;
        st_v = st_v + 1 == NSTG ? 0 : st_v + 1;
    };
    int i = 0;
    for (; i + 2 <= steps; i += 2) {
        step(i, false, sa, sb, vfa, vfb, pfa, pfb);
        step(i + 1, true, sb, sa, vfb, vfa, pfb, pfa);
    }
    if (i < steps) {
        step(i, false, sa, sb, vfa, vfb, pfa, pfb);
        pv(vfb, pfb);
    } else {
        pv(vfa, pfa);
    }
#pragma unroll
    for (int nt = 0; nt < NT; nt++) l[nt] = PREC ? row_sum4(l[nt]) : lsum[nt][0];

    if constexpr (ONE) {
        if (it.n_split == 1) {
            /* the item holds its tile's every key: the rows are final */
#pragma unroll
            for (int nt = 0; nt < NT; nt++) {
                if (!valid[nt]) continue;
                const int r = it.row0 + (wg * NT + nt) * 16 + c;
                const int qi = r / G, hg = r - qi * G;
                const float inv = l[nt] > 0.0f ? 1.0f / l[nt] : 0.0f;
                float *orow = p.out + ((long long)(b.out_tok0 + qi) * p.Hq + (g * G + hg)) * HD;
#pragma unroll
                for (int dt = 0; dt < DT; dt++) {
                    const int d = 16 * dt + 4 * j;
                    if (HD % 16 != 0 && d >= HD) continue;
                    st_stream(orow + d, o[nt][dt] * inv);
                }
            }
        } else {
            /* a split item: publish the unnormalised rows and (m, l) into
             * slot `part` with device-coherent stores, count in once, and the
             * group's last workgroup merges (as k_attn_fa's split items) */
            const long long pbase = ((long long)it.part * p.Hkv + g) * ROWS;
            const rsrc_t ro = make_rsrc(p.part_o + pbase * HD, (long long)ROWS * HD * 4);
            const rsrc_t rml = make_rsrc(p.part_ml + pbase * 2, (long long)ROWS * 2 * 4);
#pragma unroll
            for (int nt = 0; nt < NT; nt++) {
                const int rr = (wg * NT + nt) * 16 + c;
#pragma unroll
                for (int dt = 0; dt < DT; dt++) {
                    const int d = 16 * dt + 4 * j;
                    if (HD % 16 != 0 && d >= HD) continue;
                    store_f4_sc1(ro, (unsigned)((rr * HD + d) * 4), o[nt][dt]);
                }
                if (j == 0) store_f2_sc1(rml, (unsigned)(rr * 8), m[nt], l[nt]);
            }
            __atomic_signal_fence(__ATOMIC_SEQ_CST);
            __builtin_amdgcn_s_waitcnt(0);
            __atomic_signal_fence(__ATOMIC_SEQ_CST);
            __syncthreads(); /* every wave's stores are acknowledged (and every stage read is done) */
            if (tid == 0) {
                const int prev = __hip_atomic_fetch_add(p.counters + ((long long)it.group * p.Hkv + g) * SK_COUNTER_STRIDE,
                                                        1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                s_last = prev == it.n_split - 1;
            }
            __syncthreads();
            if (s_last)
                fb_merge<HD, ROWS, 64 * WPG>(p.part_o, p.part_ml, p.counters, p.out, p.Hkv, p.Hq, p.G, it, g, tid,
                                             reinterpret_cast<float *>(smem));
        }
        if (next < 0) break;
        item = next;
        __syncthreads(); /* the epilogue is done with LDS */
        continue;
    }

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
            st_stream(orow + d, o[nt][dt] * a0 + o1 * a1);
        }
    }
    if (next < 0) break;
    item = next;
    __syncthreads(); /* the epilogue is done with LDS */
    } /* items */
}

/* nt: 1 or 2 row tiles per wave with two key groups (64-row items), or 0:
 * one key group of eight waves (128-row items) */
template <int HD, bool PREC>
static int launch_fb_v(const SkParams *sp, dim3 grid, int nt, hipStream_t st, hipEvent_t e0, hipEvent_t e1) {
    const bool cap = sp->cap2 > 0.0f;
    if (nt == 0) {
        if (cap) hipExtLaunchKernelGGL((k_attn_fb<HD, 1, true, PREC, true>), grid, dim3(512), 0, st, e0, e1, 0, *sp);
        else hipExtLaunchKernelGGL((k_attn_fb<HD, 1, false, PREC, true>), grid, dim3(512), 0, st, e0, e1, 0, *sp);
    } else if (nt == 1) {
        if (cap) hipExtLaunchKernelGGL((k_attn_fb<HD, 1, true, PREC, false>), grid, dim3(512), 0, st, e0, e1, 0, *sp);
        else hipExtLaunchKernelGGL((k_attn_fb<HD, 1, false, PREC, false>), grid, dim3(512), 0, st, e0, e1, 0, *sp);
    } else if (nt == 2) {
        if (cap) hipExtLaunchKernelGGL((k_attn_fb<HD, 2, true, PREC, false>), grid, dim3(256), 0, st, e0, e1, 0, *sp);
        else hipExtLaunchKernelGGL((k_attn_fb<HD, 2, false, PREC, false>), grid, dim3(256), 0, st, e0, e1, 0, *sp);
    } else return -1;
    return hipGetLastError() == hipSuccess ? 0 : -3;
}

/* Q from the inputs (precise QK^T, head_dim 64 or 128, nt 0 or 1) */
template <int HD>
static int launch_fb_qin(const SkParams *sp, dim3 grid, int nt, hipStream_t st, hipEvent_t e0, hipEvent_t e1) {
    if constexpr (HD == 64 || HD == 128) {
        const bool cap = sp->cap2 > 0.0f;
        if (nt == 0) {
            if (cap) hipExtLaunchKernelGGL((k_attn_fb<HD, 1, true, true, true, true>), grid, dim3(512), 0, st, e0, e1, 0, *sp);
            else hipExtLaunchKernelGGL((k_attn_fb<HD, 1, false, true, true, true>), grid, dim3(512), 0, st, e0, e1, 0, *sp);
        } else if (nt == 1) {
            if (cap) hipExtLaunchKernelGGL((k_attn_fb<HD, 1, true, true, false, true>), grid, dim3(512), 0, st, e0, e1, 0, *sp);
            else hipExtLaunchKernelGGL((k_attn_fb<HD, 1, false, true, false, true>), grid, dim3(512), 0, st, e0, e1, 0, *sp);
        } else {
            return -1;
        }
        return hipGetLastError() == hipSuccess ? 0 : -3;
    }
    return -1;
}

/* precise QK^T (fp16 hi + lo operands) when the Q scratch has its lo part
 * (or Q comes from the inputs) */
template <int HD>
static int launch_fb_hd(const SkParams *sp, int n_items, int nt, hipStream_t st, hipEvent_t e0, hipEvent_t e1) {
    const int n_wg = sp->n_wg > 0 ? sp->n_wg : n_items; /* workgroups per kv head: the heads of the lists */
    const dim3 grid(n_wg * sp->Hkv);
    if (sp->q_in) {
        if (!sp->kf_lo) return -1;
        return launch_fb_qin<HD>(sp, grid, nt, st, e0, e1);
    }
    if (sp->qs_lo) {
        if (!sp->kf_lo) return -1;
        return launch_fb_v<HD, true>(sp, grid, nt, st, e0, e1);
    }
    return launch_fb_v<HD, false>(sp, grid, nt, st, e0, e1);
}

/* k_attn_fb: every key in the fresh buffers; nt: 1 or 2 row tiles per wave
 * over 64-row items (512 threads for nt 1, 256 for nt 2), or 0: 128-row items
 * of one key group (512 threads; split items merge through part_o / part_ml
 * and the counters); sp->n_wg workgroups per kv head (0: one per item) each
 * run their list of items; e0 / e1 (may be null): events recorded around the
 * kernel alone */
extern "C" int smol_launch_fb(const SkParams *sp, int hd, int n_items, int nt, hipStream_t st, hipEvent_t e0,
                              hipEvent_t e1) {
    if (n_items <= 0) return 0;
    switch (hd) {
    case 64: return launch_fb_hd<64>(sp, n_items, nt, st, e0, e1);
    case 72: return launch_fb_hd<72>(sp, n_items, nt, st, e0, e1);
    case 80: return launch_fb_hd<80>(sp, n_items, nt, st, e0, e1);
    case 96: return launch_fb_hd<96>(sp, n_items, nt, st, e0, e1);
    case 128: return launch_fb_hd<128>(sp, n_items, nt, st, e0, e1);
    default: return -1;
    }
}

