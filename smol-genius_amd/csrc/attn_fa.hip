/*
 * attn_fa.hip - k_attn_fa: prefill over a cache prefix (and head_dim 256).
 */
#include "attn_splitk.h"

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
/* PREC (precise QK^T): a stage holds the K image twice, fp16 hi then fp16
 * lo (zero for bf16 cache slabs, which fp16 holds exactly), then V^T. */
template <int HD, bool PREC>
struct FaGeom {
    static constexpr int KS = (HD + 31) / 32;
    static constexpr int DT = (HD + 15) / 16;
    static constexpr int HDP = KS * 32;
    static constexpr int KROW = HD <= 128 ? 256 : 512;
    static constexpr int K_BYTES = SMOL_SLAB * KROW;
    static constexpr int KPARTS = PREC ? 2 : 1;
    static constexpr int V_BYTES = 16 * DT * 64;
    static constexpr int STAGE = KPARTS * K_BYTES + V_BYTES;
    static constexpr int CK = SMOL_SLAB * HD / 8; /* 16-byte chunks in a K (or V^T) slab */
    static constexpr int PER = (CK + 255) / 256;  /* K (and V) chunks per thread */
};

template <int HD, int NT, int W, bool PREC>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(W, W))) void k_attn_fa(SkParams p) {
    using Gm = FaGeom<HD, PREC>;
    constexpr int KS = Gm::KS, DT = Gm::DT, HDP = Gm::HDP, KROW = Gm::KROW;
    constexpr int STAGE = Gm::STAGE, K_BYTES = Gm::K_BYTES, CK = Gm::CK, PER = Gm::PER;
    constexpr int ROWS = 4 * 16 * NT;
    constexpr unsigned SLAB_BYTES = SMOL_SLAB * HD * 2;
    /* LDS stages: slabs i, i+1 read while i+2 is stored (PREC: three, the
     * larger stages leave no room for a fourth) */
    constexpr int NSTG = PREC ? 3 : 4;
    constexpr int VOFF = Gm::KPARTS * K_BYTES; /* V^T within a stage */
    /* register sets of staged slabs in flight (two for PREC at head_dim 256,
     * whose K lo part would not leave registers for four) */
    constexpr int SETS = W == 1 && !(PREC && HD > 128) ? 4 : 2;
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
    h8 qfl[PREC ? NT : 1][KS]; /* PREC: Q lo */
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
        {
            const long long qoff = (long long)g * p.qs_head_stride + (long long)(b.q_row0 + (valid ? r : 0)) * HDP;
            const _Float16 *qrow = p.qs + qoff;
#pragma unroll
            for (int ks = 0; ks < KS; ks++) qf[nt][ks] = valid ? load_h8(qrow + 32 * ks + 8 * j) : zero_h8();
            if constexpr (PREC) {
                const _Float16 *qrl = p.qs_lo + qoff;
#pragma unroll
                for (int ks = 0; ks < KS; ks++) qfl[nt][ks] = valid ? load_h8(qrl + 32 * ks + 8 * j) : zero_h8();
            }
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
    /* the fresh K's lo part; a cache slab's lo part reads zeros (empty range) */
    const rsrc_t rkl_f = PREC ? make_rsrc(p.kf_lo + (long long)g * p.fcap * HD, (long long)p.fcap * HD * 2) : rk_f;
    const rsrc_t r_none = make_rsrc(nullptr, 0);
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
        lv_off[e] = (unsigned)(VOFF + d * 64 + 16 * (jj ^ ((d >> 1) & 3)));
        g_off[e] = c_ok[e] ? (unsigned)(q * 16) : OOB_OFF;
    }
    /* this lane's fragment addresses within a stage */
    const int kt_row = 8 * (c >> 2) + (c & 3);
    unsigned kfo[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ks++) kfo[ks] = (unsigned)(kt_row * KROW + 16 * ((4 * ks + j) ^ c));
    const unsigned vfo = (unsigned)(VOFF + c * 64 + 16 * (j ^ ((c >> 1) & 3)));

    struct Stg {
        uint4 k[PER], v[PER];
        uint4 kl[PREC ? PER : 1]; /* PREC: K lo */
        bool bf; /* bf16 cache slab (widen to fp16 when storing) */
    };
    auto issue = [&](int k0, Stg &s) __attribute__((always_inline)) {
        const bool fr = k0 >= b.fresh_pos0;
        const int kr = fr ? k0 + it.fresh_off : k0;
        const unsigned so = (unsigned)(kr / SMOL_SLAB) * SLAB_BYTES;
        const rsrc_t rk = fr ? rk_f : rk_c, rv = fr ? rv_f : rv_c;
#pragma unroll
        for (int e = 0; e < PER; e++) s.k[e] = bload(rk, g_off[e], so);
        if constexpr (PREC) {
            const rsrc_t rkl = fr ? rkl_f : r_none;
#pragma unroll
            for (int e = 0; e < PER; e++) s.kl[e] = bload(rkl, g_off[e], so);
        }
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
                if (bf16x8_out_of_h_range(kw) || bf16x8_out_of_h_range(vw)) {
                    if (p.range_flag) *p.range_flag = 1;
                }
                const h8 kh = bf16x8_to_h8(kw), vh = bf16x8_to_h8(vw);
                kw = *reinterpret_cast<const uint4 *>(&kh);
                vw = *reinterpret_cast<const uint4 *>(&vh);
            }
            *reinterpret_cast<uint4 *>(base + lk_off[e]) = kw;
            if constexpr (PREC) *reinterpret_cast<uint4 *>(base + lk_off[e] + K_BYTES) = s.kl[e];
            *reinterpret_cast<uint4 *>(base + lv_off[e]) = vw;
        }
    };
    auto lds_h8 = [&](int stage, unsigned off) __attribute__((always_inline)) -> h8 {
        const uint4 w = *reinterpret_cast<const uint4 *>(smem + stage * STAGE + off);
        return *reinterpret_cast<const h8 *>(&w);
    };
    /* S^T - m = K.Q^T - m of the slab in `stage` (raw S with a softcap);
     * PREC: Khi.Qhi + Khi.Qlo + Klo.Qhi */
    const bool capped = p.cap2 > 0.0f;
    auto qk = [&](int stage, f4 (&sacc)[NT][2]) __attribute__((always_inline)) {
#pragma unroll
        for (int t = 0; t < 2; t++) {
            h8 kfr[KS], kfl[PREC ? KS : 1];
#pragma unroll
            for (int ks = 0; ks < KS; ks++) kfr[ks] = lds_h8(stage, kfo[ks] + t * 4 * KROW);
            if constexpr (PREC) {
#pragma unroll
                for (int ks = 0; ks < KS; ks++) kfl[ks] = lds_h8(stage, kfo[ks] + t * 4 * KROW + K_BYTES);
            }
#pragma unroll
            for (int nt = 0; nt < NT; nt++) {
                f4 acc = capped ? f4{0.f, 0.f, 0.f, 0.f} : negm[nt];
#pragma unroll
                for (int ks = 0; ks < KS; ks++) {
                    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(kfr[ks], qf[nt][ks], acc, 0, 0, 0);
                    if constexpr (PREC) {
                        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(kfr[ks], qfl[nt][ks], acc, 0, 0, 0);
                        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(kfl[ks], qf[nt][ks], acc, 0, 0, 0);
                    }
                }
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
    /* P = exp2(S - m) as fp16 (PREC: hi [0] + lo [1]), row sums */
    constexpr int NP = PREC ? 2 : 1;
    auto expo = [&](const float (&sv)[NT][8], h8 (&pf)[NP][NT]) __attribute__((always_inline)) {
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
            float pe[8];
#pragma unroll
            for (int e = 0; e < 8; e++) pe[e] = __builtin_amdgcn_exp2f(sv[nt][e]);
            if constexpr (PREC) {
#pragma unroll
                for (int e = 0; e < 8; e += 2) {
                    uint32_t hi, lo;
                    split_h2(pe[e], pe[e + 1], hi, lo);
                    reinterpret_cast<uint32_t *>(&pf[0][nt])[e >> 1] = hi;
                    reinterpret_cast<uint32_t *>(&pf[1][nt])[e >> 1] = lo;
                }
            } else {
#pragma unroll
                for (int e = 0; e < 8; e++) pf[0][nt][e] = (_Float16)pe[e];
            }
            l[nt] += ((pe[0] + pe[1]) + (pe[2] + pe[3])) + ((pe[4] + pe[5]) + (pe[6] + pe[7]));
        }
    };
    auto pv = [&](int stage, const h8 (&pf)[NP][NT]) __attribute__((always_inline)) {
#pragma unroll
        for (int dt = 0; dt < DT; dt++) {
            const h8 vfr = lds_h8(stage, vfo + dt * 1024);
#pragma unroll
            for (int nt = 0; nt < NT; nt++) {
                o[nt][dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vfr, pf[0][nt], o[nt][dt], 0, 0, 0);
                if constexpr (PREC) o[nt][dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vfr, pf[1][nt], o[nt][dt], 0, 0, 0);
            }
        }
    };

    /* The item's n slabs are walked in a rotated order (slab (i + rot) mod n
     * at step i; the softmax does not depend on the order), so the
     * workgroups of one head, which start together, read different slabs.
     * Slab i sits in LDS stage i % NSTG from the barrier that ends step i-2
     * to the one that ends step i (with three stages, slab i+2 goes into the
     * stage of slab i-1, whose last read, step i-1, precedes that barrier). Step i: softmax front of slab i; then its
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
        /* u = i % 4, compile-time in each unrolled step (the register sets);
         * the stage of slab i is i % NSTG */
        auto step = [&](int i, auto u_tag, f4 (&scur)[NT][2], f4 (&snext)[NT][2]) __attribute__((always_inline)) {
            constexpr int u = decltype(u_tag)::value;
            const int sg = NSTG == 4 ? (i & 3) : i % NSTG;
            const int sg1 = sg + 1 == NSTG ? 0 : sg + 1, sg2 = sg1 + 1 == NSTG ? 0 : sg1 + 1;
            float sv[NT][8];
            h8 pf[NP][NT];
            front(slab_k(i), scur, sv);
            qk(sg1, snext);
            expo(sv, pf);
            pv(sg, pf);
            Stg &s2 = st[(u + 2) % SETS];
            store(s2, sg2);
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

/* ev0 / ev1 (may be null): events recorded around the kernel alone */
/* precise QK^T when the Q scratch has its lo part (not built for two row
 * tiles at two waves per SIMD, whose registers it would not fit) */
template <int HD, int NT, int W>
static int launch_fa_v(const SkParams *sp, dim3 grid, hipStream_t st, hipEvent_t ev0, hipEvent_t ev1) {
    if (sp->qs_lo) {
        if constexpr (NT == 2 && W == 2) return -1;
        else hipExtLaunchKernelGGL((k_attn_fa<HD, NT, W, true>), grid, dim3(256), 0, st, ev0, ev1, 0, *sp);
    } else {
        hipExtLaunchKernelGGL((k_attn_fa<HD, NT, W, false>), grid, dim3(256), 0, st, ev0, ev1, 0, *sp);
    }
    return 0;
}

/* w: waves per SIMD the kernel is built for (2 with fewer staged slabs) */
template <int HD>
static int launch_fa_hd(const SkParams *sp, int n_items, int nt, int w, hipStream_t st, hipEvent_t e0, hipEvent_t e1) {
    const dim3 grid(n_items * sp->Hkv);
    int rc = -1;
    if (nt == 1 && w == 1) rc = launch_fa_v<HD, 1, 1>(sp, grid, st, e0, e1);
    else if constexpr (HD <= 128) { /* two tiles or two waves per SIMD fit the registers */
        if (nt == 1 && w == 2) rc = launch_fa_v<HD, 1, 2>(sp, grid, st, e0, e1);
        else if (nt == 2 && w == 1) rc = launch_fa_v<HD, 2, 1>(sp, grid, st, e0, e1);
        else if (nt == 2 && w == 2) rc = launch_fa_v<HD, 2, 2>(sp, grid, st, e0, e1);
    }
    if (rc) return rc;
    return hipGetLastError() == hipSuccess ? 0 : -3;
}

extern "C" int smol_launch_fa(const SkParams *sp, int hd, int n_items, int nt, int w, hipStream_t st, hipEvent_t e0,
                              hipEvent_t e1) {
    if (n_items <= 0) return 0;
    switch (hd) {
    case 64: return launch_fa_hd<64>(sp, n_items, nt, w, st, e0, e1);
    case 72: return launch_fa_hd<72>(sp, n_items, nt, w, st, e0, e1);
    case 80: return launch_fa_hd<80>(sp, n_items, nt, w, st, e0, e1);
    case 96: return launch_fa_hd<96>(sp, n_items, nt, w, st, e0, e1);
    case 128: return launch_fa_hd<128>(sp, n_items, nt, w, st, e0, e1);
    case 256: return launch_fa_hd<256>(sp, n_items, nt, w, st, e0, e1);
    default: return -1;
    }
}

