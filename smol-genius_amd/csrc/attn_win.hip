/*
 * attn_win.hip - k_attn_win: windowed bidirectional attention with each
 * window's keys resident in LDS (common/kernels/attention.c:32-77, the
 * vision encoders' and the audio encoder's windows).
 *
 * A workgroup owns one 128-row tile of one (window, head) (or, when the
 * windows are too few to fill the GPU that way, a 64-row tile whose two
 * groups of four waves take the first and second half of the window's
 * slabs and merge their softmax states through LDS at the end): its eight
 * waves read the window's K and V rows straight from the inputs (fp32 or bf16),
 * convert them to fp16 (bf16 exactly, fp32 rounded to nearest even, as the
 * pre-pass of the other kernels does) and write them once into an LDS image
 * of the whole window; Q is read into registers the same way, times
 * scale * log2 e. After one barrier every wave runs through the window's
 * 32-key slabs with no further synchronisation: S = K.Q^T and O += V^T.P^T
 * on v_mfma_f32_16x16x32_f16, the softmax in fp32 with an exact running
 * maximum per slab. No pre-pass and no staging buffer in HBM: the inputs
 * are read once per row tile (a 104-token audio window is one tile; the
 * tiles of a window share its K and V in one XCD's L2).
 *
 * LDS image of slab s (the layout k_attn_fb reads, conflict-free):
 *   K   : 32 key rows of 256 bytes; 16-byte chunk cb of key row r sits in
 *         slot cb ^ f(r), f(r) = (r & 3) | ((r >> 3) & 3) << 2.
 *   V^T : 16*DT rows of 64 bytes (32 keys); chunk jc (keys 8jc..8jc+7) of
 *         row d sits in slot jc ^ ((d >> 1) & 3).
 *   V   : (bf16 inputs with the precise products, in place of V^T) 32 key
 *         rows of 256 bytes as in the inputs; chunk q of key row r sits in
 *         slot q ^ 2 fv(r), fv(r) = (r & 3) | ((r >> 3) & 1) << 2, and the
 *         V^T fragments are read from it with the LDS transpose read.
 * Columns past head_dim and keys past the window are zeros.
 */
#include "attn_device.h"

namespace {

/* KLO: the slab image holds K twice, fp16 hi then fp16 lo (precise QK^T on
 * fp32 inputs; bf16 inputs are exact in fp16 and need no lo part). VROW: V
 * as rows of the inputs (256-byte rows) instead of the V^T image. */
template <int HD, bool KLO, bool VROW>
struct WinGeom {
    static constexpr int KS = (HD + 31) / 32;  /* 32-wide d chunks of a K fragment */
    static constexpr int DT = (HD + 15) / 16;  /* 16-wide d tiles of the output */
    static constexpr int HDP = KS * 32;
    static constexpr int KROW = 256;
    static constexpr int K_BYTES = SMOL_SLAB * KROW;
    static constexpr int KPARTS = KLO ? 2 : 1;
    static constexpr int V_BYTES = VROW ? SMOL_SLAB * KROW : 16 * DT * 64;
    static constexpr int SLABB = KPARTS * K_BYTES + V_BYTES;
    static constexpr int NS_MAX = (160 * 1024) / SLABB; /* slabs the LDS holds */
};

/* 8 elements of an input row as fp32 (bf16 widened exactly) */
template <bool BF>
struct Raw8In {
    uint4 a, b;
    __device__ __forceinline__ void load(const void *base, long long idx) {
        if constexpr (BF) {
            a = *reinterpret_cast<const uint4 *>(reinterpret_cast<const uint16_t *>(base) + idx);
        } else {
            const float *f = reinterpret_cast<const float *>(base) + idx;
            a = *reinterpret_cast<const uint4 *>(f);
            b = *reinterpret_cast<const uint4 *>(f + 4);
        }
    }
    __device__ __forceinline__ void unpack(float *v) const {
        if constexpr (BF) {
            unpack_bf16x8(a, v);
        } else {
            v[0] = __uint_as_float(a.x); v[1] = __uint_as_float(a.y); v[2] = __uint_as_float(a.z);
            v[3] = __uint_as_float(a.w); v[4] = __uint_as_float(b.x); v[5] = __uint_as_float(b.y);
            v[6] = __uint_as_float(b.z); v[7] = __uint_as_float(b.w);
        }
    }
};

} // namespace

/* PREC: QK^T on fp16 hi + lo operands, Khi.Qhi + Khi.Qlo (+ Klo.Qhi for
 * fp32 inputs) */
template <int HD, bool BF, int NS, bool PREC>
__global__ __launch_bounds__(WIN_TPB) void k_attn_win(const WinParams p) {
    constexpr bool KLO = PREC && !BF;
    /* BFK (bf16 inputs, precise): K and V stay bf16 and go straight into
     * LDS (buffer_load ... lds, no registers), the V^T fragments come from
     * the V rows by the LDS transpose read, and the products run on bf16
     * MFMA with Q and P as bf16 hi + lo (K and V are exact, Q and P carry 16
     * bits) */
    constexpr bool BFK = BF && PREC;
    using Gm = WinGeom<HD, KLO, BFK>;
    constexpr int KS = Gm::KS, DT = Gm::DT, HDP = Gm::HDP, KROW = Gm::KROW;
    constexpr int K_BYTES = Gm::K_BYTES, SLABB = Gm::SLABB;
    static_assert(HD % 8 == 0 && HD <= 128, "head_dim");
    static_assert(NS * SLABB <= 160 * 1024, "LDS");
    __shared__ __attribute__((aligned(1024))) unsigned char smem[NS * SLABB];

    const int tid = threadIdx.x;
    const int lane = tid & 63, c = lane & 15, j = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    /* Unit u = (window u / H, head u % H) has up to tpu tiles of WIN_ROWS. The
     * units go round-robin over the XCDs and a unit's tiles to one XCD
     * (workgroup b runs on XCD b % n_xcc), so the window's K and V come
     * from memory into one L2 and its tiles share them there. */
    const int b = blockIdx.x, nx = p.n_xcc;
    const int x = b % nx, slot = b / nx;
    const int u = (slot / p.tpu) * nx + x, tile = slot % p.tpu;
    if (u >= p.n_windows * p.H) return;
    const int w = u / p.H, h = u - w * p.H;
    const int w0 = p.ws[w], len = p.ws[w + 1] - w0;
    const int split = p.ksplit == 2;
    const int row0 = tile * (WIN_ROWS >> split);
    if (row0 >= len) return;
    const int nslab = (len + SMOL_SLAB - 1) / SMOL_SLAB; /* <= NS (the host's choice of build) */
    const long long hoff = (long long)h * HD;
    /* the wave's rows and its group's slabs [s_lo, s_hi) */
    const int grp = split ? wave >> 2 : 0, wr = split ? wave & 3 : wave;
    const int s_half = (nslab + 1) >> 1;
    const int s_lo = grp == 0 ? 0 : s_half, s_hi = split && grp == 0 ? s_half : nslab;

    /* ---- Q fragments of this wave's 16 rows: row rq, dims 32 ks + 8 j ---- */
    const int rq = row0 + 16 * wr + c;
    const bool q_ok = rq < len;
    Raw8In<BF> qin[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ks++) {
        const int d0 = 32 * ks + 8 * j;
        const bool ok = q_ok && (HDP == HD || d0 < HD);
        /* rows and columns past the window read the window's first row */
        qin[ks].load(p.q, (long long)(w0 + (ok ? rq : 0)) * p.row_stride + hoff + (ok ? d0 : 0));
    }

    /* ---- the window's K and V into LDS ----
     * K: LDS chunk e (key e / 16, slot e % 16 of its 256-byte row) receives
     * the key's 8 dims cb = slot ^ f(key % 32): a wave writes 1 KB of
     * consecutive LDS, and the 16 lanes of a key read its row. Slots past
     * HDP are never read and are skipped.
     * V^T: 8 x 8 blocks, below.
     * All loads of a part are issued before any is used; out-of-range
     * lanes read the window's first row and write zeros. */
    constexpr int CK = HDP / 8;
    const int nkey = nslab * SMOL_SLAB;
    constexpr int NKT = NS * SMOL_SLAB * 16 / WIN_TPB;              /* K chunks per thread (the build's capacity) */
    constexpr int RK = (BF ? 16 : 8) < NKT ? (BF ? 16 : 8) : NKT;  /* K chunks a round */
    constexpr int NDB = 2 * DT;                                     /* 8-row blocks of a V^T image */
    constexpr int NVB = (NS * 4 * NDB + WIN_TPB - 1) / WIN_TPB;     /* 8 x 8 V blocks per thread */
    auto k_chunk = [&](int e, int &key, int &slot, int &rr, int &cb) __attribute__((always_inline)) {
        key = e >> 4; slot = e & 15; rr = key & 31;
        cb = slot ^ ((rr & 3) | (((rr >> 3) & 3) << 2));
    };
    auto k_issue = [&](int r0, Raw8In<BF> (&in)[RK]) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < RK; u++) {
            int key, slot, rr, cb;
            k_chunk(tid + WIN_TPB * (r0 + u), key, slot, rr, cb);
            const bool ok = r0 + u < NKT && key < len && cb * 8 < HD;
            in[u].load(p.k, (long long)(w0 + (ok ? key : 0)) * p.row_stride + hoff + (ok ? cb * 8 : 0));
        }
    };
    auto k_store = [&](int r0, const Raw8In<BF> (&in)[RK]) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < RK; u++) {
            int key, slot, rr, cb;
            k_chunk(tid + WIN_TPB * (r0 + u), key, slot, rr, cb);
            if (r0 + u >= NKT || key >= nkey || cb >= CK) continue;
            float v[8];
            in[u].unpack(v);
            if (key >= len || cb * 8 >= HD) {
#pragma unroll
                for (int i = 0; i < 8; i++) v[i] = 0.0f;
            }
            note_h_range(p.range_flag, v);
            unsigned char *kd = smem + (key >> 5) * SLABB + rr * KROW + 16 * slot;
            if constexpr (KLO) {
                uint4 hi, lo;
                pack_h8_hilo(v, hi, lo);
                *reinterpret_cast<uint4 *>(kd) = hi;
                *reinterpret_cast<uint4 *>(kd + K_BYTES) = lo;
            } else {
                *reinterpret_cast<uint4 *>(kd) = pack_h8(v);
            }
        }
    };
    /* V^T: block e (keys 8 kb .. 8 kb + 7, dims 8 db .. 8 db + 7; consecutive
     * lanes take consecutive dim blocks of a key row, so a load instruction
     * reads whole row segments) is eight 16-byte row loads, transposed in
     * registers into eight 16-byte chunks of V^T rows */
    const int nvb = nslab * 4 * NDB;
    auto v_issue = [&](int u, Raw8In<BF> (&in)[8]) __attribute__((always_inline)) {
        const int e = tid + WIN_TPB * u, db = e % NDB, kb = e / NDB;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const bool ok = e < nvb && 8 * kb + i < len && 8 * db < HD;
            in[i].load(p.v, (long long)(w0 + (ok ? 8 * kb + i : 0)) * p.row_stride + hoff + (ok ? 8 * db : 0));
        }
    };
    auto v_store = [&](int u, const Raw8In<BF> (&in)[8]) __attribute__((always_inline)) {
        const int e = tid + WIN_TPB * u, db = e % NDB, kb = e / NDB;
        if (e >= nvb) return;
        uint4 r[8]; /* fp16 rows: r[i] holds dims 8 db .. 8 db + 7 of key 8 kb + i */
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const bool ok = 8 * kb + i < len && 8 * db < HD;
            float v[8];
            in[i].unpack(v);
            if (!ok) {
#pragma unroll
                for (int t = 0; t < 8; t++) v[t] = 0.0f;
            }
            note_h_range(p.range_flag, v);
            r[i] = pack_h8(v);
        }
        const int sl = kb >> 2, jc = kb & 3;
        unsigned char *vbase = smem + sl * SLABB + Gm::KPARTS * K_BYTES;
#pragma unroll
        for (int dd = 0; dd < 8; dd++) {
            /* column dd: key pairs (2m, 2m + 1) of dim 8 db + dd */
            uint32_t c4[4];
#pragma unroll
            for (int mm = 0; mm < 4; mm++) {
                const uint32_t x = reinterpret_cast<const uint32_t *>(&r[2 * mm])[dd >> 1];
                const uint32_t y = reinterpret_cast<const uint32_t *>(&r[2 * mm + 1])[dd >> 1];
                c4[mm] = (dd & 1) ? (x >> 16) | (y & 0xFFFF0000u) : (x & 0xFFFFu) | (y << 16);
            }
            const int d = 8 * db + dd;
            *reinterpret_cast<uint4 *>(vbase + d * 64 + 16 * (jc ^ ((d >> 1) & 3))) = make_uint4(c4[0], c4[1], c4[2], c4[3]);
        }
    };
    if constexpr (BFK) {
        /* K and V: each wave transfers row quad `wave` (1 KB of each image)
         * of every slab; lane l lands at slot l % 16 of row 4 wave + l / 16,
         * reading the key's chunk slot ^ f(row) (K) or slot ^ 2 fv(row) (V);
         * chunks past head_dim and keys past the window are out of the
         * buffer's range (zeros). The range is the window's rows, whose first
         * element is the base. */
        const long long wbase = (long long)w0 * p.row_stride + hoff, wbytes = ((long long)(len - 1) * p.row_stride + HD) * 2;
        const rsrc_t rk = make_rsrc(reinterpret_cast<const uint16_t *>(p.k) + wbase, wbytes);
        const rsrc_t rv = make_rsrc(reinterpret_cast<const uint16_t *>(p.v) + wbase, wbytes);
        const int rr = 4 * wave + (lane >> 4), ks16 = lane & 15;
        const int cbk = ks16 ^ ((rr & 3) | (((rr >> 3) & 3) << 2));
        const int cbv = ks16 ^ (2 * ((rr & 3) | (((rr >> 3) & 1) << 2)));
        const unsigned lds0 = (unsigned)(size_t)smem + (unsigned)(wave * 1024);
#pragma unroll
        for (int e = 0; e < NS; e++) {
            const int key = e * SMOL_SLAB + rr;
            const unsigned offk = key < len && cbk < HD / 8 ? (unsigned)((key * p.row_stride + cbk * 8) * 2) : OOB_OFF;
            const unsigned offv = key < len && cbv < HD / 8 ? (unsigned)((key * p.row_stride + cbv * 8) * 2) : OOB_OFF;
            if (e < nslab) {
                dma_1k(rk, offk, 0u, __builtin_amdgcn_readfirstlane(lds0 + (unsigned)(e * SLABB)));
                dma_1k(rv, offv, 0u, __builtin_amdgcn_readfirstlane(lds0 + (unsigned)(e * SLABB + K_BYTES)));
            }
        }
    } else {
        /* the first rounds of K and V go out together */
        Raw8In<BF> kin[RK];
        Raw8In<BF> vin[8];
        k_issue(0, kin);
        v_issue(0, vin);
        k_store(0, kin);
        v_store(0, vin);
#pragma unroll
        for (int r0 = RK; r0 < NKT; r0 += RK) {
            k_issue(r0, kin);
            k_store(r0, kin);
        }
#pragma unroll
        for (int u = 1; u < NVB; u++) {
            v_issue(u, vin);
            v_store(u, vin);
        }
    }
    h8 qf[KS], qfl[PREC ? KS : 1];
    b8 qbh[BFK ? KS : 1], qbl[BFK ? KS : 1]; /* BFK: Q as bf16 hi + lo */
#pragma unroll
    for (int ks = 0; ks < KS; ks++) {
        float v[8];
        qin[ks].unpack(v);
        const bool ok = q_ok && (HDP == HD || 32 * ks + 8 * j < HD);
#pragma unroll
        for (int i = 0; i < 8; i++) v[i] = ok ? v[i] * p.qscale : 0.0f;
        if constexpr (BFK) {
            split8(v, qbh[ks], qbl[ks]);
            continue;
        }
        note_h_range(p.range_flag, v);
        if constexpr (PREC) {
            uint4 hw, lw;
            pack_h8_hilo(v, hw, lw);
            qf[ks] = *reinterpret_cast<const h8 *>(&hw);
            qfl[ks] = *reinterpret_cast<const h8 *>(&lw);
        } else {
            const uint4 hw = pack_h8(v);
            qf[ks] = *reinterpret_cast<const h8 *>(&hw);
        }
    }
    /* the LDS transfers (BFK) have landed before the barrier */
    if constexpr (BFK) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();

    /* ---- the slabs: S^T = K.Q^T (lane (c, j) holds keys 8 j + 4 t + i of
     * row c in s[t][i]), exact running max, P in fp16, O^T += V^T.P^T and
     * the row sums against a fragment of ones ---- */
    const int kt_row = 8 * (c >> 2) + (c & 3);
    unsigned kfo[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ks++) kfo[ks] = (unsigned)(kt_row * KROW + 16 * ((4 * ks + j) ^ c));
    const unsigned vfo = (unsigned)(Gm::KPARTS * K_BYTES + c * 64 + 16 * (j ^ ((c >> 1) & 3)));
    auto lds_h8 = [&](int s, unsigned off) __attribute__((always_inline)) -> h8 {
        const uint4 x = *reinterpret_cast<const uint4 *>(smem + s * SLABB + off);
        return *reinterpret_cast<const h8 *>(&x);
    };
    /* BFK: the V^T fragment of dim tile dt (lane (c, j): dim 16 dt + c, keys
     * 8 j .. 8 j + 7) as two transpose reads of the V rows. Each reads four
     * keys: within a group of 16 lanes, lane q points at 4 dims of one key
     * row (key 8 j + 4 h + q / 4, dims 16 dt + 4 (q % 4) ..) and lane c
     * receives dim 16 dt + c of the four keys its group's lanes 4 k + c / 4
     * point at. The rows of one read (keys 8 j + 4 h + 0..3, over j) take
     * distinct chunk pairs per pair of groups through fv. */
    unsigned vto[BFK ? DT : 1];
    if constexpr (BFK) {
        const int fv = (c >> 2) | ((j & 1) << 2);
        const int kr = 8 * j + (c >> 2);
#pragma unroll
        for (int dt = 0; dt < DT; dt++)
            vto[dt] = (unsigned)(K_BYTES + kr * KROW + ((((2 * dt) ^ (2 * fv)) | ((c >> 1) & 1)) << 4) + 8 * (c & 1));
    }
    auto lds_vt = [&](int s, int dt) __attribute__((always_inline)) -> h8 {
        typedef short v4s __attribute__((ext_vector_type(4)));
        typedef __attribute__((address_space(3))) v4s lds_v4s;
        const unsigned char *a = smem + s * SLABB + vto[dt];
        const v4s lo4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s *)(a));
        const v4s hi4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s *)(a + 4 * KROW));
        const uint2 x = __builtin_bit_cast(uint2, lo4), y = __builtin_bit_cast(uint2, hi4);
        const uint4 w = make_uint4(x.x, x.y, y.x, y.y);
        return *reinterpret_cast<const h8 *>(&w);
    };
    h8 ones;
#pragma unroll
    for (int i = 0; i < 8; i++) ones[i] = (_Float16)1.0f;
    /* row sums: on the matrix cores against a fragment of ones (lsum), or
     * with PREC (P = Phi + Plo) in fp32 per lane (lp), reduced at the end */
    f4 o[DT], lsum = {0.f, 0.f, 0.f, 0.f};
    float lp = 0.0f;
#pragma unroll
    for (int dt = 0; dt < DT; dt++) o[dt] = f4{0.f, 0.f, 0.f, 0.f};
    float m = -INFINITY;
    /* S of slab s + 1 is formed before the softmax of slab s: the matrix
     * cores work on it while the vector ALU does the softmax */
    /* K fragments: [0..1] hi, [2..3] lo (KLO) */
    constexpr int KF = KLO ? 4 : 2;
    auto read_k = [&](int s, h8 (&kf)[KF][KS]) __attribute__((always_inline)) {
#pragma unroll
        for (int tt = 0; tt < KF; tt++)
#pragma unroll
            for (int ks = 0; ks < KS; ks++) kf[tt][ks] = lds_h8(s, kfo[ks] + (tt & 1) * 4 * KROW + (tt >> 1) * K_BYTES);
    };
    auto qk = [&](const h8 (&kf)[KF][KS], f4 (&sc)[2]) __attribute__((always_inline)) {
#pragma unroll
        for (int tt = 0; tt < 2; tt++) {
            f4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < KS; ks++) {
                if constexpr (BFK) {
                    const b8 kb = *reinterpret_cast<const b8 *>(&kf[tt][ks]); /* the bf16 bits as staged */
                    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kb, qbh[ks], acc, 0, 0, 0);
                    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kb, qbl[ks], acc, 0, 0, 0);
                    continue;
                }
                acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf[tt][ks], qf[ks], acc, 0, 0, 0);
                if constexpr (PREC) acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf[tt][ks], qfl[ks], acc, 0, 0, 0);
                if constexpr (KLO) acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf[2 + tt][ks], qf[ks], acc, 0, 0, 0);
            }
            sc[tt] = acc;
        }
    };
    h8 kf[KF][KS];
    f4 scur[2], snext[2];
    if (s_lo < s_hi) {
        read_k(s_lo, kf);
        qk(kf, scur);
    }
    for (int s = s_lo; s < s_hi; s++) {
        h8 vf[DT];
#pragma unroll
        for (int dt = 0; dt < DT; dt++) vf[dt] = BFK ? lds_vt(s, dt) : lds_h8(s, vfo + dt * 1024);
        const bool more = s + 1 < s_hi;
        if (more) {
            read_k(s + 1, kf);
            qk(kf, snext);
        }
        float sv[8];
#pragma unroll
        for (int tt = 0; tt < 2; tt++)
#pragma unroll
            for (int i = 0; i < 4; i++) sv[4 * tt + i] = scur[tt][i];
        if (s * SMOL_SLAB + SMOL_SLAB > len) {
            /* the last slab: keys past the window */
#pragma unroll
            for (int e = 0; e < 8; e++)
                if (s * SMOL_SLAB + 8 * j + e >= len) sv[e] = -INFINITY;
        }
        float mx = sv[0];
#pragma unroll
        for (int e = 1; e < 8; e++) mx = fmaxf(mx, sv[e]);
        mx = row_max4(mx);
        const float m_new = fmaxf(m, mx); /* finite: every slab holds a key of the window */
        /* (a group without slabs keeps m = -inf, lsum = 0, o = 0) */
        const float alpha = __builtin_amdgcn_exp2f(m - m_new);
        m = m_new;
        h8 pf, pfl;
        float ps = 0.0f;
        float pe8[8];
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const float pe = __builtin_amdgcn_exp2f(sv[e] - m_new);
            pe8[e] = pe;
            if constexpr (!BFK && !PREC) pf[e] = (_Float16)pe;
            if constexpr (PREC) ps += pe;
        }
        if constexpr (!BFK && PREC) {
#pragma unroll
            for (int e = 0; e < 8; e += 2) {
                uint32_t hi, lo;
                split_h2(pe8[e], pe8[e + 1], hi, lo);
                reinterpret_cast<uint32_t *>(&pf)[e >> 1] = hi;
                reinterpret_cast<uint32_t *>(&pfl)[e >> 1] = lo;
            }
        }
        if constexpr (BFK) {
            /* P as bf16 hi + lo against the exact bf16 V^T */
            b8 pbh, pbl;
            split8(pe8, pbh, pbl);
#pragma unroll
            for (int dt = 0; dt < DT; dt++) {
                const b8 vb = *reinterpret_cast<const b8 *>(&vf[dt]);
                f4 acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vb, pbh, o[dt] * alpha, 0, 0, 0);
                o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vb, pbl, acc, 0, 0, 0);
            }
        } else {
#pragma unroll
            for (int dt = 0; dt < DT; dt++) {
                f4 acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf[dt], pf, o[dt] * alpha, 0, 0, 0);
                if constexpr (PREC) acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf[dt], pfl, acc, 0, 0, 0);
                o[dt] = acc;
            }
        }
        if constexpr (PREC) lp = lp * alpha + ps;
        else lsum = __builtin_amdgcn_mfma_f32_16x16x32_f16(ones, pf, lsum * alpha, 0, 0, 0);
        if (more) {
            scur[0] = snext[0];
            scur[1] = snext[1];
        }
    }

    /* ---- two groups: group 1 hands (O, m, l) to group 0 through LDS, lane
     * by lane (wave wr of either group holds the same rows in the same
     * lanes) ---- */
    float l = PREC ? row_sum4(lp) : lsum[0];
    if (split) {
        float *xo = reinterpret_cast<float *>(smem) + (wr * 64 + lane) * (4 * DT + 4);
        static_assert(4 * 64 * (4 * DT + 4) * 4 <= NS * SLABB, "merge scratch");
        __syncthreads(); /* every slab read is done */
        if (grp == 1) {
#pragma unroll
            for (int dt = 0; dt < DT; dt++) *reinterpret_cast<f4 *>(xo + 4 * dt) = o[dt];
            xo[4 * DT] = m;
            xo[4 * DT + 1] = l;
        }
        __syncthreads();
        if (grp == 1) return;
        const float m1 = xo[4 * DT], l1 = xo[4 * DT + 1];
        const float M = fmaxf(m, m1); /* finite: group 0 has a slab with a key of the window */
        const float w0 = __builtin_amdgcn_exp2f(m - M), w1 = __builtin_amdgcn_exp2f(m1 - M);
#pragma unroll
        for (int dt = 0; dt < DT; dt++) o[dt] = o[dt] * w0 + *reinterpret_cast<const f4 *>(xo + 4 * dt) * w1;
        l = l * w0 + l1 * w1;
    }

    /* ---- out rows of the window (rows past it are not written) ---- */
    if (!q_ok) return;
    const float inv = l > 0.0f ? 1.0f / l : 0.0f;
    float *orow = p.out + (long long)(w0 + rq) * p.row_stride + hoff;
#pragma unroll
    for (int dt = 0; dt < DT; dt++) {
        const int d = 16 * dt + 4 * j;
        if (HD % 16 != 0 && d >= HD) continue;
        *reinterpret_cast<f4 *>(orow + d) = o[dt] * inv;
    }
}

namespace {

template <int HD, bool BF, int NS, bool PREC>
int launch_win_v(const WinParams *wp, int n_tiles, hipStream_t st, hipEvent_t e0, hipEvent_t e1) {
    (void)n_tiles;
    const long long units = (long long)wp->n_windows * wp->H;
    const dim3 grid((unsigned)((units + wp->n_xcc - 1) / wp->n_xcc * wp->n_xcc * wp->tpu));
    if (e0)
        hipExtLaunchKernelGGL((k_attn_win<HD, BF, NS, PREC>), grid, dim3(WIN_TPB), 0, st, e0, e1, 0, *wp);
    else
        hipLaunchKernelGGL((k_attn_win<HD, BF, NS, PREC>), grid, dim3(WIN_TPB), 0, st, *wp);
    return hipGetLastError() == hipSuccess ? 0 : -3;
}

/* builds by window capacity: 4 or 8 slabs (the short windows of the audio
 * and vision encoders), or as many as the LDS holds */
template <int HD, bool BF, bool PREC>
int launch_win_bf(const WinParams *wp, int n_tiles, int max_len, hipStream_t st, hipEvent_t e0, hipEvent_t e1) {
    constexpr int NS_MAX = WinGeom<HD, PREC && !BF, PREC && BF>::NS_MAX;
    const int ns = (max_len + SMOL_SLAB - 1) / SMOL_SLAB;
    static_assert(NS_MAX >= 4, "the smallest build");
    if (ns <= 4) return launch_win_v<HD, BF, 4, PREC>(wp, n_tiles, st, e0, e1);
    if constexpr (NS_MAX > 8) {
        if (ns <= 8) return launch_win_v<HD, BF, 8, PREC>(wp, n_tiles, st, e0, e1);
    }
    if (ns <= NS_MAX) return launch_win_v<HD, BF, NS_MAX, PREC>(wp, n_tiles, st, e0, e1);
    return -1;
}

template <int HD>
int launch_win_hd(const WinParams *wp, int n_tiles, int max_len, hipStream_t st, hipEvent_t e0, hipEvent_t e1) {
    const bool bf = wp->in_dtype == SMOL_IN_BF16;
    if (wp->precise)
        return bf ? launch_win_bf<HD, true, true>(wp, n_tiles, max_len, st, e0, e1)
                  : launch_win_bf<HD, false, true>(wp, n_tiles, max_len, st, e0, e1);
    return bf ? launch_win_bf<HD, true, false>(wp, n_tiles, max_len, st, e0, e1)
              : launch_win_bf<HD, false, false>(wp, n_tiles, max_len, st, e0, e1);
}

template <int HD>
int win_max_keys(int in_dtype, int precise) {
    const bool bf = in_dtype == SMOL_IN_BF16;
    return (precise ? (bf ? WinGeom<HD, false, true>::NS_MAX : WinGeom<HD, true, false>::NS_MAX)
                    : WinGeom<HD, false, false>::NS_MAX) * SMOL_SLAB;
}

} // namespace

/* The longest window k_attn_win holds at head_dim hd for inputs of type
 * in_dtype, with precise QK^T or not (0: not supported) */
extern "C" int smol_win_max_keys(int hd, int in_dtype, int precise) {
    switch (hd) {
    case 64: return win_max_keys<64>(in_dtype, precise);
    case 72: return win_max_keys<72>(in_dtype, precise);
    case 80: return win_max_keys<80>(in_dtype, precise);
    case 96: return win_max_keys<96>(in_dtype, precise);
    case 128: return win_max_keys<128>(in_dtype, precise);
    default: return 0;
    }
}

/* n_tiles: 64-row tiles over all windows; max_len: the longest window;
 * e0 / e1 (may be null): events recorded around the kernel alone */
extern "C" int smol_launch_win(const WinParams *wp, int hd, int n_tiles, int max_len, hipStream_t st, hipEvent_t e0,
                               hipEvent_t e1) {
    if (n_tiles <= 0) return 0;
    switch (hd) {
    case 64: return launch_win_hd<64>(wp, n_tiles, max_len, st, e0, e1);
    case 72: return launch_win_hd<72>(wp, n_tiles, max_len, st, e0, e1);
    case 80: return launch_win_hd<80>(wp, n_tiles, max_len, st, e0, e1);
    case 96: return launch_win_hd<96>(wp, n_tiles, max_len, st, e0, e1);
    case 128: return launch_win_hd<128>(wp, n_tiles, max_len, st, e0, e1);
    default: return -1;
    }
}
