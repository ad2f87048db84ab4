/*
 * gemm.hip - k_gemm: the decoders' bf16-weight projections for more than a
 * few rows on bf16 MFMA, with the operations around them fused:
 *
 *     y[m][n] = res[m][n'] + act( r_m * sum_k (x[m][k] g[k]) W[n][k] + bias[n] )
 *
 * (smol_linear_bf16 / smol_linear_nobias_bf16 / smol_matmul_t_bf16,
 * common/kernels/matmul.c:336-358, 419-429, for seq_len > 1; bf16_linear_nobias,
 * common/decoder/qkn_bf16_decoder.c:99-117; the input RMSNorm of
 * common/kernels/rmsnorm.c:17-75 with r_m = 1 / sqrtf(sum_k x[m][k]^2 / K + eps)
 * and the gated activations of common/kernels/activation.c:55-125 on the
 * interleaved gate / up rows of the fused weight).
 *
 * Operands. W is bf16 [N][K]; x is fp32 or bf16 [M][K]. An fp32 x (times the
 * norm weight g when there is one) is split as it is staged into x_hi =
 * bf16(x) and x_lo = bf16(x - x_hi), and every W fragment feeds two MFMAs
 * (W.x_hi + W.x_lo, fp32 accumulation), which carries x to about 2^-17
 * relative; a bf16 x is used as it is. The row scale r_m is applied to the
 * accumulator: sum_k ((x g) r) W and r sum_k (x g) W differ only by fp32
 * rounding. The sum of squares comes from the same x loads.
 *
 * Tiling. One workgroup computes a BN x BM tile (outputs x rows) with
 * v_mfma_f32_16x16x32_bf16: A = W rows (outputs), B = x rows, so a lane's
 * four accumulator values are four consecutive outputs of one row (one
 * 16-byte store, and both members of a gate / up pair). Three tile sizes
 * (192 x 192 and 128 x 128 with eight waves, 64 x 64 with four and two
 * workgroups per compute unit: two waves per SIMD in each); the host picks
 * one from the launch's rounds over the device. With a bf16 x the waves
 * form a 2 x (NW / 2) grid; with an fp32 x each wave of the two smaller
 * tiles owns rows of its own (1 x NW) and so splits each element once per
 * workgroup. K advances 64 at a time through NSTG LDS
 * stages (three where they fit in 150 KB, else two): W, x and the norm
 * weight all by direct-to-LDS transfers (buffer_load ... lds), the next
 * stages in flight while one is multiplied. LDS rows are 128 or 256 bytes
 * with their 16-byte chunks XOR-swizzled by the row's low 3 bits, so the
 * fragment reads of eight consecutive lanes hit distinct banks. The tile
 * grid is cut into eight regions, one per XCD (workgroup b runs on XCD
 * b % 8), shaped to keep the fewest x and W bytes per XCD L2.
 */
#include "attn_device.h"
#include "smol_linear.h"

#define GEMM_BK 64
#define GEMM_XCD 8


namespace {

/* NSTG LDS stages of BK = 64: W [BN][64] bf16 (128-byte rows), then x
 * [BM][64] as loaded (bf16: 128-byte rows; fp32: 256-byte rows), then the
 * norm weight's 64 values */
template <int BM, int BN, bool XBF, int WN, int WM>
struct GemmGeom {
    static constexpr int NW = WN * WM;
    static constexpr int XROW = XBF ? 128 : 256;
    static constexpr int W_BYTES = BN * 128;
    static constexpr int X_BYTES = BM * XROW;
    static constexpr int G_BYTES = 1024; /* norm weight of the stage's 64 columns (the first 256 bytes) */
    static constexpr int STAGE = W_BYTES + X_BYTES + G_BYTES;
    static constexpr int NSTG = 3 * STAGE <= 150 * 1024 ? 3 : 2;
    static constexpr int TN = BN / WN, TM = BM / WM; /* wave tile */
    static constexpr int NT = TN / 16, MT = TM / 16;
    static constexpr int WDMA = W_BYTES / 1024 / NW; /* 1 KB transfers per wave per stage */
    static constexpr int XDMA = X_BYTES / 1024 / NW;
};

/* byte offset of 16-byte chunk q of row r in rows of `rb` bytes: the chunk
 * index XOR the row's low 3 bits, so eight consecutive rows read at one
 * chunk index hit distinct banks */
__device__ __forceinline__ unsigned swz(int row, int q, int rb) {
    return (unsigned)(row * rb + ((q ^ (row & 7)) << 4));
}

__device__ __forceinline__ float act_fn(float g, int act) {
    if (act == SMOL_LINEAR_ACT_SWIGLU) return g / (1.0f + expf(-g));
    const float x3 = g * g * g;
    const float inner = 0.7978845608028654f * (g + 0.044715f * x3);
    return 0.5f * g * (1.0f + tanhf(inner));
}

/* x_hi = bf16_rne(x), x_lo = bf16_rne(xc - bf16_rne(xc)) of 8 floats, xc =
 * x clamped to bf16's largest finite magnitude (about 3.39e38): the same
 * x_lo for every |x| up to that bound, 0 for an infinite x (which goes to
 * x_hi whole and so reaches y as it would in fp32), never an infinite or
 * NaN lo part beside a finite one. Per pair: one packed conversion for the
 * hi pair, two clamps, two conversions over a zero low half (which are
 * bf16(xc) as floats), two differences, one packed conversion for the lo
 * pair. */
typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
typedef float fl2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ void split_frag(const float *v, b8 &hi, b8 &lo) {
    constexpr float BF16_MAX = 3.3895313892515355e38f;
    uint32_t hw[4], lw[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float x0 = v[2 * i], x1 = v[2 * i + 1];
        hw[i] = __builtin_bit_cast(uint32_t, __builtin_convertvector((fl2){x0, x1}, bf2));
        const float c0 = __builtin_amdgcn_fmed3f(x0, -BF16_MAX, BF16_MAX);
        const float c1 = __builtin_amdgcn_fmed3f(x1, -BF16_MAX, BF16_MAX);
        const float h0 = __builtin_bit_cast(float, __builtin_convertvector((fl2){0.0f, c0}, bf2));
        const float h1 = __builtin_bit_cast(float, __builtin_convertvector((fl2){0.0f, c1}, bf2));
        lw[i] = __builtin_bit_cast(uint32_t, __builtin_convertvector((fl2){c0 - h0, c1 - h1}, bf2));
    }
    hi = as_b8(make_uint4(hw[0], hw[1], hw[2], hw[3]));
    lo = as_b8(make_uint4(lw[0], lw[1], lw[2], lw[3]));
}

} // namespace

template <int BM, int BN, int WN, int WM, bool XBF, bool YBF, bool NORM>
__global__ __launch_bounds__(64 * WN * WM) __attribute__((amdgpu_waves_per_eu(WN * WM * (BM >= 128 ? 1 : 2) / 4,
                                                                             WN * WM * (BM >= 128 ? 1 : 2) / 4)))
void k_gemm(const GemmParams p) {
    using Gm = GemmGeom<BM, BN, XBF, WN, WM>;
    constexpr int NW = Gm::NW;
    constexpr int STAGE = Gm::STAGE, W_BYTES = Gm::W_BYTES, XROW = Gm::XROW, NSTG = Gm::NSTG;
    constexpr int NT = Gm::NT, MT = Gm::MT, WDMA = Gm::WDMA, XDMA = Gm::XDMA;
    constexpr int XCH = XROW / 16;                   /* 16-byte chunks of an x row */
    static_assert(NSTG * STAGE <= 160 * 1024, "LDS");
    static_assert(WDMA * 1024 * NW == W_BYTES && XDMA * 1024 * NW == Gm::X_BYTES, "staging shape");
    __shared__ __attribute__((aligned(1024))) unsigned char smem[NSTG * STAGE];
    __shared__ float s_rinv[NORM ? BM : 1];

    /* the tile: workgroup b runs on XCD b % 8 */
    const int b = blockIdx.x, xcd = b % GEMM_XCD, idx = b / GEMM_XCD;
    int tm, tn;
    if (p.rm > 0) {
        /* XCD x: region (x / rn, x % rn) of the tile grid, so the rows of x
         * and of W that its tiles share stay in its own L2 */
        const int tiles_n = p.tiles / p.tiles_m;
        const int ri = xcd / p.rn, rj = xcd % p.rn;
        const int m_lo = ri * p.tiles_m / p.rm, m_hi = (ri + 1) * p.tiles_m / p.rm;
        const int n_lo = rj * tiles_n / p.rn, n_hi = (rj + 1) * tiles_n / p.rn;
        if (idx >= (m_hi - m_lo) * (n_hi - n_lo)) return;
        tm = m_lo + idx % (m_hi - m_lo);
        tn = n_lo + idx / (m_hi - m_lo);
    } else {
        const int t = xcd * p.per_xcd + idx;
        if (idx >= p.per_xcd || t >= p.tiles) return;
        tm = t % p.tiles_m;
        tn = t / p.tiles_m;
    }
    const int m0 = tm * BM;
    const int K = p.K;
    /* the tile's output: its segment's weight rows, y and width (a tile
     * never straddles two segments) */
    int n0 = tn * BN, NN = p.N;
    const uint16_t *Wt = p.w;
    void *Yt = p.y;
    if (p.nseg > 0) {
        const int sg = (n0 >= p.seg_c[1] ? 1 : 0) + (p.nseg > 2 && n0 >= p.seg_c[2] ? 1 : 0);
        const int c0 = sg == 0 ? 0 : sg == 1 ? p.seg_c[1] : p.seg_c[2];
        NN = (sg == 0 ? p.seg_c[1] : sg == 1 ? p.seg_c[2] : p.seg_c[3]) - c0;
        Wt = sg == 0 ? p.seg_w[0] : sg == 1 ? p.seg_w[1] : p.seg_w[2];
        Yt = sg == 0 ? p.seg_y[0] : sg == 1 ? p.seg_y[1] : p.seg_y[2];
        n0 -= c0;
    }

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wn = wave % WN, wm = wave / WN;
    const int c = lane & 15, j = lane >> 4;
    const unsigned lds0 = (unsigned)(size_t)smem;

    /* Transfer e of a wave fills 1 KB of the stage: lane L lands at the
     * stage's 16-byte position 1024 (wave + 4 e) / 16 + L, i.e. at chunk
     * position (pos % chunks-per-row) of row pos / chunks-per-row, and loads
     * the global chunk that the swizzle puts there. Rows past the operand
     * and chunks past K read zero. */
    const rsrc_t rw = make_rsrc(Wt + (long long)n0 * K, (long long)min(BN, NN - n0) * K * 2);
    const long long xes = XBF ? 2 : 4;
    const rsrc_t rx = make_rsrc(static_cast<const char *>(p.x) + (long long)m0 * K * xes,
                                (long long)min(BM, p.M - m0) * K * xes);
    /* the norm weight: staged with each step's transfers (wave 0's one
     * extra transfer; a vector load of the compiler's would make it wait for
     * every transfer in flight) */
    const rsrc_t rg = make_rsrc(NORM ? (const void *)p.g : (const void *)Wt, NORM ? (long long)K * 4 : 0);
    const int n_steps = (K + GEMM_BK - 1) / GEMM_BK;
    unsigned w_off[WDMA], x_off[XDMA];
    int w_k[WDMA], x_k[XDMA]; /* first k of the lane's chunk, within the stage */
#pragma unroll
    for (int e = 0; e < WDMA; e++) {
        const int pos = 64 * (wave + NW * e) + lane;
        const int row = pos / 8, q = (pos % 8) ^ (row & 7);
        w_k[e] = 8 * q;
        w_off[e] = (unsigned)((row * K + 8 * q) * 2);
    }
#pragma unroll
    for (int e = 0; e < XDMA; e++) {
        const int pos = 64 * (wave + NW * e) + lane;
        const int row = pos / XCH, q = (pos % XCH) ^ (row & 7);
        x_k[e] = XBF ? 8 * q : 4 * q;
        x_off[e] = (unsigned)((row * K + x_k[e]) * xes);
    }
    auto issue = [&](int s, int stage) __attribute__((always_inline)) {
        const int k0 = s * GEMM_BK;
        const unsigned st = lds0 + (unsigned)(stage * STAGE);
#pragma unroll
        for (int e = 0; e < WDMA; e++)
            dma_1k(rw, k0 + w_k[e] < K ? w_off[e] : OOB_OFF, (unsigned)(k0 * 2),
                   __builtin_amdgcn_readfirstlane(st + (wave + NW * e) * 1024));
#pragma unroll
        for (int e = 0; e < XDMA; e++)
            dma_1k(rx, k0 + x_k[e] < K ? x_off[e] : OOB_OFF, (unsigned)(k0 * xes),
                   __builtin_amdgcn_readfirstlane(st + W_BYTES + (wave + NW * e) * 1024));
        if (NORM && wave == 0)
            dma_1k(rg, lane < 16 && k0 + 4 * lane < K ? (unsigned)(lane * 16) : OOB_OFF, (unsigned)(k0 * 4),
                   __builtin_amdgcn_readfirstlane(st + W_BYTES + Gm::X_BYTES));
    };

    float ss[MT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++) ss[mt] = 0.0f;

    f4 acc[NT][MT];
#pragma unroll
    for (int t = 0; t < NT; t++)
#pragma unroll
        for (int mt = 0; mt < MT; mt++) acc[t][mt] = f4{0.f, 0.f, 0.f, 0.f};

    /* NSTG - 1 stages in flight ahead of the one being multiplied */
#pragma unroll
    for (int s = 0; s < NSTG - 1; s++)
        if (s < n_steps) issue(s, s);
    /* unrolled by the ring's length, so every stage offset is a constant */
    for (int s0 = 0; s0 < n_steps; s0 += NSTG)
#pragma unroll
    for (int u = 0; u < NSTG; u++) {
        const int s = s0 + u;
        if (s >= n_steps) break;
        /* stage s complete and visible: all of this thread's transfers
         * drained (vmcnt(0), explicit: the compiler's own waits do not count
         * the inline-asm transfers; a count that leaves the younger stage in
         * flight measured no faster, and on pages touched for the first time
         * transfers need not land in issue order), then the barrier, which
         * also tells every wave that stage s - 1 is no longer read */
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (s + NSTG - 1 < n_steps) issue(s + NSTG - 1, (u + NSTG - 1) % NSTG);
        const unsigned char *st = smem + u * STAGE;
        float gw[2][8];
        if constexpr (NORM) {
            const unsigned char *gs = st + W_BYTES + Gm::X_BYTES;
#pragma unroll
            for (int ks = 0; ks < 2; ks++) {
                const f4 a = *reinterpret_cast<const f4 *>(gs + (32 * ks + 8 * j) * 4);
                const f4 bb = *reinterpret_cast<const f4 *>(gs + (32 * ks + 8 * j) * 4 + 16);
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    gw[ks][i] = a[i];
                    gw[ks][4 + i] = bb[i];
                }
            }
        }
        /* the two half-steps (k 0-31, 32-63) as read, prepare, multiply,
         * with the second half's fragment reads issued before the first
         * half's products, so the LDS reads and the split (vector ALU) of
         * one half overlap the matrix work of the other */
        struct Raw {
            uint4 a[NT];
            f4 x[MT][XBF ? 1 : 2];
        };
        struct Frag {
            b8 a[NT], h[MT], l[XBF ? 1 : MT];
        };
        auto read = [&](int ks, Raw &r) __attribute__((always_inline)) {
#pragma unroll
            for (int t = 0; t < NT; t++)
                r.a[t] = *reinterpret_cast<const uint4 *>(st + swz(wn * Gm::TN + 16 * t + c, 4 * ks + j, 128));
#pragma unroll
            for (int mt = 0; mt < MT; mt++) {
                const int row = wm * Gm::TM + 16 * mt + c;
                if constexpr (XBF) {
                    r.x[mt][0] = *reinterpret_cast<const f4 *>(st + W_BYTES + swz(row, 4 * ks + j, 128));
                } else {
                    r.x[mt][0] = *reinterpret_cast<const f4 *>(st + W_BYTES + swz(row, 8 * ks + 2 * j, 256));
                    r.x[mt][1] = *reinterpret_cast<const f4 *>(st + W_BYTES + swz(row, 8 * ks + 2 * j + 1, 256));
                }
            }
        };
        auto prepare = [&](int ks, const Raw &r, Frag &f) __attribute__((always_inline)) {
#pragma unroll
            for (int t = 0; t < NT; t++) f.a[t] = as_b8(r.a[t]);
#pragma unroll
            for (int mt = 0; mt < MT; mt++) {
                if constexpr (XBF) {
                    const f4 v = r.x[mt][0];
                    f.h[mt] = as_b8(make_uint4(__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]),
                                               __float_as_uint(v[3])));
                } else {
                    const f4 v0 = r.x[mt][0], v1 = r.x[mt][1];
                    float v[8] = {v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
                    if constexpr (NORM) {
                        if (wn == 0) {
#pragma unroll
                            for (int i = 0; i < 8; i++) ss[mt] = fmaf(v[i], v[i], ss[mt]);
                        }
#pragma unroll
                        for (int i = 0; i < 8; i++) v[i] *= gw[ks][i];
                    }
                    split_frag(v, f.h[mt], f.l[mt]);
                }
            }
        };
        /* the hi products, then the lo ones: no MFMA waits for the one just
         * issued */
        auto multiply = [&](const Frag &f) __attribute__((always_inline)) {
#pragma unroll
            for (int t = 0; t < NT; t++)
#pragma unroll
                for (int mt = 0; mt < MT; mt++)
                    acc[t][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(f.a[t], f.h[mt], acc[t][mt], 0, 0, 0);
            if constexpr (!XBF) {
#pragma unroll
                for (int t = 0; t < NT; t++)
#pragma unroll
                    for (int mt = 0; mt < MT; mt++)
                        acc[t][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(f.a[t], f.l[mt], acc[t][mt], 0, 0, 0);
            }
        };
        {
            Raw r0, r1;
            Frag f0, f1;
            read(0, r0);
            prepare(0, r0, f0);
            read(1, r1);
            __builtin_amdgcn_sched_barrier(0);
            multiply(f0);
            prepare(1, r1, f1);
            multiply(f1);
        }
    }

    /* the rows' scale: in the waves with wn = 0, lanes c, c + 16, c + 32,
     * c + 48 hold row c's partial sums of squares */
    if constexpr (NORM) {
        if (wn == 0) {
#pragma unroll
            for (int mt = 0; mt < MT; mt++) {
                const float t = row_sum4(ss[mt]);
                if (j == 0) s_rinv[wm * Gm::TM + 16 * mt + c] = 1.0f / sqrtf(t / (float)K + p.eps);
            }
        }
        __syncthreads();
    }

    /* epilogue: lane (c, j) holds outputs n = 4 j + e of row m = c of each
     * 16 x 16 product tile */
    const bool has_act = p.act != SMOL_LINEAR_ACT_NONE;
    const int ycols = has_act ? NN / 2 : NN;
#pragma unroll
    for (int mt = 0; mt < MT; mt++) {
        const int ml = wm * Gm::TM + 16 * mt + c;
        const int m = m0 + ml;
        if (m >= p.M) continue;
        const float r = NORM ? s_rinv[ml] : 1.0f;
#pragma unroll
        for (int t = 0; t < NT; t++) {
            const int n = n0 + wn * Gm::TN + 16 * t + 4 * j;
            if (n >= NN) continue;
            float v[4] = {acc[t][mt][0], acc[t][mt][1], acc[t][mt][2], acc[t][mt][3]};
#pragma unroll
            for (int e = 0; e < 4; e++) {
                if (NORM) v[e] *= r;
                if (p.bias) v[e] += n + e < NN ? p.bias[n + e] : 0.0f;
            }
            if (has_act) {
                const int col = n / 2;
                float o[2] = {act_fn(v[0], p.act) * v[1], act_fn(v[2], p.act) * v[3]};
                const long long yi = (long long)m * ycols + col;
                const int nv = min(2, ycols - col);
                if (p.res) {
#pragma unroll
                    for (int e = 0; e < 2; e++)
                        if (e < nv) o[e] += p.res[yi + e];
                }
                if constexpr (YBF) {
                    uint16_t *y = static_cast<uint16_t *>(Yt) + yi;
#pragma unroll
                    for (int e = 0; e < 2; e++)
                        if (e < nv) y[e] = (uint16_t)(__float_as_uint(o[e]) >> 16);
                } else {
                    float *y = static_cast<float *>(Yt) + yi;
                    if (nv == 2 && ((yi & 1) == 0)) *reinterpret_cast<float2 *>(y) = make_float2(o[0], o[1]);
                    else
                        for (int e = 0; e < nv; e++) y[e] = o[e];
                }
            } else {
                const long long yi = (long long)m * ycols + n;
                const int nv = min(4, NN - n);
                if (p.res) {
#pragma unroll
                    for (int e = 0; e < 4; e++)
                        if (e < nv) v[e] += p.res[yi + e];
                }
                if constexpr (YBF) {
                    uint16_t *y = static_cast<uint16_t *>(Yt) + yi;
#pragma unroll
                    for (int e = 0; e < 4; e++)
                        if (e < nv) y[e] = (uint16_t)(__float_as_uint(v[e]) >> 16);
                } else {
                    float *y = static_cast<float *>(Yt) + yi;
                    if (nv == 4 && ((yi & 3) == 0)) *reinterpret_cast<float4 *>(y) = make_float4(v[0], v[1], v[2], v[3]);
                    else
                        for (int e = 0; e < nv; e++) y[e] = v[e];
                }
            }
        }
    }
}

/* ------------------------------------------------------------------ launch */

template <int BM, int BN, int WN, int WM, bool XBF, bool YBF>
static int launch_gemm_t(const GemmParams &p, bool norm, hipStream_t st, hipEvent_t e0, hipEvent_t e1) {
    const dim3 grid((unsigned)(GEMM_XCD * p.per_xcd)), block(64 * WN * WM);
    if constexpr (!XBF) {
        if (norm) {
            hipExtLaunchKernelGGL((k_gemm<BM, BN, WN, WM, false, YBF, true>), grid, block, 0, st, e0, e1, 0, p);
            return hipGetLastError() == hipSuccess ? 0 : -3;
        }
    }
    hipExtLaunchKernelGGL((k_gemm<BM, BN, WN, WM, XBF, YBF, false>), grid, block, 0, st, e0, e1, 0, p);
    return hipGetLastError() == hipSuccess ? 0 : -3;
}

/* wave layouts, (WNF x WMF) for an fp32 x and (WNB x WMB) for a bf16 x:
 * with an fp32 x each wave should own rows of its own (WN = 1), so each
 * element is split once per workgroup (two waves across the outputs both
 * split the same fragment: the split, not the matrix cores, bounds the fp32
 * steps); the 192-row tile keeps two waves across the outputs, since its
 * eight waves' rows would not be whole 16-row tiles otherwise, and eight
 * waves (two per SIMD, one hiding the other's LDS and split latency) beat
 * four with rows of their own */
template <int BM, int BN, int WNF, int WMF, int WNB, int WMB>
static int launch_gemm_b(const GemmParams &p, bool xbf, bool ybf, bool norm, hipStream_t st, hipEvent_t e0,
                         hipEvent_t e1) {
    if (xbf) return ybf ? launch_gemm_t<BM, BN, WNB, WMB, true, true>(p, false, st, e0, e1)
                        : launch_gemm_t<BM, BN, WNB, WMB, true, false>(p, false, st, e0, e1);
    return ybf ? launch_gemm_t<BM, BN, WNF, WMF, false, true>(p, norm, st, e0, e1)
               : launch_gemm_t<BM, BN, WNF, WMF, false, false>(p, norm, st, e0, e1);
}

/* tile sizes the host may choose (rows of x = BM, outputs = BN) */
extern "C" int smol_gemm_tile(int cfg, int *bm, int *bn) {
    static const int t[3][2] = {{192, 192}, {128, 128}, {64, 64}};
    if (cfg < 0 || cfg > 2) return -1;
    *bm = t[cfg][0];
    *bn = t[cfg][1];
    return 0;
}

/* p's tile fields are filled here from the configuration; K % 8 == 0 and a
 * 16-byte aligned W and x are the caller's to check */
extern "C" int smol_launch_gemm(GemmParams *p, int cfg, bool xbf, bool ybf, hipStream_t st, hipEvent_t e0,
                                hipEvent_t e1) {
    int bm, bn;
    if (smol_gemm_tile(cfg, &bm, &bn)) return -1;
    if (xbf && p->g) return -1;
    p->tiles_m = (p->M + bm - 1) / bm;
    const int tiles_n = (p->N + bn - 1) / bn;
    p->tiles = p->tiles_m * tiles_n;
    if (p->tiles <= 0) return 0;
    if (p->rm > 0) {
        /* the region split with the fewest operand bytes per XCD (x rows
         * of its row blocks + W rows of its column blocks); a grid smaller
         * than the split in either direction keeps the contiguous deal */
        static const int splits[4][2] = {{1, 8}, {2, 4}, {4, 2}, {8, 1}};
        const double xrow = (double)p->K * (xbf ? 2 : 4), wrow = (double)p->K * 2;
        double best = 1e300;
        p->rm = 0;
        for (const auto &sp : splits) {
            if (sp[0] > p->tiles_m || sp[1] > tiles_n) continue;
            const double bytes = (double)((p->tiles_m + sp[0] - 1) / sp[0]) * bm * xrow +
                                 (double)((tiles_n + sp[1] - 1) / sp[1]) * bn * wrow;
            if (bytes < best) {
                best = bytes;
                p->rm = sp[0];
                p->rn = sp[1];
            }
        }
    }
    if (p->rm > 0) {
        const int hm = (p->tiles_m + p->rm - 1) / p->rm, hn = (tiles_n + p->rn - 1) / p->rn;
        p->per_xcd = hm * hn;
    } else {
        p->per_xcd = (p->tiles + GEMM_XCD - 1) / GEMM_XCD;
    }
    const bool norm = p->g != nullptr;
    switch (cfg) {
    case 0: return launch_gemm_b<192, 192, 2, 4, 2, 4>(*p, xbf, ybf, norm, st, e0, e1);
    case 1: return launch_gemm_b<128, 128, 1, 8, 2, 4>(*p, xbf, ybf, norm, st, e0, e1);
    default: return launch_gemm_b<64, 64, 1, 4, 2, 2>(*p, xbf, ybf, norm, st, e0, e1);
    }
}
