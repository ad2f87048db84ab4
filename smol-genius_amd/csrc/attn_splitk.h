/*
 * attn_splitk.h - the split-K merge of k_attn_fa: merge_group (the last
 * workgroup of a group merges the partials).
 */
#ifndef SMOL_ATTN_SPLITK_H
#define SMOL_ATTN_SPLITK_H

#include "attn_device.h"

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

#endif
