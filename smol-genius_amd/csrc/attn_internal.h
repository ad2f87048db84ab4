/*
 * attn_internal.h - descriptors shared by the host dispatcher (attn_api.hip)
 * and the kernels (attn_kernels.hip). Not part of the public C ABI.
 *
 * Device data layout (one GPU):
 *   KV cache   K  : bf16 [layer][slot][kv_head][cap][head_dim]   (post-RoPE)
 *              V^T: bf16 [layer][slot][kv_head][cap/32][head_dim][32]
 *                   (transposed within 32-key slabs: the P.V product reads 8
 *                   consecutive keys of one column, and one slab of V is one
 *                   contiguous block, as one slab of K is)
 *   fresh K/V  fp16 copies of the keys a call appends (and of the cache rows
 *              that share their 32-key slab), same two layouts with `fcap`
 *              rows; attention over a call's own keys uses these, so a key
 *              rotated in fp32 is never read back through bf16 rounding.
 *              With precise QK^T the fresh K also has an fp16 lo part
 *              (K - fp16(K), same layout), so hi + lo holds the fp32 key to
 *              about 22 significant bits.
 *   Q scratch  [kv_head][row][hdp], row = q_index * G + head_in_group,
 *              rotated and pre-multiplied by scale * log2(e); hdp = head_dim
 *              rounded up to 32 and zero-filled; fp16 (with its lo part in
 *              a second array of the same layout for precise QK^T) or fp32.
 */
#ifndef SMOL_ATTN_INTERNAL_H
#define SMOL_ATTN_INTERNAL_H

#include <stdint.h>

#define SMOL_SLAB 32          /* keys per inner step of the attention kernels */
#define SK_MERGE_MAX 4096     /* max rows * n_split of one split-K merge group (the merge's LDS) */
#define SK_COUNTER_STRIDE 64  /* ints between two merge groups' counters: one 256-byte line each */
#define SMOL_ROWS_PER_TILE 16 /* query rows per MFMA tile (16x16x32 f16) */

enum { SMOL_IN_F32 = 0, SMOL_IN_BF16 = 1 };
enum { SMOL_ROPE_OFF = 0, SMOL_ROPE_NEOX_K = 1, SMOL_ROPE_INTERLEAVED_K = 2 };

/* One attention "batch": a set of query rows sharing one key range and one
 * K/V source (a sequence slot of the cache, or one bidirectional window). */
typedef struct {
    int n_rows;      /* query rows = n_q * G */
    int q_row0;      /* first Q-scratch row of this batch */
    int out_tok0;    /* first output token row */
    int q_pos0;      /* causal position of query 0 (query i sits at q_pos0 + i) */
    int key_lo;      /* visible keys are [key_lo, key_hi) (then causal / window) */
    int key_hi;
    int causal;      /* 1: key <= q_pos0 + i; 0: the whole [key_lo, key_hi) */
    int fresh_pos0;  /* keys >= fresh_pos0 come from the fresh fp16 buffers */
    int fresh_row0;  /* fresh row holding key fresh_pos0 */
    int slot;        /* cache slot, or -1 when the batch has no cache */
    int pad0, pad1;
} SkBatch;

/* One work item of the split-K kernel: a tile of rows of a batch against a
 * contiguous key range. Items of one merge group are contiguous. */
typedef struct {
    int batch;
    int row0;        /* first row (within the batch) of this item's row tiles */
    int key_begin;   /* slab-aligned */
    int key_end;
    int group;       /* merge group id (one output row tile) */
    int n_split;     /* items in the group */
    int split;       /* index of this item in its group */
    int fresh_off;   /* the batch's fresh_row0 - fresh_pos0: fresh row of key k is k + fresh_off */
} SkItem;

/* An item with its batch, loaded together (the kernels issue one round of
 * scalar loads for both instead of two dependent rounds) */
typedef struct {
    SkItem it;
    SkBatch b;
} SkItemB;

/* A work item of k_attn_fb with its batch's fields (one scalar load): a
 * 64-row tile (128 rows with one key group) of a batch against the keys
 * [key_begin, key_end), all in the fresh buffers. next: the next item of the
 * same workgroup, or -1. With one key group a tile's keys may be split over
 * several items (a merge group): the item writes its partial into slot
 * `part` and the last of the group to finish merges them. */
typedef struct {
    int key_begin, key_end, fresh_off, row0;
    int n_rows, q_row0, out_tok0, q_pos0;
    int key_lo, key_hi, causal, next;
    int group, n_split, split, part;
} FbItem;

/* Q-scratch format written by k_prep (fresh K / V^T are fp16 in both):
 *   SMOL_STAGE_F16    fp16 (the fp16-MFMA kernels k_attn_fb and k_attn_fa),
 *                     plus the fp16 lo part when PrepParams.qs_lo is set
 *   SMOL_STAGE_QF32   fp32 (k_dec splits it into bf16 hi + lo) */
enum { SMOL_STAGE_F16 = 0, SMOL_STAGE_QF32 = 1 };

typedef struct {
    const _Float16 *qs;        /* Q scratch */
    const _Float16 *qs_lo;     /* its lo part (precise QK^T; null: single-term fp16 QK^T) */
    long long qs_head_stride;  /* rows_total * hdp */
    const uint16_t *kc;        /* cache K at (layer, slot 0), or null */
    const uint16_t *vtc;       /* cache V^T at (layer, slot 0), or null */
    long long c_slot_stride;   /* elements per slot (n_kv * cap * hd) */
    int cap;                   /* cache rows per (slot, kv head) */
    const _Float16 *kf;        /* fresh K [kv][fcap][hd] */
    const _Float16 *kf_lo;     /* its lo part (precise QK^T) */
    const _Float16 *vtf;       /* fresh V^T [kv][hd][fcap] */
    const float *qs32;         /* fp32 Q scratch (SMOL_STAGE_QF32) */
    int fcap;
    float *out;                /* [token][Hq][hd] fp32 */
    int Hq, Hkv, G;
    int window;                /* > 0: sliding window (keys > pos - window) */
    float cap2;                /* > 0: softcap in log2 units (cap * log2 e) */
    const SkItemB *items;      /* k_attn_dec / k_attn_fa items with their batches */
    float *part_o;             /* [item][kv][rows][hd] unnormalised partial outputs */
    float *part_ml;            /* [item][kv][rows][2] (max, sum) */
    int *counters;             /* [group][kv] at a stride of SK_COUNTER_STRIDE; zero between calls */
    /* k_attn_fb: its items; workgroup w (per kv head) starts at item w and
     * follows the items' next links */
    const FbItem *fb_items;
    int n_wg;
    int *range_flag;           /* k_attn_fa: set to 1 when a cache value widened to fp16 overflows */
    /* k_attn_fb with Q from the inputs (q_in non-null; no Q scratch): each
     * item rotates and scales its Q rows itself, the arithmetic of k_prep's
     * Q blocks; Q-scratch row r of an item then names input token r / G,
     * head g * G + r % G */
    const void *q_in; int q_dtype; long long q_stride;
    const float *rope_cos; const float *rope_sin; int q_rope_kind;
    float qscale;
} SkParams;

/* Pre-pass: normalises (optional per-head RMSNorm), rotates and scales Q into
 * the Q scratch, appends the normalised and rotated K and V to the bf16 cache
 * and writes the fresh fp16 K/V slabs. */
typedef struct {
    int q_tok0, n_q;     /* Q input rows of this batch */
    int q_row0;          /* Q-scratch row offset (already multiplied by G) */
    int q_pos0;          /* RoPE table row of Q row 0 */
    int kv_in0, n_kv;    /* new K/V input rows */
    int kv_pos0;         /* position (cache row, RoPE row) of new K/V row 0 */
    int fresh_pos0;      /* slab-aligned first position of the fresh window */
    int n_fresh;         /* multiple of SMOL_SLAB */
    int fresh_row0;      /* fresh row of fresh_pos0 */
    int slot;            /* cache slot or -1 */
    int pad;
} PrepBatch;

/* Block work of the pre-pass: a 32-position fresh slab of one batch, or a
 * run of Q tokens of one batch. */
typedef struct {
    int batch;
    int kind;            /* 0: fresh slab, 1: Q tokens */
    int first;           /* slab index within the fresh window / first Q token */
    int count;           /* Q tokens in this block; fresh slab: 0 its K and V, 1 its K, 2 its V */
} PrepBlock;

/* A pre-pass block with its batch (one round of scalar loads) */
typedef struct {
    PrepBlock blk;
    PrepBatch b;
} PrepBlockB;

typedef struct {
    const void *q; int q_dtype; long long q_stride;
    const void *k; const void *v; int kv_dtype; long long kv_stride;
    const float *rope_cos; const float *rope_sin; int rope_kind; int rope_q; int rope_k;
    float qscale;
    int Hq, Hkv, G, hd, hdp;
    _Float16 *qs; long long qs_head_stride;
    _Float16 *qs_lo;           /* non-null: Q is also written as its fp16 lo part (Q - fp16(Q)) */
    uint16_t *kc; uint16_t *vtc; long long c_slot_stride; int cap;
    _Float16 *kf; _Float16 *vtf; int fcap;
    _Float16 *kf_lo;           /* non-null: the fresh K's fp16 lo part */
    int stage;                 /* SMOL_STAGE_F16 or SMOL_STAGE_QF32 */
    float *qs32;
    const PrepBlockB *blocks;
    /* per-head RMSNorm before RoPE (null: none): weights [hd] fp32 */
    const float *q_norm; const float *k_norm; float norm_eps;
    int *range_flag;           /* set to 1 when a value written to fp16 would overflow */
} PrepParams;

/* ---- k_attn_win: bidirectional windows resident in LDS ----
 * One workgroup per 128-row tile of a (window, head); the window's K and V
 * are read from the inputs (fp32 or bf16), converted to fp16 and written
 * to LDS once; no pre-pass. */
#ifndef WIN_ARG_WINDOWS
#define WIN_ARG_WINDOWS 255   /* windows passed in the kernel arguments */
#endif
#define WIN_TPB 512           /* threads of a k_attn_win workgroup: 8 waves, two per SIMD */
#define WIN_ROWS 128          /* rows of its tile (ksplit 1; 64 for ksplit 2): 16 per wave */
typedef struct {
    const void *q; const void *k; const void *v; int in_dtype;
    long long row_stride;      /* elements between consecutive tokens (n_heads * hd) */
    float *out; float qscale; int H; int n_windows;
    int tpu;                   /* tiles of the longest window */
    int ksplit;                /* 1: a workgroup's 8 waves hold 128 rows over every key; 2: two groups of
                                  4 waves hold 64 rows, each over half the window's slabs, merged in LDS */
    int n_xcc;                 /* XCDs: workgroup b runs on XCD b % n_xcc */
    int *range_flag;           /* set to 1 when a value written as fp16 would overflow */
    int precise;               /* 1: QK^T on fp16 hi + lo operands (Q always; K for fp32 inputs) */
    int ws[WIN_ARG_WINDOWS + 1];
} WinParams;

/* ---- k_dec: decode and short chunks, split over the workgroups of one XCD ----
 *
 * A group is one (sequence, kv head): its R = n_q * G query rows (R <= 64)
 * against the sequence's keys, split into n_split contiguous slab ranges,
 * one workgroup each. Every workgroup of a group runs on the same XCD
 * (workgroup b runs on XCD b % n_xcc, checked when a context is created), so
 * the partials and flags of a group meet in that XCD's L2. There is no
 * atomic: each split publishes its partial, waits for the stores, then
 * writes the call's epoch into its flag; the group's last split, placed
 * after every other split of its XCD in dispatch order (so each split it
 * waits for has been dispatched before it), polls the flags and merges. */
#define DEC_MAX_SPLIT 32      /* splits per group (the merge's LDS and the partial slots) */
#define DEC_ARG_SEQS 32       /* sequences passed in the kernel arguments */
#define DEC_ARG_ITEMS 320     /* workgroup items passed in the kernel arguments */
#define DEC_SPIN_LIMIT (1 << 22) /* flag polls before a merger gives up (writes NaN rows and raises
                                    the context's merge flag) */
#define SMOL_FLAG_WORDS 64       /* ints of a context's device flag block (256 bytes) */
#define SMOL_FLAG_MERGE 32       /* word of the merge flag: its own 128-byte line */

/* one workgroup of the grid (index = blockIdx.x); seq < 0: nothing to do.
 * A group's rows are cut into row blocks of at most DEC_RB(hd) rows; each
 * (sequence, kv head, row block) is merged on its own. */
typedef struct {
    short seq;
    unsigned char kvh, rb, split, n_split;
    short pad;
} DecItem;

#define DEC_RB(hd) ((hd) <= 128 ? 32 : 16) /* rows of a row block (registers of one wave) */

typedef struct {
    int pos;       /* decode: position of the new token (cache keys [0, pos) + the new key);
                      chunk: position of query 0 (keys [0, pos + n_q)) */
    int slot;      /* cache slot */
    int tok0;      /* input / output token row of query 0 (decode: the new K/V row too) */
    int n_q;       /* query tokens (1 for decode) */
} DecSeq;

typedef struct {
    /* bf16 cache of the layer: K [slot][kv][cap][hd], V^T [slot][kv][cap/32][hd][32] */
    const uint16_t *kc; const uint16_t *vtc; long long c_slot_stride; int cap;
    /* chunk mode: the call's new keys (and the older rows of their first
     * slab) in the fp16 staging; key k >= fresh_pos0 is fresh row fresh_row0 + k - fresh_pos0 */
    const _Float16 *kf; const _Float16 *vtf; int fcap; int fresh_pos0; int fresh_row0;
    const _Float16 *kf_lo;     /* the fresh K's fp16 lo part (null: K = fp16 hi alone) */
    /* chunk mode: fp32 Q scratch [kv][rows][hdp], rotated and scaled; row q * G + h */
    const float *qs32; long long qs_head_stride;
    /* decode mode (direct = 1): Q, the new K and V rows of the inputs, rotated here */
    int direct;
    const void *q_in; const void *k_in; const void *v_in; int in_dtype; long long q_stride; long long kv_stride;
    const float *rope_cos; const float *rope_sin; int rope_kind;
    const float *q_norm; const float *k_norm; float norm_eps;
    float qscale;              /* scale * log2 e */
    float *out; int Hq, Hkv, G;
    int window; float cap2;    /* window > 0: sliding window; cap2 > 0: softcap in log2 units */
    /* split-K: partial slot (merge group * DEC_MAX_SPLIT + split), merge group
     * (seq * Hkv + kvh) * n_rb + rb, of slot_floats floats:
     * O [R][hd], (m, l) [R][2], then the flag (an int) at slot_floats - 1,
     * alone in the slot's last 128 bytes */
    float *part; int slot_floats; unsigned epoch;
    /* captured launches (a HIP graph replayed at many positions): the call's
     * epoch is (*step_dev << 8) + epoch, step_dev a counter the host advances
     * before each replay and epoch the launch's own tag (1..255), and the
     * sequences come from seqs_dev; null otherwise */
    const unsigned *step_dev;
    int *err_flag;             /* set to 1 (plain store) by a merger that gave up waiting */
    int spin_limit;            /* flag polls before a merger gives up */
    int fault_merge;           /* 1: mergers wait for a flag value no split writes (tests the give-up path) */
    int n_rb;                  /* row blocks per (sequence, kv head) */
    int n_items;               /* grid size */
    const DecItem *items_dev;  /* the items when n_items > DEC_ARG_ITEMS */
    int n_seq;
    const DecSeq *seqs_dev;    /* the sequences when n_seq > DEC_ARG_SEQS or step_dev is set */
    DecSeq seqs[DEC_ARG_SEQS];
    DecItem items[DEC_ARG_ITEMS];
} DecParams;

/* ---- k_gemm (gemm.hip): the projections on bf16 MFMA ---- */
struct GemmParams {
    const uint16_t *w; /* [N][K] bf16 */
    const void *x;     /* [M][K] fp32 or bf16 */
    void *y;           /* [M][N] (act: [M][N / 2]) fp32 or bf16 (truncated) */
    const float *bias; /* [N] or null */
    const float *g;    /* [K] norm weight or null (fp32 x) */
    const float *res;  /* [M][y columns] or null; may equal y */
    float eps;
    int M, N, K;
    int act;           /* SMOL_LINEAR_ACT_* */
    int tiles_m, tiles;
    int per_xcd;       /* tiles dealt to each XCD */
    /* rm > 0: XCD x takes the tiles of region (x / rn, x % rn) of an rm x rn
     * split of the tile grid; 0: tiles [x per_xcd, (x + 1) per_xcd) in
     * row-block-fastest order */
    int rm, rn;
    /* nseg > 0: up to three outputs side by side (the Q, K and V of one x):
     * segment s covers the concatenated columns [seg_c[s], seg_c[s + 1]) of
     * the N, reads seg_w[s] and writes seg_y[s] with seg_c[s + 1] - seg_c[s]
     * columns; every boundary a multiple of the tile width; no bias or
     * activation. nseg 0: the one output w, y of N columns */
    int nseg;
    int seg_c[4];
    const uint16_t *seg_w[3];
    void *seg_y[3];
};

#endif
