/*
 * attn_api.hip - host side of libsmol_attn.so: the C ABI of include/smol_attn.h
 * and include/smol_kernels_attn.h.
 *
 * Each attention call builds small descriptor tables on the host (which rows
 * and keys each kernel block covers), copies them to the device through a
 * ring of pinned buffers, and enqueues two kernels on the context's stream:
 * k_prep (RoPE + cache append + staging) and one attention kernel:
 * k_attn_fb (prefill over new keys), k_attn_fa (prefill over a cache prefix)
 * or k_attn_dec (decode and short chunks). Nothing here computes attention on
 * the host; without a GPU every entry point fails with SMOL_ATTN_ERR_NO_GPU.
 */
#include <hip/hip_runtime.h>

#include <float.h>
#include <limits.h>
#include <math.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <atomic>
#include <mutex>
#include <numeric>
#include <queue>
#include <vector>

#include "../../include/smol_attn.h"
#include "../../include/smol_kernels_attn.h"
#include "attn_internal.h"

extern "C" int smol_launch_prep(const PrepParams *pp, int n_blocks, hipStream_t st, hipEvent_t ev0, hipEvent_t ev1);
extern "C" int smol_launch_decode(const DecParams *dp, int hd, int rows, int nw, hipStream_t st, hipEvent_t ev0,
                                  hipEvent_t ev1);
extern "C" int smol_launch_xcc_probe(unsigned *out, int n, hipStream_t st);
extern "C" int smol_decode_occupancy(int hd, int rows, int nw, int direct);
extern "C" int smol_launch_fa(const SkParams *sp, int hd, int n_items, int nt, int w, hipStream_t st, hipEvent_t ev0,
                              hipEvent_t ev1);
extern "C" int smol_launch_fb(const SkParams *sp, int hd, int n_items, int nt, hipStream_t st, hipEvent_t ev0,
                              hipEvent_t ev1);
extern "C" int smol_launch_win(const WinParams *wp, int hd, int n_tiles, int max_len, hipStream_t st, hipEvent_t e0,
                               hipEvent_t e1);
extern "C" int smol_win_max_keys(int hd, int in_dtype, int precise);
extern "C" int smol_launch_to_bf16_trunc(const float *x, uint16_t *y, long long n, hipStream_t st);
extern "C" int smol_launch_bf16_norm_rope(uint16_t *x, const float *w, uint16_t *x2, const float *w2, int H2,
                                          float eps, const float *cos_t, const float *sin_t, int pos0, int seq, int H,
                                          int hd, hipStream_t st);
extern "C" int smol_launch_norm_rope(float *x, const float *w, float eps, const float *cos_t, const float *sin_t,
                                     const int *pos, int seq, int n_heads, int hd, int kind, hipStream_t st);

#define LOG2E_D 1.4426950408889634

/* ------------------------------------------------------------------ errors */

static thread_local char g_err[512];

static int fail(int code, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}

/* the same error channel for the library's other translation units */
extern "C" int smol_internal_fail(int code, const char *msg) { return fail(code, "%s", msg); }

#define HIP_TRY(expr)                                                                    \
    do {                                                                                 \
        hipError_t e_ = (expr);                                                          \
        if (e_ != hipSuccess)                                                            \
            return fail(SMOL_ATTN_ERR_DEVICE, "%s: %s", #expr, hipGetErrorString(e_));   \
    } while (0)

extern "C" const char *smol_attn_version(void) { return "smol_attn 0.1 gfx950"; }
extern "C" const char *smol_attn_last_error(void) { return g_err; }

extern "C" int smol_attn_device_count(void) {
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n <= 0)
        return fail(SMOL_ATTN_ERR_NO_GPU, "no HIP device: %s", hipGetErrorString(e));
    return n;
}

static bool hd_supported(int hd) {
    return hd == 64 || hd == 72 || hd == 80 || hd == 96 || hd == 128 || hd == 256;
}

/* ---------------------------------------------------------------- buffers */

struct DevBuf {
    void *p = nullptr;
    size_t cap = 0;
};

/* grow a device buffer; contents are not kept. The stream is drained first
 * because earlier kernels may still read the old allocation. */
static int dev_reserve(DevBuf &b, size_t bytes, hipStream_t st, bool zero = false) {
    if (bytes <= b.cap) return 0;
    size_t want = std::max(bytes, b.cap + b.cap / 2);
    want = (want + 4095) & ~(size_t)4095;
    if (b.p) {
        HIP_TRY(hipStreamSynchronize(st));
        HIP_TRY(hipFree(b.p));
        b.p = nullptr;
        b.cap = 0;
    }
    HIP_TRY(hipMalloc(&b.p, want));
    if (zero) HIP_TRY(hipMemsetAsync(b.p, 0, want, st));
    b.cap = want;
    return 0;
}

/* ------------------------------------------------ no-alloc decode scratch */

/* k_dec's partial slots and flags for smol_attn_decode_noalloc: one copy of
 * this array per GPU, reserved when the code object loads on that GPU and
 * held until the process ends. On the host the name only stands for the
 * symbol and is never used as an address: each device's address comes from
 * hipGetSymbolAddress, called with that device current, and is kept in
 * g_scratch. */
static __device__ __align__(256) float scratch[SMOL_ATTN_NOALLOC_SCRATCH_BYTES / 4];

#define SMOL_MAX_DEVICES 64
struct ScratchDev {
    void *ptr = nullptr;               /* this device's copy of `scratch` */
    std::atomic<unsigned> epoch{0};    /* last epoch handed to a no-alloc call */
};
static ScratchDev g_scratch[SMOL_MAX_DEVICES];
static std::mutex g_scratch_mu;

/* once per device, with that device current (context creation) */
static int scratch_setup(int device) {
    if (device < 0 || device >= SMOL_MAX_DEVICES)
        return fail(SMOL_ATTN_ERR_UNSUPPORTED, "device ordinal %d (at most %d devices)", device, SMOL_MAX_DEVICES);
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (g_scratch[device].ptr) return 0;
    void *ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr)
        return fail(SMOL_ATTN_ERR_DEVICE, "decode scratch on device %d: %s", device, hipGetErrorString(e));
    g_scratch[device].ptr = ptr;
    return 0;
}

/* Ring of pinned host staging buffers for the per-call descriptor tables.
 * A slot is reused only after the copy that last read it has completed. */
struct PinnedSlot {
    void *h = nullptr;
    size_t cap = 0;
    hipEvent_t ev = nullptr;
    bool pending = false;
};

#define SMOL_RING 16
#define SMOL_TIMING_KINDS 3 /* 0: pre-pass, 1: attention, 2: other */

/* Decode launches captured into a HIP graph read their sequence record and
 * their epoch's high bits from this state's device memory, so one graph
 * replays at any position up to the planning position: before each replay
 * the host launches k_gdec_step, which writes the position and advances the
 * step counter. The partial slots are the state's own (never shared with
 * uncaptured launches, whose epochs come from the host). */
struct smol_graph_dec {
    int device = 0;
    void *mem = nullptr; /* [0, 64): the sequence record; [64, 68): the step counter; slots from 256 */
    DecSeq *seqs = nullptr;
    unsigned *step = nullptr;
    float *part = nullptr;
    size_t part_bytes = 0;
    int plan_pos = 0;
};

struct smol_attn_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    bool own_stream = false;
    PinnedSlot ring[SMOL_RING];
    int ring_next = 0;
    DevBuf desc;   /* device copy of the descriptor tables */
    std::vector<unsigned char> desc_last; /* host bytes of the last upload to `desc` */
    DevBuf qs, kf, vtf, part_o, part_ml, counters;
    DevBuf kf_lo; /* fp16 lo part of the fresh K (precise QK^T) */
    DevBuf qs32; /* fp32 Q scratch of the decode kernel */
    DevBuf out32; /* fp32 result of a call whose output is bf16 */
    DevBuf dec_part; /* k_dec partial slots and flags */
    /* device flags, 256 bytes: word 0 is set by kernels when fp16 staging
     * overflows, word 32 (its own 128-byte line) by a k_dec merger that gave
     * up waiting for its splits; synchronize reads and clears both */
    int *range_flag = nullptr;
    /* kernel arguments of k_dec and k_attn_win, built in place per context
     * (several KB: kept off the stack; one thread per context, so no two
     * calls build them at once) */
    DecParams dp;
    WinParams wp;
    int cu_count = 256;
    int n_xcc = 1;       /* XCDs of the device */
    bool xcd_ok = true;  /* workgroup b runs on XCD b % n_xcc (checked at creation) */
    unsigned epoch = 0;  /* k_dec launches so far: each one's flags carry its own value */
    int opt[SMOL_OPT_COUNT] = {};
    /* opt-in per-kernel timing: events bracketing each launch */
    bool timing = false;
    struct Mark { int kind; hipEvent_t a, b; };
    std::vector<Mark> marks;
    std::vector<hipEvent_t> event_pool;
    double t_ms[SMOL_TIMING_KINDS] = {0, 0, 0};
    int t_count[SMOL_TIMING_KINDS] = {0, 0, 0};
    /* set while a caller captures decode launches into a HIP graph
     * (smol_internal_gdec_capture): k_dec then reads its positions and epoch
     * from this state's device memory */
    smol_graph_dec *gdec = nullptr;
    bool timing_saved = false; /* timing is off while a capture runs */
};

/* for linear.hip: the context's device and its compute units */
extern "C" int smol_internal_ctx_device(smol_attn_ctx *ctx) { return ctx->device; }
extern "C" int smol_internal_ctx_cus(smol_attn_ctx *ctx) { return ctx->cu_count; }
extern "C" int smol_internal_ctx_option(smol_attn_ctx *ctx, int option) { return ctx->opt[option]; }

static hipEvent_t pool_event(smol_attn_ctx *ctx) {
    if (!ctx->event_pool.empty()) {
        hipEvent_t e = ctx->event_pool.back();
        ctx->event_pool.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    return e;
}

/* A timed launch of `kind` (-1 unless timing is enabled): the launch itself
 * records the pair (hipExtLaunchKernelGGL with start and stop events), so the
 * events bracket the kernel's own execution and nothing else in the stream. */
static int timing_begin(smol_attn_ctx *ctx, int kind) {
    if (!ctx->timing) return -1;
    hipEvent_t a = pool_event(ctx), b = pool_event(ctx);
    if (!a || !b) return -1;
    ctx->marks.push_back({kind, a, b});
    return (int)ctx->marks.size() - 1;
}

static hipEvent_t mark_a(smol_attn_ctx *ctx, int mark) { return mark >= 0 ? ctx->marks[mark].a : nullptr; }
static hipEvent_t mark_b(smol_attn_ctx *ctx, int mark) { return mark >= 0 ? ctx->marks[mark].b : nullptr; }

/* for linear.hip: the pair of events that brackets one timed launch of the
 * given kind (both null when timing is off) */
extern "C" void smol_internal_timing_events(smol_attn_ctx *ctx, int kind, hipEvent_t *a, hipEvent_t *b) {
    const int mk = timing_begin(ctx, kind);
    *a = mark_a(ctx, mk);
    *b = mark_b(ctx, mk);
}

/* Tables and caches keep their own device and stream, so destroying them
 * does not touch the context (which may already be gone). */
struct smol_rope_table {
    smol_attn_ctx *ctx;
    int device;
    hipStream_t stream;
    int hd, type, cap;
    float theta;
    float *cos_d = nullptr, *sin_d = nullptr;
};

struct smol_kv_cache {
    smol_attn_ctx *ctx;
    int device;
    hipStream_t stream;
    int n_layers, n_slots, n_kv, hd, cap;
    uint16_t *k = nullptr, *vt = nullptr;
};

static int set_device(smol_attn_ctx *ctx) {
    HIP_TRY(hipSetDevice(ctx->device));
    return 0;
}

/* copy `bytes` of descriptor data to ctx->desc via the pinned ring */
/* Copies the descriptor tables to the device, unless the device buffer already
 * holds exactly these bytes (a decoder calls with the same shapes layer after
 * layer; stream order keeps the buffer valid for every later kernel). */
static int upload_desc(smol_attn_ctx *ctx, const void *host, size_t bytes) {
    if (ctx->desc.p && bytes == ctx->desc_last.size() && memcmp(ctx->desc_last.data(), host, bytes) == 0) return 0;
    ctx->desc_last.clear();
    int rc = dev_reserve(ctx->desc, bytes, ctx->stream);
    if (rc) return rc;
    PinnedSlot &s = ctx->ring[ctx->ring_next];
    ctx->ring_next = (ctx->ring_next + 1) % SMOL_RING;
    if (s.pending) {
        HIP_TRY(hipEventSynchronize(s.ev));
        s.pending = false;
    }
    if (bytes > s.cap) {
        if (s.h) HIP_TRY(hipHostFree(s.h));
        s.h = nullptr;
        size_t want = std::max(bytes, (size_t)65536);
        HIP_TRY(hipHostMalloc(&s.h, want, hipHostMallocDefault));
        s.cap = want;
    }
    if (!s.ev) HIP_TRY(hipEventCreateWithFlags(&s.ev, hipEventDisableTiming));
    memcpy(s.h, host, bytes);
    HIP_TRY(hipMemcpyAsync(ctx->desc.p, s.h, bytes, hipMemcpyHostToDevice, ctx->stream));
    HIP_TRY(hipEventRecord(s.ev, ctx->stream));
    s.pending = true;
    ctx->desc_last.assign((const unsigned char *)host, (const unsigned char *)host + bytes);
    return 0;
}

/* ------------------------------------------------------------------ context */

/* k_dec merges the splits of a group through one XCD's L2, which needs
 * workgroup b of a launch to run on XCD b % n_xcc (the round-robin dispatch
 * of a device in one partition). A probe grid records each workgroup's XCC
 * id; when any differs, k_dec keeps every group in one workgroup. */
static int check_xcd_dispatch(smol_attn_ctx *c) {
    int nx = 0;
    if (hipDeviceGetAttribute(&nx, hipDeviceAttributeNumberOfXccs, c->device) != hipSuccess || nx <= 0) nx = 1;
    c->n_xcc = nx;
    c->xcd_ok = true;
    if (nx == 1) return 0;
    const int n = 64 * nx;
    unsigned *d = nullptr;
    HIP_TRY(hipMalloc(&d, n * sizeof(unsigned)));
    std::vector<unsigned> h(n, 0xFFFFFFFFu);
    int rc = smol_launch_xcc_probe(d, n, c->stream);
    hipError_t e = rc ? hipErrorLaunchFailure : hipMemcpyAsync(h.data(), d, n * sizeof(unsigned), hipMemcpyDeviceToHost, c->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    hipFree(d);
    if (e != hipSuccess) return fail(SMOL_ATTN_ERR_DEVICE, "XCD probe: %s", hipGetErrorString(e));
    for (int b = 0; b < n; b++)
        if (h[b] != (unsigned)(b % nx)) c->xcd_ok = false;
    return 0;
}

extern "C" int smol_attn_ctx_create(int device, void *stream, smol_attn_ctx **out) {
    if (!out) return fail(SMOL_ATTN_ERR_ARG, "out is NULL");
    *out = nullptr;
    int n = smol_attn_device_count();
    if (n < 0) return n;
    if (device < 0 || device >= n) return fail(SMOL_ATTN_ERR_ARG, "device %d of %d", device, n);
    smol_attn_ctx *c = new smol_attn_ctx();
    c->device = device;
    hipError_t e = hipSetDevice(device);
    if (e == hipSuccess) {
        /* NULL is the device's null stream, ordered with other work on it */
        c->stream = (hipStream_t)stream;
    }
    int cus = 0;
    if (e == hipSuccess && hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) == hipSuccess && cus > 0)
        c->cu_count = cus;
    if (e != hipSuccess) {
        delete c;
        return fail(SMOL_ATTN_ERR_DEVICE, "context: %s", hipGetErrorString(e));
    }
    int rc = scratch_setup(device);
    if (!rc) rc = check_xcd_dispatch(c);
    if (!rc) {
        if (hipMalloc((void **)&c->range_flag, 256) != hipSuccess ||
            hipMemset(c->range_flag, 0, 256) != hipSuccess)
            rc = fail(SMOL_ATTN_ERR_NOMEM, "range flag: %s", hipGetErrorString(hipGetLastError()));
    }
    if (rc) {
        if (c->range_flag) hipFree(c->range_flag);
        delete c;
        return rc;
    }
    *out = c;
    return SMOL_ATTN_OK;
}

extern "C" int smol_attn_ctx_destroy(smol_attn_ctx *ctx) {
    if (!ctx) return SMOL_ATTN_OK;
    hipSetDevice(ctx->device);
    hipStreamSynchronize(ctx->stream);
    DevBuf *bufs[] = {&ctx->desc, &ctx->qs, &ctx->kf, &ctx->kf_lo, &ctx->vtf, &ctx->part_o, &ctx->part_ml, &ctx->counters,
                      &ctx->qs32, &ctx->out32, &ctx->dec_part};
    for (DevBuf *b : bufs)
        if (b->p) hipFree(b->p);
    if (ctx->range_flag) hipFree(ctx->range_flag);
    for (auto &s : ctx->ring) {
        if (s.h) hipHostFree(s.h);
        if (s.ev) hipEventDestroy(s.ev);
    }
    for (auto &m : ctx->marks) {
        hipEventDestroy(m.a);
        hipEventDestroy(m.b);
    }
    for (hipEvent_t e : ctx->event_pool) hipEventDestroy(e);
    if (ctx->own_stream) hipStreamDestroy(ctx->stream);
    delete ctx;
    return SMOL_ATTN_OK;
}

extern "C" int smol_attn_ctx_synchronize(smol_attn_ctx *ctx) {
    if (!ctx) return fail(SMOL_ATTN_ERR_ARG, "ctx is NULL");
    HIP_TRY(hipSetDevice(ctx->device));
    HIP_TRY(hipStreamSynchronize(ctx->stream));
    int flag[SMOL_FLAG_WORDS] = {};
    HIP_TRY(hipMemcpy(flag, ctx->range_flag, sizeof(flag), hipMemcpyDeviceToHost));
    if (flag[0] || flag[SMOL_FLAG_MERGE]) {
        const int zero[SMOL_FLAG_WORDS] = {};
        HIP_TRY(hipMemcpy(ctx->range_flag, zero, sizeof(zero), hipMemcpyHostToDevice));
    }
    if (flag[SMOL_FLAG_MERGE])
        return fail(SMOL_ATTN_ERR_TIMEOUT, "a decode split-K merge gave up waiting for its splits (the affected "
                    "rows are NaN)");
    if (flag[0])
        return fail(SMOL_ATTN_ERR_RANGE, "a staged Q, K or V value was not finite or reached 65520 in magnitude "
                    "(fp16 staging of the prefill and bidirectional kernels)");
    return SMOL_ATTN_OK;
}

extern "C" void *smol_attn_ctx_stream(smol_attn_ctx *ctx) { return ctx ? (void *)ctx->stream : nullptr; }

extern "C" int smol_attn_ctx_set_option(smol_attn_ctx *ctx, int option, int value) {
    if (!ctx) return fail(SMOL_ATTN_ERR_ARG, "ctx is NULL");
    if (option < 0 || option >= SMOL_OPT_COUNT || option == SMOL_OPT_XCD_CHECK)
        return fail(SMOL_ATTN_ERR_ARG, "option %d cannot be set", option);
    ctx->opt[option] = value;
    return SMOL_ATTN_OK;
}

extern "C" int smol_attn_ctx_get_option(smol_attn_ctx *ctx, int option, int *value) {
    if (!ctx || !value) return fail(SMOL_ATTN_ERR_ARG, "NULL argument");
    if (option < 0 || option >= SMOL_OPT_COUNT) return fail(SMOL_ATTN_ERR_ARG, "option %d", option);
    *value = option == SMOL_OPT_XCD_CHECK ? (ctx->xcd_ok ? 1 : 0) : ctx->opt[option];
    return SMOL_ATTN_OK;
}

extern "C" int smol_attn_ctx_set_timing(smol_attn_ctx *ctx, int enable) {
    if (!ctx) return fail(SMOL_ATTN_ERR_ARG, "ctx is NULL");
    ctx->timing = enable != 0;
    return SMOL_ATTN_OK;
}

extern "C" int smol_attn_ctx_timing_read(smol_attn_ctx *ctx, double *ms, int *count) {
    if (!ctx || !ms || !count) return fail(SMOL_ATTN_ERR_ARG, "NULL argument");
    HIP_TRY(hipStreamSynchronize(ctx->stream));
    for (auto &m : ctx->marks) {
        float t = 0.0f;
        HIP_TRY(hipEventElapsedTime(&t, m.a, m.b));
        ctx->t_ms[m.kind] += t;
        ctx->t_count[m.kind] += 1;
        ctx->event_pool.push_back(m.a);
        ctx->event_pool.push_back(m.b);
    }
    ctx->marks.clear();
    for (int k = 0; k < SMOL_TIMING_KINDS; k++) {
        ms[k] = ctx->t_ms[k];
        count[k] = ctx->t_count[k];
        ctx->t_ms[k] = 0.0;
        ctx->t_count[k] = 0;
    }
    return SMOL_ATTN_OK;
}

/* --------------------------------------------------------------- RoPE table */

/* qkn_decoder.c:261-311: inv_freq[d] = 1/powf(theta, 2d/hd); angle = (float)pos * inv_freq[d] */
extern "C" void smol_rope_fill_host(float *cos_out, float *sin_out, int pos0, int n_pos, int hd,
                                    float theta, int rope_type) {
    const int half = hd / 2;
    std::vector<float> inv(half > 0 ? half : 1);
    for (int d = 0; d < half; d++) {
        volatile float e = (float)(2 * d) / (float)hd;
        inv[d] = 1.0f / powf(theta, e);
    }
    for (int r = 0; r < n_pos; r++) {
        const float p = (float)(pos0 + r);
        float *cr = cos_out + (size_t)r * hd, *sr = sin_out + (size_t)r * hd;
        for (int d = 0; d < half; d++) {
            volatile float a = p * inv[d];
            const float c = cosf(a), s = sinf(a);
            if (rope_type == SMOL_ROPE_INTERLEAVED) {
                cr[2 * d] = c; cr[2 * d + 1] = c; sr[2 * d] = s; sr[2 * d + 1] = s;
            } else {
                cr[d] = c; cr[half + d] = c; sr[d] = s; sr[half + d] = s;
            }
        }
    }
}

static int rope_upload(smol_rope_table *rt, int new_cap) {
    smol_attn_ctx *ctx = rt->ctx;
    std::vector<float> c((size_t)new_cap * rt->hd), s((size_t)new_cap * rt->hd);
    smol_rope_fill_host(c.data(), s.data(), 0, new_cap, rt->hd, rt->theta, rt->type);
    float *cd = nullptr, *sd = nullptr;
    HIP_TRY(hipStreamSynchronize(ctx->stream));
    HIP_TRY(hipMalloc(&cd, c.size() * sizeof(float)));
    HIP_TRY(hipMalloc(&sd, s.size() * sizeof(float)));
    HIP_TRY(hipMemcpy(cd, c.data(), c.size() * sizeof(float), hipMemcpyHostToDevice));
    HIP_TRY(hipMemcpy(sd, s.data(), s.size() * sizeof(float), hipMemcpyHostToDevice));
    if (rt->cos_d) hipFree(rt->cos_d);
    if (rt->sin_d) hipFree(rt->sin_d);
    rt->cos_d = cd;
    rt->sin_d = sd;
    rt->cap = new_cap;
    return 0;
}

extern "C" int smol_rope_table_create(smol_attn_ctx *ctx, int hd, float theta, int type, int cap,
                                      smol_rope_table **out) {
    if (!ctx || !out) return fail(SMOL_ATTN_ERR_ARG, "NULL argument");
    *out = nullptr;
    if (hd <= 0 || (hd & 1) || hd > 512) return fail(SMOL_ATTN_ERR_ARG, "head_dim %d", hd);
    if (type != SMOL_ROPE_NEOX && type != SMOL_ROPE_INTERLEAVED)
        return fail(SMOL_ATTN_ERR_ARG, "rope_type %d", type);
    if (!(theta > 0.0f)) return fail(SMOL_ATTN_ERR_ARG, "theta must be > 0");
    int rc = set_device(ctx);
    if (rc) return rc;
    smol_rope_table *rt = new smol_rope_table();
    rt->ctx = ctx;
    rt->device = ctx->device;
    rt->stream = ctx->stream;
    rt->hd = hd;
    rt->type = type;
    rt->theta = theta;
    rt->cap = 0;
    int c = 1024;
    while (c < cap) c *= 2;
    rc = rope_upload(rt, c);
    if (rc) { delete rt; return rc; }
    *out = rt;
    return SMOL_ATTN_OK;
}

extern "C" int smol_rope_table_ensure(smol_rope_table *rt, int required_pos) {
    if (!rt) return fail(SMOL_ATTN_ERR_ARG, "NULL table");
    if (required_pos <= rt->cap) return SMOL_ATTN_OK;
    int c = rt->cap > 0 ? rt->cap : 1024;
    while (c < required_pos) c *= 2;
    int rc = set_device(rt->ctx);
    return rc ? rc : rope_upload(rt, c);
}

extern "C" int smol_rope_table_capacity(const smol_rope_table *rt) { return rt ? rt->cap : 0; }

extern "C" int smol_rope_table_destroy(smol_rope_table *rt) {
    if (!rt) return SMOL_ATTN_OK;
    hipSetDevice(rt->device);
    hipStreamSynchronize(rt->stream);
    if (rt->cos_d) hipFree(rt->cos_d);
    if (rt->sin_d) hipFree(rt->sin_d);
    delete rt;
    return SMOL_ATTN_OK;
}

/* ----------------------------------------------------------------- KV cache */

static size_t kv_slot_elems(const smol_kv_cache *kv) { return (size_t)kv->n_kv * kv->cap * kv->hd; }
static size_t kv_layer_elems(const smol_kv_cache *kv) { return kv_slot_elems(kv) * kv->n_slots; }

extern "C" int smol_kv_cache_create(smol_attn_ctx *ctx, int n_layers, int n_slots, int n_kv, int hd,
                                    int max_seq, smol_kv_cache **out) {
    if (!ctx || !out) return fail(SMOL_ATTN_ERR_ARG, "NULL argument");
    *out = nullptr;
    if (n_layers <= 0 || n_slots <= 0 || n_kv <= 0 || max_seq <= 0)
        return fail(SMOL_ATTN_ERR_ARG, "cache shape %d/%d/%d/%d", n_layers, n_slots, n_kv, max_seq);
    if (!hd_supported(hd)) return fail(SMOL_ATTN_ERR_UNSUPPORTED, "head_dim %d", hd);
    int rc = set_device(ctx);
    if (rc) return rc;
    smol_kv_cache *kv = new smol_kv_cache();
    kv->ctx = ctx;
    kv->device = ctx->device;
    kv->stream = ctx->stream;
    kv->n_layers = n_layers;
    kv->n_slots = n_slots;
    kv->n_kv = n_kv;
    kv->hd = hd;
    kv->cap = (max_seq + 63) & ~63;
    size_t bytes = kv_layer_elems(kv) * n_layers * sizeof(uint16_t);
    hipError_t e = hipMalloc(&kv->k, bytes);
    if (e == hipSuccess) e = hipMalloc(&kv->vt, bytes);
    if (e == hipSuccess) e = hipMemsetAsync(kv->k, 0, bytes, ctx->stream);
    if (e == hipSuccess) e = hipMemsetAsync(kv->vt, 0, bytes, ctx->stream);
    if (e != hipSuccess) {
        if (kv->k) hipFree(kv->k);
        if (kv->vt) hipFree(kv->vt);
        delete kv;
        return fail(e == hipErrorOutOfMemory ? SMOL_ATTN_ERR_NOMEM : SMOL_ATTN_ERR_DEVICE,
                    "kv cache (%zu bytes): %s", bytes, hipGetErrorString(e));
    }
    *out = kv;
    return SMOL_ATTN_OK;
}

extern "C" int smol_kv_cache_destroy(smol_kv_cache *kv) {
    if (!kv) return SMOL_ATTN_OK;
    hipSetDevice(kv->device);
    hipStreamSynchronize(kv->stream);
    hipFree(kv->k);
    hipFree(kv->vt);
    delete kv;
    return SMOL_ATTN_OK;
}

extern "C" int smol_kv_cache_capacity(const smol_kv_cache *kv) { return kv ? kv->cap : 0; }

/* kv_cache_grow (qkn_decoder.c:183-210): double until it fits, keep contents */
extern "C" int smol_kv_cache_reserve(smol_kv_cache *kv, int required) {
    if (!kv) return fail(SMOL_ATTN_ERR_ARG, "NULL cache");
    if (required <= kv->cap) return SMOL_ATTN_OK;
    smol_attn_ctx *ctx = kv->ctx;
    int rc = set_device(ctx);
    if (rc) return rc;
    int nc = kv->cap;
    while (nc < required) nc *= 2;
    smol_kv_cache nkv = *kv;
    nkv.cap = nc;
    size_t bytes = kv_layer_elems(&nkv) * kv->n_layers * sizeof(uint16_t);
    uint16_t *nk = nullptr, *nvt = nullptr;
    hipError_t e = hipMalloc(&nk, bytes);
    if (e == hipSuccess) e = hipMalloc(&nvt, bytes);
    if (e != hipSuccess) {
        if (nk) hipFree(nk);
        return fail(SMOL_ATTN_ERR_NOMEM, "kv cache grow to %d: %s", nc, hipGetErrorString(e));
    }
    HIP_TRY(hipMemsetAsync(nk, 0, bytes, ctx->stream));
    HIP_TRY(hipMemsetAsync(nvt, 0, bytes, ctx->stream));
    const int hd = kv->hd;
    const size_t n_blocks = (size_t)kv->n_layers * kv->n_slots * kv->n_kv;
    /* per (layer, slot, head): K [cap][hd] and slab-blocked V^T [cap/32][hd][32]
     * are both prefixes of the grown region */
    const size_t old_bytes = (size_t)kv->cap * hd * sizeof(uint16_t);
    HIP_TRY(hipMemcpy2DAsync(nk, (size_t)nc * hd * sizeof(uint16_t), kv->k, old_bytes, old_bytes, n_blocks,
                             hipMemcpyDeviceToDevice, ctx->stream));
    HIP_TRY(hipMemcpy2DAsync(nvt, (size_t)nc * hd * sizeof(uint16_t), kv->vt, old_bytes, old_bytes, n_blocks,
                             hipMemcpyDeviceToDevice, ctx->stream));
    HIP_TRY(hipStreamSynchronize(ctx->stream));
    hipFree(kv->k);
    hipFree(kv->vt);
    kv->k = nk;
    kv->vt = nvt;
    kv->cap = nc;
    return SMOL_ATTN_OK;
}

/* ------------------------------------------------------------ the dispatcher */

struct Plan {
    std::vector<PrepBatch> pb;
    std::vector<PrepBlock> pblk;
    std::vector<SkBatch> sb;
    std::vector<SkItem> items;
    int n_groups = 0;
    int q_rows = 0;      /* Q scratch rows per KV head */
    int fresh_rows = 0;  /* fresh rows per KV head */
};

struct CallShape {
    bool dec;             /* true: fp32 Q staging + k_attn_dec; false: fp16 Q staging + k_attn_fb / k_attn_fa */
    const void *q, *k, *v;
    int dtype;
    int Hq, Hkv, hd;
    long long q_stride, kv_stride;
    float scale, cap;
    int window;
    const smol_rope_table *rope;
    int rope_q, rope_k;
    smol_kv_cache *kv;
    int layer;
    float *out;
    const float *q_norm = nullptr, *k_norm = nullptr; /* per-head RMSNorm weights [hd] or null */
    float norm_eps = 0.0f;
    bool direct = false;  /* k_attn_dec without the pre-pass (one query token and one new key per batch) */
};


/* rows_per: query rows of one work item; longest_first: order the merge
 * groups by descending key count, so the last workgroups dispatched are the
 * short ones */
static void plan_items(Plan &pl, int Hkv, int G, int window, int rows_per, int cu_count, bool longest_first,
                       bool no_split = false) {
    struct Tile { int batch, row0, lo, hi; };
    std::vector<Tile> tiles;
    long long total_slabs = 0;
    for (int bi = 0; bi < (int)pl.sb.size(); bi++) {
        const SkBatch &b = pl.sb[bi];
        for (int r0 = 0; r0 < b.n_rows; r0 += rows_per) {
            const int r1 = std::min(r0 + rows_per, b.n_rows) - 1;
            int lo = b.key_lo, hi = b.key_hi;
            if (b.causal) {
                hi = std::min(hi, b.q_pos0 + r1 / G + 1);
                if (window > 0) lo = std::max(lo, b.q_pos0 + r0 / G - window + 1);
            }
            lo = std::max(lo, 0) & ~(SMOL_SLAB - 1);
            if (hi < lo) hi = lo;
            tiles.push_back({bi, r0, lo, hi});
            total_slabs += (hi - lo + SMOL_SLAB - 1) / SMOL_SLAB;
        }
    }
    if (longest_first)
        std::stable_sort(tiles.begin(), tiles.end(),
                         [](const Tile &a, const Tile &b) { return a.hi - a.lo > b.hi - b.lo; });
    /* a workgroup per compute unit and wave slot, each wave >= 2 slabs */
    const long long target_items = (long long)cu_count;
    long long per = (total_slabs * Hkv + target_items - 1) / std::max(1LL, target_items);
    /* k_attn_fa gives each slab to all four waves: at least four slabs per item */
    int slabs_per_item = (int)std::max(4LL, per);
    if (no_split) slabs_per_item = 1 << 28;
    int group = 0;
    const int max_split = SK_MERGE_MAX / rows_per; /* the kernel's merge holds rows * n_split pairs in LDS */
    for (const Tile &t : tiles) {
        const int n_slabs = (t.hi - t.lo + SMOL_SLAB - 1) / SMOL_SLAB;
        int want = std::max(1, (n_slabs + slabs_per_item - 1) / slabs_per_item);
        const int n_split = std::min(max_split, want);
        const int per_split = (n_slabs + n_split - 1) / std::max(1, n_split);
        int made = 0;
        std::vector<SkItem> tmp;
        for (int sp = 0; sp < n_split; sp++) {
            int kb = t.lo + sp * per_split * SMOL_SLAB;
            int ke = std::min(t.hi, kb + per_split * SMOL_SLAB);
            if (sp > 0 && kb >= t.hi) break;
            if (ke < kb) ke = kb;
            const SkBatch &sb = pl.sb[t.batch];
            tmp.push_back({t.batch, t.row0, kb, ke, group, 0, made++, sb.fresh_row0 - sb.fresh_pos0});
        }
        for (SkItem &it : tmp) {
            it.n_split = made;
            pl.items.push_back(it);
        }
        group++;
    }
    pl.n_groups = group;
}

/* k_attn_fb with one key group: 128-row tiles cut into key pieces that fill
 * each workgroup's list to the same cost. The tiles, largest first, are laid
 * into lists of capacity C in turn, a tile cut exactly where a list is full
 * and continued in the next; a piece costs its slabs plus `overhead` steps
 * (start-up, epilogue, and a publish / merge when the tile is cut), and C is
 * the total cost over the workgroups a kv head gets (raised until the lists
 * fit). The pieces of a tile merge (group = tile, partial slots contiguous);
 * pl.items holds the pieces in slot order and `lists` each list's pieces. */
static void plan_fb_fill(Plan &pl, int Hkv, int G, int window, int cu_count, std::vector<std::vector<int>> &lists) {
    const int rows_per = 128, overhead = 3;
    struct Tile { int batch, row0, lo, hi, n; };
    std::vector<Tile> tiles;
    long long total = 0;
    for (int bi = 0; bi < (int)pl.sb.size(); bi++) {
        const SkBatch &b = pl.sb[bi];
        for (int r0 = 0; r0 < b.n_rows; r0 += rows_per) {
            const int r1 = std::min(r0 + rows_per, b.n_rows) - 1;
            int lo = b.key_lo, hi = b.key_hi;
            if (b.causal) {
                hi = std::min(hi, b.q_pos0 + r1 / G + 1);
                if (window > 0) lo = std::max(lo, b.q_pos0 + r0 / G - window + 1);
            }
            lo = std::max(lo, 0) & ~(SMOL_SLAB - 1);
            const int n = hi > lo ? (hi - lo + SMOL_SLAB - 1) / SMOL_SLAB : 0;
            tiles.push_back({bi, r0, lo, std::max(hi, lo), n});
            total += n + overhead;
        }
    }
    std::stable_sort(tiles.begin(), tiles.end(), [](const Tile &a, const Tile &b) { return a.n > b.n; });
    const int n_wg = std::max(1, cu_count / std::max(1, Hkv));
    const int max_split = SK_MERGE_MAX / rows_per;
    struct Piece { int tile, first, count; };
    std::vector<std::vector<Piece>> bins;
    for (double cap = std::max(1.0, (double)total / n_wg);; cap *= 1.02) {
        bins.assign(1, {});
        double room = cap;
        bool ok = true;
        for (int t = 0; t < (int)tiles.size() && ok; t++) {
            int first = 0, made = 0;
            do {
                if (room < overhead + 1 && !bins.back().empty()) {
                    bins.push_back({});
                    room = cap;
                }
                const int left = tiles[t].n - first;
                const int take = std::min(left, std::max(1, (int)(room - overhead)));
                bins.back().push_back({t, first, take});
                first += take;
                room -= take + overhead;
                if (++made > max_split) ok = false;
            } while (first < tiles[t].n);
        }
        if (ok && (int)bins.size() <= n_wg) break;
    }
    /* items in slot order: a tile's pieces contiguous, in key order */
    std::vector<std::vector<int>> pieces_of(tiles.size());
    std::vector<std::pair<int, int>> where; /* (bin, index in bin) of each piece, by piece id */
    std::vector<Piece> all;
    for (int bi = 0; bi < (int)bins.size(); bi++)
        for (int k = 0; k < (int)bins[bi].size(); k++) {
            pieces_of[bins[bi][k].tile].push_back((int)all.size());
            all.push_back(bins[bi][k]);
            where.push_back({bi, k});
        }
    std::vector<int> slot(all.size());
    pl.items.clear();
    for (int t = 0; t < (int)tiles.size(); t++) {
        const Tile &tl = tiles[t];
        const SkBatch &sb = pl.sb[tl.batch];
        const int ns = (int)pieces_of[t].size();
        for (int sp = 0; sp < ns; sp++) {
            const Piece &pc = all[pieces_of[t][sp]];
            slot[pieces_of[t][sp]] = (int)pl.items.size();
            const int kb = tl.lo + pc.first * SMOL_SLAB;
            const int ke = sp == ns - 1 ? tl.hi : tl.lo + (pc.first + pc.count) * SMOL_SLAB;
            pl.items.push_back({tl.batch, tl.row0, kb, std::max(kb, ke), t, ns, sp, sb.fresh_row0 - sb.fresh_pos0});
        }
    }
    pl.n_groups = (int)tiles.size();
    lists.assign(bins.size(), {});
    for (int p = 0; p < (int)all.size(); p++) lists[where[p].first].push_back(slot[p]);
}

/* the pre-pass blocks with their batches */
/* the pre-pass blocks with their batches; without_q: the Q blocks are left
 * out (k_attn_fb prepares its Q rows itself). A fresh slab becomes two
 * blocks, its K and its V (count 1 and 2), when the launch then still fits
 * the device in one round (`slots` workgroups at once): separate blocks keep
 * twice as many loads in flight, a second round costs more than that */
static std::vector<PrepBlockB> prep_records(const Plan &pl, bool without_q, int Hkv, int slots) {
    long long n = 0, nf = 0;
    for (const PrepBlock &b : pl.pblk) {
        if (without_q && b.kind == 1) continue;
        n++;
        nf += b.kind == 0;
    }
    const bool split = (n + nf) * Hkv <= slots;
    std::vector<PrepBlockB> r;
    r.reserve(pl.pblk.size() * 2);
    for (const PrepBlock &b : pl.pblk) {
        if (without_q && b.kind == 1) continue;
        if (split && b.kind == 0 && b.count == 0) {
            r.push_back({{b.batch, 0, b.first, 1}, pl.pb[b.batch]});
            r.push_back({{b.batch, 0, b.first, 2}, pl.pb[b.batch]});
        } else {
            r.push_back({b, pl.pb[b.batch]});
        }
    }
    return r;
}

/* k_attn_fb items with their batches' fields. With n_wg > 0 (fewer
 * workgroups per kv head than items) each item, longest first, goes to the
 * list with the least work so far: an item costs its steps (two slabs each,
 * one per key group) plus about six steps of start-up and epilogue. Item w
 * heads list w; `next` links the rest. */
static std::vector<FbItem> fb_items(const Plan &pl, int n_wg, bool one_group,
                                    const std::vector<std::vector<int>> *given = nullptr) {
    const int n = (int)pl.items.size();
    auto record = [&](int i) {
        const SkItem &it = pl.items[i];
        const SkBatch &b = pl.sb[it.batch];
        FbItem f;
        memset(&f, 0, sizeof(f));
        f.key_begin = it.key_begin; f.key_end = it.key_end; f.fresh_off = it.fresh_off; f.row0 = it.row0;
        f.n_rows = b.n_rows; f.q_row0 = b.q_row0; f.out_tok0 = b.out_tok0; f.q_pos0 = b.q_pos0;
        f.key_lo = b.key_lo; f.key_hi = b.key_hi; f.causal = b.causal; f.next = -1;
        /* merge group and partial slot: a group's items are contiguous in
         * the plan, so slot i - split is the group's first */
        f.group = it.group; f.n_split = it.n_split; f.split = it.split; f.part = i;
        return f;
    };
    std::vector<FbItem> out(n);
    if (n_wg <= 0) {
        for (int i = 0; i < n; i++) out[i] = record(i);
        return out;
    }
    std::vector<std::vector<int>> lists;
    if (given) {
        lists = *given; /* the planner's lists (plan_fb_fill) */
        n_wg = (int)lists.size();
    } else {
    std::vector<int> order(n);
    for (int i = 0; i < n; i++) order[i] = i;
    auto cost = [&](int i) {
        const SkItem &it = pl.items[i];
        const int slabs = (it.key_end - it.key_begin + SMOL_SLAB - 1) / SMOL_SLAB;
        /* a step per slab (one key group) or per two (two groups), start-up
         * and epilogue, and a publish and merge for a split item */
        return one_group ? slabs + 6 + (it.n_split > 1 ? 2 : 0) : (slabs + 1) / 2 + 6;
    };
    std::stable_sort(order.begin(), order.end(), [&](int a, int b) { return cost(a) > cost(b); });
    using Load = std::pair<long long, int>; /* (work, list) */
    std::priority_queue<Load, std::vector<Load>, std::greater<Load>> heap;
    for (int w = 0; w < n_wg; w++) heap.push({0, w});
    lists.assign(n_wg, {});
    for (int i : order) {
        Load l = heap.top();
        heap.pop();
        lists[l.second].push_back(i);
        heap.push({l.first + cost(i), l.second});
    }
    }
    /* new index of every item: the heads first, then the rest list by list */
    std::vector<int> at(n, -1);
    int k = n_wg;
    for (int w = 0; w < n_wg; w++)
        for (size_t e = 0; e < lists[w].size(); e++) at[lists[w][e]] = e == 0 ? w : k++;
    for (int w = 0; w < n_wg; w++)
        for (size_t e = 0; e < lists[w].size(); e++) {
            FbItem f = record(lists[w][e]);
            if (e + 1 < lists[w].size()) f.next = at[lists[w][e + 1]];
            out[at[lists[w][e]]] = f;
        }
    return out;
}

/* ---------------------------------------------------------------- k_dec plan */

/* query rows one k_dec workgroup holds: 8 (hi/lo packed in the MFMA columns),
 * 16, or a row block of DEC_RB(hd) */
static int dec_tile_rows(int hd, int rows) { return rows <= 8 ? 8 : rows <= 16 ? 16 : DEC_RB(hd); }

struct DecCall {
    bool direct;                  /* single-token decode, no pre-pass */
    bool noalloc = false;         /* partials in the per-device scratch; nothing allocated */
    bool whole = false;           /* one workgroup per (sequence, kv head, row block) */
    std::vector<DecSeq> seqs;
    /* chunk mode: the pre-pass's fresh window and Q scratch */
    int fresh_pos0 = 0, fresh_row0 = 0, fcap = 0;
    const _Float16 *kf_lo = nullptr; /* the fresh K's lo part (precise QK^T) */
    long long qs_head_stride = 0;
};

/* Places the (sequence, kv head) units on XCDs, longest first onto the XCD
 * with the least work so far, then splits each unit's slab range so that
 * every XCD's units fill the workgroups it holds at once (`fit`): a unit
 * gets a share of the XCD's slots in proportion to its slabs, at least
 * `min_per` slabs per workgroup (one per wave) and at most DEC_MAX_SPLIT
 * splits. Then each XCD's workgroups are ordered with every group's last
 * split after all of its other splits: the last split merges, and the
 * workgroups an XCD dispatches before it include every split it waits for.
 * Since no XCD gets more workgroups than it holds at once, none waits for
 * another to finish before it starts. Workgroup b is slot b / n_xcc of XCD
 * b % n_xcc; slots past an XCD's list are idle. SMOL_OPT_DEC_SLABS > 0
 * instead cuts every unit into workgroups of that many slabs. */
static void plan_decode(smol_attn_ctx *ctx, const DecCall &dc, int Hkv, int window, int n_rb, int fit, int min_per,
                        std::vector<DecItem> &items) {
    const int nx = ctx->n_xcc;
    const int n_seq = (int)dc.seqs.size();
    auto slabs_of = [&](const DecSeq &q) {
        const int kend = dc.direct ? q.pos : q.pos + q.n_q;
        const int klo = (window > 0 ? std::max(0, q.pos - window + 1) : 0) & ~(SMOL_SLAB - 1);
        return kend > klo ? (kend - klo + SMOL_SLAB - 1) / SMOL_SLAB : 0;
    };
    const int forced = ctx->opt[SMOL_OPT_DEC_SLABS];
    const bool no_split = !ctx->xcd_ok || ctx->opt[SMOL_OPT_DEC_SPLIT] == -1 || dc.whole;
    struct Unit { int seq, kvh, ns, n_split, xcd; };
    std::vector<Unit> units;
    for (int i = 0; i < n_seq; i++) {
        const int ns = slabs_of(dc.seqs[i]);
        for (int g = 0; g < Hkv; g++) units.push_back({i, g, ns, 1, 0});
    }
    std::vector<int> order(units.size());
    std::iota(order.begin(), order.end(), 0);
    std::stable_sort(order.begin(), order.end(), [&](int a, int b) { return units[a].ns > units[b].ns; });
    std::vector<long long> load(nx, 0);
    for (int u : order) {
        const int x = (int)(std::min_element(load.begin(), load.end()) - load.begin());
        units[u].xcd = x;
        load[x] += std::max(units[u].ns, 1);
    }
    if (!no_split && forced > 0) {
        for (Unit &u : units) u.n_split = std::max(1, std::min(DEC_MAX_SPLIT, (u.ns + forced - 1) / forced));
    } else if (!no_split) {
        for (int x = 0; x < nx; x++) {
            std::vector<Unit *> mine;
            long long groups = 0, work = 0;
            for (Unit &u : units)
                if (u.xcd == x) {
                    mine.push_back(&u);
                    groups += n_rb;
                    work += u.ns;
                }
            if (mine.empty() || groups >= fit) continue; /* every slot taken without splits */
            const double per = std::max<double>(min_per, (double)work * n_rb / fit);
            long long used = 0;
            for (Unit *u : mine) {
                const int cap = std::min(DEC_MAX_SPLIT, std::max(1, u->ns));
                u->n_split = std::max(1, std::min(cap, (int)std::lround(u->ns / per)));
                used += (long long)u->n_split * n_rb;
            }
            /* over the slots by rounding: take splits from the units whose
             * splits are shortest */
            while (used > fit) {
                Unit *v = nullptr;
                for (Unit *u : mine)
                    if (u->n_split > 1 && (!v || (double)u->ns / u->n_split < (double)v->ns / v->n_split)) v = u;
                if (!v) break;
                v->n_split--;
                used -= n_rb;
            }
        }
    }
    std::vector<std::vector<DecItem>> lists(nx), lasts(nx);
    for (const Unit &u : units)
        for (int rb = 0; rb < n_rb; rb++)
            for (int sp = 0; sp < u.n_split; sp++) {
                DecItem it;
                it.seq = (short)u.seq;
                it.kvh = (unsigned char)u.kvh;
                it.rb = (unsigned char)rb;
                it.split = (unsigned char)sp;
                it.n_split = (unsigned char)u.n_split;
                it.pad = 0;
                (sp == u.n_split - 1 ? lasts : lists)[u.xcd].push_back(it);
            }
    size_t slots = 0;
    for (int x = 0; x < nx; x++) {
        lists[x].insert(lists[x].end(), lasts[x].begin(), lasts[x].end());
        slots = std::max(slots, lists[x].size());
    }
    DecItem idle;
    memset(&idle, 0, sizeof(idle));
    idle.seq = -1;
    items.assign(slots * nx, idle);
    for (int x = 0; x < nx; x++)
        for (size_t k = 0; k < lists[x].size(); k++) items[k * nx + x] = lists[x][k];
}

/* Plans and launches k_dec for the sequences of `dc` */
/* a partial slot's floats: O [TR][hd], (m, l) [TR][2], then the flag alone
 * in the slot's last 128-byte line; 256-byte aligned */
static int dec_slot_floats(int hd, int TR) { return ((((TR * (hd + 2) + 31) & ~31) + 32) + 63) & ~63; }

static int run_decode(smol_attn_ctx *ctx, const CallShape &cs, const DecCall &dc) {
    const int hd = cs.hd, G = cs.Hq / cs.Hkv;
    int max_q = 0;
    for (const DecSeq &q : dc.seqs) max_q = std::max(max_q, q.n_q);
    const int rows = max_q * G;
    const int TR = dec_tile_rows(hd, rows);
    const int n_rb = (rows + TR - 1) / TR;
    if (n_rb > 255 || (int)dc.seqs.size() > 32767 || cs.Hkv > 255)
        return fail(SMOL_ATTN_ERR_UNSUPPORTED, "decode call too large (%d rows, %d sequences)", rows, (int)dc.seqs.size());
    const int nw = rows <= 8 && hd <= 128 ? (ctx->opt[SMOL_OPT_DEC_WAVES] == 8 ? 8 : 4) : 4;
    /* workgroups an XCD holds at once */
    const int fit = std::max(1, ctx->cu_count / ctx->n_xcc) * smol_decode_occupancy(hd, rows, nw, dc.direct ? 1 : 0);
    /* partial slots: O [TR][hd], (m, l) [TR][2], then the flag alone in the
     * slot's last 128-byte line (the merger polls that line device-coherently
     * and reads the others through L2); 256-byte aligned */
    const int slot_floats = dec_slot_floats(hd, TR);
    const size_t n_groups = dc.seqs.size() * cs.Hkv * n_rb;
    const size_t part_bytes = n_groups * DEC_MAX_SPLIT * slot_floats * 4;
    DecCall whole_dc;
    const DecCall *pdc = &dc;
    smol_graph_dec *gd = ctx->gdec;
    if (gd) {
        /* captured: one sequence, planned at the state's planning position
         * (every position up to it runs the same items; splits past a
         * shorter sequence's keys are empty) */
        if (!dc.direct || dc.noalloc || dc.seqs.size() != 1)
            return fail(SMOL_ATTN_ERR_UNSUPPORTED, "a captured decode is one sequence's direct decode step");
        if (cs.layer + 1 > 255) return fail(SMOL_ATTN_ERR_UNSUPPORTED, "captured decode: layer %d > 254", cs.layer);
        if (part_bytes > gd->part_bytes)
            return fail(SMOL_ATTN_ERR_UNSUPPORTED, "captured decode: %zu partial bytes, the state holds %zu",
                        part_bytes, gd->part_bytes);
        whole_dc = dc;
        whole_dc.seqs[0].pos = std::max(dc.seqs[0].pos, gd->plan_pos);
        pdc = &whole_dc;
    }
    if (dc.noalloc && part_bytes > SMOL_ATTN_NOALLOC_SCRATCH_BYTES) {
        /* the scratch cannot hold every group's split slots: no splits */
        whole_dc = dc;
        whole_dc.whole = true;
        pdc = &whole_dc;
    }
    /* at least one slab per wave of a split, two at head_dim 256: the merger
     * reads every split's rows x head_dim partial, and at head_dim 256 fewer,
     * longer splits win (C4: 23.4 -> 21.5 us) */
    const int min_per = hd > 128 ? 2 * nw : nw;
    std::vector<DecItem> items;
    plan_decode(ctx, *pdc, cs.Hkv, cs.window, n_rb, fit, min_per, items);
    if (dc.noalloc && items.size() > DEC_ARG_ITEMS && !pdc->whole) {
        whole_dc = dc;
        whole_dc.whole = true;
        pdc = &whole_dc;
        plan_decode(ctx, *pdc, cs.Hkv, cs.window, n_rb, fit, min_per, items);
    }
    if (gd && items.size() > DEC_ARG_ITEMS)
        return fail(SMOL_ATTN_ERR_UNSUPPORTED, "captured decode: %d workgroups exceed the kernel arguments' %d",
                    (int)items.size(), DEC_ARG_ITEMS);
    if (dc.noalloc && (items.size() > DEC_ARG_ITEMS || dc.seqs.size() > DEC_ARG_SEQS))
        return fail(SMOL_ATTN_ERR_UNSUPPORTED, "%d sequences / %d workgroups exceed what the no-alloc decode passes "
                    "in its kernel arguments (%d / %d)", (int)dc.seqs.size(), (int)items.size(), DEC_ARG_SEQS,
                    DEC_ARG_ITEMS);

    DecParams &dp = ctx->dp;
    static_assert(sizeof(DecParams) <= 4096, "kernel arguments");
    memset(&dp, 0, sizeof(dp));
    const smol_kv_cache *kv = cs.kv;
    dp.kc = kv->k + (size_t)cs.layer * kv_layer_elems(kv);
    dp.vtc = kv->vt + (size_t)cs.layer * kv_layer_elems(kv);
    dp.c_slot_stride = (long long)kv_slot_elems(kv);
    dp.cap = kv->cap;
    dp.direct = dc.direct ? 1 : 0;
    if (dc.direct) {
        dp.q_in = cs.q; dp.k_in = cs.k; dp.v_in = cs.v; dp.in_dtype = cs.dtype;
        dp.q_stride = cs.q_stride; dp.kv_stride = cs.kv_stride;
        if (cs.rope) {
            dp.rope_cos = cs.rope->cos_d;
            dp.rope_sin = cs.rope->sin_d;
            dp.rope_kind = cs.rope->type == SMOL_ROPE_INTERLEAVED ? SMOL_ROPE_INTERLEAVED_K : SMOL_ROPE_NEOX_K;
        } else {
            dp.rope_kind = SMOL_ROPE_OFF;
        }
        dp.q_norm = cs.q_norm; dp.k_norm = cs.k_norm; dp.norm_eps = cs.norm_eps;
    } else {
        dp.kf = (const _Float16 *)ctx->kf.p; dp.vtf = (const _Float16 *)ctx->vtf.p; dp.fcap = dc.fcap;
        dp.kf_lo = dc.kf_lo;
        dp.fresh_pos0 = dc.fresh_pos0; dp.fresh_row0 = dc.fresh_row0;
        dp.qs32 = (const float *)ctx->qs32.p; dp.qs_head_stride = dc.qs_head_stride;
    }
    dp.qscale = (float)(cs.scale * LOG2E_D);
    dp.out = cs.out; dp.Hq = cs.Hq; dp.Hkv = cs.Hkv; dp.G = G;
    dp.window = cs.window;
    dp.cap2 = cs.cap > 0.0f ? (float)(cs.cap * LOG2E_D) : 0.0f;
    dp.slot_floats = slot_floats;
    dp.err_flag = ctx->range_flag + SMOL_FLAG_MERGE;
    dp.spin_limit = ctx->opt[SMOL_OPT_DEC_SPIN] > 0 ? ctx->opt[SMOL_OPT_DEC_SPIN] : DEC_SPIN_LIMIT;
    dp.fault_merge = ctx->opt[SMOL_OPT_FAULT_MERGE] ? 1 : 0;
    int rc;
    if (gd) {
        /* the state's own slots; the epoch's high bits come from its step
         * counter, the low 8 bits tell this launch from the step's others */
        dp.part = gd->part;
        dp.epoch = (unsigned)cs.layer + 1;
        dp.step_dev = gd->step;
    } else if (dc.noalloc) {
        /* the per-device scratch: its flags hold earlier calls' epochs (or
         * zero), never this call's, which comes from the device's counter */
        ScratchDev &sd = g_scratch[ctx->device];
        if (!sd.ptr) return fail(SMOL_ATTN_ERR_DEVICE, "no decode scratch on device %d", ctx->device);
        dp.part = (float *)sd.ptr;
        unsigned e = sd.epoch.fetch_add(1) + 1;
        if (e == 0) e = sd.epoch.fetch_add(1) + 1;
        dp.epoch = e;
    } else {
        if ((rc = dev_reserve(ctx->dec_part, part_bytes, ctx->stream, true))) return rc;
        dp.part = (float *)ctx->dec_part.p;
        if (++ctx->epoch == 0) ctx->epoch = 1;
        dp.epoch = ctx->epoch;
    }
    dp.n_rb = n_rb;
    dp.n_items = (int)items.size();
    dp.n_seq = (int)dc.seqs.size();
    /* the items and sequences ride in the kernel arguments when they fit;
     * otherwise one upload of both */
    const bool items_arg = items.size() <= DEC_ARG_ITEMS, seqs_arg = dc.seqs.size() <= DEC_ARG_SEQS;
    if (items_arg) memcpy(dp.items, items.data(), items.size() * sizeof(DecItem));
    if (seqs_arg) memcpy(dp.seqs, dc.seqs.data(), dc.seqs.size() * sizeof(DecSeq));
    if (gd) dp.seqs_dev = gd->seqs;
    if (!items_arg || !seqs_arg) {
        const size_t o_seq = ((items_arg ? 0 : items.size() * sizeof(DecItem)) + 255) & ~(size_t)255;
        std::vector<unsigned char> host(o_seq + (seqs_arg ? 0 : dc.seqs.size() * sizeof(DecSeq)));
        if (!items_arg) memcpy(host.data(), items.data(), items.size() * sizeof(DecItem));
        if (!seqs_arg) memcpy(host.data() + o_seq, dc.seqs.data(), dc.seqs.size() * sizeof(DecSeq));
        if ((rc = upload_desc(ctx, host.data(), host.size()))) return rc;
        if (!items_arg) dp.items_dev = (const DecItem *)ctx->desc.p;
        if (!seqs_arg) dp.seqs_dev = (const DecSeq *)((unsigned char *)ctx->desc.p + o_seq);
    }
    const int mk = dc.noalloc || gd ? -1 : timing_begin(ctx, 1);
    hipEvent_t e0 = mk >= 0 ? ctx->marks[mk].a : nullptr, e1 = mk >= 0 ? ctx->marks[mk].b : nullptr;
    rc = smol_launch_decode(&dp, hd, rows, nw, ctx->stream, e0, e1);
    if (rc)
        return fail(rc == -1 ? SMOL_ATTN_ERR_UNSUPPORTED : SMOL_ATTN_ERR_DEVICE, "k_dec launch (hd %d, %d rows): %s", hd,
                    rows, rc == -1 ? "unsupported configuration" : hipGetErrorString(hipGetLastError()));
    return SMOL_ATTN_OK;
}

__global__ __launch_bounds__(64) void k_gdec_step(DecSeq *seqs, unsigned *step, int pos, int slot) {
    if (threadIdx.x == 0) {
        DecSeq q;
        q.pos = pos;
        q.slot = slot;
        q.tok0 = 0;
        q.n_q = 1;
        seqs[0] = q;
        *step = *step + 1;
    }
}

/* for qkn_attn.hip: the state of captured single-sequence decode launches
 * with n_heads query heads over n_kv_heads cache heads of head_dim hd,
 * planned at plan_pos (allocated and cleared here, before any capture) */
extern "C" int smol_internal_gdec_create(smol_attn_ctx *ctx, int n_heads, int n_kv_heads, int hd, int plan_pos,
                                         smol_graph_dec **out) {
    if (!ctx || !out || n_kv_heads <= 0 || n_heads % n_kv_heads || plan_pos < 0)
        return fail(SMOL_ATTN_ERR_ARG, "graph decode state: bad arguments");
    *out = nullptr;
    int rc = set_device(ctx);
    if (rc) return rc;
    const int rows = n_heads / n_kv_heads, TR = dec_tile_rows(hd, rows), n_rb = (rows + TR - 1) / TR;
    auto *g = new smol_graph_dec();
    g->device = ctx->device;
    g->plan_pos = plan_pos;
    g->part_bytes = (size_t)n_kv_heads * n_rb * DEC_MAX_SPLIT * dec_slot_floats(hd, TR) * 4;
    const size_t bytes = 256 + g->part_bytes;
    hipError_t e = hipMalloc(&g->mem, bytes);
    if (e == hipSuccess) e = hipMemsetAsync(g->mem, 0, bytes, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) {
        if (g->mem) hipFree(g->mem);
        delete g;
        return fail(SMOL_ATTN_ERR_NOMEM, "graph decode state: %s", hipGetErrorString(e));
    }
    g->seqs = static_cast<DecSeq *>(g->mem);
    g->step = reinterpret_cast<unsigned *>(static_cast<char *>(g->mem) + 64);
    g->part = reinterpret_cast<float *>(static_cast<char *>(g->mem) + 256);
    *out = g;
    return SMOL_ATTN_OK;
}

/* frees the state; the caller has drained every stream that replays it */
extern "C" void smol_internal_gdec_destroy(smol_graph_dec *g) {
    if (!g) return;
    hipSetDevice(g->device);
    if (g->mem) hipFree(g->mem);
    delete g;
}

/* g non-null: decode launches of this context are being captured with g's
 * state (and per-launch timing is off); null: capture ended */
extern "C" void smol_internal_gdec_capture(smol_attn_ctx *ctx, smol_graph_dec *g) {
    if (g && !ctx->gdec) {
        ctx->timing_saved = ctx->timing;
        ctx->timing = false;
    } else if (!g && ctx->gdec) {
        ctx->timing = ctx->timing_saved;
    }
    ctx->gdec = g;
}

/* before a replay: the captured launches decode position pos of cache slot
 * `slot` (enqueued on the context's stream) */
extern "C" int smol_internal_gdec_step(smol_attn_ctx *ctx, smol_graph_dec *g, int pos, int slot) {
    if (!g || pos < 0 || pos > g->plan_pos) return fail(SMOL_ATTN_ERR_ARG, "graph decode step: pos %d", pos);
    hipLaunchKernelGGL(k_gdec_step, dim3(1), dim3(64), 0, ctx->stream, g->seqs, g->step, pos, slot);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? SMOL_ATTN_OK : fail(SMOL_ATTN_ERR_DEVICE, "k_gdec_step: %s", hipGetErrorString(e));
}

static int run_plan(smol_attn_ctx *ctx, Plan &pl, const CallShape &cs) {
    const int hd = cs.hd, hdp = (hd + 31) & ~31;
    const int G = cs.Hq / cs.Hkv;
    int max_rows = 0;
    for (auto &b : pl.sb) max_rows = std::max(max_rows, b.n_rows);
    /* prefill kernel: k_attn_fb (one workgroup per 64-row tile, no merges
     * between workgroups) when every key is in the fresh buffers and the
     * call has enough tiles to occupy the device, else k_attn_fa (waves
     * split the rows, K/V shared through LDS, split-K across workgroups);
     * SMOL_OPT_PREFILL_KERNEL forces one where the keys allow it */
    const int pk = ctx->opt[SMOL_OPT_PREFILL_KERNEL];
    const bool precise = ctx->opt[SMOL_OPT_QK_FP16] != 1;
    const bool fa = !cs.dec;
    bool fb = fa && hd <= 128 && pk != 2;
    if (fb) {
        long long tiles = 0;
        for (auto &b : pl.sb) {
            if (b.key_lo < b.fresh_pos0) fb = false;
            tiles += (b.n_rows + 63) / 64;
        }
        if (pk != 1 && tiles * cs.Hkv < ctx->cu_count / 4) fb = false;
    }
    int nt = 1, w = 2, rows_per = 64;
    /* k_attn_fb with two key groups (64-row items, each group half of the
     * keys; the default) or one key group of eight waves (128-row items whose
     * key ranges may be split over workgroups and merged: each slab is staged
     * once for 128 rows and five stages fit with precise QK^T, but at C2's
     * shape the split items' start-up and merges cost more than that saves) */
    const bool fb_one = fb && ctx->opt[SMOL_OPT_FB_GROUPS] == 1 && ctx->opt[SMOL_OPT_FB_NT] != 2;
    if (fb_one) {
        nt = 0; /* the launcher's code for one key group */
        w = 2;
        rows_per = 128;
    } else if (fb) {
        /* 64-row tiles; SMOL_OPT_FB_NT 2: two row tiles per wave (four waves
         * per workgroup instead of eight) */
        nt = ctx->opt[SMOL_OPT_FB_NT] == 2 ? 2 : 1;
        w = 2;
        rows_per = 64;
    } else if (fa) {
        /* precise QK^T does not fit two row tiles into two waves per SIMD */
        nt = (hd <= 128 && max_rows > 64 && !precise) ? 2 : 1;
        w = hd > 128 ? 1 : 2;
        rows_per = 64 * nt;
    }
    /* k_attn_fb prepares its own Q rows from the inputs (head_dim 64 and
     * 128, precise QK^T, one row tile per wave, no per-head Q norm): k_prep
     * then writes no Q scratch, 4 bytes an element written and read back
     * less. (With the norm, the weights' loads and the row sums at each
     * item's start cost the attention kernel about what k_prep saves.)
     * SMOL_OPT_FB_QPREP 1: k_prep stages Q as for k_attn_fa. The item's
     * Q-scratch row q_row0 + r then names input token (q_row0 + r) / G and
     * head g * G + (q_row0 + r) % G, and its RoPE row is q_pos0 + r / G:
     * true of every plan with one pre-pass batch whose Q starts at input
     * token 0, with one attention batch when Q is rotated. */
    const bool q_in = fb && precise && (hd == 64 || hd == 128) && nt != 2 && !cs.q_norm &&
                      ctx->opt[SMOL_OPT_FB_QPREP] != 1 &&
                      pl.pb.size() == 1 && pl.pb[0].q_tok0 == 0 && pl.pb[0].q_row0 == 0 &&
                      (!(cs.rope && cs.rope_q) || (pl.sb.size() == 1 && pl.sb[0].q_pos0 == pl.pb[0].q_pos0));
    std::vector<std::vector<int>> fill_lists;
    if (fb_one) plan_fb_fill(pl, cs.Hkv, G, cs.window, ctx->cu_count, fill_lists);
    else if (fa) plan_items(pl, cs.Hkv, G, cs.window, rows_per, ctx->cu_count * w, true, fb);

    /* workspace; precise QK^T (the default) adds the lo parts of the fp16 Q
     * scratch and of the fresh K */
    int rc;
    const size_t fcap = (size_t)std::max(pl.fresh_rows, SMOL_SLAB);
    const size_t qs_elems = (size_t)cs.Hkv * std::max(pl.q_rows, 1) * hdp;
    if (cs.dec) {
        if ((rc = dev_reserve(ctx->qs32, qs_elems * 4, ctx->stream))) return rc;
    } else {
        if ((rc = dev_reserve(ctx->qs, qs_elems * 2 * (precise ? 2 : 1), ctx->stream))) return rc;
    }
    if ((rc = dev_reserve(ctx->kf, (size_t)cs.Hkv * fcap * hd * 2, ctx->stream))) return rc;
    if (precise && (rc = dev_reserve(ctx->kf_lo, (size_t)cs.Hkv * fcap * hd * 2, ctx->stream))) return rc;
    _Float16 *const qs_lo = precise && !cs.dec ? (_Float16 *)ctx->qs.p + qs_elems : nullptr;
    _Float16 *const kf_lo = precise ? (_Float16 *)ctx->kf_lo.p : nullptr;
    if ((rc = dev_reserve(ctx->vtf, (size_t)cs.Hkv * fcap * hd * 2, ctx->stream))) return rc;
    const size_t n_items = pl.items.size();
    if (fa) {
        if ((rc = dev_reserve(ctx->part_o, std::max<size_t>(1, n_items) * cs.Hkv * rows_per * hd * 4, ctx->stream))) return rc;
        if ((rc = dev_reserve(ctx->part_ml, std::max<size_t>(1, n_items) * cs.Hkv * rows_per * 2 * 4, ctx->stream))) return rc;
        /* one counter per 256-byte line: the workgroups of different groups count in
         * at about the same time, and atomics on one line are serialised */
        if ((rc = dev_reserve(ctx->counters, (size_t)std::max(1, pl.n_groups) * cs.Hkv * 4 * SK_COUNTER_STRIDE,
                              ctx->stream, true)))
            return rc;
    }

    /* k_attn_fb with more tiles than compute units: one workgroup per unit
     * and kv head runs a list of tiles, assigned longest first to the least
     * loaded list, instead of a second wave of workgroups that would each
     * start up again behind the first */
    std::vector<FbItem> fbi;
    int fb_wg = std::max(1, ctx->cu_count / cs.Hkv);
    if (!((int)n_items > fb_wg && ctx->opt[SMOL_OPT_FB_LISTS] != -1)) fb_wg = 0;
    if (fb_one && ctx->opt[SMOL_OPT_FB_LISTS] != -1) {
        /* one key group: the planner's filled lists, one workgroup each */
        fb_wg = (int)fill_lists.size();
        fbi = fb_items(pl, fb_wg, true, &fill_lists);
    } else if (fb) {
        fbi = fb_items(pl, fb_wg, fb_one);
    }

    /* descriptor tables in one upload: pre-pass blocks and items, each with
     * its batch */
    /* k_prep holds three workgroups a compute unit (registers of the normed
     * build, 33 KB of LDS each) */
    const std::vector<PrepBlockB> pbr = prep_records(pl, q_in, cs.Hkv, 3 * ctx->cu_count);
    std::vector<SkItemB> itr;
    if (fa && !fb) {
        itr.resize(pl.items.size());
        for (size_t i = 0; i < pl.items.size(); i++) itr[i] = {pl.items[i], pl.sb[pl.items[i].batch]};
    }
    auto al = [](size_t x) { return (x + 255) & ~(size_t)255; };
    const size_t o_pblk = 0;
    const size_t o_it = al(o_pblk + pbr.size() * sizeof(PrepBlockB));
    const size_t o_sc = al(o_it + itr.size() * sizeof(SkItemB));
    const size_t total = al(o_sc + fbi.size() * sizeof(FbItem));
    std::vector<unsigned char> host(total);
    memcpy(host.data() + o_pblk, pbr.data(), pbr.size() * sizeof(PrepBlockB));
    if (!itr.empty()) memcpy(host.data() + o_it, itr.data(), itr.size() * sizeof(SkItemB));
    if (!fbi.empty()) memcpy(host.data() + o_sc, fbi.data(), fbi.size() * sizeof(FbItem));
    if ((rc = upload_desc(ctx, host.data(), total))) return rc;
    unsigned char *dd = (unsigned char *)ctx->desc.p;

    const smol_kv_cache *kv = cs.kv;
    uint16_t *kc = nullptr, *vtc = nullptr;
    long long slot_stride = 0;
    int cap = 0;
    if (kv) {
        kc = kv->k + (size_t)cs.layer * kv_layer_elems(kv);
        vtc = kv->vt + (size_t)cs.layer * kv_layer_elems(kv);
        slot_stride = (long long)kv_slot_elems(kv);
        cap = kv->cap;
    }

    PrepParams pp;
    memset(&pp, 0, sizeof(pp));
    pp.q = cs.q; pp.q_dtype = cs.dtype; pp.q_stride = cs.q_stride;
    pp.k = cs.k; pp.v = cs.v; pp.kv_dtype = cs.dtype; pp.kv_stride = cs.kv_stride;
    if (cs.rope) {
        pp.rope_cos = cs.rope->cos_d;
        pp.rope_sin = cs.rope->sin_d;
        pp.rope_kind = cs.rope->type == SMOL_ROPE_INTERLEAVED ? SMOL_ROPE_INTERLEAVED_K : SMOL_ROPE_NEOX_K;
    } else {
        pp.rope_kind = SMOL_ROPE_OFF;
    }
    pp.rope_q = cs.rope_q;
    pp.rope_k = cs.rope_k;
    pp.qscale = (float)(cs.scale * LOG2E_D);
    pp.Hq = cs.Hq; pp.Hkv = cs.Hkv; pp.G = G; pp.hd = hd; pp.hdp = hdp;
    pp.qs = (_Float16 *)ctx->qs.p;
    pp.qs_head_stride = (long long)std::max(pl.q_rows, 1) * hdp;
    pp.kc = kc; pp.vtc = vtc; pp.c_slot_stride = slot_stride; pp.cap = cap;
    pp.kf = (_Float16 *)ctx->kf.p; pp.vtf = (_Float16 *)ctx->vtf.p; pp.fcap = (int)fcap;
    pp.qs_lo = qs_lo; pp.kf_lo = kf_lo;
    pp.stage = cs.dec ? SMOL_STAGE_QF32 : SMOL_STAGE_F16;
    if (cs.dec) pp.qs32 = (float *)ctx->qs32.p;
    pp.blocks = (const PrepBlockB *)(dd + o_pblk);
    pp.q_norm = cs.q_norm; pp.k_norm = cs.k_norm; pp.norm_eps = cs.norm_eps;
    pp.range_flag = ctx->range_flag;
    /* a call with no pre-pass blocks launches nothing here and records no
     * timing mark */
    int mk = pbr.empty() ? -1 : timing_begin(ctx, 0);
    rc = smol_launch_prep(&pp, (int)pbr.size(), ctx->stream, mark_a(ctx, mk), mark_b(ctx, mk));
    if (rc)
        return fail(rc == -1 ? SMOL_ATTN_ERR_UNSUPPORTED : SMOL_ATTN_ERR_DEVICE, "k_prep launch (hd %d): %s", hd,
                    rc == -1 ? "unsupported configuration" : hipGetErrorString(hipGetLastError()));

    if (cs.dec) {
        /* a short chunk: k_dec over the cache and the fresh staging, Q from the fp32 scratch */
        const SkBatch &b = pl.sb[0];
        DecCall dc;
        dc.direct = false;
        dc.seqs.push_back({b.q_pos0, b.slot, 0, b.n_rows / G});
        dc.fresh_pos0 = b.fresh_pos0;
        dc.fresh_row0 = b.fresh_row0;
        dc.fcap = (int)fcap;
        dc.kf_lo = kf_lo;
        dc.qs_head_stride = pp.qs_head_stride;
        return run_decode(ctx, cs, dc);
    }

    SkParams sp;
    memset(&sp, 0, sizeof(sp));
    sp.qs = (const _Float16 *)ctx->qs.p;
    sp.qs_head_stride = pp.qs_head_stride;
    sp.kc = kc; sp.vtc = vtc; sp.c_slot_stride = slot_stride; sp.cap = cap;
    sp.kf = (const _Float16 *)ctx->kf.p; sp.vtf = (const _Float16 *)ctx->vtf.p; sp.fcap = (int)fcap;
    sp.qs_lo = qs_lo; sp.kf_lo = kf_lo;
    sp.out = cs.out;
    sp.Hq = cs.Hq; sp.Hkv = cs.Hkv; sp.G = G;
    sp.window = cs.window;
    sp.cap2 = cs.cap > 0.0f ? (float)(cs.cap * LOG2E_D) : 0.0f;
    sp.range_flag = ctx->range_flag;
    sp.items = (const SkItemB *)(dd + o_it);
    sp.part_o = (float *)ctx->part_o.p;
    sp.part_ml = (float *)ctx->part_ml.p;
    sp.counters = (int *)ctx->counters.p;
    if (fb) {
        sp.fb_items = (const FbItem *)(dd + o_sc);
        sp.n_wg = fb_wg;
    }
    if (q_in) {
        sp.q_in = cs.q; sp.q_dtype = cs.dtype; sp.q_stride = cs.q_stride;
        sp.rope_cos = pp.rope_cos; sp.rope_sin = pp.rope_sin;
        sp.q_rope_kind = pp.rope_q ? pp.rope_kind : SMOL_ROPE_OFF;
        sp.qscale = pp.qscale;
    }
    mk = timing_begin(ctx, 1);
    rc = fb ? smol_launch_fb(&sp, hd, (int)n_items, nt, ctx->stream, mark_a(ctx, mk), mark_b(ctx, mk))
            : smol_launch_fa(&sp, hd, (int)n_items, nt, w, ctx->stream, mark_a(ctx, mk), mark_b(ctx, mk));
    if (rc)
        return fail(rc == -1 ? SMOL_ATTN_ERR_UNSUPPORTED : SMOL_ATTN_ERR_DEVICE,
                    "attention launch (hd %d): %s", hd, hipGetErrorString(hipGetLastError()));
    return SMOL_ATTN_OK;
}

static void add_q_blocks(Plan &pl, int batch, int n_q) {
    const int per = 32; /* tokens per pre-pass block */
    for (int t = 0; t < n_q; t += per) pl.pblk.push_back({batch, 1, t, std::min(per, n_q - t)});
}

static void add_fresh_blocks(Plan &pl, int batch, int n_fresh) {
    for (int s = 0; s < n_fresh / SMOL_SLAB; s++) pl.pblk.push_back({batch, 0, s, 0});
}

static int check_common(smol_attn_ctx *ctx, int dtype, int Hq, int Hkv, int hd, const void *q,
                        float *out) {
    if (!ctx) return fail(SMOL_ATTN_ERR_ARG, "ctx is NULL");
    if (dtype != SMOL_ATTN_F32 && dtype != SMOL_ATTN_BF16) return fail(SMOL_ATTN_ERR_ARG, "dtype %d", dtype);
    if (Hq <= 0 || Hkv <= 0 || Hq % Hkv != 0)
        return fail(SMOL_ATTN_ERR_ARG, "n_heads %d not a multiple of n_kv_heads %d", Hq, Hkv);
    if (!hd_supported(hd)) return fail(SMOL_ATTN_ERR_UNSUPPORTED, "head_dim %d", hd);
    if (!q || !out) return fail(SMOL_ATTN_ERR_ARG, "NULL tensor");
    if (((uintptr_t)q | (uintptr_t)out) & 15) return fail(SMOL_ATTN_ERR_ARG, "q/out must be 16-byte aligned");
    return set_device(ctx);
}

static int check_aligned(const void *a, const void *b) {
    if (((uintptr_t)a | (uintptr_t)b) & 15) return fail(SMOL_ATTN_ERR_ARG, "k/v must be 16-byte aligned");
    return 0;
}

static int check_rope(smol_attn_ctx *ctx, const smol_rope_table *rope, int hd, int need) {
    if (!rope) return 0;
    /* a table grows on its own context's stream and frees the old arrays once
     * that stream is idle: kernels of another context could still read them */
    if (rope->ctx != ctx) return fail(SMOL_ATTN_ERR_ARG, "rope table belongs to another context");
    if (rope->hd != hd) return fail(SMOL_ATTN_ERR_ARG, "rope table head_dim %d != %d", rope->hd, hd);
    return smol_rope_table_ensure(const_cast<smol_rope_table *>(rope), need);
}

/* per-head RMSNorm weights: device fp32 [hd], 4-byte aligned; a Q block of
 * the pre-pass keeps 1/rms of its 32 tokens x G heads in LDS */
static int check_norm(const float *q_norm, const float *k_norm, float eps, int G) {
    if (((uintptr_t)q_norm | (uintptr_t)k_norm) & 3) return fail(SMOL_ATTN_ERR_ARG, "norm weights must be 4-byte aligned");
    if ((q_norm || k_norm) && !(eps >= 0.0f)) return fail(SMOL_ATTN_ERR_ARG, "norm eps %g", (double)eps);
    if (q_norm && G > 256) return fail(SMOL_ATTN_ERR_UNSUPPORTED, "q norm with %d query heads per KV head", G);
    return 0;
}

extern "C" int smol_attn_prefill(smol_attn_ctx *ctx, smol_kv_cache *kv, int layer, int slot,
                                 const smol_rope_table *rope, int pos0, int seq_q, const void *q,
                                 const void *k_new, const void *v_new, int dtype, int n_heads,
                                 float scale, int window, float cap, float *out) {
    return smol_attn_prefill_qknorm(ctx, kv, layer, slot, rope, pos0, seq_q, q, k_new, v_new, dtype, n_heads, scale,
                                    window, cap, nullptr, nullptr, 0.0f, out);
}

extern "C" int smol_attn_prefill_qknorm(smol_attn_ctx *ctx, smol_kv_cache *kv, int layer, int slot,
                                        const smol_rope_table *rope, int pos0, int seq_q, const void *q,
                                        const void *k_new, const void *v_new, int dtype, int n_heads,
                                        float scale, int window, float cap, const float *q_norm,
                                        const float *k_norm, float eps, float *out) {
    if (!kv) return fail(SMOL_ATTN_ERR_ARG, "cache is NULL");
    int rc = check_common(ctx, dtype, n_heads, kv->n_kv, kv->hd, q, out);
    if (rc) return rc;
    if ((rc = check_norm(q_norm, k_norm, eps, n_heads / kv->n_kv))) return rc;
    if (kv->ctx != ctx) return fail(SMOL_ATTN_ERR_ARG, "cache belongs to another context");
    if (layer < 0 || layer >= kv->n_layers || slot < 0 || slot >= kv->n_slots)
        return fail(SMOL_ATTN_ERR_ARG, "layer %d / slot %d out of range", layer, slot);
    if (pos0 < 0 || seq_q <= 0 || !k_new || !v_new) return fail(SMOL_ATTN_ERR_ARG, "pos0 %d seq_q %d", pos0, seq_q);
    if ((rc = check_aligned(k_new, v_new))) return rc;
    if ((rc = smol_kv_cache_reserve(kv, pos0 + seq_q))) return rc;
    if ((rc = check_rope(ctx, rope, kv->hd, pos0 + seq_q))) return rc;
    const int Hkv = kv->n_kv, G = n_heads / Hkv, hd = kv->hd;
    Plan pl;
    const int f0 = pos0 & ~(SMOL_SLAB - 1);
    const int nf = ((pos0 + seq_q + SMOL_SLAB - 1) & ~(SMOL_SLAB - 1)) - f0;
    pl.pb.push_back({0, seq_q, 0, pos0, 0, seq_q, pos0, f0, nf, 0, slot, 0});
    add_q_blocks(pl, 0, seq_q); /* the Q blocks (the longer ones) dispatched first */
    add_fresh_blocks(pl, 0, nf);
    pl.sb.push_back({seq_q * G, 0, 0, pos0, 0, pos0 + seq_q, 1, f0, 0, slot, 0, 0});
    pl.q_rows = seq_q * G;
    pl.fresh_rows = nf;
    /* short chunks stream the cache like a decode step; long ones are MFMA-bound */
    const bool dec = seq_q * G <= 64;
    CallShape cs{dec, q, k_new, v_new, dtype, n_heads, Hkv, hd, (long long)n_heads * hd,
                 (long long)Hkv * hd, scale, cap, window, rope, 1, 1, kv, layer, out, q_norm, k_norm, eps};
    return run_plan(ctx, pl, cs);
}

extern "C" int smol_attn_decode(smol_attn_ctx *ctx, smol_kv_cache *kv, int layer,
                                const smol_rope_table *rope, int n_seq, const int *slots,
                                const int *pos, const void *q, const void *k_new, const void *v_new,
                                int dtype, int n_heads, float scale, int window, float cap,
                                float *out) {
    return smol_attn_decode_qknorm(ctx, kv, layer, rope, n_seq, slots, pos, q, k_new, v_new, dtype, n_heads, scale,
                                   window, cap, nullptr, nullptr, 0.0f, out);
}

extern "C" int smol_attn_decode_qknorm(smol_attn_ctx *ctx, smol_kv_cache *kv, int layer,
                                       const smol_rope_table *rope, int n_seq, const int *slots,
                                       const int *pos, const void *q, const void *k_new,
                                       const void *v_new, int dtype, int n_heads, float scale,
                                       int window, float cap, const float *q_norm,
                                       const float *k_norm, float eps, float *out) {
    if (!kv) return fail(SMOL_ATTN_ERR_ARG, "cache is NULL");
    int rc = check_common(ctx, dtype, n_heads, kv->n_kv, kv->hd, q, out);
    if (rc) return rc;
    if ((rc = check_norm(q_norm, k_norm, eps, n_heads / kv->n_kv))) return rc;
    if (kv->ctx != ctx) return fail(SMOL_ATTN_ERR_ARG, "cache belongs to another context");
    if (layer < 0 || layer >= kv->n_layers) return fail(SMOL_ATTN_ERR_ARG, "layer %d out of range", layer);
    if (n_seq <= 0 || !slots || !pos || !k_new || !v_new) return fail(SMOL_ATTN_ERR_ARG, "bad decode batch");
    if ((rc = check_aligned(k_new, v_new))) return rc;
    int max_pos = 0;
    std::vector<char> seen(kv->n_slots, 0);
    for (int i = 0; i < n_seq; i++) {
        if (slots[i] < 0 || slots[i] >= kv->n_slots) return fail(SMOL_ATTN_ERR_ARG, "slot %d out of range", slots[i]);
        if (seen[slots[i]]) return fail(SMOL_ATTN_ERR_ARG, "slot %d appears twice", slots[i]);
        seen[slots[i]] = 1;
        if (pos[i] < 0) return fail(SMOL_ATTN_ERR_ARG, "pos %d", pos[i]);
        max_pos = std::max(max_pos, pos[i]);
    }
    if ((rc = smol_kv_cache_reserve(kv, max_pos + 1))) return rc;
    if ((rc = check_rope(ctx, rope, kv->hd, max_pos + 1))) return rc;
    const int Hkv = kv->n_kv, hd = kv->hd;
    /* one launch: k_dec normalises and rotates Q and the new key itself,
     * scores the new key in fp32 and appends it to the cache */
    DecCall dc;
    dc.direct = true;
    for (int i = 0; i < n_seq; i++) dc.seqs.push_back({pos[i], slots[i], i, 1});
    CallShape cs{true, q, k_new, v_new, dtype, n_heads, Hkv, hd, (long long)n_heads * hd,
                 (long long)Hkv * hd, scale, cap, window, rope, 1, 1, kv, layer, out, q_norm, k_norm, eps, true};
    return run_decode(ctx, cs, dc);
}

extern "C" int smol_attn_decode_noalloc(smol_attn_ctx *ctx, smol_kv_cache *kv, int layer,
                                        const smol_rope_table *rope, int n_seq, const int *slots,
                                        const int *pos, const void *q, const void *k_new,
                                        const void *v_new, int dtype, int n_heads, float scale,
                                        int window, float cap, const float *q_norm,
                                        const float *k_norm, float eps, float *out) {
    if (!kv) return fail(SMOL_ATTN_ERR_ARG, "cache is NULL");
    int rc = check_common(ctx, dtype, n_heads, kv->n_kv, kv->hd, q, out);
    if (rc) return rc;
    if ((rc = check_norm(q_norm, k_norm, eps, n_heads / kv->n_kv))) return rc;
    if (kv->ctx != ctx) return fail(SMOL_ATTN_ERR_ARG, "cache belongs to another context");
    if (layer < 0 || layer >= kv->n_layers) return fail(SMOL_ATTN_ERR_ARG, "layer %d out of range", layer);
    if (n_seq <= 0 || !slots || !pos || !k_new || !v_new) return fail(SMOL_ATTN_ERR_ARG, "bad decode batch");
    if (n_seq > DEC_ARG_SEQS)
        return fail(SMOL_ATTN_ERR_UNSUPPORTED, "%d sequences: the no-alloc decode takes at most %d", n_seq,
                    DEC_ARG_SEQS);
    if ((rc = check_aligned(k_new, v_new))) return rc;
    if (rope && rope->ctx != ctx) return fail(SMOL_ATTN_ERR_ARG, "rope table belongs to another context");
    if (rope && rope->hd != kv->hd) return fail(SMOL_ATTN_ERR_ARG, "rope table head_dim %d != %d", rope->hd, kv->hd);
    DecCall dc;
    dc.direct = true;
    dc.noalloc = true;
    for (int i = 0; i < n_seq; i++) {
        if (slots[i] < 0 || slots[i] >= kv->n_slots) return fail(SMOL_ATTN_ERR_ARG, "slot %d out of range", slots[i]);
        for (int j = 0; j < i; j++)
            if (slots[j] == slots[i]) return fail(SMOL_ATTN_ERR_ARG, "slot %d appears twice", slots[i]);
        /* no growth here: the cache and the table must already hold the position */
        if (pos[i] < 0 || pos[i] >= kv->cap)
            return fail(SMOL_ATTN_ERR_ARG, "pos %d outside the cache's %d rows (reserve them first)", pos[i], kv->cap);
        if (rope && pos[i] >= rope->cap)
            return fail(SMOL_ATTN_ERR_ARG, "pos %d outside the rope table's %d rows (ensure them first)", pos[i],
                        rope->cap);
        dc.seqs.push_back({pos[i], slots[i], i, 1});
    }
    const int Hkv = kv->n_kv, hd = kv->hd;
    CallShape cs{true, q, k_new, v_new, dtype, n_heads, Hkv, hd, (long long)n_heads * hd,
                 (long long)Hkv * hd, scale, cap, window, rope, 1, 1, kv, layer, out, q_norm, k_norm, eps, true};
    return run_decode(ctx, cs, dc);
}

extern "C" int smol_attn_causal(smol_attn_ctx *ctx, const void *q, const void *k, const void *v,
                                int dtype, int seq_q, int seq_k, int n_heads, int n_kv_heads,
                                int hd, float scale, int q_offset, int window, float cap, float *out) {
    int rc = check_common(ctx, dtype, n_heads, n_kv_heads, hd, q, out);
    if (rc) return rc;
    if (seq_q <= 0 || seq_k < 0) return fail(SMOL_ATTN_ERR_ARG, "seq_q %d seq_k %d", seq_q, seq_k);
    if (seq_k > 0 && (!k || !v)) return fail(SMOL_ATTN_ERR_ARG, "NULL K/V");
    if ((rc = check_aligned(k, v))) return rc;
    const int G = n_heads / n_kv_heads;
    Plan pl;
    const int nf = (seq_k + SMOL_SLAB - 1) & ~(SMOL_SLAB - 1);
    pl.pb.push_back({0, seq_q, 0, 0, 0, seq_k, 0, 0, nf, 0, -1, 0});
    add_q_blocks(pl, 0, seq_q); /* the Q blocks (the longer ones) dispatched first */
    add_fresh_blocks(pl, 0, nf);
    pl.sb.push_back({seq_q * G, 0, 0, q_offset, 0, seq_k, 1, 0, 0, -1, 0, 0});
    pl.q_rows = seq_q * G;
    pl.fresh_rows = nf;
    CallShape cs{false, q, k, v, dtype, n_heads, n_kv_heads, hd, (long long)n_heads * hd,
                 (long long)n_kv_heads * hd, scale, cap, window, nullptr, 0, 0, nullptr, 0, out};
    return run_plan(ctx, pl, cs);
}

extern "C" int smol_attn_causal_bf16(smol_attn_ctx *ctx, const uint16_t *q, const uint16_t *k, const uint16_t *v,
                                     int seq_q, int seq_k, int n_heads, int n_kv_heads, int hd, float scale,
                                     int q_offset, int window, float cap, uint16_t *out) {
    if (!ctx) return fail(SMOL_ATTN_ERR_ARG, "ctx is NULL");
    if (!out || ((uintptr_t)out & 15)) return fail(SMOL_ATTN_ERR_ARG, "out must be a 16-byte aligned array");
    if (seq_q <= 0 || n_heads <= 0 || hd <= 0) return fail(SMOL_ATTN_ERR_ARG, "seq_q %d", seq_q);
    int rc = set_device(ctx);
    if (rc) return rc;
    const long long n = (long long)seq_q * n_heads * hd;
    if ((rc = dev_reserve(ctx->out32, (size_t)n * 4, ctx->stream))) return rc;
    if ((rc = smol_attn_causal(ctx, q, k, v, SMOL_ATTN_BF16, seq_q, seq_k, n_heads, n_kv_heads, hd, scale, q_offset,
                               window, cap, (float *)ctx->out32.p)))
        return rc;
    if (smol_launch_to_bf16_trunc((const float *)ctx->out32.p, out, n, ctx->stream))
        return fail(SMOL_ATTN_ERR_DEVICE, "bf16 output: %s", hipGetErrorString(hipGetLastError()));
    return SMOL_ATTN_OK;
}

extern "C" int smol_attn_bidirectional(smol_attn_ctx *ctx, const void *q, const void *k,
                                       const void *v, int dtype, int seq, int n_heads, int hd,
                                       float scale, const int *ws, int n_windows, float *out) {
    int rc = check_common(ctx, dtype, n_heads, n_heads, hd, q, out);
    if (rc) return rc;
    if (!ws || n_windows <= 0 || !k || !v) return fail(SMOL_ATTN_ERR_ARG, "bad windows");
    if ((rc = check_aligned(k, v))) return rc;
    for (int w = 0; w < n_windows; w++)
        if (ws[w] < 0 || ws[w + 1] < ws[w] || ws[w + 1] > seq)
            return fail(SMOL_ATTN_ERR_ARG, "window %d = [%d, %d) outside [0, %d)", w, ws[w], ws[w + 1], seq);
    /* k_attn_win reads the inputs directly (no pre-pass, no staging in
     * HBM, one launch); each tile stages its whole window, and it still
     * beats the pre-pass and k_attn_fb wherever the window fits in LDS
     * (audio encoder, 104 keys: 9.2 us against 14 us; SigLIP, 256 keys:
     * 14.3 us against 15.7 us per call) */
    {
        int max_len = 0;
        long long n_tiles = 0;
        for (int w = 0; w < n_windows; w++) {
            max_len = std::max(max_len, ws[w + 1] - ws[w]);
            n_tiles += (ws[w + 1] - ws[w] + 63) / 64;
        }
        const bool precise = ctx->opt[SMOL_OPT_QK_FP16] != 1;
        const int wmax = smol_win_max_keys(hd, dtype == SMOL_ATTN_BF16 ? SMOL_IN_BF16 : SMOL_IN_F32, precise ? 1 : 0);
        const int opt = ctx->opt[SMOL_OPT_BIDIR_WIN];
        if (opt >= 0 && wmax > 0 && max_len <= wmax && n_windows <= WIN_ARG_WINDOWS &&
            (long long)n_windows * n_heads * ((max_len + 63) / 64) + 8LL * ((max_len + 63) / 64) <= 0x7FFFFFFF) {
            if ((rc = set_device(ctx))) return rc;
            if (n_tiles == 0) return SMOL_ATTN_OK;
            WinParams &wp = ctx->wp;
            memset(&wp, 0, sizeof(wp));
            wp.q = q; wp.k = k; wp.v = v;
            wp.in_dtype = dtype == SMOL_ATTN_BF16 ? SMOL_IN_BF16 : SMOL_IN_F32;
            wp.row_stride = (long long)n_heads * hd;
            wp.out = out;
            wp.qscale = (float)(scale * LOG2E_D);
            wp.H = n_heads;
            wp.n_windows = n_windows;
            /* 128-row tiles, or 64-row tiles over two key groups when the
             * 128-row tiles would leave compute units idle */
            const long long units = (long long)n_windows * n_heads;
            const int ko = ctx->opt[SMOL_OPT_WIN_KSPLIT];
            wp.ksplit = ko == 1 || ko == 2 ? ko
                        : max_len > SMOL_SLAB && units * ((max_len + WIN_ROWS - 1) / WIN_ROWS) < ctx->cu_count ? 2 : 1;
            const int rows = WIN_ROWS / wp.ksplit;
            wp.tpu = (max_len + rows - 1) / rows;
            wp.n_xcc = std::max(1, ctx->n_xcc);
            wp.range_flag = ctx->range_flag;
            wp.precise = precise ? 1 : 0;
            memcpy(wp.ws, ws, (size_t)(n_windows + 1) * sizeof(int));
            const int mk = timing_begin(ctx, 1);
            rc = smol_launch_win(&wp, hd, (int)n_tiles, max_len, ctx->stream, mark_a(ctx, mk), mark_b(ctx, mk));
            if (rc) return fail(SMOL_ATTN_ERR_DEVICE, "k_attn_win launch: %s", hipGetErrorString(hipGetLastError()));
            return SMOL_ATTN_OK;
        }
    }
    Plan pl;
    const int nf = (seq + SMOL_SLAB - 1) & ~(SMOL_SLAB - 1);
    pl.pb.push_back({0, seq, 0, 0, 0, seq, 0, 0, nf, 0, -1, 0});
    add_q_blocks(pl, 0, seq); /* the Q blocks (the longer ones) dispatched first */
    add_fresh_blocks(pl, 0, nf);
    for (int w = 0; w < n_windows; w++) {
        const int a = ws[w], b = ws[w + 1];
        if (b <= a) continue;
        pl.sb.push_back({b - a, a, a, 0, a, b, 0, 0, 0, -1, 0, 0});
    }
    pl.q_rows = seq;
    pl.fresh_rows = nf;
    CallShape cs{false, q, k, v, dtype, n_heads, n_heads, hd, (long long)n_heads * hd,
                 (long long)n_heads * hd, scale, 0.0f, 0, nullptr, 0, 0, nullptr, 0, out};
    return run_plan(ctx, pl, cs);
}

extern "C" int smol_kv_cache_write(smol_kv_cache *kv, int layer, int slot, int pos0, int n,
                                   const void *k, const void *v, int dtype, int on_device) {
    if (!kv || !k || !v) return fail(SMOL_ATTN_ERR_ARG, "NULL argument");
    smol_attn_ctx *ctx = kv->ctx;
    if (layer < 0 || layer >= kv->n_layers || slot < 0 || slot >= kv->n_slots || pos0 < 0 || n <= 0)
        return fail(SMOL_ATTN_ERR_ARG, "layer %d slot %d pos0 %d n %d", layer, slot, pos0, n);
    if (dtype != SMOL_ATTN_F32 && dtype != SMOL_ATTN_BF16) return fail(SMOL_ATTN_ERR_ARG, "dtype %d", dtype);
    int rc = set_device(ctx);
    if (rc) return rc;
    if ((rc = smol_kv_cache_reserve(kv, pos0 + n))) return rc;
    const size_t row_bytes = (size_t)kv->n_kv * kv->hd * (dtype == SMOL_ATTN_BF16 ? 2 : 4);
    void *kd = (void *)k, *vd = (void *)v;
    if (!on_device) {
        HIP_TRY(hipMalloc(&kd, row_bytes * n));
        HIP_TRY(hipMalloc(&vd, row_bytes * n));
        HIP_TRY(hipMemcpy(kd, k, row_bytes * n, hipMemcpyHostToDevice));
        HIP_TRY(hipMemcpy(vd, v, row_bytes * n, hipMemcpyHostToDevice));
    }
    Plan pl;
    const int f0 = pos0 & ~(SMOL_SLAB - 1);
    const int nf = ((pos0 + n + SMOL_SLAB - 1) & ~(SMOL_SLAB - 1)) - f0;
    pl.pb.push_back({0, 0, 0, 0, 0, n, pos0, f0, nf, 0, slot, 0});
    add_fresh_blocks(pl, 0, nf);
    pl.fresh_rows = nf;
    const int hd = kv->hd;
    const size_t fcap = (size_t)nf;
    if ((rc = dev_reserve(ctx->kf, (size_t)kv->n_kv * fcap * hd * 2, ctx->stream))) return rc;
    if ((rc = dev_reserve(ctx->vtf, (size_t)kv->n_kv * fcap * hd * 2, ctx->stream))) return rc;
    const std::vector<PrepBlockB> pbr = prep_records(pl, false, kv->n_kv, 3 * ctx->cu_count);
    if ((rc = upload_desc(ctx, pbr.data(), pbr.size() * sizeof(PrepBlockB)))) return rc;
    PrepParams pp;
    memset(&pp, 0, sizeof(pp));
    pp.k = kd; pp.v = vd; pp.kv_dtype = dtype; pp.kv_stride = (long long)kv->n_kv * hd;
    pp.q_dtype = dtype; /* no Q blocks; the pre-pass is built per input type */
    pp.rope_kind = SMOL_ROPE_OFF;
    pp.Hq = kv->n_kv; pp.Hkv = kv->n_kv; pp.G = 1; pp.hd = hd; pp.hdp = (hd + 31) & ~31;
    pp.kc = kv->k + (size_t)layer * kv_layer_elems(kv);
    pp.vtc = kv->vt + (size_t)layer * kv_layer_elems(kv);
    pp.c_slot_stride = (long long)kv_slot_elems(kv);
    pp.cap = kv->cap;
    pp.kf = (_Float16 *)ctx->kf.p; pp.vtf = (_Float16 *)ctx->vtf.p; pp.fcap = (int)fcap;
    pp.blocks = (const PrepBlockB *)ctx->desc.p;
    rc = smol_launch_prep(&pp, (int)pbr.size(), ctx->stream, nullptr, nullptr);
    if (!on_device) {
        hipStreamSynchronize(ctx->stream);
        hipFree(kd);
        hipFree(vd);
    }
    if (rc) return fail(SMOL_ATTN_ERR_DEVICE, "cache write: %s", hipGetErrorString(hipGetLastError()));
    return SMOL_ATTN_OK;
}

extern "C" int smol_kv_cache_read(smol_kv_cache *kv, int layer, int slot, int pos0, int n,
                                  uint16_t *k_out, uint16_t *v_out) {
    if (!kv || !k_out || !v_out) return fail(SMOL_ATTN_ERR_ARG, "NULL argument");
    if (layer < 0 || layer >= kv->n_layers || slot < 0 || slot >= kv->n_slots || pos0 < 0 || n <= 0 ||
        pos0 + n > kv->cap)
        return fail(SMOL_ATTN_ERR_ARG, "layer %d slot %d rows [%d, %d) cap %d", layer, slot, pos0, pos0 + n, kv->cap);
    int rc = set_device(kv->ctx);
    if (rc) return rc;
    HIP_TRY(hipStreamSynchronize(kv->ctx->stream));
    const int hd = kv->hd, H = kv->n_kv;
    const int b0 = pos0 / SMOL_SLAB, b1 = (pos0 + n + SMOL_SLAB - 1) / SMOL_SLAB;
    std::vector<uint16_t> kt((size_t)n * hd), vt((size_t)(b1 - b0) * SMOL_SLAB * hd);
    for (int g = 0; g < H; g++) {
        const size_t base = (size_t)layer * kv_layer_elems(kv) + (size_t)slot * kv_slot_elems(kv) + (size_t)g * kv->cap * hd;
        HIP_TRY(hipMemcpy(kt.data(), kv->k + base + (size_t)pos0 * hd, kt.size() * 2, hipMemcpyDeviceToHost));
        HIP_TRY(hipMemcpy(vt.data(), kv->vt + base + (size_t)b0 * SMOL_SLAB * hd, vt.size() * 2, hipMemcpyDeviceToHost));
        for (int r = 0; r < n; r++) {
            const int pos = pos0 + r;
            const size_t vb = (size_t)(pos / SMOL_SLAB - b0) * SMOL_SLAB * hd + pos % SMOL_SLAB;
            for (int d = 0; d < hd; d++) {
                k_out[((size_t)r * H + g) * hd + d] = kt[(size_t)r * hd + d];
                v_out[((size_t)r * H + g) * hd + d] = vt[vb + (size_t)d * SMOL_SLAB];
            }
        }
    }
    return SMOL_ATTN_OK;
}

extern "C" int smol_attn_apply_rope(smol_attn_ctx *ctx, const smol_rope_table *rope, float *x,
                                    const int *positions, int seq, int n_heads) {
    if (!rope) return fail(SMOL_ATTN_ERR_ARG, "rope table is NULL");
    return smol_attn_norm_rope(ctx, rope, x, nullptr, 0.0f, positions, seq, n_heads, rope->hd);
}

extern "C" int smol_attn_norm_rope(smol_attn_ctx *ctx, const smol_rope_table *rope, float *x, const float *weight,
                                   float eps, const int *positions, int seq, int n_heads, int head_dim) {
    if (!ctx || !x || seq <= 0 || n_heads <= 0 || head_dim <= 0 || (head_dim & 1))
        return fail(SMOL_ATTN_ERR_ARG, "bad arguments");
    if (rope && (!positions || rope->hd != head_dim))
        return fail(SMOL_ATTN_ERR_ARG, "rope needs positions and head_dim %d", rope ? rope->hd : 0);
    if (rope && rope->ctx != ctx) return fail(SMOL_ATTN_ERR_ARG, "rope table belongs to another context");
    if (weight && !(eps >= 0.0f)) return fail(SMOL_ATTN_ERR_ARG, "norm eps %g", (double)eps);
    if (((uintptr_t)x | (uintptr_t)weight) & 3) return fail(SMOL_ATTN_ERR_ARG, "x / weight must be 4-byte aligned");
    int rc = set_device(ctx);
    if (rc) return rc;
    if (!rope && !weight) return SMOL_ATTN_OK;
    const int *pos_d = nullptr;
    if (rope) {
        int mx = 0;
        for (int s = 0; s < seq; s++) {
            if (positions[s] < 0) return fail(SMOL_ATTN_ERR_ARG, "position %d", positions[s]);
            mx = std::max(mx, positions[s]);
        }
        if ((rc = smol_rope_table_ensure(const_cast<smol_rope_table *>(rope), mx + 1))) return rc;
        if ((rc = upload_desc(ctx, positions, (size_t)seq * sizeof(int)))) return rc;
        pos_d = (const int *)ctx->desc.p;
    }
    const int kind = !rope ? SMOL_ROPE_OFF
                     : rope->type == SMOL_ROPE_INTERLEAVED ? SMOL_ROPE_INTERLEAVED_K : SMOL_ROPE_NEOX_K;
    if (smol_launch_norm_rope(x, weight, eps, rope ? rope->cos_d : nullptr, rope ? rope->sin_d : nullptr, pos_d, seq,
                              n_heads, head_dim, kind, ctx->stream))
        return fail(SMOL_ATTN_ERR_DEVICE, "norm/rope launch: %s", hipGetErrorString(hipGetLastError()));
    return SMOL_ATTN_OK;
}

/* the Q rows (q, q_weight, n_heads) and, when k is not NULL, the K rows (k,
 * k_weight, n_kv_heads) of one call in one launch */
static int norm_rope_bf16(smol_attn_ctx *ctx, const smol_rope_table *rope, uint16_t *x, const float *weight,
                          uint16_t *k, const float *k_weight, int n_kv_heads, float eps, int pos0, int seq,
                          int n_heads, int head_dim) {
    if (!ctx || !x || seq <= 0 || n_heads <= 0 || head_dim <= 0 || (head_dim & 7) || pos0 < 0 ||
        (k && n_kv_heads <= 0))
        return fail(SMOL_ATTN_ERR_ARG, "bad arguments (head_dim must be a multiple of 8)");
    if (rope && (rope->hd != head_dim || rope->type != SMOL_ROPE_INTERLEAVED))
        return fail(SMOL_ATTN_ERR_ARG, "the bf16 rotation needs an interleaved table of head_dim %d", head_dim);
    if (rope && rope->ctx != ctx) return fail(SMOL_ATTN_ERR_ARG, "rope table belongs to another context");
    if ((weight || k_weight) && !(eps >= 0.0f)) return fail(SMOL_ATTN_ERR_ARG, "norm eps %g", (double)eps);
    if (((uintptr_t)x & 15) || ((uintptr_t)weight & 3) || ((uintptr_t)k & 15) || ((uintptr_t)k_weight & 3))
        return fail(SMOL_ATTN_ERR_ARG, "x must be 16-byte and weight 4-byte aligned");
    int rc = set_device(ctx);
    if (rc) return rc;
    if (!rope && !weight && !k_weight) return SMOL_ATTN_OK;
    if (rope && (rc = smol_rope_table_ensure(const_cast<smol_rope_table *>(rope), pos0 + seq))) return rc;
    if (smol_launch_bf16_norm_rope(x, weight, k, k_weight, n_kv_heads, eps, rope ? rope->cos_d : nullptr,
                                   rope ? rope->sin_d : nullptr, pos0, seq, n_heads, head_dim, ctx->stream))
        return fail(SMOL_ATTN_ERR_DEVICE, "bf16 norm/rope launch: %s", hipGetErrorString(hipGetLastError()));
    return SMOL_ATTN_OK;
}

extern "C" int smol_attn_norm_rope_bf16(smol_attn_ctx *ctx, const smol_rope_table *rope, uint16_t *x,
                                        const float *weight, float eps, int pos0, int seq, int n_heads,
                                        int head_dim) {
    return norm_rope_bf16(ctx, rope, x, weight, nullptr, nullptr, 0, eps, pos0, seq, n_heads, head_dim);
}

/* for qkn_attn.hip: smol_attn_norm_rope_bf16 of a call's Q and K rows (each
 * with its own norm weight) as one launch */
extern "C" int smol_internal_norm_rope_bf16_qk(smol_attn_ctx *ctx, const smol_rope_table *rope, uint16_t *q,
                                               const float *q_weight, uint16_t *k, const float *k_weight, float eps,
                                               int pos0, int seq, int n_heads, int n_kv_heads, int head_dim) {
    if (!k) return fail(SMOL_ATTN_ERR_ARG, "k is NULL");
    return norm_rope_bf16(ctx, rope, q, q_weight, k, k_weight, n_kv_heads, eps, pos0, seq, n_heads, head_dim);
}

/* ============================================ reference-signature drop-ins */

namespace {

/* Per-thread state of the drop-ins. It is never freed: releasing device
 * memory from a thread-exit or static destructor can run after the HIP
 * runtime has shut down; the process exit reclaims it. */
struct Legacy {
    smol_attn_ctx *ctx = nullptr;
    DevBuf q, k, v, out, cs;
};

thread_local Legacy g_legacy;

[[noreturn]] void legacy_abort(const char *fn) {
    fprintf(stderr, "smol_attn: %s failed on the GPU: %s\n", fn, smol_attn_last_error());
    abort();
}

smol_attn_ctx *legacy_ctx(const char *fn) {
    if (!g_legacy.ctx && smol_attn_ctx_create(0, nullptr, &g_legacy.ctx) != SMOL_ATTN_OK) legacy_abort(fn);
    return g_legacy.ctx;
}

} // namespace

/* for linear.hip's drop-ins: the calling thread's context of the
 * reference-signature entry points (created on first use, device 0) */
extern "C" smol_attn_ctx *smol_internal_legacy_ctx(const char *fn) { return legacy_ctx(fn); }

namespace {

void legacy_upload(const char *fn, DevBuf &b, const void *h, size_t bytes) {
    smol_attn_ctx *ctx = legacy_ctx(fn);
    if (dev_reserve(b, std::max<size_t>(bytes, 4), ctx->stream)) legacy_abort(fn);
    if (bytes && hipMemcpyAsync(b.p, h, bytes, hipMemcpyHostToDevice, ctx->stream) != hipSuccess) legacy_abort(fn);
}

/* copies the result back and waits; returns SMOL_ATTN_OK or
 * SMOL_ATTN_ERR_RANGE (any other failure aborts) */
int legacy_download(const char *fn, void *h, const DevBuf &b, size_t bytes) {
    smol_attn_ctx *ctx = legacy_ctx(fn);
    if (bytes && hipMemcpyAsync(h, b.p, bytes, hipMemcpyDeviceToHost, ctx->stream) != hipSuccess) legacy_abort(fn);
    const int rc = smol_attn_ctx_synchronize(ctx);
    if (rc != SMOL_ATTN_OK && rc != SMOL_ATTN_ERR_RANGE) legacy_abort(fn);
    return rc;
}

/* The attention kernels take head_dim 64, 72, 80, 96, 128 and 256; the
 * reference takes any (attention.c:79-126). A drop-in call with another
 * head_dim up to 256 runs at the next supported one with every head row
 * zero-padded: the zero columns add nothing to Q K^T (the caller's scale is
 * passed as given) and the output's padded columns are dropped. */
int padded_hd(int hd) {
    for (int h : {64, 72, 80, 96, 128, 256})
        if (hd <= h) return h;
    return 0;
}

/* rows of hd floats into device rows of hdp floats (the padding zeroed) */
void legacy_upload_rows(const char *fn, DevBuf &b, const float *h, size_t rows, int hd, int hdp) {
    if (hd == hdp) return legacy_upload(fn, b, h, rows * hd * 4);
    smol_attn_ctx *ctx = legacy_ctx(fn);
    const size_t bytes = rows * hdp * 4;
    if (dev_reserve(b, std::max<size_t>(bytes, 4), ctx->stream)) legacy_abort(fn);
    if (!rows) return;
    if (hipMemsetAsync(b.p, 0, bytes, ctx->stream) != hipSuccess ||
        hipMemcpy2DAsync(b.p, (size_t)hdp * 4, h, (size_t)hd * 4, (size_t)hd * 4, rows, hipMemcpyHostToDevice,
                         ctx->stream) != hipSuccess)
        legacy_abort(fn);
}

int legacy_download_rows(const char *fn, float *h, const DevBuf &b, size_t rows, int hd, int hdp) {
    if (hd == hdp) return legacy_download(fn, h, b, rows * hd * 4);
    smol_attn_ctx *ctx = legacy_ctx(fn);
    if (rows && hipMemcpy2DAsync(h, (size_t)hd * 4, b.p, (size_t)hdp * 4, (size_t)hd * 4, rows,
                                 hipMemcpyDeviceToHost, ctx->stream) != hipSuccess)
        legacy_abort(fn);
    return legacy_download(fn, nullptr, b, 0);
}

/* largest |x|; *finite is cleared when a value is NaN or infinite */
float host_absmax(const float *x, size_t n, bool *finite) {
    float m = 0.0f;
    for (size_t i = 0; i < n; i++) {
        const float a = fabsf(x[i]);
        if (!(a <= FLT_MAX)) *finite = false;
        else if (a > m) m = a;
    }
    return m;
}

/* smallest e with x < 2^e (x > 0) */
int pow2_above(float x) {
    int e;
    frexpf(x, &e);
    return e;
}

/* The drop-ins' answer to a range error of the fp16 staging. The prefill
 * kernels stage Q * scale * log2 e, K and V as fp16; the same result comes
 * from Q 2^-a, K 2^a (Q K^T unchanged) and V 2^-b with the output times
 * 2^b, exactly while the scaled values stay clear of fp16's subnormal and
 * overflow ranges. This picks a to balance the largest staged |Q| and |K|
 * (both then below 2^15) and b to bring the largest |V| below 2^15.
 * Returns 0 with (a, b) set; 1 when an input is not finite (the output
 * stands as computed: non-finite inputs give non-finite scores in the
 * reference too); -1 when no such a exists
 * (max|Q| * scale * log2 e * max|K| >= 2^30). */
int legacy_range_fix(const float *Q, size_t nq, const float *K, const float *V, size_t nk, float qmul, int *a,
                     int *b) {
    bool finite = true;
    const float mq = host_absmax(Q, nq, &finite) * qmul, mk = host_absmax(K, nk, &finite);
    const float mv = host_absmax(V, nk, &finite);
    if (!finite || !(mq <= FLT_MAX)) return 1;
    const int eq = mq > 0.0f ? pow2_above(mq) : 0, ek = mk > 0.0f ? pow2_above(mk) : 0;
    const int lo = mq > 0.0f ? eq - 15 : INT_MIN / 2, hi = mk > 0.0f ? 15 - ek : INT_MAX / 2;
    if (lo > hi) return -1;
    const int x = (mq > 0.0f && mk > 0.0f) ? (eq - ek) / 2 : 0;
    *a = std::min(std::max(x, lo), hi);
    *b = mv > 0.0f ? std::max(0, pow2_above(mv) - 15) : 0;
    return 0;
}

std::vector<float> scaled_copy(const float *x, size_t n, int e) {
    std::vector<float> y(x, x + n);
    if (e)
        for (float &v : y) v = ldexpf(v, e);
    return y;
}

void scale_out(float *out, size_t n, int e) {
    if (e)
        for (size_t i = 0; i < n; i++) out[i] = ldexpf(out[i], e);
}

/* The four causal variants of attention.c. use_window / use_cap say which
 * entry point was called; the reference's rules for their values are applied
 * here (attention.c:190-192, 284-308): a window_size <= 0 leaves every row
 * without keys, so the output is zero; cap * tanhf(s / cap) is the same for
 * cap and -cap; cap == 0 turns every score into 0 (0 * tanhf(+-inf)), which
 * is plain attention with scale 0. The device entry points take window > 0
 * and cap > 0 as "on". */
void legacy_causal(const char *fn, float *out, const float *Q, const float *K, const float *V, int seq_q,
                   int seq_k, int Hq, int Hkv, int hd, float scale, int q_offset, bool use_window, int window,
                   bool use_cap, float cap) {
    if (seq_q <= 0 || Hq <= 0 || hd <= 0) return; /* no output elements */
    const size_t qb = (size_t)seq_q * Hq * hd * 4, kb = (size_t)std::max(seq_k, 0) * Hkv * hd * 4;
    if (use_window && window <= 0) {
        memset(out, 0, qb);
        return;
    }
    if (!use_window) window = 0;
    if (use_cap) {
        if (cap == 0.0f) scale = 0.0f;
        cap = fabsf(cap);
    } else {
        cap = 0.0f;
    }
    smol_attn_ctx *ctx = legacy_ctx(fn);
    const int hdp = padded_hd(hd);
    if (!hdp) {
        fail(SMOL_ATTN_ERR_UNSUPPORTED, "head_dim %d (at most 256)", hd);
        legacy_abort(fn);
    }
    const size_t q_rows = (size_t)seq_q * Hq, k_rows = (size_t)std::max(seq_k, 0) * Hkv;
    auto run = [&](const float *q, const float *k, const float *v) {
        legacy_upload_rows(fn, g_legacy.q, q, q_rows, hd, hdp);
        legacy_upload_rows(fn, g_legacy.k, k, k_rows, hd, hdp);
        legacy_upload_rows(fn, g_legacy.v, v, k_rows, hd, hdp);
        if (dev_reserve(g_legacy.out, q_rows * hdp * 4, ctx->stream)) legacy_abort(fn);
        if (smol_attn_causal(ctx, g_legacy.q.p, g_legacy.k.p, g_legacy.v.p, SMOL_ATTN_F32, seq_q, seq_k, Hq, Hkv,
                             hdp, scale, q_offset, window, cap, (float *)g_legacy.out.p) != SMOL_ATTN_OK)
            legacy_abort(fn);
        return legacy_download_rows(fn, out, g_legacy.out, q_rows, hd, hdp);
    };
    if (run(Q, K, V) == SMOL_ATTN_OK) return;
    const size_t nq = qb / 4, nk = kb / 4;
    int a = 0, b = 0;
    const int fix = legacy_range_fix(Q, nq, K, V, nk, fabsf(scale) * (float)LOG2E_D, &a, &b);
    if (fix > 0) return;
    if (fix < 0) legacy_abort(fn);
    const std::vector<float> q2 = scaled_copy(Q, nq, -a), k2 = scaled_copy(K, nk, a), v2 = scaled_copy(V, nk, -b);
    if (run(q2.data(), k2.data(), v2.data()) != SMOL_ATTN_OK) legacy_abort(fn);
    scale_out(out, nq, b);
}

}  // namespace

extern "C" void smol_causal_attention(float *out, const float *Q, const float *K, const float *V, int seq_q,
                                      int seq_k, int n_heads, int n_kv_heads, int head_dim, float scale,
                                      int q_offset) {
    legacy_causal(__func__, out, Q, K, V, seq_q, seq_k, n_heads, n_kv_heads, head_dim, scale, q_offset, false, 0,
                  false, 0.0f);
}

extern "C" void smol_sliding_window_attention(float *out, const float *Q, const float *K, const float *V,
                                              int seq_q, int seq_k, int n_heads, int n_kv_heads, int head_dim,
                                              float scale, int q_offset, int window_size) {
    legacy_causal(__func__, out, Q, K, V, seq_q, seq_k, n_heads, n_kv_heads, head_dim, scale, q_offset, true,
                  window_size, false, 0.0f);
}

extern "C" void smol_causal_attention_softcap(float *out, const float *Q, const float *K, const float *V,
                                              int seq_q, int seq_k, int n_heads, int n_kv_heads, int head_dim,
                                              float scale, int q_offset, float cap) {
    legacy_causal(__func__, out, Q, K, V, seq_q, seq_k, n_heads, n_kv_heads, head_dim, scale, q_offset, false, 0,
                  true, cap);
}

extern "C" void smol_sliding_window_attention_softcap(float *out, const float *Q, const float *K,
                                                      const float *V, int seq_q, int seq_k, int n_heads,
                                                      int n_kv_heads, int head_dim, float scale, int q_offset,
                                                      int window_size, float cap) {
    legacy_causal(__func__, out, Q, K, V, seq_q, seq_k, n_heads, n_kv_heads, head_dim, scale, q_offset, true,
                  window_size, true, cap);
}

extern "C" void smol_bidirectional_attention(float *out, const float *Q, const float *K, const float *V, int seq,
                                             int n_heads, int head_dim, float scale, const int *window_starts,
                                             int n_windows) {
    (void)seq; /* unused by the reference too (attention.c:33); the windows define the rows */
    if (n_windows <= 0 || n_heads <= 0 || head_dim <= 0) return;
    const int rows = window_starts[n_windows];
    if (rows <= 0) return;
    const char *fn = __func__;
    smol_attn_ctx *ctx = legacy_ctx(fn);
    const int hdp = padded_hd(head_dim);
    if (!hdp) {
        fail(SMOL_ATTN_ERR_UNSUPPORTED, "head_dim %d (at most 256)", head_dim);
        legacy_abort(fn);
    }
    const size_t hrows = (size_t)rows * n_heads, n = hrows * head_dim;
    /* rows outside every window are left untouched by the reference; keep
     * them (a copy, since a repeated call must start from the same rows) */
    const std::vector<float> keep(out, out + n);
    auto run = [&](const float *q, const float *k, const float *v) {
        legacy_upload_rows(fn, g_legacy.q, q, hrows, head_dim, hdp);
        legacy_upload_rows(fn, g_legacy.k, k, hrows, head_dim, hdp);
        legacy_upload_rows(fn, g_legacy.v, v, hrows, head_dim, hdp);
        legacy_upload_rows(fn, g_legacy.out, keep.data(), hrows, head_dim, hdp);
        if (smol_attn_bidirectional(ctx, g_legacy.q.p, g_legacy.k.p, g_legacy.v.p, SMOL_ATTN_F32, rows, n_heads, hdp,
                                    scale, window_starts, n_windows, (float *)g_legacy.out.p) != SMOL_ATTN_OK)
            legacy_abort(fn);
        return legacy_download_rows(fn, out, g_legacy.out, hrows, head_dim, hdp);
    };
    if (run(Q, K, V) == SMOL_ATTN_OK) return;
    int a = 0, b = 0;
    const int fix = legacy_range_fix(Q, n, K, V, n, fabsf(scale) * (float)LOG2E_D, &a, &b);
    if (fix > 0) return;
    if (fix < 0) legacy_abort(fn);
    const std::vector<float> q2 = scaled_copy(Q, n, -a), k2 = scaled_copy(K, n, a), v2 = scaled_copy(V, n, -b);
    if (run(q2.data(), k2.data(), v2.data()) != SMOL_ATTN_OK) legacy_abort(fn);
    /* only the windows' rows were computed with V 2^-b */
    const size_t row = (size_t)n_heads * head_dim;
    for (int w = 0; w < n_windows; w++) {
        const int r0 = std::max(window_starts[w], 0), r1 = std::min(window_starts[w + 1], rows);
        if (r1 > r0) scale_out(out + (size_t)r0 * row, (size_t)(r1 - r0) * row, b);
    }
}

/* rope.c:27-66: the table rows for explicit positions (host, as in the reference) */
static void compute_rope_rows(float *c, float *s, const int *positions, int seq, int hd, float theta, int type) {
    for (int i = 0; i < seq; i++)
        smol_rope_fill_host(c + (size_t)i * hd, s + (size_t)i * hd, positions[i], 1, hd, theta, type);
}

extern "C" void smol_compute_rope_neox(float *cos_out, float *sin_out, const int *positions, int seq, int head_dim,
                                       float theta) {
    compute_rope_rows(cos_out, sin_out, positions, seq, head_dim, theta, SMOL_ROPE_NEOX);
}

extern "C" void smol_compute_rope_interleaved(float *cos_out, float *sin_out, const int *positions, int seq,
                                              int head_dim, float theta) {
    compute_rope_rows(cos_out, sin_out, positions, seq, head_dim, theta, SMOL_ROPE_INTERLEAVED);
}

static void legacy_rope(const char *fn, float *x, const float *c, const float *s, int seq, int H, int hd,
                        int kind) {
    if (seq <= 0 || H <= 0) return;
    smol_attn_ctx *ctx = legacy_ctx(fn);
    const size_t xb = (size_t)seq * H * hd * 4, tb = (size_t)seq * hd * 4;
    legacy_upload(fn, g_legacy.q, x, xb);
    if (dev_reserve(g_legacy.cs, 2 * tb, ctx->stream)) legacy_abort(fn);
    if (hipMemcpyAsync(g_legacy.cs.p, c, tb, hipMemcpyHostToDevice, ctx->stream) != hipSuccess ||
        hipMemcpyAsync((char *)g_legacy.cs.p + tb, s, tb, hipMemcpyHostToDevice, ctx->stream) != hipSuccess)
        legacy_abort(fn);
    if (smol_launch_norm_rope((float *)g_legacy.q.p, nullptr, 0.0f, (const float *)g_legacy.cs.p,
                              (const float *)((char *)g_legacy.cs.p + tb), nullptr, seq, H, hd, kind, ctx->stream))
        legacy_abort(fn);
    legacy_download(fn, x, g_legacy.q, xb);
}

extern "C" void smol_apply_rope_neox(float *x, const float *cos_vals, const float *sin_vals, int seq, int n_heads,
                                     int head_dim) {
    legacy_rope(__func__, x, cos_vals, sin_vals, seq, n_heads, head_dim, SMOL_ROPE_NEOX_K);
}

extern "C" void smol_apply_rope_interleaved(float *x, const float *cos_vals, const float *sin_vals, int seq,
                                            int n_heads, int head_dim) {
    legacy_rope(__func__, x, cos_vals, sin_vals, seq, n_heads, head_dim, SMOL_ROPE_INTERLEAVED_K);
}

extern "C" void smol_rms_norm_per_head(float *x, const float *weight, int seq_len, int n_heads, int head_dim,
                                       float eps) {
    const char *fn = __func__;
    if (seq_len <= 0 || n_heads <= 0 || head_dim <= 0) return;
    smol_attn_ctx *ctx = legacy_ctx(fn);
    const size_t xb = (size_t)seq_len * n_heads * head_dim * 4, wb = (size_t)head_dim * 4;
    legacy_upload(fn, g_legacy.q, x, xb);
    legacy_upload(fn, g_legacy.cs, weight, wb);
    if (smol_launch_norm_rope((float *)g_legacy.q.p, (const float *)g_legacy.cs.p, eps, nullptr, nullptr, nullptr,
                              seq_len, n_heads, head_dim, SMOL_ROPE_OFF, ctx->stream))
        legacy_abort(fn);
    legacy_download(fn, x, g_legacy.q, xb);
}
