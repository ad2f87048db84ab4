"""The CPU oracle's answer for each workload of smol-genius_amd/workloads.py.
TEST INFRASTRUCTURE ONLY (tests, smoke check, CPU-baseline leg of the bench).

Each function follows the reference decoder's order of operations on the
same input bits: widen bf16 to fp32, build the RoPE table as fill_rope_cache
does (qkn_decoder.c:276-311), optionally apply the per-head RMSNorm
(qkn_decoder.c:487-491), rotate Q and the new K in fp32
(smol_apply_rope_*, qkn_decoder.c:493-495 / :647-649), append to the cache
(qkn_decoder.c:498-503 / :651-652), then smol_causal_attention or
smol_bidirectional_attention (attention.c:32-170). The cache is the
workloads' bf16 cache: a call attends to its own new rows at fp32 and to
rows written before it as bf16.
"""
import numpy as np

from oracle import Oracle


def _widen(b):
    return (np.ascontiguousarray(b, np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def _as_f32(a):
    a = np.asarray(a)
    return _widen(a) if a.dtype == np.uint16 else np.ascontiguousarray(a, np.float32)


def rope_rows(orc, positions, hd, theta, interleaved, cache={}):
    key = (hd, float(theta), bool(interleaved))
    need = int(np.max(positions)) + 1
    c = cache.get(key)
    if c is None or c[0].shape[0] < need:
        cap = 1024
        while cap < need:
            cap *= 2
        c = orc.fill_rope_table(0, cap, hd, theta, interleaved)
        cache[key] = c
    return c[0][positions], c[1][positions]


def _norm(orc, a, w, rows, heads, hd, eps):
    """per-head RMSNorm before RoPE (qkn_decoder.c:487-491); w None: none"""
    a = _as_f32(a)
    return a if w is None else orc.rms_norm_per_head(a, w, rows, heads, hd, eps)


def decode(orc: Oracle, wl, x, q_norm=None, k_norm=None, eps=1e-6, window=0, cap=0.0):
    """out [n_seq, Hq*hd]: per sequence, attention of the (normalised and)
    rotated new query over its widened cache plus the rotated new key
    (optionally a sliding window and a softcap, attention.c:153-170 and its
    variants)."""
    inter = wl.rope_type == 1
    outs = []
    for i, L in enumerate(wl.lengths):
        p = L - 1
        c, s = rope_rows(orc, np.array([p]), wl.hd, wl.theta, inter)
        q = orc.apply_rope(_norm(orc, x["q"][i:i + 1], q_norm, 1, wl.Hq, wl.hd, eps), c, s, 1, wl.Hq, wl.hd, inter)
        kn = orc.apply_rope(_norm(orc, x["k"][i:i + 1], k_norm, 1, wl.Hkv, wl.hd, eps), c, s, 1, wl.Hkv, wl.hd,
                            inter)
        K = np.concatenate([_widen(x["cache_k"][i]), kn], 0)
        V = np.concatenate([_widen(x["cache_v"][i]), x["v"][i:i + 1]], 0)
        outs.append(orc.causal_attention(q, K, V, 1, L, wl.Hq, wl.Hkv, wl.hd, wl.scale, p, window=window, cap=cap))
    return np.concatenate(outs, 0)


def prefill(orc: Oracle, wl, x, window=0, cap=0.0, q_norm=None, k_norm=None, eps=1e-6):
    P, S = wl.pos0, wl.seq_q
    pos = np.arange(P, P + S)
    c, s = rope_rows(orc, pos, wl.hd, wl.theta, wl.rope_type == 1)
    q = orc.apply_rope(_norm(orc, x["q"], q_norm, S, wl.Hq, wl.hd, eps), c, s, S, wl.Hq, wl.hd, wl.rope_type == 1)
    kn = orc.apply_rope(_norm(orc, x["k"], k_norm, S, wl.Hkv, wl.hd, eps), c, s, S, wl.Hkv, wl.hd,
                        wl.rope_type == 1)
    K = np.concatenate([_widen(x["cache_k"]).reshape(P, wl.Hkv * wl.hd), kn], 0)
    V = np.concatenate([_widen(x["cache_v"]).reshape(P, wl.Hkv * wl.hd), _as_f32(x["v"])], 0)
    return orc.causal_attention(q, K, V, S, P + S, wl.Hq, wl.Hkv, wl.hd, wl.scale, P, window=window, cap=cap)


def bidir(orc: Oracle, wl, x):
    return orc.bidirectional_attention(_as_f32(x["q"]), _as_f32(x["k"]), _as_f32(x["v"]), wl.seq, wl.H, wl.hd,
                                       wl.scale, wl.window_starts)


def _bf16_round(a):
    """a rounded to bf16 (nearest even) and widened back: what a bf16 cache returns"""
    u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    return _widen(((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16))


def stream(orc: Oracle, wl, x):
    """(chunk_out [chunk, Hq*hd], decode_out [steps, Hq*hd]). The cache is the
    workload's bf16 cache: each call uses its own new rows at fp32 (as the
    reference decoder does, qkn_decoder.c:498-528) and the rows appended by
    earlier calls as stored, rounded to bf16 (nearest even)."""
    P, C = wl.prefix, wl.chunk
    pos = np.arange(P, P + C)
    c, s = rope_rows(orc, pos, wl.hd, wl.theta, False)
    q = orc.apply_rope(x["q"], c, s, C, wl.Hq, wl.hd)
    kn = orc.apply_rope(x["k"], c, s, C, wl.Hkv, wl.hd)
    K = np.concatenate([_widen(x["cache_k"]), kn], 0)
    V = np.concatenate([_widen(x["cache_v"]), x["v"]], 0)
    chunk = orc.causal_attention(q, K, V, C, P + C, wl.Hq, wl.Hkv, wl.hd, wl.scale, P)
    dec = []
    for st in range(wl.steps):
        p = P + C + st
        c, s = rope_rows(orc, np.array([p]), wl.hd, wl.theta, False)
        qd = orc.apply_rope(x["dq"][st:st + 1], c, s, 1, wl.Hq, wl.hd)
        kd = orc.apply_rope(x["dk"][st:st + 1], c, s, 1, wl.Hkv, wl.hd)
        if st == 0:  # the chunk's rows come back from the bf16 cache
            K = np.concatenate([K[:P], _bf16_round(K[P:])], 0)
            V = np.concatenate([V[:P], _bf16_round(V[P:])], 0)
        else:        # so does the previous step's row
            K[-1] = _bf16_round(K[-1])
            V[-1] = _bf16_round(V[-1])
        K = np.concatenate([K, kd], 0)
        V = np.concatenate([V, x["dv"][st:st + 1]], 0)
        dec.append(orc.causal_attention(qd, K, V, 1, p + 1, wl.Hq, wl.Hkv, wl.hd, wl.scale, p))
    return chunk, np.concatenate(dec, 0)


def evaluate(orc, wl, x):
    kind = type(wl).__name__
    if getattr(wl, "qk_norm", False):
        qw, kw = wl.norm_weights()
        return {"Decode": decode, "Prefill": prefill}[kind](orc, wl, x, q_norm=qw, k_norm=kw, eps=wl.norm_eps)
    return {"Decode": decode, "Prefill": prefill, "Bidir": bidir, "Stream": stream}[kind](orc, wl, x)
