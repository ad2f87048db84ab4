"""Times the reference's CPU attention on a workload. TEST/BENCH INFRASTRUCTURE ONLY.

Uses oracle/_ref (the reference's own attention.c / rope.c / vecops /
threading.c, compiled by oracle/Makefile) when it exists, otherwise the C
restatement (liboracle). The timed call sequence is the reference decoder's
attention block for the workload: smol_apply_rope_* on Q and the new K
(qkn_decoder.c:493-495 / :647-649), then smol_causal_attention or
smol_bidirectional_attention (qkn_decoder.c:525-527 / :674-676,
siglip.c:126-128). Threads: min(nproc, 16), as the reference's pool allows
(threading.c:22).
"""
import os
import time

import numpy as np

from oracle import Oracle, RefLib, ref_path, simd_branch


def _widen(b):
    return (np.ascontiguousarray(b, np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def _f32(a):
    a = np.asarray(a)
    return _widen(a) if a.dtype == np.uint16 else np.ascontiguousarray(a, np.float32)


def host_facts():
    """nproc, the CPU model and the SIMD branch the reference's vector code takes here
    (vecops_avx.c:14: AVX-512 when the compiler targets it, else AVX2)."""
    model = None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"nproc": os.cpu_count(), "cpu_model": model, "simd": simd_branch()}


def _lib():
    cores = min(os.cpu_count() or 1, 16)
    if ref_path():
        lib, kind = RefLib(), "reference"
    else:
        lib, kind = Oracle(), "port"
    lib.set_threads(cores)
    return lib, kind, cores


def prefill_sample(wl, x, min_seconds=10.0, max_reps=50):
    """Full causal prefill (RoPE on Q and K + attention) repeated for >= min_seconds."""
    lib, kind, cores = _lib()
    orc = Oracle()
    P, S = wl.pos0, wl.seq_q
    c, s = orc.fill_rope_table(0, P + S, wl.hd, wl.theta, wl.rope_type == 1)
    c, s = c[P:], s[P:]
    q0, k0, v = _f32(x["q"]), _f32(x["k"]), _f32(x["v"])
    Kc = _widen(x["cache_k"]).reshape(P, wl.Hkv * wl.hd)
    Vc = _widen(x["cache_v"]).reshape(P, wl.Hkv * wl.hd)
    reps, t = 0, 0.0
    while reps < 2 or (t < min_seconds and reps < max_reps):
        t0 = time.perf_counter()
        q = lib.apply_rope(q0, c, s, S, wl.Hq, wl.hd, wl.rope_type == 1)
        kn = lib.apply_rope(k0, c, s, S, wl.Hkv, wl.hd, wl.rope_type == 1)
        K = np.concatenate([Kc, kn], 0)
        V = np.concatenate([Vc, v], 0)
        lib.causal_attention(q, K, V, S, P + S, wl.Hq, wl.Hkv, wl.hd, wl.scale, P)
        t += time.perf_counter() - t0
        reps += 1
    sec = t / reps
    return {"value": round(wl.flops() / sec / 1e12, 6), "unit": "TFLOP/s", "cores": cores, "kind": kind,
            "ms_per_step": round(sec * 1e3, 3), **host_facts(),
            "sample": "%d full repetitions of the %s step (RoPE on Q and K + causal attention, %d x %d, "
                      "%d heads)" % (reps, wl.name, S, P + S, wl.Hq)}


def decode_sample(wl, x, min_seconds=3.0, max_reps=200):
    """One decode step of every sequence (RoPE on q and k + attention over its cache)."""
    lib, kind, cores = _lib()
    orc = Oracle()
    inter = wl.rope_type == 1
    c, s = orc.fill_rope_table(0, max(wl.lengths), wl.hd, wl.theta, inter)
    Ks = [np.concatenate([_widen(x["cache_k"][i]), np.zeros((1, wl.Hkv * wl.hd), np.float32)], 0)
          for i in range(wl.n_seq)]
    Vs = [np.concatenate([_widen(x["cache_v"][i]), x["v"][i:i + 1]], 0) for i in range(wl.n_seq)]
    reps, t = 0, 0.0
    while reps < 2 or (t < min_seconds and reps < max_reps):
        t0 = time.perf_counter()
        for i, L in enumerate(wl.lengths):
            p = L - 1
            q = lib.apply_rope(x["q"][i:i + 1], c[p:p + 1], s[p:p + 1], 1, wl.Hq, wl.hd, inter)
            Ks[i][p] = lib.apply_rope(x["k"][i:i + 1], c[p:p + 1], s[p:p + 1], 1, wl.Hkv, wl.hd, inter)[0]
            lib.causal_attention(q, Ks[i], Vs[i], 1, L, wl.Hq, wl.Hkv, wl.hd, wl.scale, p)
        t += time.perf_counter() - t0
        reps += 1
    sec = t / reps
    return {"value": round(wl.algorithmic_bytes() / sec / 1e9, 3), "unit": "GB/s", "cores": cores, "kind": kind,
            "ms_per_step": round(sec * 1e3, 3), **host_facts(),
            "sample": "%d repetitions of one decode step of %d sequences" % (reps, wl.n_seq)}


def bidir_sample(wl, x, min_seconds=3.0, max_reps=50):
    lib, kind, cores = _lib()
    q, k, v = _widen(x["q"]), _widen(x["k"]), _widen(x["v"])
    reps, t = 0, 0.0
    while reps < 2 or (t < min_seconds and reps < max_reps):
        t0 = time.perf_counter()
        lib.bidirectional_attention(q, k, v, wl.seq, wl.H, wl.hd, wl.scale, wl.window_starts)
        t += time.perf_counter() - t0
        reps += 1
    sec = t / reps
    return {"value": round(wl.flops() / sec / 1e12, 6), "unit": "TFLOP/s", "cores": 1, "kind": kind,
            "ms_per_step": round(sec * 1e3, 3), **host_facts(),
            "sample": "%d repetitions; smol_bidirectional_attention is single-threaded "
                      "(attention.c:32-77)" % reps}


def stream_sample(wl, x, min_seconds=5.0, max_reps=20):
    """The streaming step: RoPE + the chunk's causal attention over the cache, then
    `steps` single-token decode calls against the growing cache (qkn_decoder.c:493-528,
    :647-677)."""
    lib, kind, cores = _lib()
    orc = Oracle()
    P, C, n = wl.prefix, wl.chunk, wl.steps
    total = P + C + n
    c, s = orc.fill_rope_table(0, total, wl.hd, wl.theta, False)
    w = wl.Hkv * wl.hd
    K = np.zeros((total, w), np.float32)
    V = np.zeros((total, w), np.float32)
    K[:P] = _widen(x["cache_k"]).reshape(P, w)
    V[:P] = _widen(x["cache_v"]).reshape(P, w)
    reps, t = 0, 0.0
    while reps < 1 or (t < min_seconds and reps < max_reps):
        t0 = time.perf_counter()
        q = lib.apply_rope(x["q"], c[P:P + C], s[P:P + C], C, wl.Hq, wl.hd, False)
        K[P:P + C] = lib.apply_rope(x["k"], c[P:P + C], s[P:P + C], C, wl.Hkv, wl.hd, False)
        V[P:P + C] = x["v"]
        lib.causal_attention(q, K, V, C, P + C, wl.Hq, wl.Hkv, wl.hd, wl.scale, P)
        for st in range(n):
            p = P + C + st
            q = lib.apply_rope(x["dq"][st:st + 1], c[p:p + 1], s[p:p + 1], 1, wl.Hq, wl.hd, False)
            K[p] = lib.apply_rope(x["dk"][st:st + 1], c[p:p + 1], s[p:p + 1], 1, wl.Hkv, wl.hd, False)[0]
            V[p] = x["dv"][st]
            lib.causal_attention(q, K, V, 1, p + 1, wl.Hq, wl.Hkv, wl.hd, wl.scale, p)
        t += time.perf_counter() - t0
        reps += 1
    sec = t / reps
    return {"value": round(wl.decode_bytes() / sec / 1e9, 3), "unit": "GB/s (decode bytes over the whole step)",
            "cores": cores, "kind": kind, "ms_per_step": round(sec * 1e3, 3), **host_facts(),
            "sample": "%d repetitions of the chunk call + %d decode calls" % (reps, n)}


def projections_sample(wl, x, min_seconds=3.0, max_reps=100, max_rows=64):
    """One layer's projections as the reference decoder calls them: for one token
    smol_linear_nobias_bf16_qkv + smol_linear_nobias_bf16 x 3 (qkn_decoder.c:635, 679,
    693, 699: threaded bf16 matvecs); for a prefill smol_linear_nobias_bf16 per weight
    (qkn_decoder.c:474-476, 531, 546, 552: a bf16 -> fp32 weight copy and single-threaded
    loops, matmul.c:336-346), on at most `max_rows` rows of the input (the work per row
    is the same for every row)."""
    lib, kind, cores = _lib()
    rows = min(wl.seq, max_rows)
    ws = {k: wl.layer_weights(0, k) for k in wl.kinds}
    xs = {k: np.ascontiguousarray(x["x"][k][:rows]) for k in wl.kinds}
    reps, t = 0, 0.0
    while reps < 2 or (t < min_seconds and reps < max_reps):
        t0 = time.perf_counter()
        for k in wl.kinds:
            if k == "qkv" and rows == 1 and hasattr(lib, "linear_qkv"):
                lib.linear_qkv(xs[k], *ws[k])
            else:
                for w in ws[k]:
                    lib.linear_bf16(xs[k], w)
        t += time.perf_counter() - t0
        reps += 1
    sec = t / reps * (wl.seq / rows)
    if wl.seq == 1:
        val, unit = round(wl.algorithmic_bytes() / sec / 1e9, 3), "GB/s"
        threads = cores
    else:
        val, unit = round(wl.flops() / sec / 1e12, 6), "TFLOP/s"
        threads = 1  # smol_linear's loops are not threaded (matmul.c:70-97)
    return {"value": val, "unit": unit, "cores": threads, "kind": kind, "ms_per_step": round(sec * 1e3, 3),
            **host_facts(),
            "sample": "%d repetitions of one layer's projections on %d of %d rows%s" % (
                reps, rows, wl.seq, "" if rows == wl.seq else ", scaled to all rows")}


def decoder_step_sample(n_layers=28, dim=1024, inter=3072, H=16, Hkv=8, hd=128, prefix=1024, sample_layers=2,
                        min_seconds=3.0, max_reps=50):
    """One token through Qwen3-0.6B decoder layers as qkn_decoder_forward runs them
    (qkn_decoder.c:633-705): smol_rms_norm, smol_linear_nobias_bf16_qkv, per-head
    RMSNorm, NeoX RoPE, smol_causal_attention over a `prefix`-row cache,
    smol_linear_nobias_bf16 (o_proj), the residual add, smol_rms_norm,
    smol_linear_nobias_bf16 (gate_up), smol_swiglu_multiply,
    smol_linear_nobias_bf16 (down), the residual add. Timed on `sample_layers`
    layers and scaled to n_layers (every layer does the same work)."""
    lib, kind, cores = _lib()
    orc = Oracle()
    rng = np.random.default_rng(5)

    def bits(o, i):
        w = (rng.standard_normal((o, i)) / np.sqrt(i)).astype(np.float32)
        return (w.view(np.uint32) >> 16).astype(np.uint16)

    layers = []
    for _ in range(sample_layers):
        layers.append(dict(
            inorm=(1 + 0.1 * rng.standard_normal(dim)).astype(np.float32),
            pnorm=(1 + 0.1 * rng.standard_normal(dim)).astype(np.float32),
            qn=(1 + 0.1 * rng.standard_normal(hd)).astype(np.float32),
            kn=(1 + 0.1 * rng.standard_normal(hd)).astype(np.float32),
            wq=bits(H * hd, dim), wk=bits(Hkv * hd, dim), wv=bits(Hkv * hd, dim), wo=bits(dim, H * hd),
            gu=bits(2 * inter, dim), down=bits(dim, inter),
            K=rng.standard_normal((prefix + 1, Hkv * hd)).astype(np.float32),
            V=rng.standard_normal((prefix + 1, Hkv * hd)).astype(np.float32)))
    c, s = orc.fill_rope_table(0, prefix + 1, hd, 1e6, False)
    c, s = c[prefix:prefix + 1], s[prefix:prefix + 1]
    scale = float(np.float32(1.0) / np.sqrt(np.float32(hd)))
    x0 = rng.standard_normal((1, dim)).astype(np.float32)
    reps, t = 0, 0.0
    while reps < 2 or (t < min_seconds and reps < max_reps):
        x = x0.copy()
        t0 = time.perf_counter()
        for L in layers:
            xn = lib.rms_norm(x, L["inorm"], 1e-6)
            if hasattr(lib, "linear_qkv"):
                q, k, v = lib.linear_qkv(xn, L["wq"], L["wk"], L["wv"])
            else:
                q, k, v = (lib.linear_bf16(xn, L[n])[0] for n in ("wq", "wk", "wv"))
            q = lib.rms_norm_per_head(q[None], L["qn"], 1, H, hd, 1e-6)
            k = lib.rms_norm_per_head(k[None], L["kn"], 1, Hkv, hd, 1e-6)
            q = lib.apply_rope(q, c, s, 1, H, hd, False)
            L["K"][prefix] = lib.apply_rope(k, c, s, 1, Hkv, hd, False)[0]
            L["V"][prefix] = v
            a = lib.causal_attention(q, L["K"], L["V"], 1, prefix + 1, H, Hkv, hd, scale, prefix)
            x = x + lib.linear_bf16(a, L["wo"])
            h = lib.rms_norm(x, L["pnorm"], 1e-6)
            x = x + lib.linear_bf16(lib.glu(lib.linear_bf16(h, L["gu"]), 1), L["down"])
        t += time.perf_counter() - t0
        reps += 1
    sec = t / reps * n_layers / sample_layers
    return {"value": round(1.0 / sec, 2), "unit": "tokens/s", "cores": cores, "kind": kind,
            "ms_per_token": round(sec * 1e3, 3), **host_facts(),
            "sample": "%d repetitions of one token through %d layers (%d cached tokens), scaled to %d layers" % (
                reps, sample_layers, prefix, n_layers)}


def bf16_decoder_step_sample(n_layers=28, dim=1024, inter=3072, H=16, Hkv=8, hd=128, prefix=1024, sample_layers=2,
                             min_seconds=3.0, max_reps=20):
    """One token through the bf16 decoder's layers (qkn_bf16_decoder.c:634-697) at
    the Qwen3-0.6B sizes, on the oracle's single-threaded restatement of them
    (decoder_oracle.Bf16Layer: truncating norms, projections, per-head norm,
    interleaved rotation, two-pass attention over a `prefix`-row cache of random
    bf16 rows, GeGLU, residual adds). The reference's own bf16 routines are
    static inside its decoder and are not built here, so this is a port baseline.
    Timed on `sample_layers` layers and scaled to n_layers."""
    from decoder_oracle import Bf16Block, Bf16Layer
    orc = Oracle()
    rng = np.random.default_rng(6)

    def bits(o, i):
        w = (rng.standard_normal((o, i)) / np.sqrt(i)).astype(np.float32)
        return (w.view(np.uint32) >> 16).astype(np.uint16)

    blk = Bf16Block(orc, n_layers=sample_layers, n_heads=H, n_kv_heads=Hkv, head_dim=hd, eps=1e-6,
                    rope_theta=1e6, rope_local_theta=0.0, rope_type=1, sliding_window=0, attn_logit_softcap=0.0,
                    capacity=prefix + max_reps + 4)
    weights = []
    for li in range(sample_layers):
        blk.set_layer(li, 0, (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32),
                      (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32))
        blk.ck[li, :prefix] = bits(prefix, Hkv * hd)
        blk.cv[li, :prefix] = bits(prefix, Hkv * hd)
        weights.append(dict(input_norm=(1 + 0.1 * rng.standard_normal(dim)).astype(np.float32),
                            wq=bits(H * hd, dim), wk=bits(Hkv * hd, dim), wv=bits(Hkv * hd, dim),
                            wo=bits(dim, H * hd), post_attn_norm=(1 + 0.1 * rng.standard_normal(dim)).astype(np.float32),
                            gate_up=bits(2 * inter, dim), down=bits(dim, inter)))
    layer = Bf16Layer(orc, blk, weights)
    x0 = bits(1, dim)
    reps, t = 0, 0.0
    while reps < 2 or (t < min_seconds and reps < max_reps):
        x = x0.copy()
        t0 = time.perf_counter()
        for li in range(sample_layers):
            x = layer.step(li, prefix, x)
        t += time.perf_counter() - t0
        reps += 1
    sec = t / reps * n_layers / sample_layers
    return {"value": round(1.0 / sec, 2), "unit": "tokens/s", "cores": 1, "kind": "port",
            "ms_per_token": round(sec * 1e3, 3), **host_facts(),
            "sample": "%d repetitions of one token through %d layers (%d cached tokens) on the oracle's "
                      "single-threaded bf16 layer, scaled to %d layers" % (reps, sample_layers, prefix, n_layers)}
