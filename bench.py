"""Benchmark of the MI355X attention path (one GPU).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--only NAME]

Headline line: causal prefill of Qwen3-ASR-0.6B (1536 tokens, 16 Q heads,
8 KV heads, head_dim 128, bf16 inputs, NeoX RoPE) in TFLOP/s of unmasked
attention work, with every input resident in HBM when the timed region
starts. A "step" is one smol_attn_prefill call (RoPE + cache append +
attention). Steps rotate over `layers` distinct caches and input sets
(>= 512 MB in total) so repeats stream HBM rather than the 256 MB
last-level cache.

The other workloads (decode, bidirectional, MQA decode, streaming chunk +
decode, and the decode step and prefill with the per-head Q/K RMSNorm fused
into the pre-pass) are measured the same way and reported under "detail",
as are the bf16-weight projections of one decoder layer (decode GEMV and
prefill GEMM, rotating over 28 layers of weights).

value / ms_per_step: wall clock over the timed steps with nothing but the
library's own launches in the stream.
roofline: the attention kernel's own duration, from the HIP events its
launch records around it (hipExtLaunchKernelGGL) on the context's stream, in
a second pass over the same steps; achieved = algorithmic flops (or bytes)
per launch / mean kernel time. profile_kernel_ms / profile_frac repeat the
figure from the rocprofv3 kernel trace summarised in profiles/, and traffic
is that summary's HBM bytes per launch.
cpu_baseline: the reference's own CPU attention (oracle/_ref, compiled from
the reference sources) on this host's cores, timed on the same workload.
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_MFMA_TFLOPS = 2500.0   # MI355X dense fp16/bf16 MFMA
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E
MALL_BYTES = 256 << 20


# the kernel each workload's roofline is quoted for (its profiles/<kernel>_<workload>.md summary)
DOMINANT = {"qwen06b_prefill": "k_attn_fb", "qwen06b_prefill_qknorm": "k_attn_fb", "siglip_bidir": "k_attn_win",
            "asr_encoder_bidir": "k_attn_win", "qwen06b_decode": "k_dec", "qwen06b_decode_qknorm": "k_dec",
            "gemma_mqa_decode": "k_dec", "qwen06b_decode_x28": "k_dec", "qwen17b_stream": "k_dec",
            "qwen06b_proj_decode": "k_gemv", "qwen06b_proj_prefill": "k_gemm"}


def profile_fields(workload):
    """Figures of the workload's dominant kernel as measured by rocprofv3 and summarised in
    profiles/<kernel>_<workload>.md: kernel_avg_ns (kernel trace), traffic_bytes_per_launch
    (FETCH_SIZE / WRITE_SIZE passes), mfma_busy_frac and mfma_flops_executed_per_launch (SQ
    counter passes); absent keys where the summary lacks them."""
    path = os.path.join(ROOT, "profiles", "%s_%s.md" % (DOMINANT.get(workload, "k_attn_fb").rstrip("_"), workload))
    out = {}
    try:
        for line in open(path):
            for key, conv in (("traffic_bytes_per_launch", int), ("kernel_avg_ns", float),
                              ("mfma_busy_frac", float), ("mfma_flops_executed_per_launch", int)):
                if line.startswith(key + ":"):
                    out[key] = conv(line.split(":")[1])
    except OSError:
        pass
    return out


def profiled(workload):
    """(kernel mean ns, HBM bytes per launch) of the workload's dominant kernel (profile_fields)"""
    f = profile_fields(workload)
    return f.get("kernel_avg_ns"), f.get("traffic_bytes_per_launch")


def layers_for(bytes_per_layer, lo=2, hi=64):
    n = -(-2 * MALL_BYTES // max(1, bytes_per_layer))
    return int(max(lo, min(hi, n)))


def time_steps(ctx, run, steps, warmup):
    """Wall time of `steps` steps with no instrumentation, then the kernels'
    own times from HIP events in a second pass over the same steps (the
    events sit between the launches, so they are kept out of the wall-clock
    pass)."""
    import torch
    for _ in range(warmup):
        run.step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        run.step()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ctx.timing_read()
    ctx.set_timing(True)
    for _ in range(steps):
        run.step()
    torch.cuda.synchronize()
    ctx.set_timing(False)
    kt = ctx.timing_read()
    return wall, kt


def measure(ctx, wl, steps, warmup, runner, layers=None):
    """Runs of earlier workloads hold device caches whose release (hipFree)
    synchronises the device; they are collected here, before the timing, and
    the collector stays off while the steps are timed."""
    import gc
    import torch
    gc.collect()
    torch.cuda.synchronize()
    x = wl.inputs()
    per_layer = getattr(wl, "algorithmic_bytes", lambda: 64 << 20)()
    n_layers = layers or layers_for(per_layer)
    run = runner.prepare(ctx, wl, x, layers=n_layers)
    gc.collect()
    gc.disable()
    try:
        wall, kt = time_steps(ctx, run, steps, warmup)
    finally:
        gc.enable()
    return x, run, n_layers, wall, kt


def measure_projections(ctx, sa, wl, steps, warmup):
    """One decoder layer's four projections per step (smol_linear_qkv_dev for Q/K/V,
    smol_linear_dev for o_proj, gate_up and down), rotating over wl.layers layers of
    distinct device weights (random bf16, generated on the device: values do not
    change the work). Wall clock per layer, then each kind's own launches timed by
    the HIP events the library records around them."""
    import gc
    import ctypes
    import torch
    lib = sa.load()
    gc.collect()
    torch.cuda.synchronize()
    g = torch.Generator(device="cuda")
    g.manual_seed(wl.seed)
    W = [{k: [(torch.randn((o, n_in), generator=g, device="cuda") * n_in ** -0.5).to(torch.bfloat16)
              for o in outs] for k, (n_in, outs) in wl.kinds.items()} for _ in range(wl.layers)]
    X = {k: torch.randn((wl.seq, n_in), generator=g, device="cuda") for k, (n_in, _) in wl.kinds.items()}
    Y = {k: [torch.empty((wl.seq, o), device="cuda") for o in outs] for k, (_, outs) in wl.kinds.items()}
    vp = ctypes.c_void_p
    calls = {}
    for k, (n_in, outs) in wl.kinds.items():
        x, ys = vp(X[k].data_ptr()), [vp(y.data_ptr()) for y in Y[k]]
        if k == "qkv":
            calls[k] = [(lib.smol_linear_qkv_dev, (ctx.h, ys[0], ys[1], ys[2], 0, x, 0,
                                                   vp(W[l][k][0].data_ptr()), vp(W[l][k][1].data_ptr()),
                                                   vp(W[l][k][2].data_ptr()), wl.seq, n_in, outs[0], outs[1]))
                        for l in range(wl.layers)]
        else:
            calls[k] = [(lib.smol_linear_dev, (ctx.h, ys[0], 0, x, 0, vp(W[l][k][0].data_ptr()), None, wl.seq,
                                               n_in, outs[0])) for l in range(wl.layers)]

    def layer(l):
        for k in wl.kinds:
            f, a = calls[k][l]
            if f(*a):
                raise RuntimeError(lib.smol_attn_last_error().decode())

    gc.disable()
    try:
        for i in range(warmup):
            layer(i % wl.layers)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for i in range(steps):
            layer(i % wl.layers)
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        per, launches = {}, {}
        ctx.timing_read()
        for k in wl.kinds:
            ctx.set_timing(True)
            for i in range(steps):
                f, a = calls[k][i % wl.layers]
                f(*a)
            torch.cuda.synchronize()
            ctx.set_timing(False)
            ms, cnt = ctx.timing_read()["other"]
            # per call: the GEMM path runs Q, K and V as three launches
            per[k] = ms / steps
            launches[k] = cnt / steps
    finally:
        gc.enable()
    d = {"config": wl.describe(), "ms_per_step": round(wall / steps * 1e3, 5),
         "step": "one layer: 4 projection calls"}
    tot_ms = sum(per.values())
    for k, ms in per.items():
        e = {"kernel_ms": round(ms, 5), "launches": launches[k], "bytes_per_call": wl.algorithmic_bytes(k)}
        if wl.seq <= 4:
            gbs = wl.algorithmic_bytes(k) / (ms * 1e-3) / 1e9
            e.update(GBps_kernel=round(gbs, 1), hbm_frac=round(gbs / PEAK_HBM_GBS, 4))
        else:
            tf = wl.flops(k) / (ms * 1e-3) / 1e12
            # an fp32 input runs as two bf16 products (x_hi, x_lo)
            e.update(tflops=round(tf, 2), mfma_frac_executed=round(2 * tf / PEAK_MFMA_TFLOPS, 4))
        d[k] = e
    if wl.seq <= 4:
        gbs = wl.algorithmic_bytes() / (tot_ms * 1e-3) / 1e9
        d.update(GBps_layer_kernels=round(gbs, 1), hbm_frac_layer=round(gbs / PEAK_HBM_GBS, 4),
                 GBps_layer_wall=round(wl.algorithmic_bytes() / (wall / steps) / 1e9, 1))
    else:
        tf = wl.flops() / (tot_ms * 1e-3) / 1e12
        d.update(tflops_layer_kernels=round(tf, 2), tflops_layer_wall=round(wl.flops() / (wall / steps) / 1e12, 2))
    del W, X, Y, calls
    return d


def measure_decoder(ctx, sa, steps, warmup, prefix=1024, n_layers=28, dim=1024, inter=3072):
    """Whole Qwen3-ASR-0.6B decoder layers on the device (smol_qkn_layer_*): the
    28 layers' caches filled by a `prefix`-token prefill, then single-token
    steps through all 28 layers (5 launches per layer). Random bf16 weights
    generated on the device (values do not change the work). Returns per-token
    and per-prefill-token figures."""
    import ctypes
    import gc
    import torch
    gc.collect()
    torch.cuda.synchronize()
    H, Hkv, hd = 16, 8, 128
    owner = ctypes.create_string_buffer(256)
    blk = sa.QknAttn(owner, n_layers=n_layers, n_heads=H, n_kv_heads=Hkv, head_dim=hd, eps=1e-6, rope_theta=1e6,
                     rope_local_theta=0.0, rope_type=0, sliding_window=0, attn_logit_softcap=0.0, bf16=0,
                     on_device=1, device=0, max_seq=prefix + steps + warmup + 8)
    g = torch.Generator(device="cuda")
    g.manual_seed(11)

    def proj(o, i):
        return (torch.randn((o, i), generator=g, device="cuda") * i ** -0.5).to(torch.bfloat16)

    def nw(n):
        return 1.0 + 0.1 * torch.randn((n,), generator=g, device="cuda")

    W = []
    for li in range(n_layers):
        blk.set_layer(li, 0, (1.0 + 0.1 * np.random.default_rng(li).standard_normal(hd)).astype(np.float32),
                      (1.0 + 0.1 * np.random.default_rng(100 + li).standard_normal(hd)).astype(np.float32))
        W.append(sa.QknLayerWeights(input_norm=nw(dim), wq=proj(H * hd, dim), wk=proj(Hkv * hd, dim),
                                    wv=proj(Hkv * hd, dim), wo=proj(dim, H * hd), post_attn_norm=nw(dim),
                                    pre_ffn_norm=None, post_ffn_norm=None, gate_up=proj(2 * inter, dim),
                                    down=proj(dim, inter)))
    lib = sa.load()
    addr = blk.addr
    x = torch.randn((prefix, dim), generator=g, device="cuda")
    x0 = x.clone()
    prefill_s = []
    for rep in range(3):  # the first pass pays one-time set-up (GEMM heuristics, buffers); a rewind to 0 repeats it
        x.copy_(x0)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for li in range(n_layers):
            if lib.smol_qkn_layer_prefill(addr, li, 0, prefix, ctypes.c_void_p(x.data_ptr()),
                                          ctypes.byref(W[li].s), dim, inter, 1):
                raise RuntimeError(lib.smol_attn_last_error().decode())
        blk.synchronize()
        prefill_s.append(time.perf_counter() - t0)
    prefill_cold = prefill_s[0]
    prefill_s = min(prefill_s[1:])
    xt = torch.randn((1, dim), generator=g, device="cuda")
    xp = ctypes.c_void_p(xt.data_ptr())

    def token(pos):
        for li in range(n_layers):
            if lib.smol_qkn_layer_forward(addr, li, pos, xp, ctypes.byref(W[li].s), dim, inter, 1):
                raise RuntimeError(lib.smol_attn_last_error().decode())

    pos = prefix
    gc.disable()
    try:
        for _ in range(warmup):
            token(pos)
            pos += 1
        blk.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            token(pos)
            pos += 1
        blk.synchronize()
        wall = time.perf_counter() - t0
    finally:
        gc.enable()
    # the same steps replayed from one HIP graph of the 28-layer step (two launches per token)
    graph = sa.QknStepGraph(blk, xt, W, dim, inter, 1, pos + warmup + steps + 8)
    gc.disable()
    try:
        for _ in range(warmup):
            graph.launch(pos)
            pos += 1
        blk.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            graph.launch(pos)
            pos += 1
        blk.synchronize()
        wall_graph = time.perf_counter() - t0
    finally:
        gc.enable()
        graph.close()
    wbytes = n_layers * 2 * dim * (H * hd + 2 * Hkv * hd + H * hd + 3 * inter)
    kv_bytes = n_layers * 2 * Hkv * hd * 2 * (prefix + warmup + steps / 2)
    ms_tok = wall / steps * 1e3
    d = {"config": {"workload": "qwen06b_decoder_step", "layers": n_layers, "hidden": dim, "heads": [H, Hkv, hd],
                    "intermediate": inter, "cached_tokens": prefix, "weights": "random bf16 on the device"},
         "ms_per_token": round(ms_tok, 4), "tokens_per_s": round(1e3 / ms_tok, 1),
         "launches_per_token": 5 * n_layers,
         "graph_ms_per_token": round(wall_graph / steps * 1e3, 4),
         "graph_tokens_per_s": round(steps / wall_graph, 1),
         "graph_launches_per_token": 2,
         "hbm_GBps_per_token": round((wbytes + kv_bytes) / (wall / steps) / 1e9, 1),
         "bytes_per_token": int(wbytes + kv_bytes),
         "prefill_tokens_per_s": round(prefix / prefill_s, 1),
         "prefill_ms_%d_tokens" % prefix: round(prefill_s * 1e3, 3),
         "prefill_ms_first_call": round(prefill_cold * 1e3, 3),
         "note": "decode: 28 layers per token, norms/activation/residuals fused into the projections, "
                 "one host wait per timed run; graph_*: the same step captured once "
                 "(smol_qkn_step_graph_create) and replayed per token; prefill: 28 smol_qkn_layer_prefill calls, each waiting for its "
                 "attention block"}
    blk.close()
    del W, x, xt
    return d


def measure_decoder_bf16(ctx, sa, steps, warmup, prefix=1024, n_layers=28, dim=1024, inter=3072):
    """The bf16 decoder's layers (smol_qkn_layer_*_bf16: bf16 residual stream,
    truncating projections and row operations, GeGLU) at the Qwen3-0.6B sizes
    of measure_decoder: a `prefix`-token prefill of the 28 layers, then
    single-token steps. Random bf16 weights generated on the device."""
    import ctypes
    import gc
    import torch
    gc.collect()
    torch.cuda.synchronize()
    H, Hkv, hd = 16, 8, 128
    owner = ctypes.create_string_buffer(256)
    blk = sa.QknAttn(owner, n_layers=n_layers, n_heads=H, n_kv_heads=Hkv, head_dim=hd, eps=1e-6, rope_theta=1e6,
                     rope_local_theta=0.0, rope_type=0, sliding_window=0, attn_logit_softcap=0.0, bf16=1,
                     on_device=1, device=0, max_seq=prefix + steps + warmup + 8)
    g = torch.Generator(device="cuda")
    g.manual_seed(12)

    def proj(o, i):
        return (torch.randn((o, i), generator=g, device="cuda") * i ** -0.5).to(torch.bfloat16)

    def nw(n):
        return 1.0 + 0.1 * torch.randn((n,), generator=g, device="cuda")

    W = []
    for li in range(n_layers):
        blk.set_layer(li, 0, (1.0 + 0.1 * np.random.default_rng(li).standard_normal(hd)).astype(np.float32),
                      (1.0 + 0.1 * np.random.default_rng(100 + li).standard_normal(hd)).astype(np.float32))
        W.append(sa.QknLayerWeights(input_norm=nw(dim), wq=proj(H * hd, dim), wk=proj(Hkv * hd, dim),
                                    wv=proj(Hkv * hd, dim), wo=proj(dim, H * hd), post_attn_norm=nw(dim),
                                    pre_ffn_norm=None, post_ffn_norm=None, gate_up=proj(2 * inter, dim),
                                    down=proj(dim, inter)))
    lib = sa.load()
    addr = blk.addr
    x0 = torch.randn((prefix, dim), generator=g, device="cuda").to(torch.bfloat16).view(torch.int16)
    x = x0.clone()
    prefill_s = []
    for rep in range(3):
        x.copy_(x0)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for li in range(n_layers):
            if lib.smol_qkn_layer_prefill_bf16(addr, li, 0, prefix, ctypes.c_void_p(x.data_ptr()),
                                               ctypes.byref(W[li].s), dim, inter):
                raise RuntimeError(lib.smol_attn_last_error().decode())
        blk.synchronize()
        prefill_s.append(time.perf_counter() - t0)
    prefill_s = min(prefill_s[1:])
    xt = torch.randn((1, dim), generator=g, device="cuda").to(torch.bfloat16).view(torch.int16)
    xp = ctypes.c_void_p(xt.data_ptr())

    def token(pos):
        for li in range(n_layers):
            if lib.smol_qkn_layer_forward_bf16(addr, li, pos, xp, ctypes.byref(W[li].s), dim, inter):
                raise RuntimeError(lib.smol_attn_last_error().decode())

    pos = prefix
    gc.disable()
    try:
        for _ in range(warmup):
            token(pos)
            pos += 1
        blk.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            token(pos)
            pos += 1
        blk.synchronize()
        wall = time.perf_counter() - t0
    finally:
        gc.enable()
    ms_tok = wall / steps * 1e3
    d = {"config": {"workload": "qwen06b_bf16_decoder_step", "layers": n_layers, "hidden": dim,
                    "heads": [H, Hkv, hd], "intermediate": inter, "cached_tokens": prefix,
                    "activations": "bf16 (truncating, GeGLU)", "weights": "random bf16 on the device"},
         "ms_per_token": round(ms_tok, 4), "tokens_per_s": round(1e3 / ms_tok, 1),
         "prefill_tokens_per_s": round(prefix / prefill_s, 1),
         "prefill_ms_%d_tokens" % prefix: round(prefill_s * 1e3, 3),
         "note": "the bf16 decoder's layer order (qkn_bf16_decoder.c:482-571, 634-697) at the fp32 step's "
                 "sizes"}
    blk.close()
    del W, x, xt
    return d


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--only", default=None, help="measure only this workload")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="first run 5 plain device copies of MIB MiB (a known-size reference for "
                         "the HBM byte counters of a profiler run)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: the library has no multi-GPU path (the attention would shard "
              "by KV head with no exchange inside attention). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import torch
    import __graft_entry__
    __graft_entry__.load_package()
    from smol_genius_amd import runner, smol_attn as sa, workloads

    sa.load()
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    if args.copy_calibration:
        n = args.copy_calibration << 18
        src = torch.ones(n, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print("copy calibration: 5 copies of %d MiB (%d bytes read + %d written per copy)"
              % (args.copy_calibration, 4 * n, 4 * n), flush=True)
        del src, dst
    ctx = sa.Context(0)
    wls = workloads.all_workloads()
    steps, warmup = args.steps, args.warmup

    # ---------------- headline: causal prefill
    main_wl = wls["qwen06b_prefill"]
    detail = {}
    if args.only in (None, main_wl.name):
        x, run, n_layers, wall, kt = measure(ctx, main_wl, steps, warmup, runner)
        del x, run
        flops = main_wl.flops()
        ms_step = wall / steps * 1e3
        attn_ms = kt["attn"][0] / max(1, kt["attn"][1])
        prep_ms = kt["prep"][0] / max(1, kt["prep"][1])
        value = flops / (wall / steps) / 1e12
        achieved = flops / (attn_ms * 1e-3) / 1e12
        prof_ns, traffic = profiled(main_wl.name)
        head = {
            "metric": "prefill attn TFLOP/s (causal, Qwen3-ASR-0.6B 1536 tokens)",
            "value": round(value, 3), "unit": "TFLOP/s", "n_gpus": 1, "steps": steps, "warmup": warmup,
            "ms_per_step": round(ms_step, 5), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
            "dtype": "f16 MFMA operands as hi + lo pairs (Q, K and P: QK^T and P.V to about 21 bits), f32 "
                     "softmax/accumulate (bf16 inputs and KV cache)",
            "data": "synthetic (seeded N(0,1) bf16 Q/K/V)",
            "config": dict(main_wl.describe(), layers_rotated=n_layers, parallelism="single GPU"),
            "roofline": {"bound": "mfma", "kernel": "k_attn_fb", "achieved": round(achieved, 3),
                         "peak": PEAK_MFMA_TFLOPS, "unit": "TFLOP/s", "frac": round(achieved / PEAK_MFMA_TFLOPS, 5),
                         "traffic": traffic,
                         "traffic_source": "profiles/k_attn_fb_qwen06b_prefill.md (rocprofv3 FETCH_SIZE and "
                                           "WRITE_SIZE, copy-calibrated)",
                         "kernel_ms": round(attn_ms, 5), "prep_kernel_ms": round(prep_ms, 5),
                         "kernel_ms_source": "HIP events recorded by the kernel's own launch, live in this run",
                         "flops_per_launch": flops},
        }
        if prof_ns:
            pa = flops / (prof_ns * 1e-9) / 1e12
            head["roofline"].update(profile_kernel_ms=round(prof_ns * 1e-6, 5), profile_achieved=round(pa, 3),
                                    profile_frac=round(pa / PEAK_MFMA_TFLOPS, 5))
        pf = profile_fields(main_wl.name)
        if "mfma_busy_frac" in pf:
            # matrix-core busy cycles per SIMD over the kernel's cycles (SQ counters), and the MFMA work
            # executed per launch, hi/lo products included (useful flops are `flops_per_launch`)
            head["roofline"].update(mfma_busy=pf["mfma_busy_frac"],
                                    mfma_flops_executed_per_launch=pf.get("mfma_flops_executed_per_launch"),
                                    mfma_busy_source="profiles/k_attn_fb_qwen06b_prefill.md (SQ_VALU_MFMA_BUSY_CYCLES)")
        # the same step with SMOL_OPT_QK_FP16 (single fp16 Q and K operands, P in fp16: faster, within
        # the bar for logits up to about sigma 1.4 only)
        ctx.set_option(sa.OPT_QK_FP16, 1)
        x, run, n_layers16, wall16, kt16 = measure(ctx, main_wl, steps, warmup, runner)
        ctx.set_option(sa.OPT_QK_FP16, 0)
        del x, run
        a16 = kt16["attn"][0] / max(1, kt16["attn"][1])
        detail["qwen06b_prefill_fp16qk"] = {
            "config": dict(main_wl.describe(), option="SMOL_OPT_QK_FP16=1"),
            "ms_per_step": round(wall16 / steps * 1e3, 5), "tflops_step": round(flops / (wall16 / steps) / 1e12, 3),
            "attn_kernel_ms": round(a16, 5), "tflops_kernel": round(flops / (a16 * 1e-3) / 1e12, 3),
            "mfma_frac_kernel": round(flops / (a16 * 1e-3) / 1e12 / PEAK_MFMA_TFLOPS, 5),
            "note": "not the default: single fp16 Q/K/P operands meet the bar only for logits up to about sigma 1.4"}
    else:
        head = None

    # CPU baselines: the reference's own CPU attention (oracle/_ref) on this host, after each
    # workload's GPU timing, on a bounded sample of the same inputs
    cpu_mod = None
    if not args.no_cpu:
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import cpu_baseline as cpu_mod

    # ---------------- the other workloads
    for name in ["qwen06b_decode", "gemma_mqa_decode", "siglip_bidir", "qwen17b_stream", "qwen06b_decode_qknorm",
                 "qwen06b_prefill_qknorm", "asr_encoder_bidir", "qwen06b_decode_x28"]:
        if args.only not in (None, name):
            continue
        wl = wls[name]
        if name == "qwen17b_stream":
            x, run, n_layers, wall, kt = measure(ctx, wl, max(3, steps // 10), max(1, warmup // 5), runner,
                                                 layers=8)
            del x, run
            n = max(3, steps // 10)
            attn_ms, attn_n = kt["attn"]
            # per step: 1 chunk launch + `steps` decode launches of the attention kernel
            detail[name] = {"config": wl.describe(), "ms_per_step": round(wall / n * 1e3, 4),
                            "attn_kernel_ms_total_per_step": round(attn_ms / n, 4),
                            "decode_GBps_path": round(wl.decode_bytes() / (wall / n) / 1e9, 1),
                            "note": "wall time per step includes 65 launches and their host dispatch"}
            if cpu_mod:
                detail[name]["cpu_baseline"] = cpu_mod.stream_sample(wl, wl.inputs())
            continue
        x, run, n_layers, wall, kt = measure(ctx, wl, steps, warmup, runner)
        del x, run
        attn_ms = kt["attn"][0] / max(1, kt["attn"][1])
        prep_ms = kt["prep"][0] / max(1, kt["prep"][1])
        d = {"config": wl.describe(), "layers_rotated": n_layers, "ms_per_step": round(wall / steps * 1e3, 5),
             "attn_kernel_ms": round(attn_ms, 5), "prep_kernel_ms": round(prep_ms, 5)}
        if name == "qwen06b_prefill_qknorm":
            f = wl.flops()
            d.update(tflops_kernel=round(f / (attn_ms * 1e-3) / 1e12, 3),
                     tflops_step=round(f / (wall / steps) / 1e12, 3))
        elif name in ("siglip_bidir", "asr_encoder_bidir"):
            f = wl.flops()
            d.update(tflops_kernel=round(f / (attn_ms * 1e-3) / 1e12, 3),
                     mfma_frac=round(f / (attn_ms * 1e-3) / 1e12 / PEAK_MFMA_TFLOPS, 5),
                     hbm_GBps_kernel=round(wl.algorithmic_bytes() / (attn_ms * 1e-3) / 1e9, 1))
        else:
            b = wl.algorithmic_bytes()
            d.update(GBps_kernel=round(b / (attn_ms * 1e-3) / 1e9, 1),
                     hbm_frac_kernel=round(b / (attn_ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 5),
                     GBps_path=round(b / ((attn_ms + prep_ms) * 1e-3) / 1e9, 1),
                     bytes_per_launch=b)
        pf = profile_fields(name)
        if "kernel_avg_ns" in pf:
            d["profile_kernel_ms"] = round(pf["kernel_avg_ns"] * 1e-6, 5)
            d["profile_traffic_bytes"] = pf.get("traffic_bytes_per_launch")
        if "mfma_busy_frac" in pf:
            d["profile_mfma_busy"] = pf["mfma_busy_frac"]
        if cpu_mod:
            if isinstance(wl, workloads.Decode):
                d["cpu_baseline"] = cpu_mod.decode_sample(wl, wl.inputs())
            elif isinstance(wl, workloads.Bidir):
                d["cpu_baseline"] = cpu_mod.bidir_sample(wl, wl.inputs())
            elif isinstance(wl, workloads.Prefill):
                d["cpu_baseline"] = cpu_mod.prefill_sample(wl, wl.inputs(), min_seconds=3.0)
        detail[name] = d

    # ---------------- the decoder layer's bf16-weight projections (decode GEMV, prefill GEMM)
    for name in ["qwen06b_proj_decode", "qwen06b_proj_prefill"]:
        if args.only not in (None, name):
            continue
        wl = wls[name]
        n = steps if wl.seq == 1 else max(5, steps // 5)
        d = measure_projections(ctx, sa, wl, n, max(2, warmup // 2))
        if cpu_mod:
            d["cpu_baseline"] = cpu_mod.projections_sample(wl, wl.inputs())
        detail[name] = d

    # ---------------- whole decoder layers on the device (28-layer token step)
    if args.only in (None, "qwen06b_decoder_step"):
        d = measure_decoder(ctx, sa, max(10, steps // 5), max(2, warmup // 2))
        if cpu_mod:
            d["cpu_baseline"] = cpu_mod.decoder_step_sample()
        detail["qwen06b_decoder_step"] = d
    if args.only in (None, "qwen06b_bf16_decoder_step"):
        d = measure_decoder_bf16(ctx, sa, max(10, steps // 5), max(2, warmup // 2))
        if cpu_mod:
            d["cpu_baseline"] = cpu_mod.bf16_decoder_step_sample()
        detail["qwen06b_bf16_decoder_step"] = d

    # ---------------- CPU baseline of the headline (reference CPU attention on this host)
    if cpu_mod and head is not None:
        head["cpu_baseline"] = cpu_mod.prefill_sample(main_wl, main_wl.inputs())
    if head is None:
        head = {"metric": "detail only", "value": None}
    head["detail"] = detail
    print(json.dumps(head), flush=True)
    ctx.close()


if __name__ == "__main__":
    main()
