"""HIP path against the CPU oracle (and the compiled reference's golden vectors), on the GPU.

Every case prints its name before it runs. The bar is |gpu - cpu| <= 2e-3 +
1e-2 |cpu| for every element (conftest.ATOL / RTOL), on fp32 outputs.
"""
import numpy as np
import pytest

from conftest import assert_parity, pkg, synth  # noqa: F401
from gen_golden_inputs import bidir_inputs, causal_inputs

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module")
def sa():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from smol_genius_amd import smol_attn
    smol_attn.load()
    return smol_attn


@pytest.fixture(scope="module")
def ctx(sa):
    c = sa.Context(0)
    yield c
    c.close()


@pytest.fixture
def opts(ctx):
    """Sets context options (SMOL_OPT_*) for one test and restores the defaults after it."""
    touched = []

    def set_option(option, value):
        ctx.set_option(option, value)
        touched.append(option)

    yield set_option
    for o in touched:
        ctx.set_option(o, 0)


@pytest.fixture(scope="module")
def wo():
    import workload_oracle
    return workload_oracle


def dev(a, bf16=False):
    if bf16:
        return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).cuda().view(torch.bfloat16)
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).cuda()


def widen(b):
    return synth.bf16_bits_to_f32(b)


# ------------------------------------------------------------- full workloads

@pytest.mark.parametrize("name", ["qwen06b_decode", "qwen06b_prefill", "siglip_bidir", "gemma_mqa_decode",
                                  "qwen17b_stream", "qwen06b_decode_qknorm", "qwen06b_prefill_qknorm",
                                  "asr_encoder_bidir", "qwen06b_decode_x28"])
def test_workload_full_size(ctx, oracle, wo, name):
    from smol_genius_amd import runner, workloads
    print("case", name, flush=True)
    wl = workloads.all_workloads()[name]
    x = wl.inputs()
    r = runner.prepare(ctx, wl, x)
    r.step()
    got = r.outputs()
    want = wo.evaluate(oracle, wl, x)
    if isinstance(want, tuple):
        a = assert_parity(got[0], want[0], name + " chunk")
        b = assert_parity(got[1], want[1], name + " decode")
        print(name, "chunk", a, "decode", b)
    else:
        print(name, assert_parity(got, want, name))
    # a second pass over the same inputs gives the same bits (appends are idempotent)
    r.step()
    again = r.outputs()
    if isinstance(got, list):
        for u, w in zip(got, again):
            np.testing.assert_array_equal(u, w)
    else:
        np.testing.assert_array_equal(got, again)


# ---------------------------------------------- reference golden vectors

def test_golden_causal_through_reference_signature(sa, golden):
    meta, data = golden
    for c in meta["causal"]:
        print("golden", c["name"], flush=True)
        Q, K, V = causal_inputs(c["seed"], c["Hq"], c["Hkv"], c["hd"], c["seq_q"], c["seq_k"])
        out = np.full((c["seq_q"], c["Hq"] * c["hd"]), np.nan, np.float32)
        args = (out, Q, K, V, c["seq_q"], c["seq_k"], c["Hq"], c["Hkv"], c["hd"], c["scale"], c["q_offset"])
        kind = c["kind"]
        if kind == "swa_softcap":
            sa.smol_sliding_window_attention_softcap(*args, c["window"], c["cap"])
        elif kind == "swa":
            sa.smol_sliding_window_attention(*args, c["window"])
        elif kind == "softcap":
            sa.smol_causal_attention_softcap(*args, c["cap"])
        else:
            sa.smol_causal_attention(*args)
        assert_parity(out, data[c["name"]], c["name"])


def test_golden_bidirectional_through_reference_signature(sa, golden):
    meta, data = golden
    for b in meta["bidir"]:
        print("golden", b["name"], flush=True)
        ws = b["window_starts"]
        seq = ws[-1]
        Q, K, V = bidir_inputs(b["seed"], b["H"], b["hd"], seq, b["std"])
        out = np.zeros((seq, b["H"] * b["hd"]), np.float32)
        sa.smol_bidirectional_attention(out, Q, K, V, seq, b["H"], b["hd"], b["scale"], ws, len(ws) - 1)
        assert_parity(out, data[b["name"]], b["name"])


def test_golden_rope_through_reference_signature(sa, golden):
    meta, data = golden
    for r in meta["rope"]:
        n = len(r["positions"])
        pos = np.array(r["positions"], np.int32)
        c = np.zeros((n, r["hd"]), np.float32)
        s = np.zeros_like(c)
        (sa.smol_compute_rope_interleaved if r["interleaved"] else sa.smol_compute_rope_neox)(
            c, s, pos, n, r["hd"], r["theta"])
        tol = 2e-7 * pos[:, None].astype(np.float64) + 2e-7
        assert (np.abs(c - data[r["tag"] + "_cos"]) <= tol).all(), r["tag"]
        x = synth.normal(r["seed"], (n, 3 * r["hd"]))
        (sa.smol_apply_rope_interleaved if r["interleaved"] else sa.smol_apply_rope_neox)(
            x, data[r["tag"] + "_cos"], data[r["tag"] + "_sin"], n, 3, r["hd"])
        np.testing.assert_allclose(x, data[r["tag"] + "_applied"], rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("hd", [1, 16, 32, 65, 100, 112, 200, 255])
def test_reference_signatures_any_head_dim(sa, oracle, hd):
    """The drop-ins take any head_dim up to 256 (zero-padded to a kernel
    size); the bidirectional call keeps the rows before its first window."""
    print("any head_dim", hd, flush=True)
    Hq, Hkv, sq, sk = 4, 2, 37, 90
    Q, K, V = synth.normal(61, (sq, Hq * hd)), synth.normal(62, (sk, Hkv * hd)), synth.normal(63, (sk, Hkv * hd))
    sc = 1.0 / np.sqrt(hd)
    out = np.full((sq, Hq * hd), np.nan, np.float32)
    sa.smol_sliding_window_attention_softcap(out, Q, K, V, sq, sk, Hq, Hkv, hd, sc, sk - sq, 40, 20.0)
    assert_parity(out, oracle.causal_attention(Q, K, V, sq, sk, Hq, Hkv, hd, sc, sk - sq, window=40, cap=20.0),
                  "causal hd %d" % hd)
    ws = [5, 40, 41, 90]
    out = synth.normal(64, (sk, Hkv * hd)).astype(np.float32)
    init = out.copy()
    V2 = synth.normal(65, (sk, Hkv * hd))
    sa.smol_bidirectional_attention(out, K, V, V2, sk, Hkv, hd, sc, ws, 3)
    want = oracle.bidirectional_attention(K, V, V2, sk, Hkv, hd, sc, ws)
    np.testing.assert_array_equal(out[:5], init[:5])
    assert_parity(out[5:], want[5:], "bidirectional hd %d" % hd)


# ------------------------------------------------------------ shapes and edges

CAUSAL_SHAPES = [  # Hq, Hkv, hd, seq_q, seq_k, q_offset, bf16
    (4, 4, 64, 33, 33, 0, False), (8, 2, 72, 17, 50, 33, True), (6, 2, 80, 5, 70, 65, False),
    (4, 1, 96, 40, 40, 0, True), (16, 8, 128, 1, 1, 0, False), (16, 8, 128, 70, 130, 60, True),
    (8, 1, 256, 3, 200, 197, False), (2, 2, 256, 48, 48, 0, True), (32, 2, 128, 2, 90, 88, False),
    (4, 2, 64, 9, 20, -3, False), (4, 2, 128, 6, 10, 30, False), (16, 16, 64, 100, 300, 200, True),
    (4, 2, 256, 70, 70, 0, True), (8, 4, 128, 40, 200, 160, False), (6, 3, 96, 130, 130, 0, True),
]


@pytest.mark.parametrize("shape", CAUSAL_SHAPES)
def test_causal_shapes(ctx, sa, oracle, shape):
    Hq, Hkv, hd, sq, sk, qo, bf = shape
    print("causal", shape, flush=True)
    Q = synth.normal(7, (sq, Hq * hd))
    K = synth.normal(8, (sk, Hkv * hd))
    V = synth.normal(9, (sk, Hkv * hd))
    if bf:
        Q, K, V = (synth.round_bf16(a) for a in (Q, K, V))
    sc = 1.0 / np.sqrt(hd)
    conv = (lambda a: dev(synth.f32_to_bf16_bits(a), True)) if bf else dev
    out = sa.causal(ctx, conv(Q), conv(K), conv(V), sq, sk, Hq, Hkv, hd, sc, qo)
    got = out.cpu().numpy()
    want = oracle.causal_attention(Q, K, V, sq, sk, Hq, Hkv, hd, sc, qo)
    assert_parity(got, want, str(shape))
    if qo < 0:
        assert not got[:-qo].any()


@pytest.mark.parametrize("shape", [s for s in CAUSAL_SHAPES if s[2] <= 128 and s[5] >= 0])
def test_causal_shapes_fb(ctx, sa, oracle, shape, opts):
    """The same cases through k_attn_fb (one workgroup per 64-row tile, taken
    here whatever the call's size)."""
    opts(sa.OPT_PREFILL_KERNEL, 1)
    test_causal_shapes(ctx, sa, oracle, shape)


@pytest.mark.parametrize("window,cap", [(16, 0.0), (0, 2.0), (40, 1.5), (1, 0.0), (7, 50.0)])
def test_window_softcap_fb(ctx, sa, oracle, window, cap, opts):
    opts(sa.OPT_PREFILL_KERNEL, 1)
    test_window_softcap(ctx, sa, oracle, window, cap)


@pytest.mark.parametrize("kernel", [1, 2], ids=["fb", "fa"])
def test_bidirectional_ragged_staged(ctx, sa, oracle, opts, kernel):
    """The pre-pass + k_attn_fb / k_attn_fa path of bidirectional calls."""
    opts(sa.OPT_BIDIR_WIN, -1)
    opts(sa.OPT_PREFILL_KERNEL, kernel)
    test_bidirectional_ragged(ctx, sa, oracle)


@pytest.mark.parametrize("hd", [64, 72, 80, 96, 128])
@pytest.mark.parametrize("bf", [False, True], ids=["f32", "bf16"])
def test_window_kernel(ctx, sa, oracle, opts, hd, bf):
    """k_attn_win: windows resident in LDS, read from fp32 or bf16 inputs;
    ragged windows (1, 31, 33 keys ...), a window at the LDS limit of the
    head_dim, with 128-row tiles over every key and with 64-row tiles over
    two key groups (a 1-key window leaves the second group without slabs),
    and the same call through the staged path for comparison. A window past
    the limit takes the staged path by itself."""
    # the LDS holds 160 KB of 32-key slabs; with the precise products (the
    # default) a bf16 slab is K and V as rows of 32 x 256 B, an fp32 one K hi
    # and K lo (2 x 32 x 256 B) and V^T (16 ceil(hd / 16) rows of 64 B)
    slab = 2 * 8192 if bf else 2 * 8192 + 16 * ((hd + 15) // 16) * 64
    lim = (160 * 1024 // slab) * 32
    assert lim >= 192
    H = 3
    for ws in ([0, 1, 32, 65, 130, 200], [7, 7 + lim], [0, lim + 1, lim + 40]):
        print("window kernel", hd, bf, ws, flush=True)
        seq = ws[-1]
        Q, K, V = (synth.normal(70 + i, (seq, H * hd)) for i in range(3))
        if bf:
            Q, K, V = (synth.round_bf16(a) for a in (Q, K, V))
        conv = (lambda a: dev(synth.f32_to_bf16_bits(a), True)) if bf else dev
        sc = 1.0 / np.sqrt(hd)
        want = oracle.bidirectional_attention(Q, K, V, seq, H, hd, sc, ws)
        res = []
        for w, ks in ((1, 1), (1, 2), (-1, 0)):
            opts(sa.OPT_BIDIR_WIN, w)
            opts(sa.OPT_WIN_KSPLIT, ks)
            init = synth.normal(79, (seq, H * hd)).astype(np.float32)
            out = dev(init)
            got = sa.bidirectional(ctx, conv(Q), conv(K), conv(V), seq, H, hd, sc, ws, out=out).cpu().numpy()
            np.testing.assert_array_equal(got[:ws[0]], init[:ws[0]])
            assert_parity(got[ws[0]:], want[ws[0]:], "win %d ksplit %d hd %d %s" % (w, ks, hd, ws))
            res.append(got)
        opts(sa.OPT_BIDIR_WIN, 0)
        opts(sa.OPT_WIN_KSPLIT, 0)


@pytest.mark.parametrize("case", [  # Hq, Hkv, hd, seq, window, bf16 / bidirectional window starts
    (16, 8, 128, 1536, 0, True), (32, 4, 96, 700, 0, False), (16, 4, 64, 1100, 300, False),
    (16, 16, 64, [0, 100, 700, 750, 1600, 1601, 2000]), (12, 12, 72, [3, 500, 1025, 1090, 1700, 1800]),
])
def test_fb_tile_lists(ctx, sa, oracle, case, opts):
    """More 64-row tiles than compute units: each k_attn_fb workgroup runs a
    list of tiles (longest first to the least loaded list). Every tile is
    computed as it is with one workgroup per tile, so the two launches agree
    bit for bit, and both meet the oracle."""
    print("fb lists", case, flush=True)
    opts(sa.OPT_PREFILL_KERNEL, 1)
    opts(sa.OPT_BIDIR_WIN, -1)
    bidir = isinstance(case[3], list)
    if bidir:
        H, _, hd, ws = case
        seq, Hq, Hkv = ws[-1], H, H
        Q, K, V = (synth.round_bf16(synth.normal(60 + i, (seq, H * hd))) for i in range(3))
        bf = True
    else:
        Hq, Hkv, hd, seq, window, bf = case
        Q = synth.normal(63, (seq, Hq * hd))
        K = synth.normal(64, (seq, Hkv * hd))
        V = synth.normal(65, (seq, Hkv * hd))
        if bf:
            Q, K, V = (synth.round_bf16(a) for a in (Q, K, V))
    sc = 1.0 / np.sqrt(hd)
    conv = (lambda a: dev(synth.f32_to_bf16_bits(a), True)) if bf else dev

    def run():
        if bidir:
            out = torch.zeros((seq, Hq * hd), dtype=torch.float32, device="cuda")
            return sa.bidirectional(ctx, conv(Q), conv(K), conv(V), seq, Hq, hd, sc, ws, out=out).cpu().numpy()
        return sa.causal(ctx, conv(Q), conv(K), conv(V), seq, seq, Hq, Hkv, hd, sc, 0, window=window).cpu().numpy()

    lists = run()
    opts(sa.OPT_FB_LISTS, -1)
    per_tile = run()
    assert np.array_equal(lists, per_tile)
    if bidir:
        want = oracle.bidirectional_attention(Q, K, V, seq, Hq, hd, sc, ws)
        assert_parity(lists[ws[0]:], want[ws[0]:], "fb lists %s" % (case,))
    else:
        want = oracle.causal_attention(Q, K, V, seq, seq, Hq, Hkv, hd, sc, 0, window=window)
        assert_parity(lists, want, "fb lists %s" % (case,))


@pytest.mark.parametrize("window,cap", [(16, 0.0), (0, 2.0), (40, 1.5), (1, 0.0), (7, 50.0)])
def test_window_softcap(ctx, sa, oracle, window, cap):
    # small caps so that tanh actually bends the N(0, 1) scores
    Hq, Hkv, hd, sq, sk, qo = 8, 4, 128, 37, 150, 113
    Q = synth.normal(17, (sq, Hq * hd))
    K = synth.normal(18, (sk, Hkv * hd))
    V = synth.normal(19, (sk, Hkv * hd))
    sc = 1.0 / np.sqrt(hd)
    got = sa.causal(ctx, dev(Q), dev(K), dev(V), sq, sk, Hq, Hkv, hd, sc, qo, window=window, cap=cap).cpu().numpy()
    want = oracle.causal_attention(Q, K, V, sq, sk, Hq, Hkv, hd, sc, qo, window=window, cap=cap)
    assert_parity(got, want, "window %d cap %g" % (window, cap))


def test_bidirectional_ragged(ctx, sa, oracle):
    for H, hd, ws in [(3, 72, [0, 1, 33, 34, 100, 257]), (2, 64, [5, 40, 41]), (4, 128, [0, 64, 128])]:
        seq = ws[-1]
        Q, K, V = (synth.round_bf16(synth.normal(30 + i, (seq, H * hd))) for i in range(3))
        sc = 1.0 / np.sqrt(hd)
        out = torch.zeros((seq, H * hd), dtype=torch.float32, device="cuda")
        b = lambda a: dev(synth.f32_to_bf16_bits(a), True)  # noqa: E731
        got = sa.bidirectional(ctx, b(Q), b(K), b(V), seq, H, hd, sc, ws, out=out).cpu().numpy()
        want = oracle.bidirectional_attention(Q, K, V, seq, H, hd, sc, ws)
        lo = ws[0]
        assert_parity(got[lo:], want[lo:], "bidir %s" % ws)
        assert not got[:lo].any()


@pytest.mark.parametrize("P,S", [(0, 1), (0, 33), (5, 7), (31, 1), (32, 32), (40, 64), (63, 2), (100, 26),
                                 (64, 100), (250, 130)])
@pytest.mark.parametrize("rope_type", [0, 1])
def test_prefill_chunks(ctx, sa, oracle, wo, P, S, rope_type):
    from smol_genius_amd.workloads import Prefill
    print("prefill", P, S, rope_type, flush=True)
    wl = Prefill("t", 8, 2, 128, P, S, 1e4 if rope_type else 1e6, seed=50 + P + S, in_bf16=(S % 2 == 0))
    wl.rope_type = rope_type
    x = wl.inputs()
    kv = sa.KVCache(ctx, 1, 1, 2, 128, P + S)
    if P:
        kv.write(0, 0, 0, x["cache_k"], x["cache_v"])
    rope = sa.RopeTable(ctx, 128, wl.theta, rope_type)
    bf = wl.in_bf16
    got = sa.prefill(ctx, kv, 0, 0, rope, P, dev(x["q"], bf), dev(x["k"], bf), dev(x["v"], bf), 8, wl.scale)
    want = wo.prefill(oracle, wl, x)
    assert_parity(got.cpu().numpy(), want, "prefill P=%d S=%d" % (P, S))
    # the cache now holds the rotated new K (bf16, nearest even) and V
    k_rows, v_rows = kv.read(0, 0, P, S)
    pos = np.arange(P, P + S)
    c, s = wo.rope_rows(oracle, pos, 128, wl.theta, rope_type == 1)
    kn = oracle.apply_rope(wo._as_f32(x["k"]), c, s, S, 2, 128, rope_type == 1)
    exact = (k_rows == synth.f32_to_bf16_bits(kn)).mean()
    assert exact > 0.999, exact
    np.testing.assert_array_equal(v_rows, synth.f32_to_bf16_bits(wo._as_f32(x["v"])))


@pytest.mark.parametrize("hd", [64, 72, 80, 96, 128, 256])
@pytest.mark.parametrize("rope_type", [0, 1])
@pytest.mark.parametrize("bf", [False, True])
def test_prefill_rope_every_head_dim(ctx, sa, oracle, wo, hd, rope_type, bf):
    """The pre-pass's three NeoX partner paths (lane shuffle at hd 64/128/256,
    partner chunks at 80/96, partner elements at 72) and the interleaved
    pairing, through a chunk on a prefix (fa) and a decode step (dec)."""
    from smol_genius_amd.workloads import Prefill
    for P, S in [(37, 45), (40, 1)]:
        print("prefill rope", hd, rope_type, bf, P, S, flush=True)
        wl = Prefill("t", 4, 2, hd, P, S, 1e4, seed=90 + hd + P, in_bf16=bf)
        wl.rope_type = rope_type
        x = wl.inputs()
        kv = sa.KVCache(ctx, 1, 1, 2, hd, P + S)
        kv.write(0, 0, 0, x["cache_k"], x["cache_v"])
        rope = sa.RopeTable(ctx, hd, wl.theta, rope_type)
        got = sa.prefill(ctx, kv, 0, 0, rope, P, dev(x["q"], bf), dev(x["k"], bf), dev(x["v"], bf), 4, wl.scale)
        assert_parity(got.cpu().numpy(), wo.prefill(oracle, wl, x), "hd %d rope %d P=%d S=%d" % (hd, rope_type, P, S))
        k_rows, _ = kv.read(0, 0, P, S)
        c, s = wo.rope_rows(oracle, np.arange(P, P + S), hd, wl.theta, rope_type == 1)
        kn = oracle.apply_rope(wo._as_f32(x["k"]), c, s, S, 2, hd, rope_type == 1)
        assert (k_rows == synth.f32_to_bf16_bits(kn)).mean() > 0.999


@pytest.mark.parametrize("positions", [[0], [1], [31], [32], [33], [64, 0, 95, 7], [1000, 31, 4095]])
def test_decode_positions(ctx, sa, oracle, wo, positions):
    from smol_genius_amd import runner
    from smol_genius_amd.workloads import Decode
    print("decode", positions, flush=True)
    for hq, hkv, hd, rt in [(16, 8, 128, 0), (8, 1, 256, 1), (4, 4, 64, 0)]:
        wl = Decode("t", hq, hkv, hd, [p + 1 for p in positions], 1e4, rt, seed=60 + len(positions))
        x = wl.inputs()
        r = runner.prepare(ctx, wl, x)
        r.step()
        assert_parity(r.outputs(), wo.decode(oracle, wl, x), "decode %s hd %d" % (positions, hd))


@pytest.mark.parametrize("positions", [[0], [33], [64, 0, 95, 7], [1000, 31, 4095]])
@pytest.mark.parametrize("slabs", [1, 3])
def test_decode_positions_split(ctx, sa, oracle, wo, positions, slabs, opts):
    """The same cases with every k_dec workgroup holding 1 or 3 key slabs, so
    the long sequences split into up to 32 workgroups merged through the
    flags (1000 keys in 1-slab splits: the 32-split cap)."""
    opts(sa.OPT_DEC_SLABS, slabs)
    test_decode_positions(ctx, sa, oracle, wo, positions)


@pytest.mark.parametrize("positions", [[0], [33], [64, 0, 95, 7], [1000, 31, 1400]])
def test_decode_positions_whole(ctx, sa, oracle, wo, positions, opts):
    """The same cases with one k_dec workgroup per (sequence, kv head) (no
    merge), with eight waves where the shape allows them."""
    opts(sa.OPT_DEC_SPLIT, -1)
    opts(sa.OPT_DEC_WAVES, 8)
    test_decode_positions(ctx, sa, oracle, wo, positions)


@pytest.mark.parametrize("window,cap,qk", [(0, 0.0, False), (16, 2.0, False), (0, 0.0, True)])
def test_decode_whole_window_norm(ctx, sa, oracle, wo, window, cap, qk, opts):
    """Eight-wave whole-sequence decode with a window and softcap, and with
    per-head Q/K norms (72-wide heads: a row tile's chunks past head_dim)."""
    from smol_genius_amd import runner
    from smol_genius_amd.workloads import Decode
    opts(sa.OPT_DEC_SPLIT, -1)
    opts(sa.OPT_DEC_WAVES, 8)
    for hq, hkv, hd in [(16, 8, 128), (6, 2, 72)]:
        positions = [0, 40, 200, 1000]
        print("decode whole", hd, window, cap, qk, flush=True)
        wl = Decode("t", hq, hkv, hd, [p + 1 for p in positions], 1e4, 0, seed=160 + hd)
        x = wl.inputs()
        qw = (1.0 + 0.1 * synth.normal(161, (hd,))).astype(np.float32) if qk else None
        kw = (1.0 + 0.1 * synth.normal(162, (hd,))).astype(np.float32) if qk else None
        r = runner.prepare(ctx, wl, x)
        got = sa.decode(ctx, r.kv, 0, r.rope, np.arange(wl.n_seq), wl.positions, r.q[0], r.k[0], r.v[0], wl.Hq,
                        wl.scale, window=window, cap=cap, q_norm=None if qw is None else dev(qw),
                        k_norm=None if kw is None else dev(kw), eps=1e-6).cpu().numpy()
        want = wo.decode(oracle, wl, x, q_norm=qw, k_norm=kw, eps=1e-6, window=window, cap=cap)
        assert_parity(got, want, "decode whole hd %d window %d cap %g qk %s" % (hd, window, cap, qk))


@pytest.mark.parametrize("hq,hkv,hd,rt,bf", [(16, 8, 128, 0, False), (8, 1, 256, 1, False), (6, 2, 72, 0, True),
                                             (4, 4, 80, 1, False), (8, 2, 96, 0, True), (4, 4, 64, 0, True),
                                             (32, 2, 128, 0, False), (64, 2, 64, 0, False), (24, 1, 256, 0, True)])
def test_decode_direct_cache_rows(ctx, sa, oracle, wo, hq, hkv, hd, rt, bf):
    """k_dec normalises, rotates and appends the new key itself; a one-token
    prefill at the same position goes through the pre-pass (k_prep) and
    k_dec's chunk mode. Both append the same bf16 cache rows (the rotation
    formulas are the same) and both outputs meet the oracle. G = 32 and 64
    cut the rows into row blocks; 24 heads at hd 256, into blocks of 16."""
    from smol_genius_amd import runner
    from smol_genius_amd.workloads import Decode
    positions = [0, 40, 200, 31]
    print("decode direct rows", hq, hkv, hd, rt, bf, flush=True)
    wl = Decode("t", hq, hkv, hd, [p + 1 for p in positions], 1e4, rt, seed=140 + hd)
    x = wl.inputs()
    if bf:
        for k in ("q", "k", "v"):
            x[k] = synth.f32_to_bf16_bits(x[k])
    want = wo.decode(oracle, wl, {k: (widen(a) if bf and k in ("q", "k", "v") else a) for k, a in x.items()})
    r = runner.prepare(ctx, wl, x)
    out = sa.decode(ctx, r.kv, 0, r.rope, np.arange(wl.n_seq), wl.positions, dev(x["q"], bf), dev(x["k"], bf),
                    dev(x["v"], bf), wl.Hq, wl.scale).cpu().numpy()
    assert_parity(out, want, "decode direct hd %d" % hd)
    direct_rows = [r.kv.read(0, i, p, 1) for i, p in enumerate(positions)]
    r2 = runner.prepare(ctx, wl, x)
    for i, p in enumerate(positions):
        q1, k1, v1 = (dev(x[k][i:i + 1], bf) for k in ("q", "k", "v"))
        o1 = sa.prefill(ctx, r2.kv, 0, i, r2.rope, p, q1, k1, v1, wl.Hq, wl.scale).cpu().numpy()
        assert_parity(o1, want[i:i + 1], "one-token prefill hd %d pos %d" % (hd, p))
        k_row, v_row = r2.kv.read(0, i, p, 1)
        np.testing.assert_array_equal(k_row, direct_rows[i][0])
        np.testing.assert_array_equal(v_row, direct_rows[i][1])


@pytest.mark.parametrize("case", [
    (16, 8, 128, 1536, 0, True), (32, 4, 96, 700, 0, False), (16, 4, 64, 1100, 300, False),
    (16, 16, 64, [0, 100, 700, 750, 1600, 1601, 2000]), (12, 12, 72, [3, 500, 1025, 1090, 1700, 1800]),
])
@pytest.mark.parametrize("qk_fp16", [0, 1])
def test_fb_one_key_group(ctx, sa, oracle, case, qk_fp16, opts):
    """k_attn_fb with one key group of eight waves (SMOL_OPT_FB_GROUPS 1):
    128-row items whose long key ranges are split over workgroups and merged
    by the last of each group. The same cases as the tile lists, with both
    QK^T modes; with lists and with one workgroup per item the merges add the
    same partials in the same order, so the two launches agree bit for bit."""
    opts(sa.OPT_FB_GROUPS, 1)
    opts(sa.OPT_QK_FP16, qk_fp16)
    test_fb_tile_lists(ctx, sa, oracle, case, opts)


@pytest.mark.parametrize("window,cap", [(16, 0.0), (0, 2.0), (1, 0.0), (40, 1.5), (1, 3.0)])
def test_decode_window_softcap(ctx, sa, oracle, wo, window, cap):
    """Sliding window and softcap on decode (the new key is scored apart
    from the cache slabs; window 1 leaves it alone)."""
    from smol_genius_amd import runner
    from smol_genius_amd.workloads import Decode
    positions = [0, 40, 200, 1000]
    print("decode window", window, "cap", cap, flush=True)
    wl = Decode("t", 16, 8, 128, [p + 1 for p in positions], 1e6, 0, seed=150 + window)
    x = wl.inputs()
    r = runner.prepare(ctx, wl, x)
    got = sa.decode(ctx, r.kv, 0, r.rope, np.arange(wl.n_seq), wl.positions, r.q[0], r.k[0], r.v[0], wl.Hq,
                    wl.scale, window=window, cap=cap).cpu().numpy()
    assert_parity(got, wo.decode(oracle, wl, x, window=window, cap=cap), "decode window %d cap %g" % (window, cap))


@pytest.mark.parametrize("name", ["qwen06b_decode", "gemma_mqa_decode", "qwen17b_stream"])
@pytest.mark.parametrize("split", [-1, 1])
def test_workload_full_size_dec_splits(ctx, sa, oracle, wo, name, split, opts):
    """The decode workloads with no split (one workgroup per sequence and kv
    head) and with the most splits (one slab per workgroup, capped at 32)."""
    if split == -1:
        opts(sa.OPT_DEC_SPLIT, -1)
    else:
        opts(sa.OPT_DEC_SLABS, 1)
    test_workload_full_size(ctx, oracle, wo, name)


def test_cache_roundtrip_growth_and_rewind(ctx, sa, oracle, wo):
    from smol_genius_amd.workloads import Prefill
    Hkv, hd = 2, 64
    kv = sa.KVCache(ctx, 2, 2, Hkv, hd, 40)
    assert kv.capacity == 64
    k = synth.f32_to_bf16_bits(synth.normal(70, (50, Hkv * hd)))
    v = synth.f32_to_bf16_bits(synth.normal(71, (50, Hkv * hd)))
    kv.write(1, 1, 10, k, v)
    rk, rv = kv.read(1, 1, 10, 50)
    np.testing.assert_array_equal(rk, k)
    np.testing.assert_array_equal(rv, v)
    # f32 rows are stored rounded to nearest even
    kf = synth.normal(72, (3, Hkv * hd))
    kv.write(0, 0, 0, kf, kf)
    np.testing.assert_array_equal(kv.read(0, 0, 0, 3)[0], synth.f32_to_bf16_bits(kf))
    # growth (doubling) keeps every row of every layer and slot
    kv.reserve(200)
    assert kv.capacity == 256
    rk, rv = kv.read(1, 1, 10, 50)
    np.testing.assert_array_equal(rk, k)
    np.testing.assert_array_equal(rv, v)
    np.testing.assert_array_equal(kv.read(0, 0, 0, 3)[0], synth.f32_to_bf16_bits(kf))
    # rewind: prefill 60 tokens, then re-prefill from position 20 with other tokens;
    # the second call must see rows [0, 20) of the first and its own rows only.
    rope = sa.RopeTable(ctx, hd, 1e6, 0)
    a = Prefill("a", 4, 2, 64, 0, 60, 1e6, seed=73)
    xa = a.inputs()
    sa.prefill(ctx, kv, 0, 1, rope, 0, dev(xa["q"], True), dev(xa["k"], True), dev(xa["v"], True), 4, a.scale)
    b = Prefill("b", 4, 2, 64, 20, 25, 1e6, seed=74)
    xb = b.inputs()
    ck, cv = kv.read(0, 1, 0, 20)
    xb["cache_k"], xb["cache_v"] = ck, cv
    got = sa.prefill(ctx, kv, 0, 1, rope, 20, dev(xb["q"], True), dev(xb["k"], True), dev(xb["v"], True), 4,
                     b.scale)
    assert_parity(got.cpu().numpy(), wo.prefill(oracle, b, xb), "rewind")


def test_prefill_grows_cache_and_table(ctx, sa, oracle, wo):
    from smol_genius_amd.workloads import Prefill
    kv = sa.KVCache(ctx, 1, 1, 2, 128, 16)
    rope = sa.RopeTable(ctx, 128, 1e6, 0, 16)
    wl = Prefill("g", 4, 2, 128, 0, 1100, 1e6, seed=75)
    x = wl.inputs()
    got = sa.prefill(ctx, kv, 0, 0, rope, 0, dev(x["q"], True), dev(x["k"], True), dev(x["v"], True), 4, wl.scale)
    assert kv.capacity >= 1100 and rope.capacity >= 1100
    assert_parity(got.cpu().numpy(), wo.prefill(oracle, wl, x), "grow")


def test_device_apply_rope(ctx, sa, oracle, wo):
    for hd, rt in [(128, 0), (256, 1), (72, 0)]:
        rope = sa.RopeTable(ctx, hd, 1e4, rt)
        pos = np.array([0, 3, 1500, 77], np.int32)
        x = synth.normal(80 + hd, (4, 3 * hd))
        got = sa.apply_rope(ctx, rope, dev(x), pos, 3).cpu().numpy()
        c, s = wo.rope_rows(oracle, pos, hd, 1e4, rt == 1)
        np.testing.assert_allclose(got, oracle.apply_rope(x, c, s, 4, 3, hd, rt == 1), rtol=1e-6, atol=1e-6)


def test_errors_are_reported(ctx, sa):
    with pytest.raises(sa.SmolAttnError, match="head_dim"):
        sa.KVCache(ctx, 1, 1, 2, 100, 16)
    kv = sa.KVCache(ctx, 1, 2, 2, 64, 16)
    q = torch.zeros((2, 4 * 64), device="cuda")
    k = torch.zeros((2, 2 * 64), device="cuda")
    with pytest.raises(sa.SmolAttnError, match="twice"):
        sa.decode(ctx, kv, 0, None, [1, 1], [3, 4], q, k, k, 4, 0.125)
    with pytest.raises(sa.SmolAttnError, match="multiple"):
        sa.decode(ctx, kv, 0, None, [0], [3], q[:1], k[:1], k[:1], 3, 0.125)
    with pytest.raises(sa.SmolAttnError, match="layer"):
        sa.prefill(ctx, kv, 5, 0, None, 0, q, k, k, 4, 0.125)


@pytest.mark.parametrize("Hq,Hkv,hd,sq,sk,qo,window,cap", [
    (8, 1, 256, 6, 33, 27, 0, 0.0), (8, 1, 256, 1, 300, 299, 0, 50.0), (4, 2, 128, 26, 200, 174, 64, 30.0),
    (8, 4, 64, 40, 40, 0, 16, 0.0), (4, 4, 72, 9, 9, 0, 0, 0.0)])
def test_causal_bf16_out(ctx, sa, oracle, Hq, Hkv, hd, sq, sk, qo, window, cap):
    """bf16 in / bf16 out (truncated) against the restated two-pass attention of
    the bf16 decoder (qkn_bf16_decoder.c:120-229); both sides truncate an fp32
    result, so they differ by at most one bf16 step where the fp32 results
    straddle one."""
    print("causal_bf16", Hq, Hkv, hd, sq, sk, qo, window, cap, flush=True)
    q = synth.f32_to_bf16_bits(synth.normal(110 + hd, (sq, Hq * hd)))
    k = synth.f32_to_bf16_bits(synth.normal(111 + hd, (sk, Hkv * hd)))
    v = synth.f32_to_bf16_bits(synth.normal(112 + hd, (sk, Hkv * hd)))
    sc = 1.0 / np.sqrt(hd)
    got = sa.causal_bf16(ctx, dev(q, True), dev(k, True), dev(v, True), sq, sk, Hq, Hkv, hd, sc, qo, window=window,
                         cap=cap).cpu().numpy().view(np.uint16)
    want = oracle.bf16_attention(q, k, v, sq, sk, Hq, Hkv, hd, sc, qo, window=window, cap=cap)
    assert_parity(widen(got), widen(want), "causal_bf16 hd %d" % hd)


# ------------------------------------------------------------- large sizes

def test_long_causal_prefill(ctx, sa, oracle, wo):
    """4096-token causal prefill from position 0 (k_attn_fb, 64 slabs per row tile at the end)."""
    from smol_genius_amd.workloads import Prefill
    print("long prefill 4096", flush=True)
    wl = Prefill("t", 8, 2, 128, 0, 4096, 1e6, seed=120)
    x = wl.inputs()
    kv = sa.KVCache(ctx, 1, 1, 2, 128, 4096)
    rope = sa.RopeTable(ctx, 128, wl.theta, 0)
    got = sa.prefill(ctx, kv, 0, 0, rope, 0, dev(x["q"], True), dev(x["k"], True), dev(x["v"], True), 8, wl.scale)
    assert_parity(got.cpu().numpy(), wo.prefill(oracle, wl, x), "prefill 4096")


def test_fresh_context_long_prefill(sa, oracle, wo):
    """The first call on a new context (staging buffers never touched before)
    with 8192 keys per kv head, so a tile's key slabs span more than the
    first transfers touch; LDS left by earlier kernels would show as wrong
    rows if a transfer were read before it landed."""
    from smol_genius_amd.workloads import Prefill
    print("fresh context prefill 8192", flush=True)
    c = sa.Context(0)
    try:
        wl = Prefill("t", 4, 2, 128, 0, 8192, 1e6, seed=125, in_bf16=True)
        x = wl.inputs()
        kv = sa.KVCache(c, 1, 1, 2, 128, 8192)
        rope = sa.RopeTable(c, 128, wl.theta, 0, 8192)
        got = sa.prefill(c, kv, 0, 0, rope, 0, dev(x["q"], True), dev(x["k"], True), dev(x["v"], True), 4,
                         wl.scale)
        assert_parity(got.cpu().numpy(), wo.prefill(oracle, wl, x), "fresh context prefill 8192")
        kv.close()
        rope.close()
    finally:
        c.close()


def test_long_prefix_chunk(ctx, sa, oracle, wo):
    """A 64-token chunk on a 16384-token cache (k_attn_fa, key ranges split across workgroups)."""
    from smol_genius_amd.workloads import Prefill
    print("chunk 64 on 16384", flush=True)
    wl = Prefill("t", 8, 2, 128, 16384, 64, 1e6, seed=121)
    x = wl.inputs()
    kv = sa.KVCache(ctx, 1, 1, 2, 128, 16384 + 64)
    kv.write(0, 0, 0, x["cache_k"], x["cache_v"])
    rope = sa.RopeTable(ctx, 128, wl.theta, 0)
    got = sa.prefill(ctx, kv, 0, 0, rope, 16384, dev(x["q"], True), dev(x["k"], True), dev(x["v"], True), 8,
                     wl.scale)
    assert_parity(got.cpu().numpy(), wo.prefill(oracle, wl, x), "chunk 64 on 16384")


@pytest.mark.parametrize("hq,hkv,hd", [(16, 8, 128), (8, 1, 256)])
def test_long_decode(ctx, sa, oracle, wo, hq, hkv, hd):
    """Decode at position 65535 and, in the same call, at 70 (one long and one short split group)."""
    from smol_genius_amd import runner
    from smol_genius_amd.workloads import Decode
    print("decode 65536 hd", hd, flush=True)
    wl = Decode("t", hq, hkv, hd, [65536, 71], 1e6, 0, seed=122 + hd)
    x = wl.inputs()
    r = runner.prepare(ctx, wl, x)
    r.step()
    assert_parity(r.outputs(), wo.decode(oracle, wl, x), "decode 65536 hd %d" % hd)


def test_contexts_on_two_threads(sa, oracle):
    """One context per host thread (the reference's pool is not re-entrant,
    threading.c:26-47): two threads, each with its own context and its own
    stream, run causal calls concurrently; every result matches the oracle."""
    import threading
    print("two threads", flush=True)
    cases = [(8, 2, 128, 40, 300, 260, 1), (4, 4, 64, 64, 64, 0, 2)]
    inputs = []
    for Hq, Hkv, hd, sq, sk, qo, seed in cases:
        Q = synth.normal(130 + seed, (sq, Hq * hd))
        K = synth.normal(131 + seed, (sk, Hkv * hd))
        V = synth.normal(132 + seed, (sk, Hkv * hd))
        inputs.append((Q, K, V, oracle.causal_attention(Q, K, V, sq, sk, Hq, Hkv, hd, 1.0 / np.sqrt(hd), qo)))
    results, errors = {}, []

    def worker(idx):
        try:
            Hq, Hkv, hd, sq, sk, qo, _ = cases[idx]
            Q, K, V, _ = inputs[idx]
            stream = torch.cuda.Stream()
            with torch.cuda.stream(stream):
                c = sa.Context(0, stream=stream.cuda_stream)
                q, k, v = dev(Q), dev(K), dev(V)
                outs = [sa.causal(c, q, k, v, sq, sk, Hq, Hkv, hd, 1.0 / np.sqrt(hd), qo) for _ in range(20)]
                c.synchronize()
                results[idx] = [o.cpu().numpy() for o in outs]
                c.close()
        except Exception as e:  # reported by the main thread
            errors.append(e)

    threads = [threading.Thread(target=worker, args=(i,)) for i in range(len(cases))]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors, errors
    for idx, (_, _, _, want) in enumerate(inputs):
        for got in results[idx]:
            assert_parity(got, want, "thread %d" % idx)


def test_contexts_on_two_threads_decode_bidir(sa, oracle, wo):
    """Two host threads, each with its own context and stream, interleave
    split-K decode calls (k_dec with several workgroups per sequence merged
    through the flags) and bidirectional window calls (k_attn_win) at the
    same time. Each context builds its own kernel arguments, so every result
    matches the oracle and repeats bit for bit."""
    import threading
    from smol_genius_amd import runner
    from smol_genius_amd.workloads import Bidir, Decode
    print("two threads decode + bidirectional", flush=True)
    cases = [
        (Decode("t0", 16, 8, 128, [1025, 300, 700], 1e6, 0, seed=171), Bidir("b0", 4, 72, [0, 256, 512], seed=172)),
        (Decode("t1", 8, 1, 256, [2000, 600], 1e4, 1, seed=173),
         Bidir("b1", 6, 64, [0, 104, 208, 312], seed=174, in_bf16=False)),
    ]
    inputs = [(d.inputs(), b.inputs()) for d, b in cases]
    wants = [(wo.decode(oracle, d, xd), wo.bidir(oracle, b, xb)) for (d, b), (xd, xb) in zip(cases, inputs)]
    results, errors = {}, []
    go = threading.Barrier(len(cases))

    def worker(idx):
        try:
            (d, b), (xd, xb) = cases[idx], inputs[idx]
            stream = torch.cuda.Stream()
            with torch.cuda.stream(stream):
                c = sa.Context(0, stream=stream.cuda_stream)
                c.set_option(sa.OPT_DEC_SLABS, 1)  # the most splits per sequence
                rd = runner.prepare(c, d, xd)
                rb = runner.prepare(c, b, xb)
                stream.synchronize()
                go.wait()
                outs = []
                for _ in range(25):
                    od = rd.step().clone()
                    ob = rb.step().clone()
                    outs.append((od, ob))
                c.synchronize()
                results[idx] = [(od.cpu().numpy(), ob.cpu().numpy()) for od, ob in outs]
                c.close()
        except Exception as e:  # reported by the main thread
            errors.append(e)

    threads = [threading.Thread(target=worker, args=(i,)) for i in range(len(cases))]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors, errors
    for idx, (want_d, want_b) in enumerate(wants):
        first_d, first_b = results[idx][0]
        assert_parity(first_d, want_d, "thread %d decode" % idx)
        assert_parity(first_b, want_b, "thread %d bidirectional" % idx)
        for od, ob in results[idx][1:]:
            np.testing.assert_array_equal(od, first_d)
            np.testing.assert_array_equal(ob, first_b)


def test_decode_merge_timeout_reported(ctx, sa, oracle, wo, opts):
    """A k_dec merger whose wait for its splits gives up writes NaN rows and
    raises the context's merge flag: synchronize then fails with
    SMOL_ATTN_ERR_TIMEOUT, and the next call is clean again. The give-up is
    forced from the host (mergers wait for a flag value no split stores,
    with a bound of 64 polls), so every kernel ends normally."""
    from smol_genius_amd import runner
    from smol_genius_amd.workloads import Decode
    print("decode merge timeout", flush=True)
    wl = Decode("t", 16, 8, 128, [1025, 300], 1e6, 0, seed=175)
    x = wl.inputs()
    if not ctx.get_option(sa.OPT_XCD_CHECK):
        pytest.skip("workgroups do not follow the XCD round robin here, so k_dec does not split")
    r = runner.prepare(ctx, wl, x)
    ctx.synchronize()
    opts(sa.OPT_DEC_SLABS, 1)
    opts(sa.OPT_DEC_SPIN, 64)
    opts(sa.OPT_FAULT_MERGE, 1)
    r.step()
    got = r.outputs()
    print("NaN rows after the forced give-up:", int(np.isnan(got).any(axis=1).sum()), flush=True)
    assert np.isnan(got).any(), "the merged rows of a timed-out merge are NaN"
    with pytest.raises(sa.SmolAttnTimeoutError):
        ctx.synchronize()
    ctx.set_option(sa.OPT_FAULT_MERGE, 0)
    r.step()
    ctx.synchronize()  # the flag was cleared by the failed synchronize
    assert_parity(r.outputs(), wo.decode(oracle, wl, x), "decode after a timed-out merge")
