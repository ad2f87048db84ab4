"""Per-head Q/K RMSNorm fused in front of RoPE and the cache append, against
the CPU oracle (rmsnorm.c:78-140 restated, then rope.c and attention.c), on
the GPU.

The attention outputs meet the path's bar |gpu - cpu| <= 2e-3 + 1e-2 |cpu|
(conftest.ATOL / RTOL). The normalised and rotated rows themselves are fp32 on
both sides and differ only by summation order and rounding, so they are held
to 1e-5 relative.
"""
import numpy as np
import pytest

from conftest import assert_parity, synth  # noqa: F401
from gen_golden_inputs import digest, norm_inputs

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

EPS = 1e-6


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


@pytest.fixture(scope="module")
def wo():
    import workload_oracle
    return workload_oracle


def dev(a, bf16=False):
    if bf16:
        return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).cuda().view(torch.bfloat16)
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).cuda()


def weight(seed, hd):
    return (1.0 + 0.1 * synth.normal(seed, (hd,))).astype(np.float32)


def spread_rows(a, bf16):
    """Row i of a scaled by 2^(i % 5 - 2): exact in bf16 and fp32, and far
    from unit RMS, so that a missing or misplaced norm shows (V keeps unit
    scale, to which the absolute part of the parity bar is sized)."""
    f = np.exp2((np.arange(a.shape[0]) % 5 - 2).astype(np.float32))[:, None]
    if bf16:
        return synth.f32_to_bf16_bits(synth.bf16_bits_to_f32(a) * f)
    return (np.asarray(a, np.float32) * f).astype(np.float32)


@pytest.mark.parametrize("hd", [64, 72, 80, 96, 128, 256])
@pytest.mark.parametrize("mode", ["norm", "neox", "interleaved", "norm+neox", "norm+interleaved"])
def test_norm_rope_device(ctx, sa, oracle, wo, hd, mode):
    print("norm_rope", hd, mode, flush=True)
    seq, H = 5, 3
    x = synth.normal(90 + hd, (seq, H * hd), 2.0)
    w = weight(91 + hd, hd) if "norm" in mode else None
    inter = "interleaved" in mode
    rope = None
    pos = np.array([0, 7, 1023, 1024, 3000], np.int32)
    if mode != "norm":
        rope = sa.RopeTable(ctx, hd, 1e4, sa.ROPE_INTERLEAVED if inter else sa.ROPE_NEOX)
    xt = dev(x)
    sa.norm_rope(ctx, rope, xt, None if w is None else dev(w), EPS, None if rope is None else pos, H, hd)
    got = xt.cpu().numpy()
    want = x if w is None else oracle.rms_norm_per_head(x, w, seq, H, hd, EPS)
    if rope is not None:
        c, s = wo.rope_rows(oracle, pos, hd, 1e4, inter)
        want = oracle.apply_rope(want, c, s, seq, H, hd, inter)
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-5)


def test_golden_rms_norm_through_reference_signature(sa, golden):
    meta, data = golden
    for n in meta["norm"]:
        print("golden", n["name"], flush=True)
        x, w = norm_inputs(n["seed"], n["seq"], n["H"], n["hd"], n["std"])
        assert digest(x, w) == n["digest"]
        y = x.copy()
        sa.smol_rms_norm_per_head(y, w, n["seq"], n["H"], n["hd"], n["eps"])
        np.testing.assert_allclose(y, data[n["name"]], rtol=1e-5, atol=1e-6 * n["std"])


PREFILL_CASES = [  # P, S, hd, Hq, Hkv, rope_type, bf16 inputs, q norm, k norm
    (0, 33, 128, 8, 2, 0, False, True, True),
    (40, 64, 128, 8, 2, 0, True, True, True),
    (100, 26, 128, 16, 8, 0, False, True, True),   # 52 rows: the decode kernel
    (0, 70, 72, 6, 2, 1, True, True, False),
    (31, 5, 256, 8, 1, 1, False, False, True),
    (64, 100, 64, 4, 4, 0, False, True, True),
    (0, 300, 256, 4, 2, 0, True, True, True),
]


@pytest.mark.parametrize("case", PREFILL_CASES)
def test_prefill_qknorm(ctx, sa, oracle, wo, case):
    from smol_genius_amd.workloads import Prefill
    P, S, hd, Hq, Hkv, rt, bf, qn, kn = case
    print("prefill_qknorm", case, flush=True)
    wl = Prefill("t", Hq, Hkv, hd, P, S, 1e4 if rt else 1e6, seed=70 + P + S + hd, in_bf16=bf)
    wl.rope_type = rt
    x = wl.inputs()
    # only normalised operands are spread: the bar is sized for unit-scale scores
    if qn:
        x["q"] = spread_rows(x["q"], bf)
    if kn:
        x["k"] = spread_rows(x["k"], bf)
    kv = sa.KVCache(ctx, 1, 1, Hkv, hd, P + S)
    if P:
        kv.write(0, 0, 0, x["cache_k"], x["cache_v"])
    rope = sa.RopeTable(ctx, hd, wl.theta, rt)
    qw = weight(71 + hd, hd) if qn else None
    kw = weight(72 + hd, hd) if kn else None
    got = sa.prefill(ctx, kv, 0, 0, rope, P, dev(x["q"], bf), dev(x["k"], bf), dev(x["v"], bf), Hq, wl.scale,
                     q_norm=None if qw is None else dev(qw), k_norm=None if kw is None else dev(kw), eps=EPS)
    want = wo.prefill(oracle, wl, x, q_norm=qw, k_norm=kw, eps=EPS)
    assert_parity(got.cpu().numpy(), want, "prefill_qknorm %s" % (case,))
    # the cache holds the normalised and rotated new K (bf16, nearest even)
    k_rows, _ = kv.read(0, 0, P, S)
    pos = np.arange(P, P + S)
    c, s = wo.rope_rows(oracle, pos, hd, wl.theta, rt == 1)
    kref = wo._norm(oracle, x["k"], kw, S, Hkv, hd, EPS)
    kref = oracle.apply_rope(kref, c, s, S, Hkv, hd, rt == 1)
    exact = (k_rows == synth.f32_to_bf16_bits(kref)).mean()
    assert exact > 0.999, exact


FB_Q_CASES = [  # P, S, hd, Hq, Hkv, rope_type, bf16 inputs, q norm (which keeps Q in the pre-pass)
    (5, 150, 128, 16, 8, 0, True, False),     # RoPE rows from position 5
    (0, 200, 64, 8, 2, 1, False, False),
    (0, 130, 128, 6, 3, 1, False, False),
    (17, 90, 64, 4, 4, 0, True, False),
    (0, 100, 128, 8, 2, 0, True, True),
]


@pytest.mark.parametrize("case", FB_Q_CASES)
def test_prefill_fb_q_from_inputs(ctx, sa, oracle, wo, case):
    """k_attn_fb at head_dim 64 / 128 rotates and scales its own Q rows from
    the inputs (SMOL_OPT_FB_QPREP 0), or reads them from the pre-pass's Q
    scratch (1): both meet the oracle, and they differ only by the rounding
    of the rotation (fused multiply-adds in k_attn_fb)."""
    from smol_genius_amd.workloads import Prefill
    P, S, hd, Hq, Hkv, rt, bf, qn = case
    print("prefill fb q", case, flush=True)
    wl = Prefill("t", Hq, Hkv, hd, P, S, 1e4, seed=110 + P + S + hd, in_bf16=bf)
    wl.rope_type = rt
    x = wl.inputs()
    if qn:
        x["q"] = spread_rows(x["q"], bf)
    qw = weight(111 + hd, hd) if qn else None
    want = wo.prefill(oracle, wl, x, q_norm=qw, eps=EPS)
    outs = []
    ctx.set_option(sa.OPT_PREFILL_KERNEL, 1)
    try:
        for mode in (0, 1):
            ctx.set_option(sa.OPT_FB_QPREP, mode)
            kv = sa.KVCache(ctx, 1, 1, Hkv, hd, P + S)
            if P:
                kv.write(0, 0, 0, x["cache_k"], x["cache_v"])
            rope = sa.RopeTable(ctx, hd, wl.theta, rt)
            got = sa.prefill(ctx, kv, 0, 0, rope, P, dev(x["q"], bf), dev(x["k"], bf), dev(x["v"], bf), Hq,
                             wl.scale, q_norm=None if qw is None else dev(qw), eps=EPS).cpu().numpy()
            assert_parity(got, want, "prefill fb q %s mode %d" % (case, mode))
            outs.append(got)
    finally:
        ctx.set_option(sa.OPT_FB_QPREP, 0)
        ctx.set_option(sa.OPT_PREFILL_KERNEL, 0)
    assert np.abs(outs[0] - outs[1]).max() <= 1e-4 * max(1.0, np.abs(want).max())


@pytest.mark.parametrize("hq,hkv,hd,rt,qn,kn", [(16, 8, 128, 0, True, True), (8, 1, 256, 1, True, True),
                                                (4, 4, 64, 0, True, False), (6, 2, 72, 0, False, True)])
def test_decode_qknorm(ctx, sa, oracle, wo, hq, hkv, hd, rt, qn, kn):
    from smol_genius_amd import runner
    from smol_genius_amd.workloads import Decode
    positions = [0, 31, 64, 1000]
    print("decode_qknorm", hq, hkv, hd, rt, qn, kn, flush=True)
    wl = Decode("t", hq, hkv, hd, [p + 1 for p in positions], 1e4, rt, seed=80 + hd)
    x = wl.inputs()
    if qn:
        x["q"] = spread_rows(x["q"], False)
    if kn:
        x["k"] = spread_rows(x["k"], False)
    qw = weight(81 + hd, hd) if qn else None
    kw = weight(82 + hd, hd) if kn else None
    r = runner.prepare(ctx, wl, x)
    got = sa.decode(ctx, r.kv, 0, r.rope, np.arange(wl.n_seq), wl.positions, r.q[0], r.k[0], r.v[0], wl.Hq,
                    wl.scale, q_norm=None if qw is None else dev(qw), k_norm=None if kw is None else dev(kw),
                    eps=EPS).cpu().numpy()
    assert_parity(got, wo.decode(oracle, wl, x, q_norm=qw, k_norm=kw, eps=EPS), "decode_qknorm hd %d" % hd)


def test_qknorm_argument_errors(ctx, sa):
    kv = sa.KVCache(ctx, 1, 1, 2, 64, 64)
    q = torch.zeros((1, 4 * 64), dtype=torch.float32, device="cuda")
    k = torch.zeros((1, 2 * 64), dtype=torch.float32, device="cuda")
    w = torch.ones(64, dtype=torch.float32, device="cuda")
    with pytest.raises(sa.SmolAttnError):
        sa.prefill(ctx, kv, 0, 0, None, 0, q, k, k, 4, 0.125, q_norm=w, eps=-1.0)
    with pytest.raises(sa.SmolAttnError):
        sa.prefill(ctx, kv, 0, 0, None, 0, q, k, k, 4, 0.125, q_norm=w.to(torch.bfloat16))
    with pytest.raises(sa.SmolAttnError):
        sa.norm_rope(ctx, None, q, w, 1e-6, [0, 1], 4, 64)  # two positions for one row
    rope = sa.RopeTable(ctx, 128, 1e4)
    with pytest.raises(sa.SmolAttnError):
        sa.norm_rope(ctx, rope, q, w, 1e-6, [0], 4, 64)  # table built for head_dim 128
