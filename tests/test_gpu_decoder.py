"""The decoder-level attention block (include/smol_qkn_attn.h) on the GPU,
against the CPU oracle's model of the same block (oracle/decoder_oracle.py).

Each case binds a multi-layer decoder configuration to a fake decoder
context, then runs the call sequence of a streaming decoder over every layer:
prefill at position 0, a rewind to a prefix followed by a chunk on top of
it, single-token decode steps, and a second rewind with decodes that
overwrite cache rows. Outputs meet the path's bar
|gpu - cpu| <= 2e-3 + 1e-2 |cpu| (bf16 outputs widened first). Cache bytes:
the bf16 contract appends bit-identical rows (the oracle's truncating norm
and rotation are pinned by brute force in test_oracle_math.py); the fp32
contract rotates in fp32 on both sides, so its K rows agree to one bf16
step and its V rows exactly.
"""
import ctypes

import numpy as np
import pytest

from conftest import assert_parity, synth  # noqa: F401

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
def dorc():
    import decoder_oracle
    return decoder_oracle


def _weights(seed, hd):
    return (1.0 + 0.1 * synth.normal(seed, (hd,))).astype(np.float32)


# (name, config, layers: (is_sliding, q_norm, k_norm) per layer)
CONFIGS = [
    ("qwen3", dict(n_layers=2, n_heads=16, n_kv_heads=8, head_dim=128, eps=1e-6, rope_theta=1e6,
                   rope_local_theta=0.0, rope_type=0, sliding_window=0, attn_logit_softcap=0.0),
     [(0, True, True), (0, True, True)]),
    ("gemma3", dict(n_layers=3, n_heads=8, n_kv_heads=4, head_dim=256, eps=1e-6, rope_theta=1e6,
                    rope_local_theta=1e4, rope_type=1, sliding_window=32, attn_logit_softcap=0.0),
     [(1, True, True), (1, True, True), (0, True, True)]),
    ("gemma2", dict(n_layers=2, n_heads=8, n_kv_heads=1, head_dim=256, eps=1e-6, rope_theta=1e4,
                    rope_local_theta=0.0, rope_type=1, sliding_window=48, attn_logit_softcap=50.0),
     [(1, False, False), (0, False, False)]),
    ("odd", dict(n_layers=2, n_heads=6, n_kv_heads=2, head_dim=72, eps=1e-5, rope_theta=1e4,
                 rope_local_theta=0.0, rope_type=0, sliding_window=20, attn_logit_softcap=30.0),
     [(1, True, False), (0, False, True)]),
]

# (kind, start position, rows): prefill 80 at 0; rewind to 50 and a 20-row
# chunk; 6 decode steps; rewind to 40 and 2 decode steps
SEQUENCE = [("prefill", 0, 80), ("prefill", 50, 20)] + [("forward", p, 1) for p in range(70, 76)] + \
           [("forward", 40, 1), ("forward", 41, 1)]


def _inputs(seed, rows, cfg, bf16):
    H, Hkv, hd = cfg["n_heads"], cfg["n_kv_heads"], cfg["head_dim"]
    q = synth.normal(seed, (rows, H * hd))
    k = synth.normal(seed + 1, (rows, Hkv * hd))
    v = synth.normal(seed + 2, (rows, Hkv * hd))
    if bf16:
        return tuple(synth.f32_to_bf16_bits(a) for a in (q, k, v))
    return q, k, v


def _run(sa, oracle, dorc, name, cfg, layers, bf16, on_device=0):
    owner = ctypes.create_string_buffer(256)  # stands for the decoder's qkn_ctx_t
    blk = sa.QknAttn(owner, **cfg, bf16=1 if bf16 else 0, on_device=on_device, device=0, max_seq=64)
    model = (dorc.Bf16Block if bf16 else dorc.Fp32Block)(oracle, **cfg)
    hd = cfg["head_dim"]
    for li, (sl, qn, kn) in enumerate(layers):
        wq = _weights(100 + li, hd) if qn else None
        wk = _weights(200 + li, hd) if kn else None
        blk.set_layer(li, sl, wq, wk)
        model.set_layer(li, sl, wq, wk)
    outs = []
    try:
        for step, (kind, start, rows) in enumerate(SEQUENCE):
            for li in range(cfg["n_layers"]):
                q, k, v = _inputs(1000 * step + 10 * li, rows, cfg, bf16)
                print("qkn %s bf16=%d dev=%d %s start %d rows %d layer %d" % (name, bf16, on_device, kind, start,
                                                                            rows, li), flush=True)
                if on_device:
                    t = (lambda a: torch.from_numpy(a.view(np.int16)).cuda().view(torch.bfloat16)) if bf16 else \
                        (lambda a: torch.from_numpy(a).cuda())
                    qd, kd, vd = t(q), t(k), t(v)
                    got = getattr(blk, kind)(li, start, qd, kd, vd)
                    got = got.view(torch.int16).cpu().numpy().view(np.uint16) if bf16 else got.cpu().numpy()
                else:
                    got = getattr(blk, kind)(li, start, q, k, v)
                want = model.block(li, start, q, k, v)
                outs.append(got)
                if bf16:
                    assert_parity(synth.bf16_bits_to_f32(got), synth.bf16_bits_to_f32(want),
                                  "qkn %s %s@%d L%d" % (name, kind, start, li))
                else:
                    assert_parity(got, want, "qkn %s %s@%d L%d" % (name, kind, start, li))
        # cache rows [0, 42) of every layer hold what the model's cache holds
        for li in range(cfg["n_layers"]):
            kc, vc = blk.read_cache(li, 0, 42)
            mk, mv = model.ck[li, :42], model.cv[li, :42]
            if bf16:
                np.testing.assert_array_equal(kc, mk)
                np.testing.assert_array_equal(vc, mv)
            else:
                np.testing.assert_array_equal(vc, mv)
                assert np.abs(kc.astype(np.int32) - mk.astype(np.int32)).max() <= 1
    finally:
        blk.close()
    return outs


@pytest.mark.parametrize("name,cfg,layers", CONFIGS, ids=[c[0] for c in CONFIGS])
def test_qkn_block_fp32_sequence(sa, oracle, dorc, name, cfg, layers):
    _run(sa, oracle, dorc, name, cfg, layers, bf16=False)


@pytest.mark.parametrize("name,cfg,layers", CONFIGS[1:], ids=[c[0] for c in CONFIGS[1:]])
def test_qkn_block_bf16_sequence(sa, oracle, dorc, name, cfg, layers):
    """The bf16 decoder's contract (always interleaved pairs)."""
    _run(sa, oracle, dorc, name, cfg, layers, bf16=True)


@pytest.mark.parametrize("bf16", [False, True])
def test_qkn_block_device_io_matches_host_io(sa, oracle, dorc, bf16):
    name, cfg, layers = CONFIGS[1]
    a = _run(sa, oracle, dorc, name, cfg, layers, bf16, on_device=0)
    b = _run(sa, oracle, dorc, name, cfg, layers, bf16, on_device=1)
    for x, y in zip(a, b):
        np.testing.assert_array_equal(x, y)


@pytest.mark.parametrize("hd", [64, 72, 80, 96, 128, 256])
@pytest.mark.parametrize("mode", ["norm", "rope", "norm+rope"])
@pytest.mark.parametrize("seq", [37, 1])
def test_norm_rope_bf16_bits(sa, oracle, hd, mode, seq):
    """smol_attn_norm_rope_bf16 reproduces the oracle's truncating norm and
    rotation bit for bit, over several binades and far positions; one
    position (a decode step) takes the LDS-staged kernel."""
    print("norm_rope_bf16", hd, mode, seq, flush=True)
    ctx = sa.Context(0)
    try:
        H, pos0 = 3, 4000
        r = np.random.default_rng(hd)
        x = synth.f32_to_bf16_bits((r.standard_normal((seq, H * hd)) *
                                    np.exp2(r.integers(-8, 8, (seq, H * hd)))).astype(np.float32))
        w = _weights(300 + hd, hd) if "norm" in mode else None
        rope = sa.RopeTable(ctx, hd, 1e4, sa.ROPE_INTERLEAVED) if "rope" in mode else None
        xt = torch.from_numpy(x.view(np.int16)).cuda().view(torch.bfloat16)
        wt = None if w is None else torch.from_numpy(w).cuda()
        sa.norm_rope_bf16(ctx, rope, xt, wt, 1e-6, pos0, H, hd)
        got = xt.view(torch.int16).cpu().numpy().view(np.uint16)
        want = x
        if w is not None:
            want = oracle.bf16_rms_norm_per_head(want, w, seq, H, hd, 1e-6)
        if rope is not None:
            c, s = oracle.fill_rope_table(pos0, seq, hd, 1e4, True)
            want = oracle.bf16_apply_rope_interleaved(want, c, s, seq, H, hd)
        np.testing.assert_array_equal(got, want)
    finally:
        ctx.close()
