"""The bf16-weight projections on the GPU against the CPU oracle.

Every case prints its name before it runs. Two bars on fp32 outputs:
  * the path's bar, |gpu - cpu| <= 2e-3 + 1e-2 |cpu| (conftest.ATOL / RTOL);
  * the arithmetic's own bound: both sides are fp32 sums of the same exact
    products (the GEMM path carries x as bf16 hi + lo, 2^-17 relative), so
    |gpu - cpu| <= (2 n 2^-24 + 2^-16) sum_i |x_i w_i| + |b| 2^-23.
bf16 outputs (truncated) match bit for bit when every partial sum is exact
(integer-valued inputs) and within one bf16 step otherwise.
"""
import os
import threading

import numpy as np
import pytest

from conftest import assert_parity, pkg, synth  # noqa: F401
from gen_golden_inputs import linear_inputs

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


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def dev_bits(bits):
    return torch.from_numpy(np.ascontiguousarray(bits, np.uint16).view(np.int16)).cuda()


def w32(bits):
    return synth.bf16_bits_to_f32(bits).astype(np.float64)


def bound(x, w_bits, b=None):
    a = np.abs(np.asarray(x, np.float64)) @ np.abs(w32(w_bits)).T
    n = w_bits.shape[1]
    t = a * (2 * (n + 1) * 2.0 ** -24 + 2.0 ** -16)
    if b is not None:
        t = t + np.abs(np.asarray(b, np.float64)) * 2.0 ** -22
    return t + 1e-30


def check(y, ref, x, w_bits, b, what):
    y = np.asarray(y, np.float64)
    assert_parity(y, ref, what)
    err = np.abs(y - np.asarray(ref, np.float64))
    lim = bound(x, w_bits, b)
    assert (err <= lim).all(), "%s: error %.3e above the fp32 bound (ratio %.2f)" % (
        what, err.max(), (err / lim).max())


GEMV_CASES = [
    # seq, in, out, bias
    (1, 1024, 4096, False),   # Q+K+V rows of Qwen3-0.6B, one wave per workgroup
    (1, 2048, 1024, False),   # o_proj: two waves split in_dim
    (1, 3072, 1024, True),    # down projection: three waves
    (1, 1024, 6144, False),   # gate_up
    (2, 1003, 33, True),      # in % 8 != 0: element loads
    (3, 72, 40, True),
    (4, 16384, 64, False),    # eight waves, two steps each
    (4, 7, 5, True),
    (1, 1, 3, True),
    (2, 24000, 9, False),     # eight waves, three steps, out not a multiple of 4
]


@pytest.mark.parametrize("case", GEMV_CASES, ids=lambda c: "s%d_in%d_out%d%s" % (c[0], c[1], c[2], "_b" * c[3]))
def test_gemv(ctx, sa, oracle, case):
    seq, n_in, n_out, has_b = case
    print("gemv", case, flush=True)
    x, w, b = linear_inputs(6000 + n_in + n_out, seq, n_in, n_out, has_b)
    y = sa.linear(ctx, dev(x), dev_bits(w), dev(b) if has_b else None)
    ctx.synchronize()
    check(y.cpu().numpy(), oracle.linear_bf16(x, w, b), x, w, b, "gemv %s" % (case,))


def test_gemv_bf16_io(ctx, sa, oracle):
    """bf16 x, truncated bf16 y (the bf16 decoder's contract)"""
    rng = np.random.default_rng(11)
    for seq, n_in, n_out in [(1, 1024, 256), (3, 96, 7), (4, 1003, 13)]:
        print("gemv bf16", seq, n_in, n_out, flush=True)
        xi = rng.integers(-16, 17, (seq, n_in)).astype(np.float32)
        wi = rng.integers(-16, 17, (n_out, n_in)).astype(np.float32)
        xb, wb = synth.f32_to_bf16_bits(xi), synth.f32_to_bf16_bits(wi)
        y = sa.linear(ctx, dev_bits(xb).view(torch.bfloat16), dev_bits(wb), out_bf16=True)
        ctx.synchronize()
        got = y.cpu().numpy().view(np.uint16)
        np.testing.assert_array_equal(got, oracle.bf16_linear_nobias(xb, wb))
        # random values: within one bf16 step of the oracle's truncated sum
        xb = synth.f32_to_bf16_bits(synth.normal(12 + seq, (seq, n_in)))
        wb = synth.f32_to_bf16_bits(synth.normal(13 + seq, (n_out, n_in), 1.0 / np.sqrt(n_in)))
        y = sa.linear(ctx, dev_bits(xb).view(torch.bfloat16), dev_bits(wb), out_bf16=True)
        ctx.synchronize()
        g = synth.bf16_bits_to_f32(y.cpu().numpy().view(np.uint16)).astype(np.float64)
        r = synth.bf16_bits_to_f32(oracle.bf16_linear_nobias(xb, wb)).astype(np.float64)
        assert (np.abs(g - r) <= np.abs(r) * 2.0 ** -7 + 1e-6).all()
        # fp32 x with a truncated bf16 y
        x = synth.normal(14 + seq, (seq, n_in))
        y = sa.linear(ctx, dev(x), dev_bits(wb), out_bf16=True)
        ctx.synchronize()
        g = synth.bf16_bits_to_f32(y.cpu().numpy().view(np.uint16)).astype(np.float64)
        r = oracle.linear_bf16(x, wb).astype(np.float64)
        assert (np.abs(g - r) <= np.abs(r) * 2.0 ** -7 + bound(x, wb)).all()


@pytest.mark.parametrize("shape", [(1, 1024, 2048, 1024), (3, 72, 40, 12), (1, 1003, 5, 0), (2, 64, 0, 8),
                                   (1, 2048, 2048, 1024), (26, 1024, 2048, 1024)])
def test_qkv(ctx, sa, oracle, shape):
    seq, n_in, q_dim, kv_dim = shape
    print("qkv", shape, flush=True)
    x, wq, _ = linear_inputs(7000 + n_in, seq, n_in, q_dim, False)
    _, wk, _ = linear_inputs(7100 + n_in, seq, n_in, kv_dim, False)
    _, wv, _ = linear_inputs(7200 + n_in, seq, n_in, kv_dim, False)
    q, k, v = sa.linear_qkv(ctx, dev(x), dev_bits(wq), dev_bits(wk), dev_bits(wv))
    ctx.synchronize()
    for got, w, nm in ((q, wq, "q"), (k, wk, "k"), (v, wv, "v")):
        if w.shape[0]:
            check(got.cpu().numpy(), oracle.linear_bf16(x, w), x, w, None, "qkv %s %s" % (shape, nm))


@pytest.mark.parametrize("case", [  # seq, in, q_dim, kv_dim, forced tile (0: by shape), norm, x bf16
    (1536, 1024, 2048, 1024, 0, False, False),   # Q on 128-wide tiles, K and V after it, one launch
    (1536, 1024, 2048, 1024, 3, True, False),    # 64-wide tiles, with the input norm
    (300, 512, 320, 64, 0, True, False),         # K and V one 64-wide tile column each, ragged rows
    (200, 256, 200, 40, 0, False, False),        # widths no tile divides: three launches
    (130, 1024, 256, 128, 2, False, True),       # bf16 x
    (130, 1024, 384, 192, 1, False, False),      # 192-wide tiles forced
])
def test_qkv_one_launch(ctx, sa, oracle, case):
    """Q, K and V of one x as column segments of one k_gemm launch where
    every segment boundary falls on a tile edge (else three launches); each
    output against the oracle, rows past the call untouched."""
    seq, n_in, q_dim, kv_dim, tile, norm, xbf = case
    print("qkv one launch", case, flush=True)
    x, wq, _ = linear_inputs(7300 + n_in + q_dim, seq, n_in, q_dim, False)
    _, wk, _ = linear_inputs(7400 + n_in + kv_dim, seq, n_in, kv_dim, False)
    _, wv, _ = linear_inputs(7500 + n_in + kv_dim, seq, n_in, kv_dim, False)
    g = (1.0 + 0.1 * synth.normal(7600 + n_in, (n_in,))).astype(np.float32) if norm else None
    if xbf:
        xbits = synth.f32_to_bf16_bits(x)
        x = synth.bf16_bits_to_f32(xbits)
        xd = dev_bits(xbits).view(torch.bfloat16)
    else:
        xd = dev(x)
    ctx.set_option(sa.OPT_GEMM_TILE, tile)
    try:
        if norm:
            q, k, v = sa.linear_qkv_norm(ctx, xd, dev_bits(wq), dev_bits(wk), dev_bits(wv), dev(g), 1e-6)
        else:
            q, k, v = sa.linear_qkv(ctx, xd, dev_bits(wq), dev_bits(wk), dev_bits(wv))
        ctx.synchronize()
    finally:
        ctx.set_option(sa.OPT_GEMM_TILE, 0)
    xn = oracle.rms_norm(x, g, 1e-6) if norm else x
    for got, w, nm in ((q, wq, "q"), (k, wk, "k"), (v, wv, "v")):
        ref = oracle.linear_bf16(xn, w)
        if norm:
            assert_parity(got.cpu().numpy(), ref, "qkv one launch %s %s" % (case, nm))
        else:
            check(got.cpu().numpy(), ref, x, w, None, "qkv one launch %s %s" % (case, nm))


GEMM_CASES = [
    # seq, in, out, bias, x bf16, y bf16
    (5, 1024, 4096, False, False, False),
    (26, 2048, 1024, False, False, False),
    (40, 512, 96, True, False, False),
    (7, 1003, 37, True, False, False),      # ld not a multiple of 8
    (64, 3072, 1024, False, False, False),
    (40, 512, 96, False, True, True),
    (33, 256, 80, True, False, True),
    (200, 1000, 390, True, False, False),   # K a multiple of 8 but not of the 64-wide K step; ragged tiles
    (193, 520, 200, False, True, False),    # bf16 x, tiles past M and N
    (1536, 1024, 2048, False, False, True), # the 128 x 128 tiles
]


@pytest.mark.parametrize("case", GEMM_CASES, ids=lambda c: "s%d_in%d_out%d%s%s%s" % (
    c[0], c[1], c[2], "_b" * c[3], "_xbf" * c[4], "_ybf" * c[5]))
def test_gemm(ctx, sa, oracle, case):
    seq, n_in, n_out, has_b, xbf, ybf = case
    print("gemm", case, flush=True)
    x, w, b = linear_inputs(8000 + n_in + n_out, seq, n_in, n_out, has_b)
    if xbf:
        xbits = synth.f32_to_bf16_bits(x)
        x = synth.bf16_bits_to_f32(xbits)
        xd = dev_bits(xbits).view(torch.bfloat16)
    else:
        xd = dev(x)
    y = sa.linear(ctx, xd, dev_bits(w), dev(b) if has_b else None, out_bf16=ybf)
    ctx.synchronize()
    ref = oracle.linear_bf16(x, w, b)
    if ybf:
        g = synth.bf16_bits_to_f32(y.cpu().numpy().view(np.uint16)).astype(np.float64)
        assert (np.abs(g - ref) <= np.abs(ref) * 2.0 ** -7 + bound(x, w, b)).all()
    else:
        check(y.cpu().numpy(), ref, x, w, b, "gemm %s" % (case,))


@pytest.mark.parametrize("tile", [1, 2, 3], ids=["192", "128", "64"])
def test_gemm_every_tile(ctx, sa, oracle, tile):
    """Each tile configuration forced (both wave layouts: fp32 and bf16 x), on
    ragged grids and on grids cut into per-XCD regions, plain and with the
    fused norm / activation / residual."""
    ctx.set_option(sa.OPT_GEMM_TILE, tile)
    try:
        for seq, n_in, n_out, has_b, xbf in [(200, 1000, 390, True, False), (193, 520, 200, False, True),
                                             (1536, 1024, 1024, False, False), (777, 1024, 2000, True, True)]:
            print("gemm tile", tile, seq, n_in, n_out, xbf, flush=True)
            x, w, b = linear_inputs(8500 + n_in + n_out + tile, seq, n_in, n_out, has_b)
            if xbf:
                xbits = synth.f32_to_bf16_bits(x)
                x = synth.bf16_bits_to_f32(xbits)
                xd = dev_bits(xbits).view(torch.bfloat16)
            else:
                xd = dev(x)
            y = sa.linear(ctx, xd, dev_bits(w), dev(b) if has_b else None)
            ctx.synchronize()
            check(y.cpu().numpy(), oracle.linear_bf16(x, w, b), x, w, b, "gemm tile %d %s" % (tile, (seq, n_in, n_out)))
        seq, n_in, n_out = 300, 1000, 392
        x, w, b = linear_inputs(8600 + tile, seq, n_in, n_out, True)
        g = (1.0 + 0.1 * synth.normal(8601, (n_in,))).astype(np.float32)
        r = synth.normal(8602, (seq, n_out // 2))
        ref = (r.astype(np.float64) + oracle.glu(oracle.linear_bf16(oracle.rms_norm(x, g, 1e-6), w, b), 1)).astype(
            np.float32)
        rd = dev(r)
        y = sa.linear_ops(ctx, dev(x), dev_bits(w), dev(b), norm_weight=dev(g), eps=1e-6, act=1, residual=rd, out=rd)
        ctx.synchronize()
        assert_parity(y.cpu().numpy(), ref, "gemm tile %d ops" % tile)
    finally:
        ctx.set_option(sa.OPT_GEMM_TILE, 0)


def test_gemm_full_prefill_shapes(ctx, sa, oracle):
    """Qwen3-0.6B projections of a 1536-token prefill: sampled rows against the
    oracle, every row against a float64 product on the device."""
    seq = 1536
    for n_in, n_out in [(1024, 4096), (2048, 1024), (1024, 6144), (3072, 1024)]:
        print("gemm prefill", seq, n_in, n_out, flush=True)
        x, w, _ = linear_inputs(9000 + n_out, seq, n_in, n_out, False)
        xd, wd = dev(x), dev_bits(w)
        y = sa.linear(ctx, xd, wd)
        ctx.synchronize()
        yh = y.cpu().numpy()
        rows = np.array([0, 1, 2, 511, 777, 1024, 1535])
        check(yh[rows], oracle.linear_bf16(x[rows], w), x[rows], w, None, "prefill %d->%d rows" % (n_in, n_out))
        w64 = wd.view(torch.bfloat16).to(torch.float64)
        ref = (xd.to(torch.float64) @ w64.T).cpu().numpy()
        check(yh, ref, x, w, None, "prefill %d->%d all" % (n_in, n_out))


def test_gemm_carries_the_low_part(ctx, sa):
    """x = 1 + 3 * 2^-10 is not a bf16 value (x_hi = 1, x_lo = 3 * 2^-10):
    with W = 1, every output is exactly n * x; without the low part it would be n."""
    for seq in (1, 8, 100):
        n = 1024
        x = np.full((seq, n), 1.0 + 3 * 2.0 ** -10, np.float32)
        w = synth.f32_to_bf16_bits(np.ones((16, n), np.float32))
        y = sa.linear(ctx, dev(x), dev_bits(w))
        ctx.synchronize()
        np.testing.assert_array_equal(y.cpu().numpy(), np.full((seq, 16), 1027.0, np.float32))


def test_empty_and_bias_only(ctx, sa):
    b = synth.normal(3, (9,))
    for seq in (2, 9):
        y = sa.linear(ctx, torch.zeros((seq, 0), device="cuda"), torch.zeros((9, 0), dtype=torch.int16,
                                                                               device="cuda"), dev(b))
        ctx.synchronize()
        np.testing.assert_array_equal(y.cpu().numpy(), np.broadcast_to(b, (seq, 9)))
    y = sa.linear(ctx, torch.zeros((0, 16), device="cuda"), torch.zeros((9, 16), dtype=torch.int16, device="cuda"))
    assert y.shape == (0, 9)


def test_golden_through_reference_signatures(sa):
    import json
    from conftest import GOLDEN
    with open(os.path.join(GOLDEN, "ref_linear.json")) as f:
        meta = json.load(f)
    data = np.load(os.path.join(GOLDEN, "ref_linear.npz"))
    for c in meta["cases"]:
        print("golden", c["name"], flush=True)
        n_in, n_out, seq = c["in_dim"], c["out_dim"], c["seq"]
        if c["kind"] == "qkv":
            x, wq, _ = linear_inputs(c["seed"], 1, n_in, n_out, False)
            _, wk, _ = linear_inputs(c["seed"] + 100, 1, n_in, n_out // 2, False)
            _, wv, _ = linear_inputs(c["seed"] + 200, 1, n_in, n_out // 2, False)
            q = np.zeros(n_out, np.float32)
            k = np.zeros(n_out // 2, np.float32)
            v = np.zeros(n_out // 2, np.float32)
            sa.smol_linear_nobias_bf16_qkv(q, k, v, x, wq, wk, wv, n_in, n_out, n_out // 2)
            for got, w, tag in ((q, wq, "_q"), (k, wk, "_k"), (v, wv, "_v")):
                check(got[None], data[c["name"] + tag][None], x, w, None, c["name"] + tag)
            continue
        x, w, b = linear_inputs(c["seed"], seq, n_in, n_out, c["bias"])
        y = np.zeros((seq, n_out), np.float32)
        if c["kind"] == "matmul_t":
            sa.smol_matmul_t_bf16(y, x, w, seq, n_in, n_out)
        elif b is None:
            sa.smol_linear_nobias_bf16(y, x, w, seq, n_in, n_out)
        else:
            sa.smol_linear_bf16(y, x, w, b, seq, n_in, n_out)
        check(y, data[c["name"]], x, w, b, c["name"])


def test_dropin_weight_cache(sa, oracle):
    """SMOL_BF16_CACHE_MB keeps device copies of weights by host pointer (a
    fresh thread reads the variable, as each thread has its own drop-in state)."""
    x, w1, _ = linear_inputs(31, 1, 256, 64, False)
    _, w2, _ = linear_inputs(32, 1, 256, 64, False)
    res = {}

    def body():
        os.environ["SMOL_BF16_CACHE_MB"] = "64"
        try:
            for i, w in enumerate((w1, w2, w1, w2)):
                y = np.zeros((1, 64), np.float32)
                sa.smol_linear_nobias_bf16(y, x, w, 1, 256, 64)
                res[i] = y
        finally:
            del os.environ["SMOL_BF16_CACHE_MB"]

    t = threading.Thread(target=body)
    t.start()
    t.join()
    for i, w in enumerate((w1, w2, w1, w2)):
        check(res[i], oracle.linear_bf16(x, w), x, w, None, "cached weight %d" % i)
    np.testing.assert_array_equal(res[0], res[2])
    np.testing.assert_array_equal(res[1], res[3])


# ------------------------------------------- the decoder layer's fused operations

OPS_CASES = [
    # seq, in, out, norm, act, residual ("y": in place, "sep": separate), bias
    (1, 1024, 6144, True, 1, None, False),    # post-attention norm + gate_up + SwiGLU
    (1, 2048, 1024, False, 0, "y", False),    # o_proj + residual add in place
    (1, 3072, 1024, False, 0, "y", False),    # down + residual add (three waves)
    (1, 1024, 4096, True, 0, None, False),    # input norm + projection
    (2, 512, 96, True, 2, "sep", True),       # GeGLU with bias and a separate residual
    (3, 1003, 40, True, 1, "y", True),        # element loads
    (4, 3072, 64, True, 0, "sep", False),
    (26, 1024, 6144, True, 1, None, False),   # the same operations on the GEMM path
    (26, 2048, 1024, False, 0, "y", False),
    (64, 512, 96, True, 2, "sep", True),
    (40, 1003, 40, True, 1, "y", True),
    (300, 3072, 1024, False, 0, "sep", True),
    (130, 1000, 390, True, 1, "sep", True),   # norm weight past a partial last K step
    (1536, 1024, 6144, True, 1, None, False), # the full prefill gate_up (192 x 192 tiles)
]


@pytest.mark.parametrize("case", OPS_CASES, ids=lambda c: "s%d_in%d_out%d_n%d_a%d_%s%s" % (
    c[0], c[1], c[2], c[3], c[4], c[5] or "nores", "_b" * c[6]))
def test_linear_ops(ctx, sa, oracle, case):
    seq, n_in, n_out, norm, act, res, has_b = case
    print("ops", case, flush=True)
    x, w, b = linear_inputs(9500 + n_in + n_out, seq, n_in, n_out, has_b)
    g = (1.0 + 0.1 * synth.normal(9600 + n_in, (n_in,))).astype(np.float32) if norm else None
    cols = n_out // 2 if act else n_out
    r = synth.normal(9700 + n_out, (seq, cols)) if res else None
    # oracle composition: rms_norm -> linear (+ bias) -> activation -> + residual
    xn = oracle.rms_norm(x, g, 1e-6) if norm else x
    t = oracle.linear_bf16(xn, w, b)
    ref = oracle.glu(t, act) if act else t
    if res:
        ref = (r.astype(np.float64) + ref).astype(np.float32)
    rd = dev(r) if res else None
    out = rd if res == "y" else None
    y = sa.linear_ops(ctx, dev(x), dev_bits(w), dev(b) if has_b else None, norm_weight=dev(g) if norm else None,
                      eps=1e-6, act=act, residual=rd, out=out)
    ctx.synchronize()
    got = y.cpu().numpy()
    assert got.shape == (seq, cols)
    assert_parity(got, ref, "ops %s" % (case,))
    if not act:
        # without an activation the fp32 bound of the product applies (plus the norm's rounding)
        lim = bound(xn, w, b) + 4 * 2.0 ** -24 * (np.abs(t) + (np.abs(r) if res else 0))
        assert (np.abs(got.astype(np.float64) - ref) <= lim).all()


def test_rms_norm_dev(ctx, sa, oracle):
    for seq, dim in [(1, 1024), (5, 72), (2, 7), (3, 3072), (1536, 1024)]:
        print("rms_norm", seq, dim, flush=True)
        x = synth.normal(77 + dim, (seq, dim), 3.0)
        w = (1.0 + 0.1 * synth.normal(78 + dim, (dim,))).astype(np.float32)
        ref = oracle.rms_norm(x, w, 1e-6)
        xd = dev(x)
        y = sa.rms_norm(ctx, xd, dev(w), 1e-6)
        ctx.synchronize()
        np.testing.assert_allclose(y.cpu().numpy(), ref, rtol=2e-6, atol=1e-6)
        sa.rms_norm(ctx, xd, dev(w), 1e-6, out=xd)   # in place
        ctx.synchronize()
        np.testing.assert_allclose(xd.cpu().numpy(), ref, rtol=2e-6, atol=1e-6)


def _step_diff(a, b):
    """|a - b| in bf16 steps of the bits (same-sign values)"""
    return np.abs(np.asarray(a, np.uint16).astype(np.int32) - np.asarray(b, np.uint16).astype(np.int32))


def test_bf16_row_ops(ctx, sa, oracle):
    """smol_bf16_rms_norm_dev / smol_bf16_add_norm_dev / smol_bf16_geglu_dev
    against the oracle's bf16_rms_norm, bf16_add and bf16_geglu. The device
    sums squares in another order and calls the device tanhf, so a result
    that lies on a truncation boundary may come out one bf16 step away: the
    bar is at most one step, with at least 99% of the elements bit-equal."""
    for seq, dim in [(1, 1024), (3, 72), (2, 7), (40, 320), (1536, 1024)]:
        print("bf16 rows", seq, dim, flush=True)
        x = synth.f32_to_bf16_bits(synth.normal(90 + dim, (seq, dim), 3.0))
        p = synth.f32_to_bf16_bits(synth.normal(91 + dim, (seq, dim), 0.5))
        w1 = (1.0 + 0.1 * synth.normal(92 + dim, (dim,))).astype(np.float32)
        w2 = (1.0 + 0.1 * synth.normal(93 + dim, (dim,))).astype(np.float32)
        ref = oracle.bf16_rms_norm(x, w1, 1e-6)
        xd = dev_bits(x)
        got = sa.bf16_rms_norm(ctx, xd, dev(w1), 1e-6).cpu().numpy().view(np.uint16)
        d = _step_diff(got, ref)
        assert d.max() <= 1 and (d == 0).mean() >= 0.99, (d.max(), (d == 0).mean())
        sa.bf16_rms_norm(ctx, xd, dev(w1), 1e-6, out=xd)  # in place
        assert (xd.cpu().numpy().view(np.uint16) == got).all()
        # x = x + norm(p, w1); xn = norm(x, w2), the bf16 Gemma 3 step
        xd = dev_bits(x)
        xn = sa.bf16_add_norm(ctx, xd, dev_bits(p), dev(w1), dev(w2), 1e-6)
        ctx.synchronize()
        q_ref = oracle.bf16_rms_norm(p, w1, 1e-6)
        x_ref = oracle.bf16_add(x, q_ref)
        x_got = xd.cpu().numpy().view(np.uint16)
        # a step of the normed p carries into the sum at its own size, which
        # is more than a step of the sum where x and p cancel
        err = np.abs(synth.bf16_bits_to_f32(x_got).astype(np.float64) - synth.bf16_bits_to_f32(x_ref))
        bar = 2.0 ** -7 * (np.abs(synth.bf16_bits_to_f32(x_ref)) + np.abs(synth.bf16_bits_to_f32(q_ref)))
        assert (err <= bar).all() and (x_got == x_ref).mean() >= 0.99
        # the second norm, of the x the device computed
        d = _step_diff(xn.cpu().numpy().view(np.uint16), oracle.bf16_rms_norm(x_got, w2, 1e-6))
        assert d.max() <= 1 and (d == 0).mean() >= 0.99
        # plain residual add (no norms): exact
        xd = dev_bits(x)
        sa.bf16_add_norm(ctx, xd, dev_bits(p))
        ctx.synchronize()
        assert (xd.cpu().numpy().view(np.uint16) == oracle.bf16_add(x, p)).all()
    for seq, inter in [(1, 3072), (5, 13), (1536, 3072)]:
        print("bf16 geglu", seq, inter, flush=True)
        gu = synth.f32_to_bf16_bits(synth.normal(95 + inter, (seq, 2 * inter), 2.0))
        ref = oracle.bf16_geglu(gu)
        got = sa.bf16_geglu(ctx, dev_bits(gu)).cpu().numpy().view(np.uint16)
        gf, rf = synth.bf16_bits_to_f32(got).astype(np.float64), synth.bf16_bits_to_f32(ref).astype(np.float64)
        g, u = synth.bf16_bits_to_f32(gu[:, 0::2]), synth.bf16_bits_to_f32(gu[:, 1::2])
        # one bf16 step, plus, where 1 + tanh cancels, an ulp of 1 times 0.5 g u
        bar = 2.0 ** -7 * np.abs(rf) + 2.0 ** -22 * np.abs(0.5 * g * u)
        assert (np.abs(gf - rf) <= bar).all() and (got == ref).mean() >= 0.99
