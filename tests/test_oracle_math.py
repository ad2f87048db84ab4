"""Pins the CPU oracle with what the mathematics fixes, independent of the reference.

* float64 brute force: softmax(scale * Q K^T + mask) V, with the causal,
  sliding-window and softcap variants and GQA head mapping written out
  independently of the oracle's online-softmax loop;
* closed forms: one visible key, identical keys, scale 0, empty rows, clipping;
* structural identities: decode == last row of prefill, chunked prefill ==
  rows of the full prefill, GQA == MHA with repeated K/V heads, windowed
  bidirectional == per-window calls;
* RoPE: float64 tables, position 0 is the identity, pair norms are kept,
  R(a) R(b) = R(a + b);
* planted mistakes: mutated float64 restatements (off-by-one causal limit,
  wrong RoPE sign, wrong GQA head map, transposed RoPE pairing) must fail the
  same checks, so the checks can tell a right answer from a plausible wrong one.
"""
import numpy as np
import pytest

from conftest import synth


def brute_causal(Q, K, V, seq_q, seq_k, Hq, Hkv, hd, scale, q_offset, window=0, cap=0.0,
                 kv_head=None):
    Q = Q.astype(np.float64).reshape(seq_q, Hq, hd)
    K = K.astype(np.float64).reshape(seq_k, Hkv, hd)
    V = V.astype(np.float64).reshape(seq_k, Hkv, hd)
    out = np.zeros((seq_q, Hq, hd))
    kv_head = kv_head or (lambda h: h // (Hq // Hkv))
    for h in range(Hq):
        g = kv_head(h)
        s = Q[:, h, :] @ K[:, g, :].T * scale
        if cap > 0:
            s = cap * np.tanh(s / cap)
        pos = q_offset + np.arange(seq_q)[:, None]
        j = np.arange(seq_k)[None, :]
        vis = j <= pos
        if window > 0:
            vis &= j > pos - window
        s = np.where(vis, s, -np.inf)
        for i in range(seq_q):
            if not vis[i].any():
                continue
            p = np.exp(s[i] - s[i].max())
            out[i, h] = (p @ V[:, g, :]) / p.sum()
    return out.reshape(seq_q, Hq * hd)


def rand(seed, shape, std=1.0):
    return synth.normal(seed, shape, std)


CASES = [  # Hq, Hkv, hd, seq_q, seq_k, q_offset
    (4, 2, 64, 9, 9, 0), (8, 1, 128, 1, 77, 76), (2, 2, 72, 13, 40, 27),
    (4, 4, 256, 5, 17, 12), (6, 3, 64, 8, 30, 25),
]


@pytest.mark.parametrize("case", CASES)
def test_causal_brute_force(oracle, case):
    Hq, Hkv, hd, sq, sk, qo = case
    Q, K, V = rand(1, (sq, Hq * hd)), rand(2, (sk, Hkv * hd)), rand(3, (sk, Hkv * hd))
    sc = 1.0 / np.sqrt(hd)
    got = oracle.causal_attention(Q, K, V, sq, sk, Hq, Hkv, hd, sc, qo)
    np.testing.assert_allclose(got, brute_causal(Q, K, V, sq, sk, Hq, Hkv, hd, sc, qo),
                               rtol=2e-5, atol=2e-6)


@pytest.mark.parametrize("window,cap", [(5, 0.0), (0, 20.0), (7, 5.0), (1, 0.0)])
def test_window_softcap_brute_force(oracle, window, cap):
    Hq, Hkv, hd, sq, sk, qo = 4, 2, 64, 12, 30, 18
    Q, K, V = rand(4, (sq, Hq * hd), 2.0), rand(5, (sk, Hkv * hd), 2.0), rand(6, (sk, Hkv * hd))
    sc = 1.0 / np.sqrt(hd)
    got = oracle.causal_attention(Q, K, V, sq, sk, Hq, Hkv, hd, sc, qo, window=window, cap=cap)
    want = brute_causal(Q, K, V, sq, sk, Hq, Hkv, hd, sc, qo, window=window, cap=cap)
    np.testing.assert_allclose(got, want, rtol=2e-5, atol=2e-6)


def test_bidirectional_brute_force_and_windows(oracle):
    H, hd = 3, 72
    ws = [0, 10, 11, 37]
    seq = ws[-1]
    Q, K, V = rand(7, (seq, H * hd)), rand(8, (seq, H * hd)), rand(9, (seq, H * hd))
    sc = 1.0 / np.sqrt(hd)
    got = oracle.bidirectional_attention(Q, K, V, seq, H, hd, sc, ws)
    want = np.zeros_like(got)
    for a, b in zip(ws[:-1], ws[1:]):
        n = b - a
        # a bidirectional window is causal attention of its last row over every row
        blk = brute_causal(Q[a:b], K[a:b], V[a:b], n, n, H, H, hd, sc, n - 1)
        want[a:b] = blk
        # and the windowed call equals an independent call on that window
        sub = oracle.bidirectional_attention(Q[a:b], K[a:b], V[a:b], n, H, hd, sc, [0, n])
        np.testing.assert_array_equal(sub, got[a:b])
    np.testing.assert_allclose(got, want, rtol=2e-5, atol=2e-6)


def test_closed_forms(oracle):
    Hq, Hkv, hd = 4, 2, 64
    sk = 20
    K, V = rand(10, (sk, Hkv * hd)), rand(11, (sk, Hkv * hd))
    Q = rand(12, (sk, Hq * hd))
    sc = 0.125
    out = oracle.causal_attention(Q, K, V, sk, sk, Hq, Hkv, hd, sc, 0)
    # row 0 sees one key: o = v_0 for every head of the group
    for h in range(Hq):
        g = h // 2
        np.testing.assert_array_equal(out[0, h * hd:(h + 1) * hd], V[0, g * hd:(g + 1) * hd])
    # scale 0: uniform weights, o_i = mean(v_0..v_i)
    out0 = oracle.causal_attention(Q, K, V, sk, sk, Hq, Hkv, hd, 0.0, 0)
    cm = np.cumsum(V.astype(np.float64), 0) / np.arange(1, sk + 1)[:, None]
    for h in range(Hq):
        g = h // 2
        np.testing.assert_allclose(out0[:, h * hd:(h + 1) * hd], cm[:, g * hd:(g + 1) * hd],
                                   rtol=1e-5, atol=1e-6)
    # identical keys: o = mean of the visible values
    Kc = np.tile(K[:1], (sk, 1))
    outc = oracle.causal_attention(Q, Kc, V, sk, sk, Hq, Hkv, hd, sc, 0)
    np.testing.assert_allclose(outc[:, :hd], cm[:, :hd], rtol=1e-5, atol=1e-6)
    # empty rows (q_offset + i + 1 <= 0) are zero; seq_k = 0 gives zeros
    outn = oracle.causal_attention(Q[:5], K, V, 5, sk, Hq, Hkv, hd, sc, -3)
    assert not outn[:3].any() and outn[3:].any()
    assert not oracle.causal_attention(Q[:2], K, V, 2, 0, Hq, Hkv, hd, sc, 0).any()
    # q_offset + i >= seq_k clips to seq_k visible keys
    a = oracle.causal_attention(Q[:1], K, V, 1, sk, Hq, Hkv, hd, sc, 500)
    b = oracle.causal_attention(Q[:1], K, V, 1, sk, Hq, Hkv, hd, sc, sk - 1)
    np.testing.assert_array_equal(a, b)


def test_structural_identities(oracle):
    Hq, Hkv, hd, S = 8, 2, 128, 40
    Q, K, V = rand(13, (S, Hq * hd)), rand(14, (S, Hkv * hd)), rand(15, (S, Hkv * hd))
    sc = 1.0 / np.sqrt(hd)
    full = oracle.causal_attention(Q, K, V, S, S, Hq, Hkv, hd, sc, 0)
    # decode == last prefill row
    dec = oracle.causal_attention(Q[-1:], K, V, 1, S, Hq, Hkv, hd, sc, S - 1)
    np.testing.assert_array_equal(dec, full[-1:])
    # chunked prefill == rows P..P+C-1 of the full prefill
    P, C = 29, 11
    ch = oracle.causal_attention(Q[P:P + C], K, V, C, S, Hq, Hkv, hd, sc, P)
    np.testing.assert_array_equal(ch, full[P:P + C])
    # GQA == MHA with K/V heads repeat-interleaved
    rep = Hq // Hkv
    Km = np.repeat(K.reshape(S, Hkv, hd), rep, axis=1).reshape(S, Hq * hd)
    Vm = np.repeat(V.reshape(S, Hkv, hd), rep, axis=1).reshape(S, Hq * hd)
    mha = oracle.causal_attention(Q, Km, Vm, S, S, Hq, Hq, hd, sc, 0)
    np.testing.assert_array_equal(mha, full)


def _rope64(x, pos, hd, theta, interleaved):
    inv = 1.0 / np.power(np.float64(theta), np.arange(hd // 2) * 2.0 / hd)
    a = np.asarray(pos, np.float64)[:, None] * inv[None, :]
    c, s = np.cos(a), np.sin(a)
    x = x.astype(np.float64).reshape(len(pos), -1, hd)
    if interleaved:
        x0, x1 = x[..., 0::2], x[..., 1::2]
        y = np.empty_like(x)
        y[..., 0::2] = x0 * c[:, None] - x1 * s[:, None]
        y[..., 1::2] = x1 * c[:, None] + x0 * s[:, None]
    else:
        h = hd // 2
        x1, x2 = x[..., :h], x[..., h:]
        y = np.concatenate([x1 * c[:, None] - x2 * s[:, None], x2 * c[:, None] + x1 * s[:, None]], -1)
    return y.reshape(len(pos), -1)


@pytest.mark.parametrize("hd,theta,inter", [(128, 1e6, False), (256, 1e4, True), (64, 1e4, False),
                                            (72, 1e4, False)])
def test_rope_against_float64(oracle, hd, theta, inter):
    pos = np.array([0, 1, 5, 100, 1023, 1024, 4095, 8281], np.int32)
    c, s = oracle.fill_rope_table(0, 8282, hd, theta, inter)
    c, s = c[pos], s[pos]
    inv32 = oracle.rope_inv_freq(hd, theta)
    ang = pos[:, None].astype(np.float32) * inv32[None, :]  # the float32 angle of the reference
    k = np.arange(hd) // 2 if inter else np.arange(hd) % (hd // 2)
    np.testing.assert_allclose(c, np.cos(ang.astype(np.float64))[:, k], atol=1e-6)
    np.testing.assert_allclose(s, np.sin(ang.astype(np.float64))[:, k], atol=1e-6)
    # the frequency itself is the float64 one to float32 rounding
    np.testing.assert_allclose(inv32, 1.0 / np.power(theta, np.arange(hd // 2) * 2.0 / hd),
                               rtol=3e-7)
    x = rand(16, (len(pos), 2 * hd))
    y = oracle.apply_rope(x, c, s, len(pos), 2, hd, interleaved=inter)
    # position 0 is the identity
    np.testing.assert_array_equal(y[0], x[0])
    # each rotated pair keeps its norm
    yy, xx = y.reshape(len(pos), 2, hd).astype(np.float64), x.reshape(len(pos), 2, hd).astype(np.float64)
    if inter:
        ny, nx = yy[..., 0::2] ** 2 + yy[..., 1::2] ** 2, xx[..., 0::2] ** 2 + xx[..., 1::2] ** 2
    else:
        h = hd // 2
        ny, nx = yy[..., :h] ** 2 + yy[..., h:] ** 2, xx[..., :h] ** 2 + xx[..., h:] ** 2
    np.testing.assert_allclose(ny, nx, rtol=2e-5, atol=1e-6)
    # against a rotation by tables computed in float64 from the same float32 angle
    a64 = ang.astype(np.float64)
    cc, ss = np.cos(a64)[:, k], np.sin(a64)[:, k]
    yr = oracle.apply_rope(x, cc.astype(np.float32), ss.astype(np.float32), len(pos), 2, hd, inter)
    np.testing.assert_allclose(y, yr, atol=2e-5)


def test_rope_composition(oracle):
    hd, theta = 128, 1e6
    a, b = 300, 211
    c, s = oracle.fill_rope_table(0, a + b + 1, hd, theta, False)
    x = rand(17, (1, 4 * hd))
    ya = oracle.apply_rope(x, c[a:a + 1], s[a:a + 1], 1, 4, hd)
    yab = oracle.apply_rope(ya, c[b:b + 1], s[b:b + 1], 1, 4, hd)
    yd = oracle.apply_rope(x, c[a + b:a + b + 1], s[a + b:a + b + 1], 1, 4, hd)
    np.testing.assert_allclose(yab, yd, atol=2e-4)  # float32 angles of 511 rad


# ------------------------------------------------------------ planted mistakes

def test_planted_mistakes_are_caught(oracle):
    Hq, Hkv, hd, sq, sk, qo = 4, 2, 64, 9, 20, 11
    Q, K, V = rand(18, (sq, Hq * hd)), rand(19, (sk, Hkv * hd)), rand(20, (sk, Hkv * hd))
    sc = 1.0 / np.sqrt(hd)
    got = oracle.causal_attention(Q, K, V, sq, sk, Hq, Hkv, hd, sc, qo)
    ok = lambda w: np.allclose(got, w, rtol=2e-5, atol=2e-6)  # noqa: E731
    assert ok(brute_causal(Q, K, V, sq, sk, Hq, Hkv, hd, sc, qo))
    # causal limit off by one
    assert not ok(brute_causal(Q, K, V, sq, sk, Hq, Hkv, hd, sc, qo + 1))
    assert not ok(brute_causal(Q, K, V, sq, sk, Hq, Hkv, hd, sc, qo - 1))
    # GQA head map h % Hkv instead of h // (Hq / Hkv)
    assert not ok(brute_causal(Q, K, V, sq, sk, Hq, Hkv, hd, sc, qo, kv_head=lambda h: h % Hkv))
    # dropped scale
    assert not ok(brute_causal(Q, K, V, sq, sk, Hq, Hkv, hd, 1.0, qo))
    # RoPE with the sign of the sine flipped, or pairs taken as interleaved
    pos = np.array([3, 50], np.int32)
    c, s = oracle.fill_rope_table(0, 51, hd, 1e4, False)
    x = rand(21, (2, hd))
    y = oracle.apply_rope(x, c[pos], s[pos], 2, 1, hd)
    assert np.allclose(y, _rope64(x, pos, hd, 1e4, False), atol=1e-5)
    assert not np.allclose(y, _rope64(x, -pos, hd, 1e4, False), atol=1e-5)
    assert not np.allclose(y, _rope64(x, pos, hd, 1e4, True), atol=1e-5)


def test_bf16_two_pass_attention(oracle):
    """qkn_bf16_decoder.c two-pass attention: truncating bf16 output of the exact result."""
    Hq, Hkv, hd, sq, sk, qo = 4, 1, 256, 6, 33, 27
    q = synth.f32_to_bf16_bits(rand(22, (sq, Hq * hd)))
    k = synth.f32_to_bf16_bits(rand(23, (sk, Hkv * hd)))
    v = synth.f32_to_bf16_bits(rand(24, (sk, Hkv * hd)))
    sc = 1.0 / np.sqrt(hd)
    for win, cap in [(0, 0.0), (8, 0.0), (0, 50.0)]:
        out = synth.bf16_bits_to_f32(oracle.bf16_attention(q, k, v, sq, sk, Hq, Hkv, hd, sc, qo,
                                                           window=win, cap=cap))
        want = brute_causal(synth.bf16_bits_to_f32(q), synth.bf16_bits_to_f32(k),
                            synth.bf16_bits_to_f32(v), sq, sk, Hq, Hkv, hd, sc, qo,
                            window=win, cap=cap)
        # the fp32 sums stray from float64 by at most `margin` (1e-5 relative plus 1e-6 for rows
        # that cancel: V is unit scale and the weights sum to 1)
        w32 = want.astype(np.float32)
        margin = 1e-5 * np.abs(w32) + 1e-6
        # truncation toward zero: |out| <= |want| and within one bf16 ulp (2^-7 relative) of it
        np.testing.assert_allclose(out, want, rtol=2 ** -7, atol=1e-6)
        assert (np.abs(out) <= np.abs(want) + margin).all()
        # the bits are the truncation of the float32 result wherever that result is farther
        # from a bf16 boundary than the margin
        t = synth.bf16_bits_to_f32((w32.view(np.uint32) >> 16).astype(np.uint16))
        step = np.abs(synth.bf16_bits_to_f32(((t.view(np.uint32) >> 16) + 1).astype(np.uint16)) - t)
        clear = (np.abs(w32 - t) > margin) & (np.abs(w32 - t) < step - margin)
        assert clear.mean() > 0.9
        np.testing.assert_array_equal(out[clear], t[clear])
        # planted: rounding to nearest instead of truncation breaks both checks
        rne = synth.bf16_bits_to_f32(synth.f32_to_bf16_bits(w32))
        assert (np.abs(rne) > np.abs(want) + margin).any()
        assert (rne[clear] != t[clear]).any()


# ------------------------------------------------------- per-head RMSNorm

def _norm64(x, w, seq, H, hd, eps):
    v = np.asarray(x, np.float64).reshape(seq, H, hd)
    r = 1.0 / np.sqrt((v * v).mean(-1, keepdims=True) + eps)
    return (v * r * np.asarray(w, np.float64)).reshape(seq, H * hd)


@pytest.mark.parametrize("hd", [64, 72, 80, 96, 128, 256])
def test_rms_norm_per_head_against_float64(oracle, hd):
    seq, H, eps = 3, 5, 1e-6
    x = rand(40 + hd, (seq, H * hd))
    w = 1.0 + 0.1 * rand(41 + hd, (hd,))
    for generic in (False, True):
        oracle.set_vec_generic(generic)
        try:
            y = oracle.rms_norm_per_head(x, w, seq, H, hd, eps)
        finally:
            oracle.set_vec_generic(False)
        np.testing.assert_allclose(y, _norm64(x, w, seq, H, hd, eps), rtol=2e-6, atol=1e-7)


def test_rms_norm_per_head_identities(oracle):
    seq, H, hd = 2, 3, 128
    x = rand(50, (seq, H * hd))
    one = np.ones(hd, np.float32)
    # unit weight: every head row has mean square ms / (ms + eps)
    for eps in (1e-6, 0.5):
        y = oracle.rms_norm_per_head(x, one, seq, H, hd, eps).reshape(seq, H, hd).astype(np.float64)
        ms = (x.reshape(seq, H, hd).astype(np.float64) ** 2).mean(-1)
        np.testing.assert_allclose((y ** 2).mean(-1), ms / (ms + eps), rtol=1e-5)
    # scale invariance (eps negligible) and linearity in the weight
    y1 = oracle.rms_norm_per_head(x, one, seq, H, hd, 1e-12)
    np.testing.assert_allclose(oracle.rms_norm_per_head(64.0 * x, one, seq, H, hd, 1e-12), y1, rtol=1e-6, atol=1e-7)
    w = 1.0 + 0.1 * rand(51, (hd,))
    np.testing.assert_allclose(oracle.rms_norm_per_head(x, 3.0 * w, seq, H, hd, 1e-6),
                               3.0 * oracle.rms_norm_per_head(x, w, seq, H, hd, 1e-6), rtol=1e-6, atol=1e-7)
    # a zero row stays zero; each head is normalised on its own
    z = x.copy()
    z[0, :hd] = 0.0
    yz = oracle.rms_norm_per_head(z, w, seq, H, hd, 1e-6)
    assert not yz[0, :hd].any()
    np.testing.assert_array_equal(yz[0, hd:], oracle.rms_norm_per_head(x, w, seq, H, hd, 1e-6)[0, hd:])


def test_rms_norm_planted_mistakes_are_caught(oracle):
    seq, H, hd, eps = 2, 4, 72, 1e-5
    x = 1e-3 * rand(52, (seq, H * hd))  # small values: eps is a visible part of the mean square
    w = 1.0 + 0.1 * rand(53, (hd,))
    y = oracle.rms_norm_per_head(x, w, seq, H, hd, eps)
    ok = lambda r: np.allclose(y, r, rtol=1e-5, atol=1e-7)  # noqa: E731
    assert ok(_norm64(x, w, seq, H, hd, eps))
    assert not ok(_norm64(x, w, seq, H, hd, 0.0))            # eps dropped
    assert not ok(_norm64(x, np.tile(w, H), seq, 1, H * hd, eps))  # one norm over all heads of a row
    assert not ok(_norm64(x, w[::-1].copy(), seq, H, hd, eps))  # weight reversed
    assert not ok(_norm64(x, np.ones(hd), seq, H, hd, eps))     # weight ignored


# ---- the bf16 decoder's truncating norm and rotation (qkn_bf16_decoder.c:73-91, :264-283)
#
# Brute force in exact rational arithmetic: every operation of the stated
# order is computed exactly and rounded once to float32 (round to nearest
# even), then truncated to bf16, independently of the C restatement.

from fractions import Fraction  # noqa: E402
import math  # noqa: E402


def _f32_round(q):
    """The float32 nearest to the rational q (ties to even), as a Fraction."""
    q = Fraction(q)
    if q == 0:
        return Fraction(0)
    sign = -1 if q < 0 else 1
    a = abs(q)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    e = max(e, -126)
    scaled = a / Fraction(2) ** (e - 23)
    m = scaled.numerator // scaled.denominator
    rem = scaled - m
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and m % 2 == 1):
        m += 1
    return sign * Fraction(m) * Fraction(2) ** (e - 23)


def _f32_sqrt(x):
    """Correctly rounded float32 square root of a float32 x >= 0."""
    r = Fraction(float(np.float32(math.sqrt(float(x)))))
    best = None
    for cand in (r, *(Fraction(float(np.nextafter(np.float32(r), np.float32(d)))) for d in (0, np.inf))):
        err = abs(cand * cand - x)
        if best is None or err < best[0]:
            best = (err, cand)
    return best[1]


def _bits(q):
    return int(np.float32(float(q)).view(np.uint32))


def _trunc16(q):
    return _bits(q) >> 16


def _widen16(b):
    return Fraction(float(np.uint32(int(b) << 16).view(np.float32)))


def _bf16_norm_exact(x, w, seq, H, hd, eps):
    y = np.array(x, np.uint16, copy=True).reshape(seq * H, hd)
    e = Fraction(float(np.float32(eps)))
    for r in range(seq * H):
        v = [_widen16(b) for b in y[r]]
        ss = Fraction(0)
        for a in v:
            ss = _f32_round(a * a + ss)
        ri = _f32_round(1 / _f32_sqrt(_f32_round(_f32_round(ss / hd) + e)))
        y[r] = [_trunc16(_f32_round(_f32_round(a * ri) * Fraction(float(w[d])))) for d, a in enumerate(v)]
    return y.reshape(seq, H * hd)


def _bf16_rope_exact(x, c, s, seq, H, hd):
    y = np.array(x, np.uint16, copy=True).reshape(seq, H, hd)
    for t in range(seq):
        for h in range(H):
            for i in range(hd // 2):
                x0, x1 = _widen16(y[t, h, 2 * i]), _widen16(y[t, h, 2 * i + 1])
                cc, sn = Fraction(float(c[t, 2 * i])), Fraction(float(s[t, 2 * i]))
                p1, p0 = _f32_round(x1 * sn), _f32_round(x0 * sn)
                y[t, h, 2 * i] = _trunc16(_f32_round(x0 * cc - p1))
                y[t, h, 2 * i + 1] = _trunc16(_f32_round(x1 * cc + p0))
    return y.reshape(seq, H * hd)


def _bf16_inputs(seed, shape):
    """bf16 bits over several binades (exponents 2^-6 .. 2^5), both signs"""
    r = np.random.default_rng(seed)
    v = r.standard_normal(shape) * np.exp2(r.integers(-6, 6, shape))
    return synth.f32_to_bf16_bits(v.astype(np.float32))


@pytest.mark.parametrize("hd,eps", [(8, 1e-6), (16, 1e-5), (8, 0.25)])
def test_bf16_norm_brute_force(oracle, hd, eps):
    seq, H = 3, 2
    x = _bf16_inputs(70 + hd, (seq, H * hd))
    w = (1.0 + 0.25 * np.random.default_rng(71).standard_normal(hd)).astype(np.float32)
    got = oracle.bf16_rms_norm_per_head(x, w, seq, H, hd, eps)
    np.testing.assert_array_equal(got, _bf16_norm_exact(x, w, seq, H, hd, eps))


@pytest.mark.parametrize("hd,theta", [(8, 1e4), (16, 1e6)])
def test_bf16_rope_brute_force(oracle, hd, theta):
    seq, H = 4, 3
    x = _bf16_inputs(80 + hd, (seq, H * hd))
    c, s = oracle.fill_rope_table(0, 4096, hd, theta, True)
    pos = np.array([0, 1, 1000, 4095])
    got = oracle.bf16_apply_rope_interleaved(x, c[pos], s[pos], seq, H, hd)
    np.testing.assert_array_equal(got, _bf16_rope_exact(x, c[pos], s[pos], seq, H, hd))
    # position 0 is the identity (cos 1, sin 0): the bits come back unchanged
    np.testing.assert_array_equal(got[0], x[0])


def test_bf16_norm_rope_planted_mistakes_are_caught(oracle):
    """Rounding to nearest instead of truncating, rotating with the partner
    swapped and the NeoX pairing all change bits that the restatement keeps.
    (Fusing or not fusing the first product moves a result by at most one
    float32 ulp, which survives the truncation to bf16 only rarely: the
    brute-force tests above pin that choice on their inputs.)"""
    seq, H, hd = 4, 4, 16
    x = _bf16_inputs(90, (seq, H * hd))
    w = np.ones(hd, np.float32)
    ref = oracle.bf16_rms_norm_per_head(x, w, seq, H, hd, 1e-6)
    xf = synth.bf16_bits_to_f32(x).reshape(seq * H, hd).astype(np.float64)
    r = 1.0 / np.sqrt((xf ** 2).mean(-1, keepdims=True) + 1e-6)
    rne = synth.f32_to_bf16_bits((xf * r).astype(np.float32)).reshape(seq, H * hd)
    trunc = ((xf * r).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16).reshape(seq, H * hd)
    assert (rne != ref).any()                                    # rounding to nearest
    assert np.abs(trunc.astype(np.int32) - ref.astype(np.int32)).max() <= 1   # float64 norm: within one step
    c, s = oracle.fill_rope_table(0, 2048, hd, 1e4, True)
    pos = np.array([3, 100, 1500, 2047])
    rot = oracle.bf16_apply_rope_interleaved(x, c[pos], s[pos], seq, H, hd).reshape(seq, H, hd // 2, 2)
    xv = synth.bf16_bits_to_f32(x).reshape(seq, H, hd // 2, 2).astype(np.float64)
    cc, ss = c[pos][:, None, 0::2], s[pos][:, None, 0::2]
    x0, x1 = xv[..., 0], xv[..., 1]
    tr = lambda a: (a.astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)  # noqa: E731
    good = np.stack([x0 * cc - x1 * ss, x1 * cc + x0 * ss], -1)
    assert np.abs(tr(good).astype(np.int32) - rot.astype(np.int32)).max() <= 1
    assert (synth.f32_to_bf16_bits(good.astype(np.float32)) != rot).any()          # rounding to nearest
    assert (tr(np.stack([x1 * cc - x0 * ss, x0 * cc + x1 * ss], -1)) != rot).any()  # partner swapped
    xn = synth.bf16_bits_to_f32(x).reshape(seq, H, 2, hd // 2).astype(np.float64)   # NeoX halves
    cn, sn = c[pos][:, None, :hd // 2], s[pos][:, None, :hd // 2]
    neox = np.stack([xn[:, :, 0] * cn - xn[:, :, 1] * sn, xn[:, :, 1] * cn + xn[:, :, 0] * sn], 2)
    assert (tr(neox).reshape(seq, H, hd // 2, 2) != rot).any()


@pytest.mark.parametrize("dim,eps", [(24, 1e-6), (40, 0.5)])
def test_bf16_row_norm_brute_force(oracle, dim, eps):
    """bf16_rms_norm over whole rows is the per-head norm with the row as one
    head: exact rational arithmetic, each step rounded to float32."""
    seq = 3
    x = _bf16_inputs(110 + dim, (seq, dim))
    w = (1.0 + 0.25 * np.random.default_rng(111).standard_normal(dim)).astype(np.float32)
    got = oracle.bf16_rms_norm(x, w, eps)
    np.testing.assert_array_equal(got, _bf16_norm_exact(x, w, seq, 1, dim, eps))
    # a per-head norm over halves of the row gives different bits
    assert (oracle.bf16_rms_norm_per_head(x, w[:dim // 2], seq, 2, dim // 2, eps) != got).any()


def test_bf16_add_exact(oracle):
    """trunc(a + b): the float32 sum of two bf16 values is correctly rounded
    by numpy, so the truncated bits are fixed; rounding to nearest differs."""
    a = _bf16_inputs(120, (4, 64))
    b = _bf16_inputs(121, (4, 64))
    got = oracle.bf16_add(a, b)
    s = synth.bf16_bits_to_f32(a) + synth.bf16_bits_to_f32(b)
    np.testing.assert_array_equal(got, (s.astype(np.float32).view(np.uint32) >> 16).astype(np.uint16))
    assert (synth.f32_to_bf16_bits(s.astype(np.float32)) != got).any()


def test_bf16_geglu_against_float64(oracle):
    """trunc(gelu_tanh(g) * u) within one bf16 step of the same formula
    evaluated step by step in numpy float32 (its tanh may differ from the C
    library's by an ulp), equal on most elements; planted mistakes (gate and
    up swapped, rounding to nearest, the erf GELU) are caught. (float64 is no
    reference here: for g below about -5, 1 + tanh cancels to 0 in float32.)"""
    inter = 256
    gu = _bf16_inputs(130, (3, 2 * inter))
    got = oracle.bf16_geglu(gu)
    v = synth.bf16_bits_to_f32(gu)
    g, u = v[:, 0::2], v[:, 1::2]
    f = np.float32

    def gelu(a):
        inner = f(0.7978845608028654) * (a + f(0.044715) * (a * a * a))
        return f(0.5) * a * (f(1.0) + np.tanh(inner))

    tr = lambda a: (a.astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)  # noqa: E731
    want = tr(gelu(g) * u)
    d = np.abs(want.astype(np.int32) - got.astype(np.int32))
    assert (d == 0).mean() > 0.95
    # one bf16 step, plus, where 1 + tanh cancels, an ulp of 1 times 0.5 g u
    err = np.abs(synth.bf16_bits_to_f32(got).astype(np.float64) - synth.bf16_bits_to_f32(want))
    bar = 2.0 ** -7 * np.abs(synth.bf16_bits_to_f32(want)) + 2.0 ** -22 * np.abs(0.5 * g * u)
    assert (err <= bar).all()
    assert (np.abs(tr(gelu(u) * g).astype(np.int32) - got.astype(np.int32)) > 1).any()
    assert (synth.f32_to_bf16_bits((gelu(g) * u).astype(np.float32)) != got).any()
    from scipy.special import erf
    g64 = g.astype(np.float64)
    gelu_erf = 0.5 * g64 * (1.0 + erf(g64 / np.sqrt(2.0)))
    assert (np.abs(tr(gelu_erf * u).astype(np.int32) - got.astype(np.int32)) > 1).any()
