"""The CPU oracle of the bf16-weight projections, pinned.

* golden vectors written by the reference's own matmul.c / bf16_matvec_*.c,
  compiled by oracle/Makefile (tests/golden/gen_golden_linear.py), for every
  entry point: smol_linear_bf16 (with and without bias, matvec and loop
  paths), smol_linear_nobias_bf16_qkv, smol_matmul_t_bf16;
* a float64 brute force with the fp32 summation bound;
* closed forms: identity weights, integer-valued inputs (every partial sum
  exact in fp32, so any order gives the same bits), bias only;
* the bf16 decoder's truncating projection against exact integer sums;
* planted mistakes (transposed weights, dropped bias, bf16-rounded x, RNE
  instead of truncation) that the same checks reject.
"""
import json
import os

import numpy as np
import pytest

from conftest import GOLDEN, synth
from gen_golden_inputs import digest, linear_inputs


@pytest.fixture(scope="module")
def golden_linear():
    with open(os.path.join(GOLDEN, "ref_linear.json")) as f:
        meta = json.load(f)
    return meta, np.load(os.path.join(GOLDEN, "ref_linear.npz"))


def fp32_bound(x, w32, b=None):
    """|fp32 sum - exact| <= n * 2^-24 * sum |terms| (terms in any order)"""
    a = np.abs(np.asarray(x, np.float64)) @ np.abs(np.asarray(w32, np.float64)).T
    if b is not None:
        a = a + np.abs(np.asarray(b, np.float64))
    n = w32.shape[1] + 1
    return a * n * 2.0 ** -24 + 1e-30


def w32_of(bits):
    return synth.bf16_bits_to_f32(bits).astype(np.float64)


def case_inputs(c):
    return linear_inputs(c["seed"], c["seq"], c["in_dim"], c["out_dim"], c["bias"])


def test_golden_inputs_unchanged(golden_linear):
    meta, _ = golden_linear
    assert len(meta["cases"]) == 11
    for c in meta["cases"]:
        if c["kind"] == "qkv":
            continue
        x, w, b = case_inputs(c)
        assert (digest(x, w) if b is None else digest(x, w, b)) == c["digest"]


@pytest.mark.parametrize("idx", range(11))
def test_oracle_matches_reference(golden_linear, oracle, idx):
    meta, data = golden_linear
    c = meta["cases"][idx]
    if c["kind"] == "qkv":
        x, wq, _ = linear_inputs(c["seed"], 1, c["in_dim"], c["out_dim"], False)
        _, wk, _ = linear_inputs(c["seed"] + 100, 1, c["in_dim"], c["out_dim"] // 2, False)
        _, wv, _ = linear_inputs(c["seed"] + 200, 1, c["in_dim"], c["out_dim"] // 2, False)
        assert digest(x, wq, wk, wv) == c["digest"]
        for w, tag in ((wq, "_q"), (wk, "_k"), (wv, "_v")):
            y = oracle.linear_bf16(x, w)[0]
            bound = fp32_bound(x, w32_of(w))[0] * 2
            assert (np.abs(y.astype(np.float64) - data[c["name"] + tag]) <= bound).all()
        return
    x, w, b = case_inputs(c)
    y = oracle.linear_bf16(x, w, b)
    ref = data[c["name"]]
    # both are fp32 sums of the same products; the reference's order differs
    bound = 2 * fp32_bound(x, w32_of(w), b)
    assert (np.abs(y.astype(np.float64) - ref) <= bound).all()


@pytest.mark.parametrize("seq,n_in,n_out", [(1, 64, 8), (3, 72, 5), (2, 7, 3), (4, 300, 17)])
def test_brute_force_float64(oracle, seq, n_in, n_out):
    x, w, b = linear_inputs(77 + n_in, seq, n_in, n_out, True)
    y = oracle.linear_bf16(x, w, b).astype(np.float64)
    exact = x.astype(np.float64) @ w32_of(w).T + b
    assert (np.abs(y - exact) <= fp32_bound(x, w32_of(w), b)).all()
    y0 = oracle.linear_bf16(x, w).astype(np.float64)
    assert (np.abs(y0 - (exact - b)) <= fp32_bound(x, w32_of(w))).all()


def test_closed_forms(oracle):
    # identity weights: y = x exactly
    n = 40
    x = synth.normal(5, (3, n))
    eye = synth.f32_to_bf16_bits(np.eye(n, dtype=np.float32))
    np.testing.assert_array_equal(oracle.linear_bf16(x, eye), x)
    # a weight row with one non-zero entry picks (and scales by a power of two) one input
    w = np.zeros((2, n), np.float32)
    w[0, 7] = 1.0
    w[1, 31] = -0.25
    y = oracle.linear_bf16(x, synth.f32_to_bf16_bits(w))
    np.testing.assert_array_equal(y[:, 0], x[:, 7])
    np.testing.assert_array_equal(y[:, 1], -0.25 * x[:, 31])
    # integer-valued inputs: every partial sum is an integer below 2^24, exact in any order
    rng = np.random.default_rng(3)
    xi = rng.integers(-8, 9, (5, 200)).astype(np.float32)
    wi = rng.integers(-8, 9, (11, 200)).astype(np.float32)
    bi = rng.integers(-50, 51, 11).astype(np.float32)
    y = oracle.linear_bf16(xi, synth.f32_to_bf16_bits(wi), bi)
    np.testing.assert_array_equal(y, (xi.astype(np.int64) @ wi.astype(np.int64).T + bi.astype(np.int64)))
    # zero input: the bias (or zero)
    np.testing.assert_array_equal(oracle.linear_bf16(np.zeros((2, 9), np.float32), synth.f32_to_bf16_bits(wi[:, :9]), bi),
                                  np.broadcast_to(bi, (2, 11)))


def test_bf16_linear_truncates(oracle):
    rng = np.random.default_rng(4)
    # exact integer sums: the output is the truncated exact value, bit for bit
    xi = rng.integers(-16, 17, (3, 96)).astype(np.float32)
    wi = rng.integers(-16, 17, (7, 96)).astype(np.float32)
    y = oracle.bf16_linear_nobias(synth.f32_to_bf16_bits(xi), synth.f32_to_bf16_bits(wi))
    exact = (xi.astype(np.int64) @ wi.astype(np.int64).T).astype(np.float32)
    np.testing.assert_array_equal(y, (exact.view(np.uint32) >> 16).astype(np.uint16))
    # 256 + 2 + 1 = 259 (0x43818000) truncates to 258 where round-to-nearest-even gives 260
    xs = synth.f32_to_bf16_bits(np.array([[1.0, 1.0, 1.0]], np.float32))
    ws = synth.f32_to_bf16_bits(np.array([[256.0, 2.0, 1.0]], np.float32))
    assert synth.bf16_bits_to_f32(oracle.bf16_linear_nobias(xs, ws))[0, 0] == 258.0
    # random inputs: within one bf16 step below the float64 value
    xb = synth.f32_to_bf16_bits(synth.normal(8, (4, 128)))
    wb = synth.f32_to_bf16_bits(synth.normal(9, (9, 128), 0.1))
    y = synth.bf16_bits_to_f32(oracle.bf16_linear_nobias(xb, wb)).astype(np.float64)
    ex = w32_of(xb) @ w32_of(wb).T
    assert (np.abs(y) <= np.abs(ex) * (1 + 1e-5) + 1e-6).all()
    assert (np.abs(ex - y) <= np.abs(ex) * 2.0 ** -7 + 1e-6).all()


def test_planted_mistakes_are_caught(golden_linear, oracle):
    """Mutated restatements (float64, numpy) fail the checks the oracle passes."""
    meta, data = golden_linear
    c = next(c for c in meta["cases"] if c["name"] == "lin_s5_1000_33_b")
    x, w, b = case_inputs(c)
    ref = data[c["name"]].astype(np.float64)
    w32 = w32_of(w)
    bound = 2 * fp32_bound(x, w32, b)

    def ok(y):
        return bool((np.abs(np.asarray(y, np.float64) - ref) <= bound).all())

    assert ok(oracle.linear_bf16(x, w, b))
    assert ok(x.astype(np.float64) @ w32.T + b)                     # the float64 truth passes
    assert not ok(x.astype(np.float64) @ w32.T)                     # dropped bias
    xr = synth.bf16_bits_to_f32(synth.f32_to_bf16_bits(x)).astype(np.float64)
    assert not ok(xr @ w32.T + b)                                   # x rounded to bf16 (no lo part)
    wt = w32.reshape(w32.shape[1], w32.shape[0]).T
    assert not ok(x.astype(np.float64) @ wt.T + b)                  # weights read transposed
    assert not ok(x.astype(np.float64)[:, ::-1] @ w32.T + b)        # input read backwards
    # the bf16 projection: RNE instead of truncation is caught by the exact-sum case
    xs = synth.f32_to_bf16_bits(np.array([[1.0, 1.0, 1.0]], np.float32))
    ws = synth.f32_to_bf16_bits(np.array([[256.0, 2.0, 1.0]], np.float32))
    rne = synth.bf16_bits_to_f32(synth.f32_to_bf16_bits(np.array([259.0], np.float32)))[0]
    assert rne == 260.0 and synth.bf16_bits_to_f32(oracle.bf16_linear_nobias(xs, ws))[0, 0] != rne


# ------------------------------------------------- RMSNorm and the gated activations

def test_rms_norm_matches_reference(golden_linear, oracle):
    from gen_golden_inputs import norm_row_inputs
    meta, data = golden_linear
    assert len(meta["norm"]) == 4
    for c in meta["norm"]:
        x, w = norm_row_inputs(c["seed"], c["seq"], c["dim"])
        assert digest(x, w) == c["digest"]
        y = oracle.rms_norm(x, w, c["eps"])
        np.testing.assert_allclose(y, data[c["name"]], rtol=4e-6, atol=1e-7)


def test_rms_norm_closed_forms(oracle):
    # a constant row normalises to the weight times the sign; float64 brute force elsewhere
    w = (1.0 + 0.1 * synth.normal(41, (96,))).astype(np.float32)
    x = np.full((2, 96), 3.0, np.float32)
    x[1] *= -1
    y = oracle.rms_norm(x, w, 0.0)
    np.testing.assert_allclose(y[0], w, rtol=2e-7)
    np.testing.assert_allclose(y[1], -w, rtol=2e-7)
    x = synth.normal(42, (3, 200), 5.0)
    w2 = (1.0 + 0.1 * synth.normal(43, (200,))).astype(np.float32)
    r = 1.0 / np.sqrt((x.astype(np.float64) ** 2).mean(1, keepdims=True) + 1e-5)
    np.testing.assert_allclose(oracle.rms_norm(x, w2, 1e-5), x * w2 * r, rtol=2e-6)
    # eps matters for a tiny row
    t = np.full((1, 16), 1e-4, np.float32)
    np.testing.assert_allclose(oracle.rms_norm(t, np.ones(16, np.float32), 1e-6)[0],
                               1e-4 / np.sqrt(1e-8 + 1e-6), rtol=1e-5)


def test_glu_matches_reference(golden_linear, oracle):
    from gen_golden_inputs import glu_inputs
    meta, data = golden_linear
    assert len(meta["glu"]) == 4
    for c in meta["glu"]:
        gu = glu_inputs(c["seed"], c["seq"], c["inter"])
        assert digest(gu) == c["digest"]
        np.testing.assert_allclose(oracle.glu(gu, c["act"]), data[c["name"]], rtol=5e-5, atol=1e-6)


def test_glu_closed_forms_and_float64(oracle):
    gu = np.array([[0.0, 5.0, 30.0, 2.0, -30.0, 2.0, 1.0, 1.0]], np.float32)
    s = oracle.glu(gu, 1)[0]
    assert s[0] == 0.0 and abs(s[1] - 60.0) < 1e-4 and abs(s[2]) < 1e-10
    g = oracle.glu(gu, 2)[0]
    assert g[0] == 0.0 and abs(g[1] - 60.0) < 1e-4 and abs(g[2]) < 1e-10
    x = synth.normal(44, (3, 2 * 64), 2.0).astype(np.float64)
    gate, up = x[:, 0::2], x[:, 1::2]
    silu = gate / (1 + np.exp(-gate)) * up
    gelu = 0.5 * gate * (1 + np.tanh(np.sqrt(2 / np.pi) * (gate + 0.044715 * gate ** 3))) * up
    np.testing.assert_allclose(oracle.glu(x, 1), silu, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(oracle.glu(x, 2), gelu, rtol=1e-5, atol=1e-6)
    # planted: gate and up swapped, or the pairs read as halves, are caught
    assert not np.allclose(up / (1 + np.exp(-up)) * gate, oracle.glu(x, 1), rtol=1e-3)
    halves = x[:, :64] / (1 + np.exp(-x[:, :64])) * x[:, 64:]
    assert not np.allclose(halves, oracle.glu(x, 1), rtol=1e-3)
