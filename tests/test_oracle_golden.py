"""The CPU oracle against the golden vectors written by the compiled reference.

The fixtures in tests/golden/ come from the reference's own attention.c /
rope.c / vecops / threading.c, compiled by oracle/Makefile (see
tests/golden/gen_golden.py). Inputs are regenerated from the recorded seeds;
their checksum must match the one stored with the outputs.
"""
import numpy as np
import pytest

from conftest import synth
from gen_golden_inputs import bidir_inputs, causal_inputs, digest


def _meta(golden, kind):
    return golden[0][kind]


def test_fixture_generator_unchanged(golden):
    meta, _ = golden
    for c in meta["causal"][:3]:
        Q, K, V = causal_inputs(c["seed"], c["Hq"], c["Hkv"], c["hd"], c["seq_q"], c["seq_k"])
        assert digest(Q, K, V) == c["digest"]


@pytest.mark.parametrize("idx", range(23))
def test_causal_matches_reference(golden, oracle, idx):
    meta, data = golden
    c = meta["causal"][idx]
    Q, K, V = causal_inputs(c["seed"], c["Hq"], c["Hkv"], c["hd"], c["seq_q"], c["seq_k"])
    assert digest(Q, K, V) == c["digest"]
    out = oracle.causal_attention(Q, K, V, c["seq_q"], c["seq_k"], c["Hq"], c["Hkv"], c["hd"],
                                  c["scale"], c["q_offset"], window=c["window"], cap=c["cap"],
                                  kind=c["kind"])
    np.testing.assert_allclose(out, data[c["name"]], rtol=1e-5, atol=1e-5)


def test_golden_case_count(golden):
    assert len(golden[0]["causal"]) == 23


@pytest.mark.parametrize("idx", range(5))
def test_bidirectional_matches_reference(golden, oracle, idx):
    meta, data = golden
    b = meta["bidir"][idx]
    seq = b["window_starts"][-1]
    Q, K, V = bidir_inputs(b["seed"], b["H"], b["hd"], seq, b["std"])
    assert digest(Q, K, V) == b["digest"]
    out = oracle.bidirectional_attention(Q, K, V, seq, b["H"], b["hd"], b["scale"],
                                         b["window_starts"])
    np.testing.assert_allclose(out, data[b["name"]], rtol=1e-5, atol=1e-5)


def test_rope_tables_match_reference(golden, oracle):
    meta, data = golden
    for r in meta["rope"]:
        pos = np.array(r["positions"], np.int32)
        c, s = oracle.compute_rope(pos, r["hd"], r["theta"], interleaved=r["interleaved"])
        # The reference is built with -ffast-math, which computes the frequency
        # 1/powf(theta, 2d/hd) to within ~1 ulp; the angle error grows with pos.
        tol = 2e-7 * pos[:, None].astype(np.float64) + 2e-7
        assert (np.abs(c - data[r["tag"] + "_cos"]) <= tol).all(), r["tag"]
        assert (np.abs(s - data[r["tag"] + "_sin"]) <= tol).all(), r["tag"]
        # fill_rope_table (the decoder's table, qkn_decoder.c:276-311) uses the
        # same formula as compute_rope (rope.c:27-66): rows must agree exactly.
        for p in r["positions"]:
            ct, st = oracle.fill_rope_table(p, 1, r["hd"], r["theta"], r["interleaved"])
            k = r["positions"].index(p)
            assert np.array_equal(ct[0], c[k]) and np.array_equal(st[0], s[k])


def test_rope_apply_matches_reference(golden, oracle):
    meta, data = golden
    for r in meta["rope"]:
        n = len(r["positions"])
        x = synth.normal(r["seed"], (n, 3 * r["hd"]))
        assert digest(x) == r["digest"]
        # the reference's tables are the input here, so only the rotation is compared
        y = oracle.apply_rope(x, data[r["tag"] + "_cos"], data[r["tag"] + "_sin"], n, 3, r["hd"],
                              interleaved=r["interleaved"])
        np.testing.assert_allclose(y, data[r["tag"] + "_applied"], rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("idx", range(8))
def test_rms_norm_per_head_matches_reference(golden, oracle, idx):
    from gen_golden_inputs import norm_inputs
    meta, data = golden
    n = meta["norm"][idx]
    x, w = norm_inputs(n["seed"], n["seq"], n["H"], n["hd"], n["std"])
    assert digest(x, w) == n["digest"]
    y = oracle.rms_norm_per_head(x, w, n["seq"], n["H"], n["hd"], n["eps"])
    # the reference is built with -ffast-math (1/sqrtf may become an estimate
    # refined by one Newton step); the restatement computes it exactly
    np.testing.assert_allclose(y, data[n["name"]], rtol=2e-6, atol=1e-7 * n["std"])
