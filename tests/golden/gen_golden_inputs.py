"""Seeded inputs of the golden fixtures (shared by gen_golden.py and the tests)."""
import hashlib
import os
import sys

import numpy as np

sys.path.insert(0, os.path.join(os.path.dirname(os.path.dirname(os.path.dirname(
    os.path.abspath(__file__)))), "smol-genius_amd"))
import synth  # noqa: E402


def digest(*arrays):
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()[:16]


def causal_inputs(seed, Hq, Hkv, hd, seq_q, seq_k):
    Q = synth.normal(seed * 3 + 0, (seq_q, Hq * hd))
    K = synth.normal(seed * 3 + 1, (seq_k, Hkv * hd))
    V = synth.normal(seed * 3 + 2, (seq_k, Hkv * hd))
    return Q, K, V


def bidir_inputs(seed, H, hd, seq, std):
    return tuple(synth.normal(seed * 3 + i, (seq, H * hd), std) for i in range(3))


def norm_inputs(seed, seq, H, hd, std):
    """x [seq, H*hd] and a per-head weight [hd] near 1 (loaders fold Gemma's
    1 + w into the stored weight, gemma.c:166-169)."""
    x = synth.normal(seed * 3 + 0, (seq, H * hd), std)
    w = (1.0 + 0.1 * synth.normal(seed * 3 + 1, (hd,))).astype(np.float32)
    return x, w


def linear_inputs(seed, seq, n_in, n_out, bias):
    """x [seq, n_in] ~N(0, 1) fp32, W [n_out, n_in] as bf16 bits of
    N(0, 1/n_in) samples (the scale of a trained projection), and a bias
    [n_out] ~N(0, 0.1) or None."""
    x = synth.normal(seed * 3 + 0, (seq, n_in))
    w = synth.f32_to_bf16_bits(synth.normal(seed * 3 + 1, (n_out, n_in), 1.0 / np.sqrt(max(n_in, 1))))
    b = synth.normal(seed * 3 + 2, (n_out,), 0.1) if bias else None
    return x, w, b


def norm_row_inputs(seed, seq, dim):
    """x [seq, dim] ~N(0, 1) and a weight [dim] near 1"""
    x = synth.normal(seed * 3 + 0, (seq, dim))
    w = (1.0 + 0.1 * synth.normal(seed * 3 + 1, (dim,))).astype(np.float32)
    return x, w


def glu_inputs(seed, seq, inter):
    """interleaved (gate, up) rows [seq, 2 * inter] ~N(0, 2^2)"""
    return synth.normal(seed * 3, (seq, 2 * inter), 2.0)
