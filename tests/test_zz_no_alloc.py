"""smol_attn_decode_noalloc, called through the C ABI, against
smol_attn_decode_qknorm on the same inputs: two calls in a row on one
context, the second smaller, each on two caches that hold the same rows.

Where both entry points split the work the same way (the scratch holds the
call's split partials) the outputs and the appended cache rows are
bit-identical. A call whose partials exceed the scratch runs unsplit on the
no-alloc side; its outputs then meet the path's bar
|a - b| <= 2e-3 + 1e-2 |b| against the splitting entry point.
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


def _dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _call(sa, fn, ctx, kv, rope, slots, pos, q, k, v, n_heads, hd, window, cap, qn, kn, out):
    slots = np.ascontiguousarray(slots, np.int32)
    pos = np.ascontiguousarray(pos, np.int32)
    ptr = lambda t: None if t is None else ctypes.c_void_p(t.data_ptr())  # noqa: E731
    return getattr(sa.load(), fn)(ctx.h, kv.h, 0, rope.h, len(slots), slots.ctypes.data_as(ctypes.POINTER(ctypes.c_int)),
                                  pos.ctypes.data_as(ctypes.POINTER(ctypes.c_int)), ptr(q), ptr(k), ptr(v), sa.F32,
                                  n_heads, ctypes.c_float(hd ** -0.5), window, ctypes.c_float(cap), ptr(qn), ptr(kn),
                                  ctypes.c_float(1e-6), ptr(out))


class Pair:
    """two caches with the same rows, one per entry point"""

    def __init__(self, sa, ctx, n_slots, Hq, Hkv, hd, lengths, seed, rope_type):
        self.sa, self.ctx, self.Hq, self.Hkv, self.hd = sa, ctx, Hq, Hkv, hd
        cap = 1024
        while cap < max(lengths) + 64:
            cap *= 2
        self.kv = [sa.KVCache(ctx, 1, n_slots, Hkv, hd, cap) for _ in range(2)]
        self.rope = sa.RopeTable(ctx, hd, 1e4 if rope_type else 1e6, rope_type, cap)
        for s, L in enumerate(lengths):
            kb = synth.f32_to_bf16_bits(synth.normal(seed + 2 * s, (L, Hkv * hd)))
            vb = synth.f32_to_bf16_bits(synth.normal(seed + 2 * s + 1, (L, Hkv * hd)))
            for kv in self.kv:
                kv.write(0, s, 0, kb, vb)
        self.qn = _dev((1.0 + 0.1 * synth.normal(seed + 90, (hd,))).astype(np.float32))
        self.kn = _dev((1.0 + 0.1 * synth.normal(seed + 91, (hd,))).astype(np.float32))

    def step(self, slots, pos, seed, window=0, cap=0.0, expect_exact=True):
        n, Hq, Hkv, hd = len(slots), self.Hq, self.Hkv, self.hd
        q = _dev(synth.normal(seed, (n, Hq * hd)))
        k = _dev(synth.normal(seed + 1, (n, Hkv * hd)))
        v = _dev(synth.normal(seed + 2, (n, Hkv * hd)))
        outs = []
        for fn, kv in (("smol_attn_decode_qknorm", self.kv[0]), ("smol_attn_decode_noalloc", self.kv[1])):
            out = torch.full((n, Hq * hd), float("nan"), device="cuda")
            print("no-alloc", fn, "n_seq", n, "Hq", Hq, "Hkv", Hkv, "hd", hd, "pos", list(pos)[:4], flush=True)
            rc = _call(self.sa, fn, self.ctx, kv, self.rope, slots, pos, q, k, v, Hq, hd, window, cap, self.qn,
                       self.kn, out)
            assert rc == 0, (fn, rc, self.sa.load().smol_attn_last_error())
            torch.cuda.synchronize()
            outs.append(out.cpu().numpy())
        if expect_exact:
            np.testing.assert_array_equal(outs[1], outs[0])
        else:
            assert_parity(outs[1], outs[0], "no-alloc unsplit vs split")
        for s, p in zip(slots, pos):
            a = self.kv[0].read(0, s, p, 1)
            b = self.kv[1].read(0, s, p, 1)
            np.testing.assert_array_equal(a[0], b[0])
            np.testing.assert_array_equal(a[1], b[1])
        return outs

    def close(self):
        for kv in self.kv:
            kv.close()
        self.rope.close()


def test_noalloc_matches_decode_two_calls(sa):
    ctx = sa.Context(0)
    try:
        # MQA decode of 16 sequences (hd 256), then 3 shorter ones on other slots
        lengths = [int(x) for x in 512 + np.random.default_rng(5).integers(0, 3585, 16)] + [100, 40, 7]
        pr = Pair(sa, ctx, 19, 8, 1, 256, lengths, 700, 1)
        pr.step(list(range(16)), [L - 1 for L in lengths[:16]], 800, cap=50.0)
        pr.step([16, 17, 18], [99, 39, 6], 810, window=24)
        # the same two calls again: the scratch keeps the last call's contents
        pr.step(list(range(16)), [L for L in lengths[:16]], 820)
        pr.step([16, 17, 18], [100, 40, 7], 830)
        pr.close()
        # GQA, 28 sequences of 1025 keys: the split partials exceed the
        # scratch, so the no-alloc call runs unsplit
        pr = Pair(sa, ctx, 28, 16, 8, 128, [1024] * 28, 900, 0)
        pr.step(list(range(28)), [1024] * 28, 950, expect_exact=False)
        pr.step([3, 5], [1025, 1025], 960)
        pr.close()
    finally:
        ctx.close()


def test_noalloc_limits(sa):
    ctx = sa.Context(0)
    try:
        pr = Pair(sa, ctx, 40, 8, 1, 128, [64] * 40, 1000, 0)
        q = _dev(synth.normal(1, (40, 8 * 128)))
        kv1 = _dev(synth.normal(2, (40, 128)))
        out = torch.zeros((40, 8 * 128), device="cuda")
        rc = _call(sa, "smol_attn_decode_noalloc", ctx, pr.kv[1], pr.rope, list(range(33)), [64] * 33, q, kv1, kv1, 8,
                   128, 0, 0.0, None, None, out)
        assert rc == -4 and b"at most 32" in sa.load().smol_attn_last_error()
        cap = pr.kv[1].capacity
        rc = _call(sa, "smol_attn_decode_noalloc", ctx, pr.kv[1], pr.rope, [0], [cap], q, kv1, kv1, 8, 128, 0, 0.0,
                   None, None, out)
        assert rc == -1 and b"reserve" in sa.load().smol_attn_last_error()
        assert pr.kv[1].capacity == cap   # nothing grew
        pr.close()
    finally:
        ctx.close()
