"""Runs the workloads of workloads.py through the C ABI on one GPU.

``prepare(ctx, wl, inputs, layers=1)`` uploads the inputs, fills the device KV
cache(s) and returns a ``Run`` whose ``step()`` enqueues one pass of the path
(calls whose arguments were converted once, so the host issues a step in a few
microseconds and short kernels run back to back instead of each waking an idle
GPU)
(on the context's stream) and whose ``outputs()`` returns the fp32 results
as numpy. ``layers > 1`` gives every layer its own cache region and inputs,
so repeated steps stream distinct HBM buffers instead of re-reading data
that is still in the 256 MB last-level cache.
"""
import numpy as np

from . import smol_attn as sa
from .workloads import ROPE_INTERLEAVED, Bidir, Decode, Prefill, Stream


def _t(a, device, bf16=False):
    import torch
    if bf16:
        return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).to(device).view(torch.bfloat16)
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(device)


class Run:
    def __init__(self):
        self.layer = 0
        self.n_layers = 1
        self.outs = []

    def step(self):
        """one pass over the next layer (round-robin); returns the output tensor(s)"""
        r = self._step(self.layer)
        self.layer = (self.layer + 1) % self.n_layers
        return r

    def outputs(self, layer=0):
        import torch
        torch.cuda.synchronize()
        o = self.outs[layer]
        if isinstance(o, list):
            return [x.cpu().numpy() for x in o]
        return o.cpu().numpy()


def _norm_tensors(wl, device):
    qw, kw = wl.norm_weights()
    return tuple(None if w is None else _t(w, device) for w in (qw, kw))


def _fill_cache(kv, layer, slot, ck, cv):
    if len(ck):
        kv.write(layer, slot, 0, ck, cv)


def prepare(ctx, wl, inputs, layers=1, device="cuda"):
    if isinstance(wl, Decode):
        return _prep_decode(ctx, wl, inputs, layers, device)
    if isinstance(wl, Prefill):
        return _prep_prefill(ctx, wl, inputs, layers, device)
    if isinstance(wl, Bidir):
        return _prep_bidir(ctx, wl, inputs, layers, device)
    if isinstance(wl, Stream):
        return _prep_stream(ctx, wl, inputs, layers, device)
    raise TypeError(wl)


def _prep_decode(ctx, wl, x, layers, device):
    import torch
    r = Run()
    r.n_layers = layers
    r.kv = sa.KVCache(ctx, layers, wl.n_seq, wl.Hkv, wl.hd, max(wl.lengths))
    r.rope = sa.RopeTable(ctx, wl.hd, wl.theta, wl.rope_type, max(wl.lengths))
    for l in range(layers):
        for i in range(wl.n_seq):
            _fill_cache(r.kv, l, i, x["cache_k"][i], x["cache_v"][i])
    torch.cuda.synchronize()
    r.q = [_t(x["q"], device) for _ in range(layers)]
    r.k = [_t(x["k"], device) for _ in range(layers)]
    r.v = [_t(x["v"], device) for _ in range(layers)]
    r.outs = [torch.empty((wl.n_seq, wl.Hq * wl.hd), dtype=torch.float32, device=device) for _ in range(layers)]
    slots = np.arange(wl.n_seq, dtype=np.int32)
    pos = wl.positions
    qn, kn = _norm_tensors(wl, device)

    calls = [sa.decode_call(ctx, r.kv, l, r.rope, slots, pos, r.q[l], r.k[l], r.v[l], wl.Hq, wl.scale,
                            out=r.outs[l], q_norm=qn, k_norm=kn, eps=wl.norm_eps) for l in range(layers)]
    r._step = lambda l: calls[l]()
    return r


def _prep_prefill(ctx, wl, x, layers, device):
    import torch
    r = Run()
    r.n_layers = layers
    r.kv = sa.KVCache(ctx, layers, 1, wl.Hkv, wl.hd, wl.pos0 + wl.seq_q)
    r.rope = sa.RopeTable(ctx, wl.hd, wl.theta, wl.rope_type, wl.pos0 + wl.seq_q)
    for l in range(layers):
        _fill_cache(r.kv, l, 0, x["cache_k"], x["cache_v"])
    torch.cuda.synchronize()
    bf = wl.in_bf16
    r.q = [_t(x["q"], device, bf) for _ in range(layers)]
    r.k = [_t(x["k"], device, bf) for _ in range(layers)]
    r.v = [_t(x["v"], device, bf) for _ in range(layers)]
    r.outs = [torch.empty((wl.seq_q, wl.Hq * wl.hd), dtype=torch.float32, device=device) for _ in range(layers)]
    qn, kn = _norm_tensors(wl, device)

    calls = [sa.prefill_call(ctx, r.kv, l, 0, r.rope, wl.pos0, r.q[l], r.k[l], r.v[l], wl.Hq, wl.scale,
                             out=r.outs[l], q_norm=qn, k_norm=kn, eps=wl.norm_eps) for l in range(layers)]
    r._step = lambda l: calls[l]()
    return r


def _prep_bidir(ctx, wl, x, layers, device):
    import torch
    r = Run()
    r.n_layers = layers
    r.q = [_t(x["q"], device, wl.in_bf16) for _ in range(layers)]
    r.k = [_t(x["k"], device, wl.in_bf16) for _ in range(layers)]
    r.v = [_t(x["v"], device, wl.in_bf16) for _ in range(layers)]
    r.outs = [torch.empty((wl.seq, wl.H * wl.hd), dtype=torch.float32, device=device) for _ in range(layers)]

    calls = [sa.bidirectional_call(ctx, r.q[l], r.k[l], r.v[l], wl.seq, wl.H, wl.hd, wl.scale, wl.window_starts,
                                   out=r.outs[l]) for l in range(layers)]
    r._step = lambda l: calls[l]()
    return r


def _prep_stream(ctx, wl, x, layers, device):
    import torch
    r = Run()
    r.n_layers = layers
    total = wl.prefix + wl.chunk + wl.steps
    r.kv = sa.KVCache(ctx, layers, 1, wl.Hkv, wl.hd, total)
    r.rope = sa.RopeTable(ctx, wl.hd, wl.theta, wl.rope_type, total)
    for l in range(layers):
        _fill_cache(r.kv, l, 0, x["cache_k"], x["cache_v"])
    torch.cuda.synchronize()
    r.q = [_t(x["q"], device) for _ in range(layers)]
    r.k = [_t(x["k"], device) for _ in range(layers)]
    r.v = [_t(x["v"], device) for _ in range(layers)]
    r.dq = [_t(x["dq"], device) for _ in range(layers)]
    r.dk = [_t(x["dk"], device) for _ in range(layers)]
    r.dv = [_t(x["dv"], device) for _ in range(layers)]
    r.outs = [[torch.empty((wl.chunk, wl.Hq * wl.hd), dtype=torch.float32, device=device),
               torch.empty((wl.steps, wl.Hq * wl.hd), dtype=torch.float32, device=device)] for _ in range(layers)]
    slot0 = np.zeros(1, np.int32)
    calls = []
    for l in range(layers):
        oc, od = r.outs[l]
        cl = [sa.prefill_call(ctx, r.kv, l, 0, r.rope, wl.prefix, r.q[l], r.k[l], r.v[l], wl.Hq, wl.scale, out=oc)]
        for s in range(wl.steps):
            p = np.array([wl.prefix + wl.chunk + s], np.int32)
            cl.append(sa.decode_call(ctx, r.kv, l, r.rope, slot0, p, r.dq[l][s:s + 1], r.dk[l][s:s + 1],
                                     r.dv[l][s:s + 1], wl.Hq, wl.scale, out=od[s:s + 1]))
        calls.append(cl)

    def _step(l):
        for c in calls[l]:
            c()
        return r.outs[l]
    r._step = _step
    return r
