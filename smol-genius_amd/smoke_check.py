"""One small decode and one small chunked prefill on cuda:0, checked against the CPU oracle.

Used by __graft_entry__.smoke(). The oracle (oracle/) is the checker here,
never the thing computed: the outputs come from libsmol_attn.so.
"""
import numpy as np

ATOL, RTOL = 2e-3, 1e-2


def _check(name, got, want):
    d = np.abs(got.astype(np.float64) - want)
    ratio = float((d / (ATOL + RTOL * np.abs(want))).max())
    print("smoke %-8s max_abs %.3e ratio %.3f" % (name, d.max(), ratio), flush=True)
    if not np.isfinite(got).all() or ratio > 1.0:
        raise AssertionError("smoke %s: GPU output differs from the oracle" % name)


def run():
    import torch
    from oracle import Oracle
    import workload_oracle as wo

    from . import runner, smol_attn as sa
    from .workloads import Decode, Prefill

    if not torch.cuda.is_available():
        raise RuntimeError("smoke needs a GPU")
    sa.load()
    orc = Oracle()
    ctx = sa.Context(0)
    dec = Decode("smoke_decode", 16, 8, 128, [77, 300], 1e6, 0, seed=11)
    x = dec.inputs()
    r = runner.prepare(ctx, dec, x)
    r.step()
    _check("decode", r.outputs(), wo.decode(orc, dec, x))
    pre = Prefill("smoke_prefill", 8, 2, 128, 40, 50, 1e6, seed=12)
    x = pre.inputs()
    r = runner.prepare(ctx, pre, x)
    r.step()
    _check("prefill", r.outputs(), wo.prefill(orc, pre, x))
    r.kv.close()
    r.rope.close()
    ctx.close()
