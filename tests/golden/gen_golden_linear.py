"""Writes the projection fixtures (ref_linear.json / ref_linear.npz) from the
compiled reference.

The reference's common/kernels/matmul.c, bf16_matvec_{avx,generic}.c,
rmsnorm.c, activation.c and threading.c are compiled by ``oracle/Makefile`` into ``oracle/_ref/``; this
script calls smol_linear_bf16, smol_linear_nobias_bf16,
smol_linear_nobias_bf16_qkv, smol_matmul_t_bf16, smol_rms_norm,
smol_swiglu_multiply and smol_geglu_multiply there (one thread) on
seeded inputs and stores the outputs. Inputs are regenerated from the seeds by
``linear_inputs``; their checksum is stored with the outputs.

Run from the repository root:  python tests/golden/gen_golden_linear.py
"""
import json
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
from oracle import RefLib, simd_branch  # noqa: E402
from gen_golden_inputs import digest, glu_inputs, linear_inputs, norm_row_inputs  # noqa: E402

OUT = os.path.dirname(os.path.abspath(__file__))

# (name, kind, seq, in_dim, out_dim, bias). kind: "linear" (smol_linear_bf16 /
# smol_linear_nobias_bf16), "qkv" (out_dim = q_dim, kv_dim = out_dim // 2),
# "matmul_t" (smol_matmul_t_bf16: M = seq, K = in_dim, N = out_dim).
# seq 1 takes the reference's matvec (bf16_matvec_fused), seq > 1 its loops;
# in_dim 72 / 1000 / 7 are not multiples of the SIMD widths.
CASES = [
    ("lin_s1_1024_512_b", "linear", 1, 1024, 512, True),
    ("lin_s1_1024_256", "linear", 1, 1024, 256, False),
    ("lin_s1_7_5_b", "linear", 1, 7, 5, True),
    ("lin_s3_72_40", "linear", 3, 72, 40, False),
    ("lin_s5_1000_33_b", "linear", 5, 1000, 33, True),
    ("lin_s26_512_96", "linear", 26, 512, 96, False),
    ("lin_s2_3072_64", "linear", 2, 3072, 64, False),
    ("qkv_1024_256", "qkv", 1, 1024, 256, False),
    ("qkv_72_24", "qkv", 1, 72, 24, False),
    ("mmt_4_256_130", "matmul_t", 4, 256, 130, False),
    ("mmt_1_128_64", "matmul_t", 1, 128, 64, False),
]


# (seq, dim) of the full-row RMSNorm cases; 72 and 7 have a scalar tail
NORM_ROWS = [(1, 1024), (3, 2048), (2, 72), (2, 7)]
# (seq, intermediate, act): 1 SwiGLU, 2 GeGLU
GLU = [(1, 3072, 1), (4, 100, 1), (1, 3072, 2), (3, 17, 2)]


def main():
    ref = RefLib()
    ref.set_threads(1)
    arrays, meta = {}, {"simd": simd_branch(), "ref": os.path.basename(ref.path), "cases": []}
    for i, (name, kind, seq, n_in, n_out, has_b) in enumerate(CASES):
        seed = 5000 + i
        if kind == "qkv":
            x, wq, _ = linear_inputs(seed, 1, n_in, n_out, False)
            _, wk, _ = linear_inputs(seed + 100, 1, n_in, n_out // 2, False)
            _, wv, _ = linear_inputs(seed + 200, 1, n_in, n_out // 2, False)
            q, k, v = ref.linear_qkv(x, wq, wk, wv)
            arrays[name + "_q"], arrays[name + "_k"], arrays[name + "_v"] = q, k, v
            dg = digest(x, wq, wk, wv)
        else:
            x, w, b = linear_inputs(seed, seq, n_in, n_out, has_b)
            if kind == "matmul_t":
                arrays[name] = ref.matmul_t_bf16(x, w)
            else:
                arrays[name] = ref.linear_bf16(x, w, b)
            dg = digest(x, w) if b is None else digest(x, w, b)
        meta["cases"].append(dict(name=name, kind=kind, seed=seed, seq=seq, in_dim=n_in, out_dim=n_out,
                                  bias=has_b, digest=dg))
    # smol_rms_norm (rmsnorm.c:17-75) and the gated activations (activation.c:55-125)
    meta["norm"], meta["glu"] = [], []
    for i, (seq, dim) in enumerate(NORM_ROWS):
        seed = 5500 + i
        x, w = norm_row_inputs(seed, seq, dim)
        name = "rms_%d_%d" % (seq, dim)
        arrays[name] = ref.rms_norm(x, w, 1e-6)
        meta["norm"].append(dict(name=name, seed=seed, seq=seq, dim=dim, eps=1e-6, digest=digest(x, w)))
    for i, (seq, inter, act) in enumerate(GLU):
        seed = 5600 + i
        gu = glu_inputs(seed, seq, inter)
        name = "%s_%d_%d" % ("swiglu" if act == 1 else "geglu", seq, inter)
        arrays[name] = ref.glu(gu, act)
        meta["glu"].append(dict(name=name, seed=seed, seq=seq, inter=inter, act=act, digest=digest(gu)))
    np.savez_compressed(os.path.join(OUT, "ref_linear.npz"), **arrays)
    with open(os.path.join(OUT, "ref_linear.json"), "w") as f:
        json.dump(meta, f, indent=1)
    print("wrote", len(arrays), "arrays; simd", meta["simd"])


if __name__ == "__main__":
    main()
