"""The attention workloads, as seeded synthetic inputs (numpy, host).

Each workload is named by what it is; sizes follow the calls the reference's
callers make (common/decoder/qkn_decoder.c:525-527 / :674-676,
common/vision/siglip.c:126-128, exports/qwen_asr/qwen_asr.c:1595-1620):

  qwen06b_decode      Qwen3-ASR-0.6B decoder, one decode step: Hq 16, Hkv 8,
                      hd 128, 1024 cached keys + the new token at position
                      1024 (seq_k 1025); NeoX RoPE theta 1e6.
  qwen06b_prefill     Qwen3-ASR-0.6B causal prefill, 1536 tokens, Hq 16,
                      Hkv 8, hd 128, bf16 Q/K/V, NeoX RoPE theta 1e6 over
                      positions 0..1535.
  siglip_bidir        SigLIP-so400m vision attention, 4 images x 256 patch
                      tokens, 16 heads, hd 72, bf16 ~N(0, 0.5^2), one window per
                      image, no RoPE, scale 1/sqrt(72).
  gemma_mqa_decode    Gemma-2B-style MQA decode of 16 independent sequences:
                      Hq 8, Hkv 1, hd 256, lengths L_i = 512 + (u64 % 3585),
                      the new token at position L_i - 1; interleaved RoPE
                      theta 1e4 (the Gemma / PaliGemma pairing).
  qwen17b_stream      Qwen3-ASR-1.7B streaming: a 26-token chunk at positions
                      8192..8217 on an 8192-token bf16 cache (chunked
                      prefill), then 64 single-token decode steps.
  qwen06b_decode_x28  qwen06b_decode's step for 28 sequences in one call.
  asr_encoder_bidir   Qwen3-ASR-0.6B audio encoder self-attention: 14 heads of
                      64, fp32 Q/K/V, 104-token windows over 900 tokens (the
                      last one 68 tokens), no RoPE, scale 1/8.
  *_qknorm            qwen06b_decode / qwen06b_prefill with the decoder's
                      per-head Q/K RMSNorm (weights near 1, eps 1e-6) in
                      front of RoPE (qkn_decoder.c:487-491).
  qwen06b_proj_decode / qwen06b_proj_prefill
                      the bf16-weight projections of one Qwen3-ASR-0.6B
                      decoder layer (hidden 1024, Q 16 x 128, K/V 8 x 128,
                      intermediate 3072): fused Q/K/V 1024 -> 2048 + 1024 +
                      1024, o_proj 2048 -> 1024, gate_up 1024 -> 6144, down
                      3072 -> 1024 (qkn_decoder.c:474-476, 531, 546, 552 and
                      :635, 679, 693, 699), for 1 token and for 1536 tokens;
                      28 layers of distinct weights.

Cached rows are bf16 (round to nearest even) and are already rotated, as a
decoder leaves them; the tokens a call appends are fp32 (projection outputs)
unless the workload says bf16. The CPU oracle consumes the same bits widened
to fp32.
"""
import numpy as np

from . import synth

ROPE_NEOX, ROPE_INTERLEAVED = 0, 1


def scale_of(hd):
    return float(np.float32(1.0) / np.sqrt(np.float32(hd)))


class Workload:
    name = ""
    qk_norm = False   # per-head Q/K RMSNorm in front of RoPE (the Qwen3 decoders' q_norm / k_norm)
    norm_eps = 1e-6

    def describe(self):
        return {"workload": self.name}

    def norm_weights(self):
        """(q_norm, k_norm) weights [hd] fp32 near 1, seeded, when qk_norm is set."""
        if not self.qk_norm:
            return None, None
        s = self.seed * 100
        return tuple((1.0 + 0.1 * synth.normal(s + 20 + i, (self.hd,))).astype(np.float32) for i in range(2))


def with_qk_norm(wl, name):
    wl.name, wl.qk_norm = name, True
    return wl


class Decode(Workload):
    """Batched single-token decode: per sequence i, cache rows [0, pos_i) and one new token at pos_i."""

    def __init__(self, name, Hq, Hkv, hd, lengths, theta, rope_type, seed, std=1.0):
        self.name, self.Hq, self.Hkv, self.hd = name, Hq, Hkv, hd
        self.lengths = [int(x) for x in lengths]  # seq_k of each sequence (new token included)
        self.theta, self.rope_type, self.seed, self.std = theta, rope_type, seed, std
        self.scale = scale_of(hd)

    @property
    def n_seq(self):
        return len(self.lengths)

    @property
    def positions(self):
        return np.array([L - 1 for L in self.lengths], np.int32)

    def inputs(self):
        """cache_k/cache_v: list of bf16 bit arrays [L_i - 1, Hkv*hd]; q [n, Hq*hd] f32; k/v new [n, Hkv*hd] f32."""
        s = self.seed * 100
        w = self.Hkv * self.hd
        ck = [synth.f32_to_bf16_bits(synth.normal(s + 10 + 2 * i, (L - 1, w), self.std))
              for i, L in enumerate(self.lengths)]
        cv = [synth.f32_to_bf16_bits(synth.normal(s + 11 + 2 * i, (L - 1, w), self.std))
              for i, L in enumerate(self.lengths)]
        q = synth.normal(s + 1, (self.n_seq, self.Hq * self.hd), self.std)
        k = synth.normal(s + 2, (self.n_seq, w), self.std)
        v = synth.normal(s + 3, (self.n_seq, w), self.std)
        return dict(cache_k=ck, cache_v=cv, q=q, k=k, v=v)

    def kv_bytes(self):
        return sum(self.lengths) * self.Hkv * self.hd * 2 * 2

    def algorithmic_bytes(self):
        """K+V bf16 of every visible key, Q and out fp32 (and the appended row)."""
        return self.kv_bytes() + self.n_seq * self.Hq * self.hd * 4 * 2

    def flops(self):
        return sum(4 * self.hd * self.Hq * L for L in self.lengths)

    def describe(self):
        d = {"workload": self.name, "n_seq": self.n_seq, "n_heads": self.Hq, "n_kv_heads": self.Hkv,
             "head_dim": self.hd, "seq_k": self.lengths if self.n_seq <= 4 else
             {"sum": int(sum(self.lengths)), "min": min(self.lengths), "max": max(self.lengths)},
             "rope_theta": self.theta, "rope": "neox" if self.rope_type == ROPE_NEOX else "interleaved"}
        if self.qk_norm:
            d["qk_norm_eps"] = self.norm_eps
        return d


class Prefill(Workload):
    """Causal (chunked) prefill of one sequence: cache rows [0, pos0) + seq_q new tokens."""

    def __init__(self, name, Hq, Hkv, hd, pos0, seq_q, theta, seed, in_bf16=True, std=1.0):
        self.name, self.Hq, self.Hkv, self.hd = name, Hq, Hkv, hd
        self.pos0, self.seq_q, self.theta, self.seed = pos0, seq_q, theta, seed
        self.in_bf16, self.std = in_bf16, std
        self.rope_type = ROPE_NEOX
        self.scale = scale_of(hd)

    def inputs(self):
        s = self.seed * 100
        w = self.Hkv * self.hd
        q = synth.normal(s + 1, (self.seq_q, self.Hq * self.hd), self.std)
        k = synth.normal(s + 2, (self.seq_q, w), self.std)
        v = synth.normal(s + 3, (self.seq_q, w), self.std)
        if self.in_bf16:
            q, k, v = (synth.f32_to_bf16_bits(x) for x in (q, k, v))
        ck = synth.f32_to_bf16_bits(synth.normal(s + 4, (self.pos0, w), self.std))
        cv = synth.f32_to_bf16_bits(synth.normal(s + 5, (self.pos0, w), self.std))
        return dict(cache_k=ck, cache_v=cv, q=q, k=k, v=v)

    def pairs(self):
        """unmasked (query, key) pairs: sum over rows of pos0 + i + 1"""
        return self.seq_q * self.pos0 + self.seq_q * (self.seq_q + 1) // 2

    def flops(self):
        return 4 * self.hd * self.Hq * self.pairs()

    def algorithmic_bytes(self):
        e = 2 if self.in_bf16 else 4
        return (self.seq_q * (self.Hq + 2 * self.Hkv) * self.hd * e + self.pos0 * self.Hkv * self.hd * 4
                + self.seq_q * self.Hq * self.hd * 4)

    def describe(self):
        d = {"workload": self.name, "n_heads": self.Hq, "n_kv_heads": self.Hkv, "head_dim": self.hd,
             "pos0": self.pos0, "seq_q": self.seq_q, "causal": True, "rope_theta": self.theta,
             "inputs": "bf16" if self.in_bf16 else "f32"}
        if self.qk_norm:
            d["qk_norm_eps"] = self.norm_eps
        return d


class Bidir(Workload):
    def __init__(self, name, H, hd, window_starts, seed, std=0.5, in_bf16=True):
        self.name, self.H, self.hd = name, H, hd
        self.window_starts = list(window_starts)
        self.seq = window_starts[-1]
        self.seed, self.std, self.in_bf16 = seed, std, in_bf16
        self.scale = scale_of(hd)

    def inputs(self):
        s = self.seed * 100
        shp = (self.seq, self.H * self.hd)
        cvt = synth.f32_to_bf16_bits if self.in_bf16 else (lambda a: a)
        return dict(q=cvt(synth.normal(s + 1, shp, self.std)),
                    k=cvt(synth.normal(s + 2, shp, self.std)),
                    v=cvt(synth.normal(s + 3, shp, self.std)))

    def flops(self):
        ws = self.window_starts
        return sum(4 * self.hd * self.H * (b - a) ** 2 for a, b in zip(ws[:-1], ws[1:]))

    def algorithmic_bytes(self):
        return self.seq * self.H * self.hd * (3 * (2 if self.in_bf16 else 4) + 4)

    def describe(self):
        return {"workload": self.name, "n_heads": self.H, "head_dim": self.hd,
                "windows": len(self.window_starts) - 1, "tokens": self.seq,
                "inputs": "bf16" if self.in_bf16 else "f32"}


class Stream(Workload):
    """Chunked prefill of `chunk` tokens on a `prefix`-token cache, then `steps` decode steps."""

    def __init__(self, name, Hq, Hkv, hd, prefix, chunk, steps, theta, seed, std=1.0):
        self.name, self.Hq, self.Hkv, self.hd = name, Hq, Hkv, hd
        self.prefix, self.chunk, self.steps, self.theta, self.seed = prefix, chunk, steps, theta, seed
        self.rope_type = ROPE_NEOX
        self.scale = scale_of(hd)
        self.std = std

    def inputs(self):
        s, sd = self.seed * 100, self.std
        w = self.Hkv * self.hd
        return dict(cache_k=synth.f32_to_bf16_bits(synth.normal(s + 4, (self.prefix, w), sd)),
                    cache_v=synth.f32_to_bf16_bits(synth.normal(s + 5, (self.prefix, w), sd)),
                    q=synth.normal(s + 1, (self.chunk, self.Hq * self.hd), sd),
                    k=synth.normal(s + 2, (self.chunk, w), sd),
                    v=synth.normal(s + 3, (self.chunk, w), sd),
                    dq=synth.normal(s + 6, (self.steps, self.Hq * self.hd), sd),
                    dk=synth.normal(s + 7, (self.steps, w), sd),
                    dv=synth.normal(s + 8, (self.steps, w), sd))

    def chunk_flops(self):
        return 4 * self.hd * self.Hq * sum(self.prefix + i + 1 for i in range(self.chunk))

    def decode_bytes(self):
        p = self.prefix + self.chunk
        return sum((p + s + 1) * self.Hkv * self.hd * 4 for s in range(self.steps))

    def describe(self):
        return {"workload": self.name, "n_heads": self.Hq, "n_kv_heads": self.Hkv, "head_dim": self.hd,
                "prefix": self.prefix, "chunk": self.chunk, "decode_steps": self.steps,
                "rope_theta": self.theta}


class Projections(Workload):
    """The four bf16-weight projections of one decoder layer on `seq` fp32 rows.
    kinds: name -> (in_dim, [out_dim of each weight]); "qkv" has three weights."""

    def __init__(self, name, seq, hidden, q_dim, kv_dim, inter, layers, seed):
        self.name, self.seq, self.layers, self.seed = name, seq, layers, seed
        self.kinds = {"qkv": (hidden, [q_dim, kv_dim, kv_dim]), "o_proj": (q_dim, [hidden]),
                      "gate_up": (hidden, [2 * inter]), "down": (inter, [hidden])}

    def weight_bytes(self, kind):
        n_in, outs = self.kinds[kind]
        return 2 * n_in * sum(outs)

    def algorithmic_bytes(self, kind=None):
        """weights (bf16) + x (fp32) + y (fp32) of one launch (or one layer)"""
        kinds = [kind] if kind else list(self.kinds)
        b = 0
        for k in kinds:
            n_in, outs = self.kinds[k]
            b += self.weight_bytes(k) + 4 * self.seq * (n_in + sum(outs))
        return b

    def flops(self, kind=None):
        kinds = [kind] if kind else list(self.kinds)
        return sum(2 * self.seq * self.kinds[k][0] * sum(self.kinds[k][1]) for k in kinds)

    def inputs(self):
        """x [seq, in] fp32 per kind, and bf16 weight bits per (layer, kind) as a list per kind"""
        x = {k: synth.normal(self.seed * 10 + i, (self.seq, n_in)) for i, (k, (n_in, _)) in
             enumerate(self.kinds.items())}
        return {"x": x}

    def layer_weights(self, layer, kind):
        """bf16 bits of the weights of one kind in one layer (seeded; for the CPU side)"""
        n_in, outs = self.kinds[kind]
        ki = list(self.kinds).index(kind)
        return [synth.f32_to_bf16_bits(synth.normal(self.seed * 1000 + layer * 16 + ki * 4 + j, (o, n_in),
                                                    1.0 / np.sqrt(n_in)))
                for j, o in enumerate(outs)]

    def describe(self):
        return {"workload": self.name, "tokens": self.seq, "layers_rotated": self.layers,
                "projections": {k: {"in": v[0], "out": v[1]} for k, v in self.kinds.items()},
                "weights": "bf16 [out][in], N(0, 1/in)", "x": "fp32 N(0,1)"}


def gemma_lengths(seed=4, n=16, lo=512, hi=4096):
    return [int(x) for x in synth.uniform_int(seed * 1000 + 7, n, lo, hi)]


def all_workloads():
    return {
        "qwen06b_decode": Decode("qwen06b_decode", 16, 8, 128, [1025], 1e6, ROPE_NEOX, seed=1),
        "qwen06b_prefill": Prefill("qwen06b_prefill", 16, 8, 128, 0, 1536, 1e6, seed=2),
        "siglip_bidir": Bidir("siglip_bidir", 16, 72, [0, 256, 512, 768, 1024], seed=3),
        "gemma_mqa_decode": Decode("gemma_mqa_decode", 8, 1, 256, gemma_lengths(), 1e4, ROPE_INTERLEAVED,
                                   seed=4),
        "qwen17b_stream": Stream("qwen17b_stream", 16, 8, 128, 8192, 26, 64, 1e6, seed=5),
        # C1's decode step for 28 sequences in one call (28 x 4.2 MB): the same kernel when the launch
        # and the memory latency are spread over enough bytes
        "qwen06b_decode_x28": Decode("qwen06b_decode_x28", 16, 8, 128, [1025] * 28, 1e6, ROPE_NEOX, seed=7),
        # Qwen3-ASR-0.6B audio encoder self-attention: 14 heads of 64, fp32 projections, 104-token
        # windows (encoder.c:426-434) over 900 tokens, the last window ragged
        "asr_encoder_bidir": Bidir("asr_encoder_bidir", 14, 64, list(range(0, 900, 104)) + [900], seed=6, std=1.0,
                                   in_bf16=False),
        # the same decode step and prefill with the per-head Q/K RMSNorm fused in front of RoPE
        "qwen06b_decode_qknorm": with_qk_norm(Decode("", 16, 8, 128, [1025], 1e6, ROPE_NEOX, seed=1),
                                              "qwen06b_decode_qknorm"),
        "qwen06b_prefill_qknorm": with_qk_norm(Prefill("", 16, 8, 128, 0, 1536, 1e6, seed=2),
                                               "qwen06b_prefill_qknorm"),
        "qwen06b_proj_decode": Projections("qwen06b_proj_decode", 1, 1024, 2048, 1024, 3072, 28, seed=8),
        "qwen06b_proj_prefill": Projections("qwen06b_proj_prefill", 1536, 1024, 2048, 1024, 3072, 28, seed=9),
    }
