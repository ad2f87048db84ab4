"""The reference decoders' attention block, one layer per call, on the CPU
oracle. TEST INFRASTRUCTURE ONLY (the tests and the smoke check).

Each model keeps its own per-layer KV cache and follows the block between
the projections and o_proj:

  Fp32Block   common/decoder/qkn_decoder.c:460-528 (prefill) / :625-677
              (decode): table choice (global theta, or the local theta on a
              sliding layer when it differs, :460-468 and :326-337),
              per-head RMSNorm (rmsnorm.c:78-140 restated), RoPE
              (rope.c restated), cache write, then the four-way dispatch
              (is_sliding && sliding_window > 0, softcap > 0) of :505-528
              with scale 1/sqrtf(head_dim) (:430). The reference's cache is
              fp32; the device cache it is compared with is bf16, so rows
              written by an earlier call are read back through bf16 (round to
              nearest even) and a call's own rows are used at fp32.
  Bf16Block   common/decoder/qkn_bf16_decoder.c:486-546 / :638-674:
              truncating per-head norm and interleaved rotation
              (orc_bf16_rms_norm_per_head, orc_bf16_apply_rope_interleaved),
              byte-copy cache write, two-pass attention with truncated bf16
              output (orc_bf16_attention_softcap).
"""
import numpy as np

from workload_oracle import _widen


def _rne16(a):
    u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


class _Block:
    def __init__(self, orc, n_layers, n_heads, n_kv_heads, head_dim, eps, rope_theta, rope_local_theta,
                 rope_type, sliding_window, attn_logit_softcap, capacity=4096):
        self.orc = orc
        self.L, self.H, self.Hkv, self.hd = n_layers, n_heads, n_kv_heads, head_dim
        self.eps = eps
        self.theta, self.local_theta, self.rope_type = rope_theta, rope_local_theta, rope_type
        self.window, self.cap = sliding_window, attn_logit_softcap
        self.scale = float(np.float32(1.0) / np.sqrt(np.float32(head_dim)))
        self.sliding = [0] * n_layers
        self.qn = [None] * n_layers
        self.kn = [None] * n_layers
        kvd = n_kv_heads * head_dim
        self.ck = np.zeros((n_layers, capacity, kvd), np.uint16)
        self.cv = np.zeros((n_layers, capacity, kvd), np.uint16)

    def set_layer(self, layer, is_sliding=0, q_norm=None, k_norm=None):
        self.sliding[layer] = 1 if is_sliding else 0
        self.qn[layer], self.kn[layer] = q_norm, k_norm

    def _layer_args(self, layer, interleaved):
        local = self.local_theta > 0 and self.local_theta != self.theta
        theta = self.local_theta if (self.sliding[layer] and local) else self.theta
        window = self.window if (self.sliding[layer] and self.window > 0) else 0
        cap = self.cap if self.cap > 0 else 0.0
        return theta, window, cap

    def _table(self, theta, pos0, n, interleaved):
        c, s = self.orc.fill_rope_table(0, pos0 + n, self.hd, theta, interleaved)
        return c[pos0:], s[pos0:]


class Fp32Block(_Block):
    def block(self, layer, start, q, k, v):
        """out [S, H*hd] fp32 for the projections q [S, H*hd], k, v [S, Hkv*hd] (fp32)"""
        o, S, H, Hkv, hd = self.orc, q.shape[0], self.H, self.Hkv, self.hd
        inter = self.rope_type == 1
        theta, window, cap = self._layer_args(layer, inter)
        c, s = self._table(theta, start, S, inter)
        qx = np.ascontiguousarray(q, np.float32)
        kx = np.ascontiguousarray(k, np.float32)
        if self.qn[layer] is not None:
            qx = o.rms_norm_per_head(qx, self.qn[layer], S, H, hd, self.eps)
        if self.kn[layer] is not None:
            kx = o.rms_norm_per_head(kx, self.kn[layer], S, Hkv, hd, self.eps)
        qr = o.apply_rope(qx, c, s, S, H, hd, inter)
        kr = o.apply_rope(kx, c, s, S, Hkv, hd, inter)
        K = np.concatenate([_widen(self.ck[layer, :start]), kr], 0)
        V = np.concatenate([_widen(self.cv[layer, :start]), np.asarray(v, np.float32)], 0)
        out = o.causal_attention(qr, K, V, S, start + S, H, Hkv, hd, self.scale, start, window=window, cap=cap)
        self.ck[layer, start:start + S] = _rne16(kr)
        self.cv[layer, start:start + S] = _rne16(v)
        return out


class Bf16Block(_Block):
    def block(self, layer, start, q, k, v):
        """out [S, H*hd] bf16 bits for bf16-bit projections q, k, v"""
        o, S, H, Hkv, hd = self.orc, q.shape[0], self.H, self.Hkv, self.hd
        theta, window, cap = self._layer_args(layer, True)
        c, s = self._table(theta, start, S, True)
        qb = np.ascontiguousarray(q, np.uint16)
        kb = np.ascontiguousarray(k, np.uint16)
        if self.qn[layer] is not None:
            qb = o.bf16_rms_norm_per_head(qb, self.qn[layer], S, H, hd, self.eps)
        if self.kn[layer] is not None:
            kb = o.bf16_rms_norm_per_head(kb, self.kn[layer], S, Hkv, hd, self.eps)
        qb = o.bf16_apply_rope_interleaved(qb, c, s, S, H, hd)
        kb = o.bf16_apply_rope_interleaved(kb, c, s, S, Hkv, hd)
        self.ck[layer, start:start + S] = kb
        self.cv[layer, start:start + S] = np.asarray(v, np.uint16)
        return o.bf16_attention(qb, self.ck[layer, :start + S], self.cv[layer, :start + S], S, start + S, H, Hkv,
                                hd, self.scale, start, window=window, cap=cap)


class Fp32Layer:
    """A whole fp32 decoder layer around Fp32Block: qkn_decoder.c:633-705 (one
    token) / :470-560 (prefill), with the restated smol_rms_norm, the bf16
    projections (orc_linear_bf16), SwiGLU / GeGLU and the residual adds:

      xn = rms_norm(x, input_norm); q, k, v = xn Wq^T, xn Wk^T, xn Wv^T
      a  = block(q, k, v); p = a Wo^T
      Qwen3:   x = x + p;             h = rms_norm(x, post_attn_norm)
      Gemma 3: x = x + rms_norm(p, post_attn_norm); h = rms_norm(x, pre_ffn_norm)
      f = act(h Wgu^T) Wd^T; x = x + f (or x + rms_norm(f, post_ffn_norm))

    `weights[layer]` holds numpy arrays under the smol_qkn_layer_weights
    names (bf16 bits for the projections)."""

    def __init__(self, orc, block, weights, act):
        self.orc, self.block, self.w, self.act = orc, block, weights, act
        self.gain = 1.0  # of the last step: max(1, 1 / rms of the rows post_attn_norm rescales)

    def step(self, layer, start, x):
        o, w, eps = self.orc, self.w[layer], self.block.eps
        x = np.asarray(x, np.float32)
        xn = o.rms_norm(x, w["input_norm"], eps)
        q, k, v = o.linear_bf16(xn, w["wq"]), o.linear_bf16(xn, w["wk"]), o.linear_bf16(xn, w["wv"])
        a = self.block.block(layer, start, q, k, v)
        p = o.linear_bf16(a, w["wo"])
        self.gain = 1.0
        if w.get("pre_ffn_norm") is not None:
            # the norm rescales the attention sublayer's output (and its error) by 1 / rms(p)
            rms = np.sqrt((p.astype(np.float64) ** 2).mean(1) + eps)
            self.gain = float(max(1.0, (1.0 / rms).max()))
            x = x + o.rms_norm(p, w["post_attn_norm"], eps)
            h = o.rms_norm(x, w["pre_ffn_norm"], eps)
        else:
            x = x + p
            h = o.rms_norm(x, w["post_attn_norm"], eps)
        f = o.linear_bf16(o.glu(o.linear_bf16(h, w["gate_up"]), self.act), w["down"])
        if w.get("post_ffn_norm") is not None:
            f = o.rms_norm(f, w["post_ffn_norm"], eps)
        return (x + f).astype(np.float32)


class Bf16Layer:
    """A whole bf16 decoder layer around Bf16Block: qkn_bf16_decoder.c:634-697
    (one token) / :482-571 (prefill). Every array is bf16 bits and every step
    truncates its result to bf16 (orc_bf16_rms_norm, orc_bf16_linear_nobias,
    orc_bf16_geglu, orc_bf16_add_inplace):

      xn = norm(x, input_norm); q, k, v = xn Wq^T, xn Wk^T, xn Wv^T
      a  = block(q, k, v); p = a Wo^T
      pre_ffn_norm set: p = norm(p, post_attn_norm); x = x + p; h = norm(x, pre_ffn_norm)
      otherwise:        x = x + p;                    h = norm(x, post_attn_norm)
      f = geglu(h Wgu^T) Wd^T; f = norm(f, post_ffn_norm) when set; x = x + f

    `weights[layer]` holds numpy arrays under the smol_qkn_layer_weights
    names (bf16 bits for the projections, fp32 norm weights)."""

    def __init__(self, orc, block, weights):
        self.orc, self.block, self.w = orc, block, weights

    def step(self, layer, start, x):
        o, w, eps = self.orc, self.w[layer], self.block.eps
        x = np.asarray(x, np.uint16)
        xn = o.bf16_rms_norm(x, w["input_norm"], eps)
        q, k, v = (o.bf16_linear_nobias(xn, w[n]) for n in ("wq", "wk", "wv"))
        a = self.block.block(layer, start, q, k, v)
        p = o.bf16_linear_nobias(a, w["wo"])
        if w.get("pre_ffn_norm") is not None:
            p = o.bf16_rms_norm(p, w["post_attn_norm"], eps)
            x = o.bf16_add(x, p)
            h = o.bf16_rms_norm(x, w["pre_ffn_norm"], eps)
        else:
            x = o.bf16_add(x, p)
            h = o.bf16_rms_norm(x, w["post_attn_norm"], eps)
        f = o.bf16_linear_nobias(o.bf16_geglu(o.bf16_linear_nobias(h, w["gate_up"])), w["down"])
        if w.get("post_ffn_norm") is not None:
            f = o.bf16_rms_norm(f, w["post_ffn_norm"], eps)
        return o.bf16_add(x, f)
