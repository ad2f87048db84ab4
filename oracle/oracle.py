"""ctypes loader for the CPU oracle. TEST INFRASTRUCTURE ONLY.

Two libraries share one Python interface:

* ``liboracle_v{3,4}.so`` - this repository's C restatement of the reference's
  CPU attention and RoPE (``oracle/smol_oracle.c``; each function there cites
  the reference file:line it follows), symbol prefix ``orc_``.
* ``_ref/libsmolref_v{3,4}.so`` - the reference's own
  ``common/kernels/{attention,rope,vecops_*,threading}.c`` compiled from the
  reference tree by ``oracle/Makefile``, symbol prefix ``smol_``. It exists
  only where it was built; tests that need it skip otherwise.

Only ``tests/``, ``__graft_entry__.smoke()`` and the CPU-baseline leg of
``bench.py`` import this module. Arrays are numpy, C-contiguous.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))

_F = ctypes.POINTER(ctypes.c_float)
_I = ctypes.POINTER(ctypes.c_int)
_U16 = ctypes.POINTER(ctypes.c_uint16)


def cpu_has_avx512():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("flags"):
                    fl = line.split()
                    return all(x in fl for x in ("avx512f", "avx512bw", "avx512vl", "avx512dq"))
    except OSError:
        pass
    return False


def simd_branch():
    return "avx512" if cpu_has_avx512() else "avx2"


def causal_kind(window, cap):
    """The entry point the reference decoders call for (window, cap)
    (qkn_decoder.c:505-528: a sliding window when > 0, a softcap when > 0)."""
    if window > 0 and cap > 0:
        return "swa_softcap"
    if window > 0:
        return "swa"
    return "softcap" if cap > 0 else "causal"


def _fp(a):
    return a.ctypes.data_as(_F)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


class _Lib:
    """Common wrapper; ``prefix`` is ``orc_`` (restatement) or ``smol_`` (reference)."""

    def __init__(self, path, prefix):
        self.path = path
        self.prefix = prefix
        self.lib = ctypes.CDLL(path)
        self._bind()

    def _fn(self, name, argtypes, restype=None):
        f = getattr(self.lib, self.prefix + name)
        f.argtypes = argtypes
        f.restype = restype
        return f

    def _bind(self):
        ci, cf = ctypes.c_int, ctypes.c_float
        causal = [_F, _F, _F, _F, ci, ci, ci, ci, ci, cf, ci]
        self._causal = self._fn("causal_attention", causal)
        self._swa = self._fn("sliding_window_attention", causal + [ci])
        self._softcap = self._fn("causal_attention_softcap", causal + [cf])
        self._swa_softcap = self._fn("sliding_window_attention_softcap", causal + [ci, cf])
        self._bidir = self._fn("bidirectional_attention", [_F, _F, _F, _F, ci, ci, ci, cf, _I, ci])
        self._crope_neox = self._fn("compute_rope_neox", [_F, _F, _I, ci, ci, cf])
        self._crope_inter = self._fn("compute_rope_interleaved", [_F, _F, _I, ci, ci, cf])
        self._arope_neox = self._fn("apply_rope_neox", [_F, _F, _F, ci, ci, ci])
        self._arope_inter = self._fn("apply_rope_interleaved", [_F, _F, _F, ci, ci, ci])
        set_threads = "set_threads"
        self._set_threads = self._fn(set_threads, [ci])
        # rmsnorm.c is part of the reference build since per-head RMSNorm joined
        # the path; an older _ref build lacks it
        self._rms_ph = (self._fn("rms_norm_per_head", [_F, _F, ci, ci, ci, cf])
                        if hasattr(self.lib, self.prefix + "rms_norm_per_head") else None)

    def set_threads(self, n):
        self._set_threads(int(n))

    # -- attention ---------------------------------------------------------
    def causal_attention(self, Q, K, V, seq_q, seq_k, n_heads, n_kv_heads, head_dim,
                         scale, q_offset, window=0, cap=0.0, kind=None):
        """kind picks the entry point: "causal", "swa" (window), "softcap" (cap) or
        "swa_softcap"; None picks it from the values (window > 0, cap > 0), the
        dispatch of the reference decoders (qkn_decoder.c:505-528)."""
        Q, K, V = _f32(Q), _f32(K), _f32(V)
        assert Q.size >= seq_q * n_heads * head_dim
        assert K.size >= seq_k * n_kv_heads * head_dim and V.size == K.size
        out = np.zeros((seq_q, n_heads * head_dim), np.float32)
        args = (_fp(out), _fp(Q), _fp(K), _fp(V), seq_q, seq_k, n_heads, n_kv_heads,
                head_dim, ctypes.c_float(scale), q_offset)
        if kind is None:
            kind = causal_kind(window, cap)
        if kind == "swa_softcap":
            self._swa_softcap(*args, int(window), ctypes.c_float(cap))
        elif kind == "swa":
            self._swa(*args, int(window))
        elif kind == "softcap":
            self._softcap(*args, ctypes.c_float(cap))
        elif kind == "causal":
            self._causal(*args)
        else:
            raise ValueError(kind)
        return out

    def bidirectional_attention(self, Q, K, V, seq, n_heads, head_dim, scale, window_starts):
        Q, K, V = _f32(Q), _f32(K), _f32(V)
        ws = np.ascontiguousarray(window_starts, dtype=np.int32)
        assert ws[-1] <= seq and Q.size >= seq * n_heads * head_dim
        out = np.zeros((seq, n_heads * head_dim), np.float32)
        self._bidir(_fp(out), _fp(Q), _fp(K), _fp(V), seq, n_heads, head_dim,
                    ctypes.c_float(scale), ws.ctypes.data_as(_I), len(ws) - 1)
        return out

    # -- per-head RMSNorm ----------------------------------------------------
    def rms_norm_per_head(self, x, weight, seq, n_heads, head_dim, eps):
        """x [seq, n_heads*head_dim] normalised per head_dim segment (a copy)."""
        if self._rms_ph is None:
            raise NotImplementedError("%s has no rms_norm_per_head" % self.path)
        y = np.array(x, dtype=np.float32, copy=True, order="C")
        w = _f32(weight)
        assert y.size >= seq * n_heads * head_dim and w.size >= head_dim
        self._rms_ph(_fp(y), _fp(w), seq, n_heads, head_dim, ctypes.c_float(eps))
        return y

    # -- RoPE ----------------------------------------------------------------
    def compute_rope(self, positions, head_dim, theta, interleaved=False):
        pos = np.ascontiguousarray(positions, dtype=np.int32)
        c = np.zeros((len(pos), head_dim), np.float32)
        s = np.zeros_like(c)
        f = self._crope_inter if interleaved else self._crope_neox
        f(_fp(c), _fp(s), pos.ctypes.data_as(_I), len(pos), head_dim, ctypes.c_float(theta))
        return c, s

    def apply_rope(self, x, cos, sin, seq, n_heads, head_dim, interleaved=False):
        y = np.array(x, dtype=np.float32, copy=True, order="C")
        c, s = _f32(cos), _f32(sin)
        assert c.size >= seq * head_dim
        f = self._arope_inter if interleaved else self._arope_neox
        f(_fp(y), _fp(c), _fp(s), seq, n_heads, head_dim)
        return y


class Oracle(_Lib):
    """The C restatement (``orc_`` symbols) plus its extra entry points."""

    def __init__(self, path=None):
        if path is None:
            path = os.path.join(HERE, "liboracle_v4.so" if cpu_has_avx512() else "liboracle_v3.so")
        super().__init__(path, "orc_")
        ci, cf = ctypes.c_int, ctypes.c_float
        self._fill = self._fn("fill_rope_table", [_F, _F, ci, ci, ci, cf, ci])
        self._inv = self._fn("rope_inv_freq", [_F, ci, cf])
        self._generic = self._fn("set_vec_generic", [ci])
        self._bf16_attn = self._fn("bf16_attention_softcap",
                                   [_U16, _U16, _U16, _U16, ci, ci, ci, ci, ci, cf, ci, ci, cf])
        self._bf16_norm = self._fn("bf16_rms_norm_per_head", [_U16, _F, ci, ci, ci, cf])
        self._bf16_rope = self._fn("bf16_apply_rope_interleaved", [_U16, _F, _F, ci, ci, ci])
        self._linear = self._fn("linear_bf16", [_F, _F, _U16, _F, ci, ci, ci])
        self._rms = self._fn("rms_norm", [_F, _F, _F, ci, ci, cf])
        self._swiglu = self._fn("swiglu", [_F, _F, ci, ci])
        self._geglu = self._fn("geglu", [_F, _F, ci, ci])
        self._bf16_linear = self._fn("bf16_linear_nobias", [_U16, _U16, _U16, ci, ci, ci])
        self._bf16_rms = self._fn("bf16_rms_norm", [_U16, _U16, _F, ci, ci, cf])
        self._bf16_geglu = self._fn("bf16_geglu", [_U16, _U16, ci, ci])
        self._bf16_add = self._fn("bf16_add_inplace", [_U16, _U16, ctypes.c_size_t])

    def rms_norm(self, x, w, eps):
        """smol_rms_norm (rmsnorm.c:17-75) of rows x [seq, dim]"""
        x = _f32(x)
        y = np.zeros_like(x)
        self._rms(_fp(y), _fp(x), _fp(_f32(w)), x.shape[0], x.shape[1], ctypes.c_float(eps))
        return y

    def glu(self, gu, act):
        """act 1: SwiGLU, 2: GeGLU of interleaved (gate, up) rows gu [seq, 2 * inter]"""
        gu = _f32(gu)
        y = np.zeros((gu.shape[0], gu.shape[1] // 2), np.float32)
        (self._swiglu if act == 1 else self._geglu)(_fp(y), _fp(gu), gu.shape[0], gu.shape[1] // 2)
        return y

    def linear_bf16(self, x, w_bits, bias=None):
        """y [seq, out] = x [seq, in] W^T (+ bias), W given as bf16 bits [out, in]"""
        x = _f32(x)
        w = np.ascontiguousarray(w_bits, np.uint16)
        seq, n_in = x.shape
        n_out = w.shape[0]
        y = np.zeros((seq, n_out), np.float32)
        b = _f32(bias) if bias is not None else None
        self._linear(_fp(y), _fp(x), w.ctypes.data_as(_U16), _fp(b) if b is not None else None, seq, n_in, n_out)
        return y

    def bf16_linear_nobias(self, x_bits, w_bits):
        """bf16 bits y [seq, out] = trunc(x W^T), x [seq, in] and W [out, in] bf16 bits"""
        x = np.ascontiguousarray(x_bits, np.uint16)
        w = np.ascontiguousarray(w_bits, np.uint16)
        y = np.zeros((x.shape[0], w.shape[0]), np.uint16)
        u = lambda a: a.ctypes.data_as(_U16)  # noqa: E731
        self._bf16_linear(u(y), u(x), u(w), x.shape[0], x.shape[1], w.shape[0])
        return y

    def bf16_rms_norm(self, x_bits, w, eps):
        """bf16_rms_norm (qkn_bf16_decoder.c:51-71): bf16 bits rows [seq, dim] -> truncated bf16 bits"""
        x = np.ascontiguousarray(x_bits, np.uint16)
        y = np.zeros_like(x)
        self._bf16_rms(y.ctypes.data_as(_U16), x.ctypes.data_as(_U16), _fp(_f32(w)), x.shape[0], x.shape[1],
                       ctypes.c_float(eps))
        return y

    def bf16_geglu(self, gu_bits):
        """bf16_geglu (qkn_bf16_decoder.c:235-251) of interleaved (gate, up) bf16 bits [seq, 2 * inter]"""
        gu = np.ascontiguousarray(gu_bits, np.uint16)
        y = np.zeros((gu.shape[0], gu.shape[1] // 2), np.uint16)
        self._bf16_geglu(y.ctypes.data_as(_U16), gu.ctypes.data_as(_U16), gu.shape[0], gu.shape[1] // 2)
        return y

    def bf16_add(self, a_bits, b_bits):
        """bf16_add_inplace (qkn_bf16_decoder.c:255-258): trunc(a + b) as new bf16 bits"""
        a = np.array(a_bits, np.uint16, copy=True, order="C")
        b = np.ascontiguousarray(b_bits, np.uint16)
        assert a.size == b.size
        self._bf16_add(a.ctypes.data_as(_U16), b.ctypes.data_as(_U16), a.size)
        return a

    def set_vec_generic(self, on):
        self._generic(1 if on else 0)

    def rope_inv_freq(self, head_dim, theta):
        inv = np.zeros(head_dim // 2, np.float32)
        self._inv(_fp(inv), head_dim, ctypes.c_float(theta))
        return inv

    def fill_rope_table(self, pos0, n_pos, head_dim, theta, interleaved=False):
        c = np.zeros((n_pos, head_dim), np.float32)
        s = np.zeros_like(c)
        self._fill(_fp(c), _fp(s), pos0, n_pos, head_dim, ctypes.c_float(theta),
                   1 if interleaved else 0)
        return c, s

    def bf16_attention(self, q, k, v, seq_q, seq_k, n_heads, n_kv_heads, head_dim, scale,
                       q_offset, window=0, cap=0.0):
        q = np.ascontiguousarray(q, np.uint16)
        k = np.ascontiguousarray(k, np.uint16)
        v = np.ascontiguousarray(v, np.uint16)
        out = np.zeros((seq_q, n_heads * head_dim), np.uint16)
        u = lambda a: a.ctypes.data_as(_U16)  # noqa: E731
        self._bf16_attn(u(out), u(q), u(k), u(v), seq_q, seq_k, n_heads, n_kv_heads,
                        head_dim, ctypes.c_float(scale), q_offset, window, ctypes.c_float(cap))
        return out


    def bf16_rms_norm_per_head(self, x, w, seq, n_heads, head_dim, eps):
        """bf16 bits [seq, n_heads*head_dim] -> normalised bf16 bits (truncating)"""
        y = np.array(x, np.uint16, copy=True, order="C")
        w = np.ascontiguousarray(w, np.float32)
        self._bf16_norm(y.ctypes.data_as(_U16), _fp(w), seq, n_heads, head_dim, ctypes.c_float(eps))
        return y

    def bf16_apply_rope_interleaved(self, x, cos, sin, seq, n_heads, head_dim):
        """bf16 bits [seq, n_heads*head_dim] rotated with table rows cos/sin [seq, head_dim] (truncating)"""
        y = np.array(x, np.uint16, copy=True, order="C")
        c = np.ascontiguousarray(cos, np.float32)
        s = np.ascontiguousarray(sin, np.float32)
        self._bf16_rope(y.ctypes.data_as(_U16), _fp(c), _fp(s), seq, n_heads, head_dim)
        return y


def ref_path():
    """Path of the compiled reference library for this host, or None."""
    p = os.path.join(HERE, "_ref", "libsmolref_v4.so" if cpu_has_avx512() else "libsmolref_v3.so")
    return p if os.path.exists(p) else None


class RefLib(_Lib):
    """The reference's own sources, compiled by oracle/Makefile (``smol_`` symbols)."""

    def __init__(self, path=None):
        path = path or ref_path()
        if path is None:
            raise FileNotFoundError("oracle/_ref was not built")
        super().__init__(path, "smol_")
        ci = ctypes.c_int
        self._lin = self._fn("linear_bf16", [_F, _F, _U16, _F, ci, ci, ci])
        self._lin_nb = self._fn("linear_nobias_bf16", [_F, _F, _U16, ci, ci, ci])
        self._lin_qkv = self._fn("linear_nobias_bf16_qkv", [_F, _F, _F, _F, _U16, _U16, _U16, ci, ci, ci])
        self._mm_t = self._fn("matmul_t_bf16", [_F, _F, _U16, ci, ci, ci])
        cf = ctypes.c_float
        self._rms_ref = self._fn("rms_norm", [_F, _F, _F, ci, ci, cf])
        self._swiglu_ref = self._fn("swiglu_multiply", [_F, _F, ci, ci])
        self._geglu_ref = self._fn("geglu_multiply", [_F, _F, ci, ci])

    def linear_bf16(self, x, w_bits, bias=None):
        """smol_linear_bf16 / smol_linear_nobias_bf16 (matmul.c:336-358)"""
        x = _f32(x)
        w = np.ascontiguousarray(w_bits, np.uint16)
        seq, n_in = x.shape
        y = np.zeros((seq, w.shape[0]), np.float32)
        if bias is None:
            self._lin_nb(_fp(y), _fp(x), w.ctypes.data_as(_U16), seq, n_in, w.shape[0])
        else:
            b = _f32(bias)
            self._lin(_fp(y), _fp(x), w.ctypes.data_as(_U16), _fp(b), seq, n_in, w.shape[0])
        return y

    def linear_qkv(self, x, wq, wk, wv):
        """smol_linear_nobias_bf16_qkv (matmul.c:308-334): one token"""
        x = _f32(x).reshape(-1)
        ws = [np.ascontiguousarray(w, np.uint16) for w in (wq, wk, wv)]
        q = np.zeros(ws[0].shape[0], np.float32)
        k = np.zeros(ws[1].shape[0], np.float32)
        v = np.zeros(ws[2].shape[0], np.float32)
        u = lambda a: a.ctypes.data_as(_U16)  # noqa: E731
        self._lin_qkv(_fp(q), _fp(k), _fp(v), _fp(x), u(ws[0]), u(ws[1]), u(ws[2]), x.shape[0], q.shape[0],
                      k.shape[0])
        return q, k, v

    def matmul_t_bf16(self, a, b_bits):
        """smol_matmul_t_bf16 (matmul.c:419-429): C [M, N] = A [M, K] B^T"""
        a = _f32(a)
        b = np.ascontiguousarray(b_bits, np.uint16)
        c = np.zeros((a.shape[0], b.shape[0]), np.float32)
        self._mm_t(_fp(c), _fp(a), b.ctypes.data_as(_U16), a.shape[0], a.shape[1], b.shape[0])
        return c

    def rms_norm(self, x, w, eps):
        x = _f32(x)
        y = np.zeros_like(x)
        self._rms_ref(_fp(y), _fp(x), _fp(_f32(w)), x.shape[0], x.shape[1], ctypes.c_float(eps))
        return y

    def glu(self, gu, act):
        gu = _f32(gu)
        y = np.zeros((gu.shape[0], gu.shape[1] // 2), np.float32)
        (self._swiglu_ref if act == 1 else self._geglu_ref)(_fp(y), _fp(gu), gu.shape[0], gu.shape[1] // 2)
        return y
