"""Python mirror of the C ABI in include/smol_attn.h and include/smol_kernels_attn.h.

The library is loaded from this directory (libsmol_attn.so, built by
build.py); importing this module fails loudly when it is missing. Device
tensors are torch tensors on a ROCm device: torch provides memory and the
stream, the computation is the library's. Host arrays are numpy.

The names mirror the reference's kernel API (common/kernels/smol_kernels.h):
``smol_causal_attention``, ``smol_bidirectional_attention``,
``smol_sliding_window_attention``, ``smol_causal_attention_softcap``,
``smol_sliding_window_attention_softcap``, ``smol_compute_rope_neox`` ... with
the same argument meaning (``out`` is overwritten in place).
"""
import atexit
import ctypes
import os
import weakref

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# SMOL_ATTN_LIB selects another build of the library (same C ABI)
LIB_PATH = os.environ.get("SMOL_ATTN_LIB") or os.path.join(HERE, "libsmol_attn.so")

F32, BF16 = 0, 1
ROPE_NONE, ROPE_NEOX, ROPE_INTERLEAVED = -1, 0, 1

_c_int, _c_float, _vp = ctypes.c_int, ctypes.c_float, ctypes.c_void_p
_FP = ctypes.POINTER(ctypes.c_float)
_IP = ctypes.POINTER(ctypes.c_int)
_U16P = ctypes.POINTER(ctypes.c_uint16)

# (name, argtypes, restype) of every exported entry point; the ABI test checks
# this list against the header declarations and the library's symbol table.
SIGNATURES = [
    ("smol_attn_version", [], ctypes.c_char_p),
    ("smol_attn_last_error", [], ctypes.c_char_p),
    ("smol_attn_device_count", [], _c_int),
    ("smol_attn_ctx_create", [_c_int, _vp, ctypes.POINTER(_vp)], _c_int),
    ("smol_attn_ctx_destroy", [_vp], _c_int),
    ("smol_attn_ctx_synchronize", [_vp], _c_int),
    ("smol_attn_ctx_stream", [_vp], _vp),
    ("smol_attn_ctx_set_timing", [_vp, _c_int], _c_int),
    ("smol_attn_ctx_set_option", [_vp, _c_int, _c_int], _c_int),
    ("smol_attn_ctx_get_option", [_vp, _c_int, _IP], _c_int),
    ("smol_attn_ctx_timing_read", [_vp, ctypes.POINTER(ctypes.c_double), _IP], _c_int),
    ("smol_rope_table_create", [_vp, _c_int, _c_float, _c_int, _c_int, ctypes.POINTER(_vp)], _c_int),
    ("smol_rope_table_ensure", [_vp, _c_int], _c_int),
    ("smol_rope_table_capacity", [_vp], _c_int),
    ("smol_rope_table_destroy", [_vp], _c_int),
    ("smol_rope_fill_host", [_FP, _FP, _c_int, _c_int, _c_int, _c_float, _c_int], None),
    ("smol_kv_cache_create", [_vp, _c_int, _c_int, _c_int, _c_int, _c_int, ctypes.POINTER(_vp)], _c_int),
    ("smol_kv_cache_destroy", [_vp], _c_int),
    ("smol_kv_cache_capacity", [_vp], _c_int),
    ("smol_kv_cache_reserve", [_vp, _c_int], _c_int),
    ("smol_kv_cache_write", [_vp, _c_int, _c_int, _c_int, _c_int, _vp, _vp, _c_int, _c_int], _c_int),
    ("smol_kv_cache_read", [_vp, _c_int, _c_int, _c_int, _c_int, _U16P, _U16P], _c_int),
    ("smol_attn_prefill", [_vp, _vp, _c_int, _c_int, _vp, _c_int, _c_int, _vp, _vp, _vp, _c_int,
                           _c_int, _c_float, _c_int, _c_float, _vp], _c_int),
    ("smol_attn_decode", [_vp, _vp, _c_int, _vp, _c_int, _IP, _IP, _vp, _vp, _vp, _c_int, _c_int,
                          _c_float, _c_int, _c_float, _vp], _c_int),
    ("smol_attn_causal", [_vp, _vp, _vp, _vp, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int,
                          _c_float, _c_int, _c_int, _c_float, _vp], _c_int),
    ("smol_attn_causal_bf16", [_vp, _vp, _vp, _vp, _c_int, _c_int, _c_int, _c_int, _c_int, _c_float, _c_int, _c_int,
                               _c_float, _vp], _c_int),
    ("smol_attn_bidirectional", [_vp, _vp, _vp, _vp, _c_int, _c_int, _c_int, _c_int, _c_float, _IP,
                                 _c_int, _vp], _c_int),
    ("smol_attn_prefill_qknorm", [_vp, _vp, _c_int, _c_int, _vp, _c_int, _c_int, _vp, _vp, _vp, _c_int,
                                  _c_int, _c_float, _c_int, _c_float, _vp, _vp, _c_float, _vp], _c_int),
    ("smol_attn_decode_qknorm", [_vp, _vp, _c_int, _vp, _c_int, _IP, _IP, _vp, _vp, _vp, _c_int, _c_int,
                                 _c_float, _c_int, _c_float, _vp, _vp, _c_float, _vp], _c_int),
    ("smol_attn_decode_noalloc", [_vp, _vp, _c_int, _vp, _c_int, _IP, _IP, _vp, _vp, _vp, _c_int, _c_int,
                                  _c_float, _c_int, _c_float, _vp, _vp, _c_float, _vp], _c_int),
    ("smol_attn_apply_rope", [_vp, _vp, _vp, _IP, _c_int, _c_int], _c_int),
    ("smol_attn_norm_rope", [_vp, _vp, _vp, _vp, _c_float, _IP, _c_int, _c_int, _c_int], _c_int),
    ("smol_attn_norm_rope_bf16", [_vp, _vp, _vp, _vp, _c_float, _c_int, _c_int, _c_int, _c_int], _c_int),
    # decoder attention block keyed by the decoder context (include/smol_qkn_attn.h)
    ("smol_qkn_attn_bind", [_vp, _vp], _c_int),
    ("smol_qkn_attn_set_layer", [_vp, _c_int, _c_int, _FP, _FP], _c_int),
    ("smol_qkn_attn_prefill", [_vp, _c_int, _c_int, _c_int, _vp, _vp, _vp, _vp], _c_int),
    ("smol_qkn_attn_forward", [_vp, _c_int, _c_int, _vp, _vp, _vp, _vp], _c_int),
    ("smol_qkn_attn_read_cache", [_vp, _c_int, _c_int, _c_int, _U16P, _U16P], _c_int),
    ("smol_qkn_attn_unbind", [_vp], _c_int),
    ("smol_qkn_layer_forward", [_vp, _c_int, _c_int, _vp, _vp, _c_int, _c_int, _c_int], _c_int),
    ("smol_qkn_layer_prefill", [_vp, _c_int, _c_int, _c_int, _vp, _vp, _c_int, _c_int, _c_int], _c_int),
    ("smol_qkn_layer_forward_bf16", [_vp, _c_int, _c_int, _vp, _vp, _c_int, _c_int], _c_int),
    ("smol_qkn_layer_prefill_bf16", [_vp, _c_int, _c_int, _c_int, _vp, _vp, _c_int, _c_int], _c_int),
    ("smol_qkn_layer_synchronize", [_vp], _c_int),
    ("smol_qkn_step_graph_create", [_vp, _vp, _vp, _c_int, _c_int, _c_int, _c_int, ctypes.POINTER(_vp)], _c_int),
    ("smol_qkn_step_graph_launch", [_vp, _c_int], _c_int),
    ("smol_qkn_step_graph_destroy", [_vp], _c_int),
    ("smol_qkn_attn_stream", [_vp], _vp),
    # bf16-weight projections on device pointers (include/smol_linear.h)
    ("smol_linear_dev", [_vp, _vp, _c_int, _vp, _c_int, _vp, _vp, _c_int, _c_int, _c_int], _c_int),
    ("smol_linear_qkv_dev", [_vp, _vp, _vp, _vp, _c_int, _vp, _c_int, _vp, _vp, _vp, _c_int, _c_int, _c_int,
                             _c_int], _c_int),
    ("smol_linear_ops_dev", [_vp, _vp, _vp, _vp, _vp, _c_int, _c_int, _c_int, _vp], _c_int),
    ("smol_rms_norm_dev", [_vp, _vp, _vp, _vp, _vp, _c_int, _c_int, _c_float], _c_int),
    ("smol_bf16_rms_norm_dev", [_vp, _vp, _vp, _vp, _c_int, _c_int, _c_float], _c_int),
    ("smol_bf16_add_norm_dev", [_vp, _vp, _vp, _vp, _vp, _vp, _c_int, _c_int, _c_float], _c_int),
    ("smol_bf16_geglu_dev", [_vp, _vp, _vp, _c_int, _c_int], _c_int),
    ("smol_linear_qkv_norm_dev", [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_int, _c_int, _c_int, _c_int, _vp,
                                  _c_float], _c_int),
    # reference-signature drop-ins (host fp32 arrays)
    ("smol_linear_bf16", [_FP, _FP, _U16P, _FP, _c_int, _c_int, _c_int], None),
    ("smol_linear_nobias_bf16", [_FP, _FP, _U16P, _c_int, _c_int, _c_int], None),
    ("smol_linear_nobias_bf16_qkv", [_FP, _FP, _FP, _FP, _U16P, _U16P, _U16P, _c_int, _c_int, _c_int], None),
    ("smol_matmul_t_bf16", [_FP, _FP, _U16P, _c_int, _c_int, _c_int], None),
    ("smol_bidirectional_attention", [_FP, _FP, _FP, _FP, _c_int, _c_int, _c_int, _c_float, _IP, _c_int], None),
    ("smol_causal_attention", [_FP, _FP, _FP, _FP, _c_int, _c_int, _c_int, _c_int, _c_int, _c_float, _c_int], None),
    ("smol_sliding_window_attention", [_FP, _FP, _FP, _FP, _c_int, _c_int, _c_int, _c_int, _c_int, _c_float,
                                       _c_int, _c_int], None),
    ("smol_causal_attention_softcap", [_FP, _FP, _FP, _FP, _c_int, _c_int, _c_int, _c_int, _c_int, _c_float,
                                       _c_int, _c_float], None),
    ("smol_sliding_window_attention_softcap", [_FP, _FP, _FP, _FP, _c_int, _c_int, _c_int, _c_int, _c_int,
                                               _c_float, _c_int, _c_int, _c_float], None),
    ("smol_compute_rope_neox", [_FP, _FP, _IP, _c_int, _c_int, _c_float], None),
    ("smol_apply_rope_neox", [_FP, _FP, _FP, _c_int, _c_int, _c_int], None),
    ("smol_compute_rope_interleaved", [_FP, _FP, _IP, _c_int, _c_int, _c_float], None),
    ("smol_apply_rope_interleaved", [_FP, _FP, _FP, _c_int, _c_int, _c_int], None),
    ("smol_rms_norm_per_head", [_FP, _FP, _c_int, _c_int, _c_int, _c_float], None),
]

_lib = None
_live = weakref.WeakSet()  # open handles, closed at interpreter exit before the HIP runtime goes away


@atexit.register
def _close_all():
    # caches and tables before contexts
    objs = sorted(list(_live), key=lambda o: isinstance(o, Context))
    for o in objs:
        try:
            o.close()
        except Exception:
            pass


class SmolAttnError(RuntimeError):
    pass


class SmolAttnRangeError(SmolAttnError):
    """SMOL_ATTN_ERR_RANGE: a prefill or bidirectional call's fp16 staging
    overflowed since the last synchronize; those calls' outputs are not valid."""


class SmolAttnTimeoutError(SmolAttnError):
    """SMOL_ATTN_ERR_TIMEOUT: a decode split-K merge gave up waiting for its
    splits since the last synchronize; the rows it merged are NaN."""


ERR_RANGE = -6  # SMOL_ATTN_ERR_RANGE
ERR_TIMEOUT = -7  # SMOL_ATTN_ERR_TIMEOUT


def load(path=LIB_PATH):
    """The loaded library (ctypes.CDLL). Raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise SmolAttnError("%s is missing: run `python smol-genius_amd/build.py` "
                            "(the attention path has no CPU fallback)" % path)
    # torch carries its own HIP runtime under the soname the library links
    # against: with torch imported first the library binds to that one copy;
    # loaded the other way round, torch's runtime and the library's each
    # initialise separately and the library's finds no device
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    lib = ctypes.CDLL(path)
    for name, argtypes, restype in SIGNATURES:
        f = getattr(lib, name)
        f.argtypes = argtypes
        f.restype = restype
    _lib = lib
    return lib


def _check(rc, what):
    if rc != 0:
        cls = {ERR_RANGE: SmolAttnRangeError, ERR_TIMEOUT: SmolAttnTimeoutError}.get(rc, SmolAttnError)
        raise cls("%s failed (%d): %s" % (what, rc, load().smol_attn_last_error().decode()))


def _dtype_code(t):
    import torch
    if t.dtype == torch.float32:
        return F32
    if t.dtype == torch.bfloat16:
        return BF16
    raise SmolAttnError("inputs must be float32 or bfloat16, got %s" % t.dtype)


def _dev(t, what):
    if not t.is_cuda or not t.is_contiguous():
        raise SmolAttnError("%s must be a contiguous device tensor" % what)
    return ctypes.c_void_p(t.data_ptr())


# context options (include/smol_attn.h SMOL_OPT_*)
(OPT_PREFILL_KERNEL, OPT_FB_LISTS, OPT_FB_NT, OPT_DEC_SLABS, OPT_DEC_WAVES, OPT_DEC_SPLIT, OPT_XCD_CHECK,
 OPT_BIDIR_WIN, OPT_WIN_KSPLIT, OPT_DEC_SPIN, OPT_FAULT_MERGE, OPT_QK_FP16, OPT_FB_GROUPS, OPT_GEMM_TILE,
 OPT_FB_QPREP) = range(15)


class Context:
    """Device + stream + workspace (smol_attn_ctx). Defaults to torch's current stream."""

    def __init__(self, device=0, stream=None):
        lib = load()
        if stream is None:
            import torch
            stream = torch.cuda.current_stream(device).cuda_stream
        self.h = ctypes.c_void_p()
        _check(lib.smol_attn_ctx_create(device, ctypes.c_void_p(stream), ctypes.byref(self.h)),
               "smol_attn_ctx_create")
        self.device = device
        _live.add(self)

    def synchronize(self):
        _check(load().smol_attn_ctx_synchronize(self.h), "synchronize")

    def set_timing(self, enable):
        _check(load().smol_attn_ctx_set_timing(self.h, 1 if enable else 0), "set_timing")

    def set_option(self, option, value):
        """Context switch SMOL_OPT_* (OPT_* here); 0 is the default choice by call shape."""
        _check(load().smol_attn_ctx_set_option(self.h, int(option), int(value)), "set_option")

    def get_option(self, option):
        v = ctypes.c_int()
        _check(load().smol_attn_ctx_get_option(self.h, int(option), ctypes.byref(v)), "get_option")
        return v.value

    def timing_read(self):
        """{'prep': (ms, n), 'attn': (ms, n), 'other': (ms, n)} since the last read (synchronizes)."""
        ms = (ctypes.c_double * 3)()
        n = (ctypes.c_int * 3)()
        _check(load().smol_attn_ctx_timing_read(self.h, ms, n), "timing_read")
        return {"prep": (ms[0], n[0]), "attn": (ms[1], n[1]), "other": (ms[2], n[2])}

    def close(self):
        if self.h:
            load().smol_attn_ctx_destroy(self.h)
            self.h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class RopeTable:
    def __init__(self, ctx, head_dim, theta, rope_type=ROPE_NEOX, capacity=1024):
        self.ctx = ctx
        self.h = ctypes.c_void_p()
        _check(load().smol_rope_table_create(ctx.h, head_dim, ctypes.c_float(theta), rope_type, capacity,
                                             ctypes.byref(self.h)), "smol_rope_table_create")
        self.head_dim, self.theta, self.rope_type = head_dim, theta, rope_type
        _live.add(self)

    @property
    def capacity(self):
        return load().smol_rope_table_capacity(self.h)

    def ensure(self, required_pos):
        _check(load().smol_rope_table_ensure(self.h, required_pos), "smol_rope_table_ensure")

    def close(self):
        if self.h:
            load().smol_rope_table_destroy(self.h)
            self.h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def rope_fill_host(pos0, n_pos, head_dim, theta, rope_type=ROPE_NEOX):
    """Host rows [pos0, pos0 + n_pos) of the cos/sin table (qkn_decoder.c:261-311)."""
    c = np.zeros((n_pos, head_dim), np.float32)
    s = np.zeros_like(c)
    load().smol_rope_fill_host(c.ctypes.data_as(_FP), s.ctypes.data_as(_FP), pos0, n_pos, head_dim,
                               ctypes.c_float(theta), rope_type)
    return c, s


class KVCache:
    """Device bf16 KV cache: layers x slots x kv_heads x capacity x head_dim."""

    def __init__(self, ctx, n_layers, n_slots, n_kv_heads, head_dim, max_seq):
        self.ctx = ctx
        self.h = ctypes.c_void_p()
        _check(load().smol_kv_cache_create(ctx.h, n_layers, n_slots, n_kv_heads, head_dim, max_seq,
                                           ctypes.byref(self.h)), "smol_kv_cache_create")
        self.n_layers, self.n_slots, self.n_kv_heads, self.head_dim = n_layers, n_slots, n_kv_heads, head_dim
        _live.add(self)

    @property
    def capacity(self):
        return load().smol_kv_cache_capacity(self.h)

    def reserve(self, required_pos):
        _check(load().smol_kv_cache_reserve(self.h, required_pos), "smol_kv_cache_reserve")

    def write(self, layer, slot, pos0, k, v):
        """Write already-rotated rows [pos0, pos0+n) from host numpy (f32 or bf16 bits as uint16) or device tensors."""
        if isinstance(k, np.ndarray):
            dt = BF16 if k.dtype == np.uint16 else F32
            k = np.ascontiguousarray(k, np.uint16 if dt == BF16 else np.float32)
            v = np.ascontiguousarray(v, k.dtype)
            n = k.shape[0]
            _check(load().smol_kv_cache_write(self.h, layer, slot, pos0, n, k.ctypes.data_as(_vp),
                                              v.ctypes.data_as(_vp), dt, 0), "smol_kv_cache_write")
        else:
            n = k.shape[0]
            _check(load().smol_kv_cache_write(self.h, layer, slot, pos0, n, _dev(k, "k"), _dev(v, "v"),
                                              _dtype_code(k), 1), "smol_kv_cache_write")

    def read(self, layer, slot, pos0, n):
        """bf16 bits (uint16) [n][kv_heads*head_dim] of K and V."""
        w = self.n_kv_heads * self.head_dim
        k = np.zeros((n, w), np.uint16)
        v = np.zeros((n, w), np.uint16)
        _check(load().smol_kv_cache_read(self.h, layer, slot, pos0, n, k.ctypes.data_as(_U16P),
                                         v.ctypes.data_as(_U16P)), "smol_kv_cache_read")
        return k, v

    def close(self):
        if self.h:
            load().smol_kv_cache_destroy(self.h)
            self.h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def _out_like(q_rows, n_heads, head_dim, device, out):
    import torch
    if out is None:
        out = torch.empty((q_rows, n_heads * head_dim), dtype=torch.float32, device=device)
    return out


def _norm_w(w, what):
    if w is None:
        return None
    import torch
    if w.dtype != torch.float32:
        raise SmolAttnError("%s must be float32" % what)
    return _dev(w, what)


class Prepared:
    """One C call with its arguments converted once, for loops that repeat it
    (the bench): calling it runs the call and raises on a failure status.
    `out` is the output tensor the call writes."""

    def __init__(self, fn, args, name, out, keep=()):
        self.fn, self.args, self.name, self.out, self.keep = fn, args, name, out, keep

    def __call__(self):
        rc = self.fn(*self.args)
        if rc:
            _check(rc, self.name)
        return self.out


def prefill_call(ctx, kv, layer, slot, rope, pos0, q, k_new, v_new, n_heads, scale, window=0, cap=0.0, out=None,
                 q_norm=None, k_norm=None, eps=1e-6):
    """smol_attn_prefill(_qknorm) as a Prepared call"""
    seq_q = q.shape[0]
    out = _out_like(seq_q, n_heads, kv.head_dim, q.device, out)
    args = (ctx.h, kv.h, layer, slot, rope.h if rope else None, pos0, seq_q, _dev(q, "q"), _dev(k_new, "k"),
            _dev(v_new, "v"), _dtype_code(q), n_heads, ctypes.c_float(scale), window, ctypes.c_float(cap))
    # the call holds only raw device addresses: keep the tensors behind them alive with it
    keep = (q, k_new, v_new, out, q_norm, k_norm)
    if q_norm is None and k_norm is None:
        return Prepared(load().smol_attn_prefill, args + (_dev(out, "out"),), "smol_attn_prefill", out, keep)
    return Prepared(load().smol_attn_prefill_qknorm,
                    args + (_norm_w(q_norm, "q_norm"), _norm_w(k_norm, "k_norm"), ctypes.c_float(eps),
                            _dev(out, "out")), "smol_attn_prefill_qknorm", out, keep)


def prefill(ctx, kv, layer, slot, rope, pos0, q, k_new, v_new, n_heads, scale, window=0, cap=0.0, out=None,
            q_norm=None, k_norm=None, eps=1e-6):
    """Chunked prefill of one sequence; see smol_attn_prefill. q_norm / k_norm
    (device float32 [head_dim]) select smol_attn_prefill_qknorm."""
    return prefill_call(ctx, kv, layer, slot, rope, pos0, q, k_new, v_new, n_heads, scale, window, cap, out,
                        q_norm, k_norm, eps)()


def decode_call(ctx, kv, layer, rope, slots, pos, q, k_new, v_new, n_heads, scale, window=0, cap=0.0, out=None,
                q_norm=None, k_norm=None, eps=1e-6):
    """smol_attn_decode(_qknorm) as a Prepared call"""
    slots = np.ascontiguousarray(slots, np.int32)
    pos = np.ascontiguousarray(pos, np.int32)
    n = len(slots)
    out = _out_like(n, n_heads, kv.head_dim, q.device, out)
    args = (ctx.h, kv.h, layer, rope.h if rope else None, n, slots.ctypes.data_as(_IP), pos.ctypes.data_as(_IP),
            _dev(q, "q"), _dev(k_new, "k"), _dev(v_new, "v"), _dtype_code(q), n_heads, ctypes.c_float(scale),
            window, ctypes.c_float(cap))
    keep = (slots, pos, q, k_new, v_new, out, q_norm, k_norm)
    if q_norm is None and k_norm is None:
        return Prepared(load().smol_attn_decode, args + (_dev(out, "out"),), "smol_attn_decode", out, keep)
    return Prepared(load().smol_attn_decode_qknorm,
                    args + (_norm_w(q_norm, "q_norm"), _norm_w(k_norm, "k_norm"), ctypes.c_float(eps),
                            _dev(out, "out")), "smol_attn_decode_qknorm", out, keep)


def decode(ctx, kv, layer, rope, slots, pos, q, k_new, v_new, n_heads, scale, window=0, cap=0.0, out=None,
           q_norm=None, k_norm=None, eps=1e-6):
    """Batched single-token decode; see smol_attn_decode. q_norm / k_norm
    (device float32 [head_dim]) select smol_attn_decode_qknorm."""
    return decode_call(ctx, kv, layer, rope, slots, pos, q, k_new, v_new, n_heads, scale, window, cap, out,
                       q_norm, k_norm, eps)()


def causal(ctx, q, k, v, seq_q, seq_k, n_heads, n_kv_heads, head_dim, scale, q_offset, window=0, cap=0.0,
           out=None):
    out = _out_like(seq_q, n_heads, head_dim, q.device, out)
    _check(load().smol_attn_causal(ctx.h, _dev(q, "q"), _dev(k, "k"), _dev(v, "v"), _dtype_code(q), seq_q,
                                   seq_k, n_heads, n_kv_heads, head_dim, ctypes.c_float(scale), q_offset,
                                   window, ctypes.c_float(cap), _dev(out, "out")), "smol_attn_causal")
    return out


def causal_bf16(ctx, q, k, v, seq_q, seq_k, n_heads, n_kv_heads, head_dim, scale, q_offset, window=0, cap=0.0,
                out=None):
    """bf16 in, bf16 out (truncated); see smol_attn_causal_bf16. Returns a
    torch int16 tensor holding the bf16 bits."""
    import torch
    for t, nm in ((q, "q"), (k, "k"), (v, "v")):
        if t.dtype != torch.bfloat16:
            raise SmolAttnError("%s must be bfloat16" % nm)
    if out is None:
        out = torch.empty((seq_q, n_heads * head_dim), dtype=torch.int16, device=q.device)
    _check(load().smol_attn_causal_bf16(ctx.h, _dev(q, "q"), _dev(k, "k"), _dev(v, "v"), seq_q, seq_k, n_heads,
                                        n_kv_heads, head_dim, ctypes.c_float(scale), q_offset, window,
                                        ctypes.c_float(cap), _dev(out, "out")), "smol_attn_causal_bf16")
    return out


def bidirectional_call(ctx, q, k, v, seq, n_heads, head_dim, scale, window_starts, out=None):
    """smol_attn_bidirectional as a Prepared call"""
    ws = np.ascontiguousarray(window_starts, np.int32)
    out = _out_like(seq, n_heads, head_dim, q.device, out)
    args = (ctx.h, _dev(q, "q"), _dev(k, "k"), _dev(v, "v"), _dtype_code(q), seq, n_heads, head_dim,
            ctypes.c_float(scale), ws.ctypes.data_as(_IP), len(ws) - 1, _dev(out, "out"))
    return Prepared(load().smol_attn_bidirectional, args, "smol_attn_bidirectional", out, (ws, q, k, v, out))


def bidirectional(ctx, q, k, v, seq, n_heads, head_dim, scale, window_starts, out=None):
    return bidirectional_call(ctx, q, k, v, seq, n_heads, head_dim, scale, window_starts, out)()


def apply_rope(ctx, rope, x, positions, n_heads):
    pos = np.ascontiguousarray(positions, np.int32)
    _check(load().smol_attn_apply_rope(ctx.h, rope.h, _dev(x, "x"), pos.ctypes.data_as(_IP), len(pos), n_heads),
           "smol_attn_apply_rope")
    return x


def norm_rope(ctx, rope, x, weight, eps, positions, n_heads, head_dim):
    """In place: per-head RMSNorm (weight None: skipped) then RoPE (rope None:
    skipped); see smol_attn_norm_rope."""
    seq = x.shape[0]
    pos = None if positions is None else np.ascontiguousarray(positions, np.int32)
    if pos is not None and len(pos) != seq:
        raise SmolAttnError("%d positions for %d rows" % (len(pos), seq))
    _check(load().smol_attn_norm_rope(ctx.h, rope.h if rope else None, _dev(x, "x"), _norm_w(weight, "weight"),
                                      ctypes.c_float(eps), None if pos is None else pos.ctypes.data_as(_IP), seq,
                                      n_heads, head_dim), "smol_attn_norm_rope")
    return x


def norm_rope_bf16(ctx, rope, x, weight, eps, pos0, n_heads, head_dim):
    """In place on a device bf16 tensor [seq, n_heads*head_dim]: the bf16
    decoder's truncating per-head norm (weight None: skipped) and interleaved
    rotation at rows pos0.. (rope None: skipped); see smol_attn_norm_rope_bf16."""
    _check(load().smol_attn_norm_rope_bf16(ctx.h, rope.h if rope else None, _dev(x, "x"), _norm_w(weight, "weight"),
                                           ctypes.c_float(eps), pos0, x.shape[0], n_heads, head_dim),
           "smol_attn_norm_rope_bf16")
    return x


class QknConfig(ctypes.Structure):
    """smol_qkn_attn_config (include/smol_qkn_attn.h): the qkn_config_t fields of the attention block."""
    _fields_ = [("n_layers", _c_int), ("n_heads", _c_int), ("n_kv_heads", _c_int), ("head_dim", _c_int),
                ("eps", _c_float), ("rope_theta", _c_float), ("rope_local_theta", _c_float),
                ("rope_type", _c_int), ("sliding_window", _c_int), ("attn_logit_softcap", _c_float),
                ("bf16", _c_int), ("on_device", _c_int), ("device", _c_int), ("max_seq", _c_int)]


class _LayerWeights(ctypes.Structure):
    _fields_ = [(n, _vp) for n in ("input_norm", "wq", "wk", "wv", "wo", "post_attn_norm", "pre_ffn_norm",
                                   "post_ffn_norm", "gate_up", "down")]


class QknLayerWeights:
    """smol_qkn_layer_weights from device tensors (fp32 norms, bf16 / int16-bit weights);
    the tensors are kept alive with the struct."""

    def __init__(self, **t):
        self.t = t
        self.s = _LayerWeights(**{k: (ctypes.c_void_p(v.data_ptr()) if v is not None else None)
                                  for k, v in t.items()})


class QknStepGraph:
    """smol_qkn_step_graph_*: one decode step of every layer of a binding,
    captured on x [1, dim] (device fp32) with weights (one QknLayerWeights per
    layer); launch(pos) replays it at pos. The tensors are kept alive with it."""

    def __init__(self, blk, x, weights, dim, inter, act, max_pos):
        self.blk, self.x, self.weights = blk, x, list(weights)
        arr_t = type(self.weights[0].s) * len(self.weights)
        self._arr = arr_t(*[w.s for w in self.weights])
        self.h = _vp()
        _check(load().smol_qkn_step_graph_create(blk.addr, _dev(x, "x"), self._arr, dim, inter, act, max_pos,
                                                 ctypes.byref(self.h)), "smol_qkn_step_graph_create")

    def launch(self, pos):
        _check(load().smol_qkn_step_graph_launch(self.h, pos), "smol_qkn_step_graph_launch")

    def close(self):
        if self.h:
            load().smol_qkn_step_graph_destroy(self.h)
            self.h = _vp()


class QknAttn:
    """The decoder attention block bound to a decoder context (`owner`, any
    object whose address keys the registry; a ctypes buffer stands for the
    qkn_ctx_t). Host numpy arrays in and out when on_device is 0 (fp32, or
    bf16 bits as uint16 with bf16=1); device tensors when on_device is 1."""

    def __init__(self, owner, **cfg):
        self.owner = owner
        self.cfg = QknConfig(**cfg)
        self.addr = ctypes.c_void_p(ctypes.addressof(owner))
        _check(load().smol_qkn_attn_bind(self.addr, ctypes.byref(self.cfg)), "smol_qkn_attn_bind")
        _live.add(self)

    def set_layer(self, layer, is_sliding=0, q_norm=None, k_norm=None):
        def w(a):
            if a is None:
                return None
            a = np.ascontiguousarray(a, np.float32)
            self._keep = getattr(self, "_keep", []) + [a]
            return a.ctypes.data_as(_FP)
        _check(load().smol_qkn_attn_set_layer(self.addr, layer, 1 if is_sliding else 0, w(q_norm), w(k_norm)),
               "smol_qkn_attn_set_layer")

    def _io(self, q, k, v, rows):
        c = self.cfg
        qd, kvd = c.n_heads * c.head_dim, c.n_kv_heads * c.head_dim
        if c.on_device:
            import torch
            out = torch.empty((rows, qd), dtype=torch.bfloat16 if c.bf16 else torch.float32, device=q.device)
            return (_dev(q, "q"), _dev(k, "k"), _dev(v, "v"), _dev(out, "attn_out")), out
        dt = np.uint16 if c.bf16 else np.float32
        q = np.ascontiguousarray(q, dt).reshape(rows, qd)
        k = np.ascontiguousarray(k, dt).reshape(rows, kvd)
        v = np.ascontiguousarray(v, dt).reshape(rows, kvd)
        out = np.zeros((rows, qd), dt)
        self._hold = (q, k, v)
        return tuple(ctypes.c_void_p(a.ctypes.data) for a in (q, k, v, out)), out

    def prefill(self, layer, start_pos, q, k, v):
        rows = q.shape[0]
        ptrs, out = self._io(q, k, v, rows)
        _check(load().smol_qkn_attn_prefill(self.addr, layer, start_pos, rows, *ptrs), "smol_qkn_attn_prefill")
        return out

    def forward(self, layer, pos, q, k, v):
        ptrs, out = self._io(q, k, v, 1)
        _check(load().smol_qkn_attn_forward(self.addr, layer, pos, *ptrs), "smol_qkn_attn_forward")
        return out

    def layer_forward(self, layer, pos, x, weights, dim, inter, act=1):
        """smol_qkn_layer_forward: x [1, dim] device fp32, updated in place;
        weights a QknLayerWeights of device tensors"""
        _check(load().smol_qkn_layer_forward(self.addr, layer, pos, _dev(x, "x"), ctypes.byref(weights.s), dim,
                                             inter, act), "smol_qkn_layer_forward")
        return x

    def layer_prefill(self, layer, start_pos, x, weights, dim, inter, act=1):
        _check(load().smol_qkn_layer_prefill(self.addr, layer, start_pos, x.shape[0], _dev(x, "x"),
                                             ctypes.byref(weights.s), dim, inter, act), "smol_qkn_layer_prefill")
        return x

    def layer_forward_bf16(self, layer, pos, x, weights, dim, inter):
        """smol_qkn_layer_forward_bf16: x [1, dim] device bf16 bits, updated in place"""
        _check(load().smol_qkn_layer_forward_bf16(self.addr, layer, pos, _dev(x, "x"), ctypes.byref(weights.s),
                                                  dim, inter), "smol_qkn_layer_forward_bf16")
        return x

    def layer_prefill_bf16(self, layer, start_pos, x, weights, dim, inter):
        _check(load().smol_qkn_layer_prefill_bf16(self.addr, layer, start_pos, x.shape[0], _dev(x, "x"),
                                                  ctypes.byref(weights.s), dim, inter),
               "smol_qkn_layer_prefill_bf16")
        return x

    def synchronize(self):
        _check(load().smol_qkn_layer_synchronize(self.addr), "smol_qkn_layer_synchronize")

    def read_cache(self, layer, pos0, n):
        kvd = self.cfg.n_kv_heads * self.cfg.head_dim
        k = np.zeros((n, kvd), np.uint16)
        v = np.zeros_like(k)
        _check(load().smol_qkn_attn_read_cache(self.addr, layer, pos0, n, k.ctypes.data_as(_U16P),
                                               v.ctypes.data_as(_U16P)), "smol_qkn_attn_read_cache")
        return k, v

    def close(self):
        if self.addr:
            load().smol_qkn_attn_unbind(self.addr)
            self.addr = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


# ----------------------------------------------- reference-signature drop-ins

def _f32(a):
    a = np.ascontiguousarray(a, np.float32)
    return a, a.ctypes.data_as(_FP)


def smol_causal_attention(out, Q, K, V, seq_q, seq_k, n_heads, n_kv_heads, head_dim, scale, q_offset):
    assert out.dtype == np.float32 and out.flags.c_contiguous
    Qa, q = _f32(Q); Ka, k = _f32(K); Va, v = _f32(V)
    load().smol_causal_attention(out.ctypes.data_as(_FP), q, k, v, seq_q, seq_k, n_heads, n_kv_heads, head_dim,
                                 ctypes.c_float(scale), q_offset)


def smol_sliding_window_attention(out, Q, K, V, seq_q, seq_k, n_heads, n_kv_heads, head_dim, scale, q_offset,
                                  window_size):
    assert out.dtype == np.float32 and out.flags.c_contiguous
    Qa, q = _f32(Q); Ka, k = _f32(K); Va, v = _f32(V)
    load().smol_sliding_window_attention(out.ctypes.data_as(_FP), q, k, v, seq_q, seq_k, n_heads, n_kv_heads,
                                         head_dim, ctypes.c_float(scale), q_offset, window_size)


def smol_causal_attention_softcap(out, Q, K, V, seq_q, seq_k, n_heads, n_kv_heads, head_dim, scale, q_offset, cap):
    assert out.dtype == np.float32 and out.flags.c_contiguous
    Qa, q = _f32(Q); Ka, k = _f32(K); Va, v = _f32(V)
    load().smol_causal_attention_softcap(out.ctypes.data_as(_FP), q, k, v, seq_q, seq_k, n_heads, n_kv_heads,
                                         head_dim, ctypes.c_float(scale), q_offset, ctypes.c_float(cap))


def smol_sliding_window_attention_softcap(out, Q, K, V, seq_q, seq_k, n_heads, n_kv_heads, head_dim, scale,
                                          q_offset, window_size, cap):
    assert out.dtype == np.float32 and out.flags.c_contiguous
    Qa, q = _f32(Q); Ka, k = _f32(K); Va, v = _f32(V)
    load().smol_sliding_window_attention_softcap(out.ctypes.data_as(_FP), q, k, v, seq_q, seq_k, n_heads,
                                                 n_kv_heads, head_dim, ctypes.c_float(scale), q_offset,
                                                 window_size, ctypes.c_float(cap))


def smol_bidirectional_attention(out, Q, K, V, seq, n_heads, head_dim, scale, window_starts, n_windows):
    assert out.dtype == np.float32 and out.flags.c_contiguous
    Qa, q = _f32(Q); Ka, k = _f32(K); Va, v = _f32(V)
    ws = np.ascontiguousarray(window_starts, np.int32)
    load().smol_bidirectional_attention(out.ctypes.data_as(_FP), q, k, v, seq, n_heads, head_dim,
                                        ctypes.c_float(scale), ws.ctypes.data_as(_IP), n_windows)


def smol_compute_rope_neox(cos_out, sin_out, positions, seq, head_dim, theta):
    pos = np.ascontiguousarray(positions, np.int32)
    load().smol_compute_rope_neox(cos_out.ctypes.data_as(_FP), sin_out.ctypes.data_as(_FP),
                                  pos.ctypes.data_as(_IP), seq, head_dim, ctypes.c_float(theta))


def smol_compute_rope_interleaved(cos_out, sin_out, positions, seq, head_dim, theta):
    pos = np.ascontiguousarray(positions, np.int32)
    load().smol_compute_rope_interleaved(cos_out.ctypes.data_as(_FP), sin_out.ctypes.data_as(_FP),
                                         pos.ctypes.data_as(_IP), seq, head_dim, ctypes.c_float(theta))


def smol_apply_rope_neox(x, cos_vals, sin_vals, seq, n_heads, head_dim):
    assert x.dtype == np.float32 and x.flags.c_contiguous
    Ca, c = _f32(cos_vals); Sa, s = _f32(sin_vals)
    load().smol_apply_rope_neox(x.ctypes.data_as(_FP), c, s, seq, n_heads, head_dim)


def smol_apply_rope_interleaved(x, cos_vals, sin_vals, seq, n_heads, head_dim):
    assert x.dtype == np.float32 and x.flags.c_contiguous
    Ca, c = _f32(cos_vals); Sa, s = _f32(sin_vals)
    load().smol_apply_rope_interleaved(x.ctypes.data_as(_FP), c, s, seq, n_heads, head_dim)


def smol_rms_norm_per_head(x, weight, seq_len, n_heads, head_dim, eps):
    assert x.dtype == np.float32 and x.flags.c_contiguous
    Wa, w = _f32(weight)
    load().smol_rms_norm_per_head(x.ctypes.data_as(_FP), w, seq_len, n_heads, head_dim, ctypes.c_float(eps))


# ------------------------------------------------ bf16-weight projections

GEMV_MAX_SEQ = 4  # SMOL_LINEAR_GEMV_MAX_SEQ


def _wbits(w, what):
    """a device weight as bf16 bits: a bfloat16 tensor, or int16 / uint16 bits"""
    import torch
    if w.dtype not in (torch.bfloat16, torch.int16, torch.uint16):
        raise SmolAttnError("%s must be bfloat16 (or its bits as int16)" % what)
    return _dev(w, what)


def linear(ctx, x, w, bias=None, out=None, out_bf16=False):
    """y = x W^T (+ bias) on the device (smol_linear_dev). x [seq, in] float32 or
    bfloat16; w [out, in] bf16; bias [out] float32 or None. Returns y
    [seq, out], float32, or the truncated bf16 bits as int16 when out_bf16."""
    import torch
    seq, in_dim = x.shape
    out_dim = w.shape[0]
    if w.shape[1] != in_dim:
        raise SmolAttnError("w must be [out, in]")
    if out is None:
        out = torch.empty((seq, out_dim), dtype=torch.int16 if out_bf16 else torch.float32, device=x.device)
    b = _dev(bias, "bias") if bias is not None else None
    _check(load().smol_linear_dev(ctx.h, _dev(out, "out"), BF16 if out_bf16 else F32, _dev(x, "x"),
                                  _dtype_code(x), _wbits(w, "w"), b, seq, in_dim, out_dim), "smol_linear_dev")
    return out


def linear_qkv(ctx, x, wq, wk, wv, out_bf16=False):
    """q, k, v = x Wq^T, x Wk^T, x Wv^T (smol_linear_qkv_dev)"""
    import torch
    seq, in_dim = x.shape
    q_dim, kv_dim = wq.shape[0], wk.shape[0]
    dt = torch.int16 if out_bf16 else torch.float32
    q = torch.empty((seq, q_dim), dtype=dt, device=x.device)
    k = torch.empty((seq, kv_dim), dtype=dt, device=x.device)
    v = torch.empty((seq, kv_dim), dtype=dt, device=x.device)
    _check(load().smol_linear_qkv_dev(ctx.h, _dev(q, "q"), _dev(k, "k"), _dev(v, "v"), BF16 if out_bf16 else F32,
                                      _dev(x, "x"), _dtype_code(x), _wbits(wq, "wq"), _wbits(wk, "wk"),
                                      _wbits(wv, "wv"), seq, in_dim, q_dim, kv_dim), "smol_linear_qkv_dev")
    return q, k, v


ACT_NONE, ACT_SWIGLU, ACT_GEGLU = 0, 1, 2


class _LinearOps(ctypes.Structure):
    _fields_ = [("norm_weight", _vp), ("norm_eps", _c_float), ("act", _c_int), ("residual", _vp)]


def linear_ops(ctx, x, w, bias=None, norm_weight=None, eps=1e-6, act=ACT_NONE, residual=None, out=None):
    """y = residual + act(rmsnorm(x) W^T + bias) on the device (smol_linear_ops_dev); fp32 x [seq, in],
    bf16 w [out, in]; y [seq, out] (or [seq, out / 2] with an activation). `out` may be `residual`."""
    import torch
    seq, in_dim = x.shape
    out_dim = w.shape[0]
    if out is None:
        out = torch.empty((seq, out_dim // 2 if act else out_dim), dtype=torch.float32, device=x.device)
    ops = _LinearOps(_dev(norm_weight, "norm_weight") if norm_weight is not None else None, eps, act,
                     _dev(residual, "residual") if residual is not None else None)
    _check(load().smol_linear_ops_dev(ctx.h, _dev(out, "out"), _dev(x, "x"), _wbits(w, "w"),
                                      _dev(bias, "bias") if bias is not None else None, seq, in_dim, out_dim,
                                      ctypes.byref(ops)), "smol_linear_ops_dev")
    return out


def rms_norm(ctx, x, weight, eps, out=None, residual=None):
    """smol_rms_norm_dev: fp32 rows [seq, dim] (+ residual)"""
    import torch
    seq, dim = x.shape
    if out is None:
        out = torch.empty_like(x)
    _check(load().smol_rms_norm_dev(ctx.h, _dev(out, "out"), _dev(x, "x"), _dev(weight, "weight"),
                                    _dev(residual, "residual") if residual is not None else None, seq, dim,
                                    ctypes.c_float(eps)), "smol_rms_norm_dev")
    return out


def bf16_rms_norm(ctx, x, weight, eps, out=None):
    """smol_bf16_rms_norm_dev: bf16-bit rows [seq, dim] (int16 or bfloat16 tensor); out may be x"""
    import torch
    seq, dim = x.shape
    if out is None:
        out = torch.empty_like(x)
    _check(load().smol_bf16_rms_norm_dev(ctx.h, _dev(out, "out"), _dev(x, "x"), _dev(weight, "weight"), seq, dim,
                                         ctypes.c_float(eps)), "smol_bf16_rms_norm_dev")
    return out


def bf16_add_norm(ctx, x, p=None, p_norm=None, next_norm=None, eps=1e-6, xn=None):
    """smol_bf16_add_norm_dev: x = x + (p_norm ? norm(p) : p) in place, then xn = norm(x, next_norm)"""
    import torch
    seq, dim = x.shape
    if next_norm is not None and xn is None:
        xn = torch.empty_like(x)
    opt = lambda t, n: _dev(t, n) if t is not None else None  # noqa: E731
    _check(load().smol_bf16_add_norm_dev(ctx.h, _dev(x, "x"), opt(p, "p"), opt(p_norm, "p_norm"),
                                         opt(next_norm, "next_norm"), opt(xn, "xn"), seq, dim, ctypes.c_float(eps)),
           "smol_bf16_add_norm_dev")
    return xn


def bf16_geglu(ctx, gate_up, out=None):
    """smol_bf16_geglu_dev: bf16-bit rows [seq, 2 * inter] -> [seq, inter]"""
    import torch
    seq, two = gate_up.shape
    if out is None:
        out = torch.empty((seq, two // 2), dtype=gate_up.dtype, device=gate_up.device)
    _check(load().smol_bf16_geglu_dev(ctx.h, _dev(out, "out"), _dev(gate_up, "gate_up"), seq, two // 2),
           "smol_bf16_geglu_dev")
    return out


def linear_qkv_norm(ctx, x, wq, wk, wv, norm_weight, eps):
    """smol_linear_qkv_norm_dev: q, k, v of rmsnorm(x) (fp32)"""
    import torch
    seq, in_dim = x.shape
    q_dim, kv_dim = wq.shape[0], wk.shape[0]
    q = torch.empty((seq, q_dim), dtype=torch.float32, device=x.device)
    k = torch.empty((seq, kv_dim), dtype=torch.float32, device=x.device)
    v = torch.empty((seq, kv_dim), dtype=torch.float32, device=x.device)
    _check(load().smol_linear_qkv_norm_dev(ctx.h, _dev(q, "q"), _dev(k, "k"), _dev(v, "v"), _dev(x, "x"),
                                           _wbits(wq, "wq"), _wbits(wk, "wk"), _wbits(wv, "wv"), seq, in_dim,
                                           q_dim, kv_dim,
                                           _dev(norm_weight, "norm") if norm_weight is not None else None,
                                           ctypes.c_float(eps)), "smol_linear_qkv_norm_dev")
    return q, k, v


def _u16(a):
    a = np.ascontiguousarray(a, np.uint16)
    return a, a.ctypes.data_as(_U16P)


def smol_linear_bf16(y, x, W_bf16, b, seq_len, in_dim, out_dim):
    assert y.dtype == np.float32 and y.flags.c_contiguous
    Xa, xp = _f32(x); Wa, wp = _u16(W_bf16)
    Ba, bp = _f32(b) if b is not None else (None, None)
    load().smol_linear_bf16(y.ctypes.data_as(_FP), xp, wp, bp, seq_len, in_dim, out_dim)


def smol_linear_nobias_bf16(y, x, W_bf16, seq_len, in_dim, out_dim):
    assert y.dtype == np.float32 and y.flags.c_contiguous
    Xa, xp = _f32(x); Wa, wp = _u16(W_bf16)
    load().smol_linear_nobias_bf16(y.ctypes.data_as(_FP), xp, wp, seq_len, in_dim, out_dim)


def smol_linear_nobias_bf16_qkv(q, k, v, x, Wq_bf16, Wk_bf16, Wv_bf16, in_dim, q_dim, kv_dim):
    for a in (q, k, v):
        assert a.dtype == np.float32 and a.flags.c_contiguous
    Xa, xp = _f32(x)
    Qa, wq = _u16(Wq_bf16); Ka, wk = _u16(Wk_bf16); Va, wv = _u16(Wv_bf16)
    load().smol_linear_nobias_bf16_qkv(q.ctypes.data_as(_FP), k.ctypes.data_as(_FP), v.ctypes.data_as(_FP), xp,
                                       wq, wk, wv, in_dim, q_dim, kv_dim)


def smol_matmul_t_bf16(C, A, B_bf16, M, K, N):
    assert C.dtype == np.float32 and C.flags.c_contiguous
    Aa, ap = _f32(A); Ba, bp = _u16(B_bf16)
    load().smol_matmul_t_bf16(C.ctypes.data_as(_FP), ap, bp, M, K, N)
