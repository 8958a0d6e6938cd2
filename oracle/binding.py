"""ctypes binding of the CPU oracle (liboracle.so) -- TEST INFRASTRUCTURE ONLY.

Imported only by tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg, where the
oracle is what results are compared against (or the timed CPU baseline), never the product path.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

_f32p = ctypes.POINTER(ctypes.c_float)
_u16p = ctypes.POINTER(ctypes.c_uint16)
_ip = ctypes.POINTER(ctypes.c_int)


class OracleConfig(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int) for n in (
        "dim", "hidden_dim", "head_dim", "n_layers", "n_heads", "n_kv_heads", "vocab_size",
        "max_seq_len", "rotary_dim")] + [
        ("rope_theta", ctypes.c_float), ("norm_eps", ctypes.c_float), ("qkv_clip", ctypes.c_float),
        ("act", ctypes.c_int)]


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            raise RuntimeError(f"oracle library not built: {_LIB_PATH} (run `make -C oracle`)")
        L = ctypes.CDLL(_LIB_PATH)
        L.oracle_h2f.restype = ctypes.c_float
        L.oracle_h2f.argtypes = [ctypes.c_uint16]
        L.oracle_f2h.restype = ctypes.c_uint16
        L.oracle_f2h.argtypes = [ctypes.c_float]
        L.oracle_h2f_array.argtypes = [_u16p, _f32p, ctypes.c_size_t]
        L.oracle_f2h_array.argtypes = [_f32p, _u16p, ctypes.c_size_t]
        L.oracle_matmul_f16.argtypes = [_f32p, _f32p, _u16p, ctypes.c_int, ctypes.c_int]
        L.oracle_matmul_f32.argtypes = [_f32p, _f32p, _f32p, ctypes.c_int, ctypes.c_int]
        L.oracle_rmsnorm.argtypes = [_f32p, _f32p, _f32p, ctypes.c_int, ctypes.c_float]
        L.oracle_softmax.argtypes = [_f32p, _f32p, ctypes.c_int]
        L.oracle_silu.restype = ctypes.c_float
        L.oracle_silu.argtypes = [ctypes.c_float]
        L.oracle_gelu.restype = ctypes.c_float
        L.oracle_gelu.argtypes = [ctypes.c_float]
        L.oracle_rope.argtypes = [_f32p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_float, ctypes.c_int]
        L.oracle_k_cache_idx.restype = ctypes.c_int
        L.oracle_k_cache_idx.argtypes = [ctypes.c_int] * 3
        L.oracle_attn.argtypes = [_f32p, _f32p, _f32p, _u16p, _u16p] + [ctypes.c_int] * 4
        L.oracle_mha.argtypes = [_f32p, _f32p, _u16p, _u16p, _f32p] + [ctypes.c_int] * 5
        L.oracle_ffn.argtypes = [_f32p, _f32p, _u16p, _u16p, _u16p] + [ctypes.c_int] * 3
        L.oracle_argmax.restype = ctypes.c_int
        L.oracle_argmax.argtypes = [_f32p, ctypes.c_int]
        L.oracle_positions.argtypes = [ctypes.c_int, ctypes.c_int, _ip, _ip, _ip]
        L.oracle_create.restype = ctypes.c_int
        L.oracle_create.argtypes = [ctypes.POINTER(OracleConfig), ctypes.POINTER(ctypes.c_void_p)]
        L.oracle_destroy.argtypes = [ctypes.c_void_p]
        L.oracle_set_layer.restype = ctypes.c_int
        L.oracle_set_layer.argtypes = [ctypes.c_void_p, ctypes.c_int, _f32p, _f32p] + [_u16p] * 7
        L.oracle_set_globals.restype = ctypes.c_int
        L.oracle_set_globals.argtypes = [ctypes.c_void_p, _u16p, _f32p, _u16p]
        L.oracle_forward.restype = ctypes.c_int
        L.oracle_forward.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int, _f32p]
        L.oracle_key_cache.restype = _u16p
        L.oracle_key_cache.argtypes = [ctypes.c_void_p, ctypes.c_int]
        L.oracle_value_cache.restype = _u16p
        L.oracle_value_cache.argtypes = [ctypes.c_void_p, ctypes.c_int]
        L.oracle_x.restype = _f32p
        L.oracle_x.argtypes = [ctypes.c_void_p]
        L.oracle_set_rope_freqs.restype = ctypes.c_int
        L.oracle_set_rope_freqs.argtypes = [ctypes.c_void_p, _f32p, ctypes.c_int]
        _lib = L
    return _lib


def _f32(a):
    a = np.ascontiguousarray(a, dtype=np.float32)
    return a, a.ctypes.data_as(_f32p)


def _u16(a):
    a = np.ascontiguousarray(a)
    if a.dtype == np.float16:
        a = a.view(np.uint16)
    a = np.ascontiguousarray(a, dtype=np.uint16)
    return a, a.ctypes.data_as(_u16p)


def matmul_f16(x, w):
    """W (d, n) fp16 times x (n) -> (d) fp32 (infer.cpp:63-100)."""
    d, n = w.shape
    x, xp = _f32(x)
    w, wp = _u16(w)
    out = np.zeros(d, np.float32)
    lib().oracle_matmul_f16(out.ctypes.data_as(_f32p), xp, wp, n, d)
    return out


def matmul_f32(x, w):
    d, n = w.shape
    x, xp = _f32(x)
    w, wp = _f32(w)
    out = np.zeros(d, np.float32)
    lib().oracle_matmul_f32(out.ctypes.data_as(_f32p), xp, wp, n, d)
    return out


def rmsnorm(x, g, eps):
    x, xp = _f32(x)
    g, gp = _f32(g)
    out = np.zeros_like(x)
    lib().oracle_rmsnorm(out.ctypes.data_as(_f32p), xp, gp, x.size, eps)
    return out


def softmax(x):
    x, xp = _f32(x)
    out = np.zeros_like(x)
    lib().oracle_softmax(out.ctypes.data_as(_f32p), xp, x.size)
    return out


def rope(vec, head_dim, pos, theta, rotary_dim):
    v = np.array(vec, dtype=np.float32, copy=True)
    lib().oracle_rope(v.ctypes.data_as(_f32p), v.size, head_dim, pos, theta, rotary_dim)
    return v


def attn(q, kh, vh, head_dim, max_seq_len, kv_len):
    """One head over a (head_dim, max_seq_len) cache slice; returns (xout, att)."""
    q, qp = _f32(q)
    kh, kp = _u16(kh)
    vh, vp = _u16(vh)
    out = np.zeros(head_dim, np.float32)
    att = np.zeros(max(kv_len, 1), np.float32)
    lib().oracle_attn(out.ctypes.data_as(_f32p), att.ctypes.data_as(_f32p), qp, kp, vp, head_dim, 1, max_seq_len, kv_len)
    return out, att


def mha(q, kb, vb, head_dim, kv_len, max_seq_len, n_heads, n_kv_heads):
    q, qp = _f32(q)
    kb, kp = _u16(kb)
    vb, vp = _u16(vb)
    out = np.zeros(n_heads * head_dim, np.float32)
    att = np.zeros(n_heads * max_seq_len, np.float32)
    lib().oracle_mha(out.ctypes.data_as(_f32p), att.ctypes.data_as(_f32p), kp, vp, qp, head_dim, kv_len,
                     max_seq_len, n_heads, n_kv_heads)
    return out, att.reshape(n_heads, max_seq_len)


def ffn(x, w1, w2, w3, act=1):
    hidden, dim = w1.shape
    x, xp = _f32(x)
    w1, p1 = _u16(w1)
    w2, p2 = _u16(w2)
    w3, p3 = _u16(w3)
    out = np.zeros(dim, np.float32)
    lib().oracle_ffn(out.ctypes.data_as(_f32p), xp, p1, p2, p3, hidden, dim, act)
    return out


def argmax(logits):
    lg, p = _f32(logits)
    return int(lib().oracle_argmax(p, lg.size))


def positions(pos, max_seq_len):
    a, b, c = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    lib().oracle_positions(pos, max_seq_len, ctypes.byref(a), ctypes.byref(b), ctypes.byref(c))
    return a.value, b.value, c.value


def k_cache_idx(hi, t, max_seq_len):
    return int(lib().oracle_k_cache_idx(hi, t, max_seq_len))


def h2f(bits):
    b, bp = _u16(bits)
    out = np.zeros(b.size, np.float32)
    lib().oracle_h2f_array(bp, out.ctypes.data_as(_f32p), b.size)
    return out


def f2h(vals):
    v, vp = _f32(vals)
    out = np.zeros(v.size, np.uint16)
    lib().oracle_f2h_array(vp, out.ctypes.data_as(_u16p), v.size)
    return out


def make_config(cfg) -> OracleConfig:
    """Accepts any object (or dict) with the Config field names (model.h:56-82)."""
    get = (lambda k: cfg[k]) if isinstance(cfg, dict) else (lambda k: getattr(cfg, k))
    act = get("act")
    if isinstance(act, str):
        act = 1 if act == "silu" else 0
    return OracleConfig(get("dim"), get("hidden_dim"), get("head_dim"), get("n_layers"), get("n_heads"),
                        get("n_kv_heads"), get("vocab_size"), get("max_seq_len"), get("rotary_dim"),
                        float(get("rope_theta")), float(get("norm_eps")), float(get("qkv_clip")), int(act))


class OracleModel:
    """Whole-model CPU forward over borrowed weight arrays (names as in the .yalm file)."""

    def __init__(self, cfg, tensors):
        self.cfg = make_config(cfg)
        self._keep = []
        h = ctypes.c_void_p()
        if lib().oracle_create(ctypes.byref(self.cfg), ctypes.byref(h)) != 0:
            raise ValueError("oracle_create rejected the config")
        self.h = h
        c = self.cfg
        for i in range(c.n_layers):
            p = f"model.layers.{i}."
            ra, rap = _f32(tensors[p + "attn.norm.weight"])
            rf, rfp = _f32(tensors[p + "mlp.norm.weight"])
            ws = [_u16(tensors[p + n]) for n in ("attn.wq.weight", "attn.wk.weight", "attn.wv.weight", "attn.wo.weight",
                                                 "mlp.w1.weight", "mlp.w2.weight", "mlp.w3.weight")]
            self._keep += [ra, rf] + [w for w, _ in ws]
            rc = lib().oracle_set_layer(h, i, rap, rfp, *[wp for _, wp in ws])
            assert rc == 0
        e, ep = _u16(tensors["model.embed.weight"])
        g, gp = _f32(tensors["model.norm.weight"])
        if "model.output.weight" in tensors:
            o, op = _u16(tensors["model.output.weight"])
        else:
            o, op = e, ep
        self._keep += [e, g, o]
        assert lib().oracle_set_globals(h, ep, gp, op) == 0

    def forward(self, token, pos, mode=1):
        logits = np.zeros(self.cfg.vocab_size, np.float32)
        rc = lib().oracle_forward(self.h, token, pos, mode, logits.ctypes.data_as(_f32p))
        if rc != 0:
            raise ValueError(f"oracle_forward failed (token={token}, pos={pos})")
        return logits if mode == 1 else None

    def kv(self, layer):
        c = self.cfg
        n = c.n_kv_heads * c.head_dim * c.max_seq_len
        k = np.ctypeslib.as_array(lib().oracle_key_cache(self.h, layer), shape=(n,)).copy()
        v = np.ctypeslib.as_array(lib().oracle_value_cache(self.h, layer), shape=(n,)).copy()
        return k, v

    def set_kv(self, layer, k, v):
        c = self.cfg
        n = c.n_kv_heads * c.head_dim * c.max_seq_len
        kd = np.ctypeslib.as_array(lib().oracle_key_cache(self.h, layer), shape=(n,))
        vd = np.ctypeslib.as_array(lib().oracle_value_cache(self.h, layer), shape=(n,))
        kd[:] = np.asarray(k).view(np.uint16).reshape(-1)
        vd[:] = np.asarray(v).view(np.uint16).reshape(-1)

    def x(self):
        return np.ctypeslib.as_array(lib().oracle_x(self.h), shape=(self.cfg.dim,)).copy()

    def set_rope_freqs(self, freqs=None):
        """Rotate with these head_dim / 2 frequencies instead of the reference's expression
        (None restores it)."""
        f = np.ascontiguousarray(freqs if freqs is not None else [], np.float32)
        if lib().oracle_set_rope_freqs(self.h, f.ctypes.data_as(_f32p), int(f.size)) != 0:
            raise ValueError("oracle_set_rope_freqs: expected head_dim / 2 frequencies")

    def close(self):
        if self.h:
            lib().oracle_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
