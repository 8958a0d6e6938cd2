"""ctypes binding of libyalm_hip.so (the C-ABI declared in include/yalm_hip.h).

This is what a Python caller (the tests, bench.py) uses to reach the HIP decode path. It loads the
in-tree library and fails loudly if it has not been built: there is no CPU fallback.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libyalm_hip.so")

_f32p = ctypes.POINTER(ctypes.c_float)
_u16p = ctypes.POINTER(ctypes.c_uint16)
_ip = ctypes.POINTER(ctypes.c_int)

MODE_HYDRATE = 0
MODE_LOGITS = 1

# Launch structure of a decode step (yhip_step_plan), as include/yalm_hip.h's YHIP_STEP_*.
STEP_SEPARATE, STEP_ATTN_O, STEP_SPLIT_O, STEP_SINGLE = 0, 1, 2, 3

# Every symbol include/yalm_hip.h declares.
EXPORTS = (
    "yhip_create", "yhip_destroy", "yhip_upload_layer", "yhip_upload_globals", "yhip_forward",
    "yhip_forward_argmax", "yhip_prefill", "yhip_logits_host", "yhip_kv_read", "yhip_kv_write", "yhip_set_option",
    "yhip_debug_read", "yhip_last_error", "yhip_step_stats", "yhip_test_matvec", "yhip_test_ffn", "yhip_test_attention",
    "yhip_test_qkv", "yhip_test_gemm", "yhip_test_argmax", "yhip_bench_kernel", "yhip_bench_attention",
    "yhip_bench_gemm", "yhip_gemm_variant", "yhip_attention_noalloc", "yhip_kv_fill_normal", "yhip_bench_stream",
    "yhip_step_plan",
)


class HipConfig(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int) for n in (
        "dim", "hidden_dim", "head_dim", "n_layers", "n_heads", "n_kv_heads", "vocab_size",
        "max_seq_len", "rotary_dim")] + [
        ("rope_theta", ctypes.c_float), ("norm_eps", ctypes.c_float), ("qkv_clip", ctypes.c_float),
        ("act", ctypes.c_int)]


class HipError(RuntimeError):
    pass


_lib = None


def lib():
    """Load libyalm_hip.so; raises if it is missing (build with __graft_entry__.build())."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise HipError(f"HIP library not built: {LIB_PATH}")
    L = ctypes.CDLL(LIB_PATH)
    vp = ctypes.c_void_p
    sig = {
        "yhip_create": (ctypes.c_int, [ctypes.POINTER(HipConfig), ctypes.c_int, ctypes.POINTER(vp)]),
        "yhip_destroy": (ctypes.c_int, [vp]),
        "yhip_upload_layer": (ctypes.c_int, [vp, ctypes.c_int, _f32p, _f32p] + [_u16p] * 7),
        "yhip_upload_globals": (ctypes.c_int, [vp, _u16p, _f32p, _u16p]),
        "yhip_forward": (ctypes.c_int, [vp, ctypes.c_int, ctypes.c_int, ctypes.c_int, _f32p]),
        "yhip_forward_argmax": (ctypes.c_int, [vp, ctypes.c_int, ctypes.c_int, _ip]),
        "yhip_prefill": (ctypes.c_int, [vp, _ip, ctypes.c_int, ctypes.c_int, _f32p]),
        "yhip_logits_host": (_f32p, [vp]),
        "yhip_kv_read": (ctypes.c_int, [vp, ctypes.c_int, _u16p, _u16p]),
        "yhip_kv_write": (ctypes.c_int, [vp, ctypes.c_int, _u16p, _u16p]),
        "yhip_set_option": (ctypes.c_int, [vp, ctypes.c_char_p, ctypes.c_int]),
        "yhip_debug_read": (ctypes.c_int, [vp, ctypes.c_int, _f32p, ctypes.c_size_t]),
        "yhip_last_error": (ctypes.c_char_p, [vp]),
        "yhip_step_stats": (ctypes.c_int, [vp, ctypes.POINTER(ctypes.c_double), _ip]),
        "yhip_step_plan": (ctypes.c_int, [vp, ctypes.c_int, _ip, _ip, _ip]),
        "yhip_test_matvec": (ctypes.c_int, [_f32p, _f32p, ctypes.c_float, _u16p, ctypes.c_int, ctypes.c_int,
                                            _f32p, _f32p]),
        "yhip_test_ffn": (ctypes.c_int, [_f32p, _f32p, ctypes.c_float, _u16p, _u16p, _u16p, ctypes.c_int,
                                         ctypes.c_int, ctypes.c_int, _f32p, _f32p]),
        "yhip_test_attention": (ctypes.c_int, [_f32p, _u16p, _u16p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                               ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_float,
                                               ctypes.c_int, _f32p]),
        "yhip_test_qkv": (ctypes.c_int, [_f32p, _f32p, ctypes.c_float, _u16p, _u16p, _u16p] + [ctypes.c_int] * 6
                          + [ctypes.c_float, ctypes.c_float, ctypes.c_int, _f32p, _u16p, _u16p]),
        "yhip_test_gemm": (ctypes.c_int, [_u16p, _u16p, _u16p] + [ctypes.c_int] * 5 + [_f32p, _u16p]),
        "yhip_test_argmax": (ctypes.c_int, [_f32p, ctypes.c_int, _ip]),
        "yhip_gemm_variant": (ctypes.c_int, [ctypes.c_int] * 4 + [_ip] * 3),
        "yhip_kv_fill_normal": (ctypes.c_int, [vp, ctypes.c_int, ctypes.c_ulonglong]),
        "yhip_attention_noalloc": (ctypes.c_int, [vp, vp, vp] + [ctypes.c_int] * 6 + [ctypes.c_float, ctypes.c_int,
                                                                                        vp, vp]),
        "yhip_bench_kernel": (ctypes.c_int, [ctypes.c_int] * 7 + [_f32p]),
        "yhip_bench_attention": (ctypes.c_int, [ctypes.c_int] * 10 + [_f32p]),
        "yhip_bench_gemm": (ctypes.c_int, [ctypes.c_int] * 6 + [_f32p]),
        "yhip_bench_stream": (ctypes.c_int, [ctypes.POINTER(HipConfig), ctypes.c_int, _f32p, _f32p]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


def _check(rc, ctx=None):
    if rc != 0:
        msg = lib().yhip_last_error(ctx)
        raise HipError(f"yalm_hip error {rc}: {msg.decode() if msg else ''}")


def _f32(a):
    a = np.ascontiguousarray(a, dtype=np.float32)
    return a, a.ctypes.data_as(_f32p)


def _u16(a):
    a = np.asarray(a)
    if a.dtype == np.float16:
        a = a.view(np.uint16)
    a = np.ascontiguousarray(a, dtype=np.uint16)
    return a, a.ctypes.data_as(_u16p)


def make_config(cfg) -> HipConfig:
    get = (lambda k: cfg[k]) if isinstance(cfg, dict) else (lambda k: getattr(cfg, k))
    act = get("act")
    if isinstance(act, str):
        act = 1 if act == "silu" else 0
    return HipConfig(get("dim"), get("hidden_dim"), get("head_dim"), get("n_layers"), get("n_heads"),
                     get("n_kv_heads"), get("vocab_size"), get("max_seq_len"), get("rotary_dim"),
                     float(get("rope_theta")), float(get("norm_eps")), float(get("qkv_clip")), int(act))


class HipModel:
    """A device context holding one model's weights and KV caches (one decode stream)."""

    def __init__(self, cfg, tensors=None, device=0):
        self.cfg = make_config(cfg)
        h = ctypes.c_void_p()
        _check(lib().yhip_create(ctypes.byref(self.cfg), device, ctypes.byref(h)))
        self.h = h
        self.owned = True
        if tensors is not None:
            self.upload(tensors)

    @classmethod
    def attach(cls, ctx_ptr, cfg):
        """Non-owning view of a context created elsewhere (e.g. by a host-library session)."""
        self = cls.__new__(cls)
        self.cfg = make_config(cfg)
        self.h = ctypes.c_void_p(ctx_ptr)
        self.owned = False
        return self

    def upload(self, tensors):
        c = self.cfg
        for i in range(c.n_layers):
            p = f"model.layers.{i}."
            keep = [_u16(tensors[p + n]) for n in ("attn.wq.weight", "attn.wk.weight", "attn.wv.weight",
                                                   "attn.wo.weight", "mlp.w1.weight", "mlp.w2.weight",
                                                   "mlp.w3.weight")]
            ra_arr = np.ascontiguousarray(tensors[p + "attn.norm.weight"], np.float32)
            rf_arr = np.ascontiguousarray(tensors[p + "mlp.norm.weight"], np.float32)
            _check(lib().yhip_upload_layer(self.h, i, ra_arr.ctypes.data_as(_f32p), rf_arr.ctypes.data_as(_f32p),
                                           *[ptr for _, ptr in keep]), self.h)
        e, ep = _u16(tensors["model.embed.weight"])
        g, gp = _f32(tensors["model.norm.weight"])
        if "model.output.weight" in tensors:
            o, op = _u16(tensors["model.output.weight"])
        else:
            op = None
        _check(lib().yhip_upload_globals(self.h, ep, gp, op), self.h)

    def forward(self, token, pos, mode=MODE_LOGITS):
        if mode == MODE_HYDRATE:
            _check(lib().yhip_forward(self.h, token, pos, mode, None), self.h)
            return None
        out = np.zeros(self.cfg.vocab_size, np.float32)
        _check(lib().yhip_forward(self.h, token, pos, mode, out.ctypes.data_as(_f32p)), self.h)
        return out

    def forward_argmax(self, token, pos):
        nxt = ctypes.c_int()
        _check(lib().yhip_forward_argmax(self.h, token, pos, ctypes.byref(nxt)), self.h)
        return nxt.value

    def prefill(self, tokens, start_pos=0, logits=True):
        """Batched prompt prefill; returns the last token's logits (or None with logits=False)."""
        toks = np.ascontiguousarray(tokens, dtype=np.int32)
        out = np.zeros(self.cfg.vocab_size, np.float32) if logits else None
        _check(lib().yhip_prefill(self.h, toks.ctypes.data_as(_ip), len(toks), start_pos,
                                  out.ctypes.data_as(_f32p) if logits else None), self.h)
        return out

    def kv(self, layer):
        c = self.cfg
        n = c.n_kv_heads * c.head_dim * c.max_seq_len
        k = np.zeros(n, np.uint16)
        v = np.zeros(n, np.uint16)
        _check(lib().yhip_kv_read(self.h, layer, k.ctypes.data_as(_u16p), v.ctypes.data_as(_u16p)), self.h)
        return k, v

    def set_kv(self, layer, k, v):
        k, kp = _u16(k)
        v, vp = _u16(v)
        _check(lib().yhip_kv_write(self.h, layer, kp, vp), self.h)

    def kv_fill_normal(self, n_positions, seed):
        """Every layer's K/V = fp16 N(0, 1) draws below n_positions, zeros above (on the device)."""
        _check(lib().yhip_kv_fill_normal(self.h, int(n_positions), int(seed)), self.h)

    def set_option(self, key, value):
        _check(lib().yhip_set_option(self.h, key.encode(), int(value)), self.h)

    def step_plan(self, pos):
        """(variant, slices per kv head holding keys, keys per slice) of the decode step at pos under
        the current options; variant is one of STEP_*."""
        out = [ctypes.c_int() for _ in range(3)]
        _check(lib().yhip_step_plan(self.h, int(pos), *[ctypes.byref(o) for o in out]), self.h)
        return tuple(o.value for o in out)

    def step_stats(self):
        """(device microseconds, steps) timed since set_option("stats", 1)."""
        us = ctypes.c_double()
        n = ctypes.c_int()
        _check(lib().yhip_step_stats(self.h, ctypes.byref(us), ctypes.byref(n)), self.h)
        return us.value, n.value

    def debug_read(self, which, n):
        out = np.zeros(n, np.float32)
        _check(lib().yhip_debug_read(self.h, which, out.ctypes.data_as(_f32p), n), self.h)
        return out

    def close(self):
        if self.h and getattr(self, "owned", True):
            lib().yhip_destroy(self.h)
        self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


# ---- kernel-level hooks --------------------------------------------------------------------
def set_test_bpc(n):
    """Workgroups per CU used by the kernel-level hooks (0 = the decode path's default)."""
    _check(lib().yhip_set_option(None, b"test_bpc", int(n)))


def set_gemm_stages(n, bk=32, bm=128):
    """Prefill GEMM variant: -1 = chosen per shape (default); 2..4 = LDS pipeline stages with k-step
    bk and workgroup rows bm (4 stages with 32-deep k-steps, 2 or 3 with 64-deep ones); 6 = the
    eight-wave 256 x 256 kernel (64-deep k-steps, K % 64 == 0)."""
    _check(lib().yhip_set_option(None, b"gemm_stages", int(n)))
    _check(lib().yhip_set_option(None, b"gemm_bk", int(bk)))
    _check(lib().yhip_set_option(None, b"gemm_bm", int(bm)))


def set_gemm_ppsplit(on=True):
    """Process-wide: the eight-wave prefill GEMM splits its last, partial round of tiles along K."""
    _check(lib().yhip_set_option(None, b"gemm_ppsplit", int(bool(on))))


def set_gemm_ksplit(n=0):
    """Prefill GEMM K splits on the LDS-pipeline kernel: 0 = chosen per shape (split when the output
    has too few tiles to fill the GPU), n >= 1 = forced (must divide the k-steps)."""
    _check(lib().yhip_set_option(None, b"gemm_ksplit", int(n)))


def gemm_variant(M, N, K, mode):
    """(stages, k-step, workgroup rows) of the prefill GEMM yhip_prefill runs for this shape and mode
    under the current process-wide options (stages 6 = the eight-wave 256 x 256 kernel, 2..4 = the
    LDS pipeline's depth)."""
    out = [ctypes.c_int() for _ in range(3)]
    _check(lib().yhip_gemm_variant(M, N, K, mode, *[ctypes.byref(o) for o in out]))
    return tuple(o.value for o in out)


def set_upload(stage_mb=64, threads=8):
    """Weight upload: pinned staging chunk size in MB (0 = direct copies from pageable memory) and
    the host threads that fill a chunk."""
    _check(lib().yhip_set_option(None, b"upload_stage_mb", int(stage_mb)))
    _check(lib().yhip_set_option(None, b"upload_threads", int(threads)))


def bench_stream(cfg, reps=10):
    """Memory-only ceiling of one decode step: (ms per token through the step's launch sequence,
    ms per token as one launch)."""
    a, b = ctypes.c_float(), ctypes.c_float()
    c = make_config(cfg)
    _check(lib().yhip_bench_stream(ctypes.byref(c), reps, ctypes.byref(a), ctypes.byref(b)))
    return a.value, b.value


def bench_gemm(M, N, K, mode, warmup=3, reps=20):
    us = ctypes.c_float()
    _check(lib().yhip_bench_gemm(M, N, K, mode, warmup, reps, ctypes.byref(us)))
    return us.value


def set_attn_mfma(on):
    """Attention kernel of the kernel-level hooks: MFMA (where the shape allows) or SIMT."""
    _check(lib().yhip_set_option(None, b"attn_mfma", int(bool(on))))


def matvec(x, w, gain=None, eps=1e-5, resid=None):
    d, n = w.shape
    x, xp = _f32(x)
    w, wp = _u16(w)
    g_keep = np.ascontiguousarray(gain, np.float32) if gain is not None else None
    gp = g_keep.ctypes.data_as(_f32p) if g_keep is not None else None
    r_keep = np.ascontiguousarray(resid, np.float32) if resid is not None else None
    rp = r_keep.ctypes.data_as(_f32p) if r_keep is not None else None
    out = np.zeros(d, np.float32)
    _check(lib().yhip_test_matvec(xp, gp, eps, wp, n, d, rp, out.ctypes.data_as(_f32p)))
    return out


def ffn(x, w1, w2, w3, gain=None, eps=1e-5, act=1, resid=None):
    hidden, dim = w1.shape
    x, xp = _f32(x)
    a1, p1 = _u16(w1)
    a2, p2 = _u16(w2)
    a3, p3 = _u16(w3)
    g_keep = np.ascontiguousarray(gain, np.float32) if gain is not None else None
    r_keep = np.ascontiguousarray(resid, np.float32) if resid is not None else None
    out = np.zeros(dim, np.float32)
    _check(lib().yhip_test_ffn(xp, g_keep.ctypes.data_as(_f32p) if g_keep is not None else None, eps, p1, p2, p3,
                               hidden, dim, act, r_keep.ctypes.data_as(_f32p) if r_keep is not None else None,
                               out.ctypes.data_as(_f32p)))
    return out


def attention(q, kcache, vcache, head_dim, pos, max_seq_len, n_heads, n_kv_heads, nsplit=0, rope_theta=1e6,
              rotary_dim=None):
    """Returns (att_out, kcache_after) -- the K cache changes only in sink mode (pos >= msl)."""
    q, qp = _f32(q)
    k = np.array(np.asarray(kcache).view(np.uint16) if np.asarray(kcache).dtype == np.float16 else kcache,
                 dtype=np.uint16, copy=True)
    v, vp = _u16(vcache)
    out = np.zeros(n_heads * head_dim, np.float32)
    _check(lib().yhip_test_attention(qp, k.ctypes.data_as(_u16p), vp, head_dim, pos, max_seq_len, n_heads,
                                     n_kv_heads, nsplit, rope_theta, rotary_dim or head_dim,
                                     out.ctypes.data_as(_f32p)))
    return out, k


def qkv(x, gain, wq, wk, wv, n_heads, n_kv_heads, head_dim, max_seq_len, pos, kcache, vcache, eps=1e-5,
        rope_theta=1e6, rotary_dim=None, qkv_clip=3.4028234663852886e38):
    dim = wq.shape[1]
    x, xp = _f32(x)
    g_keep = np.ascontiguousarray(gain, np.float32) if gain is not None else None
    aq, pq = _u16(wq)
    ak, pk = _u16(wk)
    av, pv = _u16(wv)
    k = np.array(kcache, dtype=np.uint16, copy=True)
    v = np.array(vcache, dtype=np.uint16, copy=True)
    q = np.zeros(n_heads * head_dim, np.float32)
    _check(lib().yhip_test_qkv(xp, g_keep.ctypes.data_as(_f32p) if g_keep is not None else None, eps, pq, pk, pv,
                               dim, n_heads, n_kv_heads, head_dim, max_seq_len, rotary_dim or head_dim, rope_theta,
                               qkv_clip, pos, q.ctypes.data_as(_f32p), k.ctypes.data_as(_u16p),
                               v.ctypes.data_as(_u16p)))
    return q, k, v


def gemm(a, b, mode=0, b3=None, c=None, act=1):
    """Prefill GEMM hook: mode 0 a @ b.T, mode 1 c + a @ b.T, mode 2 fp16(act(a @ b.T) * (a @ b3.T))."""
    A, ap = _u16(a)
    B, bp = _u16(b)
    M, K = A.shape
    N = B.shape[0]
    if mode == 2:
        B3, b3p = _u16(b3)
        h = np.zeros((M, N), np.uint16)
        _check(lib().yhip_test_gemm(ap, bp, b3p, M, N, K, mode, act, None, h.ctypes.data_as(_u16p)))
        return h
    out = np.zeros((M, N), np.float32) if c is None else np.ascontiguousarray(c, np.float32).copy()
    _check(lib().yhip_test_gemm(ap, bp, None, M, N, K, mode, act, out.ctypes.data_as(_f32p), None))
    return out


def argmax(logits):
    lg, p = _f32(logits)
    out = ctypes.c_int()
    _check(lib().yhip_test_argmax(p, lg.size, ctypes.byref(out)))
    return out.value


def bench_kernel(kind, rows, cols, copies=4, warmup=20, reps=200, blocks_per_cu=0):
    us = ctypes.c_float()
    _check(lib().yhip_bench_kernel(kind, rows, cols, copies, warmup, reps, blocks_per_cu, ctypes.byref(us)))
    return us.value


def bench_attention(kv_len, max_seq_len=4096, nsplit=32, min_slice=64, head_dim=128, n_heads=32, n_kv_heads=8,
                    copies=8, warmup=10, reps=100):
    us = ctypes.c_float()
    _check(lib().yhip_bench_attention(head_dim, n_heads, n_kv_heads, max_seq_len, kv_len, nsplit, min_slice, copies,
                                      warmup, reps, ctypes.byref(us)))
    return us.value
