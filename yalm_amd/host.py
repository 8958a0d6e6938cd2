"""ctypes binding of libyalm_host.so (include/yalm_host.h): the C++ Model/InferenceState/Sampler
session behind one handle, for Python callers (bench.py, tests)."""
from __future__ import annotations

import ctypes
import os

import numpy as np

from . import hip as _hip

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libyalm_host.so")

EXPORTS = (
    "yalm_session_open", "yalm_session_synthetic", "yalm_session_write", "yalm_session_hip", "yalm_session_close",
    "yalm_session_error", "yalm_session_config", "yalm_session_tensor", "yalm_session_hip_ctx",
    "yalm_session_forward", "yalm_session_prefill", "yalm_session_generate", "yalm_session_active_bytes",
    "yalm_uniform_ids",
    "yalm_fill_normal_f16", "yalm_f32_to_f16", "yalm_f16_to_f32",
)

DTYPES = {0: np.float32, 1: np.float16, 2: None, 3: np.uint8, 4: np.uint8, 5: np.int32, 6: np.int16, 7: np.int8,
          8: np.uint8}


class SynthSpec(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int) for n in ("dim", "hidden_dim", "head_dim", "n_layers", "n_heads", "n_kv_heads",
                                            "vocab_size", "max_seq_len")] + [
        ("rope_theta", ctypes.c_float), ("norm_eps", ctypes.c_float), ("std", ctypes.c_float),
        ("seed", ctypes.c_uint64), ("tied_embeddings", ctypes.c_int)]


class HostError(RuntimeError):
    pass


_lib = None
_f32p = ctypes.POINTER(ctypes.c_float)
_u16p = ctypes.POINTER(ctypes.c_uint16)
_ip = ctypes.POINTER(ctypes.c_int)
_dp = ctypes.POINTER(ctypes.c_double)


def lib():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise HostError(f"host library not built: {LIB_PATH}")
    L = ctypes.CDLL(LIB_PATH)
    vp = ctypes.c_void_p
    sig = {
        "yalm_session_open": (ctypes.c_int, [ctypes.c_char_p, ctypes.c_int, ctypes.POINTER(vp)]),
        "yalm_session_synthetic": (ctypes.c_int, [ctypes.POINTER(SynthSpec), ctypes.c_int, ctypes.POINTER(vp)]),
        "yalm_session_write": (ctypes.c_int, [vp, ctypes.c_char_p]),
        "yalm_session_hip": (ctypes.c_int, [vp, ctypes.c_int]),
        "yalm_session_close": (None, [vp]),
        "yalm_session_error": (ctypes.c_char_p, [vp]),
        "yalm_session_config": (ctypes.c_int, [vp, ctypes.POINTER(_hip.HipConfig)]),
        "yalm_session_tensor": (ctypes.c_int, [vp, ctypes.c_char_p, ctypes.POINTER(vp),
                                               ctypes.POINTER(ctypes.c_size_t), _ip, _ip]),
        "yalm_session_hip_ctx": (vp, [vp]),
        "yalm_session_forward": (ctypes.c_int, [vp, ctypes.c_int, ctypes.c_int, ctypes.c_int, _f32p]),
        "yalm_session_prefill": (ctypes.c_int, [vp, _ip, ctypes.c_int, ctypes.c_int, _f32p]),
        "yalm_session_generate": (ctypes.c_int, [vp, _ip, ctypes.c_int, ctypes.c_int, ctypes.c_float, ctypes.c_int,
                                                 ctypes.c_int, ctypes.c_int, _ip, _dp, _dp]),
        "yalm_session_active_bytes": (ctypes.c_size_t, [vp, ctypes.c_size_t]),
        "yalm_uniform_ids": (None, [_ip, ctypes.c_size_t, ctypes.c_uint64, ctypes.c_int]),
        "yalm_fill_normal_f16": (None, [_u16p, ctypes.c_size_t, ctypes.c_uint64, ctypes.c_char_p, ctypes.c_float]),
        "yalm_f32_to_f16": (None, [_f32p, _u16p, ctypes.c_size_t]),
        "yalm_f16_to_f32": (None, [_u16p, _f32p, ctypes.c_size_t]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


SEED = 0x59414C4D

MISTRAL_7B = dict(dim=4096, hidden_dim=14336, head_dim=128, n_layers=32, n_heads=32, n_kv_heads=8, vocab_size=32000,
                  max_seq_len=32768)
TINY = dict(dim=256, hidden_dim=768, head_dim=32, n_layers=4, n_heads=8, n_kv_heads=2, vocab_size=32000,
            max_seq_len=512)


def uniform_ids(n, seed, hi):
    out = np.zeros(n, np.int32)
    lib().yalm_uniform_ids(out.ctypes.data_as(_ip), n, seed, hi)
    return out


def f32_to_f16(a):
    a = np.ascontiguousarray(a, np.float32).reshape(-1)
    out = np.zeros(a.size, np.uint16)
    lib().yalm_f32_to_f16(a.ctypes.data_as(_f32p), out.ctypes.data_as(_u16p), a.size)
    return out


def f16_to_f32(a):
    a = np.ascontiguousarray(a, np.uint16).reshape(-1)
    out = np.zeros(a.size, np.float32)
    lib().yalm_f16_to_f32(a.ctypes.data_as(_u16p), out.ctypes.data_as(_f32p), a.size)
    return out


class Session:
    """Model + InferenceState + Sampler (reference src/main.cpp:121-211 objects)."""

    def __init__(self, handle):
        self.h = handle
        self.on_hip = False

    @classmethod
    def open(cls, path, context=0):
        h = ctypes.c_void_p()
        if lib().yalm_session_open(str(path).encode(), context, ctypes.byref(h)) != 0:
            raise HostError(lib().yalm_session_error(None).decode())
        return cls(h)

    @classmethod
    def synthetic(cls, shape, context=0, seed=SEED, std=0.02, rope_theta=1e6, norm_eps=1e-5, tied=False):
        spec = SynthSpec(shape["dim"], shape["hidden_dim"], shape["head_dim"], shape["n_layers"], shape["n_heads"],
                         shape["n_kv_heads"], shape["vocab_size"], shape["max_seq_len"], rope_theta, norm_eps, std,
                         seed, int(tied))
        h = ctypes.c_void_p()
        if lib().yalm_session_synthetic(ctypes.byref(spec), context, ctypes.byref(h)) != 0:
            raise HostError(lib().yalm_session_error(None).decode())
        return cls(h)

    def _check(self, rc):
        if rc < 0:
            raise HostError(lib().yalm_session_error(self.h).decode())
        return rc

    def write(self, path):
        self._check(lib().yalm_session_write(self.h, str(path).encode()))

    def hip(self, device=0):
        self._check(lib().yalm_session_hip(self.h, device))
        self.on_hip = True

    def config(self):
        c = _hip.HipConfig()
        self._check(lib().yalm_session_config(self.h, ctypes.byref(c)))
        return {f: getattr(c, f) for f, _ in c._fields_}

    def tensor(self, name):
        """Zero-copy NumPy view of a host tensor (fp16 returned as uint16 bit patterns)."""
        data = ctypes.c_void_p()
        nbytes = ctypes.c_size_t()
        dt = ctypes.c_int()
        shape = (ctypes.c_int * 4)()
        self._check(lib().yalm_session_tensor(self.h, name.encode(), ctypes.byref(data), ctypes.byref(nbytes),
                                              ctypes.byref(dt), shape))
        np_dt = {0: np.float32, 1: np.uint16, 8: np.uint8}.get(dt.value)
        if np_dt is None:
            raise HostError(f"unsupported dtype code {dt.value} for {name}")
        n = nbytes.value // np.dtype(np_dt).itemsize
        buf = (ctypes.c_char * nbytes.value).from_address(data.value)
        arr = np.frombuffer(buf, dtype=np_dt, count=n)
        dims = [d for d in shape if d > 0]
        return arr.reshape(dims) if dims else arr

    def tensors(self):
        c = self.config()
        names = ["model.embed.weight", "model.norm.weight", "model.output.weight"]
        for i in range(c["n_layers"]):
            p = f"model.layers.{i}."
            names += [p + n for n in ("attn.norm.weight", "mlp.norm.weight", "attn.wq.weight", "attn.wk.weight",
                                      "attn.wv.weight", "attn.wo.weight", "mlp.w1.weight", "mlp.w2.weight",
                                      "mlp.w3.weight")]
        out = {}
        for n in names:
            try:
                out[n] = self.tensor(n)
            except HostError:
                if n != "model.output.weight":
                    raise
        return out

    def hip_ctx(self):
        return lib().yalm_session_hip_ctx(self.h)

    def forward(self, token, pos, mode=1):
        c = self.config()
        out = np.zeros(c["vocab_size"], np.float32) if mode == 1 else None
        self._check(lib().yalm_session_forward(self.h, token, pos, mode,
                                               out.ctypes.data_as(_f32p) if out is not None else None))
        return out

    def prefill(self, tokens, start_pos=0):
        """Model::prefill: the tokens in one batched pass; returns the last token's logits."""
        tokens = np.ascontiguousarray(tokens, np.int32)
        out = np.zeros(self.config()["vocab_size"], np.float32)
        self._check(lib().yalm_session_prefill(self.h, tokens.ctypes.data_as(_ip), tokens.size, start_pos,
                                               out.ctypes.data_as(_f32p)))
        return out

    def generate(self, prompt, n_steps, temperature=0.0, device_argmax=True, stop_at_eos=False, prefill=False):
        """Returns (tokens, step_seconds, hydrate_seconds) of the reference completion loop; with
        prefill=True the prompt goes through one batched Model::prefill instead of token steps."""
        prompt = np.ascontiguousarray(prompt, np.int32)
        toks = np.zeros(max(n_steps, 1), np.int32)
        secs = np.zeros(max(n_steps, 1), np.float64)
        hyd = ctypes.c_double()
        n = self._check(lib().yalm_session_generate(self.h, prompt.ctypes.data_as(_ip), prompt.size, n_steps,
                                                    temperature, int(device_argmax), int(prefill), int(stop_at_eos),
                                                    toks.ctypes.data_as(_ip), secs.ctypes.data_as(_dp),
                                                    ctypes.byref(hyd)))
        return toks[:n], secs[:n], hyd.value

    def active_bytes(self, pos):
        return lib().yalm_session_active_bytes(self.h, pos)

    def close(self):
        if self.h:
            lib().yalm_session_close(self.h)
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
