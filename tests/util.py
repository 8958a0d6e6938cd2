"""Shared helpers for the test suite: small model configs and seeded NumPy weights."""
from __future__ import annotations

import numpy as np

# A very small Mistral-style model used by the oracle and kernel tests.
MICRO = dict(dim=64, hidden_dim=128, head_dim=16, n_layers=2, n_heads=4, n_kv_heads=2, vocab_size=512,
             max_seq_len=64, rotary_dim=16, rope_theta=1e6, norm_eps=1e-5, qkv_clip=3.4028234663852886e38, act=1)

# The tiny Mistral-architecture model run on the CPU path (dim 256, hidden 768, 4 layers, 8/2 heads).
TINY = dict(dim=256, hidden_dim=768, head_dim=32, n_layers=4, n_heads=8, n_kv_heads=2, vocab_size=32000,
            max_seq_len=512, rotary_dim=32, rope_theta=1e6, norm_eps=1e-5, qkv_clip=3.4028234663852886e38, act=1)


def np_tensors(cfg, seed=0, std=0.02, gain=1.0):
    """Seeded N(0, std) fp16 weights (as uint16 bit patterns) and fp32 gains, keyed like a .yalm file."""
    rng = np.random.default_rng(seed)
    d, hd, nh, nkv, hid, V = (cfg["dim"], cfg["head_dim"], cfg["n_heads"], cfg["n_kv_heads"], cfg["hidden_dim"],
                              cfg["vocab_size"])

    def w(*shape):
        return (rng.standard_normal(shape, dtype=np.float32) * std).astype(np.float16).view(np.uint16)

    def gvec():
        if gain == "random":
            return (1.0 + 0.1 * rng.standard_normal(d)).astype(np.float32)
        return np.full(d, gain, np.float32)

    t = {"model.embed.weight": w(V, d)}
    for i in range(cfg["n_layers"]):
        p = f"model.layers.{i}."
        t[p + "attn.norm.weight"] = gvec()
        t[p + "mlp.norm.weight"] = gvec()
        t[p + "attn.wq.weight"] = w(nh * hd, d)
        t[p + "attn.wk.weight"] = w(nkv * hd, d)
        t[p + "attn.wv.weight"] = w(nkv * hd, d)
        t[p + "attn.wo.weight"] = w(d, nh * hd)
        t[p + "mlp.w1.weight"] = w(hid, d)
        t[p + "mlp.w2.weight"] = w(d, hid)
        t[p + "mlp.w3.weight"] = w(hid, d)
    t["model.norm.weight"] = gvec()
    t["model.output.weight"] = w(V, d)
    return t


def f16(a):
    """float array -> fp16 bit patterns (RNE)."""
    return np.asarray(a, np.float32).astype(np.float16).view(np.uint16)


def h2f(bits):
    return np.asarray(bits, np.uint16).view(np.float16).astype(np.float32)
