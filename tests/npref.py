"""Float64 NumPy brute-force model of the decode step, written from the mathematics.

It is the independent check of the C++ oracle: every quantity is computed in float64 except
where the reference defines the arithmetic itself (RoPE frequencies and angles are fp32,
infer.cpp:205-206; cached K/V are rounded to fp16, infer.cpp:300-305). It deliberately shares
no code with oracle/oracle.cpp.
"""
from __future__ import annotations

import numpy as np


def f16_to_f64(a):
    a = np.asarray(a)
    if a.dtype == np.uint16:
        a = a.view(np.float16)
    return a.astype(np.float64)


def rmsnorm(x, g, eps):
    x = np.asarray(x, np.float64)
    return x / np.sqrt(np.mean(x * x) + eps) * np.asarray(g, np.float64)


def softmax(s):
    s = np.asarray(s, np.float64)
    e = np.exp(s - s.max())
    return e / e.sum()


def silu(x):
    return x / (1.0 + np.exp(-x))


def gelu(x):
    return 0.5 * x * (1.0 + np.tanh(0.797885 * (x + 0.044715 * x ** 3)))


def rope_angles(n, head_dim, pos, theta, rotary_dim):
    """fp32 angle per pair, as the reference defines it."""
    j = (np.arange(0, n, 2) % head_dim).astype(np.float32)
    freq = np.where(j >= rotary_dim, np.float32(0.0),
                    np.float32(1.0) / np.power(np.float32(theta), j / np.float32(rotary_dim), dtype=np.float32))
    return (np.float32(pos) * freq.astype(np.float32)).astype(np.float32).astype(np.float64)


def rope(v, head_dim, pos, theta, rotary_dim):
    v = np.asarray(v, np.float64).copy()
    a = rope_angles(v.size, head_dim, pos, theta, rotary_dim)
    c, s = np.cos(a), np.sin(a)
    x0, x1 = v[0::2].copy(), v[1::2].copy()
    v[0::2] = x0 * c - x1 * s
    v[1::2] = x0 * s + x1 * c
    return v


def k_index(j, t, msl):
    return (j // 16) * 16 * msl + t * 16 + j % 16


class NpModel:
    """Float64 model with fp16 KV caches in the reference layout."""

    def __init__(self, cfg, tensors):
        self.c = cfg
        get = (lambda k: cfg[k]) if isinstance(cfg, dict) else (lambda k: getattr(cfg, k))
        self.g = get
        self.t = {k: (f16_to_f64(v) if np.asarray(v).dtype in (np.uint16, np.float16) else np.asarray(v, np.float64))
                  for k, v in tensors.items()}
        L, nkv, hd, msl = get("n_layers"), get("n_kv_heads"), get("head_dim"), get("max_seq_len")
        self.k = [np.zeros(nkv * hd * msl, np.float16) for _ in range(L)]
        self.v = [np.zeros(nkv * hd * msl, np.float16) for _ in range(L)]
        self.x = None

    def forward(self, token, pos):
        g, t = self.g, self.t
        dim, hd, nh, nkv = g("dim"), g("head_dim"), g("n_heads"), g("n_kv_heads")
        msl, eps, theta, rd = g("max_seq_len"), g("norm_eps"), g("rope_theta"), g("rotary_dim")
        act = g("act")
        act_fn = silu if act in (1, "silu") else gelu
        clip = float(g("qkv_clip"))
        x = t["model.embed.weight"][token].copy()
        kv_len = pos + 1
        assert pos < msl
        for layer in range(g("n_layers")):
            p = f"model.layers.{layer}."
            xb = rmsnorm(x, t[p + "attn.norm.weight"], eps)
            q = np.clip(t[p + "attn.wq.weight"] @ xb, -clip, clip)
            k = np.clip(t[p + "attn.wk.weight"] @ xb, -clip, clip)
            v = np.clip(t[p + "attn.wv.weight"] @ xb, -clip, clip)
            q = rope(q, hd, pos, theta, rd)
            k = rope(k, hd, pos, theta, rd)
            K, V = self.k[layer], self.v[layer]
            for gi in range(nkv):
                for j in range(hd):
                    K[gi * hd * msl + k_index(j, pos, msl)] = np.float16(k[gi * hd + j])
                    V[gi * hd * msl + j * msl + pos] = np.float16(v[gi * hd + j])
            out = np.zeros(nh * hd)
            grp = nh // nkv
            for h in range(nh):
                gi = h // grp
                base = gi * hd * msl
                Kh = np.array([[K[base + k_index(j, tt, msl)] for j in range(hd)] for tt in range(kv_len)], np.float64)
                Vh = np.array([[V[base + j * msl + tt] for tt in range(kv_len)] for j in range(hd)], np.float64)
                a = softmax(Kh @ q[h * hd:(h + 1) * hd] / np.sqrt(hd))
                out[h * hd:(h + 1) * hd] = Vh @ a
            x = x + t[p + "attn.wo.weight"] @ out
            xb = rmsnorm(x, t[p + "mlp.norm.weight"], eps)
            hb = act_fn(t[p + "mlp.w1.weight"] @ xb) * (t[p + "mlp.w3.weight"] @ xb)
            x = x + t[p + "mlp.w2.weight"] @ hb
        self.x = x
        xf = rmsnorm(x, t["model.norm.weight"], eps)
        wcls = t.get("model.output.weight", t["model.embed.weight"])
        return wcls @ xf


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


# ---- StreamingLLM ring mode (pos >= max_seq_len), written from its definition ------------------
# When decoding past the context, two "sink" tokens stay in the cache and the other max_seq_len - 2
# slots hold the most recent positions in ring order (reference src/infer.cpp:307-325, 489-494).
# Sink r must keep a fixed distance from the current position, so after s wrapped steps its key is
# the position-r projection rotated to angle (r + s) * freq. This model builds that key set
# directly from the pre-RoPE projections of every past token, with one fp16 rounding per cached
# value, instead of updating a cache in place: it shares neither code nor mechanism with the oracle.
def rope_freqs(head_dim, rotary_dim, theta, n):
    """fp32 frequency of every rotary pair of an n-vector (0 past rotary_dim), as float64."""
    j = (np.arange(0, n, 2) % head_dim).astype(np.float32)
    f = np.where(j >= rotary_dim, np.float32(0.0),
                 np.float32(1.0) / np.power(np.float32(theta), j / np.float32(rotary_dim), dtype=np.float32))
    return f.astype(np.float32).astype(np.float64)


def rotate(v, angles):
    """Rotate the pairs (v[2i], v[2i+1]) by angles[i] (float64)."""
    v = np.asarray(v, np.float64).copy()
    c, s = np.cos(angles), np.sin(angles)
    x0, x1 = v[0::2].copy(), v[1::2].copy()
    v[0::2] = x0 * c - x1 * s
    v[1::2] = x0 * s + x1 * c
    return v


def ring_keys(p, msl, sinks=2):
    """Which past positions the cache holds at step p, and the angle multiplier of each key."""
    if p < msl:
        return [(t, t) for t in range(p + 1)]
    s = p - msl + 1
    return [(r, r + s) for r in range(sinks)] + [(t, t) for t in range(p - (msl - sinks) + 1, p + 1)]


class NpRingModel:
    """Float64 model over an unbounded token history; attention at step p runs over ring_keys(p)."""

    def __init__(self, cfg, tensors):
        self.base = NpModel(cfg, tensors)
        self.hist = [[] for _ in range(cfg["n_layers"])]  # per layer: (k before RoPE, v) per position

    def forward(self, token, pos):
        b = self.base
        g, t = b.g, b.t
        dim, hd, nh, nkv = g("dim"), g("head_dim"), g("n_heads"), g("n_kv_heads")
        msl, eps, theta, rd = g("max_seq_len"), g("norm_eps"), g("rope_theta"), g("rotary_dim")
        act_fn = silu if g("act") in (1, "silu") else gelu
        clip = float(g("qkv_clip"))
        x = t["model.embed.weight"][token].copy()
        fk = rope_freqs(hd, rd, theta, nkv * hd)
        fq = rope_freqs(hd, rd, theta, nh * hd)
        assert len(self.hist[0]) == pos, "positions must be fed in order"
        keys = ring_keys(pos, msl)
        for layer in range(g("n_layers")):
            p = f"model.layers.{layer}."
            xb = rmsnorm(x, t[p + "attn.norm.weight"], eps)
            q = np.clip(t[p + "attn.wq.weight"] @ xb, -clip, clip)
            k = np.clip(t[p + "attn.wk.weight"] @ xb, -clip, clip)
            v = np.clip(t[p + "attn.wv.weight"] @ xb, -clip, clip)
            self.hist[layer].append((k, v))
            q = rotate(q, np.float32(pos) * fq.astype(np.float32))
            Kc = np.stack([np.float16(rotate(self.hist[layer][tt][0], mult * fk)).astype(np.float64)
                           for tt, mult in keys])        # [n_keys][kv_dim]
            Vc = np.stack([np.float16(self.hist[layer][tt][1]).astype(np.float64) for tt, _ in keys])
            out = np.zeros(nh * hd)
            grp = nh // nkv
            for h in range(nh):
                gi = h // grp
                a = softmax(Kc[:, gi * hd:(gi + 1) * hd] @ q[h * hd:(h + 1) * hd] / np.sqrt(hd))
                out[h * hd:(h + 1) * hd] = a @ Vc[:, gi * hd:(gi + 1) * hd]
            x = x + t[p + "attn.wo.weight"] @ out
            xb = rmsnorm(x, t[p + "mlp.norm.weight"], eps)
            hb = act_fn(t[p + "mlp.w1.weight"] @ xb) * (t[p + "mlp.w3.weight"] @ xb)
            x = x + t[p + "mlp.w2.weight"] @ hb
        xf = rmsnorm(x, t["model.norm.weight"], eps)
        wcls = t.get("model.output.weight", t["model.embed.weight"])
        return wcls @ xf
