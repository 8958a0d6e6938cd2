"""Writes the golden fixtures of the decode path from the float64 brute-force model (tests/npref.py).

micro.npz -- the 2-layer dim-64 model of tests/util.py (seeded NumPy weights, std 0.2, norm gains
  1 + N(0, 0.1)): the float64 logits of 8 steps fed a fixed token list, both layers' fp16 K/V caches
  after them, and a 24-token greedy continuation of a 4-token prompt (fresh caches) with the top-2
  logit margin of every step.
tiny.npz -- the dim-256, 4-layer, 32000-vocab model made by the host's synthetic generator (seed
  0x59414C4D, N(0, 0.02), context 512): 16 prompt ids (uniform, seed 16), the logits of positions 0-3
  (stored as fp16), the written part of layer 0's K/V after the whole run, and the 32 greedy tokens
  that follow the prompt with their margins.

The greedy rule is the first index of the maximum (reference src/sampler.cpp:27-38); prompt tokens are
fed one at a time as the reference's hydrate does (src/main.cpp:169-177). Each file keeps a SHA-256 of
the weight bytes, so a change of a weight generator shows up as a fixture mismatch instead of a parity
failure.

Run from the repository root once the host library is built (a few seconds):
    python tests/golden/make_golden.py
"""
from __future__ import annotations

import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

from tests import npref  # noqa: E402
from tests.util import MICRO, np_tensors  # noqa: E402

MICRO_SEED, MICRO_STD, MICRO_GAIN = 41, 0.2, "random"
MICRO_STEPS = [7, 300, 511, 0, 42, 42, 129, 5]
MICRO_PROMPT = [3, 99, 250, 17]
MICRO_GEN = 24
TINY_PROMPT_SEED, TINY_PROMPT_LEN, TINY_GEN, TINY_CTX = 16, 16, 32, 512
TINY_SHAPE = dict(dim=256, hidden_dim=768, head_dim=32, n_layers=4, n_heads=8, n_kv_heads=2, vocab_size=32000,
                  max_seq_len=512)
TINY_LOGIT_POSITIONS = 4


def weights_digest(tensors):
    h = hashlib.sha256()
    for name in sorted(tensors):
        h.update(name.encode())
        h.update(np.ascontiguousarray(tensors[name]).tobytes())
    return h.hexdigest()


def argmax_first(v):
    return int(np.flatnonzero(v == v.max())[0])


def margin(v):
    s = np.sort(v)
    return float(s[-1] - s[-2])


def greedy(model, prompt, n_gen):
    lg = None
    for pos, tok in enumerate(prompt):
        lg = model.forward(int(tok), pos)
    out, margins = [], []
    pos = len(prompt)
    for _ in range(n_gen):
        nxt = argmax_first(lg)
        out.append(nxt)
        margins.append(margin(lg))
        lg = model.forward(nxt, pos)
        pos += 1
    return np.array(out, np.int32), np.array(margins, np.float64)


def micro_fixture():
    cfg = dict(MICRO)
    t = np_tensors(cfg, seed=MICRO_SEED, std=MICRO_STD, gain=MICRO_GAIN)
    m = npref.NpModel(cfg, t)
    logits = np.stack([m.forward(tok, pos) for pos, tok in enumerate(MICRO_STEPS)])
    k = np.stack([kk.view(np.uint16) for kk in m.k])
    v = np.stack([vv.view(np.uint16) for vv in m.v])
    gen, margins = greedy(npref.NpModel(cfg, t), MICRO_PROMPT, MICRO_GEN)
    return dict(seed=MICRO_SEED, std=MICRO_STD, digest=weights_digest(t), steps=np.array(MICRO_STEPS, np.int32),
                logits=logits, k=k, v=v, prompt=np.array(MICRO_PROMPT, np.int32), greedy=gen, margins=margins)


def tiny_session():
    from yalm_amd import host
    return host.Session.synthetic(dict(TINY_SHAPE), context=TINY_CTX)


def tiny_fixture():
    from yalm_amd import host
    sess = tiny_session()
    cfg = sess.config()
    t = {k: np.array(v) for k, v in sess.tensors().items()}
    sess.close()
    prompt = host.uniform_ids(TINY_PROMPT_LEN, TINY_PROMPT_SEED, cfg["vocab_size"])
    m = npref.NpModel(dict(cfg, act=1), t)
    logits = []
    lg = None
    for pos, tok in enumerate(prompt):
        lg = m.forward(int(tok), pos)
        if pos < TINY_LOGIT_POSITIONS:
            logits.append(lg)
    out, margins = [], []
    pos = len(prompt)
    for _ in range(TINY_GEN):
        nxt = argmax_first(lg)
        out.append(nxt)
        margins.append(margin(lg))
        lg = m.forward(nxt, pos)
        pos += 1
    n_written = pos
    hd, msl, nkv = cfg["head_dim"], cfg["max_seq_len"], cfg["n_kv_heads"]
    K = m.k[0].view(np.uint16).reshape(nkv, hd // 16, msl, 16)[:, :, :n_written, :]
    V = m.v[0].view(np.uint16).reshape(nkv, hd, msl)[:, :, :n_written]
    return dict(digest=weights_digest(t), prompt=prompt.astype(np.int32),
                logits=np.stack(logits).astype(np.float16), greedy=np.array(out, np.int32),
                margins=np.array(margins, np.float64), k0=np.ascontiguousarray(K), v0=np.ascontiguousarray(V),
                n_written=n_written)


def main():
    np.savez_compressed(os.path.join(HERE, "micro.npz"), **micro_fixture())
    np.savez_compressed(os.path.join(HERE, "tiny.npz"), **tiny_fixture())
    for f in ("micro.npz", "tiny.npz"):
        print(f, os.path.getsize(os.path.join(HERE, f)), "bytes")


if __name__ == "__main__":
    main()
