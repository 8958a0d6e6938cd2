"""Pins the oracle's StreamingLLM ring mode (pos >= max_seq_len) from its definition.

Reference behaviour (src/infer.cpp:307-325 and 489-494): past the context, slots 0 and 1 keep the
first two tokens as attention sinks, the other max_seq_len - 2 slots take new positions in ring
order, and before attending each step re-rotates the sinks' keys by one position, so that after s
wrapped steps sink r sits at angle (r + s) * freq.

Nothing here restates the oracle's in-place update. The checks are built from
  * the pre-RoPE projections of the tokens (layer 0 depends only on the token), rotated in
    float64 to the angle the definition fixes, and
  * npref.NpRingModel, which rebuilds the attended key set at every step from the whole token
    history instead of updating a cache,
and a planted-mistake section shows that the cache check rejects the plausible mistakes (sinks
rotated by the position instead of one step, a skipped step, a ring slot touched, sinks swapped).
"""
import numpy as np
import pytest

from oracle import binding as O
from tests import npref
from tests.util import MICRO, np_tensors, h2f

# One kv head of 16 dims; theta 1e4 so that several rotary pairs turn by a visible angle per step
# (pair 0 by 1 rad, pair 1 by 0.32 rad, ...).
RING = dict(MICRO, n_layers=1, max_seq_len=16, rope_theta=1e4)
HALF_ULP = 2.0 ** -11  # fp16 relative rounding bound


def _k_slots(kcache, cfg, t):
    """Cached K of slot t for every kv head, as a float64 [kv_dim] vector."""
    hd, msl, nkv = cfg["head_dim"], cfg["max_seq_len"], cfg["n_kv_heads"]
    out = np.zeros(nkv * hd)
    for g in range(nkv):
        for j in range(hd):
            out[g * hd + j] = h2f(kcache[g * hd * msl + npref.k_index(j, t, msl)])
    return out


def _v_slots(vcache, cfg, t):
    hd, msl, nkv = cfg["head_dim"], cfg["max_seq_len"], cfg["n_kv_heads"]
    return np.array([h2f(vcache[g * hd * msl + j * msl + t]) for g in range(nkv) for j in range(hd)], np.float64)


def _projections(cfg, t, token):
    """Layer 0's pre-RoPE k and v of a token (float64)."""
    emb = npref.f16_to_f64(t["model.embed.weight"][token])
    xb = npref.rmsnorm(emb, t["model.layers.0.attn.norm.weight"], cfg["norm_eps"])
    k = npref.f16_to_f64(t["model.layers.0.attn.wk.weight"]) @ xb
    v = npref.f16_to_f64(t["model.layers.0.attn.wv.weight"]) @ xb
    return k, v


def _pair_norms(v):
    return np.repeat(np.hypot(v[0::2], v[1::2]), 2)


def check_ring_cache(kcache, vcache, cfg, kpre, vpre, p):
    """Raises AssertionError unless the layer-0 cache after step p holds exactly what the ring
    definition fixes (K within the fp16 roundings the sinks accumulate, the rest within one)."""
    msl = cfg["max_seq_len"]
    f = npref.rope_freqs(cfg["head_dim"], cfg["rotary_dim"], cfg["rope_theta"], cfg["n_kv_heads"] * cfg["head_dim"])
    slot_of = {}
    for tt, mult in npref.ring_keys(p, msl):
        slot = tt if tt < 2 or p < msl else 2 + (tt - 2) % (msl - 2)
        slot_of[slot] = (tt, mult)
    assert sorted(slot_of) == list(range(min(p + 1, msl)))
    s = max(0, p - msl + 1)
    for slot, (tt, mult) in slot_of.items():
        want = npref.rotate(kpre[tt], mult * f)
        got = _k_slots(kcache, cfg, slot)
        # each fp16 store moves a pair by at most sqrt(2) half-ulps of its norm; the rotations
        # between stores keep the norm, so a sink carries at most s + 1 of them
        n_round = (s + 1) if (tt < 2 and p >= msl) else 1
        bound = n_round * 1.5 * HALF_ULP * _pair_norms(want) + 1e-6
        err = np.abs(got - want)
        assert np.all(err <= bound), (p, slot, tt, float(np.max(err / bound)))
        vw = vpre[tt]
        assert np.all(np.abs(_v_slots(vcache, cfg, slot) - vw) <= 2 * HALF_ULP * np.abs(vw) + 1e-6), (p, slot)


def _run_oracle(cfg, tensors, tokens, on_step):
    om = O.OracleModel(cfg, tensors)
    try:
        for p, tok in enumerate(tokens):
            lg = om.forward(int(tok), p)
            on_step(p, om, lg)
    finally:
        om.close()


def test_ring_cache_follows_the_sink_definition():
    cfg = dict(RING)
    t = np_tensors(cfg, seed=31, std=0.1)
    rng = np.random.default_rng(32)
    tokens = rng.integers(0, cfg["vocab_size"], 3 * cfg["max_seq_len"] + 5)
    kpre, vpre = zip(*[_projections(cfg, t, int(tok)) for tok in tokens])
    checked = []

    def step(p, om, _):
        if p >= cfg["max_seq_len"] - 2:
            k, v = om.kv(0)
            check_ring_cache(k, v, cfg, kpre, vpre, p)
            checked.append(p)

    _run_oracle(cfg, t, tokens, step)
    assert len(checked) > 2 * cfg["max_seq_len"]


def test_ring_logits_match_float64_ring_model():
    # two layers: layer 1's keys depend on layer 0's ring attention, so a wrong key set anywhere
    # changes the logits
    cfg = dict(RING, n_layers=2, n_kv_heads=2, n_heads=4)
    t = np_tensors(cfg, seed=33, std=0.1)
    rng = np.random.default_rng(34)
    tokens = rng.integers(0, cfg["vocab_size"], 2 * cfg["max_seq_len"] + 7)
    ref = npref.NpRingModel(cfg, t)
    worst = []

    def step(p, om, lg):
        want = ref.forward(int(tokens[p]), p)
        worst.append(npref.rel_l2(lg, want))

    _run_oracle(cfg, t, tokens, step)
    worst = np.array(worst)
    msl = cfg["max_seq_len"]
    # past the context the sinks carry one extra fp16 rounding per step
    assert np.max(worst[:msl]) < 1e-4
    assert np.max(worst[msl:]) < 2e-3
    # and a model that attends over the plain last max_seq_len positions (no sinks) is far off, so
    # the comparison has teeth
    orig = npref.ring_keys
    om = O.OracleModel(cfg, t)
    alt = npref.NpRingModel(cfg, t)
    try:
        npref.ring_keys = lambda p, m, sinks=2: [(tt, tt) for tt in range(max(0, p - m + 1), p + 1)]
        diffs = [npref.rel_l2(om.forward(int(tok), p), alt.forward(int(tok), p)) for p, tok in enumerate(tokens)]
    finally:
        npref.ring_keys = orig
        om.close()
    assert max(diffs[msl + 2:]) > 50 * np.max(worst[msl:])


# ---- planted mistakes: the cache check must reject each one -----------------------------------
def _rotate_slot(kcache, cfg, slot, angles):
    """A copy of the K cache with slot `slot` of every kv head rotated by `angles` (per pair)."""
    k = kcache.copy()
    hd, msl, nkv = cfg["head_dim"], cfg["max_seq_len"], cfg["n_kv_heads"]
    cur = _k_slots(k, cfg, slot)
    new = npref.rotate(cur, angles)
    for g in range(nkv):
        for j in range(hd):
            k[g * hd * msl + npref.k_index(j, slot, msl)] = np.float16(new[g * hd + j]).view(np.uint16)
    return k


@pytest.mark.parametrize("mistake", ["rotate_by_pos", "skipped_step", "extra_step", "ring_slot_touched",
                                     "sinks_swapped"])
def test_ring_cache_check_rejects_planted_mistakes(mistake):
    cfg = dict(RING)
    t = np_tensors(cfg, seed=31, std=0.1)
    rng = np.random.default_rng(35)
    msl = cfg["max_seq_len"]
    p_last = msl + 9
    tokens = rng.integers(0, cfg["vocab_size"], p_last + 1)
    kpre, vpre = zip(*[_projections(cfg, t, int(tok)) for tok in tokens])
    f = npref.rope_freqs(cfg["head_dim"], cfg["rotary_dim"], cfg["rope_theta"], cfg["n_kv_heads"] * cfg["head_dim"])
    state = {}

    def step(p, om, _):
        if p == p_last:
            state["kv"] = om.kv(0)

    _run_oracle(cfg, t, tokens, step)
    k, v = state["kv"]
    check_ring_cache(k, v, cfg, kpre, vpre, p_last)  # the oracle itself passes
    if mistake == "rotate_by_pos":  # the last step rotated the sinks by p instead of 1
        bad = k
        for r in (0, 1):
            bad = _rotate_slot(bad, cfg, r, (p_last - 1) * f)
    elif mistake == "skipped_step":
        bad = _rotate_slot(_rotate_slot(k, cfg, 0, -f), cfg, 1, -f)
    elif mistake == "extra_step":
        bad = _rotate_slot(k, cfg, 1, f)
    elif mistake == "ring_slot_touched":  # the re-rotation also hit the slot just written
        kv_pos = 2 + (p_last - 2) % (msl - 2)
        bad = _rotate_slot(k, cfg, kv_pos, f)
    else:
        bad = k.copy()
        hd = cfg["head_dim"]
        for g in range(cfg["n_kv_heads"]):
            for j in range(hd):
                i0 = g * hd * msl + npref.k_index(j, 0, msl)
                i1 = g * hd * msl + npref.k_index(j, 1, msl)
                bad[i0], bad[i1] = k[i1], k[i0]
    with pytest.raises(AssertionError):
        check_ring_cache(bad, v, cfg, kpre, vpre, p_last)
