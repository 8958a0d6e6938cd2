"""Pins the CPU oracle against known answers, closed forms and a float64 brute-force model.

Nothing here retypes the oracle's formulas: each check is either a value the reference's own
tests hold (src/test.cpp:67-125), a property the mathematics fixes, or the independent float64
model in npref.py.
"""
import numpy as np
import pytest

from oracle import binding as O
from tests import npref
from tests.util import MICRO, np_tensors, f16, h2f


# ---- fp16 conversion (infer.cpp:10-16) -------------------------------------------------------
def test_h2f_all_bit_patterns():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = O.h2f(bits)
    want = bits.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_f2h_round_to_nearest_even():
    rng = np.random.default_rng(1)
    vals = np.concatenate([
        rng.standard_normal(100000).astype(np.float32) * 10,
        rng.standard_normal(1000).astype(np.float32) * 1e-6,   # subnormals
        np.array([65504, 65519.99, 0.0, -0.0], np.float32),
        # exact halfway points between fp16 neighbours: ties must go to even
        (np.arange(1024, 2048, dtype=np.float32) + 0.5) * np.float32(2.0 ** -10),
    ])
    got = O.f2h(vals)
    want = vals.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)


# ---- matvec (infer.cpp:63-100) --------------------------------------------------------------
def test_matmul_one_hot_returns_column_exactly():
    rng = np.random.default_rng(2)
    w = f16(rng.standard_normal((48, 64)))
    for j in (0, 7, 63):
        x = np.zeros(64, np.float32)
        x[j] = 1.0
        assert np.array_equal(O.matmul_f16(x, w), h2f(w[:, j]))


def test_matmul_matches_float64():
    rng = np.random.default_rng(3)
    for d, n in ((32, 16), (100, 256), (384, 4096)):
        w = f16(rng.standard_normal((d, n)) * 0.02)
        x = rng.standard_normal(n).astype(np.float32)
        ref = h2f(w).astype(np.float64) @ x.astype(np.float64)
        got = O.matmul_f16(x, w)
        assert npref.rel_l2(got, ref) < 1e-5
        wf = rng.standard_normal((d, n)).astype(np.float32)
        assert npref.rel_l2(O.matmul_f32(x, wf), wf.astype(np.float64) @ x) < 1e-5


def test_matmul_rejects_n_not_multiple_of_16():
    # infer.cpp:66 asserts n % 16 == 0; the oracle aborts rather than read past the row.
    import subprocess
    import sys
    code = ("from oracle import binding as O; import numpy as np; "
            "O.matmul_f16(np.ones(8, np.float32), np.zeros((2, 8), np.uint16))")
    r = subprocess.run([sys.executable, "-c", code], cwd=npref.__file__.rsplit("/tests/", 1)[0],
                       capture_output=True, timeout=120)
    assert r.returncode != 0


# ---- rmsnorm / softmax / activations ----------------------------------------------------------
def test_rmsnorm_constant_vector_closed_form():
    for c in (0.5, -3.0, 1e-3):
        x = np.full(256, c, np.float32)
        got = O.rmsnorm(x, np.ones(256, np.float32), 1e-5)
        want = np.sign(c) / np.sqrt(1.0 + 1e-5 / (c * c))
        assert np.allclose(got, want, rtol=1e-6, atol=0)


def test_rmsnorm_matches_float64():
    rng = np.random.default_rng(4)
    x = rng.standard_normal(4096).astype(np.float32)
    g = (1 + 0.1 * rng.standard_normal(4096)).astype(np.float32)
    assert npref.rel_l2(O.rmsnorm(x, g, 1e-5), npref.rmsnorm(x, g, 1e-5)) < 1e-6


def test_softmax_properties():
    rng = np.random.default_rng(5)
    s = rng.standard_normal(1000).astype(np.float32) * 5
    p = O.softmax(s)
    assert abs(p.sum() - 1.0) < 1e-5
    assert npref.rel_l2(p, npref.softmax(s)) < 1e-5
    assert npref.rel_l2(O.softmax(s + 100.0), p) < 1e-5  # shift invariance (max subtraction)


def test_activations_match_textbook():
    for x in np.linspace(-20, 20, 81, dtype=np.float32):
        assert abs(O.lib().oracle_silu(float(x)) - npref.silu(float(x))) <= 1e-6 * max(1, abs(x))
        assert abs(O.lib().oracle_gelu(float(x)) - npref.gelu(float(x))) <= 1e-5 * max(1, abs(x))


# ---- RoPE (infer.cpp:202-215) -----------------------------------------------------------------
def test_rope_identity_at_pos0():
    rng = np.random.default_rng(6)
    v = rng.standard_normal(256).astype(np.float32)
    assert np.array_equal(O.rope(v, 32, 0, 1e6, 32), v)


def test_rope_preserves_pair_norm_and_composes():
    rng = np.random.default_rng(7)
    v = rng.standard_normal(128).astype(np.float32)
    r = O.rope(v, 128, 37, 1e6, 128)
    n0 = v[0::2] ** 2 + v[1::2] ** 2
    n1 = r[0::2] ** 2 + r[1::2] ** 2
    assert np.allclose(n0, n1, rtol=1e-5)
    # RoPE(a) then RoPE(b) equals RoPE(a+b) up to fp32 angle rounding
    ab = O.rope(O.rope(v, 128, 5, 1e6, 128), 128, 9, 1e6, 128)
    assert npref.rel_l2(ab, O.rope(v, 128, 14, 1e6, 128)) < 1e-5


def test_rope_matches_float64_and_partial_rotary():
    rng = np.random.default_rng(8)
    v = rng.standard_normal(256).astype(np.float32)
    # The fp32 frequency may differ by an ulp between libm builds (the reference is built with
    # -ffast-math); the angle error is then about pos * 2^-22, so the bound grows with pos.
    for pos in (1, 100, 4095, 16447):
        tol = 1e-5 + 3e-7 * pos
        assert npref.rel_l2(O.rope(v, 128, pos, 1e6, 128), npref.rope(v, 128, pos, 1e6, 128)) < tol
    # rotary_dim < head_dim leaves the tail of each head untouched (freq = 0)
    r = O.rope(v, 128, 77, 1e4, 64)
    assert np.array_equal(r[64:128], v[64:128]) and np.array_equal(r[192:], v[192:])


# ---- KV layout and positions (model.h:12-17, infer.cpp:489-494) -------------------------------
def test_k_cache_idx_is_a_bijection_in_16_tiles():
    msl, hd = 40, 128
    seen = set()
    for t in range(msl):
        for j in range(hd):
            idx = O.k_cache_idx(j, t, msl)
            assert idx == (j // 16) * 16 * msl + t * 16 + (j % 16)
            seen.add(idx)
    assert seen == set(range(msl * hd))


def test_positions():
    msl = 8
    for pos in range(40):
        sink, kv_pos, kv_len = O.positions(pos, msl)
        if pos < msl:
            assert (sink, kv_pos, kv_len) == (0, pos, pos + 1)
        else:
            assert sink == 2 and kv_len == msl
            assert 2 <= kv_pos < msl and kv_pos == 2 + (pos - 2) % (msl - 2)


# ---- attention (infer.cpp:218-250; known answer test.cpp:67-125) ------------------------------
def test_attn_reference_known_answer():
    seq, hd = 4, 3
    q = np.array([0., 1e4, 0., 0., 0., 1e4], np.float32)
    kb = np.zeros(16 * seq, np.uint16)
    kb[0] = f16([1.0])[0]
    kb[17] = f16([1.0])[0]
    kb[34] = f16([1.0])[0]
    kb[48] = f16([-1.0])[0]
    vb = f16([1., 0., 0., -1., 0., 1., 0., 0., 0., 0., 1., 0.])
    out, att = O.mha(q, kb, vb, hd, seq, seq, 2, 1)
    assert np.allclose(att[0], [0, 1, 0, 0], atol=1e-4)
    assert np.allclose(att[1], [0, 0, 1, 0], atol=1e-4)
    assert np.allclose(out, [0, 1, 0, 0, 0, 1], atol=1e-4)


def test_attn_kv_len_one_returns_v0():
    rng = np.random.default_rng(9)
    hd, msl = 32, 16
    kh = f16(rng.standard_normal(hd * msl))
    vh = f16(rng.standard_normal(hd * msl))
    out, att = O.attn(rng.standard_normal(hd).astype(np.float32), kh, vh, hd, msl, 1)
    assert att[0] == 1.0
    assert np.array_equal(out, h2f(vh.reshape(hd, msl)[:, 0]))


def test_mha_gqa_matches_float64():
    rng = np.random.default_rng(10)
    hd, msl, nh, nkv, kv_len = 32, 48, 8, 2, 37
    kb = f16(rng.standard_normal(nkv * hd * msl))
    vb = f16(rng.standard_normal(nkv * hd * msl))
    q = rng.standard_normal(nh * hd).astype(np.float32)
    out, _ = O.mha(q, kb, vb, hd, kv_len, msl, nh, nkv)
    K, V = h2f(kb).astype(np.float64), h2f(vb).astype(np.float64)
    for h in range(nh):
        g = h // (nh // nkv)
        base = g * hd * msl
        Kh = np.array([[K[base + npref.k_index(j, t, msl)] for j in range(hd)] for t in range(kv_len)])
        Vh = V[base:base + hd * msl].reshape(hd, msl)[:, :kv_len]
        want = Vh @ npref.softmax(Kh @ q[h * hd:(h + 1) * hd] / np.sqrt(hd))
        assert npref.rel_l2(out[h * hd:(h + 1) * hd], want) < 1e-5


def test_ffn_matches_float64():
    rng = np.random.default_rng(11)
    dim, hid = 64, 192
    w1, w2, w3 = (f16(rng.standard_normal(s) / 8) for s in ((hid, dim), (dim, hid), (hid, dim)))
    x = rng.standard_normal(dim).astype(np.float32)
    W1, W2, W3 = (h2f(w).astype(np.float64) for w in (w1, w2, w3))
    for act, fn in ((1, npref.silu), (0, npref.gelu)):
        want = W2 @ (fn(W1 @ x) * (W3 @ x))
        assert npref.rel_l2(O.ffn(x, w1, w2, w3, act), want) < 1e-5


# ---- sampler (sampler.cpp:27-38) --------------------------------------------------------------
def test_argmax_first_index_tie_rule():
    assert O.argmax(np.array([1., 3., 3., 2.], np.float32)) == 1
    assert O.argmax(np.array([-5., -5.], np.float32)) == 0
    assert O.argmax(np.array([0., 0., 7.], np.float32)) == 2


# ---- whole forward (infer.cpp:256-392, 460-527) vs the float64 brute-force model ---------------
@pytest.mark.parametrize("gain", [1.0, "random"])
def test_forward_matches_float64_model(gain):
    cfg = dict(MICRO)
    t = np_tensors(cfg, seed=12, std=0.1, gain=gain)
    om = O.OracleModel(cfg, t)
    nm = npref.NpModel(cfg, t)
    toks = [3, 17, 400, 5, 99, 250]
    for pos, tok in enumerate(toks):
        lo = om.forward(tok, pos)
        ln = nm.forward(tok, pos)
        assert npref.rel_l2(lo, ln) < 1e-4, pos
    for layer in range(cfg["n_layers"]):
        k, v = om.kv(layer)
        # fp16 stores of nearly equal fp32/fp64 values: at most one ulp apart
        for a, b in ((k, nm.k[layer].view(np.uint16)), (v, nm.v[layer].view(np.uint16))):
            fa, fb = h2f(a), h2f(b)
            assert np.all(np.abs(fa - fb) <= np.abs(fb) * 2e-3 + 1e-6)
            assert np.array_equal(a != 0, b != 0) or np.all(np.abs(fa - fb) < 1e-6)


def test_forward_tied_lm_head_reads_the_embedding():
    # Without model.output.weight the logits come from the embedding table (reference
    # src/model.cpp:425-434): equal bit for bit to the same model with the embedding passed as an
    # explicit output matrix, and within 1e-4 of the float64 model
    cfg = dict(MICRO)
    t = np_tensors(cfg, seed=13, std=0.1)
    t.pop("model.output.weight", None)
    explicit = dict(t, **{"model.output.weight": t["model.embed.weight"].copy()})
    om, oe, nm = O.OracleModel(cfg, t), O.OracleModel(cfg, explicit), npref.NpModel(cfg, t)
    for pos, tok in enumerate([7, 300, 41, 2]):
        lo = om.forward(tok, pos)
        assert np.array_equal(lo, oe.forward(tok, pos)), pos
        assert npref.rel_l2(lo, nm.forward(tok, pos)) < 1e-4, pos
    om.close()
    oe.close()


def test_forward_hydrate_mode_writes_kv_only():
    cfg = dict(MICRO)
    t = np_tensors(cfg, seed=13, std=0.1)
    a = O.OracleModel(cfg, t)
    b = O.OracleModel(cfg, t)
    a.forward(5, 0, mode=0)
    b.forward(5, 0, mode=1)
    for layer in range(cfg["n_layers"]):
        assert all(np.array_equal(x, y) for x, y in zip(a.kv(layer), b.kv(layer)))
    assert np.array_equal(a.forward(9, 1), b.forward(9, 1))


def test_forward_kv_write_lands_at_reference_index_pos0():
    # At pos 0 RoPE is the identity, so K/V are exactly the fp16 of the clipped projections.
    cfg = dict(MICRO)
    t = np_tensors(cfg, seed=14, std=0.1)
    om = O.OracleModel(cfg, t)
    om.forward(11, 0, mode=0)
    x = h2f(t["model.embed.weight"][11])
    xb = O.rmsnorm(x, t["model.layers.0.attn.norm.weight"], cfg["norm_eps"])
    k = O.matmul_f16(xb, t["model.layers.0.attn.wk.weight"])
    v = O.matmul_f16(xb, t["model.layers.0.attn.wv.weight"])
    K, V = om.kv(0)
    hd, msl = cfg["head_dim"], cfg["max_seq_len"]
    for i in range(k.size):
        g, j = divmod(i, hd)
        assert K[g * hd * msl + npref.k_index(j, 0, msl)] == f16([k[i]])[0]
        assert V[g * hd * msl + j * msl + 0] == f16([v[i]])[0]
    assert np.count_nonzero(K) <= k.size and np.count_nonzero(V) <= v.size


def test_forward_rejects_bad_token():
    cfg = dict(MICRO)
    om = O.OracleModel(cfg, np_tensors(cfg, seed=15))
    with pytest.raises(ValueError):
        om.forward(cfg["vocab_size"], 0)


def test_rope_frequency_hook_zero_frequencies_equal_no_rotation():
    # oracle_set_rope_freqs (the test hook that lets the oracle rotate with a given frequency table):
    # all-zero frequencies make every rotation the identity, as rotary_dim 0 does through the
    # reference's own expression (src/infer.cpp:205: freq = 0 for j >= rotary_dim); setting no table
    # restores the reference's expression.
    from tests.util import MICRO, np_tensors
    cfg = dict(MICRO)
    t = np_tensors(cfg, seed=91)
    m = O.OracleModel(cfg, t)
    m.set_rope_freqs(np.zeros(cfg["head_dim"] // 2, np.float32))
    norot = O.OracleModel(dict(cfg, rotary_dim=0), t)
    plain = O.OracleModel(cfg, t)
    for pos, tok in enumerate((3, 77, 5, 300)):
        assert np.array_equal(m.forward(tok, pos), norot.forward(tok, pos))
    m2 = O.OracleModel(cfg, t)
    m2.set_rope_freqs(np.zeros(cfg["head_dim"] // 2, np.float32))
    m2.set_rope_freqs(None)
    for pos, tok in enumerate((3, 77, 5, 300)):
        assert np.array_equal(m2.forward(tok, pos), plain.forward(tok, pos))
    with pytest.raises(ValueError):
        m.set_rope_freqs(np.zeros(3, np.float32))
