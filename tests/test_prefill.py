"""Batched prefill (MFMA GEMMs + causal MFMA attention) against the reference's sequential hydrate.

The reference has no batched prefill: a prompt goes through forward() one token at a time
(src/main.cpp:169-177). Prefill must leave the same K/V cache entries (indices exact, values within
fp16-activation tolerance) and the same last-token logits (rel-L2 <= 1e-2, the decode contract).
Activations enter the matrix cores as fp16, so the values differ from the fp32 oracle by about the
fp16 rounding of an activation (~1e-3 relative)."""
import numpy as np
import pytest

from oracle import binding as O
from tests import npref
from tests.util import MICRO, TINY, np_tensors, h2f, f16

pytestmark = pytest.mark.gpu

PREFILL_LOGIT_TOL = 1e-2


def hip():
    from yalm_amd import hip as H
    H.lib()
    return H


# (LDS stages, k-step, workgroup rows): -1 = chosen per shape; 2..4 = the LDS pipeline; 6 = the
# eight-wave 256 x 256 kernel (K % 64 == 0; otherwise it falls back to the 32-deep LDS pipeline)
GEMM_VARIANTS = [(-1, 32, 128), (4, 32, 128), (2, 64, 128), (3, 64, 128), (2, 64, 256), (3, 64, 256),
                 (6, 64, 256)]


@pytest.fixture(params=GEMM_VARIANTS, ids=[f"s{s}k{k}m{m}" for s, k, m in GEMM_VARIANTS])
def gemm_variant(request):
    hip().set_gemm_stages(*request.param)
    yield request.param
    hip().set_gemm_stages(-1)


@pytest.mark.parametrize("M,N,K", [(128, 128, 32), (200, 384, 256), (37, 64, 96), (300, 256, 4096),
                                   (130, 128, 448), (520, 256, 128), (70, 200, 64)])
def test_gemm_store_and_residual(M, N, K, gemm_variant):
    H = hip()
    rng = np.random.default_rng(M * 7 + N)
    a = f16(rng.standard_normal((M, K)))
    b = f16(rng.standard_normal((N, K)) * 0.05)
    want = h2f(a).astype(np.float64) @ h2f(b).astype(np.float64).T
    got = H.gemm(a, b, mode=0)
    assert npref.rel_l2(got, want) < 1e-6
    c0 = rng.standard_normal((M, N)).astype(np.float32)
    got = H.gemm(a, b, mode=1, c=c0)
    assert npref.rel_l2(got, c0 + want) < 1e-6


@pytest.mark.parametrize("M,N,K", [(128, 64, 64), (150, 192, 256), (33, 96, 32)])
def test_gemm_swiglu(M, N, K, gemm_variant):
    H = hip()
    rng = np.random.default_rng(M + N)
    a = f16(rng.standard_normal((M, K)))
    b1 = f16(rng.standard_normal((N, K)) * 0.1)
    b3 = f16(rng.standard_normal((N, K)) * 0.1)
    A = h2f(a).astype(np.float64)
    g = A @ h2f(b1).astype(np.float64).T
    u = A @ h2f(b3).astype(np.float64).T
    want = g / (1 + np.exp(-g)) * u
    got = h2f(H.gemm(a, b1, mode=2, b3=b3))
    assert npref.rel_l2(got, want) < 2e-3  # fp16 output


@pytest.mark.parametrize("ksplit", [2, 4, 8])
@pytest.mark.parametrize("M,N,K", [(37, 192, 1024), (128, 256, 4096), (200, 128, 512)])
def test_gemm_split_k(M, N, K, ksplit):
    # K split over workgroups: fp32 partials summed in split order by the reduce kernel, which then
    # applies the epilogue (store, residual add, SwiGLU).
    H = hip()
    rng = np.random.default_rng(M + N + K + ksplit)
    a = f16(rng.standard_normal((M, K)))
    b = f16(rng.standard_normal((N, K)) * 0.05)
    b3 = f16(rng.standard_normal((N, K)) * 0.05)
    A = h2f(a).astype(np.float64)
    want = A @ h2f(b).astype(np.float64).T
    u = A @ h2f(b3).astype(np.float64).T
    c0 = rng.standard_normal((M, N)).astype(np.float32)
    try:
        H.set_gemm_stages(2, 64, 128)
        H.set_gemm_ksplit(ksplit)
        assert npref.rel_l2(H.gemm(a, b, mode=0), want) < 1e-6
        assert npref.rel_l2(H.gemm(a, b, mode=1, c=c0), c0 + want) < 1e-6
        got = h2f(H.gemm(a, b, mode=2, b3=b3))
        assert npref.rel_l2(got, want / (1 + np.exp(-want)) * u) < 2e-3  # fp16 output
    finally:
        H.set_gemm_ksplit(0)
        H.set_gemm_stages(-1)


def test_gemm_split_k_must_divide_the_k_steps():
    H = hip()
    a = f16(np.ones((64, 192)))
    b = f16(np.ones((64, 192)))
    try:
        H.set_gemm_stages(2, 64, 128)
        H.set_gemm_ksplit(2)  # 192 / 64 = 3 k-steps
        with pytest.raises(H.HipError):
            H.gemm(a, b, mode=0)
    finally:
        H.set_gemm_ksplit(0)
        H.set_gemm_stages(-1)


def _sequential(om, toks, start=0):
    for i, t in enumerate(toks):
        lo = om.forward(int(t), start + i, 1 if i == len(toks) - 1 else 0)
    return lo


def _check_kv_close(om, hm, n_layers, positions, k_zero_pattern=True):
    # k_zero_pattern False: keys small enough that fp16 rounds some of them to zero on one side only
    for layer in range(n_layers):
        ko, vo = om.kv(layer)
        kh, vh = hm.kv(layer)
        if k_zero_pattern:
            assert np.array_equal(ko != 0, kh != 0)  # the same entries are written
        assert np.array_equal(vo != 0, vh != 0)
        for a, b in ((kh, ko), (vh, vo)):
            fa, fb = h2f(a), h2f(b)
            assert npref.rel_l2(fa, fb) < 1e-2, layer
            assert np.max(np.abs(fa - fb)) <= 3e-2 * np.max(np.abs(fb)), layer


@pytest.mark.parametrize("cfg_name,n", [("tiny", 40), ("tiny", 97), ("micro", 20)])
def test_prefill_matches_sequential_hydrate(cfg_name, n):
    # micro has head_dim 16: prefill runs it token by token through the decode path
    cfg = dict(TINY if cfg_name == "tiny" else MICRO)
    t = np_tensors(cfg, seed=41, std=0.02 if cfg_name == "tiny" else 0.1)
    om = O.OracleModel(cfg, t)
    hm = hip().HipModel(cfg, t)
    toks = np.random.default_rng(42).integers(0, cfg["vocab_size"], n)
    lo = _sequential(om, toks)
    lh = hm.prefill(toks)
    assert npref.rel_l2(lh, lo) < PREFILL_LOGIT_TOL
    _check_kv_close(om, hm, cfg["n_layers"], n)
    # decoding continues from the prefilled cache
    nxt = O.argmax(lo)
    assert npref.rel_l2(hm.forward(nxt, n), om.forward(nxt, n)) < PREFILL_LOGIT_TOL
    hm.close()


@pytest.mark.parametrize("graph", [1, 0])
def test_odd_vocabulary_lm_head_and_argmax(graph):
    # An odd vocabulary streams the lm_head one row per group and takes the greedy argmax in a
    # launch of its own (the fused argmax works on row pairs), and the single launch is not
    # offered. Batched prefill's last-token logits and decode logits against the oracle; the
    # device's greedy token against the reference tie rule on the device's own logits.
    cfg = dict(TINY, vocab_size=1001)
    t = np_tensors(cfg, seed=66, std=0.02)
    om = O.OracleModel(cfg, t)
    hm = hip().HipModel(cfg, t)
    hm.set_option("graph", graph)
    with pytest.raises(hip().HipError):
        hm.set_option("single_launch", 1)
    toks = np.random.default_rng(67).integers(0, cfg["vocab_size"], 40)
    lo = _sequential(om, toks)
    assert npref.rel_l2(hm.prefill(toks), lo) < PREFILL_LOGIT_TOL
    tok = O.argmax(lo)
    for pos in range(len(toks), len(toks) + 8):
        lo = om.forward(tok, pos)
        lh = hm.forward(tok, pos)
        assert npref.rel_l2(lh, lo) < PREFILL_LOGIT_TOL, pos
        nxt = hm.forward_argmax(tok, pos)  # the same step again: the same K/V entries, then the token
        assert nxt == O.argmax(lh), pos
        tok = nxt
    hm.close()


# Batched-path shapes beyond tiny: one kv head of 32 dims (the V-cache transpose covers half a
# 64-dim tile), 2 and 8 query heads per kv head, head_dim 64 and partial rotary; prompt lengths
# that are not multiples of the 64-position transpose tile, after a few decode steps.
PREFILL_SHAPES = {
    "hd32_kv1_g4": dict(TINY, dim=128, head_dim=32, n_heads=4, n_kv_heads=1, rotary_dim=32, n_layers=2),
    "hd64_g2": dict(TINY, dim=256, head_dim=64, n_heads=4, n_kv_heads=2, rotary_dim=32, n_layers=2),
    "hd32_g8": dict(TINY, dim=256, head_dim=32, n_heads=8, n_kv_heads=1, rotary_dim=32, n_layers=2),
}


@pytest.mark.parametrize("shape", list(PREFILL_SHAPES))
def test_prefill_shapes_match_sequential_hydrate(shape):
    cfg = PREFILL_SHAPES[shape]
    t = np_tensors(cfg, seed=46, std=0.05)
    om = O.OracleModel(cfg, t)
    hm = hip().HipModel(cfg, t)
    toks = np.random.default_rng(47).integers(0, cfg["vocab_size"], 3 + 131)
    for i in range(3):
        om.forward(int(toks[i]), i, 0)
        hm.forward(int(toks[i]), i, 0)
    lh = hm.prefill(toks[3:], start_pos=3)
    lo = _sequential(om, toks[3:], start=3)
    assert npref.rel_l2(lh, lo) < PREFILL_LOGIT_TOL
    _check_kv_close(om, hm, cfg["n_layers"], len(toks))
    hm.close()


def test_prefill_in_chunks_and_after_decode_steps():
    cfg = dict(TINY)
    t = np_tensors(cfg, seed=43)
    om = O.OracleModel(cfg, t)
    hm = hip().HipModel(cfg, t)
    toks = np.random.default_rng(44).integers(0, cfg["vocab_size"], 80)
    for i in range(5):  # five decode steps first
        om.forward(int(toks[i]), i, 0)
        hm.forward(int(toks[i]), i, 0)
    hm.prefill(toks[5:45], start_pos=5, logits=False)  # then two prefill chunks
    lh = hm.prefill(toks[45:80], start_pos=45)
    lo = _sequential(om, toks[5:80], start=5)
    assert npref.rel_l2(lh, lo) < PREFILL_LOGIT_TOL
    _check_kv_close(om, hm, cfg["n_layers"], 80)
    hm.close()


def test_prefill_mistral_shape_two_layers():
    cfg = dict(TINY, dim=4096, hidden_dim=14336, head_dim=128, n_layers=2, n_heads=32, n_kv_heads=8,
               max_seq_len=512, rotary_dim=128)
    t = np_tensors(cfg, seed=45)
    om = O.OracleModel(cfg, t)
    hm = hip().HipModel(cfg, t)
    toks = np.random.default_rng(46).integers(0, cfg["vocab_size"], 200)
    lo = _sequential(om, toks)
    lh = hm.prefill(toks)
    assert npref.rel_l2(lh, lo) < PREFILL_LOGIT_TOL
    _check_kv_close(om, hm, cfg["n_layers"], 200)
    hm.close()


def test_prefill_ring_positions_fall_back_to_steps():
    # start + n beyond max_seq_len: the StreamingLLM ring (src/infer.cpp:489-494) runs step by step
    cfg = dict(TINY, max_seq_len=64)
    t = np_tensors(cfg, seed=47)
    om = O.OracleModel(cfg, t)
    hm = hip().HipModel(cfg, t)
    toks = np.random.default_rng(48).integers(0, cfg["vocab_size"], 80)
    lo = _sequential(om, toks)
    lh = hm.prefill(toks)
    assert npref.rel_l2(lh, lo) < 1e-4  # the decode path: fp32 throughout
    hm.close()


def test_prefill_rejects_bad_arguments():
    H = hip()
    cfg = dict(TINY)
    with H.HipModel(cfg, np_tensors(cfg, seed=49)) as m:
        with pytest.raises(H.HipError):
            m.prefill([1, 2, cfg["vocab_size"]])
        with pytest.raises(H.HipError):
            m.prefill([1, 2], start_pos=-1)


# ---- the long-context workload at its own size ------------------------------------------------
MISTRAL2 = dict(TINY, dim=4096, hidden_dim=14336, head_dim=128, n_layers=2, n_heads=32, n_kv_heads=8,
                max_seq_len=4096, rotary_dim=128)


def test_gemm_variants_chosen_per_shape():
    # the per-shape choice the prefill runs (checked before the parity tests rely on it): at 3200
    # rows every Mistral-7B GEMM takes the eight-wave 256 x 256 kernel; with fewer rows (the
    # 256 x 256 grid under 9/16 of the CUs) the 128-row LDS pipeline, 256-row workgroups for W1/W3
    H = hip()
    for mode, N, K in [(2, 14336, 4096), (1, 4096, 14336), (0, 6144, 4096), (1, 4096, 4096)]:
        assert H.gemm_variant(3200, N, K, mode) == (6, 64, 256)
    assert H.gemm_variant(256, 14336, 4096, 2) == (2, 64, 256)
    assert H.gemm_variant(512, 14336, 4096, 2) == (6, 64, 256)
    assert H.gemm_variant(1024, 4096, 4096, 1) == (2, 64, 128)
    assert H.gemm_variant(200, 6144, 4096, 0) == (2, 64, 128)
    assert H.gemm_variant(3200, 6144, 4000, 0)[0] == 4  # K % 64 != 0: the 32-deep LDS pipeline


@pytest.mark.parametrize("mode", [0, 1, 2])
@pytest.mark.parametrize("M,N,K", [(6400, 4096, 1024), (1024, 4096, 4096)])
def test_gemm_eight_wave_split_round(M, N, K, mode):
    # The eight-wave kernel's split of its last, partial round of tiles (on a 256-CU GPU):
    # 6400 x 4096 has 400 tiles, a whole round and 144 more (more than half the CUs: one tail piece
    # per tile, two per tail worker, main parts over 11 of 16 k-steps); 1024 x 4096 has 64 (four
    # parts per tile side by side). Checked against a float64 product on sampled rows and columns,
    # bit-reproducible across calls, and within fp32 rounding of the unsplit kernel.
    H = hip()
    rng = np.random.default_rng(M + N + K + mode)
    n_out = N // 2 if mode == 2 else N
    a = f16(rng.standard_normal((M, K), dtype=np.float32))
    b = f16(rng.standard_normal((n_out, K), dtype=np.float32) * 0.02)
    b3 = f16(rng.standard_normal((n_out, K), dtype=np.float32) * 0.02) if mode == 2 else None
    c0 = rng.standard_normal((M, n_out), dtype=np.float32) if mode == 1 else None
    H.set_gemm_stages(6, 64, 256)
    try:
        got = H.gemm(a, b, mode=mode, b3=b3, c=c0)
        again = H.gemm(a, b, mode=mode, b3=b3, c=c0)
        H.set_gemm_ppsplit(False)
        whole = H.gemm(a, b, mode=mode, b3=b3, c=c0)
    finally:
        H.set_gemm_ppsplit(True)
        H.set_gemm_stages(-1)
    assert np.array_equal(got, again)
    rows = np.unique(np.concatenate([[0, 255, 256, M - 257, M - 256, M - 1], rng.choice(M, 40, replace=False)]))
    cols = np.unique(np.concatenate([[0, 63, 64, 255, 256, n_out - 1], rng.choice(n_out, 120, replace=False)]))
    A = h2f(a[rows]).astype(np.float64)
    want = A @ h2f(b[cols]).astype(np.float64).T
    if mode == 2:
        u = A @ h2f(b3[cols]).astype(np.float64).T
        want = want / (1 + np.exp(-want)) * u
        g = h2f(got[np.ix_(rows, cols)]).astype(np.float64)
        assert npref.rel_l2(g, want) < 2e-3  # fp16 output
        assert npref.rel_l2(h2f(got).astype(np.float64), h2f(whole).astype(np.float64)) < 1e-3
    else:
        if mode == 1:
            want = want + c0[np.ix_(rows, cols)]
        assert npref.rel_l2(got[np.ix_(rows, cols)].astype(np.float64), want) < 1e-6
        assert npref.rel_l2(got.astype(np.float64), whole.astype(np.float64)) < 1e-6


@pytest.mark.parametrize("mode,N,K", [(2, 14336, 4096), (1, 4096, 14336), (0, 6144, 4096), (1, 4096, 4096)])
def test_gemm_production_shapes_at_3200_rows(mode, N, K):
    # The Mistral-7B prefill GEMMs at M = 3200 with the auto-selected variants, against a float64
    # product on sampled rows and columns (tile edges of both tile sizes included).
    H = hip()
    M = 3200
    rng = np.random.default_rng(N + K + mode)
    a = f16(rng.standard_normal((M, K), dtype=np.float32))
    b = f16(rng.standard_normal((N, K), dtype=np.float32) * 0.02)
    b3 = f16(rng.standard_normal((N, K), dtype=np.float32) * 0.02) if mode == 2 else None
    c0 = rng.standard_normal((M, N), dtype=np.float32) if mode == 1 else None
    try:
        got = H.gemm(a, b, mode=mode, b3=b3, c=c0)
    finally:
        H.set_gemm_stages(-1)
    edges = [0, 1, 127, 128, 255, 256, 3071, 3072, 3199]
    rows = np.unique(np.concatenate([edges, rng.choice(M, 40, replace=False)]))
    cedges = [0, 63, 64, 127, 128, 255, 256, N - 129, N - 128, N - 1]
    cols = np.unique(np.concatenate([cedges, rng.choice(N, 200, replace=False)]))
    A = h2f(a[rows]).astype(np.float64)
    want = A @ h2f(b[cols]).astype(np.float64).T
    if mode == 2:
        u = A @ h2f(b3[cols]).astype(np.float64).T
        want = want / (1 + np.exp(-want)) * u
        g = h2f(got[np.ix_(rows, cols)]).astype(np.float64)
        assert npref.rel_l2(g, want) < 2e-3  # fp16 output
        assert np.max(np.abs(g - want)) <= 2e-3 * np.max(np.abs(want))
    else:
        if mode == 1:
            want = want + c0[np.ix_(rows, cols)]
        g = got[np.ix_(rows, cols)].astype(np.float64)
        assert npref.rel_l2(g, want) < 1e-6
        assert np.max(np.abs(g - want)) <= 1e-5 * np.max(np.abs(want))


def test_prefill_3200_tokens_mistral_shape_then_30_decode_steps():
    # The long-context workload at its own size on a two-layer Mistral-shape model (ctx 4096): one
    # batched prefill of 3200 seeded ids (eight-wave 256 x 256 GEMM tiles for all four GEMMs, 100
    # query tiles of prefill attention) against the reference's sequential hydrate
    # (src/main.cpp:169-177), then 30 decode steps at kv ~3200 on both sides from their own caches.
    cfg = dict(MISTRAL2)
    t = np_tensors(cfg, seed=3200)
    toks = np.random.default_rng(3201).integers(0, cfg["vocab_size"], 3200)
    hm = hip().HipModel(cfg, t)
    lh = hm.prefill(toks)
    om = O.OracleModel(cfg, t)
    lo = _sequential(om, toks)
    assert npref.rel_l2(lh, lo) < PREFILL_LOGIT_TOL
    _check_kv_close(om, hm, cfg["n_layers"], len(toks))
    worst = 0.0
    tok = O.argmax(lo)
    for i in range(30):
        lo = om.forward(tok, 3200 + i)
        lh = hm.forward(tok, 3200 + i)
        worst = max(worst, npref.rel_l2(lh, lo))
        tok = O.argmax(lo)  # both sides take the oracle's token
    assert worst < PREFILL_LOGIT_TOL, worst
    om.close()
    hm.close()


def _huge_query_tensors(cfg, seed):
    # Wq x 3e5 (fp16 std ~6000): q ~ N(0, 1e5), past the fp16 range; Wk x 1e-4 keeps the scores
    # O(10) so the softmax is not one-hot. The reference keeps q in fp32 (src/infer.cpp:218-250).
    t = np_tensors(cfg, seed=seed)
    for layer in range(cfg["n_layers"]):
        p = f"model.layers.{layer}."
        t[p + "attn.wq.weight"] = f16(h2f(t[p + "attn.wq.weight"]) * 3e5)
        t[p + "attn.wk.weight"] = f16(h2f(t[p + "attn.wk.weight"]) * 1e-4)
    return t


def test_prefill_query_beyond_fp16_range():
    cfg = dict(TINY, n_layers=2)
    t = _huge_query_tensors(cfg, 51)
    om = O.OracleModel(cfg, t)
    hm = hip().HipModel(cfg, t)
    toks = np.random.default_rng(52).integers(0, cfg["vocab_size"], 150)
    lo = _sequential(om, toks)
    lh = hm.prefill(toks)
    assert np.all(np.isfinite(lh))
    assert npref.rel_l2(lh, lo) < PREFILL_LOGIT_TOL
    # keys ~3e-5 are fp16 subnormals: some round to zero on one side only
    _check_kv_close(om, hm, cfg["n_layers"], len(toks), k_zero_pattern=False)
    nxt = O.argmax(lo)
    assert npref.rel_l2(hm.forward(nxt, len(toks)), om.forward(nxt, len(toks))) < PREFILL_LOGIT_TOL
    om.close()
    hm.close()
