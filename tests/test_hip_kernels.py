"""Kernel-level parity of the HIP path against the CPU oracle (reference src/infer.cpp semantics).

Tolerances: integer/index work bit-exact; fp32-accumulated matvecs and attention within
rel-L2 1e-5 of the oracle (both accumulate in fp32, only the summation order differs).
"""
import numpy as np
import pytest

from oracle import binding as O
from tests import npref
from tests.util import f16, h2f

pytestmark = pytest.mark.gpu

H = None


def hip():
    global H
    if H is None:
        from yalm_amd import hip as _h
        _h.lib()
        H = _h
    return H


RTOL = 1e-5


@pytest.fixture(params=[0, 1], ids=["bpc_default", "bpc_1"])
def bpc(request):
    """Runs a test with the decode path's grid and with one workgroup per CU (many row groups per
    wave, exercising the row loop of every fused matvec)."""
    hip().set_test_bpc(request.param)
    yield request.param
    hip().set_test_bpc(0)


# (1002, 4096) and (6, 14336): more waves than row groups on the unrolled paths (the idle waves'
# first loads go through zero-length descriptors); (4096, 4096) and (32000, 4096): the O projection
# (with the residual) and the lm_head (with the final norm) at the Mistral-7B shape
@pytest.mark.parametrize("d,n", [(32, 64), (100, 256), (384, 768), (6144, 4096), (4096, 14336), (1000, 4096),
                                 (1002, 4096), (6, 14336), (4096, 4096), (32000, 4096)])
@pytest.mark.parametrize("norm", [False, True])
def test_matvec_parity(d, n, norm, bpc):
    rng = np.random.default_rng(d * 7 + n)
    w = f16(rng.standard_normal((d, n)) * 0.02)
    x = rng.standard_normal(n).astype(np.float32)
    g = (1 + 0.1 * rng.standard_normal(n)).astype(np.float32) if norm else None
    got = hip().matvec(x, w, gain=g, eps=1e-5)
    xin = O.rmsnorm(x, g, 1e-5) if norm else x
    want = O.matmul_f16(xin, w)
    assert npref.rel_l2(got, want) < RTOL
    # the residual epilogue (x += W v: the O and W2 projections) takes its input as it is
    r = rng.standard_normal(d).astype(np.float32)
    if norm:
        with pytest.raises(hip().HipError):
            hip().matvec(x, w, gain=g, eps=1e-5, resid=r)
    else:
        got_r = hip().matvec(x, w, resid=r)
        assert npref.rel_l2(got_r, want + r) < RTOL


def test_tensor_parallel_shard_kernels_match_oracle():
    # One GPU's share of an 8-way tensor-parallel split of the Mistral-7B layer, at the shapes the
    # benchmark times: QKV of one kv head and its 4 query heads (768 x 4096, RMSNorm in), O by input
    # columns (4096 x 512 plus the residual), W1/W3 by rows (1792 x 4096) with SwiGLU then W2 by
    # input columns (4096 x 1792 plus the residual) and lm_head by vocabulary rows (4000 x 4096), each
    # against the oracle (reference src/infer.cpp:63-100, 136-146, 339-390); the shard's attention (one
    # kv head at 16417 keys) is an attention case below.
    rng = np.random.default_rng(8)
    x = h2f(f16(rng.standard_normal(4096)))
    g = (1 + 0.1 * rng.standard_normal(4096)).astype(np.float32)
    xn = O.rmsnorm(x, g, 1e-5)
    r = rng.standard_normal(4096).astype(np.float32)

    def w(d, n):
        return f16(rng.standard_normal((d, n), dtype=np.float32) * 0.02)

    for rows in (768, 4000):
        wm = w(rows, 4096)
        assert npref.rel_l2(hip().matvec(x, wm, gain=g, eps=1e-5), O.matmul_f16(xn, wm)) < RTOL
    att = h2f(f16(rng.standard_normal(512)))
    wo = w(4096, 512)
    assert npref.rel_l2(hip().matvec(att, wo, resid=r), O.matmul_f16(att, wo) + r) < RTOL
    w1, w3, w2 = w(1792, 4096), w(1792, 4096), w(4096, 1792)
    got = hip().ffn(x, w1, w2, w3, gain=g, eps=1e-5, act=1, resid=r)
    assert npref.rel_l2(got, O.ffn(xn, w1, w2, w3, 1) + r) < RTOL


@pytest.mark.parametrize("n", [64, 4096, 14336])
def test_matvec_one_hot_is_exact(n):
    rng = np.random.default_rng(n)
    w = f16(rng.standard_normal((64, n)))
    for j in (0, n // 3, n - 1):
        x = np.zeros(n, np.float32)
        x[j] = 1.0
        assert np.array_equal(hip().matvec(x, w), h2f(w[:, j]))


@pytest.mark.parametrize("dim,hidden", [(64, 128), (256, 768), (4096, 14336)])
@pytest.mark.parametrize("act", [1, 0])
def test_ffn_parity(dim, hidden, act, bpc):
    rng = np.random.default_rng(dim + hidden + act)
    w1 = f16(rng.standard_normal((hidden, dim)) * 0.02)
    w2 = f16(rng.standard_normal((dim, hidden)) * 0.02)
    w3 = f16(rng.standard_normal((hidden, dim)) * 0.02)
    x = rng.standard_normal(dim).astype(np.float32)
    g = np.ones(dim, np.float32)
    resid = rng.standard_normal(dim).astype(np.float32)
    got = hip().ffn(x, w1, w2, w3, gain=g, eps=1e-5, act=act, resid=resid)
    want = O.ffn(O.rmsnorm(x, g, 1e-5), w1, w2, w3, act) + resid
    assert npref.rel_l2(got, want) < RTOL


def test_per_layer_kernels_of_the_microbenchmark_workload():
    # The per-layer kernel workload at the Mistral-7B shape, as the benchmark runs it: x fp16 [4096]
    # ~ N(0, 1) (seed 2), weights N(0, 0.02), RMSNorm (eps 1e-5, unit gains) feeding QKV
    # 4096 -> 6144, O 4096 -> 4096 plus the residual, W1/W3 4096 -> 14336 with SwiGLU then W2
    # 14336 -> 4096 plus the residual, and the lm_head 4096 -> 32000; each against the oracle's
    # fp32-accumulated matvec (reference src/infer.cpp:63-100, 136-146, 339-344, 362-390, 501-527).
    rng = np.random.default_rng(2)
    x = h2f(f16(rng.standard_normal(4096)))
    g = np.ones(4096, np.float32)
    xn = O.rmsnorm(x, g, 1e-5)
    r = rng.standard_normal(4096).astype(np.float32)

    def w(d, n):
        return f16(rng.standard_normal((d, n), dtype=np.float32) * 0.02)

    wqkv = w(6144, 4096)
    assert npref.rel_l2(hip().matvec(x, wqkv, gain=g, eps=1e-5), O.matmul_f16(xn, wqkv)) < RTOL
    wo = w(4096, 4096)
    assert npref.rel_l2(hip().matvec(x, wo, resid=r), O.matmul_f16(x, wo) + r) < RTOL
    w1, w3, w2 = w(14336, 4096), w(14336, 4096), w(4096, 14336)
    got = hip().ffn(x, w1, w2, w3, gain=g, eps=1e-5, act=1, resid=r)
    assert npref.rel_l2(got, O.ffn(xn, w1, w2, w3, 1) + r) < RTOL
    wcls = w(32000, 4096)
    assert npref.rel_l2(hip().matvec(x, wcls, gain=g, eps=1e-5), O.matmul_f16(xn, wcls)) < RTOL


@pytest.mark.parametrize("hidden", [1024, 4096, 8192])
def test_swiglu_rows_exact_over_row_loop(hidden, bpc):
    # Square down-projection with identity rows makes the FFN output equal hb itself, so every
    # SwiGLU row (rows past the first pass of the row loop included) is checked on its own.
    rng = np.random.default_rng(hidden)
    dim = 4096
    x = rng.standard_normal(dim).astype(np.float32)
    w1 = f16(rng.standard_normal((hidden, dim)) * 0.02)
    w3 = f16(rng.standard_normal((hidden, dim)) * 0.02)
    w2 = np.zeros((dim, hidden), np.float16)
    k = min(dim, hidden)
    w2[np.arange(k), np.arange(k)] = 1.0
    got = hip().ffn(x, w1, w2.view(np.uint16), w3, gain=None, act=1)[:k]
    a = O.matmul_f16(x, w1)[:k]
    b = O.matmul_f16(x, w3)[:k]
    want = a / (1 + np.exp(-a)) * b
    assert np.max(np.abs(got - want)) <= 1e-5 * np.max(np.abs(want))


ATTN_CASES = [
    # hd, nh, nkv, msl, kv_len, nsplit; nsplit 0 = the decode step's own slice plan (7/8 of the CUs
    # over the kv heads; on the matrix cores one slice up to 320 keys, then 64-, 128- and 384-key
    # slices: 16417 keys as 27 slices of 608 on a 256-CU part), else nsplit slices of at least 64
    (16, 4, 2, 64, 1, 0),
    (32, 8, 2, 512, 17, 0),
    (32, 8, 2, 512, 512, 3),
    (64, 8, 8, 200, 199, 7),
    (128, 32, 8, 4096, 93, 0),
    (128, 32, 8, 4096, 3201, 0),
    (128, 32, 8, 4096, 4096, 64),
    (128, 32, 8, 16448, 16417, 0),
    (128, 4, 1, 16448, 16417, 0),  # one kv head: a GPU's share of an 8-way tensor-parallel split
    (128, 8, 1, 1024, 700, 1),
    (64, 8, 8, 100, 99, 0),       # max_seq_len not a multiple of 8: scalar V path
    (128, 32, 8, 4096, 64, 32),   # exactly one 64-token slice
    (128, 32, 8, 4096, 65, 32),   # a second slice holding one token
    (128, 32, 8, 4096, 700, 0),   # 64-key slices, merged across 11 workgroups
    (128, 32, 8, 4096, 3216, 0),  # 128-key slices
    (32, 8, 2, 520, 300, 5),
    (16, 8, 1, 333, 333, 0),
    (128, 8, 8, 256, 200, 0),     # one query head per kv head
    (128, 16, 8, 512, 300, 0),    # two
    (64, 16, 2, 208, 150, 4),     # eight, head_dim 64
    (32, 4, 1, 1024, 1000, 64),   # many slices
    (128, 32, 8, 4096, 256, 32),
    (128, 32, 8, 4096, 257, 32),
    # waves with no tile in their slice skip their loads: one tile, one key past it, seven tiles
    # and a key, a last slice holding a single key, a last slice shorter than one tile
    (128, 32, 8, 4096, 32, 0),
    (128, 32, 8, 4096, 33, 0),
    (128, 32, 8, 4096, 225, 0),
    (128, 32, 8, 4096, 225, 32),
    (128, 32, 8, 4096, 513, 2),
    (128, 32, 8, 4096, 1030, 4),
]


@pytest.fixture(params=[1, 0], ids=["mfma", "simt"])
def attn_impl(request):
    """Runs a test with the MFMA decode attention (where the shape allows it) and with the SIMT kernel."""
    hip().set_attn_mfma(request.param)
    yield request.param
    hip().set_attn_mfma(1)


@pytest.mark.parametrize("hd,nh,nkv,msl,kv_len,nsplit", ATTN_CASES)
def test_attention_parity(hd, nh, nkv, msl, kv_len, nsplit, attn_impl):
    rng = np.random.default_rng(hd * nh + kv_len)
    kb = f16(rng.standard_normal(nkv * hd * msl))
    vb = f16(rng.standard_normal(nkv * hd * msl))
    q = rng.standard_normal(nh * hd).astype(np.float32)
    got, k_after = hip().attention(q, kb, vb, hd, kv_len - 1, msl, nh, nkv, nsplit=nsplit)
    want, _ = O.mha(q, kb, vb, hd, kv_len, msl, nh, nkv)
    assert npref.rel_l2(got, want) < RTOL
    assert np.array_equal(k_after, kb)  # no sink rotation below max_seq_len


def test_attention_kv_len_one_returns_v0_exactly(attn_impl):
    rng = np.random.default_rng(5)
    hd, nh, nkv, msl = 128, 32, 8, 256
    kb = f16(rng.standard_normal(nkv * hd * msl))
    vb = f16(rng.standard_normal(nkv * hd * msl))
    q = rng.standard_normal(nh * hd).astype(np.float32)
    got, _ = hip().attention(q, kb, vb, hd, 0, msl, nh, nkv)
    V = h2f(vb).reshape(nkv, hd, msl)
    want = np.concatenate([V[h // (nh // nkv), :, 0] for h in range(nh)])
    assert np.array_equal(got, want)


def test_attention_known_answer_one_hot_softmax(attn_impl):
    # The reference's known-answer construction (src/test.cpp:67-125) at head_dim 16: huge query
    # entries make each head's softmax one-hot on a chosen position.
    hd, msl, nh, nkv = 16, 4, 2, 1
    kb = np.zeros(16 * msl, np.uint16)
    kb[0 * 16 + 0] = f16([1.0])[0]    # t=0, dim 0
    kb[1 * 16 + 1] = f16([1.0])[0]    # t=1, dim 1
    kb[2 * 16 + 2] = f16([1.0])[0]    # t=2, dim 2
    kb[3 * 16 + 0] = f16([-1.0])[0]   # t=3, dim 0
    V = np.zeros((hd, msl), np.float32)
    V[0] = [1, 0, 0, -1]
    V[1] = [0, 1, 0, 0]
    V[2] = [0, 0, 1, 0]
    vb = f16(V.reshape(-1))
    q = np.zeros(nh * hd, np.float32)
    q[1] = 1e4
    q[hd + 2] = 1e4
    got, _ = hip().attention(q, kb, vb, hd, msl - 1, msl, nh, nkv)
    want = np.zeros(nh * hd, np.float32)
    want[1] = 1.0
    want[hd + 2] = 1.0
    assert np.allclose(got, want, atol=1e-4)


@pytest.mark.parametrize("hd,nh,nkv,msl,kv_len", [(32, 8, 2, 512, 300), (128, 32, 8, 4096, 3201),
                                                   (128, 32, 8, 4096, 93)])
@pytest.mark.parametrize("qmag", [1e5, 1e-4])
def test_attention_query_magnitude_beyond_fp16(hd, nh, nkv, msl, kv_len, qmag, attn_impl):
    # The reference keeps q in fp32 (src/infer.cpp:218-250), and with qkv_clip = FLT_MAX nothing
    # bounds it. Queries of 1e5 (past the fp16 range) and 1e-4 (fp16 subnormal territory) must give
    # the oracle's result on both kernels; the matrix-core one scales each head into range.
    rng = np.random.default_rng(hd + kv_len + int(qmag > 1))
    # keys scaled so that the scores stay O(10): the softmax is not one-hot and q's precision counts
    kb = f16(rng.standard_normal(nkv * hd * msl) * (1e-4 if qmag > 1 else 1.0))
    vb = f16(rng.standard_normal(nkv * hd * msl))
    q = (rng.standard_normal(nh * hd) * qmag).astype(np.float32)
    got, _ = hip().attention(q, kb, vb, hd, kv_len - 1, msl, nh, nkv)
    want, _ = O.mha(q, kb, vb, hd, kv_len, msl, nh, nkv)
    assert np.all(np.isfinite(got))
    assert npref.rel_l2(got, want) < RTOL


@pytest.mark.parametrize("hd", [32, 128])
def test_attention_known_answer_query_1e5(hd, attn_impl):
    # The reference's known-answer construction (src/test.cpp:67-125) with query entries of 1e5:
    # each head's softmax is one-hot on a chosen key, and the output is that key's V column.
    nh, nkv, msl, kv_len = 4, 1, 64, 40
    kb = np.zeros(nkv * hd * msl, np.uint16)
    V = np.zeros((hd, msl), np.float32)
    targets = [3, 17, 30, 39]  # key position chosen by head h
    for h, tpos in enumerate(targets):
        kb[O.k_cache_idx(h, tpos, msl)] = f16([1.0])[0]  # key tpos points along dim h
        V[:, tpos] = np.arange(hd) * 0.01 + h
    vb = f16(V.reshape(-1))
    q = np.zeros(nh * hd, np.float32)
    for h in range(nh):
        q[h * hd + h] = 1e5
    got, _ = hip().attention(q, kb, vb, hd, kv_len - 1, msl, nh, nkv)
    want = np.concatenate([h2f(vb).reshape(hd, msl)[:, t] for t in targets])
    assert np.allclose(got, want, atol=1e-4)


def _oracle_qkv(x, g, wq, wk, wv, nh, nkv, hd, msl, pos, kc, vc, theta=1e6, clip=3.4028234663852886e38):
    xb = O.rmsnorm(x, g, 1e-5) if g is not None else x.astype(np.float32)
    q = np.clip(O.matmul_f16(xb, wq), -clip, clip)
    k = np.clip(O.matmul_f16(xb, wk), -clip, clip)
    v = np.clip(O.matmul_f16(xb, wv), -clip, clip)
    q = O.rope(q, hd, pos, theta, hd)
    k = O.rope(k, hd, pos, theta, hd)
    kc = kc.copy()
    vc = vc.copy()
    kv_pos = O.positions(pos, msl)[1]  # the ring slot once pos >= max_seq_len
    for i in range(k.size):
        gi, j = divmod(i, hd)
        kc[gi * hd * msl + O.k_cache_idx(j, kv_pos, msl)] = O.f2h([k[i]])[0]
        vc[gi * hd * msl + j * msl + kv_pos] = O.f2h([v[i]])[0]
    return q, kc, vc


def test_qkv_kv_write_bit_exact_at_pos0():
    # One-hot input, no norm, pos 0 (RoPE = identity): every K/V entry is an exact fp16 weight and
    # must land at the reference index.
    rng = np.random.default_rng(6)
    dim, nh, nkv, hd, msl = 4096, 32, 8, 128, 64
    wq = f16(rng.standard_normal((nh * hd, dim)))
    wk = f16(rng.standard_normal((nkv * hd, dim)))
    wv = f16(rng.standard_normal((nkv * hd, dim)))
    x = np.zeros(dim, np.float32)
    x[123] = 1.0
    kc = np.zeros(nkv * hd * msl, np.uint16)
    vc = np.zeros(nkv * hd * msl, np.uint16)
    q, k2, v2 = hip().qkv(x, None, wq, wk, wv, nh, nkv, hd, msl, 0, kc, vc)
    qo, ko, vo = _oracle_qkv(x, None, wq, wk, wv, nh, nkv, hd, msl, 0, kc, vc)
    assert np.array_equal(q, h2f(wq[:, 123]))
    assert np.array_equal(k2, ko)
    assert np.array_equal(v2, vo)


@pytest.mark.parametrize("pos", [0, 5, 4095])
@pytest.mark.parametrize("shape", [(256, 8, 2, 32, 512), (4096, 32, 8, 128, 4096)])
def test_qkv_rope_parity(pos, shape, bpc):
    dim, nh, nkv, hd, msl = shape
    rng = np.random.default_rng(pos + dim)
    wq = f16(rng.standard_normal((nh * hd, dim)) * 0.02)
    wk = f16(rng.standard_normal((nkv * hd, dim)) * 0.02)
    wv = f16(rng.standard_normal((nkv * hd, dim)) * 0.02)
    x = rng.standard_normal(dim).astype(np.float32)
    g = (1 + 0.1 * rng.standard_normal(dim)).astype(np.float32)
    kc = f16(rng.standard_normal(nkv * hd * msl))
    vc = f16(rng.standard_normal(nkv * hd * msl))
    q, k2, v2 = hip().qkv(x, g, wq, wk, wv, nh, nkv, hd, msl, pos, kc, vc)
    qo, ko, vo = _oracle_qkv(x, g, wq, wk, wv, nh, nkv, hd, msl, pos, kc, vc)
    # the RoPE angle error grows with pos (fp32 frequencies can differ by an ulp between libms)
    assert npref.rel_l2(q, qo) < 1e-5 + 3e-7 * pos
    changed = (k2 != kc) | (ko != kc)
    # only the entries of slot kv_pos may change, and they are all at reference indices
    kv_pos = O.positions(pos, msl)[1]
    idx = np.array([gi * hd * msl + O.k_cache_idx(j, kv_pos, msl) for gi in range(nkv) for j in range(hd)])
    mask = np.zeros_like(changed)
    mask[idx] = True
    assert not np.any(changed & ~mask)
    assert npref.rel_l2(h2f(k2[idx]), h2f(ko[idx])) < 2e-3
    vidx = np.array([gi * hd * msl + j * msl + kv_pos for gi in range(nkv) for j in range(hd)])
    vmask = np.zeros(vc.size, bool)
    vmask[vidx] = True
    assert np.array_equal(v2[~vmask], vc[~vmask])
    assert npref.rel_l2(h2f(v2[vidx]), h2f(vo[vidx])) < 2e-3


@pytest.mark.parametrize("pos", [5, 4095])
@pytest.mark.parametrize("shape,clip", [((256, 8, 2, 32, 512), 0.05), ((256, 8, 2, 32, 512), 0.2),
                                        ((4096, 32, 8, 128, 4096), 0.05), ((4096, 32, 8, 128, 4096), 1.0)])
def test_qkv_finite_clip_before_rope(pos, shape, clip):
    # A finite qkv_clip (metadata key, reference src/model.cpp:59) clamps q, k and v before RoPE
    # (src/infer.cpp:284-294). With q ~ N(0, 1.3) at the Mistral shape most entries saturate, so a
    # clip applied after RoPE (rotated pairs reach clip * sqrt(2)) or not at all shows at once.
    dim, nh, nkv, hd, msl = shape
    rng = np.random.default_rng(pos + dim + 7)
    wq = f16(rng.standard_normal((nh * hd, dim)) * 0.02)
    wk = f16(rng.standard_normal((nkv * hd, dim)) * 0.02)
    wv = f16(rng.standard_normal((nkv * hd, dim)) * 0.02)
    x = rng.standard_normal(dim).astype(np.float32)
    g = (1 + 0.1 * rng.standard_normal(dim)).astype(np.float32)
    kc = np.zeros(nkv * hd * msl, np.uint16)
    vc = np.zeros(nkv * hd * msl, np.uint16)
    q, k2, v2 = hip().qkv(x, g, wq, wk, wv, nh, nkv, hd, msl, pos, kc, vc, qkv_clip=clip)
    qo, ko, vo = _oracle_qkv(x, g, wq, wk, wv, nh, nkv, hd, msl, pos, kc, vc, clip=clip)
    raw = O.matmul_f16(O.rmsnorm(x, g, 1e-5), wq)
    assert np.mean(np.abs(raw) >= clip) > 0.2  # the clip is active on many entries
    assert npref.rel_l2(q, qo) < 1e-5 + 3e-7 * pos
    # rotated clipped pairs leave the [-clip, clip] box: the clip ran before RoPE
    assert np.max(np.abs(q)) > 1.2 * clip
    assert np.max(np.abs(q)) <= clip * np.sqrt(2) * (1 + 1e-5)
    kv_pos = O.positions(pos, msl)[1]
    idx = np.array([gi * hd * msl + O.k_cache_idx(j, kv_pos, msl) for gi in range(nkv) for j in range(hd)])
    vidx = np.array([gi * hd * msl + j * msl + kv_pos for gi in range(nkv) for j in range(hd)])
    assert npref.rel_l2(h2f(k2[idx]), h2f(ko[idx])) < 2e-3
    # V is clipped and not rotated: every entry within the box, equal to the oracle's to an ulp
    assert np.max(np.abs(h2f(v2[vidx]))) <= clip * (1 + 2 ** -10)
    assert np.max(np.abs(h2f(v2[vidx]) - h2f(vo[vidx]))) <= 2 ** -10 * clip


def test_argmax_tie_rule():
    lg = np.zeros(32000, np.float32)
    assert hip().argmax(lg) == 0
    lg[[7, 300, 31999]] = 5.0
    assert hip().argmax(lg) == 7
    rng = np.random.default_rng(8)
    lg = rng.standard_normal(32000).astype(np.float32)
    assert hip().argmax(lg) == O.argmax(lg)
    lg[-1] = np.inf
    assert hip().argmax(lg) == 31999
