"""The HF -> .yalm converter (yalm_amd/convert.py) against what fixes its output independently:

  - the rotary row permutation: scores of HF's rotate-half RoPE on the HF rows equal the adjacent-
    pair RoPE of the decode path (reference src/infer.cpp:202-215) on the permuted rows;
  - the GPT-2 byte alphabet: a bijection onto the 256 bytes with the published anchors (space is
    U+0120, newline U+010A, '!' itself);
  - a whole model: a small random MistralForCausalLM from `transformers` (its own PyTorch forward,
    fp32) saved as an HF checkpoint and converted; the CPU oracle on the .yalm reproduces its logits,
    and the same conversion without the permutation does not (the planted mistake);
  - on the GPU, the HIP decode path on the converted file reproduces the same logits.
"""
import json
import os

import numpy as np
import pytest

from yalm_amd import convert as C

TINY_HF = dict(vocab_size=512, hidden_size=128, intermediate_size=384, num_hidden_layers=2,
               num_attention_heads=4, num_key_value_heads=2, head_dim=32, max_position_embeddings=256,
               rope_theta=1e6, rms_norm_eps=1e-5, tie_word_embeddings=False, bos_token_id=1, eos_token_id=2,
               sliding_window=None)
PROMPT = [1, 17, 300, 5, 511, 42, 42, 9, 100, 250, 3, 77]
TEXT_IDS = [1, 260, 261]  # BOS, " hello", " world" in the test vocabulary
GEN = 8
HF = {}  # checkpoint dir -> (greedy ids after TEXT_IDS, top-2 margins)


# ---- rotary permutation -------------------------------------------------------------------------
def rope_rotate_half(x, pos, theta, rd):
    """HF form: pairs (i, i + rd/2), angle pos * theta^(-2i/rd)."""
    half = rd // 2
    ang = pos * theta ** (-np.arange(half) * 2.0 / rd)
    c, s = np.cos(ang), np.sin(ang)
    y = x.copy()
    a, b = x[..., :half], x[..., half:rd]
    y[..., :half] = a * c - b * s
    y[..., half:rd] = a * s + b * c
    return y


def rope_adjacent(x, pos, theta, rd):
    """Decode-path form (reference src/infer.cpp:202-215): pairs (2i, 2i + 1), the same angles."""
    half = rd // 2
    ang = pos * theta ** (-np.arange(half) * 2.0 / rd)
    c, s = np.cos(ang), np.sin(ang)
    y = x.copy()
    a, b = x[..., 0:rd:2], x[..., 1:rd:2]
    y[..., 0:rd:2] = a * c - b * s
    y[..., 1:rd:2] = a * s + b * c
    return y


@pytest.mark.parametrize("hd,rd", [(32, 32), (64, 64), (64, 32)])
def test_rotary_permutation_preserves_scores(hd, rd):
    rng = np.random.default_rng(hd + rd)
    nh, nkv, d = 4, 2, 48
    wq = rng.standard_normal((nh * hd, d))
    wk = rng.standard_normal((nkv * hd, d))
    xq, xk = rng.standard_normal(d), rng.standard_normal(d)
    pq, pk = 37, 11
    q_hf = rope_rotate_half((wq @ xq).reshape(nh, hd), pq, 1e4, rd)
    k_hf = rope_rotate_half((wk @ xk).reshape(nkv, hd), pk, 1e4, rd)
    q_y = rope_adjacent((C.rotary_rows_to_adjacent(wq, nh, rd) @ xq).reshape(nh, hd), pq, 1e4, rd)
    k_y = rope_adjacent((C.rotary_rows_to_adjacent(wk, nkv, rd) @ xk).reshape(nkv, hd), pk, 1e4, rd)
    s_hf = q_hf.reshape(nkv, nh // nkv, hd) @ k_hf[:, :, None]
    s_y = q_y.reshape(nkv, nh // nkv, hd) @ k_y[:, :, None]
    np.testing.assert_allclose(s_y, s_hf, rtol=1e-12, atol=1e-12)
    # the identity (a converter that forgets the permutation) does not preserve them
    q_bad = rope_adjacent((wq @ xq).reshape(nh, hd), pq, 1e4, rd)
    k_bad = rope_adjacent((wk @ xk).reshape(nkv, hd), pk, 1e4, rd)
    s_bad = q_bad.reshape(nkv, nh // nkv, hd) @ k_bad[:, :, None]
    assert np.max(np.abs(s_bad - s_hf)) > 1e-3 * np.max(np.abs(s_hf))


def test_rotary_permutation_is_a_row_permutation():
    w = np.arange(2 * 8 * 3).reshape(16, 3)
    p = C.rotary_rows_to_adjacent(w, 2, 6)
    rows = p[:, 0] // 3
    assert rows.tolist() == [0, 3, 1, 4, 2, 5, 6, 7, 8, 11, 9, 12, 10, 13, 14, 15]


# ---- tokenizer ----------------------------------------------------------------------------------
def test_byte_level_alphabet():
    t = C.byte_level_decoder()
    assert sorted(t.values()) == list(range(256))
    assert t["Ġ"] == 0x20 and t["Ċ"] == 0x0A and t["!"] == 0x21 and t["Ā"] == 0x00
    assert t["ÿ"] == 0xFF and t["Ń"] == 0xAD


def sentencepiece_tokenizer(vocab_size):
    vocab = {"<unk>": 0, "<s>": 1, "</s>": 2}
    for b in range(256):
        vocab[f"<0x{b:02X}>"] = 3 + b
    words = ["▁the", "▁hello", "▁world", "ing", "é", "▁a▁b"]
    for i, w in enumerate(words):
        vocab[w] = 259 + i
    for i in range(259 + len(words), vocab_size):
        vocab[f"tok{i}"] = i
    return {"model": {"type": "BPE", "vocab": vocab, "merges": [], "byte_fallback": True},
            "added_tokens": [{"id": 0, "content": "<unk>"}, {"id": 1, "content": "<s>"}, {"id": 2, "content": "</s>"}]}


def test_token_bytes_sentencepiece_and_byte_level():
    tb = C.token_bytes(sentencepiece_tokenizer(300), 300)
    assert tb[1] == b"<s>" and tb[3 + 0x41] == b"<0x41>"
    assert tb[260] == b" hello" and tb[263] == "é".encode() and tb[264] == b" a b"
    bl = {"model": {"type": "BPE", "vocab": {"Ġworld": 0, "hello": 1, "Ċ": 2, "cafÃ©": 3}},
          "added_tokens": [{"id": 4, "content": "<|endoftext|>"}]}
    tb = C.token_bytes(bl, 6)
    assert tb[0] == b" world" and tb[1] == b"hello" and tb[2] == b"\n"
    assert tb[3] == "café".encode() and tb[4] == b"<|endoftext|>" and tb[5] == b""
    with pytest.raises(C.ConvertError):
        C.token_bytes(bl, 2)


# ---- whole model against transformers -----------------------------------------------------------
@pytest.fixture(scope="module")
def hf_checkpoint(tmp_path_factory):
    torch = pytest.importorskip("torch")
    tr = pytest.importorskip("transformers")
    torch.manual_seed(0)
    cfg = tr.MistralConfig(**TINY_HF)
    model = tr.MistralForCausalLM(cfg).eval()
    with torch.no_grad():
        for name, p in model.named_parameters():
            if "q_proj" in name or "k_proj" in name:
                p.mul_(6.0)  # scores of order 1, so a wrong rotary pairing shows in the logits
            p.copy_(p.half().float())  # fp16-exact, so the converted weights equal the HF ones
        logits = model(torch.tensor([PROMPT])).logits[0].double().numpy()
        # greedy continuation of the text prompt " hello world" (BOS, " hello", " world") and each
        # step's top-2 logit margin
        ids, margins = list(TEXT_IDS), []
        for _ in range(GEN):
            lg = model(torch.tensor([ids])).logits[0, -1].double().numpy()
            top = np.sort(lg)[-2:]
            margins.append(float(top[1] - top[0]))
            ids.append(int(np.argmax(lg)))
    d = tmp_path_factory.mktemp("hf_mistral")
    model.save_pretrained(d)
    with open(d / "tokenizer.json", "w") as f:
        json.dump(sentencepiece_tokenizer(TINY_HF["vocab_size"]), f)
    HF[d] = (ids[len(TEXT_IDS):], margins)
    return d, logits


def converted(hf_dir, out):
    C.convert(str(hf_dir), str(out))
    from yalm_amd import host
    sess = host.Session.open(str(out))
    cfg = dict(sess.config())
    t = {k: np.array(v) for k, v in sess.tensors().items()}
    sess.close()
    return cfg, t


def oracle_logits(cfg, t):
    from oracle import binding as O
    om = O.OracleModel(dict(cfg, act=1), t)
    return np.stack([om.forward(tok, pos) for pos, tok in enumerate(PROMPT)])


def rel_l2(a, b):
    return float(np.linalg.norm(a - b) / np.linalg.norm(b))


def test_convert_matches_transformers_on_the_oracle(hf_checkpoint, tmp_path):
    hf_dir, ref = hf_checkpoint
    cfg, t = converted(hf_dir, tmp_path / "m.yalm")
    assert (cfg["dim"], cfg["hidden_dim"], cfg["head_dim"], cfg["n_layers"], cfg["n_heads"], cfg["n_kv_heads"],
            cfg["vocab_size"], cfg["rotary_dim"]) == (128, 384, 32, 2, 4, 2, 512, 32)
    assert t["model.layers.0.attn.norm.weight"].dtype == np.float32
    assert cfg["rope_theta"] == 1e6
    got = oracle_logits(cfg, t)
    for pos in range(len(PROMPT)):
        assert rel_l2(got[pos], ref[pos]) < 2e-3, pos  # fp16 K/V cache on the oracle side
    assert [int(np.argmax(g)) for g in got] == [int(np.argmax(r)) for r in ref]


def test_convert_without_the_permutation_is_caught(hf_checkpoint, tmp_path, monkeypatch):
    hf_dir, ref = hf_checkpoint
    monkeypatch.setattr(C, "rotary_rows_to_adjacent", lambda w, n, r: w)
    cfg, t = converted(hf_dir, tmp_path / "bad.yalm")
    got = oracle_logits(cfg, t)
    assert max(rel_l2(got[p], ref[p]) for p in range(1, len(PROMPT))) > 2e-2


def test_converted_file_header_and_vocabulary(hf_checkpoint, tmp_path):
    hf_dir, _ = hf_checkpoint
    out = tmp_path / "m.yalm"
    C.convert(str(hf_dir), str(out))
    from safetensors import safe_open
    with safe_open(str(out), framework="numpy") as f:
        meta = f.metadata()
        tok = f.get_tensor("tokenizer.tokens")
        assert "model.output.weight" in f.keys() and "lm_head.weight" not in f.keys()
    assert meta["arch"] == "MistralForCausalLM" and meta["dtype"] == "fp16" and meta["act_type"] == "silu"
    assert meta["bos_token_id"] == "1" and meta["eos_token_id"] == "2" and float(meta["rope_theta"]) == 1e6
    strings = bytes(tok).split(b"\0")[:-1]
    assert len(strings) == TINY_HF["vocab_size"] and strings[260] == b" hello" and strings[1] == b"<s>"


def test_convert_rejects_unsupported_input(tmp_path):
    with pytest.raises(C.ConvertError):
        C.metadata(dict(TINY_HF, architectures=["MixtralForCausalLM"], hidden_act="silu"), "fp16")
    with pytest.raises(C.ConvertError):
        C.metadata(dict(TINY_HF, architectures=["MistralForCausalLM"], attention_bias=True), "fp16")
    with pytest.raises(C.ConvertError):
        C.metadata(dict(TINY_HF, architectures=["MistralForCausalLM"]), "fp8")
    with pytest.raises(C.ConvertError):  # scaled RoPE (e.g. Llama 3.1) would convert into a wrong model
        C.metadata(dict(TINY_HF, architectures=["LlamaForCausalLM"],
                        rope_parameters={"rope_type": "llama3", "rope_theta": 5e5, "factor": 8.0}), "fp16")
    # both spellings of the RoPE base: a top-level key (older configs) and rope_parameters (newer)
    m = C.metadata(dict(TINY_HF, architectures=["MistralForCausalLM"]), "fp16")
    assert float(m["rope_theta"]) == 1e6
    m = C.metadata(dict({k: v for k, v in TINY_HF.items() if k != "rope_theta"}, architectures=["MistralForCausalLM"],
                        rope_parameters={"rope_type": "default", "rope_theta": 5e5}), "fp16")
    assert float(m["rope_theta"]) == 5e5
    with pytest.raises(C.ConvertError):
        C.convert(str(tmp_path), str(tmp_path / "x.yalm"))  # no config.json
    assert C.main([str(tmp_path / "x.yalm"), str(tmp_path)]) == 1


@pytest.mark.gpu
def test_hip_decode_on_converted_file_matches_transformers(hf_checkpoint, tmp_path):
    from yalm_amd import host
    hf_dir, ref = hf_checkpoint
    out = tmp_path / "m.yalm"
    C.convert(str(hf_dir), str(out))
    with host.Session.open(str(out)) as sess:
        sess.hip(0)
        got = np.stack([sess.forward(tok, pos) for pos, tok in enumerate(PROMPT)])
    for pos in range(len(PROMPT)):
        assert rel_l2(got[pos], ref[pos]) < 2e-3, pos
    assert [int(np.argmax(g)) for g in got] == [int(np.argmax(r)) for r in ref]


@pytest.mark.gpu
def test_cli_text_prompt_on_converted_file(hf_checkpoint, tmp_path):
    # yalm <file> -i " hello world" -t 0: the converted vocabulary through the host tokenizer, then
    # greedy decoding on the HIP device against the transformers model's greedy continuation (up to
    # the first step whose top-2 margin is too small to be decided by fp32 noise).
    import subprocess
    hf_dir, _ = hf_checkpoint
    exe = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "yalm_amd", "bin", "yalm")
    if not os.path.exists(exe):
        pytest.skip("CLI not built")
    out = tmp_path / "m.yalm"
    C.convert(str(hf_dir), str(out))
    r = subprocess.run([exe, str(out), "-i", " hello world", "-t", "0", "-n", str(GEN)], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    line = [ln for ln in r.stdout.splitlines() if ln.startswith("tokens:")][-1]
    toks = [int(v) for v in line.split()[1:]]
    assert toks[:len(TEXT_IDS)] == TEXT_IDS
    want, margins = HF[hf_dir]
    sure = next((i for i, m in enumerate(margins) if m < 1e-3), len(margins))
    assert sure >= 1
    assert toks[len(TEXT_IDS):len(TEXT_IDS) + sure] == want[:sure]


@pytest.mark.gpu
def test_cli_perplexity_and_passkey_modes_on_converted_file(hf_checkpoint, tmp_path):
    # yalm <file> -m perplexity -p <ids> on the HIP device (reference src/main.cpp:213-294): the
    # perplexity of the prompt's next tokens, exp(-mean log p), and its error term, against the same
    # sums over the oracle's logits on the converted file. Then -m passkey (src/main.cpp:296-378)
    # runs its haystack prompt token by token and batched, and prints its greedy answer.
    import re
    import subprocess
    hf_dir, _ = hf_checkpoint
    exe = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "yalm_amd", "bin", "yalm")
    if not os.path.exists(exe):
        pytest.skip("CLI not built")
    out = tmp_path / "m.yalm"
    cfg, t = converted(hf_dir, out)
    r = subprocess.run([exe, str(out), "-m", "perplexity", "-p", ",".join(map(str, PROMPT))], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    m = re.search(r"perplexity: ([0-9.e+-]+) ± ([0-9.e+-]+)", r.stdout)
    assert m, r.stdout
    lg = oracle_logits(cfg, t).astype(np.float64)
    lp = np.array([lg[p, PROMPT[p + 1]] - lg[p].max() - np.log(np.exp(lg[p] - lg[p].max()).sum())
                   for p in range(len(PROMPT) - 1)])
    n = len(lp)
    ppl = float(np.exp(-lp.sum() / n))
    err = ppl * float(np.sqrt((np.sum(lp * lp) - lp.sum() ** 2 / n) / n / n))
    assert abs(float(m.group(1)) - ppl) <= 1e-3 * ppl, (m.group(0), ppl, err)
    assert abs(float(m.group(2)) - err) <= 1e-2 * err + 1e-4, (m.group(0), ppl, err)
    for batched in ("0", "1"):
        r = subprocess.run([exe, str(out), "-m", "passkey", "-n", "4", "-l", "1", "-b", batched], capture_output=True,
                           timeout=120)  # the answer of a random model can hold partial UTF-8 byte tokens
        so = r.stdout.decode("utf-8", errors="replace")
        assert r.returncode == 0, r.stderr.decode("utf-8", errors="replace")
        assert "Passkey test:" in so and "What is the pass key? The pass key is" in so, so
