"""CPU tests of the host library (libyalm_host.so): .yalm codec, Config parsing, synthetic writer,
fp16 conversion. Mirrors the reference's codec rules (src/codec.cpp:39-156) and Config keys
(src/model.cpp:18-71). No device calls."""
import json
import os
import struct
import subprocess

import numpy as np
import pytest

from tests.util import TINY

H = pytest.importorskip("yalm_amd.host")

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def small_shape(**kw):
    d = dict(dim=64, hidden_dim=128, head_dim=16, n_layers=2, n_heads=4, n_kv_heads=2, vocab_size=300,
             max_seq_len=128)
    d.update(kw)
    return d


def write_raw(path, header: dict, payload: bytes, pad=True):
    h = json.dumps(header).encode()
    if pad:
        h += b" " * ((8 - (len(h) + 8) % 8) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)) + h + payload)


def meta(**over):
    m = {"dim": "16", "hidden_dim": "32", "head_dim": "16", "n_layers": "0", "n_heads": "1", "n_kv_heads": "1",
         "vocab_size": "4", "max_seq_len": "64", "rope_theta": "10000.0", "rotary_dim": "16", "dtype": "fp16",
         "bos_token_id": "1", "eos_token_id": "2", "act_type": "silu"}
    m.update(over)
    return m


def good_header(**over):
    e = 4 * 16 * 2
    return {"__metadata__": meta(**over),
            "model.embed.weight": {"dtype": "F16", "shape": [4, 16], "data_offsets": [0, e]},
            "model.norm.weight": {"dtype": "F32", "shape": [16], "data_offsets": [e, e + 64]},
            "tokenizer.tokens": {"dtype": "U8", "shape": [8], "data_offsets": [e + 64, e + 72]}}


def good_payload():
    return np.zeros(4 * 16, np.float16).tobytes() + np.ones(16, np.float32).tobytes() + b"a\0b\0c\0d\0"


def test_fp16_conversion_matches_numpy():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    f = H.f16_to_f32(bits)
    want = bits.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(f), nan)
    assert np.array_equal(f[~nan].view(np.uint32), want[~nan].view(np.uint32))
    rng = np.random.default_rng(0)
    vals = np.concatenate([rng.standard_normal(200000).astype(np.float32) * s for s in (1e-6, 1e-3, 1, 100, 3e4)]
                          + [np.array([65504, 65519.99, 65520, 1e10, -0.0, 0.0, np.inf, -np.inf], np.float32),
                             (np.arange(0, 4096, dtype=np.float32) + 0.5) * np.float32(2.0 ** -24),
                             (np.arange(1024, 2048, dtype=np.float32) + 0.5) * np.float32(2.0 ** -10)])
    with np.errstate(over="ignore"):
        want = vals.astype(np.float16).view(np.uint16)
    assert np.array_equal(H.f32_to_f16(vals), want)


def test_synthetic_roundtrip_and_determinism(tmp_path):
    shp = small_shape()
    a = H.Session.synthetic(shp, seed=7)
    b = H.Session.synthetic(shp, seed=7)
    c = H.Session.synthetic(shp, seed=8)
    w = a.tensor("model.layers.1.mlp.w2.weight")
    assert w.shape == (64, 128) and w.dtype == np.uint16
    assert np.array_equal(w, b.tensor("model.layers.1.mlp.w2.weight"))
    assert not np.array_equal(w, c.tensor("model.layers.1.mlp.w2.weight"))
    p = tmp_path / "m.yalm"
    a.write(p)
    d = H.Session.open(p)
    for name, t in a.tensors().items():
        assert np.array_equal(t, d.tensor(name)), name
    cfg = d.config()
    assert cfg["dim"] == 64 and cfg["n_layers"] == 2 and cfg["act"] == 1 and cfg["rotary_dim"] == 16
    assert abs(cfg["rope_theta"] - 1e6) < 1 and abs(cfg["norm_eps"] - 1e-5) < 1e-9


def test_synthetic_weights_are_normal_002():
    s = H.Session.synthetic(dict(TINY), seed=0x59414C4D)
    w = s.tensor("model.layers.0.mlp.w1.weight").view(np.float16).astype(np.float64).reshape(-1)
    assert abs(w.std() - 0.02) < 2e-4 and abs(w.mean()) < 2e-4
    # Gaussian shape: about 68.3% within one sigma, 95.4% within two
    f1 = np.mean(np.abs(w) < 0.02)
    f2 = np.mean(np.abs(w) < 0.04)
    assert abs(f1 - 0.6827) < 0.01 and abs(f2 - 0.9545) < 0.005
    assert np.all(s.tensor("model.norm.weight") == 1.0)


def test_context_cap_and_override(tmp_path):
    s = H.Session.synthetic(small_shape(max_seq_len=32768))
    assert s.config()["max_seq_len"] == 4096  # capped like the reference (src/model.cpp:30-34)
    s2 = H.Session.synthetic(small_shape(max_seq_len=32768), context=16448)
    assert s2.config()["max_seq_len"] == 16448


def test_uniform_ids():
    ids = H.uniform_ids(10000, 32, 32000)
    assert ids.min() >= 0 and ids.max() < 32000
    assert np.array_equal(ids, H.uniform_ids(10000, 32, 32000))
    assert len(np.unique(ids)) > 8000


def test_active_bytes_matches_reference_formula():
    s = H.Session.synthetic(small_shape())
    d, hid, hd, L, nh, nkv, V, msl = 64, 128, 16, 2, 4, 2, 300, 128
    for pos in (0, 5, 500):
        kv_len = min(msl, pos + 1)
        per = 2 * d * 4 + nh * hd * d * 2 + 2 * nkv * hd * d * 2 + nh * hd * d * 2 + 3 * d * hid * 2
        per += 2 * kv_len * nkv * hd * 2
        want = d * 2 + L * per + d * 4 + V * d * 4
        assert s.active_bytes(pos) == want


@pytest.mark.parametrize("case", ["short", "zero_header", "header_too_long", "bad_dtype", "offsets_beyond",
                                  "offsets_reversed", "size_mismatch", "three_offsets", "bad_json"])
def test_codec_rejects_malformed_files(tmp_path, case):
    p = tmp_path / f"{case}.yalm"
    hdr = good_header()
    pay = good_payload()
    if case == "short":
        p.write_bytes(b"\x01\x02")
    elif case == "zero_header":
        p.write_bytes(struct.pack("<Q", 0) + b"{}")
    elif case == "header_too_long":
        p.write_bytes(struct.pack("<Q", 1000) + b"{}")
    elif case == "bad_json":
        p.write_bytes(struct.pack("<Q", 5) + b"{oops")
    else:
        if case == "bad_dtype":
            hdr["model.embed.weight"]["dtype"] = "F64"
        elif case == "offsets_beyond":
            hdr["tokenizer.tokens"]["data_offsets"] = [192, 10000]
        elif case == "offsets_reversed":
            hdr["model.norm.weight"]["data_offsets"] = [192, 128]
        elif case == "size_mismatch":
            hdr["model.norm.weight"]["shape"] = [15]
        elif case == "three_offsets":
            hdr["model.norm.weight"]["data_offsets"] = [128, 192, 200]
        write_raw(p, hdr, pay)
    with pytest.raises(H.HostError):
        H.Session.open(p)


def test_model_rejects_missing_tensor_and_bad_dtype(tmp_path):
    hdr = good_header(n_layers="1")
    p = tmp_path / "missing.yalm"
    write_raw(p, hdr, good_payload())
    with pytest.raises(H.HostError, match="missing tensor"):
        H.Session.open(p)
    p2 = tmp_path / "dtype.yalm"
    write_raw(p2, good_header(dtype="fp8"), good_payload())
    with pytest.raises(H.HostError, match="unsupported dtype"):
        H.Session.open(p2)
    p3 = tmp_path / "ok.yalm"
    write_raw(p3, good_header(), good_payload())
    s = H.Session.open(p3)  # zero-layer model with a tied lm_head opens fine
    assert s.config()["vocab_size"] == 4


def test_cli_usage_and_device_errors(tmp_path):
    exe = os.path.join(ROOT, "yalm_amd", "bin", "yalm")
    r = subprocess.run([exe], capture_output=True, text=True, timeout=60)
    assert r.returncode != 0 and "Usage" in r.stderr
    r = subprocess.run([exe, "x.yalm", "-d", "cpu", "-i", "hi"], capture_output=True, text=True, timeout=60)
    assert r.returncode != 0 and "reference" in r.stderr
    out = tmp_path / "tiny.yalm"
    r = subprocess.run([exe, "--synth", str(out), "tiny", "7"], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr
    s = H.Session.open(out)
    ref = H.Session.synthetic(dict(TINY), seed=7)
    assert np.array_equal(s.tensor("model.layers.2.attn.wk.weight"), ref.tensor("model.layers.2.attn.wk.weight"))
