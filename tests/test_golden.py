"""The committed golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py from the
float64 brute-force model) against the CPU oracle and, on a GPU, against the HIP path.

micro: a 2-layer dim-64 model (logits of 8 steps, both layers' K/V, a 24-token greedy run).
tiny: the dim-256 4-layer 32000-vocab synthetic model at context 512 (logits of positions 0-3 kept as
fp16, layer 0's written K/V, the 32 greedy tokens after a 16-token prompt).
"""
import os
import subprocess

import numpy as np
import pytest

from oracle import binding as O
from tests import npref
from tests.golden import make_golden as G
from tests.util import MICRO, np_tensors, h2f

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    with np.load(os.path.join(GOLDEN, name + ".npz")) as d:
        return {k: d[k] for k in d.files}


def micro_weights():
    return np_tensors(dict(MICRO), seed=G.MICRO_SEED, std=G.MICRO_STD, gain=G.MICRO_GAIN)


def tiny_weights():
    sess = G.tiny_session()
    cfg = sess.config()
    t = {k: np.array(v) for k, v in sess.tensors().items()}
    sess.close()
    return dict(cfg, act=1), t


def check_kv_close(a, b, exact_frac):
    """fp16 caches from fp32 and float64 arithmetic: identical where written, an ulp apart at most."""
    assert np.array_equal(a != 0, b != 0)
    fa, fb = h2f(a), h2f(b)
    assert np.all(np.abs(fa - fb) <= 2e-3 * np.abs(fb) + 1e-7)
    written = (a != 0) | (b != 0)
    assert np.mean(a[written] == b[written]) >= exact_frac


def run_steps(fwd, steps):
    return np.stack([fwd(int(tok), pos) for pos, tok in enumerate(steps)])


def run_greedy(fwd, prompt, n_gen, argmax=O.argmax):
    lg = None
    for pos, tok in enumerate(prompt):
        lg = fwd(int(tok), pos)
    out, pos = [], len(prompt)
    for _ in range(n_gen):
        out.append(argmax(lg))
        lg = fwd(out[-1], pos)
        pos += 1
    return out


def tiny_kv0(k, v, cfg, n):
    hd, msl, nkv = cfg["head_dim"], cfg["max_seq_len"], cfg["n_kv_heads"]
    return (k.reshape(nkv, hd // 16, msl, 16)[:, :, :n, :], v.reshape(nkv, hd, msl)[:, :, :n])


# ---- the fixtures themselves -------------------------------------------------------------------
def test_fixture_weights_are_reproduced():
    assert G.weights_digest(micro_weights()) == str(load("micro")["digest"])
    assert G.weights_digest(tiny_weights()[1]) == str(load("tiny")["digest"])


def test_fixture_margins_leave_room_for_fp32():
    # every greedy step is decided by more than fp32 accumulation noise (~1e-6 relative)
    for name in ("micro", "tiny"):
        assert load(name)["margins"].min() > 5e-4


def cli():
    exe = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "yalm_amd", "bin", "yalm")
    if not os.path.exists(exe):
        pytest.skip("CLI not built")
    return exe


def test_cli_synth_tiny_is_the_fixture_model(tmp_path):
    from yalm_amd import host
    out = tmp_path / "tiny.yalm"
    r = subprocess.run([cli(), "--synth", str(out), "tiny"], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr
    with host.Session.open(out) as sess:
        assert G.weights_digest({k: np.array(v) for k, v in sess.tensors().items()}) == str(load("tiny")["digest"])


# ---- CPU oracle against the fixtures -----------------------------------------------------------
def test_oracle_micro_logits_kv_and_greedy():
    g = load("micro")
    cfg, t = dict(MICRO), micro_weights()
    om = O.OracleModel(cfg, t)
    lg = run_steps(om.forward, g["steps"])
    for step in range(len(g["steps"])):
        assert npref.rel_l2(lg[step], g["logits"][step]) < 1e-5, step
    for layer in range(cfg["n_layers"]):
        k, v = om.kv(layer)
        check_kv_close(k, g["k"][layer], 0.99 if layer == 0 else 0.9)
        check_kv_close(v, g["v"][layer], 0.99 if layer == 0 else 0.9)
    assert run_greedy(O.OracleModel(cfg, t).forward, g["prompt"], len(g["greedy"])) == g["greedy"].tolist()


def test_oracle_tiny_greedy_logits_and_kv():
    g = load("tiny")
    cfg, t = tiny_weights()
    om = O.OracleModel(cfg, t)
    lgs = []

    def fwd(tok, pos):
        lg = om.forward(tok, pos)
        if pos < len(g["logits"]):
            lgs.append(lg)
        return lg

    assert run_greedy(fwd, g["prompt"], len(g["greedy"])) == g["greedy"].tolist()
    for pos, lg in enumerate(lgs):
        assert npref.rel_l2(lg, g["logits"][pos].astype(np.float64)) < 1e-3, pos  # fp16-stored fixture
    k, v = tiny_kv0(*om.kv(0), cfg, int(g["n_written"]))
    check_kv_close(k, g["k0"], 0.99)
    check_kv_close(v, g["v0"], 0.99)


def test_planted_mistake_in_oracle_input_is_caught():
    # The fixture check fails when the oracle sees a perturbed model: one gain off by 1%.
    g = load("micro")
    cfg, t = dict(MICRO), micro_weights()
    t["model.layers.1.mlp.norm.weight"] = t["model.layers.1.mlp.norm.weight"] * np.float32(1.01)
    lg = run_steps(O.OracleModel(cfg, t).forward, g["steps"])
    assert max(npref.rel_l2(lg[s], g["logits"][s]) for s in range(len(g["steps"]))) > 1e-4


# ---- HIP path against the fixtures -------------------------------------------------------------
def _hip():
    from yalm_amd import hip as H
    H.lib()
    return H


@pytest.mark.gpu
@pytest.mark.parametrize("path", ["graph", "single"])
def test_hip_micro_matches_fixture(path):
    from tests.test_hip_model import use_path
    g = load("micro")
    cfg, t = dict(MICRO), micro_weights()
    with _hip().HipModel(cfg, t) as hm:
        use_path(hm, path)
        lg = run_steps(hm.forward, g["steps"])
        for step in range(len(g["steps"])):
            assert npref.rel_l2(lg[step], g["logits"][step]) < 1e-4, step
        for layer in range(cfg["n_layers"]):
            k, v = hm.kv(layer)
            check_kv_close(k, g["k"][layer], 0.99 if layer == 0 else 0.9)
            check_kv_close(v, g["v"][layer], 0.99 if layer == 0 else 0.9)
    with _hip().HipModel(cfg, t) as hm:
        use_path(hm, path)
        assert run_greedy(hm.forward, g["prompt"], len(g["greedy"])) == g["greedy"].tolist()


@pytest.mark.gpu
def test_hip_session_tiny_generate_matches_fixture():
    # The host Model/InferenceState/Sampler loop on the HIP device, greedy on the device.
    g = load("tiny")
    sess = G.tiny_session()
    sess.hip(0)
    toks, _, _ = sess.generate(g["prompt"], len(g["greedy"]))
    assert toks.tolist() == g["greedy"].tolist()
    sess.close()
    sess = G.tiny_session()
    sess.hip(0)
    for pos in range(len(g["logits"])):
        lg = sess.forward(int(g["prompt"][pos]), pos)
        assert npref.rel_l2(lg, g["logits"][pos].astype(np.float64)) < 1e-3, pos
    sess.close()


def tokens_line(stdout):
    line = [ln for ln in stdout.splitlines() if ln.startswith("tokens:")][-1]
    return [int(v) for v in line.split()[1:]]


def sure_steps(g):
    low = g["margins"] < 5e-3
    return int(np.argmax(low)) if np.any(low) else len(g["margins"])


@pytest.mark.gpu
@pytest.mark.parametrize("batched", [0, 1])
def test_hip_cli_greedy_completion_matches_fixture(tmp_path, batched):
    # yalm <file> -p <ids> -t 0 -n 32 [-b 1]: the command-line completion on the HIP device.
    g = load("tiny")
    out = tmp_path / "tiny.yalm"
    r = subprocess.run([cli(), "--synth", str(out), "tiny"], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr
    ids = ",".join(str(int(v)) for v in g["prompt"])
    r = subprocess.run([cli(), str(out), "-p", ids, "-t", "0", "-n", str(len(g["greedy"])), "-b", str(batched)],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    toks = tokens_line(r.stdout)
    assert toks[:len(g["prompt"])] == g["prompt"].tolist()
    gen = toks[len(g["prompt"]):]
    n = len(g["greedy"]) if not batched else sure_steps(g)
    assert gen[:n] == g["greedy"][:n].tolist()


@pytest.mark.gpu
def test_hip_session_batched_prefill_generate_matches_fixture():
    g = load("tiny")
    sess = G.tiny_session()
    sess.hip(0)
    toks, _, _ = sess.generate(g["prompt"], len(g["greedy"]), prefill=True)
    n = sure_steps(g)
    assert toks[:n].tolist() == g["greedy"][:n].tolist()
    lg = sess.prefill(g["prompt"][:4])  # restart at 0: overwrites positions 0-3 and returns position 3's logits
    assert npref.rel_l2(lg, g["logits"][3].astype(np.float64)) < 1e-2
    sess.close()


@pytest.mark.gpu
def test_hip_prefill_tiny_matches_fixture():
    # Batched MFMA prefill of the prompt, then device-greedy decode. Prefill feeds fp16 activations
    # to its GEMMs, so its logits and K/V sit within the prefill tolerance (rel-L2 1e-2) rather than
    # fp32 noise; the greedy tokens must agree up to the first step whose top-2 margin is below 5e-3.
    g = load("tiny")
    cfg, t = tiny_weights()
    n_sure = sure_steps(g)
    assert n_sure >= 16
    with _hip().HipModel(cfg, t) as hm:
        lg = hm.prefill(g["prompt"])
        pos = len(g["prompt"])
        nxt = O.argmax(lg)
        out = [nxt]
        for _ in range(len(g["greedy"]) - 1):
            nxt = hm.forward_argmax(nxt, pos)
            out.append(nxt)
            pos += 1
        assert out[:n_sure] == g["greedy"][:n_sure].tolist()
    with _hip().HipModel(cfg, t) as hm:
        prompt = np.concatenate([g["prompt"], g["greedy"]]).astype(np.int32)
        hm.prefill(prompt)
        k, v = tiny_kv0(*hm.kv(0), cfg, int(g["n_written"]))
        for a, b in ((k, g["k0"]), (v, g["v0"])):
            assert np.array_equal(a != 0, b != 0)  # same entries written
            fa, fb = h2f(a), h2f(b)
            assert npref.rel_l2(fa, fb) < 1e-2
            assert np.max(np.abs(fa - fb)) <= 3e-2 * np.max(np.abs(fb))
