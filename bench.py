#!/usr/bin/env python3
"""Batch-1 fp16 decode benchmark on one MI355X, Mistral-7B-shaped random-init weights.

    python bench.py [--steps K] [--warmup W] [--workload decode|long|attn] [--path single|graph|direct]

Workloads (synthetic, seeded; no checkpoint download):
  decode  dim 4096, hidden 14336, 32 layers, 32/8 heads, vocab 32000, ctx 4096: 32 prompt ids then
          K greedy tokens (default 120). This is the headline line.
  long    same model; a 3200-token prompt prefilled in one batched call (MFMA GEMMs + causal MFMA
          attention; reported separately as prefill tok/s, TFLOP/s and matrix-core utilisation),
          then K greedy tokens at kv ~3200.
  attn    same model at ctx 16448 with the KV cache pre-filled ~N(0,1) to 16384 positions, then K
          greedy tokens at kv ~16400.

A step is one decode token: the reference loop's sample -> Model::forward (src/main.cpp:182-192),
greedy, with the argmax taken on the device. W untimed warm-up steps run first on a throwaway
sequence; then the prompt is hydrated again (untimed) and exactly K steps are timed with a steady
clock around each step (every step ends with a stream synchronisation).

Printed JSON line extras:
  roofline      the dominant kernel (fused RMSNorm + W1/W3 + SwiGLU matvec, 234.9 MB of fp16 weights
                per launch) timed live with HIP events on its launch stream over rotating weight copies
  step_roofline algorithmic bytes per token (all weights once + K/V read + K/V write) / step time
  cpu_baseline  the CPU oracle (a restatement of the reference -d cpu path, OpenMP over all host
                cores) on the same host weights, over a bounded sample of the same workload
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "batch-1 decode tok/s, Mistral-7B-shape fp16; % of 8 TB/s HBM roofline"
PEAK_GBS = 8000.0
WEIGHT_BYTES = 14_221_860_864       # all layer weights + lm_head + one embedding row + fp32 gains
KV_BYTES_PER_POS = 131_072          # 32 layers x 8 kv heads x 128 x (K + V) x 2 bytes
W13_BYTES = 2 * 14336 * 4096 * 2 + 4096 * 4 * 2 + 14336 * 4  # weights + x + gain + hb out
PEAK_FP16_TFLOPS = 2500.0  # MI355X dense fp16 matrix peak


def prefill_flops(cfg, n, start=0):
    """Dense matmul FLOPs of n prompt tokens through every layer (2 per weight per token) plus the
    causal attention (QK^T and PV: 4 * head_dim * n_heads per key-query pair)."""
    d, hid, hd, nh, nkv = cfg["dim"], cfg["hidden_dim"], cfg["head_dim"], cfg["n_heads"], cfg["n_kv_heads"]
    w_layer = (nh * hd + 2 * nkv * hd) * d + d * nh * hd + 3 * d * hid
    pairs = sum(start + i + 1 for i in range(n))
    return cfg["n_layers"] * (2.0 * n * w_layer + 4.0 * hd * nh * pairs)


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def bytes_per_token(kv_len):
    return WEIGHT_BYTES + KV_BYTES_PER_POS * kv_len + KV_BYTES_PER_POS


def cpu_baseline(session, cfg, prompt, gpu_tokens, budget_s):
    """The oracle on the host cores: hydrate the prompt, then greedy decode until the budget ends."""
    from oracle import binding as O  # the checker, timed here as the CPU baseline
    ocfg = dict(cfg)
    om = O.OracleModel(ocfg, session.tensors())
    t0 = time.perf_counter()
    lg = None
    for i, tok in enumerate(prompt):
        lg = om.forward(int(tok), i, 1 if i == len(prompt) - 1 else 0)
    hydrate = time.perf_counter() - t0
    steps, spent, toks = 0, 0.0, []
    pos = len(prompt)
    nxt = O.argmax(lg)
    while spent < budget_s and steps < len(gpu_tokens):
        toks.append(nxt)
        s = time.perf_counter()
        lg = om.forward(int(nxt), pos)
        nxt = O.argmax(lg)
        spent += time.perf_counter() - s
        steps += 1
        pos += 1
    om.close()
    match = 0
    for a, b in zip(toks, gpu_tokens):
        if a != b:
            break
        match += 1
    cores = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    return {
        "value": round(steps / spent, 4) if spent > 0 else None,
        "unit": "tok/s",
        "cores": cores,
        "kind": "port",
        "sample": f"{len(prompt)}-token prompt hydrated ({hydrate:.1f} s), then {steps} greedy decode steps "
                  f"timed ({spent:.1f} s) on the same weights; greedy tokens equal to the GPU's for the first "
                  f"{match} of {steps}",
        "greedy_match": match,
    }


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--workload", choices=["decode", "long", "attn"], default="decode")
    ap.add_argument("--path", choices=["graph", "single", "direct"], default="graph",
                    help="graph: per-op kernels replayed from a captured hipGraph; single: one launch per token "
                         "(dataflow of workgroups); direct: the per-op kernels launched one by one")
    ap.add_argument("--cpu-seconds", type=float, default=15.0, help="CPU-baseline decode budget (0 = skip)")
    ap.add_argument("--kernel-reps", type=int, default=200)
    ap.add_argument("--attn-min-slice", type=int, default=0, help="override the attention slice floor")
    ap.add_argument("--option", action="append", default=[], metavar="KEY=VALUE",
                    help="a context option of the HIP library (yhip_set_option), repeatable")
    ap.add_argument("--profile-kernel", choices=["w13", "copy"], default=None,
                    help="run only that kernel (for hardware-counter passes) and exit")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py runs on one GPU only: this build has no multi-GPU path (the sharding design is "
              "described in DESIGN.md); rerun with --gpus 1", file=sys.stderr)
        sys.exit(2)

    from yalm_amd import hip, host

    if args.profile_kernel:
        # W1/W3 (2 x 14336 x 4096 fp16) or a plain copy of the same 234.9 MB; 7 rotating copies
        kind = 2 if args.profile_kernel == "w13" else 5
        rows = 14336 if kind == 2 else 2 * 14336
        us = hip.bench_kernel(kind, rows, 4096, copies=7, warmup=2, reps=args.kernel_reps)
        print(json.dumps({"kernel": args.profile_kernel, "us_per_launch": round(us, 3), "reps": args.kernel_reps}))
        return

    wl = args.workload
    steps = args.steps if args.steps is not None else {"decode": 120, "long": 30, "attn": 64}[wl]
    ctx_len = 16448 if wl == "attn" else 4096
    n_prompt = {"decode": 32, "long": 3200, "attn": 1}[wl]
    prompt_seed = {"decode": 32, "long": 3200, "attn": 16385}[wl]
    shape = dict(host.MISTRAL_7B)

    t0 = time.perf_counter()
    sess = host.Session.synthetic(shape, context=ctx_len)
    cfg = sess.config()
    log(f"[bench] synthetic Mistral-7B-shape model built in {time.perf_counter() - t0:.1f} s")
    t0 = time.perf_counter()
    sess.hip(0)
    log(f"[bench] weights uploaded in {time.perf_counter() - t0:.1f} s")
    ctxp = sess.hip_ctx()
    opts = [(b"single_launch", int(args.path == "single")), (b"graph", int(args.path == "graph"))]
    if args.attn_min_slice:
        opts.append((b"attn_min_slice", args.attn_min_slice))
    for kv in args.option:
        key, _, val = kv.partition("=")
        opts.append((key.encode(), int(val)))
    for key, val in opts:
        if hip.lib().yhip_set_option(ctxp, key, val) != 0:
            raise RuntimeError(hip.lib().yhip_last_error(ctxp).decode())

    prompt = host.uniform_ids(n_prompt, prompt_seed, cfg["vocab_size"])
    start_pos = 0
    if wl == "attn":
        # KV cache pre-filled ~N(0,1) fp16 at positions [0, 16384) for every layer, written into the
        # reference layout through the C-ABI; decoding starts at position 16384.
        n = cfg["n_kv_heads"] * cfg["head_dim"] * cfg["max_seq_len"]
        fill_pos = 16384
        rng = np.random.default_rng(16384)
        for layer in range(cfg["n_layers"]):
            k = rng.standard_normal(n, dtype=np.float32).astype(np.float16).view(np.uint16)
            v = rng.standard_normal(n, dtype=np.float32).astype(np.float16).view(np.uint16)
            hd, msl = cfg["head_dim"], cfg["max_seq_len"]
            # zero the slots past the prefill in both layouts (positions >= fill_pos)
            kk = k.reshape(cfg["n_kv_heads"], hd // 16, msl, 16)
            kk[:, :, fill_pos:, :] = 0
            vv = v.reshape(cfg["n_kv_heads"], hd, msl)
            vv[:, :, fill_pos:] = 0
            rc = hip.lib().yhip_kv_write(ctxp, layer, k.ctypes.data_as(hip._u16p), v.ctypes.data_as(hip._u16p))
            if rc != 0:
                raise RuntimeError(hip.lib().yhip_last_error(ctxp).decode())
        start_pos = fill_pos
        log(f"[bench] KV cache pre-filled to {fill_pos} positions")

    prefill = None
    if wl == "long":
        view = hip.HipModel.attach(ctxp, cfg)
        view.prefill(prompt[:256])  # warm-up (kernels loaded, workspace sized)
        view.prefill(prompt)
        t0 = time.perf_counter()
        lg = view.prefill(prompt)
        pf_s = time.perf_counter() - t0
        fl = prefill_flops(cfg, n_prompt)
        prefill = {"tokens": n_prompt, "seconds": round(pf_s, 5), "tok_s": round(n_prompt / pf_s, 1),
                   "tflops": round(fl / pf_s / 1e12, 1), "mfma_frac": round(fl / pf_s / 1e12 / PEAK_FP16_TFLOPS, 4),
                   "flops": fl, "peak_tflops": PEAK_FP16_TFLOPS}
        log(f"[bench] prefill {n_prompt} tokens: {pf_s * 1e3:.1f} ms = {n_prompt / pf_s:.0f} tok/s, "
            f"{fl / pf_s / 1e12:.0f} TFLOP/s ({100 * fl / pf_s / 1e12 / PEAK_FP16_TFLOPS:.1f}% of fp16 peak)")
        first_tok = int(np.argmax(lg))

    def run(n_steps):
        if wl == "long":
            # greedy decode from the prefilled cache
            toks, secs = [], []
            tok = first_tok
            view = hip.HipModel.attach(ctxp, cfg)
            for i in range(n_steps):
                s = time.perf_counter()
                tok = view.forward_argmax(tok, n_prompt + i)
                secs.append(time.perf_counter() - s)
                toks.append(tok)
            return np.array(toks), np.array(secs), 0.0
        if wl != "attn":
            return sess.generate(prompt, n_steps, temperature=0.0, device_argmax=True)
        # decode directly from position 16384 with greedy argmax on the device
        toks, secs = [], []
        tok = int(prompt[0])
        view = hip.HipModel.attach(ctxp, cfg)
        for i in range(n_steps):
            s = time.perf_counter()
            tok = view.forward_argmax(tok, start_pos + i)
            secs.append(time.perf_counter() - s)
            toks.append(tok)
        return np.array(toks), np.array(secs), 0.0

    log(f"[bench] warm-up: {args.warmup} steps")
    run(max(args.warmup, 1))
    log(f"[bench] timed: {steps} steps")
    view = hip.HipModel.attach(ctxp, cfg)
    view.set_option("stats", 1)  # HIP events around each step's kernels on the context's stream
    toks, secs, hydrate_s = run(steps)
    dev_us, dev_steps = view.step_stats()
    view.set_option("stats", 0)
    assert len(secs) == steps, "decode stopped early"
    total = float(np.sum(secs))
    tok_s = steps / total
    first = start_pos + n_prompt
    kv_mean = first + (steps - 1) / 2.0 + 1
    step_bytes = bytes_per_token(kv_mean)
    step_gbs = step_bytes * tok_s / 1e9
    log(f"[bench] {tok_s:.1f} tok/s ({1e3 * total / steps:.3f} ms/step), {step_gbs:.0f} GB/s algorithmic")

    # device time per timed step (HIP events on the decode stream)
    step_us = dev_us / max(dev_steps, 1)
    log(f"[bench] device time per step: {step_us:.1f} us over {dev_steps} steps "
        f"({step_bytes / (step_us * 1e-6) / 1e9:.0f} GB/s algorithmic)")

    # fused rmsnorm + W1/W3 + SwiGLU matvec, timed on its own stream with HIP events over rotating
    # weight copies (7 x 235 MB, far beyond the 256 MB last-level cache)
    us = hip.bench_kernel(2, 14336, 4096, copies=7, warmup=20, reps=args.kernel_reps)
    w13_gbs = W13_BYTES / (us * 1e-6) / 1e9
    log(f"[bench] fused rmsnorm+W1/W3+SwiGLU: {us:.2f} us/launch, {w13_gbs:.0f} GB/s")

    cpu = None
    if args.cpu_seconds > 0 and wl == "decode":
        log(f"[bench] CPU baseline (oracle, {args.cpu_seconds:.0f} s decode budget)")
        cpu = cpu_baseline(sess, cfg, prompt, [int(t) for t in toks], args.cpu_seconds)
        log(f"[bench] CPU: {cpu['value']} tok/s on {cpu['cores']} cores; {cpu['sample']}")

    def traffic_of(name):
        tf = os.path.join(ROOT, "profiles", name)
        if os.path.exists(tf):
            with open(tf) as f:
                return json.load(f).get("bytes_per_launch")
        return None

    w13 = {"bound": "hbm", "achieved": round(w13_gbs, 1), "peak": PEAK_GBS, "unit": "GB/s",
           "frac": round(w13_gbs / PEAK_GBS, 4), "traffic": traffic_of("w13_swiglu_traffic.json"),
           "kernel": "matvec_kernel<8,2> as rmsnorm + W1/W3 + SwiGLU (14336 x 4096 x 2)",
           "bytes_per_launch": W13_BYTES, "us_per_launch": round(us, 3)}
    if args.path == "single":
        # one launch per token: the dominant kernel is the whole step
        achieved = step_bytes / (step_us * 1e-6) / 1e9
        roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_GBS, "unit": "GB/s",
                    "frac": round(achieved / PEAK_GBS, 4), "traffic": traffic_of("decode_step_traffic.json"),
                    "kernel": "decode_flow_kernel<128,4> (the whole token, one launch)",
                    "bytes_per_launch": int(step_bytes), "us_per_launch": round(step_us, 3)}
    else:
        roofline = w13

    out = {
        "metric": METRIC,
        "value": round(tok_s, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": round(1e3 * total / steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic",
        "config": {
            "workload": {"decode": "Mistral-7B-shape fp16 decode: 32 random prompt ids then greedy tokens, ctx 4096",
                         "long": "Mistral-7B-shape fp16 decode after a 3200-token batched prefill, ctx 4096",
                         "attn": "Mistral-7B-shape fp16 decode over a KV cache pre-filled to 16384, ctx 16448"}[wl],
            "dim": 4096, "hidden_dim": 14336, "n_layers": 32, "n_heads": 32, "n_kv_heads": 8, "head_dim": 128,
            "vocab": 32000, "context": ctx_len, "prompt_tokens": n_prompt, "global_batch": 1,
            "accumulate": "fp32", "activations": "fp32", "path": args.path, "parallelism": "none (1 GPU)",
        },
        "step_roofline": {"bytes_per_token": int(step_bytes), "achieved_GBps": round(step_gbs, 1),
                          "peak_GBps": PEAK_GBS, "frac": round(step_gbs / PEAK_GBS, 4), "kv_len_mean": kv_mean},
        "roofline": roofline,
        "w13_kernel": w13,
        "device_us_per_step": round(step_us, 2),
        "cpu_baseline": cpu,
    }
    if args.option:
        out["config"]["options"] = dict(kv.partition("=")[::2] for kv in args.option)
    if prefill is not None:
        out["prefill"] = prefill
    print(json.dumps(out), flush=True)
    sess.close()


if __name__ == "__main__":
    main()
