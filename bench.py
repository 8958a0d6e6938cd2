#!/usr/bin/env python3
"""Batch-1 fp16 decode benchmark on one MI355X, Mistral-7B-shaped random-init weights.

    python bench.py [--steps K] [--warmup W] [--workload decode|long|attn] [--path single|graph|direct]

Workloads (synthetic, seeded; no checkpoint download):
  decode  dim 4096, hidden 14336, 32 layers, 32/8 heads, vocab 32000, ctx 4096: 32 prompt ids then
          K greedy tokens (default 120). This is the headline line.
  long    same model; a 3200-token prompt prefilled in one batched call (MFMA GEMMs + causal MFMA
          attention; reported separately as prefill tok/s, TFLOP/s and matrix-core utilisation),
          then 30 greedy tokens at kv ~3200.
  attn    same model at ctx 16448 with the KV cache pre-filled ~N(0,1) on the device to 16384
          positions, then 64 greedy tokens at kv ~16400.
Without --workload the run is the headline decode line with the long and attn workloads appended as
extra keys ("long", "attn"), each with its own step_roofline.

A step is one decode token: the reference loop's sample -> Model::forward (src/main.cpp:182-192),
greedy, with the argmax taken on the device. W untimed warm-up steps run first on a throwaway
sequence; then the prompt is hydrated again (untimed) and exactly K steps are timed with a steady
clock around each step (every step ends with a stream synchronisation).

Printed JSON line extras:
  roofline      the dominant kernel (fused RMSNorm + W1/W3 + SwiGLU matvec, 234.9 MB of fp16 weights
                per launch) timed live with HIP events on its launch stream over rotating weight copies
  step_roofline algorithmic bytes per token (all weights once + K/V read + K/V write) / step time
  microbench    the per-layer kernels at the Mistral-7B shape (fused RMSNorm + QKV, O + residual,
                RMSNorm + W1/W3 + SwiGLU, W2 + residual, RMSNorm + lm_head), each timed with HIP
                events on its own stream over >= 1 GiB of rotating weight copies: microseconds,
                GB/s of algorithmic bytes, fraction of 8 TB/s, and the recorded traffic ratio
  tp8_shard     the same kernels at one GPU's share of an 8-way tensor-parallel split (QKV 768 rows,
                O 4096 x 512, W1/W3 1792 rows, W2 4096 x 1792, lm_head 4000 rows) and the attention
                of one kv head, measured on this GPU (no collectives: nothing here uses a second GPU)
  cpu_baseline  the CPU oracle (a restatement of the reference -d cpu path, OpenMP over the host
                cores given to this process) on the same host weights, over a bounded sample of the
                decode workload: decode tok/s, and the reference's own figure (prompt + generated
                tokens over hydrate + decode time, src/main.cpp:194-210)
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

# OpenMP placement of the CPU baseline, read by the OpenMP runtime when it first loads (with the
# native libraries below): threads on cores, packed. The thread count is the environment's own
# (OMP_NUM_THREADS, else the runtime's default of one per logical CPU of this process).
os.environ.setdefault("OMP_PROC_BIND", "close")
os.environ.setdefault("OMP_PLACES", "cores")

import numpy as np  # noqa: E402

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "batch-1 decode tok/s, Mistral-7B-shape fp16; % of 8 TB/s HBM roofline"
PEAK_GBS = 8000.0
WEIGHT_BYTES = 14_221_860_864       # all layer weights + lm_head + one embedding row + fp32 gains
KV_BYTES_PER_POS = 131_072          # 32 layers x 8 kv heads x 128 x (K + V) x 2 bytes
W13_BYTES = 2 * 14336 * 4096 * 2 + 4096 * 4 * 2 + 14336 * 4  # weights + x + gain + hb out
PEAK_FP16_TFLOPS = 2500.0  # MI355X dense fp16 matrix peak
GREEDY_CHECK = 32  # generated tokens the CPU baseline compares with the GPU's, at least

# The per-layer kernel workload at the Mistral-7B shape (fused RMSNorm feeding the fp16 matvecs):
# (name, yhip_bench_kernel kind, output rows, row length, RMSNorm on the input, residual added).
MICRO_KERNELS = [("qkv", 0, 6144, 4096, True, False), ("o", 1, 4096, 4096, False, True),
                 ("w13", 2, 14336, 4096, True, False), ("w2", 3, 4096, 14336, False, True),
                 ("lm_head", 4, 32000, 4096, True, False)]
MICRO_WORKING_SET = 1 << 30  # rotating weight copies per kernel: at least 4 and at least 1 GiB in total
# One GPU's share of an 8-way tensor-parallel split of the same layer: kv head r and its 4 query
# heads (QKV rows 768), Wo by input columns (4096 x 512, partial x), W1/W3 by rows (1792), W2 by
# input columns (4096 x 1792, partial x), lm_head by vocabulary rows (4000)
TP8_KERNELS = [("qkv", 0, 768, 4096, True, False), ("o", 1, 4096, 512, False, True),
               ("w13", 2, 1792, 4096, True, False), ("w2", 3, 4096, 1792, False, True),
               ("lm_head", 4, 4000, 4096, True, False)]


def micro_bytes(kind, rows, cols, norm, resid):
    """Algorithmic bytes of one launch: fp16 weights once (W1 and W3 for kind 2), the fp32 input,
    the fp32 gain when normed, the fp32 outputs (SwiGLU: one per row pair), the residual read."""
    nmat = 2 if kind == 2 else 1
    return rows * cols * 2 * nmat + 4 * cols + (4 * cols if norm else 0) + 4 * rows + (4 * rows if resid else 0)


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


def step_roofline(kv_mean, tok_s):
    b = bytes_per_token(kv_mean)
    gbs = b * tok_s / 1e9
    return {"bytes_per_token": int(b), "achieved_GBps": round(gbs, 1), "peak_GBps": PEAK_GBS,
            "frac": round(gbs / PEAK_GBS, 4), "kv_len_mean": kv_mean}


def host_cpu():
    """CPU model, logical CPUs and physical cores this process may run on, and the OpenMP settings.
    Called at start-up: once the OpenMP runtime binds the main thread, its affinity is one core."""
    model = None
    try:
        import subprocess
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.startswith("Model name:"):
                model = line.split(":", 1)[1].strip()
                break
    except (OSError, subprocess.SubprocessError):
        pass
    if not model:
        try:
            with open("/proc/cpuinfo") as f:
                for line in f:
                    if line.startswith("model name"):
                        model = line.split(":", 1)[1].strip()
                        break
        except OSError:
            pass
    cpus = sorted(os.sched_getaffinity(0))
    cores = set()
    for c in cpus:
        try:
            base = f"/sys/devices/system/cpu/cpu{c}/topology/"
            with open(base + "physical_package_id") as f1, open(base + "core_id") as f2:
                cores.add((f1.read().strip(), f2.read().strip()))
        except OSError:
            cores.add(("?", str(c)))
    return {"model": model, "logical_cpus": len(cpus), "physical_cores": len(cores),
            "omp_num_threads": os.environ.get("OMP_NUM_THREADS"), "omp_proc_bind": os.environ.get("OMP_PROC_BIND"),
            "omp_places": os.environ.get("OMP_PLACES")}


HOST_CPU = host_cpu()


def cpu_baseline(session, cfg, prompt, gpu_tokens, budget_s):
    """The oracle on the host cores: hydrate the prompt, then greedy decode until the budget ends (or
    the context does); its first tokens are compared with the GPU's."""
    from oracle import binding as O  # the oracle, timed here as the CPU baseline
    om = O.OracleModel(dict(cfg), session.tensors())
    t0 = time.perf_counter()
    lg = None
    for i, tok in enumerate(prompt):
        lg = om.forward(int(tok), i, 1 if i == len(prompt) - 1 else 0)
    hydrate = time.perf_counter() - t0
    steps, spent, toks = 0, 0.0, []
    pos = len(prompt)
    nxt = O.argmax(lg)
    while spent < budget_s and pos < cfg["max_seq_len"]:
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
    compared = min(len(toks), len(gpu_tokens))
    hc = HOST_CPU
    threads = int(hc["omp_num_threads"] or hc["logical_cpus"])
    return {
        "value": round(steps / spent, 4) if spent > 0 else None,
        "unit": "tok/s",
        "cores": threads,
        "kind": "port",
        "sample": f"{len(prompt)}-token prompt hydrated ({hydrate:.1f} s), then {steps} greedy decode steps "
                  f"timed ({spent:.1f} s) on the same weights; greedy tokens equal to the GPU's for the first "
                  f"{match} of {compared} compared",
        "reference_style_tok_s": round((len(prompt) + steps) / (hydrate + spent), 4),
        "host": hc,
        "threads": threads,
        "greedy_match": match,
        "greedy_compared": compared,
    }


def timed_steps(view, first_tok, start_pos, n):
    """n greedy steps on the device from start_pos; per-step wall time."""
    toks, secs = [], []
    tok = first_tok
    for i in range(n):
        s = time.perf_counter()
        tok = view.forward_argmax(tok, start_pos + i)
        secs.append(time.perf_counter() - s)
        toks.append(tok)
    return np.array(toks), np.array(secs)


def run_long(hip, host, ctxp, cfg, steps=30, n_prompt=3200):
    """3200-token batched prefill, then greedy decode at kv ~3200 (the long-context workload)."""
    view = hip.HipModel.attach(ctxp, cfg)
    prompt = host.uniform_ids(n_prompt, 3200, cfg["vocab_size"])
    view.prefill(prompt[:256])  # warm-up (kernels loaded, workspace sized)
    view.prefill(prompt)
    t0 = time.perf_counter()
    lg = view.prefill(prompt)
    pf_s = time.perf_counter() - t0
    fl = prefill_flops(cfg, n_prompt)
    prefill = {"tokens": n_prompt, "ms": round(pf_s * 1e3, 3), "tok_s": round(n_prompt / pf_s, 1),
               "tflops": round(fl / pf_s / 1e12, 1), "mfma_frac": round(fl / pf_s / 1e12 / PEAK_FP16_TFLOPS, 4),
               "flops": fl, "peak_tflops": PEAK_FP16_TFLOPS}
    log(f"[bench] long: prefill {n_prompt} tokens {pf_s * 1e3:.1f} ms = {n_prompt / pf_s:.0f} tok/s, "
        f"{fl / pf_s / 1e12:.0f} TFLOP/s ({100 * fl / pf_s / 1e12 / PEAK_FP16_TFLOPS:.1f}% of the fp16 peak)")
    first = int(np.argmax(lg))
    timed_steps(view, first, n_prompt, 3)  # warm-up at this context length
    lg = view.prefill(prompt)  # the cache as the timed decode expects it
    toks, secs = timed_steps(view, int(np.argmax(lg)), n_prompt, steps)
    tok_s = steps / float(np.sum(secs))
    kv_mean = n_prompt + (steps - 1) / 2.0 + 1
    log(f"[bench] long: decode {tok_s:.1f} tok/s at kv ~{kv_mean:.0f}")
    return {"workload": "Mistral-7B-shape fp16: 3200-token batched prefill, then greedy decode, ctx 4096",
            "prefill": prefill, "decode_steps": steps, "decode_tok_s": round(tok_s, 2),
            "decode_ms_per_step": round(1e3 / tok_s, 4), "step_roofline": step_roofline(kv_mean, tok_s)}


def run_attn(hip, host, sess, cfg, steps=64, fill=16384, ctx_len=16448, opts=()):
    """KV cache pre-filled on the device to 16384 positions, greedy decode at kv ~16400."""
    c16 = dict(cfg, max_seq_len=ctx_len)
    t0 = time.perf_counter()
    m = hip.HipModel(c16, sess.tensors())
    for key, val in opts:  # the same context options as the headline context
        m.set_option(key.decode(), val)
    m.kv_fill_normal(fill, 16384)
    log(f"[bench] attn: context {ctx_len} set up, KV pre-filled to {fill} in {time.perf_counter() - t0:.1f} s")
    first = int(host.uniform_ids(1, 16385, cfg["vocab_size"])[0])
    timed_steps(m, first, fill, 3)  # warm-up (rewrites the same positions as the timed run)
    toks, secs = timed_steps(m, first, fill, steps)
    m.close()
    tok_s = steps / float(np.sum(secs))
    kv_mean = fill + (steps - 1) / 2.0 + 1
    log(f"[bench] attn: decode {tok_s:.1f} tok/s at kv ~{kv_mean:.0f}")
    return {"workload": "Mistral-7B-shape fp16 decode over a KV cache pre-filled to 16384, ctx 16448",
            "decode_steps": steps, "decode_tok_s": round(tok_s, 2), "decode_ms_per_step": round(1e3 / tok_s, 4),
            "step_roofline": step_roofline(kv_mean, tok_s)}


def recorded_traffic():
    """Per-kernel HBM traffic over algorithmic bytes, recorded from rocprofv3 FETCH_SIZE/WRITE_SIZE
    passes of `bench.py --profile-kernel micro` (copy-calibrated); {} when not recorded."""
    tf = os.path.join(ROOT, "profiles", "microbench_traffic.json")
    if not os.path.exists(tf):
        return {}
    with open(tf) as f:
        return json.load(f).get("kernels", {})


def run_microbench(hip, reps, warmup=20, kernels=MICRO_KERNELS, label="microbench", recorded=True):
    """Each per-layer kernel on its own stream, HIP-event timed over rotating weight copies."""
    traffic = recorded_traffic() if recorded else {}
    out = {}
    for name, kind, rows, cols, norm, resid in kernels:
        wbytes = rows * cols * 2 * (2 if kind == 2 else 1)
        copies = max(4, -(-MICRO_WORKING_SET // wbytes))
        us = hip.bench_kernel(kind, rows, cols, copies=copies, warmup=warmup, reps=reps)
        alg = micro_bytes(kind, rows, cols, norm, resid)
        gbs = alg / (us * 1e-6) / 1e9
        rec = traffic.get(name)
        out[name] = {"shape": f"{rows}x{cols}" + (" x2" if kind == 2 else ""), "us_per_launch": round(us, 3),
                     "bytes_per_launch": alg, "GBps": round(gbs, 1), "frac": round(gbs / PEAK_GBS, 4),
                     "copies": copies, "traffic_ratio_recorded": rec.get("ratio") if rec else None}
        log(f"[bench] {label} {name} {rows}x{cols}: {us:.2f} us/launch, {gbs:.0f} GB/s "
            f"({100 * gbs / PEAK_GBS:.1f}% of 8 TB/s)")
    if recorded:
        out["traffic_source"] = ("profiles/microbench_traffic.json: recorded rocprofv3 FETCH_SIZE / WRITE_SIZE "
                                 "passes of these launches, scaled by a plain copy's counters" if traffic else None)
    return out


def run_tp8_shard(hip, reps, warmup=20):
    """One GPU's share of an 8-way tensor-parallel decode step, measured on this GPU: the per-layer
    kernels at their shard shapes and the attention of one kv head (4 query heads) at the three
    workloads' context lengths; the collectives (two 16 KB all-reduces of x per layer) are not
    measured here."""
    out = run_microbench(hip, reps, warmup, TP8_KERNELS, "tp8 shard", recorded=False)
    attn = {}
    for kv in (92, 3216, 16417):
        msl = 16448 if kv > 4096 else 4096
        attn[str(kv)] = round(hip.bench_attention(kv, max_seq_len=msl, nsplit=0, min_slice=0, n_heads=4, n_kv_heads=1,
                                                  warmup=warmup, reps=reps), 3)
        log(f"[bench] tp8 shard attention, 1 kv head, kv {kv}: {attn[str(kv)]:.2f} us/launch")
    out["attention_us_one_kv_head"] = attn
    layer = sum(out[k]["us_per_launch"] for k in ("qkv", "o", "w13", "w2"))
    out["layer_matvec_us"] = round(layer, 3)
    out["token_ms_without_collectives_kv92"] = round((32 * (layer + attn["92"]) + out["lm_head"]["us_per_launch"]) / 1e3, 4)
    out["note"] = ("kernels at one GPU's share of an 8-way split (QKV 768x4096, O 4096x512, W1/W3 1792x4096, "
                   "W2 4096x1792, lm_head 4000x4096, attention of one kv head), each timed alone; no collectives")
    return out


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--workload", choices=["decode", "long", "attn"], default=None,
                    help="one workload only (default: the decode headline with long and attn as extra keys)")
    ap.add_argument("--path", choices=["graph", "single", "direct"], default="graph",
                    help="graph: per-op kernels replayed from a captured hipGraph; single: one launch per token "
                         "(a cooperative persistent kernel, one workgroup per CU); direct: the per-op kernels launched one by one")
    ap.add_argument("--cpu-seconds", type=float, default=15.0, help="CPU-baseline decode budget (0 = skip)")
    ap.add_argument("--kernel-reps", type=int, default=200)
    ap.add_argument("--attn-min-slice", type=int, default=0, help="override the attention slice floor")
    ap.add_argument("--option", action="append", default=[], metavar="KEY=VALUE",
                    help="a context option of the HIP library (yhip_set_option), repeatable")
    ap.add_argument("--profile-kernel", choices=["w13", "copy", "micro"], default=None,
                    help="run only that kernel (micro: the five per-layer kernels, then the copy) for "
                         "hardware-counter passes, and exit")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py runs on one GPU only: there is no multi-GPU path (the decode step is measured "
              "on one GPU's share); rerun with --gpus 1", file=sys.stderr)
        sys.exit(2)

    from yalm_amd import hip, host

    if args.profile_kernel == "micro":
        res = {name: round(hip.bench_kernel(kind, rows, cols, copies=4, warmup=2, reps=args.kernel_reps), 3)
               for name, kind, rows, cols, _, _ in MICRO_KERNELS}
        res["copy"] = round(hip.bench_kernel(5, 2 * 14336, 4096, copies=4, warmup=2, reps=args.kernel_reps), 3)
        print(json.dumps({"kernel": "micro", "us_per_launch": res, "reps": args.kernel_reps}))
        return
    if args.profile_kernel:
        # W1/W3 (2 x 14336 x 4096 fp16) or a plain copy of the same 234.9 MB; 7 rotating copies
        kind = 2 if args.profile_kernel == "w13" else 5
        rows = 14336 if kind == 2 else 2 * 14336
        us = hip.bench_kernel(kind, rows, 4096, copies=7, warmup=2, reps=args.kernel_reps)
        print(json.dumps({"kernel": args.profile_kernel, "us_per_launch": round(us, 3), "reps": args.kernel_reps}))
        return

    wl = args.workload or "decode"
    extras = args.workload is None
    steps = args.steps if args.steps is not None else {"decode": 120, "long": 30, "attn": 64}[wl]
    shape = dict(host.MISTRAL_7B)

    t0 = time.perf_counter()
    sess = host.Session.synthetic(shape, context=4096)
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

    if wl == "long":
        res = run_long(hip, host, ctxp, cfg, steps)
        print(json.dumps({"metric": METRIC, "value": res["decode_tok_s"], "unit": "tok/s", "n_gpus": 1,
                          "steps": steps, "warmup": 3, "ms_per_step": res["decode_ms_per_step"],
                          "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "fp16",
                          "data": "synthetic", "config": {"workload": res["workload"], "path": args.path}, **res}))
        sess.close()
        return
    if wl == "attn":
        res = run_attn(hip, host, sess, cfg, steps, opts=opts)
        print(json.dumps({"metric": METRIC, "value": res["decode_tok_s"], "unit": "tok/s", "n_gpus": 1,
                          "steps": steps, "warmup": 3, "ms_per_step": res["decode_ms_per_step"],
                          "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "fp16",
                          "data": "synthetic", "config": {"workload": res["workload"], "path": args.path}, **res}))
        sess.close()
        return

    # ---- the headline: 32 prompt ids, then greedy decode at ctx 4096 ----
    n_prompt = 32
    prompt = host.uniform_ids(n_prompt, 32, cfg["vocab_size"])
    log(f"[bench] warm-up: {args.warmup} steps")
    sess.generate(prompt, max(args.warmup, 1), temperature=0.0, device_argmax=True)
    log(f"[bench] timed: {steps} steps")
    view = hip.HipModel.attach(ctxp, cfg)
    view.set_option("stats", 1)  # HIP events around each step's kernels on the context's stream
    toks, secs, hydrate_s = sess.generate(prompt, steps, temperature=0.0, device_argmax=True)
    dev_us, dev_steps = view.step_stats()
    view.set_option("stats", 0)
    assert len(secs) == steps, "decode stopped early"
    total = float(np.sum(secs))
    tok_s = steps / total
    kv_mean = n_prompt + (steps - 1) / 2.0 + 1
    sr = step_roofline(kv_mean, tok_s)
    log(f"[bench] {tok_s:.1f} tok/s ({1e3 * total / steps:.3f} ms/step), {sr['achieved_GBps']:.0f} GB/s algorithmic")
    step_us = dev_us / max(dev_steps, 1)
    step_bytes = bytes_per_token(kv_mean)
    log(f"[bench] device time per step: {step_us:.1f} us over {dev_steps} steps "
        f"({step_bytes / (step_us * 1e-6) / 1e9:.0f} GB/s algorithmic)")

    # fused rmsnorm + W1/W3 + SwiGLU matvec, timed on its own stream with HIP events over rotating
    # weight copies (7 x 235 MB, far beyond the 256 MB last-level cache)
    us = hip.bench_kernel(2, 14336, 4096, copies=7, warmup=20, reps=args.kernel_reps)
    w13_gbs = W13_BYTES / (us * 1e-6) / 1e9
    log(f"[bench] fused rmsnorm+W1/W3+SwiGLU: {us:.2f} us/launch, {w13_gbs:.0f} GB/s")
    micro = run_microbench(hip, args.kernel_reps)
    tp8 = run_tp8_shard(hip, args.kernel_reps)

    # what the step's launch structure allows: the same weight bytes through memory-only launches
    # of the same sizes and order (matvec access pattern), and through one launch
    ms_seq, ms_one = hip.bench_stream(cfg, reps=5)
    weights = WEIGHT_BYTES
    ceiling = {"ms_per_token": round(ms_seq, 4), "tok_s": round(1e3 / ms_seq, 1),
               "GBps": round(weights / (ms_seq * 1e-3) / 1e9, 1),
               "one_launch_ms": round(ms_one, 4), "one_launch_tok_s": round(1e3 / ms_one, 1),
               "value_frac": round(tok_s / (1e3 / ms_seq), 4),
               "note": "memory-only streaming launches with the decode step's weight bytes per launch "
                       "(129 launches) and as one launch"}
    log(f"[bench] launch-structure ceiling: {ms_seq:.3f} ms/token ({1e3 / ms_seq:.0f} tok/s), one launch "
        f"{ms_one:.3f} ms ({1e3 / ms_one:.0f} tok/s); decode at {100 * ceiling['value_frac']:.1f}% of the first")

    extra = {}
    if extras:
        extra["long"] = run_long(hip, host, ctxp, cfg)
        extra["attn"] = run_attn(hip, host, sess, cfg, opts=opts)

    cpu = None
    if args.cpu_seconds > 0:
        log(f"[bench] CPU baseline (oracle, {args.cpu_seconds:.0f} s decode budget)")
        gpu_toks = [int(t) for t in toks]
        if len(gpu_toks) < GREEDY_CHECK:  # the greedy contract covers the first 32 generated tokens
            more, _, _ = sess.generate(prompt, GREEDY_CHECK, temperature=0.0, device_argmax=True)
            gpu_toks = [int(t) for t in more]
        cpu = cpu_baseline(sess, cfg, prompt, gpu_toks, args.cpu_seconds)
        log(f"[bench] CPU: {cpu['value']} tok/s on {cpu['cores']} threads ({cpu['host']['model']}); {cpu['sample']}")

    def traffic_of(name):
        tf = os.path.join(ROOT, "profiles", name)
        if os.path.exists(tf):
            with open(tf) as f:
                return json.load(f).get("bytes_per_launch")
        return None

    w13 = {"bound": "hbm", "achieved": round(w13_gbs, 1), "peak": PEAK_GBS, "unit": "GB/s",
           "frac": round(w13_gbs / PEAK_GBS, 4), "traffic": traffic_of("w13_swiglu_traffic.json"),
           "traffic_kind": "recorded: profiles/w13_swiglu_traffic.json (rocprofv3 FETCH_SIZE + WRITE_SIZE "
                           "per dispatch, copy-calibrated), not measured in this run",
           "kernel": "matvec_kernel<8,2> as rmsnorm + W1/W3 + SwiGLU (14336 x 4096 x 2)",
           "bytes_per_launch": W13_BYTES, "us_per_launch": round(us, 3)}
    if args.path == "single":
        # one launch per token: the dominant kernel is the whole step
        achieved = step_bytes / (step_us * 1e-6) / 1e9
        roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_GBS, "unit": "GB/s",
                    "frac": round(achieved / PEAK_GBS, 4), "traffic": traffic_of("decode_step_traffic.json"),
                    "traffic_kind": "recorded (profiles/decode_step_traffic.json), not measured in this run",
                    "kernel": "decode_step_kernel<128,4,8,14> (the whole token, one cooperative launch)",
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
            "workload": "Mistral-7B-shape fp16 decode: 32 random prompt ids then greedy tokens, ctx 4096",
            "dim": 4096, "hidden_dim": 14336, "n_layers": 32, "n_heads": 32, "n_kv_heads": 8, "head_dim": 128,
            "vocab": 32000, "context": 4096, "prompt_tokens": n_prompt, "global_batch": 1,
            "accumulate": "fp32", "activations": "fp32", "path": args.path, "parallelism": "none (1 GPU)",
        },
        "step_roofline": sr,
        "reference_style_tok_s": round((n_prompt + steps) / (hydrate_s + total), 2),
        "roofline": roofline,
        "w13_kernel": w13,
        "microbench": micro,
        "tp8_shard": tp8,
        "device_us_per_step": round(step_us, 2),
        "launch_ceiling": ceiling,
        "cpu_baseline": cpu,
        **extra,
    }
    if args.option:
        out["config"]["options"] = dict(kv.partition("=")[::2] for kv in args.option)
    print(json.dumps(out), flush=True)
    sess.close()


if __name__ == "__main__":
    main()
