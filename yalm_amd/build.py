"""In-tree build of the native libraries (no cmake): hipcc for the gfx950 kernels, g++ for the host.

    python -m yalm_amd.build        # builds everything under yalm_amd/ and oracle/

Outputs (git-ignored, shipped with the tree):
    yalm_amd/libyalm_hip.so     HIP kernels + C-ABI (include/yalm_hip.h)
    yalm_amd/libyalm_host.so    C++ host: codec, Model/InferenceState (Device::HIP), sampler, tokenizer, synth
    yalm_amd/bin/yalm           CLI (reference main.cpp contract, -d hip)
"""
from __future__ import annotations

import os
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = os.environ.get("YALM_OFFLOAD_ARCH", "gfx950")

# Packed-FP32 instructions are kept out of every HIP build.
HIP_FLAGS = ["-O3", "-std=c++17", f"--offload-arch={ARCH}", "-fPIC", "-Wall", "-Wno-unused-value",
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
HOST_FLAGS = ["-O3", "-std=c++20", "-fPIC", "-Wall", "-Wextra", "-fopenmp"]


def _run(cmd):
    print("+", " ".join(cmd), flush=True)
    r = subprocess.run(cmd, cwd=ROOT, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError(f"build step failed: {' '.join(cmd[:3])} ...")
    noisy = [ln for ln in (r.stdout + r.stderr).splitlines() if "packed-fp32-ops" not in ln and ln.strip()]
    if noisy:
        sys.stderr.write("\n".join(noisy) + "\n")


def build_hip():
    src = os.path.join(PKG, "csrc", "yalm_hip.hip")
    out = os.path.join(PKG, "libyalm_hip.so")
    _run([HIPCC, *HIP_FLAGS, "-shared", "-o", out, src])
    return out


def build_host():
    hdir = os.path.join(PKG, "host")
    if not os.path.isdir(hdir):
        return None
    srcs = sorted(os.path.join(hdir, f) for f in os.listdir(hdir) if f.endswith(".cpp") and f != "main.cpp")
    if not srcs:
        return None
    lib = os.path.join(PKG, "libyalm_host.so")
    inc = ["-I", os.path.join(ROOT, "include"), "-I", hdir]
    _run(["g++", *HOST_FLAGS, *inc, "-shared", "-o", lib, *srcs, "-L", PKG, "-lyalm_hip", "-Wl,-rpath,$ORIGIN"])
    main = os.path.join(hdir, "main.cpp")
    if os.path.exists(main):
        os.makedirs(os.path.join(PKG, "bin"), exist_ok=True)
        _run(["g++", *HOST_FLAGS, *inc, "-o", os.path.join(PKG, "bin", "yalm"), main, "-L", PKG, "-lyalm_host",
              "-lyalm_hip", "-Wl,-rpath,$ORIGIN/.."])
    return lib


def build_oracle():
    _run(["make", "-B", "-s", "-C", os.path.join(ROOT, "oracle")])


def build_all():
    build_hip()
    build_host()
    build_oracle()


if __name__ == "__main__":
    build_all()
