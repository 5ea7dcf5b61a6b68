"""Builds libmidman_hip.so for gfx950 in-tree (midman-ai_amd/libmidman_hip.so).

HIP sources are compiled with hipcc for gfx950 only; the host-only sources
(error handling, the RNG and rotary tables that must match the reference bit
for bit, SHA-256, the safetensors format, token shards and the batcher) are
compiled with g++ -ffp-contract=off. Objects go to midman-ai_amd/_build/.

    python midman-ai_amd/build.py [--jobs N]
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libmidman_hip.so")
ARCH = "gfx950"

HIP_SOURCES = ["runtime.hip", "gemm.hip", "rowops.hip", "attention.hip", "attention_bwd.hip",
               "train.hip", "checkpoint.hip", "model.hip", "noalloc.hip", "fused_forward.hip"]
# Host code with no HIP in it (also built with the sanitizers: build_sanitized.py)
HOST_SOURCES = ["host_errors.cpp", "host_math.cpp", "host_sha256.cpp", "host_safetensors.cpp",
                "host_data.cpp"]

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
HIP_FLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", "-Wall",
    "-Wno-unused-result",
    # No multiply-add contraction: element-wise ops round where the reference's
    # Rust code rounds (hipcc's default would fuse x*c - y*s into one FMA;
    # the __fmul_rn-style intrinsics are not a barrier against that).
    "-ffp-contract=off",
    # Packed FP32 instructions stay off: v_pk_{add,mul,fma}_f32 are not used.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]
HOST_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-ffp-contract=off", "-Wall", "-Wextra"]


def _run(cmd):
    p = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if p.returncode != 0:
        raise RuntimeError(f"command failed ({p.returncode}): {' '.join(cmd)}\n{p.stdout}")
    return p.stdout


def build(jobs: int = 8, verbose: bool = False) -> str:
    os.makedirs(BUILD, exist_ok=True)
    jobs_list = []
    for src in HIP_SOURCES:
        obj = os.path.join(BUILD, src + ".o")
        jobs_list.append([HIPCC, *HIP_FLAGS, "-c", os.path.join(CSRC, src), "-o", obj])
    for src in HOST_SOURCES:
        obj = os.path.join(BUILD, src + ".o")
        jobs_list.append(["g++", *HOST_FLAGS, "-c", os.path.join(CSRC, src), "-o", obj])
    with cf.ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        outs = list(ex.map(_run, jobs_list))
    if verbose:
        for o in outs:
            if o.strip():
                print(o)
    objs = [os.path.join(BUILD, s + ".o") for s in HIP_SOURCES + HOST_SOURCES]
    tmp = LIB + ".tmp"
    _run([HIPCC, "-shared", f"--offload-arch={ARCH}", "-o", tmp, *objs, "-lpthread"])
    os.replace(tmp, LIB)
    return LIB


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=min(8, os.cpu_count() or 1))
    ap.add_argument("-v", "--verbose", action="store_true")
    a = ap.parse_args()
    print(build(a.jobs, a.verbose))


if __name__ == "__main__":
    sys.exit(main())
