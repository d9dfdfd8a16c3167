"""Builds libllima_sampler.so (all HIP kernels + the C ABI) for gfx950, in-tree.

hipcc flags:
  -ffp-contract=off      every product/sum is the IEEE operation in the source
                         (no fused multiply-add the host restatement lacks)
  -packed-fp32-ops off   no packed FP32 instructions are generated
"""
from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libllima_sampler.so")
SOURCES = ["argmax.hip", "sample.hip", "verify.hip", "score.hip", "lmhead.hip", "tree.hip", "stop.hip"]
ARCH = os.environ.get("LLIMA_OFFLOAD_ARCH", "gfx950")


def hipcc_cmd(out: str) -> list[str]:
    return ["hipcc", f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-shared",
            "-ffp-contract=off", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
            "-Wno-unused-command-line-argument",
            "-I", os.path.join(ROOT, "include"), "-o", out] + \
           [os.path.join(CSRC, s) for s in SOURCES]


def build(verbose: bool = False) -> str:
    tmp = LIB + ".tmp"
    cmd = hipcc_cmd(tmp)
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError("hipcc failed building libllima_sampler.so")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
