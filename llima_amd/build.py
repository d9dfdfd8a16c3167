"""Builds libllima_sampler.so (all HIP kernels + the C ABI) for gfx950, in-tree.

Each source is compiled to its own object (in parallel, under
llima_amd/_build/), then the objects are linked into the shared library.

hipcc flags:
  -ffp-contract=off      every product/sum is the IEEE operation in the source
                         (no fused multiply-add the host restatement lacks)
  -packed-fp32-ops off   no packed FP32 instructions are generated

`python -m llima_amd.build --incremental` recompiles only the objects older
than their source or a shared header; build() recompiles everything.
"""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libllima_sampler.so")
SOURCES = ["argmax.hip", "sample.hip", "verify.hip", "score.hip", "lmhead.hip", "tree.hip", "stop.hip"]
HEADERS = [os.path.join(CSRC, "common.hpp"), os.path.join(ROOT, "include", "llima_sampler.h")]
ARCH = os.environ.get("LLIMA_OFFLOAD_ARCH", "gfx950")
FLAGS = ["-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
         "-Wno-unused-command-line-argument"]


def compile_cmd(src: str, out: str, extra: list[str] | None = None) -> list[str]:
    return (["hipcc", f"--offload-arch={ARCH}"] + FLAGS + (extra or []) +
            ["-I", os.path.join(ROOT, "include"), "-c", "-o", out, src])


def link_cmd(objs: list[str], out: str) -> list[str]:
    return ["hipcc", f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", out] + objs


def hipcc_cmd(out: str, extra: list[str] | None = None) -> list[str]:
    """One command that compiles and links every source (used by tools that
    build a variant of the library, e.g. with a trace flag)."""
    return (["hipcc", f"--offload-arch={ARCH}"] + FLAGS + (extra or []) + ["-shared"] +
            ["-I", os.path.join(ROOT, "include"), "-o", out] +
            [os.path.join(CSRC, s) for s in SOURCES])


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError(f"hipcc failed: {' '.join(cmd[-1:])}")


def build(verbose: bool = False, incremental: bool = False) -> str:
    os.makedirs(OBJ, exist_ok=True)
    newest_hdr = max(os.path.getmtime(h) for h in HEADERS)
    jobs, objs = [], []
    for s in SOURCES:
        src = os.path.join(CSRC, s)
        obj = os.path.join(OBJ, s.replace(".hip", ".o"))
        objs.append(obj)
        stale = (not incremental or not os.path.exists(obj) or
                 os.path.getmtime(obj) < max(os.path.getmtime(src), newest_hdr))
        if stale:
            jobs.append(compile_cmd(src, obj))
    workers = max(1, min(len(jobs), int(os.environ.get("MAX_JOBS", os.cpu_count() or 1))))
    with ThreadPoolExecutor(max_workers=workers) as ex:
        for f in [ex.submit(_run, j, verbose) for j in jobs]:
            f.result()
    tmp = LIB + ".tmp"
    _run(link_cmd(objs, tmp), verbose)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True, incremental="--incremental" in sys.argv))
