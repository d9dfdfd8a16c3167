"""Per-phase trace of the sampler's finish kernel on one workload.

Builds a copy of the library with -DLLIMA_FINISH_TRACE (sample_finish then
stores the wall clock, 100 MHz, at each phase mark of the first 512 rows) into
OUT_DIR, runs llima_sample on the workload's inputs, and prints, per mark, the
median time since the row's workgroup started and since the previous mark
reached.  The traced build writes a few extra stores per row; its step times
are not the product's.

    python -m llima_amd.finish_trace [--workload batched_penalties] [--calls 200] [--out DIR]
"""
from __future__ import annotations

import argparse
import ctypes
import os
import subprocess
import sys

import numpy as np

from . import build as _build

DIRECT = {
    0: "start (row config)",
    1: "first-round slots and history ids arrived",
    2: "row facts reduced (1 barrier)",
    3: "direct path entered (id bitmap cleared)",
    4: "top-k boundary: histogram rounds done",
    5: "survivors staged (scan + 1 barrier)",
    6: "survivor-id bitmap built (1 barrier)",
    7: "history ids counted against the survivors",
    8: "penalties applied (1 barrier)",
    9: "temperature, keys, weights staged",
    10: "pairwise ranking (1 barrier)",
    11: "tau, top-k mass",
    12: "top-p / min-p cut, draw written",
    13: "end",
}
GATHER = {
    0: "start (row config)",
    1: "first-round slots arrived",
    2: "row facts reduced (1 barrier)",
    3: "gather: chunk counts scanned (2 barriers)",
    4: "gather: candidates in LDS (1 barrier)",
    5: "keys, row max / min (2 barriers)",
    6: "top-k boundary rounds",
    7: "survivor count scanned",
    8: "weights computed",
    9: "top-p boundary (value bins, pairwise in one bin)",
    10: "min-p cut, per-thread kept mass",
    11: "id-order scan of the kept mass (block scan)",
    12: "draw written",
    13: "end",
}
ROWS, NMARK = 512, 16
TICK_NS = 10.0


def build_traced(out_dir: str) -> str:
    os.makedirs(out_dir, exist_ok=True)
    lib = os.path.join(out_dir, "libllima_sampler_trace.so")
    cmd = _build.hipcc_cmd(lib)
    cmd.insert(1, "-DLLIMA_FINISH_TRACE")
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError("hipcc failed building the traced library")
    return lib


def main(argv=None) -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--workload", default="batched_penalties")
    ap.add_argument("--calls", type=int, default=200)
    ap.add_argument("--out", default="/tmp/llima_finish_trace")
    a = ap.parse_args(argv)
    lib = build_traced(a.out)
    print(f"[trace] built {lib}", flush=True)
    from . import _lib
    _lib.LIB_PATH = lib
    import torch
    import llima_amd
    from llima_amd import workloads as wl
    L = _lib.lib()
    L.llima_finish_trace_read.restype = ctypes.c_int
    L.llima_finish_trace_read.argtypes = [ctypes.c_void_p]
    dev = torch.device("cuda:0")
    w = wl.WORKLOADS[a.workload]()
    lg = w["logits"]
    x = (torch.from_numpy(lg.view(np.int16)).to(dev).view(torch.bfloat16) if lg.dtype == np.uint16
         else torch.from_numpy(lg).to(dev))
    hist = None if w["history"] is None else torch.from_numpy(w["history"]).to(dev)
    mask = None if w["bitmask"] is None else torch.from_numpy(w["bitmask"].view(np.int32)).to(dev)
    u = torch.from_numpy(w["uniforms"]).to(dev)
    cfg = llima_amd.SamplerConfig(**w["cfg"])
    B = lg.shape[0]
    buf = np.zeros((ROWS, NMARK), np.uint64)
    rel, step = [], []
    for i in range(a.calls + 10):
        llima_amd.sample(x, u, cfg, history=hist, bitmask=mask)
        torch.cuda.synchronize()
        if i < 10:
            continue
        if L.llima_finish_trace_read(buf.ctypes.data) != 0:
            raise RuntimeError("llima_finish_trace_read failed")
        t = buf[:min(B, ROWS)].astype(np.int64)
        rel.append(np.where(t[:, :14] > 0, t[:, :14] - t[:, :1], -1))
        rel[-1][:, 0] = 0
        step.append(t[:, 14:16])
    r = np.concatenate(rel)                       # [calls * rows, 14]
    path = np.concatenate(step)[:, 1]
    print(f"[trace] {a.workload}: {B} rows x {a.calls} calls; median over rows that reach each mark, "
          f"wall clock {TICK_NS:.0f} ns per tick", flush=True)
    for pid, names, title in [(1, DIRECT, "direct path"), (2, GATHER, "gather path")]:
        rr = r[path == pid]
        if len(rr) == 0:
            continue
        print(f"[trace] {title}: {100 * len(rr) / len(r):.1f}% of rows")
        print(f"{'mark':>4}  {'phase':<45} {'rows %':>7} {'us since start':>15} {'us since previous':>18}")
        prev = np.zeros(len(rr))
        for m in range(14):
            hit = rr[:, m] >= 0
            if not hit.any():
                continue
            since = np.median(rr[hit, m]) * TICK_NS / 1000
            d = np.median((rr[hit, m] - prev[hit])) * TICK_NS / 1000
            print(f"{m:>4}  {names[m]:<45} {100 * hit.mean():>6.1f}% {since:>15.2f} {d:>18.2f}")
            prev = np.where(hit, rr[:, m], prev)
    print(f"[trace] candidate slots per row (median) {np.median(np.concatenate(step)[:, 0]):.0f}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
