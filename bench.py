#!/usr/bin/env python3
"""Benchmark of the token-selection step on one MI355X.

Default workload: batched full penalty stack, B=64, V=128256 fp32 logits
(Llama-3 head shape) ~ N(0, 4^2), 2048-id Zipf(1.1) history per row,
repetition 1.15 / presence 0.5 / frequency 0.3, T 0.8, top-k 50, top-p 0.95,
min-p 0.05, one seeded uniform per row.  One step = one llima_sample launch over
one batch.  Inputs rotate over >= 1 GiB of distinct device buffers so that the
256 MB Infinity Cache cannot serve them; they are resident in HBM before the
timed region starts.

Prints ONE JSON line.  value = sampled rows/s (whole job), ms_per_step from a
HIP-graph replay of K steps bracketed by synchronisation and timed with HIP
events on the launch stream.  One step is one entry-point call (for the sampler
its kernels: sweep and finish, or the dense path's five), so roofline.achieved = algorithmic bytes per
step / ms_per_step; eager_call_us is the mean of per-call HIP events without the
graph (host launch gaps included).  roofline.traffic = HBM bytes per step from
the committed rocprofv3 counter runs (profiles/traffic.json), when measured for
this workload.  cpu_baseline = the CPU oracle on a bounded sample of the same
workload on this host (for the LM-head workloads, numpy float32 products on a
slice of the vocabulary, scaled to the whole).

--workload selects the other configurations: single_row, constrained,
large_vocab_bf16(_greedy), argmax_bf16, speculative, score_bf16,
mtp_masked_argmax, top_p_only (the default rows with top-p alone: the
sampler's dense path, five kernels), and lm_head_argmax /
lm_head_argmax_b64/b128/b256 (the LM head with its argmax at B = 1 to 256)
and lm_head_argmax_b32/b64/b128_packed (over a weight packed at load time);
lm_head_score_b64_packed: the packed LM head with its scoring epilogue (the
log-softmax at 64 target ids, no logits written); lm_head_verify_b16_d7: the
LM head over 16 sequences x 8 rows with greedy chain verification fused (no
logits written).  batched_penalties_rows: the default batch with every setting
given per row (SamplerConfig tensors).  mixed_topk_rows: even rows top-k 50 /
top-p 0.95, odd rows top-p 0.9 alone, no history.  constrained_half: the
constrained rows under a mask allowing half of the ids.  topk_bf16: llima_topk, k 5
over 5 bf16 rows of 32000 (the EAGLE3 draft head's top-k).  eagle3_tree: one
whole EAGLE3 draft tree (K 5, depth 4, 15 tokens; draft vocabulary 32000,
target 128256): tree_begin, three tree_grow, tree_finish.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

METRIC = "sampled rows/sec + µs/step at B=64,V=128256; achieved HBM GB/s vs peak"
HBM_PEAK_GBS = 8000.0


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default="batched_penalties",
                    choices=["batched_penalties", "batched_penalties_rows", "mixed_topk_rows",
                             "topk_bf16", "eagle3_tree",
                             "single_row", "constrained", "constrained_half", "top_p_only",
                             "large_vocab_bf16", "large_vocab_bf16_greedy", "argmax_bf16",
                             "speculative", "score_bf16", "mtp_masked_argmax",
                             "lm_head_argmax", "lm_head_argmax_b64", "lm_head_argmax_b128",
                             "lm_head_argmax_b256", "lm_head_argmax_b32_packed",
                             "lm_head_argmax_b64_packed", "lm_head_argmax_b128_packed",
                             "lm_head_score_b64_packed", "lm_head_verify_b16_d7"])
    ap.add_argument("--rotate-gib", type=float, default=1.0)
    ap.add_argument("--no-graph", action="store_true")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=16.0)
    ap.add_argument("--profile-steps", type=int, default=0,
                    help="only run this many plain launches (for rocprofv3 counter runs)")
    return ap.parse_args()


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: the selection step shards by rows with no exchange, "
              "and multi-GPU runs are not part of this build (use --gpus 1).", file=sys.stderr)
        sys.exit(2)
    import torch
    import llima_amd
    from llima_amd import _lib, workloads as wl
    from llima_amd._lib import lib, check

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    L = lib()
    stream = torch.cuda.current_stream(dev)
    sptr = stream.cuda_stream

    name = args.workload
    greedy_variant = name.endswith("_greedy")
    argmax_only = name == "argmax_bf16"          # llima_argmax on the same rows
    gen = wl.WORKLOADS["large_vocab_bf16" if (greedy_variant or argmax_only) else name]
    w = gen()
    t0 = time.time()

    launches = []          # one callable per rotated input, taking a stream pointer
    data_note = None
    if name.startswith("lm_head_"):
        B, H, V = w["B"], w["H"], w["V"]
        scoring = name.startswith("lm_head_score")
        verifying = name.startswith("lm_head_verify")
        g = torch.Generator(device=dev)
        g.manual_seed(w["seed"])
        weight = (torch.randn((V, H), generator=g, device=dev) * (1.0 / H ** 0.5)).to(torch.bfloat16)
        hid = [torch.from_numpy(w["hidden"].view(np.int16)).to(dev).view(torch.bfloat16)]
        hid += [torch.randn((B, H), generator=g, device=dev).to(torch.bfloat16) for _ in range(7)]
        ids_o = torch.empty(B, dtype=torch.int32, device=dev)
        vals_o = torch.empty(B, dtype=torch.float32, device=dev)
        packed = name.endswith("_packed")
        if scoring:
            nws = (L.llima_lm_head_score_packed_workspace_bytes(B, H, V) if packed
                   else L.llima_lm_head_score_workspace_bytes(B, V))
        elif verifying:                  # B hidden rows = seqs sequences of D + 1
            nseq, D = w["seqs"], w["D"]
            nws = (L.llima_lm_head_verify_greedy_packed_workspace_bytes(nseq, D, H, V) if packed
                   else L.llima_lm_head_verify_greedy_workspace_bytes(nseq, D, V))
        else:
            nws = (L.llima_lm_head_argmax_packed_workspace_bytes(B, H, V) if packed
                   else L.llima_lm_head_argmax_workspace_bytes(B, V))
        ws = torch.zeros(nws, dtype=torch.uint8, device=dev)
        if packed:       # the load-time layout, built once before any timing
            wp = torch.empty(L.llima_lm_head_packed_bytes(V, H), dtype=torch.uint8, device=dev)
            check(L.llima_lm_head_pack(weight.data_ptr(), V, H, wp.data_ptr(), wp.numel(),
                                       torch.cuda.current_stream().cuda_stream), "llima_lm_head_pack")
            torch.cuda.synchronize()
            del weight
            weight = wp
        if scoring:
            fn = L.llima_lm_head_score_packed if packed else L.llima_lm_head_score
            tgs = [torch.randint(0, V, (B,), generator=g, device=dev, dtype=torch.int32)
                   for _ in hid]
            lp_o = torch.empty(B, dtype=torch.float64, device=dev)
            for x, tg in zip(hid, tgs):
                launches.append(lambda sp, x=x, tg=tg: check(fn(
                    x.data_ptr(), weight.data_ptr(), B, H, V, 0.0, 1, tg.data_ptr(),
                    lp_o.data_ptr(), ids_o.data_ptr(), ws.data_ptr(), nws, sp),
                    "llima_lm_head_score"))
        elif verifying:
            fn = (L.llima_lm_head_verify_greedy_packed if packed
                  else L.llima_lm_head_verify_greedy)
            drs = [torch.randint(0, V, (nseq, D), generator=g, device=dev, dtype=torch.int32)
                   for _ in hid]
            em_o = torch.empty((nseq, D + 1), dtype=torch.int32, device=dev)
            for x, dr in zip(hid, drs):
                launches.append(lambda sp, x=x, dr=dr: check(fn(
                    x.data_ptr(), weight.data_ptr(), nseq, D, H, V, 0.0, 1, dr.data_ptr(),
                    ids_o.data_ptr(), em_o.data_ptr(), ws.data_ptr(), nws, sp),
                    "llima_lm_head_verify_greedy"))
        else:
            fn = L.llima_lm_head_argmax_packed if packed else L.llima_lm_head_argmax
            for x in hid:
                launches.append(lambda sp, x=x: check(fn(
                    x.data_ptr(), weight.data_ptr(), B, H, V, 0.0, 1, ids_o.data_ptr(),
                    vals_o.data_ptr(), None, ws.data_ptr(), nws, sp), "llima_lm_head_argmax"))
        per = V * H * 2
        # weight, hidden rows, then the argmax's ids and values, the targets,
        # log-probabilities and flags, or the drafts and the verification
        # outputs
        alg_bytes = V * H * 2 + B * H * 2 + (B * 16 if scoring else B * 8)
        if verifying:
            alg_bytes = V * H * 2 + B * H * 2 + nseq * D * 4 + nseq * (D + 2) * 4
        rows = B
        unit_rows = "rows/s"
        dtype = "bf16"
        fin = "lmh_score_finish" if scoring else "lmh_finish"
        if verifying:
            rows, unit_rows = nseq, "sequences/s"
        kernel_names = (["lmh_packed", fin] if packed else
                        ["lmh_mfma" if B > 4 else "lmh_rows", fin])
        config = {"workload": name, "B": B, "H": H, "V": V,
                  "weight": "bf16 [V, H] packed at load time" if packed else "bf16 [V, H]"}
        data_note = ("synthetic (seeded; one bf16 [%d, %d] weight, %.2f GiB, above the 256 MB "
                     "Infinity Cache; 8 rotating hidden rows)" % (V, H, per / 2**30))
    elif name == "speculative":
        B, D, V = w["target"].shape[0], w["target"].shape[1] - 1, w["target"].shape[2]
        per = w["target"].nbytes + w["draft"].nbytes
        nbuf = max(2, int(np.ceil(args.rotate_gib * 2**30 / per)))
        g = torch.Generator(device=dev)
        g.manual_seed(1004)
        base_t = torch.from_numpy(w["target"]).to(dev)
        base_d = torch.from_numpy(w["draft"]).to(dev)
        ids = torch.from_numpy(w["draft_ids"]).to(dev)
        ua = torch.from_numpy(w["u_accept"]).to(dev)
        ur = torch.from_numpy(w["u_resample"]).to(dev)
        acc = torch.empty(B, dtype=torch.int32, device=dev)
        em = torch.empty((B, D + 1), dtype=torch.int32, device=dev)
        nws = L.llima_verify_rejection_workspace_bytes(B, D, V)
        ws = torch.zeros(nws, dtype=torch.uint8, device=dev)
        bufs = [(base_t, base_d)]
        for i in range(1, nbuf):
            tt = torch.randn(base_t.shape, generator=g, device=dev) * 4.0
            dd = tt[:, :D] + torch.randn(base_d.shape, generator=g, device=dev) * 1.5
            bufs.append((tt.contiguous(), dd.contiguous()))
        for tt, dd in bufs:
            launches.append(lambda sp, tt=tt, dd=dd: check(L.llima_verify_rejection(
                tt.data_ptr(), dd.data_ptr(), B, D, V, ids.data_ptr(), ua.data_ptr(),
                ur.data_ptr(), acc.data_ptr(), em.data_ptr(), ws.data_ptr(), nws, sp),
                "verify_rejection"))
        alg_bytes = w["target"].nbytes + w["draft"].nbytes + ids.numel() * 4 + ua.numel() * 4 + \
            ur.numel() * 4 + acc.numel() * 4 + em.numel() * 4
        rows = B
        unit_rows = "sequences/s"
        dtype = "f32"
        kernel_names = ["vr_rowpass", "vr_draw"]
        config = {"workload": "speculative", "B": B, "draft_len": D, "V": V}
    elif name in ("topk_bf16", "eagle3_tree"):
        # EAGLE3 drafting: the inputs are small (a few hundred KB) and the draft
        # model's LM head has just written them, so they rotate over a handful
        # of buffers only (and may sit in the Infinity Cache, as in the loop)
        nbuf = 8
        g = torch.Generator(device=dev)
        g.manual_seed(2002)
        rows = 1
        dtype = "bf16"
        if name == "topk_bf16":
            k = w["k"]
            R_, C_ = w["logits"].shape
            bufs = [torch.from_numpy(w["logits"].view(np.int16)).to(dev).view(torch.bfloat16)]
            for i in range(1, nbuf):
                bufs.append((torch.randn((R_, C_), generator=g, device=dev) * 3.0).to(torch.bfloat16))
            idx_o = torch.empty((R_, k), dtype=torch.int32, device=dev)
            val_o = torch.empty((R_, k), dtype=torch.float32, device=dev)
            for x in bufs:
                launches.append(lambda sp, x=x, R_=R_, C_=C_, k=k: check(L.llima_topk(
                    x.data_ptr(), _lib.LLIMA_BF16, R_, C_, C_, k, idx_o.data_ptr(), val_o.data_ptr(),
                    sp), "llima_topk"))
            per = R_ * C_ * 2
            alg_bytes = per + R_ * k * 8
            unit_rows = "calls/s"
            kernel_names = ["topk_rows_kernel"]
            config = {"workload": name, "rows": R_, "cols": C_, "k": k, "logits_dtype": "bf16"}
        else:
            K, depth, total, Vd = w["K"], w["depth"], w["total"], w["root"].shape[0]
            d2t = torch.from_numpy(w["d2t"]).to(dev)
            nb = L.llima_eagle3_tree_bytes(K, depth)
            state = torch.empty(nb, dtype=torch.uint8, device=dev)
            roots = [torch.from_numpy(w["root"].view(np.int16)).to(dev).view(torch.bfloat16)]
            levs = [torch.from_numpy(w["levels"].view(np.int16)).to(dev).view(torch.bfloat16)]
            for i in range(1, nbuf):
                roots.append((torch.randn((Vd,), generator=g, device=dev) * 3.0).to(torch.bfloat16))
                levs.append((torch.randn((depth - 1, K, Vd), generator=g, device=dev) * 3.0)
                            .to(torch.bfloat16))
            N = total + 1
            ids_o = torch.empty(K, dtype=torch.int32, device=dev)
            prow_o = torch.empty(K, dtype=torch.int32, device=dev)
            mask_o = torch.empty((K, K * depth), dtype=torch.float32, device=dev)
            tok_o = torch.empty(N, dtype=torch.int32, device=dev)
            tm_o = torch.empty((N, N), dtype=torch.float32, device=dev)
            pos_o = torch.empty(N, dtype=torch.int32, device=dev)
            ret_o = torch.empty((N, N), dtype=torch.int32, device=dev)
            dims_o = torch.empty(2, dtype=torch.int32, device=dev)

            def tree(sp, r, lv, K=K, depth=depth, total=total, Vd=Vd):   # bound now: main reuses K
                check(L.llima_eagle3_tree_begin(r.data_ptr(), _lib.LLIMA_BF16, Vd, d2t.data_ptr(), K,
                                                depth, state.data_ptr(), nb, ids_o.data_ptr(), sp),
                      "llima_eagle3_tree_begin")
                for lvl in range(1, depth):
                    check(L.llima_eagle3_tree_grow(lv[lvl - 1].data_ptr(), _lib.LLIMA_BF16, Vd, Vd,
                                                   d2t.data_ptr(), K, depth, lvl, state.data_ptr(), nb,
                                                   ids_o.data_ptr(), prow_o.data_ptr(),
                                                   mask_o.data_ptr(), sp), "llima_eagle3_tree_grow")
                check(L.llima_eagle3_tree_finish(state.data_ptr(), nb, K, depth, total,
                                                 w["sample_token"], tok_o.data_ptr(), tm_o.data_ptr(),
                                                 pos_o.data_ptr(), ret_o.data_ptr(), dims_o.data_ptr(),
                                                 sp), "llima_eagle3_tree_finish")
            for r, lv in zip(roots, levs):
                launches.append(lambda sp, r=r, lv=lv: tree(sp, r, lv))
            per = (1 + (depth - 1) * K) * Vd * 2
            alg_bytes = per + Vd * 4 + N * 4 * 3 + N * N * 8
            unit_rows = "trees/s"
            kernel_names = ["eagle3_begin_kernel", "eagle3_rows_kernel", "eagle3_combine_kernel",
                            "eagle3_finish_kernel"]
            config = {"workload": name, "K": K, "depth": depth, "total_tokens": total,
                      "draft_vocab": Vd, "logits_dtype": "bf16",
                      "calls": "begin + %d grow + finish" % (depth - 1)}
        data_note = ("synthetic (seeded; %d input sets of %d KB, small enough for the Infinity "
                     "Cache, as a draft LM head's fresh output is)" % (nbuf, per // 1024))
    elif name in ("score_bf16", "mtp_masked_argmax"):
        lg = w["logits"]
        B, V = lg.shape
        dt = _lib.LLIMA_BF16
        per = lg.nbytes
        nbuf = max(2, int(np.ceil(args.rotate_gib * 2**30 / per)))
        g = torch.Generator(device=dev)
        g.manual_seed(2001)
        bufs = [torch.from_numpy(lg.view(np.int16)).to(dev).view(torch.bfloat16)]
        for i in range(1, nbuf):
            x = torch.randn((B, V), generator=g, device=dev) * 5.0
            bufs.append((30.0 * torch.tanh(x / 30.0)).to(torch.bfloat16).contiguous())
        rows = B
        unit_rows = "rows/s"
        dtype = "bf16"
        if name == "score_bf16":
            tg = torch.from_numpy(w["targets"]).to(dev)
            lp = torch.empty(B, dtype=torch.float64, device=dev)
            gr = torch.empty(B, dtype=torch.int32, device=dev)
            nws = L.llima_score_logits_workspace_bytes(B, V, dt)
            ws = torch.zeros(nws, dtype=torch.uint8, device=dev)
            for x in bufs:
                launches.append(lambda sp, x=x: check(L.llima_score_logits(
                    x.data_ptr(), dt, B, V, V, tg.data_ptr(), lp.data_ptr(), gr.data_ptr(),
                    ws.data_ptr(), nws, sp), "llima_score_logits"))
            alg_bytes = lg.nbytes + B * (4 + 8 + 4)
            kernel_names = ["score_sweep", "score_finish"]
            config = {"workload": name, "B": B, "V": V, "logits_dtype": "bf16"}
        else:
            C, k = w["centroids"].shape[1], w["top_k"]
            cent = torch.from_numpy(w["centroids"].view(np.int16)).to(dev)
            order = torch.from_numpy(w["ordering"].view(np.int32)).to(dev)
            ids_o = torch.empty(B, dtype=torch.int32, device=dev)
            st_o = torch.empty(B, dtype=torch.int32, device=dev)
            nws = L.llima_mtp_masked_argmax_workspace_bytes(B)
            ws = torch.zeros(nws, dtype=torch.uint8, device=dev)
            for x in bufs:
                launches.append(lambda sp, x=x: check(L.llima_mtp_masked_argmax(
                    cent.data_ptr(), C, C, order.data_ptr(), k, x.data_ptr(), dt, B, V, V,
                    ids_o.data_ptr(), st_o.data_ptr(), None, ws.data_ptr(), nws, sp),
                    "llima_mtp_masked_argmax"))
            # centroid row, the selected ordering runs and their logits, the outputs
            alg_bytes = B * (C * 2 + k * (V // C) * (4 + 2) + 4 + 4)
            kernel_names = ["mtp_select_gather", "mtp_combine"]
            config = {"workload": name, "B": B, "V": V, "centroids": C, "top_k": k,
                      "logits_dtype": "bf16"}
    else:
        lg = w["logits"]
        B, V = lg.shape
        is_bf16 = lg.dtype == np.uint16
        dt = _lib.LLIMA_BF16 if is_bf16 else _lib.LLIMA_F32
        per = lg.nbytes
        nbuf = max(2, int(np.ceil(args.rotate_gib * 2**30 / per)))
        if is_bf16:
            base = torch.from_numpy(lg.view(np.int16)).to(dev).view(torch.bfloat16)
        else:
            base = torch.from_numpy(lg).to(dev)
        g = torch.Generator(device=dev)
        g.manual_seed(2000)
        sigma = {"single_row": 3.0, "batched_penalties": 4.0, "batched_penalties_rows": 4.0,
                 "mixed_topk_rows": 4.0, "constrained": 3.0, "constrained_half": 3.0,
                 "top_p_only": 4.0}.get(name, 5.0)
        bufs = [base]
        for i in range(1, nbuf):
            x = torch.randn((B, V), generator=g, device=dev) * sigma
            if is_bf16:
                x = (30.0 * torch.tanh(x / 30.0)).to(torch.bfloat16)
            bufs.append(x.contiguous())
        hist = None if w["history"] is None else torch.from_numpy(w["history"]).to(dev)
        H = 0 if hist is None else hist.shape[1]
        mask = None if w["bitmask"] is None else \
            torch.from_numpy(w["bitmask"].view(np.int32)).to(dev)
        u = torch.from_numpy(w["uniforms"]).to(dev)
        # histories, masks and uniforms rotate with the logits (their own
        # buffers per step, so no step finds them in a cache)
        hists = [hist] + [None if hist is None else torch.roll(hist, i, 0).contiguous()
                          for i in range(1, nbuf)]
        masks = [mask] + [None if mask is None else torch.roll(mask, i, 0).contiguous()
                          for i in range(1, nbuf)]
        us = [u] + [torch.rand(u.shape, generator=g, device=dev) for _ in range(1, nbuf)]
        cfgd = dict(w["cfg"])
        if greedy_variant:
            cfgd = dict(greedy=True)
        cfg_c = dict(cfgd)
        # per-row settings, from host memory as a serving loop holds its requests'
        # settings (uploaded once, before timing)
        for k, arr in (w.get("cfg_rows") or {}).items():
            cfg_c[k] = torch.from_numpy(arr)
        cfg, keep_alive = llima_amd.SamplerConfig(**cfg_c).to_c(B, dev, V)
        out_ids = torch.empty(B, dtype=torch.int32, device=dev)
        out_p = torch.empty(B, dtype=torch.float32, device=dev)
        nws = L.llima_sample_workspace_bytes(B, V, dt)
        ws = torch.zeros(nws, dtype=torch.uint8, device=dev)
        cref = ctypes.byref(cfg)
        if argmax_only:
            nwa = L.llima_argmax_workspace_bytes(B, V, dt)
            wsa = torch.zeros(max(nwa, 1), dtype=torch.uint8, device=dev)
            for x in bufs:
                launches.append(lambda sp, x=x: check(L.llima_argmax(
                    x.data_ptr(), dt, B, V, V, 0, _lib.ARGMAX_SPLIT_FIRST, out_ids.data_ptr(), None,
                    wsa.data_ptr(), nwa, sp), "llima_argmax"))
            alg_bytes = lg.nbytes + out_ids.numel() * 4
            kernel_names = ["argmax_sweep", "argmax_finish"]
            config = {"workload": name, "B": B, "V": V, "logits_dtype": "bf16" if is_bf16 else "fp32"}
        else:
            for x, hh, mm, uu in zip(bufs, hists, masks, us):
                launches.append(lambda sp, x=x, hh=hh, mm=mm, uu=uu: check(L.llima_sample(
                    x.data_ptr(), dt, B, V, V, None if hh is None else hh.data_ptr(), None, H,
                    None if mm is None else mm.data_ptr(), uu.data_ptr(), cref,
                    out_ids.data_ptr(), out_p.data_ptr(), None, ws.data_ptr(), nws, sp),
                    "llima_sample"))
            alg_bytes = lg.nbytes + (0 if hist is None else hist.numel() * 4) + \
                (0 if mask is None else mask.numel() * 4) + u.numel() * 4 + out_ids.numel() * 4 + \
                out_p.numel() * 4
            # rows without top-k, mask or greedy take the library's dense path
            dense = mask is None and not cfgd.get("greedy") and cfgd.get("temperature", 1.0) > 0 and \
                not (0 < cfgd.get("top_k", 0) < V)
            kernel_names = (["dense_stats"] + (["dense_hist", "dense_bound"] if cfgd.get("top_p", 1.0) < 1
                                               else []) + ["dense_keep", "dense_final"]
                            if dense else ["sample_sweep"] +
                            (["sample_finish_wide"] if mask is not None and not cfgd.get("greedy") and
                             not (0 < cfgd.get("top_k", 0) < V) else []) + ["sample_finish"])
            config = {"workload": name, "B": B, "V": V, "history": H,
                      "logits_dtype": "bf16" if is_bf16 else "fp32"}
            config.update({k: v for k, v in cfgd.items()})
            for k, arr in (w.get("cfg_rows") or {}).items():
                vals = sorted(set(arr.tolist()))
                config[k] = "per-row array: " + ", ".join(str(round(v, 6)) for v in vals)
        rows = B
        unit_rows = "rows/s"
        dtype = "bf16" if is_bf16 else "f32"
    torch.cuda.synchronize()
    setup_s = time.time() - t0

    if args.profile_steps:
        for i in range(args.profile_steps):
            launches[i % len(launches)](sptr)
        torch.cuda.synchronize()
        print(json.dumps({"profile_steps": args.profile_steps, "workload": name}), flush=True)
        return

    # ---- warmup
    for i in range(args.warmup):
        launches[i % len(launches)](sptr)
    torch.cuda.synchronize()

    # ---- per-launch kernel time with HIP events on the launch stream
    K = args.steps
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(K)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(K)]
    for i in range(K):
        starts[i].record(stream)
        launches[i % len(launches)](sptr)
        ends[i].record(stream)
    torch.cuda.synchronize()
    per_launch_ms = np.array([s.elapsed_time(e) for s, e in zip(starts, ends)])
    launch_ms = float(np.mean(per_launch_ms))

    # ---- timed region: K steps, HIP graph replay (no host gaps) unless --no-graph
    graph = None
    if not args.no_graph:
        try:
            graph = torch.cuda.CUDAGraph()
            cap = torch.cuda.Stream(dev)
            cap.wait_stream(stream)
            with torch.cuda.graph(graph, stream=cap):
                for i in range(K):
                    launches[i % len(launches)](cap.cuda_stream)
            torch.cuda.synchronize()
        except Exception as e:  # pragma: no cover - reported, then eager timing
            print(f"graph capture failed ({e}); timing eager launches", file=sys.stderr)
            graph = None
    torch.cuda.synchronize()
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    if graph is not None:
        graph.replay()          # one untimed replay
        torch.cuda.synchronize()
        ev0.record(stream)
        graph.replay()
        ev1.record(stream)
    else:
        ev0.record(stream)
        for i in range(K):
            launches[i % len(launches)](sptr)
        ev1.record(stream)
    torch.cuda.synchronize()
    total_ms = ev0.elapsed_time(ev1)
    ms_per_step = total_ms / K

    achieved = alg_bytes / (ms_per_step * 1e-3) / 1e9
    traffic = None
    try:
        with open(os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                               "traffic.json")) as f:
            traffic = json.load(f).get(name, {}).get("bytes_per_step")
    except (OSError, ValueError):
        pass
    result = {
        "metric": METRIC,
        "value": rows / (ms_per_step * 1e-3),
        "unit": unit_rows,
        "n_gpus": 1,
        "steps": K,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "us_per_step": ms_per_step * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": dtype,
        "data": data_note or "synthetic (seeded; inputs rotate over %d device buffers, %.2f GiB)" % (
            len(launches), len(launches) * per / 2**30),
        "config": config,
        "timing": "graph replay" if graph is not None else "eager launches",
        "roofline": {
            "bound": "hbm",
            "achieved": achieved,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": achieved / HBM_PEAK_GBS,
            "traffic": traffic,
            "kernel": kernel_names,
            "algorithmic_bytes_per_step": int(alg_bytes),
            "eager_call_us": launch_ms * 1e3,
            "eager_call_median_us": float(np.median(per_launch_ms)) * 1e3,
        },
    }
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(name, w, args.cpu_seconds, greedy_variant)
    result["setup_s"] = round(setup_s, 2)
    print(json.dumps(result), flush=True)


def cpu_baseline(name, w, seconds, greedy_variant):
    """The CPU oracle (oracle/llima_oracle.cpp, built -O3 for x86-64-v3, OpenMP
    over rows) timed on bounded samples of the same workload on this host, at
    1 thread and at OMP_NUM_THREADS threads (the host's CPU share; every
    core otherwise).  The greedy workloads run the reference's own shape: one
    row at a time with four threads (_calc_next_token_id,
    language_model.cpp:3689-3714).  `value` is the many-thread figure."""
    from oracle import oracle as orc
    nproc = os.cpu_count() or 1
    many = int(os.environ.get("OMP_NUM_THREADS", "0")) or nproc
    orc.lib()
    leg = seconds / 2

    def timed(fn, threads):
        orc.set_threads(threads)
        t0 = time.time()
        n = reps = 0
        while time.time() < t0 + leg or reps == 0:
            n += fn()
            reps += 1
        return n / (time.time() - t0), reps, time.time() - t0

    info = {"kind": "port", "cpu": _cpu_model(), "nproc": nproc,
            "omp_num_threads": os.environ.get("OMP_NUM_THREADS")}
    if name.startswith("lm_head_"):
        # numpy float32 matrix-vector products + argmax over a 16384-row slice
        # of a weight of the same shape, scaled to the full vocabulary
        rng = np.random.default_rng(w["seed"])
        nv = 16384
        wt = (rng.standard_normal((nv, w["H"]), dtype=np.float32) * np.float32(w["H"] ** -0.5))
        xs = np.ascontiguousarray(w["hidden"].astype(np.uint32) << 16).view(np.float32)
        t0 = time.time()
        reps = 0
        scoring = name.startswith("lm_head_score")
        while time.time() < t0 + seconds or reps == 0:
            lg = xs @ wt.T
            if scoring:                                      # the log-sum-exp of each row
                m = lg.max(axis=1, keepdims=True)
                np.log(np.exp(lg - m).sum(axis=1))
            else:
                np.argmax(lg, axis=1)
            reps += 1
        dt = time.time() - t0
        full = dt * (w["V"] / nv) / reps                     # seconds per full-vocabulary call
        per_call, unit_c = (w["seqs"], "sequences/s") if "seqs" in w else (w["B"], "rows/s")
        info.update({"value": per_call / full, "unit": unit_c, "cores": many,
                     "sample": "%d x numpy float32 [%d, %d] x [%d, %d]^T + %s (a %d-row slice "
                               "of the vocabulary, scaled by V / %d), %.1f s" % (
                                   reps, w["B"], w["H"], nv, w["H"],
                                   "log-sum-exp" if scoring else "argmax", nv, nv, dt)})
        return info
    if name in ("topk_bf16", "eagle3_tree"):
        if name == "topk_bf16":
            unit = "calls/s"

            def fn():                    # topk<bf16> over the K rows (OpenMP over rows)
                orc.topk(w["logits"], w["k"])
                return 1
            what = "topk<bf16> calls over [%d, %d], k = %d" % (w["logits"].shape + (w["k"],))
        else:
            unit = "trees/s"

            def fn():
                orc.eagle3_tree(w["root"], w["levels"], w["d2t"], w["K"], w["depth"], w["total"],
                                w["sample_token"], cr=False)
                return 1
            what = "trees (K = %d, depth %d, %d tokens, Vd = %d)" % (
                w["K"], w["depth"], w["total"], w["root"].shape[0])
        v, reps, dt = timed(fn, 1)
        info.update({"value": v, "unit": unit, "cores": 1, "sample": f"{reps} {what}, {dt:.1f} s"})
        return info
    if name == "speculative":
        unit = "sequences/s"
        B = w["target"].shape[0]

        def fn():
            orc.verify_rejection(w["target"], w["draft"], w["draft_ids"], w["u_accept"],
                                 w["u_resample"])
            return B
        what = "verify_rejection over the full [16,8,128256] batch"
        one_row = False
    elif name in ("score_bf16", "mtp_masked_argmax"):
        unit = "rows/s"
        lg = w["logits"]
        state = {"r": 0}

        def fn():                        # one row per call, as the reference's functions
            r = state["r"] % lg.shape[0]
            state["r"] += 1
            if name == "score_bf16":
                orc.score_logits(lg[r], int(w["targets"][r]))
            else:
                cand = orc.select_candidate_tokens(w["centroids"][r], w["ordering"], w["top_k"])
                orc.masked_argmax(lg[r], cand)
            return 1
        what = f"rows of the {list(lg.shape)} batch, one call per row"
        one_row = True
    elif name == "argmax_bf16" or greedy_variant:
        unit = "rows/s"
        lg = w["logits"]
        state = {"r": 0}

        def fn():                        # _calc_next_token_id: one row, four threads
            r = state["r"] % lg.shape[0]
            state["r"] += 1
            orc.calc_next_token_id_omp4(lg[r])
            return 1
        what = f"rows of the {list(lg.shape)} batch, one _calc_next_token_id call (4 threads) per row"
        one_row = True
    else:
        unit = "rows/s"
        lg = w["logits"]
        cfg = orc.SamplerConfig(**w["cfg"])
        if w.get("cfg_rows"):                       # per-row settings: one config per row
            cfg = [orc.SamplerConfig(**{**w["cfg"], **{k: a[b].item() for k, a in
                                                       w["cfg_rows"].items()}})
                   for b in range(lg.shape[0])]

        def fn():
            orc.sample(lg, w["uniforms"], cfg, history=w["history"], bitmask=w["bitmask"])
            return lg.shape[0]
        what = f"the full {list(lg.shape)} batch"
        one_row = False
    if one_row:
        v, reps, dt = timed(fn, 1)
        info.update({"value": v, "unit": unit, "cores": 4 if "4 threads" in what else 1,
                     "sample": f"{reps} {what}, {dt:.1f} s"})
        return info
    v1, r1, d1 = timed(fn, 1)
    vm, rm, dm = timed(fn, many)
    info.update({"value": vm, "unit": unit, "cores": many,
                 "sample": f"{rm} x {what} at {many} threads, {dm:.1f} s",
                 "single_thread": {"value": v1, "unit": unit, "cores": 1,
                                   "sample": f"{r1} x {what}, {d1:.1f} s"}})
    return info


def _cpu_model():
    """lscpu's model name with its CPU family and model numbers (the
    /proc/cpuinfo line as a fallback)."""
    import subprocess
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        f = {}
        for line in out.splitlines():
            if ":" in line:
                k, v = line.split(":", 1)
                f[k.strip()] = v.strip()
        if "Model name" in f:
            extra = ", ".join("%s %s" % (k.lower(), f[k]) for k in ("CPU family", "Model") if k in f)
            return f["Model name"] + (" (%s)" % extra if extra else "")
    except (OSError, subprocess.SubprocessError):
        pass
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


if __name__ == "__main__":
    main()
