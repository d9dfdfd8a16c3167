"""Seeded synthetic inputs for the five token-selection workloads (NumPy PCG64,
seed = 1000 + workload number).  Shapes follow the head shapes of the models the
reference runtime ships configs for (Qwen2.5 V=151936, Llama-3 V=128256, Gemma
V=262144: tests/compilation/configuration/references/*_vlm_config.json in the
reference).  Every generator accepts smaller B / V / H for quick tests.

Each returns a dict of host numpy arrays:
  logits  float32 [B, V]   (or uint16 bf16 bit patterns for the bf16 workload)
  history int32 [B, H] or None, uniforms float32 [B], bitmask uint32 [B, V/32] or None,
  cfg     dict of sampler settings (SamplerConfig field names).
"""
from __future__ import annotations

import numpy as np


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even fp32 -> bf16 bit patterns (NaN stays NaN)."""
    x = np.ascontiguousarray(x, np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(x)
    if nan.any():
        r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def bf16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(h, np.uint16).astype(np.uint32) << 16).view(np.float32)


def _normal(rng, shape, sigma):
    return (rng.standard_normal(shape, dtype=np.float32) * np.float32(sigma)).astype(np.float32)


def single_row(B=1, V=151936, H=64, seed=1001):
    """Batch 1, fp32 vocab 151936 (Qwen2.5 head), N(0, 3^2) with 20 hot ids +8;
    repetition 1.1 over a 64-id uniform history, T 0.7, top-k 40, top-p 0.9."""
    rng = np.random.Generator(np.random.PCG64(seed))
    logits = _normal(rng, (B, V), 3.0)
    for b in range(B):
        hot = rng.choice(V, size=min(20, V), replace=False)
        logits[b, hot] += np.float32(8.0)
    history = rng.integers(0, V, size=(B, H), dtype=np.int32)
    u = rng.random(B, dtype=np.float32)
    cfg = dict(temperature=0.7, top_k=40, top_p=0.9, repetition_penalty=1.1)
    return dict(name="single_row", logits=logits, history=history, uniforms=u, bitmask=None,
                cfg=cfg)


def zipf_ids(rng, V, n, s=1.1):
    """n ids from a Zipf(s) law truncated to ranks 1..V, ranks mapped to ids by
    a seeded permutation."""
    ranks = np.arange(1, V + 1, dtype=np.float64)
    cdf = np.cumsum(ranks ** -s)
    cdf /= cdf[-1]
    perm = rng.permutation(V).astype(np.int32)
    r = np.searchsorted(cdf, rng.random(n), side="right")
    return perm[np.minimum(r, V - 1)]


def batched_penalties(B=64, V=128256, H=2048, seed=1002):
    """B=64, fp32 vocab 128256 (Llama-3 head), N(0, 4^2); 2048-id Zipf(1.1)
    history per row; repetition 1.15, presence 0.5, frequency 0.3, T 0.8,
    top-k 50, top-p 0.95, min-p 0.05."""
    rng = np.random.Generator(np.random.PCG64(seed))
    logits = _normal(rng, (B, V), 4.0)
    history = np.stack([zipf_ids(rng, V, H) for _ in range(B)]).astype(np.int32)
    u = rng.random(B, dtype=np.float32)
    cfg = dict(temperature=0.8, top_k=50, top_p=0.95, min_p=0.05, repetition_penalty=1.15,
               presence_penalty=0.5, frequency_penalty=0.3)
    return dict(name="batched_penalties", logits=logits, history=history, uniforms=u,
                bitmask=None, cfg=cfg)


def constrained(B=32, V=151936, runs=47, seed=1003):
    """B=32, fp32 vocab 151936, N(0, 3^2); a packed uint32 grammar bitmask with
    about 2% of the ids allowed in 64-id runs at 64-aligned starts; each row's
    maximum is moved onto a masked-out id; T 1.0, top-p 0.9."""
    rng = np.random.Generator(np.random.PCG64(seed))
    logits = _normal(rng, (B, V), 3.0)
    nw = (V + 31) // 32
    mask = np.zeros((B, nw), np.uint32)
    nblocks = V // 64
    for b in range(B):
        blocks = rng.choice(nblocks, size=min(runs, nblocks), replace=False)
        for blk in blocks:
            mask[b, 2 * blk] = 0xFFFFFFFF
            mask[b, 2 * blk + 1] = 0xFFFFFFFF
        allowed = ((mask[b, np.arange(V) >> 5] >> (np.arange(V) & 31).astype(np.uint32)) & 1)
        banned = np.flatnonzero(allowed == 0)
        j = banned[rng.integers(0, len(banned))]
        logits[b, j] = logits[b].max() + np.float32(5.0)
    u = rng.random(B, dtype=np.float32)
    cfg = dict(temperature=1.0, top_p=0.9)
    return dict(name="constrained", logits=logits, history=None, uniforms=u, bitmask=mask,
                cfg=cfg)


def constrained_half(B=32, V=151936, seed=1011):
    """The C3 rows (B=32, fp32 vocab 151936, N(0, 3^2)) under a grammar mask
    that allows about half of the ids (independent bits), each row's maximum
    moved onto a masked-out id; T 1.0, top-p 0.9.  About 4700 candidates per
    16 KB chunk pass the weight window: no candidate region holds them, so
    the finish takes every row through its full-row path."""
    rng = np.random.Generator(np.random.PCG64(seed))
    logits = _normal(rng, (B, V), 3.0)
    nw = (V + 31) // 32
    mask = rng.integers(0, 2**32, size=(B, nw), dtype=np.uint64).astype(np.uint32)
    ids = np.arange(V)
    for b in range(B):
        allowed = (mask[b, ids >> 5] >> (ids & 31).astype(np.uint32)) & 1
        banned = np.flatnonzero(allowed == 0)
        j = banned[rng.integers(0, len(banned))]
        logits[b, j] = logits[b].max() + np.float32(5.0)
    u = rng.random(B, dtype=np.float32)
    return dict(name="constrained_half", logits=logits, history=None, uniforms=u, bitmask=mask,
                cfg=dict(temperature=1.0, top_p=0.9))


def _softmax64(x):
    x = x.astype(np.float64)
    x = x - x.max(axis=-1, keepdims=True)
    e = np.exp(x)
    return e / e.sum(axis=-1, keepdims=True)


def speculative(B=16, D=7, V=128256, seed=1004):
    """EAGLE3-style verification: target [B, D+1, V] ~ N(0, 4^2); draft =
    target[:, :D] + N(0, 1.5^2); draft ids drawn from the draft softmax."""
    rng = np.random.Generator(np.random.PCG64(seed))
    tgt = _normal(rng, (B, D + 1, V), 4.0)
    drf = (tgt[:, :D] + _normal(rng, (B, D, V), 1.5)).astype(np.float32)
    ids = np.empty((B, D), np.int32)
    for b in range(B):
        p = _softmax64(drf[b])
        c = np.cumsum(p, axis=-1)
        r = rng.random(D)
        ids[b] = np.minimum((c < r[:, None]).sum(axis=-1), V - 1)
    ua = rng.random((B, D), dtype=np.float32)
    ur = rng.random(B, dtype=np.float32)
    return dict(name="speculative", target=tgt, draft=drf, draft_ids=ids, u_accept=ua,
                u_resample=ur)


def large_vocab_bf16(B=256, V=262144, H=512, seed=1005):
    """B=256, bf16 vocab 262144 (Gemma head), N(0, 5^2) soft-capped 30*tanh(x/30);
    repetition 1.05 over a 512-id uniform history, T 1.0, top-k 64, top-p 0.95."""
    rng = np.random.Generator(np.random.PCG64(seed))
    x = _normal(rng, (B, V), 5.0)
    x = (np.float32(30.0) * np.tanh(x / np.float32(30.0))).astype(np.float32)
    logits = f32_to_bf16_bits(x)
    history = rng.integers(0, V, size=(B, H), dtype=np.int32)
    u = rng.random(B, dtype=np.float32)
    cfg = dict(temperature=1.0, top_k=64, top_p=0.95, repetition_penalty=1.05)
    return dict(name="large_vocab_bf16", logits=logits, history=history, uniforms=u,
                bitmask=None, cfg=cfg)


def score_bf16(B=256, V=262144, seed=1006):
    """Log-likelihood scoring (score_logits) of B target ids over the bf16
    Gemma-head rows of large_vocab_bf16 (same logits, seeded targets)."""
    w = large_vocab_bf16(B=B, V=V, H=1)
    rng = np.random.Generator(np.random.PCG64(seed))
    targets = rng.integers(0, V, size=B, dtype=np.int32)
    return dict(name="score_bf16", logits=w["logits"], targets=targets)


def mtp_masked_argmax(B=16, C=2048, V=262144, top_k=32, seed=1007):
    """Gemma4 MTP drafting: B rows of bf16 centroid logits [B, C] (2048 centroids,
    top-32, the reference's defaults: vlm_config.py:780-781), a seeded token
    ordering (a permutation of V) and bf16 N(0, 5^2) soft-capped logits [B, V]."""
    rng = np.random.Generator(np.random.PCG64(seed))
    cent = f32_to_bf16_bits(_normal(rng, (B, C), 2.0))
    ordering = rng.permutation(V).astype(np.uint32)
    x = _normal(rng, (B, V), 5.0)
    x = (np.float32(30.0) * np.tanh(x / np.float32(30.0))).astype(np.float32)
    return dict(name="mtp_masked_argmax", logits=f32_to_bf16_bits(x), centroids=cent,
                ordering=ordering, top_k=top_k)


def lm_head_argmax(B=1, H=4096, V=128256, seed=1008):
    """LM head + argmax at decode: B bf16 hidden rows of width H = 4096 against a
    bf16 [V, H] weight with V = 128256 (a Llama-3-8B head, 1.05 GB).  The weight,
    N(0, 1/H), is generated on the device from the seed (torch), the hidden rows
    ~ N(0, 1) here."""
    rng = np.random.Generator(np.random.PCG64(seed))
    hidden = f32_to_bf16_bits(_normal(rng, (B, H), 1.0))
    return dict(name="lm_head_argmax", hidden=hidden, B=B, H=H, V=V, seed=seed)


def top_p_only(B=64, V=128256, seed=1002):
    """The headline rows (B=64, fp32 vocab 128256, N(0, 4^2)) sampled with
    top-p alone: T 1.0, top-p 0.9, no top-k, no penalties, no mask.  Nearly
    every value lies within 27 T of its chunk's maximum, so no candidate bound
    narrows the row: the sampler's dense path (every chunk's workgroup takes
    part in each of its passes)."""
    rng = np.random.Generator(np.random.PCG64(seed))
    logits = _normal(rng, (B, V), 4.0)
    u = rng.random(B, dtype=np.float32)
    return dict(name="top_p_only", logits=logits, history=None, uniforms=u, bitmask=None,
                cfg=dict(temperature=1.0, top_p=0.9))


def batched_penalties_rows(B=64, V=128256, H=2048, seed=1002):
    """The headline workload with every setting passed as a per-row array (a
    serving batch whose requests each carry their own sampler settings); the
    values are the headline's.  cfg_rows names the fields given per row."""
    w = batched_penalties(B, V, H, seed)
    w["name"] = "batched_penalties_rows"
    w["cfg_rows"] = {k: np.full(B, v, np.int32 if k == "top_k" else np.float32)
                     for k, v in w["cfg"].items()}
    return w


def mixed_topk_rows(B=64, V=128256, seed=1002):
    """The headline rows (no history) as a per-request serving batch: even
    rows sample with top-k 50 and top-p 0.95, odd rows with top-p 0.9 alone
    (per-row top_k 0), all at T 1.0."""
    rng = np.random.Generator(np.random.PCG64(seed))
    logits = _normal(rng, (B, V), 4.0)
    u = rng.random(B, dtype=np.float32)
    even = (np.arange(B) % 2) == 0
    rows = dict(top_k=np.where(even, 50, 0).astype(np.int32),
                top_p=np.where(even, 0.95, 0.9).astype(np.float32))
    return dict(name="mixed_topk_rows", logits=logits, history=None, uniforms=u, bitmask=None,
                cfg=dict(temperature=1.0, top_k=50, top_p=0.95), cfg_rows=rows)


def topk_bf16(rows=5, cols=32000, k=5, seed=1009):
    """One EAGLE3 draft level's row top-k as the reference calls it
    (language_model_eagle3.cpp:914-920): topk<bf16> over K = 5 rows of a
    32000-id draft vocabulary, k = 5.  Draft logits ~ N(0, 3^2), bf16."""
    rng = np.random.Generator(np.random.PCG64(seed))
    x = f32_to_bf16_bits(_normal(rng, (rows, cols), 3.0))
    return dict(name="topk_bf16", logits=x, k=k)


def eagle3_tree(K=5, depth=4, total=15, Vd=32000, V=128256, seed=1010):
    """The EAGLE3 draft tree at the reference's shape (topk_generate,
    language_model_eagle3.cpp:808-1164): K = 5, depth 4, 15 draft tokens, a
    32000-id bf16 draft vocabulary mapped to 128256 target ids by d2t.  The
    draft logits of every level are given (the draft model's forward passes
    between levels are the caller's): root [Vd], levels [depth - 1, K, Vd],
    ~ N(0, 3^2)."""
    rng = np.random.Generator(np.random.PCG64(seed))
    root = f32_to_bf16_bits(_normal(rng, (Vd,), 3.0))
    levels = f32_to_bf16_bits(_normal(rng, (depth - 1, K, Vd), 3.0))
    d2t = (np.sort(rng.choice(V, Vd, replace=False)) - np.arange(Vd)).astype(np.int32)
    return dict(name="eagle3_tree", root=root, levels=levels, d2t=d2t, K=K, depth=depth,
                total=total, sample_token=int(rng.integers(0, V)))


WORKLOADS = {
    "topk_bf16": topk_bf16,
    "eagle3_tree": eagle3_tree,
    "batched_penalties_rows": batched_penalties_rows,
    "mixed_topk_rows": mixed_topk_rows,
    "single_row": single_row,
    "batched_penalties": batched_penalties,
    "constrained": constrained,
    "constrained_half": constrained_half,
    "top_p_only": top_p_only,
    "speculative": speculative,
    "large_vocab_bf16": large_vocab_bf16,
    "score_bf16": score_bf16,
    "mtp_masked_argmax": mtp_masked_argmax,
    "lm_head_argmax": lm_head_argmax,
    "lm_head_argmax_b64": lambda: dict(lm_head_argmax(B=64), name="lm_head_argmax_b64"),
    "lm_head_argmax_b128": lambda: dict(lm_head_argmax(B=128), name="lm_head_argmax_b128"),
    "lm_head_argmax_b256": lambda: dict(lm_head_argmax(B=256), name="lm_head_argmax_b256"),
    "lm_head_argmax_b64_packed": lambda: dict(lm_head_argmax(B=64), name="lm_head_argmax_b64_packed"),
    "lm_head_argmax_b32_packed": lambda: dict(lm_head_argmax(B=32), name="lm_head_argmax_b32_packed"),
    "lm_head_argmax_b128_packed": lambda: dict(lm_head_argmax(B=128), name="lm_head_argmax_b128_packed"),
    "lm_head_score_b64_packed": lambda: dict(lm_head_argmax(B=64), name="lm_head_score_b64_packed"),
    "lm_head_verify_b16_d7": lambda: dict(lm_head_argmax(B=128), name="lm_head_verify_b16_d7",
                                          seqs=16, D=7),
}
