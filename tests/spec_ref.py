"""Independent float64 model of the sampler specification, used to pin the oracle.

It shares nothing with the oracle's arithmetic: probabilities are float64
softmaxes with numpy's exp, sums are float64, thresholds are compared as real
numbers.  The oracle's fixed-point weights must reproduce these decisions
except where a decision is within a relative 1e-6 of its boundary; such rows
are reported as "boundary" and excluded from id comparison.
"""
from __future__ import annotations

import numpy as np

EPS = 1e-6


def transformed_row(l, history=None, mask=None, cfg=None):
    """Mask / NaN / repetition / frequency / presence in float32 (same IEEE
    operations as the specification), then returns (l2, counts)."""
    cfg = cfg or {}
    l = np.array(l, dtype=np.float32)
    V = l.shape[0]
    l[np.isnan(l)] = -np.inf
    if mask is not None:
        bits = (mask[np.arange(V) >> 5] >> (np.arange(V) & 31).astype(np.uint32)) & 1
        l[bits == 0] = -np.inf
    counts = np.zeros(V, np.int64)
    if history is not None:
        h = np.asarray(history)
        h = h[(h >= 0) & (h < V)]
        np.add.at(counts, h, 1)
    R = np.float32(cfg.get("repetition_penalty", 1.0))
    a = np.float32(cfg.get("presence_penalty", 0.0))
    b = np.float32(cfg.get("frequency_penalty", 0.0))
    hit = counts > 0
    lh = l[hit]
    with np.errstate(invalid="ignore", over="ignore"):
        lh = np.where(lh < 0, lh * R, lh / R).astype(np.float32)
        lh = ((lh - b * counts[hit].astype(np.float32)).astype(np.float32) - a).astype(np.float32)
    l[hit] = lh
    return l, counts


def sample_row(l, u, history=None, mask=None, cfg=None):
    """Returns (token, prob, kept_bool_array, boundary_flag)."""
    cfg = cfg or {}
    l2, _ = transformed_row(l, history, mask, cfg)
    V = l2.shape[0]
    T = cfg.get("temperature", 1.0)
    if cfg.get("greedy", False) or not T > 0:
        if not np.isfinite(l2).any() and not (l2 == np.inf).any():
            return -1, 0.0, np.zeros(V, bool), False
        tok = int(np.argmax(l2))
        if l2[tok] == -np.inf:
            return -1, 0.0, np.zeros(V, bool), False
        kept = np.zeros(V, bool)
        kept[tok] = True
        return tok, 1.0, kept, False
    with np.errstate(over="ignore"):
        x = (l2 / np.float32(T)).astype(np.float32)
    k = int(cfg.get("top_k", 0))
    tau = -np.inf
    if 0 < k < V:
        tau = np.sort(x)[::-1][k - 1]
    kept = (x > -np.inf) & (x >= tau)
    if not kept.any():
        return -1, 0.0, kept, False
    xmax = x[kept].max()
    p = np.zeros(V, np.float64)
    with np.errstate(invalid="ignore"):
        d = x[kept].astype(np.float64) - np.float64(xmax)
    d[x[kept] == xmax] = 0.0
    p[kept] = np.exp(d)
    boundary = False
    top_p = cfg.get("top_p", 1.0)
    if top_p < 1.0:
        Z = p[kept].sum()
        xs = x[kept]
        ps = p[kept]
        order = np.argsort(-xs, kind="stable")
        xs_o, ps_o = xs[order], ps[order]
        # mass strictly above each value
        uniq, first = np.unique(-xs_o, return_index=True)
        cum = np.concatenate([[0.0], np.cumsum(ps_o)])
        above_o = cum[first[np.searchsorted(uniq, -xs_o)]]
        thr = top_p * Z
        keep_o = (above_o < thr) | (xs_o == xmax)
        if np.any(np.abs(above_o - thr) <= EPS * Z):
            boundary = True
        keep_p = np.zeros(len(xs), bool)
        keep_p[order] = keep_o
        idx = np.flatnonzero(kept)
        kept[idx[~keep_p]] = False
    min_p = cfg.get("min_p", 0.0)
    if min_p > 0:
        m = min(min_p, 1.0)
        pm = p[kept]
        if np.any(np.abs(pm - m) <= EPS):
            boundary = True
        idx = np.flatnonzero(kept)
        kept[idx[pm < m]] = False
    Zf = p[kept].sum()
    idx = np.flatnonzero(kept)
    c = np.cumsum(p[idx])
    t = np.float64(u) * Zf
    j = int(np.searchsorted(c, t, side="right"))
    j = min(j, len(idx) - 1)
    lo = c[j - 1] if j > 0 else 0.0
    if abs(t - lo) <= EPS * Zf or abs(c[j] - t) <= EPS * Zf:
        boundary = True
    tok = int(idx[j])
    return tok, float(p[tok] / Zf), kept, boundary


def verify_rejection_seq(tgt, drf, ids, ua, ur):
    """Float64 rejection sampling of one sequence -> (accepted_len, emitted, boundary)."""
    D = drf.shape[0]
    pt = _softmax(tgt)
    pd = _softmax(drf)
    em = [-1] * (D + 1)
    boundary = False
    for k in range(D):
        x = int(ids[k])
        lhs, rhs = pt[k, x], ua[k] * pd[k, x]
        if abs(lhs - rhs) <= EPS * max(lhs, rhs, 1e-300):
            boundary = True
        if lhs >= rhs:
            em[k] = x
            continue
        r = np.maximum(pt[k] - pd[k], 0.0)
        dist = r if r.sum() > 0 else pt[k]
        tok, b = _draw(dist, ur)
        em[k] = tok
        return k, em, boundary or b
    tok, b = _draw(pt[D], ur)
    em[D] = tok
    return D, em, boundary or b


def _softmax(x):
    x = np.asarray(x, np.float64)
    m = x.max(axis=-1, keepdims=True)
    e = np.exp(x - m)
    return e / e.sum(axis=-1, keepdims=True)


def _draw(p, u):
    Z = p.sum()
    c = np.cumsum(p)
    t = u * Z
    j = min(int(np.searchsorted(c, t, side="right")), len(p) - 1)
    lo = c[j - 1] if j > 0 else 0.0
    b = abs(t - lo) <= EPS * Z or abs(c[j] - t) <= EPS * Z
    return j, b
