"""CPU oracle for the logits -> token-selection path (numpy front end).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, always as the checker, never as the thing that is
measured for the GPU number or shipped.  The arithmetic lives in
oracle/llima_oracle.cpp (built by oracle/Makefile into oracle/_build/); this
module only marshals numpy arrays.  Each function names the reference code it
restates (sima-neat/llima, paths relative to that repository).
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from dataclasses import dataclass

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "liboracle.so")
_lib = None

F32, BF16 = 0, 1
ARGMAX_SPLIT_FIRST, ARGMAX_NEG_INF, ARGMAX_QUARTERS, ARGMAX_LOWEST = 0, 1, 2, 3


def build() -> str:
    """Compile the oracle with its Makefile (g++); returns the library path."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        _lib.orc_exp_neg.restype = ctypes.c_float
        _lib.orc_exp_neg.argtypes = [ctypes.c_float]
        _lib.orc_weight.restype = ctypes.c_uint64
        _lib.orc_weight.argtypes = [ctypes.c_float, ctypes.c_float]
    return _lib


class SamplerConfigC(ctypes.Structure):
    _fields_ = [
        ("temperature", ctypes.c_float),
        ("top_k", ctypes.c_int32),
        ("top_p", ctypes.c_float),
        ("min_p", ctypes.c_float),
        ("repetition_penalty", ctypes.c_float),
        ("presence_penalty", ctypes.c_float),
        ("frequency_penalty", ctypes.c_float),
        ("greedy", ctypes.c_int32),
    ]


@dataclass
class SamplerConfig:
    temperature: float = 1.0
    top_k: int = 0
    top_p: float = 1.0
    min_p: float = 0.0
    repetition_penalty: float = 1.0
    presence_penalty: float = 0.0
    frequency_penalty: float = 0.0
    greedy: bool = False

    def c(self) -> SamplerConfigC:
        return SamplerConfigC(self.temperature, self.top_k, self.top_p, self.min_p,
                              self.repetition_penalty, self.presence_penalty,
                              self.frequency_penalty, int(self.greedy))


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _logits(x):
    """Returns (contiguous array, dtype code). bf16 rows are passed as uint16 bits."""
    x = np.ascontiguousarray(x)
    if x.dtype == np.float32:
        return x, F32
    if x.dtype == np.uint16:
        return x, BF16
    raise TypeError(f"logits must be float32 or uint16 (bf16 bits), got {x.dtype}")


def exp_neg(d: float) -> float:
    return lib().orc_exp_neg(float(d))


def weight(x: float, xmax: float) -> int:
    return int(lib().orc_weight(float(x), float(xmax)))


def _bounds(V, split_dim, bounds):
    if bounds is None:
        sd = V if split_dim <= 0 or split_dim >= V else split_dim
        bounds = range(0, V, sd)
    return np.ascontiguousarray(list(bounds), np.int64)


def argmax(logits, split_dim: int = 0, mode: int = ARGMAX_SPLIT_FIRST, bounds=None):
    """argmax_bf16 / _argmax_lm_head_row semantics (utils.hpp:80-152,
    language_model.cpp:3616-3633, 3689-3714, language_model_eagle3.cpp:486-522,
    the spec path's multi-split scan language_model.cpp:1556-1575 as mode 3).
    bounds: explicit split starts (mode 0) instead of split_dim."""
    x, dt = _logits(logits)
    x2 = x.reshape(-1, x.shape[-1])
    B, V = x2.shape
    bd = _bounds(V, split_dim, bounds)
    ids = np.empty(B, np.int32)
    vals = np.empty(B, np.float32)
    rc = lib().orc_argmax_bounds(_ptr(x2), dt, B, V, ctypes.c_int64(V), _ptr(bd), len(bd), mode,
                                 _ptr(ids), _ptr(vals))
    if rc:
        raise ValueError(f"orc_argmax rc={rc}")
    return ids.reshape(x.shape[:-1]), vals.reshape(x.shape[:-1])


def sample(logits, uniforms, cfg, history=None, hist_len=None, bitmask=None,
           want_keep=False):
    """Written sampler specification (mask, penalties, temperature, top-k, top-p,
    min-p, inverse-CDF draw on fixed-point weights).  cfg: SamplerConfig or a
    list of B of them."""
    x, dt = _logits(logits)
    B, V = x.shape
    if isinstance(cfg, SamplerConfig):
        cfgs = (SamplerConfigC * 1)(cfg.c())
        stride = 0
    else:
        assert len(cfg) == B
        cfgs = (SamplerConfigC * B)(*[c.c() for c in cfg])
        stride = 1
    u = np.ascontiguousarray(uniforms, np.float32).reshape(B)
    H = 0
    if history is not None:
        history = np.ascontiguousarray(history, np.int32)
        H = history.shape[1]
        if hist_len is not None:
            hist_len = np.ascontiguousarray(hist_len, np.int32)
    if bitmask is not None:
        bitmask = np.ascontiguousarray(bitmask, np.uint32)
        assert bitmask.shape == (B, (V + 31) // 32)
    ids = np.empty(B, np.int32)
    probs = np.empty(B, np.float32)
    keep = np.zeros((B, (V + 31) // 32), np.uint32) if want_keep else None
    rc = lib().orc_sample(_ptr(x), dt, B, V, ctypes.c_int64(V), _ptr(history), _ptr(hist_len),
                          H, _ptr(bitmask), _ptr(u), cfgs, stride, _ptr(ids), _ptr(probs),
                          _ptr(keep))
    if rc:
        raise ValueError(f"orc_sample rc={rc}")
    return (ids, probs, keep) if want_keep else (ids, probs)


def resolve_draft_tokens(drafts, targets):
    """gemma4_mtp_helpers.cpp:81-111. Returns [(token, accepted)], raises RuntimeError."""
    d = np.ascontiguousarray(drafts, np.int32)
    t = np.ascontiguousarray(targets, np.int32)
    em = np.empty(len(d) + 1, np.int32)
    fl = np.empty(len(d) + 1, np.int32)
    n = ctypes.c_int(0)
    rc = lib().orc_resolve_draft_tokens(_ptr(d), len(d), _ptr(t), len(t), _ptr(em), _ptr(fl),
                                        ctypes.byref(n))
    if rc:
        raise RuntimeError("Invalid verification result" if len(t) == 0 or len(t) > len(d) + 1
                           else "verification ended without a mismatch or bonus token")
    return [(int(em[i]), bool(fl[i])) for i in range(n.value)]


def verify_greedy(target_logits, draft_ids, split_dim: int = 0, mode: int = ARGMAX_SPLIT_FIRST,
                  bounds=None):
    """Per-row argmax (as argmax) of [B, D+1, V] target rows, then
    resolve_draft_tokens per sequence -> (accepted_len [B], emitted [B, D+1])."""
    x, dt = _logits(target_logits)
    B, D1, V = x.shape
    bd = _bounds(V, split_dim, bounds)
    d = np.ascontiguousarray(draft_ids, np.int32).reshape(B, D1 - 1)
    acc = np.empty(B, np.int32)
    em = np.empty((B, D1), np.int32)
    rc = lib().orc_verify_greedy(_ptr(x), dt, B, D1 - 1, V, _ptr(bd), len(bd), mode, _ptr(d),
                                 _ptr(acc), _ptr(em))
    if rc:
        raise ValueError(f"orc_verify_greedy rc={rc}")
    return acc, em


def verify_rejection(target_logits, draft_logits, draft_ids, u_accept, u_resample):
    t = np.ascontiguousarray(target_logits, np.float32)
    dl = np.ascontiguousarray(draft_logits, np.float32)
    B, D1, V = t.shape
    D = D1 - 1
    assert dl.shape == (B, D, V)
    ids = np.ascontiguousarray(draft_ids, np.int32).reshape(B, D)
    ua = np.ascontiguousarray(u_accept, np.float32).reshape(B, D)
    ur = np.ascontiguousarray(u_resample, np.float32).reshape(B)
    acc = np.empty(B, np.int32)
    em = np.empty((B, D1), np.int32)
    rc = lib().orc_verify_rejection(_ptr(t), _ptr(dl), B, D, V, _ptr(ids), _ptr(ua), _ptr(ur),
                                    _ptr(acc), _ptr(em))
    if rc:
        raise ValueError(f"orc_verify_rejection rc={rc}")
    return acc, em


def evaluate_posterior(next_ids, candidates):
    """eagle_helpers.hpp:153-195 -> (best_candidate, accept_length, bonus_token)."""
    n = np.ascontiguousarray(next_ids, np.int32)
    c = np.ascontiguousarray(candidates, np.int32)
    P, L = c.shape
    best, acc, bonus = ctypes.c_int32(), ctypes.c_int32(), ctypes.c_int32()
    rc = lib().orc_evaluate_posterior(_ptr(n), _ptr(c), P, L, ctypes.byref(best),
                                      ctypes.byref(acc), ctypes.byref(bonus))
    if rc:
        raise ValueError(f"orc_evaluate_posterior rc={rc}")
    return best.value, acc.value, bonus.value


def tree_gather(row_tokens, retrieve):
    """language_model_eagle3.cpp:551-567."""
    r = np.ascontiguousarray(row_tokens, np.int32)
    ri = np.ascontiguousarray(retrieve, np.int32)
    P, L = ri.shape
    out = np.empty((P, L), np.int32)
    rc = lib().orc_tree_gather(_ptr(r), len(r), _ptr(ri), P, L, _ptr(out))
    if rc:
        raise ValueError(f"orc_tree_gather rc={rc}")
    return out


def select_candidate_tokens(centroid_bf16_bits, ordering, top_k):
    """gemma4_mtp_helpers.cpp:113-167. Raises RuntimeError like the reference."""
    c = np.ascontiguousarray(centroid_bf16_bits, np.uint16)
    o = np.ascontiguousarray(ordering, np.uint32)
    out = np.empty(max(len(o), 1), np.uint32)
    n = ctypes.c_int(0)
    rc = lib().orc_select_candidate_tokens(_ptr(c), len(c), _ptr(o), len(o), int(top_k),
                                           _ptr(out), ctypes.byref(n))
    if rc:
        raise RuntimeError(f"select_candidate_tokens rc={rc}")
    return out[:n.value].copy()


def masked_argmax(row, candidates):
    """language_model_gemma4_mtp.cpp:31-97 (argmax over candidate ids only)."""
    x, dt = _logits(row)
    c = np.ascontiguousarray(candidates, np.uint32)
    out = ctypes.c_int32()
    rc = lib().orc_masked_argmax(_ptr(x), dt, x.shape[-1], _ptr(c), len(c), ctypes.byref(out))
    if rc:
        raise RuntimeError("masked lm_head selected no token")
    return out.value


def score_logits(row, target):
    """language_model.cpp:29-62 -> (logprob: float64, is_greedy: bool)."""
    x, dt = _logits(row)
    lp = ctypes.c_double()
    g = ctypes.c_int32()
    rc = lib().orc_score_logits(_ptr(x), dt, x.shape[-1], int(target), ctypes.byref(lp),
                                ctypes.byref(g))
    if rc:
        raise RuntimeError(f"Target token id {target} is outside logits vocabulary size")
    return lp.value, bool(g.value)


# ---------------------------------------------------------------- helpers for tests
def f32_to_bf16_bits(x):
    """Round-to-nearest-even fp32 -> bf16 bit pattern (NaN kept quiet)."""
    x = np.ascontiguousarray(x, np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(x)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def bf16_bits_to_f32(h):
    return (np.ascontiguousarray(h, np.uint16).astype(np.uint32) << 16).view(np.float32)


def topk(x, k: int):
    """topk<T> (utils.hpp:216-281): heap top-k per row -> (indices int32
    [rows, k], values float32 [rows, k]) in the heap's output order."""
    a, dt = _logits(x)
    a2 = a.reshape(-1, a.shape[-1])
    rows, cols = a2.shape
    idx = np.empty((rows, k), np.int32)
    val = np.empty((rows, k), np.float32)
    rc = lib().orc_topk(_ptr(a2), dt, rows, ctypes.c_int64(cols), ctypes.c_int64(cols), k,
                        _ptr(idx), _ptr(val))
    if rc:
        raise ValueError(f"orc_topk rc={rc}")
    return idx.reshape(a.shape[:-1] + (k,)), val.reshape(a.shape[:-1] + (k,))


def logsoftmax(values, cr: bool = False):
    """logsoftmax<T> (utils.hpp:283-301) in float; cr selects exp/log rounded
    once from double (the HIP path's arithmetic) instead of the C library's."""
    v = np.ascontiguousarray(values, np.float32).reshape(-1)
    out = np.empty_like(v)
    rc = lib().orc_logsoftmax(_ptr(v), len(v), int(cr), _ptr(out))
    if rc:
        raise ValueError(f"orc_logsoftmax rc={rc}")
    return out


def eagle3_tree(root_logits, level_logits, d2t, K: int, depth: int, total_tokens: int,
                sample_token: int, cr: bool = True):
    """The selection side of the EAGLE3 draft tree (language_model_eagle3.cpp:
    808-1164).  root_logits [Vd], level_logits [depth-1, K, Vd] (float32 or
    bf16 bits), d2t int32 [Vd].  Returns a dict of the per-level input ids and
    parent rows, the draft masks, and the final tokens, tree mask, position
    ids and retrieve indices."""
    r, dt = _logits(root_logits)
    Vd = r.shape[-1]
    if depth > 1:
        lv, dt2 = _logits(level_logits)
        assert dt2 == dt and lv.shape == (depth - 1, K, Vd)
    else:
        lv = np.zeros((1, K, Vd), r.dtype)
    d = np.ascontiguousarray(d2t, np.int32)
    N = total_tokens + 1
    inputs = np.zeros((depth, K), np.int32)
    prow = np.zeros((max(depth - 1, 1), K), np.int32)
    masks = np.zeros((max(depth - 1, 1), K, K * depth), np.float32)
    tokens = np.zeros(N, np.int32)
    mask = np.zeros((N, N), np.float32)
    pos = np.zeros(N, np.int32)
    retrieve = np.zeros((N, N), np.int32)
    dims = np.zeros(2, np.int32)
    node_scores = np.zeros(K + (depth - 1) * K * K, np.float32)
    rc = lib().orc_eagle3_tree(_ptr(r), _ptr(lv), dt, Vd, _ptr(d), K, depth, total_tokens,
                               int(sample_token), int(cr), _ptr(inputs), _ptr(prow), _ptr(masks),
                               _ptr(tokens), _ptr(mask), _ptr(pos), _ptr(retrieve), _ptr(dims),
                               _ptr(node_scores))
    if rc:
        raise ValueError(f"orc_eagle3_tree rc={rc}")
    leaves, rcols = int(dims[0]), int(dims[1])
    return dict(inputs=inputs, parent_rows=prow[:depth - 1], masks=masks[:depth - 1],
                tokens=tokens, tree_mask=mask, position_ids=pos,
                retrieve=retrieve[:leaves, :rcols], node_scores=node_scores)


def stop_check(tokens, stop_ids, count=None, room=None):
    """The decode loops' stop rule -> (keep [B], status [B]: 0 none, 1 stop
    token, 2 cut by the cache room)."""
    t = np.ascontiguousarray(tokens, np.int32)
    B, M = t.shape
    st = np.ascontiguousarray(list(stop_ids), np.int32)
    c = None if count is None else np.ascontiguousarray(count, np.int32)
    r = None if room is None else np.ascontiguousarray(room, np.int32)
    keep = np.empty(B, np.int32)
    status = np.empty(B, np.int32)
    rc = lib().orc_stop_check(_ptr(t), _ptr(c), B, M, _ptr(st), len(st), _ptr(r), _ptr(keep),
                              _ptr(status))
    if rc:
        raise ValueError(f"orc_stop_check rc={rc}")
    return keep, status


def calc_next_token_id_omp4(row) -> int:
    """_calc_next_token_id (language_model.cpp:3689-3714) with its four OpenMP
    threads (CPU baseline of the greedy workloads)."""
    x, dt = _logits(np.ascontiguousarray(row).reshape(-1))
    out = ctypes.c_int32()
    rc = lib().orc_calc_next_token_id_omp4(_ptr(x), dt, len(x), ctypes.byref(out))
    if rc:
        raise ValueError(f"orc_calc_next_token_id_omp4 rc={rc}")
    return int(out.value)


def set_threads(n: int) -> None:
    lib().orc_set_threads(int(n))


def vr_weights(row):
    """Rejection verification's per-id weights W (uint64) and Z (int) of one row."""
    x = np.ascontiguousarray(row, np.float32).reshape(-1)
    W = np.empty(len(x), np.uint64)
    Z2 = np.empty(2, np.uint64)
    rc = lib().orc_vr_weights(_ptr(x), len(x), _ptr(W), _ptr(Z2))
    if rc:
        raise ValueError(f"orc_vr_weights rc={rc}")
    return W, int(Z2[0]) + (int(Z2[1]) << 64)
