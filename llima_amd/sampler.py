"""Host API of the MI355X token-selection path.

Function names and argument meanings follow the reference runtime's selection
functions (sima-neat/llima, paths relative to that repository); the compute
runs in the HIP kernels of libllima_sampler.so, and torch ROCm tensors are only
the buffers handed to it (inputs must already be on the GPU).

  argmax_bf16(values)                 utils.hpp:80-152
  calc_next_token_id(logits)          language_model.cpp:3689-3714
  argmax_lm_head_rows(rows, drafts)   language_model.cpp:3636-3687
  spec_path_argmax(logits, row)       language_model.cpp:1518-1611
  resolve_draft_tokens(...)           gemma4_mtp_helpers.cpp:81-111 (via verify_greedy)
  evaluate_posterior / verify_tree    eagle_helpers.hpp:153-195, language_model_eagle3.cpp:530-567
  sample(...)                         the sampler stages (no reference counterpart)
  verify_rejection(...)               stochastic draft verification (no reference counterpart)
  score_logits(logits, target)        language_model.cpp:29-62
  select_candidate_tokens(...)        gemma4_mtp_helpers.cpp:113-167
  argmax_gemma4_mtp_masked_row(s)     language_model_gemma4_mtp.cpp:31-97
  topk(x, k)                          utils.hpp:216-281
  stop_check(tokens, stop_mask, V)    language_model.cpp:643-671 (the decode loops' stop rule)
  Eagle3DraftTree                     language_model_eagle3.cpp:808-1164 (topk_generate's selection)

Errors: the reference throws std::invalid_argument / std::runtime_error; here
ValueError / RuntimeError are raised for the same conditions.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np
from typing import Optional

import torch

from . import _lib
from ._lib import check, lib

__all__ = [
    "SamplerConfig", "argmax", "argmax_bf16", "calc_next_token_id", "argmax_lm_head_rows",
    "spec_path_argmax",
    "sample", "verify_greedy", "resolve_draft_tokens", "verify_tree", "verify_rejection",
    "Workspace", "score_logits", "select_candidate_tokens", "argmax_gemma4_mtp_masked_rows",
    "argmax_gemma4_mtp_masked_row", "topk", "Eagle3DraftTree", "stop_mask", "stop_check",
    "lm_head_argmax", "lm_head_pack", "PackedLmHead",
]


@dataclass
class SamplerConfig:
    """Per-step sampler settings (HF GenerationConfig names plus OpenAI
    presence/frequency penalties).  Any field may instead be a CUDA tensor of
    shape [B] giving a per-row value."""
    temperature: float | torch.Tensor = 1.0
    top_k: int | torch.Tensor = 0
    top_p: float | torch.Tensor = 1.0
    min_p: float | torch.Tensor = 0.0
    repetition_penalty: float | torch.Tensor = 1.0
    presence_penalty: float | torch.Tensor = 0.0
    frequency_penalty: float | torch.Tensor = 0.0
    greedy: bool = False
    # per-row top_k only: every row's entry is in (0, V).  Found by itself when
    # the per-row top_k is given in host memory; a device tensor needs the
    # caller's word.  It lets the call skip the finish that can split rows
    # without top-k; a wrong True costs time (such a row takes the slower
    # full-row path), never the result.
    top_k_every_row: bool = False

    def to_c(self, B: int, device, V: int | None = None) -> tuple[_lib.SamplerConfigC, list]:
        c = _lib.SamplerConfigC()
        keep = []
        for name, dtype, default in (("temperature", torch.float32, 1.0),
                                     ("top_k", torch.int32, 0),
                                     ("top_p", torch.float32, 1.0),
                                     ("min_p", torch.float32, 0.0),
                                     ("repetition_penalty", torch.float32, 1.0),
                                     ("presence_penalty", torch.float32, 0.0),
                                     ("frequency_penalty", torch.float32, 0.0)):
            v = getattr(self, name)
            if isinstance(v, torch.Tensor):
                t = v.to(device=device, dtype=dtype).contiguous()
                if t.numel() != B:
                    raise ValueError(f"{name} has {t.numel()} values for {B} rows")
                keep.append(t)
                setattr(c, name, default)
                setattr(c, name + "_rows", t.data_ptr())
            else:
                setattr(c, name, v)
                setattr(c, name + "_rows", None)
        c.greedy = int(bool(self.greedy))
        k = self.top_k
        if isinstance(k, torch.Tensor):
            every = self.top_k_every_row
            if not every and k.device.type == "cpu" and k.numel() > 0:
                every = bool((k > 0).all()) and (V is None or bool((k < V).all()))
            c.top_k = 1 if every else 0                  # the statement (header: top_k)
        return c, keep


class Workspace:
    """Scratch buffers per (device, current stream, entry point), grown on
    demand.  The kernels keep no state in them between calls, so one buffer
    serves calls of any shape; allocation happens only when a call needs more
    than any earlier call on that stream.  Calls on one stream are ordered, so
    they may share a buffer; each stream has its own, so calls on different
    streams never race on scratch, and a buffer is allocated on (and returned
    to torch's caching allocator under) the stream that uses it."""
    _bufs: dict = {}

    @classmethod
    def get(cls, device: torch.device, kind: str, nbytes: int) -> torch.Tensor:
        stream = torch.cuda.current_stream(device)
        key = (device.index, stream.cuda_stream, kind)
        buf = cls._bufs.get(key)
        if buf is None or buf.numel() < nbytes:
            with torch.cuda.stream(stream):
                buf = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=device)
            cls._bufs[key] = buf
        return buf


def _stream(device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _dtype_code(t: torch.Tensor) -> int:
    if t.dtype == torch.float32:
        return _lib.LLIMA_F32
    if t.dtype == torch.bfloat16:
        return _lib.LLIMA_BF16
    raise ValueError(f"logits must be float32 or bfloat16, got {t.dtype}")


def _on_gpu(*ts):
    for t in ts:
        if t is not None and not t.is_cuda:
            raise ValueError("tensors must be on a ROCm device")


def _ptr(t: Optional[torch.Tensor]):
    return None if t is None else t.data_ptr()


def _rows2d(logits: torch.Tensor) -> torch.Tensor:
    if logits.dim() == 1:
        logits = logits.unsqueeze(0)
    if logits.dim() != 2:
        raise ValueError("logits must be [V] or [B, V]")
    if logits.stride(-1) != 1:
        logits = logits.contiguous()
    return logits


MODES = {"split_first": _lib.ARGMAX_SPLIT_FIRST, "neg_inf": _lib.ARGMAX_NEG_INF,
         "quarters": _lib.ARGMAX_QUARTERS, "lowest": _lib.ARGMAX_LOWEST}


def _split_arrays(splits):
    """Host arrays describing split buffers [..., w_i] (last dim contiguous):
    (pointers, widths, row strides, rows, V, dtype code, keep-alive list)."""
    if not 1 <= len(splits) <= _lib.MAX_SPLITS:
        raise ValueError(f"1..{_lib.MAX_SPLITS} split buffers are supported")
    xs = []
    for t in splits:
        t = t.reshape(-1, t.shape[-1])
        if t.stride(-1) != 1:
            t = t.contiguous()
        xs.append(t)
    rows, dt = xs[0].shape[0], _dtype_code(xs[0])
    for t in xs:
        if t.shape[0] != rows or _dtype_code(t) != dt or t.device != xs[0].device:
            raise ValueError("split buffers must share rows, dtype and device")
    _on_gpu(*xs)
    n = len(xs)
    ptrs = (ctypes.c_void_p * n)(*[t.data_ptr() for t in xs])
    widths = (ctypes.c_int32 * n)(*[t.shape[1] for t in xs])
    strides = (ctypes.c_int64 * n)(*[t.stride(0) for t in xs])
    return ptrs, widths, strides, rows, sum(t.shape[1] for t in xs), dt, xs


def argmax(logits, split_dim: int = 0, mode: str = "split_first"):
    """Greedy selection over [B, V] rows -> (ids int32 [B], values float32 [B]).

    logits: one [B, V] tensor, or a list of split buffers [B, w_i] holding
    consecutive vocabulary ranges (the reference's n{N}_lm_split{i} buffers,
    language_model.cpp:3584-3613), each buffer then being a split.
    mode "split_first": per split of split_dim values, argmax_bf16 semantics
    (utils.hpp:80-152) merged as _argmax_lm_head_row (language_model.cpp:3616-3633);
    "neg_inf": the EAGLE3 verify scan (language_model_eagle3.cpp:486-522);
    "quarters": _calc_next_token_id's four-way split (language_model.cpp:3689-3714);
    "lowest": the speculative path's multi-split scan from bf16 lowest()
    (language_model.cpp:1556-1575)."""
    if isinstance(logits, (list, tuple)):
        ptrs, widths, strides, B, V, dt, keep = _split_arrays(logits)
        dev = keep[0].device
        ids = torch.empty(B, dtype=torch.int32, device=dev)
        vals = torch.empty(B, dtype=torch.float32, device=dev)
        ws = Workspace.get(dev, "argmax", lib().llima_argmax_workspace_bytes(B, V, dt))
        check(lib().llima_argmax_splits(ptrs, widths, strides, len(keep), dt, B, MODES[mode],
                                        ids.data_ptr(), vals.data_ptr(), ws.data_ptr(),
                                        ws.numel(), _stream(dev)), "llima_argmax_splits")
        return ids, vals
    x = _rows2d(logits)
    _on_gpu(x)
    B, V = x.shape
    if V == 0:
        raise ValueError("argmax_bf16 requires at least one value")
    dev = x.device
    ids = torch.empty(B, dtype=torch.int32, device=dev)
    vals = torch.empty(B, dtype=torch.float32, device=dev)
    dt = _dtype_code(x)
    nb = lib().llima_argmax_workspace_bytes(B, V, dt)
    ws = Workspace.get(dev, "argmax", nb)
    check(lib().llima_argmax(x.data_ptr(), dt, B, V, x.stride(0), split_dim, MODES[mode],
                             ids.data_ptr(), vals.data_ptr(), ws.data_ptr(), ws.numel(),
                             _stream(dev)), "llima_argmax")
    return ids, vals


def argmax_bf16(values: torch.Tensor):
    """{maximum value, lowest index containing it} of one row (utils.hpp:80-152)."""
    ids, vals = argmax(values.reshape(1, -1))
    return float(vals[0]), int(ids[0])


def calc_next_token_id(logits: torch.Tensor) -> int:
    """Next token of a non-speculative decode step (language_model.cpp:3689-3714)."""
    ids, _ = argmax(logits.reshape(1, -1), mode="quarters")
    return int(ids[0])


def spec_path_argmax(logits, row: int) -> int:
    """The speculative path's next token in run_model_once
    (language_model.cpp:1518-1611): row `row` of one [N, V] buffer is scanned
    from its first value (argmax_bf16); split buffers [N, w_i] are scanned in
    order from bf16 lowest() with a strict '>'."""
    if isinstance(logits, (list, tuple)) and len(logits) > 1:
        ids, _ = argmax([t[row:row + 1] for t in logits], mode="lowest")
    else:
        x = logits[0] if isinstance(logits, (list, tuple)) else logits
        ids, _ = argmax(x[row:row + 1], mode="split_first")
    return int(ids[0])


def argmax_lm_head_rows(rows, expected_draft_tokens, split_dim: int = 0):
    """_argmax_lm_head_rows (language_model.cpp:3636-3687): per-row argmax of the
    first len(expected)+1 rows, truncated after the first row whose argmax differs
    from the expected draft token.  rows: [N, V] (splits of split_dim values)
    or the list of split buffers [N, w_i]."""
    n = len(expected_draft_tokens) + 1
    nrows = rows[0].shape[0] if isinstance(rows, (list, tuple)) else rows.shape[0]
    if n > nrows:
        raise RuntimeError(f"Requested {n} lm_head rows from n{nrows} output")
    if isinstance(rows, (list, tuple)):
        ids, _ = argmax([t[:n] for t in rows])
    else:
        ids, _ = argmax(rows[:n], split_dim=split_dim)
    ids = ids.tolist()
    out = []
    for r, t in enumerate(ids):
        out.append(t)
        if r < len(expected_draft_tokens) and t != int(expected_draft_tokens[r]):
            break
    return out


def sample(logits: torch.Tensor, uniforms: torch.Tensor, config: SamplerConfig,
           history: Optional[torch.Tensor] = None, history_len: Optional[torch.Tensor] = None,
           bitmask: Optional[torch.Tensor] = None, return_keep: bool = False):
    """One sampling step over [B, V] logits.

    history: int32 [B, H] token ids (ids outside [0, V) are padding), with an
    optional int32 [B] history_len; bitmask: int32/uint32 [B, ceil(V/32)]
    (bit i of word i>>5, LSB first, 0 = masked); uniforms: float32 [B] in [0,1).
    Returns (ids int32 [B], probs float32 [B]) and, if return_keep, the final
    kept set as a [B, ceil(V/32)] int32 bitmask.  A row with no admissible
    token yields id -1."""
    x = _rows2d(logits)
    B, V = x.shape
    dev = x.device
    u = uniforms.to(device=dev, dtype=torch.float32).contiguous()
    if u.numel() != B:
        raise ValueError("one uniform per row is required")
    H = 0
    if history is not None:
        history = history.to(device=dev, dtype=torch.int32).contiguous()
        if history.dim() != 2 or history.shape[0] != B:
            raise ValueError("history must be [B, H]")
        H = history.shape[1]
        if history_len is not None:
            history_len = history_len.to(device=dev, dtype=torch.int32).contiguous()
    nw = (V + 31) // 32
    if bitmask is not None:
        bitmask = bitmask.to(device=dev).contiguous()
        if bitmask.dtype not in (torch.int32, torch.uint32):
            raise ValueError("bitmask must be 32-bit words")
        if tuple(bitmask.shape) != (B, nw):
            raise ValueError(f"bitmask must be [{B}, {nw}]")
    _on_gpu(x, u, history, history_len, bitmask)
    cfg, keep_alive = config.to_c(B, dev, V)
    ids = torch.empty(B, dtype=torch.int32, device=dev)
    probs = torch.empty(B, dtype=torch.float32, device=dev)
    keep = torch.empty((B, nw), dtype=torch.int32, device=dev) if return_keep else None
    dt = _dtype_code(x)
    ws = Workspace.get(dev, "sample", lib().llima_sample_workspace_bytes(B, V, dt))
    check(lib().llima_sample(x.data_ptr(), dt, B, V, x.stride(0), _ptr(history),
                             _ptr(history_len), H, _ptr(bitmask), u.data_ptr(),
                             ctypes.byref(cfg), ids.data_ptr(), probs.data_ptr(), _ptr(keep),
                             ws.data_ptr(), ws.numel(), _stream(dev)), "llima_sample")
    del keep_alive
    return (ids, probs, keep) if return_keep else (ids, probs)


def verify_greedy(target_logits, draft_ids: torch.Tensor, split_dim: int = 0,
                  mode: str = "split_first"):
    """Greedy chain verification: target_logits [B, D+1, V] (or a list of split
    buffers [B, D+1, w_i]), draft_ids [B, D] -> (accepted_len int32 [B],
    emitted int32 [B, D+1], -1 padded).  Each target row's argmax follows
    split_dim and mode as argmax (the default with the head's split_dim is
    _argmax_lm_head_rows, language_model.cpp:3636-3687)."""
    if isinstance(target_logits, (list, tuple)):
        if target_logits[0].dim() != 3:
            raise ValueError("split target buffers must be [B, D+1, w_i]")
        B, D1 = target_logits[0].shape[:2]
        ptrs, widths, strides, _, V, dt, keep = _split_arrays(target_logits)
        dev = keep[0].device
    else:
        t = target_logits.contiguous()
        if t.dim() != 3:
            raise ValueError("target_logits must be [B, D+1, V]")
        B, D1, V = t.shape
        dt = _dtype_code(t)
        dev = t.device
        _on_gpu(t)
    D = D1 - 1
    d = draft_ids.to(device=dev, dtype=torch.int32).contiguous().reshape(B, D)
    _on_gpu(d)
    acc = torch.empty(B, dtype=torch.int32, device=dev)
    em = torch.empty((B, D1), dtype=torch.int32, device=dev)
    ws = Workspace.get(dev, "verify_greedy", lib().llima_verify_greedy_workspace_bytes(B, D, V, dt))
    if isinstance(target_logits, (list, tuple)):
        check(lib().llima_verify_greedy_splits(ptrs, widths, strides, len(keep), dt, B, D,
                                               MODES[mode], d.data_ptr(), acc.data_ptr(),
                                               em.data_ptr(), ws.data_ptr(), ws.numel(),
                                               _stream(dev)), "llima_verify_greedy_splits")
    else:
        check(lib().llima_verify_greedy(t.data_ptr(), dt, B, D, V, split_dim, MODES[mode],
                                        d.data_ptr(), acc.data_ptr(), em.data_ptr(), ws.data_ptr(),
                                        ws.numel(), _stream(dev)), "llima_verify_greedy")
    return acc, em


def resolve_draft_tokens(draft_token_ids, target_next_token_ids):
    """gemma4_mtp_helpers.cpp:81-111 on host lists (the device path computes the
    same rule inside verify_greedy)."""
    drafts = [int(x) for x in draft_token_ids]
    targets = [int(x) for x in target_next_token_ids]
    if not targets or len(targets) > len(drafts) + 1:
        raise RuntimeError("Invalid Gemma4 MTP verification result")
    out = []
    for depth, tgt in enumerate(targets):
        if depth == len(drafts) or drafts[depth] != tgt:
            out.append((tgt, False))
            return out
        out.append((drafts[depth], True))
    raise RuntimeError("Gemma4 MTP verification ended without a mismatch or bonus token")


def verify_tree(tree_logits: torch.Tensor, retrieve_indices: torch.Tensor,
                candidates: torch.Tensor):
    """EAGLE3 tree verification: argmax of each tree row (from -inf,
    language_model_eagle3.cpp:486-522), gather along retrieve_indices (-1 -> last
    row), evaluate_posterior -> (best_candidate, accept_length, bonus_token)."""
    t = _rows2d(tree_logits).contiguous()
    K, V = t.shape
    dev = t.device
    ri = retrieve_indices.to(device=dev, dtype=torch.int32).contiguous()
    ca = candidates.to(device=dev, dtype=torch.int32).contiguous()
    if ri.shape != ca.shape or ri.dim() != 2:
        raise ValueError("retrieve_indices and candidates must both be [n_paths, L]")
    P, L = ri.shape
    out = torch.empty(3, dtype=torch.int32, device=dev)
    dt = _dtype_code(t)
    ws = Workspace.get(dev, "verify_tree", lib().llima_verify_tree_workspace_bytes(K, V, dt))
    check(lib().llima_verify_tree(t.data_ptr(), dt, K, V, ri.data_ptr(), ca.data_ptr(), P, L,
                                  out.data_ptr(), ws.data_ptr(), ws.numel(), _stream(dev)),
          "llima_verify_tree")
    o = out.tolist()
    return o[0], o[1], o[2]


def verify_rejection(target_logits: torch.Tensor, draft_logits: torch.Tensor,
                     draft_ids: torch.Tensor, u_accept: torch.Tensor, u_resample: torch.Tensor):
    """Stochastic verification: target [B, D+1, V] and draft [B, D, V] fp32
    logits, draft ids [B, D], uniforms u_accept [B, D] and u_resample [B] ->
    (accepted_len int32 [B], emitted int32 [B, D+1], -1 padded)."""
    t = target_logits.contiguous()
    dl = draft_logits.contiguous()
    if t.dtype != torch.float32 or dl.dtype != torch.float32:
        raise ValueError("verify_rejection takes fp32 logits")
    B, D1, V = t.shape
    D = D1 - 1
    if tuple(dl.shape) != (B, D, V):
        raise ValueError("draft_logits must be [B, D, V]")
    dev = t.device
    ids = draft_ids.to(device=dev, dtype=torch.int32).contiguous()
    ua = u_accept.to(device=dev, dtype=torch.float32).contiguous()
    ur = u_resample.to(device=dev, dtype=torch.float32).contiguous()
    _on_gpu(t, dl, ids, ua, ur)
    acc = torch.empty(B, dtype=torch.int32, device=dev)
    em = torch.empty((B, D1), dtype=torch.int32, device=dev)
    ws = Workspace.get(dev, "verify_rejection", lib().llima_verify_rejection_workspace_bytes(B, D, V))
    check(lib().llima_verify_rejection(t.data_ptr(), dl.data_ptr(), B, D, V, ids.data_ptr(),
                                       ua.data_ptr(), ur.data_ptr(), acc.data_ptr(),
                                       em.data_ptr(), ws.data_ptr(), ws.numel(), _stream(dev)),
          "llima_verify_rejection")
    return acc, em


def score_logits(logits: torch.Tensor, target):
    """score_logits (language_model.cpp:29-62): the log-softmax of the target
    token and whether the target is the (first) argmax.

    logits [V] with an int target -> (logprob float, is_greedy bool), raising
    RuntimeError for a target outside the vocabulary as the reference does;
    logits [B, V] with int targets [B] -> (float64 [B], bool [B]) tensors."""
    single = logits.dim() == 1
    x = _rows2d(logits)
    B, V = x.shape
    dev = x.device
    if single:
        t = int(target)
        if t < 0 or t >= V:
            raise RuntimeError(f"Target token id {t} is outside logits vocabulary size {V}")
        tg = torch.full((1,), t, dtype=torch.int32, device=dev)
    else:
        tg = torch.as_tensor(target).to(device=dev, dtype=torch.int32).contiguous().reshape(-1)
        if tg.numel() != B:
            raise ValueError("one target per row is required")
    _on_gpu(x, tg)
    lp = torch.empty(B, dtype=torch.float64, device=dev)
    gr = torch.empty(B, dtype=torch.int32, device=dev)
    dt = _dtype_code(x)
    ws = Workspace.get(dev, "score", lib().llima_score_logits_workspace_bytes(B, V, dt))
    check(lib().llima_score_logits(x.data_ptr(), dt, B, V, x.stride(0), tg.data_ptr(),
                                   lp.data_ptr(), gr.data_ptr(), ws.data_ptr(), ws.numel(),
                                   _stream(dev)), "llima_score_logits")
    if single:
        return float(lp[0]), bool(gr[0] == 1)
    if bool((gr < 0).any()):
        raise RuntimeError(f"a target token id is outside logits vocabulary size {V}")
    return lp, gr == 1


def _mtp_args(centroid_logits: torch.Tensor, token_ordering, top_k: int):
    c = centroid_logits
    if c.dim() == 1:
        c = c.unsqueeze(0)
    if c.dtype != torch.bfloat16 or c.dim() != 2:
        raise ValueError("centroid_logits must be bfloat16 [C] or [B, C]")
    if c.stride(-1) != 1:
        c = c.contiguous()
    o = torch.as_tensor(token_ordering)
    if o.dtype == torch.int64:
        o = (o & 0xFFFFFFFF).to(torch.int32)         # uint32 bit patterns
    o = o.to(device=c.device, dtype=torch.int32).contiguous().reshape(-1)
    C, V = c.shape[1], o.numel()
    # the reference's own argument checks (gemma4_mtp_helpers.cpp:118-128)
    if C == 0 or V == 0 or V % C != 0:
        raise RuntimeError("Gemma4 masked lm_head vocabulary must divide evenly across centroids")
    if top_k <= 0 or top_k > C:
        raise RuntimeError("Invalid Gemma4 masked lm_head centroid top-k")
    if C > 8192:
        raise ValueError("at most 8192 centroids per row")
    _on_gpu(c, o)
    return c, o, C, V


def _mtp_status(st: torch.Tensor):
    s = st.tolist()
    if any(v == _lib.LLIMA_E_RANGE for v in s):
        raise RuntimeError("Gemma4 token_ordering contains an out-of-range token ID")
    if any(v == _lib.LLIMA_E_INVAL for v in s):
        raise RuntimeError("Gemma4 masked lm_head selected no token")


def select_candidate_tokens(centroid_logits: torch.Tensor, token_ordering, top_k_centroids: int):
    """select_candidate_tokens (gemma4_mtp_helpers.cpp:113-167): the tokens of
    the top_k centroids by (value desc, index asc), in that order.  One row [C]
    -> list of ints; rows [B, C] -> int32 [B, top_k * V / C]."""
    c, o, C, V = _mtp_args(centroid_logits, token_ordering, int(top_k_centroids))
    B, k = c.shape[0], int(top_k_centroids)
    cand = torch.empty((B, k * (V // C)), dtype=torch.int32, device=c.device)
    st = torch.empty(B, dtype=torch.int32, device=c.device)
    ws = Workspace.get(c.device, "mtp", lib().llima_mtp_masked_argmax_workspace_bytes(B))
    check(lib().llima_mtp_masked_argmax(c.data_ptr(), c.stride(0), C, o.data_ptr(), k, None,
                                        _lib.LLIMA_BF16, B, V, V, None, st.data_ptr(),
                                        cand.data_ptr(), ws.data_ptr(), ws.numel(),
                                        _stream(c.device)),
          "llima_mtp_masked_argmax")
    _mtp_status(st)
    return cand[0].tolist() if centroid_logits.dim() == 1 else cand


def argmax_gemma4_mtp_masked_rows(centroid_logits: torch.Tensor, token_ordering, top_k: int,
                                  logits: torch.Tensor):
    """_argmax_gemma4_mtp_masked_row (language_model_gemma4_mtp.cpp:31-97) over
    B rows: the candidate token (select_candidate_tokens) with the greatest
    logit, the lowest token id on equal values.  centroid_logits bf16 [B, C],
    token_ordering [V], logits [B, V] -> int32 [B]."""
    c, o, C, V = _mtp_args(centroid_logits, token_ordering, int(top_k))
    x = _rows2d(logits)
    if x.shape[0] != c.shape[0] or x.shape[1] != V:
        raise ValueError("logits must be [B, V] with V = len(token_ordering)")
    _on_gpu(x)
    B = x.shape[0]
    ids = torch.empty(B, dtype=torch.int32, device=x.device)
    st = torch.empty(B, dtype=torch.int32, device=x.device)
    ws = Workspace.get(x.device, "mtp", lib().llima_mtp_masked_argmax_workspace_bytes(B))
    check(lib().llima_mtp_masked_argmax(c.data_ptr(), c.stride(0), C, o.data_ptr(), int(top_k),
                                        x.data_ptr(), _dtype_code(x), B, V, x.stride(0),
                                        ids.data_ptr(), st.data_ptr(), None, ws.data_ptr(),
                                        ws.numel(), _stream(x.device)),
          "llima_mtp_masked_argmax")
    _mtp_status(st)
    return ids


def argmax_gemma4_mtp_masked_row(centroid_logits: torch.Tensor, token_ordering, top_k: int,
                                 logits: torch.Tensor) -> int:
    """One row of argmax_gemma4_mtp_masked_rows: centroid_logits [C], logits [V]."""
    return int(argmax_gemma4_mtp_masked_rows(centroid_logits.reshape(1, -1), token_ordering,
                                             top_k, logits.reshape(1, -1))[0])


class PackedLmHead:
    """An LM head weight prepacked once, at model load, by lm_head_pack: the
    bf16 [V, H] weight rearranged into the MFMA's operand order (1 KB per 32
    vocab rows x 16 ids, zero rows up to a multiple of 32, 8 KB groups per 32
    rows and 128 ids), so that each wave streams contiguous memory straight
    into the matrix cores.  `data` is the uint8 device tensor; V and H are the
    weight's shape.  It is read once per 64 hidden rows."""

    def __init__(self, data: torch.Tensor, V: int, H: int):
        self.data, self.V, self.H = data, V, H


def lm_head_pack(weight: torch.Tensor) -> PackedLmHead:
    """Prepack a bf16 [V, H] LM head weight (H a multiple of 256) for
    lm_head_argmax (llima_lm_head_pack)."""
    if weight.dtype != torch.bfloat16 or weight.dim() != 2:
        raise ValueError("lm_head_pack takes a bf16 [V, H] weight")
    w = weight.contiguous()
    V, H = w.shape
    _on_gpu(w)
    n = lib().llima_lm_head_packed_bytes(V, H)
    if n == 0:
        raise ValueError("lm_head_pack needs H a multiple of 256 (at most 65536)")
    data = torch.empty(n, dtype=torch.uint8, device=w.device)
    check(lib().llima_lm_head_pack(w.data_ptr(), V, H, data.data_ptr(), n, _stream(w.device)),
          "llima_lm_head_pack")
    return PackedLmHead(data, V, H)


def lm_head_argmax(hidden: torch.Tensor, weight, softcap: float = 0.0,
                   return_logits: bool = False, logit_dtype: str = "bf16",
                   logits_out: str = "f32"):
    """LM head + softcap + argmax, as the reference's graph computes them before
    the host reads one int32 (language_part_base.py:171-180,
    language_model.cpp:1607-1609): hidden bf16 [B, H] (or [H]), weight bf16
    [V, H] -> (ids int32 [B], values float32 [B]) and, if return_logits, the
    logits [B, V].  logit_dtype "bf16" rounds each logit to bf16 before the
    argmax, as the reference's bf16 graphs produce them (equal bf16 logits
    tie, the lower index wins); "f32" keeps the fp32 sums.  logits_out "bf16"
    (with logit_dtype "bf16") returns the logits as a bfloat16 tensor, half
    the bytes of the float32 one and the same values, ready for sample().
    weight may be a PackedLmHead (lm_head_pack): the same logits, read in the
    packed order (llima_lm_head_argmax_packed)."""
    x = hidden.reshape(1, -1) if hidden.dim() == 1 else hidden
    packed = isinstance(weight, PackedLmHead)
    if x.dtype != torch.bfloat16 or (not packed and weight.dtype != torch.bfloat16):
        raise ValueError("lm_head_argmax takes bf16 hidden states and weights")
    if logit_dtype not in ("bf16", "f32"):
        raise ValueError("logit_dtype must be 'bf16' or 'f32'")
    if logits_out not in ("bf16", "f32"):
        raise ValueError("logits_out must be 'bf16' or 'f32'")
    if logits_out == "bf16" and logit_dtype != "bf16":
        raise ValueError("bf16 logits output needs logit_dtype 'bf16'")
    x = x.contiguous()
    w = weight.data if packed else weight.contiguous()
    B, H = x.shape
    if packed:
        if weight.H != H:
            raise ValueError("hidden width differs from the packed weight's H")
        V = weight.V
    else:
        if w.dim() != 2 or w.shape[1] != H:
            raise ValueError("weight must be [V, H]")
        V = w.shape[0]
    dev = w.device
    _on_gpu(x, w)
    ids = torch.empty(B, dtype=torch.int32, device=dev)
    vals = torch.empty(B, dtype=torch.float32, device=dev)
    ldt = torch.bfloat16 if logits_out == "bf16" else torch.float32
    logits = torch.empty((B, V), dtype=ldt, device=dev) if return_logits else None
    nws = (lib().llima_lm_head_argmax_packed_workspace_bytes(B, H, V) if packed
           else lib().llima_lm_head_argmax_workspace_bytes(B, V))
    ws = Workspace.get(dev, "lm_head", nws)
    ld = _lib.LLIMA_BF16 if logit_dtype == "bf16" else _lib.LLIMA_F32
    if logits_out == "bf16":
        ld |= _lib.LLIMA_LOGITS_OUT_BF16
    fn = lib().llima_lm_head_argmax_packed if packed else lib().llima_lm_head_argmax
    check(fn(x.data_ptr(), w.data_ptr(), B, H, V, float(softcap), ld, ids.data_ptr(),
             vals.data_ptr(), _ptr(logits), ws.data_ptr(), ws.numel(), _stream(dev)),
          "llima_lm_head_argmax_packed" if packed else "llima_lm_head_argmax")
    return (ids, vals, logits) if return_logits else (ids, vals)


def lm_head_score(hidden: torch.Tensor, weight, target, softcap: float = 0.0,
                  logit_dtype: str = "bf16"):
    """The LM head followed by score_logits (language_model.cpp:29-62) in one
    call, the logits never written (llima_lm_head_score): hidden bf16 [B, H]
    with int targets [B] -> (float64 [B] log-probabilities, bool [B] greedy
    flags), or hidden [H] with an int target -> (float, bool).  The logits are
    lm_head_argmax's (the same softcap and logit_dtype); weight may be a
    PackedLmHead.  A target outside the vocabulary raises RuntimeError, as
    score_logits does."""
    single = hidden.dim() == 1
    x = hidden.reshape(1, -1) if single else hidden
    packed = isinstance(weight, PackedLmHead)
    if x.dtype != torch.bfloat16 or (not packed and weight.dtype != torch.bfloat16):
        raise ValueError("lm_head_score takes bf16 hidden states and weights")
    if logit_dtype not in ("bf16", "f32"):
        raise ValueError("logit_dtype must be 'bf16' or 'f32'")
    x = x.contiguous()
    w = weight.data if packed else weight.contiguous()
    B, H = x.shape
    if packed:
        if weight.H != H:
            raise ValueError("hidden width differs from the packed weight's H")
        V = weight.V
    else:
        if w.dim() != 2 or w.shape[1] != H:
            raise ValueError("weight must be [V, H]")
        V = w.shape[0]
    dev = w.device
    if single:
        t = int(target)
        if t < 0 or t >= V:
            raise RuntimeError(f"Target token id {t} is outside logits vocabulary size {V}")
        tg = torch.full((1,), t, dtype=torch.int32, device=dev)
    else:
        tg = torch.as_tensor(target).to(device=dev, dtype=torch.int32).contiguous().reshape(-1)
        if tg.numel() != B:
            raise ValueError("one target per row is required")
    _on_gpu(x, w, tg)
    lp = torch.empty(B, dtype=torch.float64, device=dev)
    gr = torch.empty(B, dtype=torch.int32, device=dev)
    nws = (lib().llima_lm_head_score_packed_workspace_bytes(B, H, V) if packed
           else lib().llima_lm_head_score_workspace_bytes(B, V))
    ws = Workspace.get(dev, "lm_head_score", nws)
    ld = _lib.LLIMA_BF16 if logit_dtype == "bf16" else _lib.LLIMA_F32
    fn = lib().llima_lm_head_score_packed if packed else lib().llima_lm_head_score
    check(fn(x.data_ptr(), w.data_ptr(), B, H, V, float(softcap), ld, tg.data_ptr(),
             lp.data_ptr(), gr.data_ptr(), ws.data_ptr(), ws.numel(), _stream(dev)),
          "llima_lm_head_score_packed" if packed else "llima_lm_head_score")
    if single:
        return float(lp[0]), bool(gr[0] == 1)
    if bool((gr < 0).any()):
        raise RuntimeError(f"a target token id is outside logits vocabulary size {V}")
    return lp, gr == 1


def lm_head_verify_greedy(hidden: torch.Tensor, weight, draft_ids: torch.Tensor,
                          softcap: float = 0.0, logit_dtype: str = "bf16"):
    """The verification step's LM head and greedy chain rule in one call, no
    logits written (llima_lm_head_verify_greedy): hidden bf16 [B, D+1, H],
    draft_ids int [B, D] -> (accepted_len int32 [B], emitted int32 [B, D+1]),
    as verify_greedy over the logits lm_head_argmax would write (the same
    softcap and logit_dtype).  weight may be a PackedLmHead."""
    if hidden.dim() != 3:
        raise ValueError("hidden must be [B, D+1, H]")
    B, D1, H = hidden.shape
    D = D1 - 1
    packed = isinstance(weight, PackedLmHead)
    if hidden.dtype != torch.bfloat16 or (not packed and weight.dtype != torch.bfloat16):
        raise ValueError("lm_head_verify_greedy takes bf16 hidden states and weights")
    if logit_dtype not in ("bf16", "f32"):
        raise ValueError("logit_dtype must be 'bf16' or 'f32'")
    x = hidden.contiguous()
    w = weight.data if packed else weight.contiguous()
    if packed:
        if weight.H != H:
            raise ValueError("hidden width differs from the packed weight's H")
        V = weight.V
    else:
        if w.dim() != 2 or w.shape[1] != H:
            raise ValueError("weight must be [V, H]")
        V = w.shape[0]
    dev = w.device
    dr = torch.as_tensor(draft_ids).to(device=dev, dtype=torch.int32).contiguous()
    if tuple(dr.shape) != (B, D):
        raise ValueError("draft_ids must be [B, D]")
    _on_gpu(x, w, dr)
    acc = torch.empty(B, dtype=torch.int32, device=dev)
    em = torch.empty((B, D1), dtype=torch.int32, device=dev)
    nws = (lib().llima_lm_head_verify_greedy_packed_workspace_bytes(B, D, H, V) if packed
           else lib().llima_lm_head_verify_greedy_workspace_bytes(B, D, V))
    ws = Workspace.get(dev, "lm_head_verify", nws)
    ld = _lib.LLIMA_BF16 if logit_dtype == "bf16" else _lib.LLIMA_F32
    if packed:
        st = lib().llima_lm_head_verify_greedy_packed(
            x.data_ptr(), w.data_ptr(), B, D, H, V, float(softcap), ld, dr.data_ptr(),
            acc.data_ptr(), em.data_ptr(), ws.data_ptr(), ws.numel(), _stream(dev))
    else:
        st = lib().llima_lm_head_verify_greedy(
            x.data_ptr(), w.data_ptr(), B, D, H, V, float(softcap), ld, dr.data_ptr(),
            acc.data_ptr(), em.data_ptr(), ws.data_ptr(), ws.numel(), _stream(dev))
    check(st, "llima_lm_head_verify_greedy_packed" if packed else "llima_lm_head_verify_greedy")
    return acc, em


def lm_head_verify_tree(hidden: torch.Tensor, weight, retrieve_indices: torch.Tensor,
                        candidates: torch.Tensor, softcap: float = 0.0,
                        logit_dtype: str = "bf16"):
    """The EAGLE3 tree step's LM head and verification in one call, no logits
    written (llima_lm_head_verify_tree): hidden bf16 [K, H] (the tree rows),
    retrieve_indices and candidates [n_paths, L] -> (best_candidate,
    accept_length, bonus_token), as verify_tree over the logits lm_head_argmax
    would write.  weight may be a PackedLmHead."""
    x = hidden.contiguous()
    packed = isinstance(weight, PackedLmHead)
    if x.dim() != 2 or x.dtype != torch.bfloat16 or (not packed and weight.dtype != torch.bfloat16):
        raise ValueError("lm_head_verify_tree takes bf16 hidden rows [K, H] and a bf16 weight")
    if logit_dtype not in ("bf16", "f32"):
        raise ValueError("logit_dtype must be 'bf16' or 'f32'")
    K, H = x.shape
    w = weight.data if packed else weight.contiguous()
    if packed:
        if weight.H != H:
            raise ValueError("hidden width differs from the packed weight's H")
        V = weight.V
    else:
        if w.dim() != 2 or w.shape[1] != H:
            raise ValueError("weight must be [V, H]")
        V = w.shape[0]
    dev = w.device
    ri = retrieve_indices.to(device=dev, dtype=torch.int32).contiguous()
    ca = candidates.to(device=dev, dtype=torch.int32).contiguous()
    if ri.shape != ca.shape or ri.dim() != 2:
        raise ValueError("retrieve_indices and candidates must both be [n_paths, L]")
    P, L = ri.shape
    _on_gpu(x, w, ri, ca)
    out = torch.empty(3, dtype=torch.int32, device=dev)
    nws = (lib().llima_lm_head_verify_tree_packed_workspace_bytes(K, H, V) if packed
           else lib().llima_lm_head_verify_tree_workspace_bytes(K, V))
    ws = Workspace.get(dev, "lm_head_tree", nws)
    ld = _lib.LLIMA_BF16 if logit_dtype == "bf16" else _lib.LLIMA_F32
    fn = lib().llima_lm_head_verify_tree_packed if packed else lib().llima_lm_head_verify_tree
    check(fn(x.data_ptr(), w.data_ptr(), K, H, V, float(softcap), ld, ri.data_ptr(),
             ca.data_ptr(), P, L, out.data_ptr(), ws.data_ptr(), ws.numel(), _stream(dev)),
          "llima_lm_head_verify_tree_packed" if packed else "llima_lm_head_verify_tree")
    o = out.tolist()
    return o[0], o[1], o[2]


def topk(x: torch.Tensor, k: int):
    """topk<T> (utils.hpp:216-281) over the rows of x ([cols] or [rows, cols],
    fp32 or bf16) -> (indices int32 [rows, k], values float32 [rows, k]) in the
    reference heap's output order, ties included.  k in [1, 32]."""
    single = x.dim() == 1
    a = _rows2d(x)
    _on_gpu(a)
    rows, cols = a.shape
    if not 1 <= k <= 32:
        raise RuntimeError("topk: k out of supported range [1, 32]")
    if cols < k:
        raise ValueError("topk needs at least k values per row")
    idx = torch.empty((rows, k), dtype=torch.int32, device=a.device)
    val = torch.empty((rows, k), dtype=torch.float32, device=a.device)
    check(lib().llima_topk(a.data_ptr(), _dtype_code(a), rows, cols, a.stride(0), k,
                           idx.data_ptr(), val.data_ptr(), _stream(a.device)), "llima_topk")
    return (idx[0], val[0]) if single else (idx, val)


class Eagle3DraftTree:
    """The selection side of the EAGLE3 draft tree (topk_generate,
    language_model_eagle3.cpp:808-1164) on the GPU.  The draft model runs
    between the calls:

        tree = Eagle3DraftTree(d2t, topk=5, depth=4)
        ids = tree.begin(root_logits)              # [Vd] -> first draft inputs [K]
        for level in range(1, depth):
            ids, parent_rows, mask = tree.grow(draft_logits)   # [K, Vd]
        out = tree.finish(total_tokens=15, sample_token=tok)

    finish returns the draft tokens [N], tree mask [N, N], position ids [N]
    and retrieve indices [leaves, columns] (N = total_tokens + 1)."""

    def __init__(self, d2t: torch.Tensor, topk: int = 5, depth: int = 4):
        self.d2t = d2t.to(dtype=torch.int32).contiguous()
        _on_gpu(self.d2t)
        self.K, self.depth = int(topk), int(depth)
        nb = lib().llima_eagle3_tree_bytes(self.K, self.depth)
        if nb == 0:
            raise ValueError("topk must be 1..32 and depth 1..16 (at most 16384 nodes)")
        self.dev = self.d2t.device
        self.state = torch.empty(nb, dtype=torch.uint8, device=self.dev)
        self.level = 0

    def _logits(self, x, rows):
        a = _rows2d(x)
        _on_gpu(a)
        if a.shape[0] != rows:
            raise ValueError(f"expected {rows} logits rows, got {a.shape[0]}")
        if a.shape[1] > self.d2t.numel():
            raise ValueError("d2t must hold an offset for every draft id")
        return a

    def begin(self, root_logits: torch.Tensor) -> torch.Tensor:
        a = self._logits(root_logits.reshape(1, -1), 1)
        ids = torch.empty(self.K, dtype=torch.int32, device=self.dev)
        check(lib().llima_eagle3_tree_begin(a.data_ptr(), _dtype_code(a), a.shape[1],
                                            self.d2t.data_ptr(), self.K, self.depth,
                                            self.state.data_ptr(), self.state.numel(),
                                            ids.data_ptr(), _stream(self.dev)),
              "llima_eagle3_tree_begin")
        self.level = 1
        return ids

    def grow(self, logits: torch.Tensor):
        if not 1 <= self.level < self.depth:
            raise RuntimeError("grow: begin first, and at most depth - 1 levels")
        a = self._logits(logits, self.K)
        ids = torch.empty(self.K, dtype=torch.int32, device=self.dev)
        prow = torch.empty(self.K, dtype=torch.int32, device=self.dev)
        mask = torch.empty((self.K, self.K * (self.level + 1)), dtype=torch.float32,
                           device=self.dev)
        check(lib().llima_eagle3_tree_grow(a.data_ptr(), _dtype_code(a), a.shape[1], a.stride(0),
                                           self.d2t.data_ptr(), self.K, self.depth, self.level,
                                           self.state.data_ptr(), self.state.numel(),
                                           ids.data_ptr(), prow.data_ptr(), mask.data_ptr(),
                                           _stream(self.dev)), "llima_eagle3_tree_grow")
        self.level += 1
        return ids, prow, mask

    def node_scores(self) -> torch.Tensor:
        """The cumulative log-probability of every node grown so far, in the
        reference's flat order (scores_list flattened, language_model_eagle3.cpp:
        1040-1048): the K root scores, then K*K per level.  A float32 view into
        the tree state, whose regions (each on a 256-byte boundary) are: the
        current scores [K], the parent groups [1 + (depth-1)K], the node
        scores, ..."""
        def take(o, nbytes):
            return o + ((nbytes + 255) & ~255)
        K, depth = self.K, self.depth
        off = take(take(0, 4 * K), 4 * (1 + (depth - 1) * K))
        n = K + (self.level - 1) * K * K if self.level else 0
        return self.state[off:off + 4 * n].view(torch.float32)

    def finish(self, total_tokens: int, sample_token: int):
        if self.level != self.depth:
            raise RuntimeError("finish: grow depth - 1 levels first")
        N = int(total_tokens) + 1
        tok = torch.empty(N, dtype=torch.int32, device=self.dev)
        tmask = torch.empty((N, N), dtype=torch.float32, device=self.dev)
        pos = torch.empty(N, dtype=torch.int32, device=self.dev)
        ret = torch.empty((N, N), dtype=torch.int32, device=self.dev)
        dims = torch.empty(2, dtype=torch.int32, device=self.dev)
        check(lib().llima_eagle3_tree_finish(self.state.data_ptr(), self.state.numel(), self.K,
                                             self.depth, int(total_tokens), int(sample_token),
                                             tok.data_ptr(), tmask.data_ptr(), pos.data_ptr(),
                                             ret.data_ptr(), dims.data_ptr(), _stream(self.dev)),
              "llima_eagle3_tree_finish")
        leaves, cols = dims.tolist()
        return dict(tokens=tok, tree_mask=tmask, position_ids=pos,
                    retrieve=ret[:leaves, :cols])


def stop_mask(stop_token_ids, V: int, device) -> torch.Tensor:
    """The stop set as the [ceil(V/32)] bitmask llima_stop_check reads (ids
    outside [0, V) are dropped: they never stop)."""
    words = np.zeros((V + 31) // 32, np.uint32)
    for t in stop_token_ids:
        t = int(t)
        if 0 <= t < V:
            words[t >> 5] |= np.uint32(1 << (t & 31))
    return torch.from_numpy(words.view(np.int32)).to(device)


def stop_check(tokens: torch.Tensor, stop: torch.Tensor, V: int,
               count: Optional[torch.Tensor] = None, room: Optional[torch.Tensor] = None):
    """The decode loops' stop rule (language_model.cpp:643-671,
    language_model_dflash.cpp:570-579, language_model_gemma4_mtp.cpp:940-956)
    on emitted tokens [B, M] (count [B] valid each, room [B] cache space left)
    with the stop set as the bitmask of stop_mask -> (keep int32 [B],
    status int32 [B]: STOP_NONE / STOP_TOKEN / STOP_CACHE_FULL)."""
    t = tokens.to(dtype=torch.int32)
    if t.dim() == 1:
        t = t.unsqueeze(1)
    t = t.contiguous()
    B, M = t.shape
    dev = t.device
    c = None if count is None else count.to(device=dev, dtype=torch.int32).contiguous()
    r = None if room is None else room.to(device=dev, dtype=torch.int32).contiguous()
    m = stop.to(device=dev).contiguous()
    if m.numel() != (V + 31) // 32:
        raise ValueError("the stop mask must hold ceil(V / 32) words")
    _on_gpu(t, c, r, m)
    keep = torch.empty(B, dtype=torch.int32, device=dev)
    status = torch.empty(B, dtype=torch.int32, device=dev)
    check(lib().llima_stop_check(t.data_ptr(), _ptr(c), B, M, m.data_ptr(), V, _ptr(r),
                                 keep.data_ptr(), status.data_ptr(), _stream(dev)),
          "llima_stop_check")
    return keep, status
