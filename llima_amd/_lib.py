"""ctypes binding of libllima_sampler.so (declarations in include/llima_sampler.h).

The library is the product: there is no fallback.  If it is missing, loading
raises and every API call fails loudly.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libllima_sampler.so")

LLIMA_OK, LLIMA_E_INVAL, LLIMA_E_RANGE, LLIMA_E_HIP, LLIMA_E_WORKSPACE = 0, -1, -2, -3, -4
LLIMA_E_SCRATCH = -5
LLIMA_E_CAPTURE = -6
LLIMA_F32, LLIMA_BF16 = 0, 1
LLIMA_LOGITS_OUT_BF16 = 0x100   # with LLIMA_BF16 in the LM head's logit_dtype: bf16 logits out
ARGMAX_SPLIT_FIRST, ARGMAX_NEG_INF, ARGMAX_QUARTERS, ARGMAX_LOWEST = 0, 1, 2, 3
MAX_SPLITS = 16
STOP_NONE, STOP_TOKEN, STOP_CACHE_FULL = 0, 1, 2

# name -> (restype, argtypes) for every entry point of include/llima_sampler.h
_vp, _sz, _i32, _i64 = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int32, ctypes.c_int64
SIGNATURES = {
    "llima_argmax_workspace_bytes": (_sz, [_i32, _i32, _i32]),
    "llima_argmax": (ctypes.c_int, [_vp, _i32, _i32, _i32, _i64, _i32, _i32, _vp, _vp, _vp, _sz,
                                    _vp]),
    "llima_argmax_splits": (ctypes.c_int, [_vp, _vp, _vp, _i32, _i32, _i32, _i32, _vp, _vp, _vp,
                                           _sz, _vp]),
    "llima_sample_workspace_bytes": (_sz, [_i32, _i32, _i32]),
    "llima_sample": (ctypes.c_int, [_vp, _i32, _i32, _i32, _i64, _vp, _vp, _i32, _vp, _vp, _vp,
                                    _vp, _vp, _vp, _vp, _sz, _vp]),
    "llima_sample_noalloc_max_bytes": (_sz, []),
    "llima_sample_noalloc": (ctypes.c_int, [_vp, _i32, _i32, _i32, _i64, _vp, _vp, _i32, _vp, _vp,
                                            _vp, _vp, _vp, _vp, _vp]),
    "llima_verify_greedy_workspace_bytes": (_sz, [_i32, _i32, _i32, _i32]),
    "llima_verify_greedy": (ctypes.c_int, [_vp, _i32, _i32, _i32, _i32, _i32, _i32, _vp, _vp, _vp,
                                           _vp, _sz, _vp]),
    "llima_verify_greedy_splits": (ctypes.c_int, [_vp, _vp, _vp, _i32, _i32, _i32, _i32, _i32, _vp,
                                                  _vp, _vp, _vp, _sz, _vp]),
    "llima_verify_tree_workspace_bytes": (_sz, [_i32, _i32, _i32]),
    "llima_verify_tree": (ctypes.c_int, [_vp, _i32, _i32, _i32, _vp, _vp, _i32, _i32, _vp, _vp,
                                         _sz, _vp]),
    "llima_verify_rejection_workspace_bytes": (_sz, [_i32, _i32, _i32]),
    "llima_verify_rejection": (ctypes.c_int, [_vp, _vp, _i32, _i32, _i32, _vp, _vp, _vp, _vp, _vp,
                                              _vp, _sz, _vp]),
    "llima_score_logits_workspace_bytes": (_sz, [_i32, _i32, _i32]),
    "llima_score_logits": (ctypes.c_int, [_vp, _i32, _i32, _i32, _i64, _vp, _vp, _vp, _vp, _sz,
                                          _vp]),
    "llima_mtp_masked_argmax_workspace_bytes": (_sz, [_i32]),
    "llima_mtp_masked_argmax": (ctypes.c_int, [_vp, _i64, _i32, _vp, _i32, _vp, _i32, _i32, _i32,
                                               _i64, _vp, _vp, _vp, _vp, _sz, _vp]),
    "llima_lm_head_argmax_workspace_bytes": (_sz, [_i32, _i32]),
    "llima_lm_head_argmax": (ctypes.c_int, [_vp, _vp, _i32, _i32, _i32, ctypes.c_float, _i32, _vp,
                                            _vp, _vp, _vp, _sz, _vp]),
    "llima_lm_head_packed_bytes": (_sz, [_i32, _i32]),
    "llima_lm_head_argmax_packed_workspace_bytes": (_sz, [_i32, _i32, _i32]),
    "llima_lm_head_pack": (ctypes.c_int, [_vp, _i32, _i32, _vp, _sz, _vp]),
    "llima_lm_head_argmax_packed": (ctypes.c_int, [_vp, _vp, _i32, _i32, _i32, ctypes.c_float, _i32,
                                                   _vp, _vp, _vp, _vp, _sz, _vp]),
    "llima_lm_head_score_workspace_bytes": (_sz, [_i32, _i32]),
    "llima_lm_head_score": (ctypes.c_int, [_vp, _vp, _i32, _i32, _i32, ctypes.c_float, _i32, _vp,
                                           _vp, _vp, _vp, _sz, _vp]),
    "llima_lm_head_score_packed_workspace_bytes": (_sz, [_i32, _i32, _i32]),
    "llima_lm_head_score_packed": (ctypes.c_int, [_vp, _vp, _i32, _i32, _i32, ctypes.c_float,
                                                  _i32, _vp, _vp, _vp, _vp, _sz, _vp]),
    "llima_lm_head_verify_greedy_workspace_bytes": (_sz, [_i32, _i32, _i32]),
    "llima_lm_head_verify_greedy": (ctypes.c_int, [_vp, _vp, _i32, _i32, _i32, _i32,
                                                   ctypes.c_float, _i32, _vp, _vp, _vp, _vp, _sz,
                                                   _vp]),
    "llima_lm_head_verify_greedy_packed_workspace_bytes": (_sz, [_i32, _i32, _i32, _i32]),
    "llima_lm_head_verify_greedy_packed": (ctypes.c_int, [_vp, _vp, _i32, _i32, _i32, _i32,
                                                          ctypes.c_float, _i32, _vp, _vp, _vp,
                                                          _vp, _sz, _vp]),
    "llima_lm_head_verify_tree_workspace_bytes": (_sz, [_i32, _i32]),
    "llima_lm_head_verify_tree": (ctypes.c_int, [_vp, _vp, _i32, _i32, _i32, ctypes.c_float,
                                                 _i32, _vp, _vp, _i32, _i32, _vp, _vp, _sz, _vp]),
    "llima_lm_head_verify_tree_packed_workspace_bytes": (_sz, [_i32, _i32, _i32]),
    "llima_lm_head_verify_tree_packed": (ctypes.c_int, [_vp, _vp, _i32, _i32, _i32,
                                                        ctypes.c_float, _i32, _vp, _vp, _i32,
                                                        _i32, _vp, _vp, _sz, _vp]),
    "llima_topk": (ctypes.c_int, [_vp, _i32, _i32, _i32, _i64, _i32, _vp, _vp, _vp]),
    "llima_eagle3_tree_bytes": (_sz, [_i32, _i32]),
    "llima_eagle3_tree_begin": (ctypes.c_int, [_vp, _i32, _i32, _vp, _i32, _i32, _vp, _sz, _vp,
                                               _vp]),
    "llima_eagle3_tree_grow": (ctypes.c_int, [_vp, _i32, _i32, _i64, _vp, _i32, _i32, _i32, _vp,
                                              _sz, _vp, _vp, _vp, _vp]),
    "llima_eagle3_tree_finish": (ctypes.c_int, [_vp, _sz, _i32, _i32, _i32, _i32, _vp, _vp, _vp,
                                                _vp, _vp, _vp]),
    "llima_stop_check": (ctypes.c_int, [_vp, _vp, _i32, _i32, _vp, _i32, _vp, _vp, _vp, _vp]),
    "llima_status_string": (ctypes.c_char_p, [ctypes.c_int]),
    "llima_abi_version": (ctypes.c_int, []),
}


class SamplerConfigC(ctypes.Structure):
    """Mirror of llima_sampler_config."""
    _fields_ = [
        ("temperature", ctypes.c_float),
        ("top_k", ctypes.c_int32),
        ("top_p", ctypes.c_float),
        ("min_p", ctypes.c_float),
        ("repetition_penalty", ctypes.c_float),
        ("presence_penalty", ctypes.c_float),
        ("frequency_penalty", ctypes.c_float),
        ("greedy", ctypes.c_int32),
        ("temperature_rows", ctypes.c_void_p),
        ("top_k_rows", ctypes.c_void_p),
        ("top_p_rows", ctypes.c_void_p),
        ("min_p_rows", ctypes.c_void_p),
        ("repetition_penalty_rows", ctypes.c_void_p),
        ("presence_penalty_rows", ctypes.c_void_p),
        ("frequency_penalty_rows", ctypes.c_void_p),
    ]


_lib = None


def lib() -> ctypes.CDLL:
    """Loads the HIP library (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python llima_amd/build.py` "
                "(there is no non-HIP implementation)")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


class LlimaError(RuntimeError):
    def __init__(self, status: int, where: str):
        msg = lib().llima_status_string(status).decode()
        super().__init__(f"{where}: {msg} (status {status})")
        self.status = status


def check(status: int, where: str) -> None:
    if status == LLIMA_E_INVAL or status == LLIMA_E_RANGE:
        # the reference raises std::invalid_argument / std::runtime_error here
        raise ValueError(f"{where}: {lib().llima_status_string(status).decode()} (status {status})")
    if status != LLIMA_OK:
        raise LlimaError(status, where)
