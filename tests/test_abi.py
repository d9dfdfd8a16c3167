"""CPU tests of the C ABI library and the host-side Python logic (no GPU calls)."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "llima_sampler.h")


def _declared():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(llima_[a-z_0-9]+)\s*\(", src)))


def test_header_declares_the_entry_points():
    names = _declared()
    for n in ["llima_argmax", "llima_sample", "llima_verify_greedy", "llima_verify_tree",
              "llima_verify_rejection", "llima_topk", "llima_score_logits",
              "llima_mtp_masked_argmax"]:
        assert n in names


def test_library_exports_every_declared_symbol():
    from llima_amd import _lib
    L = ctypes.CDLL(_lib.LIB_PATH)
    for name in _declared():
        assert hasattr(L, name), name
    assert set(_lib.SIGNATURES) == set(_declared())


def test_host_only_entry_points():
    from llima_amd._lib import lib
    L = lib()
    assert L.llima_abi_version() == 2
    assert L.llima_status_string(-4).decode() == "workspace missing or too small"
    assert L.llima_sample_workspace_bytes(64, 128256, 0) > 0
    assert L.llima_argmax_workspace_bytes(0, 10, 0) == 0
    # argument validation happens before any launch
    assert L.llima_argmax(None, 0, 1, 10, 10, 0, 0, None, None, None, 0, None) == -1
    assert L.llima_sample(ctypes.c_void_p(16), 7, 1, 10, 10, None, None, 0, None,
                          ctypes.c_void_p(16), None, ctypes.c_void_p(16), None, None, None, 0,
                          None) == -1
    assert L.llima_verify_rejection(ctypes.c_void_p(16), ctypes.c_void_p(16), 1, 1, (1 << 22) + 4,
                                    ctypes.c_void_p(16), ctypes.c_void_p(16), ctypes.c_void_p(16),
                                    ctypes.c_void_p(16), ctypes.c_void_p(16), None, 0, None) == -1
    p = ctypes.c_void_p(16)
    # split buffers: QUARTERS is refused, as are more than 16 splits and empty splits
    ptrs = (ctypes.c_void_p * 17)(*([16] * 17))
    widths = (ctypes.c_int32 * 17)(*([64] * 17))
    assert L.llima_argmax_splits(ptrs, widths, None, 2, 0, 1, 2, p, None, p, 1 << 20, None) == -1
    assert L.llima_argmax_splits(ptrs, widths, None, 17, 0, 1, 0, p, None, p, 1 << 20, None) == -1
    assert L.llima_argmax_splits(ptrs, widths, None, 0, 0, 1, 0, p, None, p, 1 << 20, None) == -1
    zero = (ctypes.c_int32 * 2)(64, 0)
    assert L.llima_argmax_splits(ptrs, zero, None, 2, 0, 1, 0, p, None, p, 1 << 20, None) == -1
    assert L.llima_argmax_splits(ptrs, widths, None, 2, 0, 1, 3, p, None, None, 0, None) == -4
    assert L.llima_verify_greedy_splits(ptrs, widths, None, 2, 0, 1, 2, 2, p, p, p, p, 1 << 20,
                                        None) == -1
    assert L.llima_verify_greedy(p, 0, 1, 2, 64, 0, 4, p, p, p, p, 1 << 20, None) == -1
    assert L.llima_sample_noalloc(p, 0, 4096, 128256, 128256, None, None, 0, None, p,
                                  ctypes.byref(_lib_cfg()), p, None, None, None) == -5
    assert L.llima_score_logits(None, 0, 1, 10, 10, p, p, p, p, 1 << 20, None) == -1
    assert L.llima_score_logits(p, 0, 1, 10, 10, p, p, p, None, 0, None) == -4
    assert L.llima_score_logits_workspace_bytes(256, 262144, 1) > 0
    # the reference's own checks: V a multiple of C, top_k in [1, C]
    wsb = L.llima_mtp_masked_argmax_workspace_bytes(1)
    assert wsb > 0
    assert L.llima_mtp_masked_argmax(p, 4, 4, p, 2, p, 1, 1, 10, 10, p, p, None, p, wsb,
                                     None) == -1
    assert L.llima_mtp_masked_argmax(p, 4, 4, p, 5, p, 1, 1, 8, 8, p, p, None, p, wsb, None) == -1
    assert L.llima_mtp_masked_argmax(p, 4, 4, p, 0, p, 1, 1, 8, 8, p, p, None, p, wsb, None) == -1
    assert L.llima_mtp_masked_argmax(p, 9000, 9000, p, 1, p, 1, 1, 9000, 9000, p, p, None, p,
                                     wsb, None) == -1         # beyond 8192 centroids
    assert L.llima_mtp_masked_argmax(p, 4, 4, p, 1, None, 1, 1, 8, 8, None, p, None, p, wsb,
                                     None) == -1
    assert L.llima_mtp_masked_argmax(p, 4, 4, p, 1, p, 1, 1, 8, 8, p, p, None, None, 0,
                                     None) == -4              # no workspace


def _lib_cfg():
    from llima_amd._lib import SamplerConfigC
    c = SamplerConfigC()
    c.temperature, c.repetition_penalty = 1.0, 1.0
    return c


def test_config_struct_layout_matches_header():
    from llima_amd._lib import SamplerConfigC
    # 8 scalar 4-byte fields then 7 pointers
    assert ctypes.sizeof(SamplerConfigC) == 8 * 4 + 7 * 8
    assert SamplerConfigC.temperature_rows.offset == 32


def test_sampler_config_rows_to_c():
    import torch
    from llima_amd import SamplerConfig
    cfg = SamplerConfig(temperature=torch.tensor([0.5, 0.7]), top_k=3, top_p=0.9)
    c, keep = cfg.to_c(2, torch.device("cpu"))
    assert c.top_k == 3 and abs(c.top_p - 0.9) < 1e-7
    assert c.temperature_rows == keep[0].data_ptr()
    assert c.top_k_rows is None
    with pytest.raises(ValueError):
        cfg.to_c(3, torch.device("cpu"))


def test_python_api_rejects_host_tensors():
    import torch
    import llima_amd
    with pytest.raises(ValueError):
        llima_amd.argmax(torch.zeros(2, 8))
    assert llima_amd.resolve_draft_tokens([1, 2], [1, 3]) == [(1, True), (3, False)]
    with pytest.raises(RuntimeError):
        llima_amd.resolve_draft_tokens([1, 2], [1, 2])
