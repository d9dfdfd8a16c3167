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
    assert L.llima_status_string(-6).decode() == "first call on this device made under stream capture"
    assert L.llima_sample_workspace_bytes(64, 128256, 0) > 0
    # the documented size rule: B (5120 S + 64) bytes, S chunks of 4096 fp32
    # or 8192 bf16 values; the C5 shape fits the no-allocation scratch
    for B, V, dt, S in ((64, 128256, 0, 32), (32, 151936, 0, 38), (256, 262144, 1, 32), (3, 8193, 1, 2)):
        assert L.llima_sample_workspace_bytes(B, V, dt) == B * (5120 * S + 64)
    assert L.llima_sample_noalloc_max_bytes() == 48 << 20
    assert L.llima_sample_workspace_bytes(256, 262144, 1) <= L.llima_sample_noalloc_max_bytes()
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
    # heap top-k: k in [1, 32] (topk<T> throws outside it), at most the row's width
    assert L.llima_topk(p, 0, 1, 100, 100, 0, p, p, None) == -1
    assert L.llima_topk(p, 0, 1, 100, 100, 33, p, p, None) == -1
    assert L.llima_topk(p, 0, 1, 4, 4, 5, p, p, None) == -1
    assert L.llima_topk(p, 0, 1, 100, 50, 5, p, p, None) == -1      # stride below the width
    assert L.llima_topk(p, 2, 1, 100, 100, 5, p, p, None) == -1      # dtype
    assert L.llima_topk(None, 0, 0, 100, 100, 5, None, None, None) == 0
    # EAGLE3 tree: K in [1, 32], depth in [1, 16], a state buffer of the stated size
    tb = L.llima_eagle3_tree_bytes(5, 4)
    assert tb > 0 and L.llima_eagle3_tree_bytes(0, 4) == 0
    assert L.llima_eagle3_tree_begin(p, 1, 32000, p, 0, 4, p, tb, p, None) == -1
    assert L.llima_eagle3_tree_begin(p, 1, 32000, p, 33, 4, p, tb, p, None) == -1
    assert L.llima_eagle3_tree_begin(p, 1, 32000, p, 5, 17, p, tb, p, None) == -1
    assert L.llima_eagle3_tree_begin(p, 1, 3, p, 5, 4, p, tb, p, None) == -1     # Vd < K
    assert L.llima_eagle3_tree_begin(p, 1, 32000, p, 5, 4, p, tb - 1, p, None) == -4
    assert L.llima_eagle3_tree_grow(p, 1, 32000, 32000, p, 5, 4, 0, p, tb, p, p, p, None) == -1
    assert L.llima_eagle3_tree_grow(p, 1, 32000, 32000, p, 5, 4, 4, p, tb, p, p, p, None) == -1
    assert L.llima_eagle3_tree_finish(p, tb, 5, 4, 33, 0, p, p, p, p, p, None) == -1
    assert L.llima_eagle3_tree_finish(p, tb, 2, 2, 7, 0, p, p, p, p, p, None) == -1  # > nodes
    # stop check: a vocabulary and a stop mask are required; B = 0 launches nothing
    assert L.llima_stop_check(p, None, 1, 4, None, 100, None, p, None, None) == -1
    assert L.llima_stop_check(p, None, 1, 4, p, 0, None, p, None, None) == -1
    assert L.llima_stop_check(None, None, 0, 4, p, 100, None, None, None, None) == 0
    # LM head: H a multiple of 8, a finite softcap, logit dtype f32 or bf16
    wl = L.llima_lm_head_argmax_workspace_bytes(1, 1000)
    assert L.llima_lm_head_argmax(p, p, 1, 12, 1000, 0.0, 1, p, None, None, p, wl, None) == -1
    assert L.llima_lm_head_argmax(p, p, 1, 16, 1000, float("nan"), 1, p, None, None, p, wl,
                                  None) == -1
    assert L.llima_lm_head_argmax(p, p, 1, 16, 1000, 0.0, 7, p, None, None, p, wl, None) == -1
    # bf16 logits output only with bf16 logits
    assert L.llima_lm_head_argmax(p, p, 1, 16, 1000, 0.0, 0x100, p, None, None, p, wl, None) == -1
    assert L.llima_lm_head_argmax(p, p, 1, 16, 1000, 0.0, 0x300, p, None, None, p, wl, None) == -1
    assert L.llima_lm_head_argmax(None, p, 0, 16, 1000, 0.0, 0x101, None, None, None, None, 0,
                                  None) == 0
    assert L.llima_lm_head_argmax(p, p, 1, 16, 1000, 0.0, 1, p, None, None, p, 0, None) == -4
    # packed LM head: H a multiple of 256 (at most 65536), the packed size as stated
    assert L.llima_lm_head_packed_bytes(1000, 100) == 0
    assert L.llima_lm_head_packed_bytes(1000, 65536 + 256) == 0
    assert L.llima_lm_head_packed_bytes(1000, 256) == 32 * 32 * 256 * 2      # 1000 -> 1024 rows
    assert L.llima_lm_head_pack(p, 1000, 100, p, 1 << 20, None) == -1
    assert L.llima_lm_head_pack(p, 1000, 256, p, 32 * 32 * 256 * 2 - 1, None) == -4
    assert L.llima_lm_head_pack(ctypes.c_void_p(24), 1000, 256, p, 1 << 20, None) == -1
    assert L.llima_lm_head_argmax_packed_workspace_bytes(1, 100, 1000) == 0
    wp = L.llima_lm_head_argmax_packed_workspace_bytes(1, 256, 1000)
    assert wp >= 32 * 8                                       # a key per 32 vocab rows and row
    assert L.llima_lm_head_argmax_packed(p, p, 1, 100, 1000, 0.0, 1, p, None, None, p, wp,
                                         None) == -1
    assert L.llima_lm_head_argmax_packed(p, p, 1, 256, 1000, float("inf"), 1, p, None, None, p,
                                         wp, None) == -1
    assert L.llima_lm_head_argmax_packed(p, p, 1, 256, 1000, 0.0, 1, p, None, None, p, wp - 1,
                                         None) == -4
    assert L.llima_lm_head_argmax_packed(p, p, 1, 256, 1000, 0.0, 1, p, None, None, p, 0,
                                         None) == -4
    assert L.llima_lm_head_argmax_packed(None, p, 0, 256, 1000, 0.0, 1, None, None, None, None,
                                         0, None) == 0
    # LM head scoring: the argmax checks, targets and both outputs required, no
    # logits output flag; its workspace holds the keys and the slot sums
    ws = L.llima_lm_head_score_workspace_bytes(2, 1000)
    assert ws > L.llima_lm_head_argmax_workspace_bytes(2, 1000)
    assert L.llima_lm_head_score_workspace_bytes(0, 1000) == 0
    assert L.llima_lm_head_score(p, p, 1, 12, 1000, 0.0, 1, p, p, p, p, ws, None) == -1
    assert L.llima_lm_head_score(p, p, 1, 16, 1000, float("nan"), 1, p, p, p, p, ws, None) == -1
    assert L.llima_lm_head_score(p, p, 1, 16, 1000, 0.0, 0x101, p, p, p, p, ws, None) == -1
    assert L.llima_lm_head_score(p, p, 1, 16, 1000, 0.0, 1, None, p, p, p, ws, None) == -1
    assert L.llima_lm_head_score(p, p, 1, 16, 1000, 0.0, 1, p, None, p, p, ws, None) == -1
    assert L.llima_lm_head_score(p, p, 1, 16, 1000, 0.0, 1, p, p, None, p, ws, None) == -1
    assert L.llima_lm_head_score(p, p, 2, 16, 1000, 0.0, 1, p, p, p, p, ws - 1, None) == -4
    assert L.llima_lm_head_score(None, p, 0, 16, 1000, 0.0, 1, None, None, None, None, 0,
                                 None) == 0
    wsp = L.llima_lm_head_score_packed_workspace_bytes(2, 256, 1000)
    assert wsp > L.llima_lm_head_argmax_packed_workspace_bytes(2, 256, 1000)
    assert L.llima_lm_head_score_packed_workspace_bytes(2, 100, 1000) == 0
    assert L.llima_lm_head_score_packed(p, p, 1, 100, 1000, 0.0, 1, p, p, p, p, wsp, None) == -1
    assert L.llima_lm_head_score_packed(p, p, 1, 256, 1000, 0.0, 0x101, p, p, p, p, wsp,
                                        None) == -1
    assert L.llima_lm_head_score_packed(p, p, 1, 256, 1000, 0.0, 1, None, p, p, p, wsp,
                                        None) == -1
    assert L.llima_lm_head_score_packed(p, p, 2, 256, 1000, 0.0, 1, p, p, p, p, wsp - 1,
                                        None) == -4
    assert L.llima_lm_head_score_packed(None, p, 0, 256, 1000, 0.0, 1, None, None, None, None,
                                        0, None) == 0
    # LM head greedy verification: the head's checks over B (D + 1) rows, outputs required
    wv = L.llima_lm_head_verify_greedy_workspace_bytes(2, 3, 1000)
    assert wv > L.llima_lm_head_argmax_workspace_bytes(8, 1000)
    assert L.llima_lm_head_verify_greedy_workspace_bytes(2, -1, 1000) == 0
    assert L.llima_lm_head_verify_greedy(p, p, 2, -1, 16, 1000, 0.0, 1, p, p, p, p, wv, None) == -1
    assert L.llima_lm_head_verify_greedy(p, p, 2, 3, 12, 1000, 0.0, 1, p, p, p, p, wv, None) == -1
    assert L.llima_lm_head_verify_greedy(p, p, 2, 3, 16, 1000, 0.0, 0x101, p, p, p, p, wv,
                                         None) == -1
    assert L.llima_lm_head_verify_greedy(p, p, 2, 3, 16, 1000, 0.0, 1, None, p, p, p, wv,
                                         None) == -1
    assert L.llima_lm_head_verify_greedy(p, p, 2, 3, 16, 1000, 0.0, 1, p, None, p, p, wv,
                                         None) == -1
    assert L.llima_lm_head_verify_greedy(p, p, 2, 3, 16, 1000, 0.0, 1, p, p, p, p, wv - 1,
                                         None) == -4
    assert L.llima_lm_head_verify_greedy(None, p, 0, 3, 16, 1000, 0.0, 1, None, None, None,
                                         None, 0, None) == 0
    wvp = L.llima_lm_head_verify_greedy_packed_workspace_bytes(2, 3, 256, 1000)
    assert wvp > 0 and L.llima_lm_head_verify_greedy_packed_workspace_bytes(2, 3, 100, 1000) == 0
    assert L.llima_lm_head_verify_greedy_packed(p, p, 2, 3, 100, 1000, 0.0, 1, p, p, p, p, wvp,
                                                None) == -1
    assert L.llima_lm_head_verify_greedy_packed(p, p, 2, 3, 256, 1000, 0.0, 1, p, p, p, p,
                                                wvp - 1, None) == -4
    # LM head tree verification: K, n_paths, L positive, the index arrays and out required
    wt = L.llima_lm_head_verify_tree_workspace_bytes(16, 1000)
    assert wt > L.llima_lm_head_argmax_workspace_bytes(16, 1000)
    assert L.llima_lm_head_verify_tree_workspace_bytes(0, 1000) == 0
    assert L.llima_lm_head_verify_tree(p, p, 0, 16, 1000, 0.0, 1, p, p, 2, 3, p, p, wt, None) == -1
    assert L.llima_lm_head_verify_tree(p, p, 16, 16, 1000, 0.0, 1, p, p, 0, 3, p, p, wt, None) == -1
    assert L.llima_lm_head_verify_tree(p, p, 16, 16, 1000, 0.0, 1, None, p, 2, 3, p, p, wt,
                                       None) == -1
    assert L.llima_lm_head_verify_tree(p, p, 16, 12, 1000, 0.0, 1, p, p, 2, 3, p, p, wt, None) == -1
    assert L.llima_lm_head_verify_tree(p, p, 16, 16, 1000, 0.0, 0x101, p, p, 2, 3, p, p, wt,
                                       None) == -1
    assert L.llima_lm_head_verify_tree(p, p, 16, 16, 1000, 0.0, 1, p, p, 2, 3, p, p, wt - 1,
                                       None) == -4
    wtp = L.llima_lm_head_verify_tree_packed_workspace_bytes(16, 256, 1000)
    assert wtp > 0 and L.llima_lm_head_verify_tree_packed_workspace_bytes(16, 100, 1000) == 0
    assert L.llima_lm_head_verify_tree_packed(p, p, 16, 256, 1000, 0.0, 1, p, p, 2, 3, p, p,
                                              wtp - 1, None) == -4
    # rejection verification: V % 4 == 0, D <= 255, 16-byte aligned rows
    vw = L.llima_verify_rejection_workspace_bytes(1, 1, 4096)
    assert L.llima_verify_rejection(p, p, 1, 1, 4094, p, p, p, p, p, p, vw, None) == -1
    assert L.llima_verify_rejection(p, p, 1, 256, 4096, p, p, p, p, p, p, vw, None) == -1
    assert L.llima_verify_rejection(ctypes.c_void_p(20), p, 1, 1, 4096, p, p, p, p, p, p, vw,
                                    None) == -1
    assert L.llima_verify_rejection(p, p, 1, 1, 4096, p, p, p, p, p, p, vw - 1, None) == -4


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


def test_sampler_config_top_k_statement():
    """Per-row top_k from host memory: the scalar states whether every row has
    top-k in (0, V) (1) or makes no statement (0); a device tensor needs the
    caller's word (top_k_every_row)."""
    import torch
    from llima_amd import SamplerConfig
    dev = torch.device("cpu")
    assert SamplerConfig(top_k=torch.tensor([5, 50])).to_c(2, dev, 100)[0].top_k == 1
    assert SamplerConfig(top_k=torch.tensor([5, 0])).to_c(2, dev, 100)[0].top_k == 0
    assert SamplerConfig(top_k=torch.tensor([5, 100])).to_c(2, dev, 100)[0].top_k == 0
    assert SamplerConfig(top_k=torch.tensor([0, 0]), top_k_every_row=True).to_c(2, dev, 100)[0].top_k == 1
    assert SamplerConfig(top_k=7).to_c(2, dev, 100)[0].top_k == 7


def test_python_api_rejects_host_tensors():
    import torch
    import llima_amd
    with pytest.raises(ValueError):
        llima_amd.argmax(torch.zeros(2, 8))
    assert llima_amd.resolve_draft_tokens([1, 2], [1, 3]) == [(1, True), (3, False)]
    with pytest.raises(RuntimeError):
        llima_amd.resolve_draft_tokens([1, 2], [1, 2])
