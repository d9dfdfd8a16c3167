"""llima_sample_noalloc (the sampler with its workspace in the library's static
device scratch) against llima_sample with a caller workspace, both called
through the C ABI on identical inputs: ids, probabilities and kept-set bitmasks
bit for bit, on consecutive calls whose second is smaller (the scratch keeps
the first call's contents), and the sampler's outputs against the oracle."""
import ctypes

import numpy as np
import pytest

from llima_amd import workloads as wl

pytestmark = pytest.mark.gpu


def _say(*a):
    print("[gpu-case]", *a, flush=True)


def _t(a, dev):
    import torch
    if a is None:
        return None
    if a.dtype == np.uint16:
        return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).to(dev).view(torch.bfloat16)
    if a.dtype == np.uint32:
        return torch.from_numpy(np.ascontiguousarray(a).view(np.int32)).to(dev)
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _call(L, entry, w, dev, ws=None):
    """One llima_sample / llima_sample_noalloc call on workload dict w; returns
    (ids, probs, keep) as numpy arrays."""
    import torch
    from llima_amd import SamplerConfig, _lib
    x = _t(w["logits"], dev)
    B, V = x.shape
    dt = _lib.LLIMA_BF16 if x.dtype == torch.bfloat16 else _lib.LLIMA_F32
    h = _t(w["history"], dev)
    m = _t(w["bitmask"], dev)
    u = _t(w["uniforms"], dev)
    cfg, keep_alive = SamplerConfig(**w["cfg"]).to_c(B, dev)
    nw = (V + 31) // 32
    ids = torch.full((B,), -7, dtype=torch.int32, device=dev)
    probs = torch.full((B,), -7.0, dtype=torch.float32, device=dev)
    keep = torch.zeros((B, nw), dtype=torch.int32, device=dev)
    H = 0 if h is None else h.shape[1]
    hp = None if h is None else h.data_ptr()
    mp = None if m is None else m.data_ptr()
    stream = torch.cuda.current_stream(dev).cuda_stream
    common = (x.data_ptr(), dt, B, V, V, hp, None, H, mp, u.data_ptr(), ctypes.byref(cfg),
              ids.data_ptr(), probs.data_ptr(), keep.data_ptr())
    if entry == "noalloc":
        rc = L.llima_sample_noalloc(*common, stream)
    else:
        rc = L.llima_sample(*common, ws.data_ptr(), ws.numel(), stream)
    assert rc == 0, (entry, rc)
    torch.cuda.synchronize(dev)
    del keep_alive
    return ids.cpu().numpy(), probs.cpu().numpy(), keep.cpu().numpy()


def _workloads():
    big = wl.batched_penalties(B=64, V=128256, H=2048)
    small = wl.constrained(B=3, V=20000, runs=40, seed=11)
    dense = wl.top_p_only(B=16, V=50000, seed=12)             # the dense path (no top-k)
    return big, small, dense


def test_noalloc_matches_workspace_entry_point(gpu, oracle):
    import torch
    from llima_amd import _lib
    L = _lib.lib()
    big, small, dense = _workloads()
    wsb = L.llima_sample_workspace_bytes(64, 128256, _lib.LLIMA_F32)
    assert wsb <= L.llima_sample_noalloc_max_bytes()
    ws = torch.empty(wsb, dtype=torch.uint8, device=gpu)
    for w, what in ((big, "batched_penalties B=64 V=128256"), (small, "constrained B=3 V=20000"),
                    (dense, "top_p_only B=16 V=50000"),
                    (big, "batched_penalties B=64 V=128256 again")):
        _say("llima_sample_noalloc vs llima_sample:", what)
        a = _call(L, "noalloc", w, gpu)
        b = _call(L, "workspace", w, gpu, ws)
        for x, y in zip(a, b):
            assert np.array_equal(x, y)
        from oracle import oracle as orc
        eids, eprobs = orc.sample(w["logits"], w["uniforms"], orc.SamplerConfig(**w["cfg"]),
                                  history=w["history"], bitmask=w["bitmask"])
        assert np.array_equal(a[0], eids) and np.array_equal(a[1], eprobs)


def test_noalloc_rejects_calls_beyond_the_scratch(gpu):
    from llima_amd import SamplerConfig, _lib
    L = _lib.lib()
    cfg, _ = SamplerConfig(top_k=5).to_c(4096, gpu)
    p = ctypes.c_void_p(256)
    # 4096 rows of 128256 fp32 values need 4096 * 32 regions of 4 KB = 512 MiB
    assert L.llima_sample_workspace_bytes(4096, 128256, 0) > L.llima_sample_noalloc_max_bytes()
    rc = L.llima_sample_noalloc(p, 0, 4096, 128256, 128256, None, None, 0, None, p,
                                ctypes.byref(cfg), p, None, None, None)
    assert rc == _lib.LLIMA_E_SCRATCH
