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
    # 4096 rows of 128256 fp32 values need 4096 * 32 regions of 5 KB = 640 MiB
    assert L.llima_sample_workspace_bytes(4096, 128256, 0) > L.llima_sample_noalloc_max_bytes()
    rc = L.llima_sample_noalloc(p, 0, 4096, 128256, 128256, None, None, 0, None, p,
                                ctypes.byref(cfg), p, None, None, None)
    assert rc == _lib.LLIMA_E_SCRATCH


def test_noalloc_graph_replays(gpu, oracle):
    """llima_sample_noalloc captured into a HIP graph (its first call on the
    device made eagerly, as the header requires) and replayed on new inputs
    loaded into the captured buffers between replays: every replay equals the
    oracle on that replay's inputs and an eager llima_sample call with a
    workspace, bit for bit."""
    import torch
    from llima_amd import SamplerConfig, _lib
    from oracle.oracle import SamplerConfig as OC
    L = _lib.lib()
    _say("graph replay llima_sample_noalloc")
    B, V, H = 16, 50000, 300
    cfgd = dict(temperature=0.8, top_k=40, top_p=0.9, min_p=0.02, repetition_penalty=1.2,
                presence_penalty=0.3, frequency_penalty=0.2)
    rng = np.random.default_rng(91)
    xs = [rng.normal(0, 3, (B, V)).astype(np.float32) for _ in range(3)]
    hs = [rng.integers(0, V, size=(B, H)).astype(np.int32) for _ in range(3)]
    us = [rng.random(B).astype(np.float32) for _ in range(3)]
    x = torch.empty((B, V), dtype=torch.float32, device=gpu)
    h = torch.empty((B, H), dtype=torch.int32, device=gpu)
    u = torch.empty(B, dtype=torch.float32, device=gpu)
    ids = torch.empty(B, dtype=torch.int32, device=gpu)
    probs = torch.empty(B, dtype=torch.float32, device=gpu)
    cfg, keep_alive = SamplerConfig(**cfgd).to_c(B, gpu)

    def launch(stream):
        rc = L.llima_sample_noalloc(x.data_ptr(), _lib.LLIMA_F32, B, V, V, h.data_ptr(), None, H,
                                    None, u.data_ptr(), ctypes.byref(cfg), ids.data_ptr(),
                                    probs.data_ptr(), None, stream)
        assert rc == 0, rc

    def load(i):
        x.copy_(torch.from_numpy(xs[i]))
        h.copy_(torch.from_numpy(hs[i]))
        u.copy_(torch.from_numpy(us[i]))

    load(0)
    launch(torch.cuda.current_stream(gpu).cuda_stream)        # eager: the first call on the device
    torch.cuda.synchronize(gpu)
    graph = torch.cuda.CUDAGraph()
    cap = torch.cuda.Stream(gpu)
    cap.wait_stream(torch.cuda.current_stream(gpu))
    with torch.cuda.graph(graph, stream=cap):
        launch(cap.cuda_stream)
    torch.cuda.synchronize(gpu)
    wsb = L.llima_sample_workspace_bytes(B, V, _lib.LLIMA_F32)
    ws = torch.empty(wsb, dtype=torch.uint8, device=gpu)
    for i in range(3):
        load(i)
        ids.fill_(-7)
        torch.cuda.synchronize(gpu)
        graph.replay()
        torch.cuda.synchronize(gpu)
        gi, gp = ids.cpu().numpy(), probs.cpu().numpy()
        eids, eprobs = oracle.sample(xs[i], us[i], OC(**cfgd), history=hs[i])
        assert np.array_equal(gi, eids), (i, np.flatnonzero(gi != eids)[:8])
        assert np.array_equal(gp.view(np.uint32), eprobs.view(np.uint32)), i
        # an eager call of the workspace entry point between replays
        w = dict(logits=xs[i], history=hs[i], bitmask=None, uniforms=us[i], cfg=cfgd)
        a = _call(L, "workspace", w, gpu, ws)
        assert np.array_equal(a[0], gi) and np.array_equal(a[1].view(np.uint32), gp.view(np.uint32))
    del keep_alive
