"""HIP graph replay: one llima_sample call (the sweep + finish kernels, or the
dense path), one llima_verify_rejection call, and the LM head's scoring and
greedy verification entry points captured into graphs through
the C ABI, then replayed several times.  Between replays the program's own
eager work writes new inputs into the captured buffers and synchronises; every
replay is checked against the oracle on that replay's inputs."""
import ctypes

import numpy as np
import pytest

from llima_amd import workloads as wl

pytestmark = pytest.mark.gpu

REPLAYS = 3


def _say(*a):
    print("[gpu-case]", *a, flush=True)


SAMPLE_CFGS = {
    "sweep_finish": dict(temperature=0.8, top_k=40, top_p=0.9, min_p=0.02, repetition_penalty=1.2,
                         presence_penalty=0.3, frequency_penalty=0.2),
    "dense": dict(temperature=0.9, top_p=0.9, min_p=0.01, repetition_penalty=1.1),
    "dense_plain": dict(temperature=1.0),
    "masked_wide": dict(temperature=1.0, top_p=0.9),          # with a sparse mask: the wide finish
}


@pytest.mark.parametrize("name", list(SAMPLE_CFGS))
def test_sample_graph_replays(gpu, oracle, name):
    import torch
    from llima_amd import SamplerConfig, _lib
    from oracle.oracle import SamplerConfig as OC
    _say("graph replay llima_sample", name)
    L = _lib.lib()
    cfgd = SAMPLE_CFGS[name]
    rng = np.random.default_rng(31 + list(SAMPLE_CFGS).index(name))
    B, V, H = 16, 50000, 300
    xs = [rng.normal(0, 3, (B, V)).astype(np.float32) for _ in range(REPLAYS)]
    hs = [rng.integers(0, V, size=(B, H)).astype(np.int32) for _ in range(REPLAYS)]
    us = [rng.random(B).astype(np.float32) for _ in range(REPLAYS)]
    x = torch.empty((B, V), dtype=torch.float32, device=gpu)
    h = torch.empty((B, H), dtype=torch.int32, device=gpu)
    u = torch.empty(B, dtype=torch.float32, device=gpu)
    nw = (V + 31) // 32
    masked = name == "masked_wide"
    ms = [(rng.random((B, nw)) < 0.05).astype(np.uint32) * np.uint32(0xFFFFFFFF) for _ in range(REPLAYS)]
    m = torch.empty((B, nw), dtype=torch.int32, device=gpu)
    ids = torch.empty(B, dtype=torch.int32, device=gpu)
    probs = torch.empty(B, dtype=torch.float32, device=gpu)
    keep = torch.empty((B, nw), dtype=torch.int32, device=gpu)
    nws = L.llima_sample_workspace_bytes(B, V, _lib.LLIMA_F32)
    ws = torch.empty(nws, dtype=torch.uint8, device=gpu)
    cfg, keep_alive = SamplerConfig(**cfgd).to_c(B, gpu)

    def launch(stream):
        rc = L.llima_sample(x.data_ptr(), _lib.LLIMA_F32, B, V, V, h.data_ptr(), None, H,
                            m.data_ptr() if masked else None, u.data_ptr(), ctypes.byref(cfg),
                            ids.data_ptr(), probs.data_ptr(), keep.data_ptr(), ws.data_ptr(), nws,
                            stream)
        assert rc == 0

    def load(i):
        x.copy_(torch.from_numpy(xs[i]))
        h.copy_(torch.from_numpy(hs[i]))
        u.copy_(torch.from_numpy(us[i]))
        m.copy_(torch.from_numpy(ms[i].view(np.int32)))

    load(0)
    launch(torch.cuda.current_stream(gpu).cuda_stream)        # eager warmup
    torch.cuda.synchronize(gpu)
    graph = torch.cuda.CUDAGraph()
    cap = torch.cuda.Stream(gpu)
    cap.wait_stream(torch.cuda.current_stream(gpu))
    with torch.cuda.graph(graph, stream=cap):
        launch(cap.cuda_stream)
    torch.cuda.synchronize(gpu)
    for i in range(REPLAYS):
        load(i)
        ids.fill_(-7)
        torch.cuda.synchronize(gpu)
        graph.replay()
        torch.cuda.synchronize(gpu)
        eids, eprobs, ekeep = oracle.sample(xs[i], us[i], OC(**cfgd), history=hs[i],
                                            bitmask=ms[i] if masked else None, want_keep=True)
        gi = ids.cpu().numpy()
        assert (gi == eids).all(), (name, i, np.flatnonzero(gi != eids)[:8])
        assert (probs.cpu().numpy().view(np.uint32) == eprobs.view(np.uint32)).all(), (name, i)
        assert (keep.cpu().numpy().view(np.uint32) == ekeep).all(), (name, i)
    del keep_alive


def test_verify_rejection_graph_replays(gpu, oracle):
    import torch
    import llima_amd
    _say("graph replay llima_verify_rejection")
    ws_ = [wl.speculative(B=4, D=5, V=30000, seed=40 + i) for i in range(REPLAYS)]

    def dev(a):
        return torch.from_numpy(np.ascontiguousarray(a)).to(gpu)
    cur = {k: dev(ws_[0][k]) for k in ("target", "draft", "draft_ids", "u_accept", "u_resample")}
    out = llima_amd.verify_rejection(cur["target"], cur["draft"], cur["draft_ids"],
                                     cur["u_accept"], cur["u_resample"])       # eager warmup
    torch.cuda.synchronize(gpu)
    graph = torch.cuda.CUDAGraph()
    cap = torch.cuda.Stream(gpu)
    cap.wait_stream(torch.cuda.current_stream(gpu))
    with torch.cuda.graph(graph, stream=cap):
        out = llima_amd.verify_rejection(cur["target"], cur["draft"], cur["draft_ids"],
                                         cur["u_accept"], cur["u_resample"])
    torch.cuda.synchronize(gpu)
    for i in range(REPLAYS):
        for k in cur:
            cur[k].copy_(dev(ws_[i][k]))
        torch.cuda.synchronize(gpu)
        graph.replay()
        torch.cuda.synchronize(gpu)
        w = ws_[i]
        exp = oracle.verify_rejection(w["target"], w["draft"], w["draft_ids"], w["u_accept"],
                                      w["u_resample"])
        for got, want in zip(out, exp):
            assert np.array_equal(got.cpu().numpy(), want), i


def test_lm_head_score_graph_replays(gpu, oracle):
    """llima_lm_head_score_packed captured through the C ABI: each replay, on new
    hidden rows and targets, equals an eager call bit for bit and the oracle's
    score_logits over the head's logits within 1e-5."""
    import torch
    import llima_amd
    from llima_amd import _lib
    _say("graph replay llima_lm_head_score_packed")
    L = _lib.lib()
    rng = np.random.default_rng(77)
    B, H, V = 40, 512, 20000
    xs = [wl.f32_to_bf16_bits(rng.normal(0, 1, (B, H)).astype(np.float32)) for _ in range(REPLAYS)]
    ts = [rng.integers(0, V, B).astype(np.int32) for _ in range(REPLAYS)]
    wf = wl.f32_to_bf16_bits(rng.normal(0, 4.0 / np.sqrt(H), (V, H)).astype(np.float32))
    w = torch.from_numpy(wf.view(np.int16)).to(gpu).view(torch.bfloat16)
    pk = llima_amd.lm_head_pack(w)
    x = torch.empty((B, H), dtype=torch.bfloat16, device=gpu)
    tg = torch.empty(B, dtype=torch.int32, device=gpu)
    lp = torch.empty(B, dtype=torch.float64, device=gpu)
    gr = torch.empty(B, dtype=torch.int32, device=gpu)
    nws = L.llima_lm_head_score_packed_workspace_bytes(B, H, V)
    ws = torch.empty(nws, dtype=torch.uint8, device=gpu)

    def launch(stream):
        rc = L.llima_lm_head_score_packed(x.data_ptr(), pk.data.data_ptr(), B, H, V, 0.0,
                                          _lib.LLIMA_BF16, tg.data_ptr(), lp.data_ptr(),
                                          gr.data_ptr(), ws.data_ptr(), nws, stream)
        assert rc == 0

    def load(i):
        x.copy_(torch.from_numpy(xs[i].view(np.int16)).view(torch.bfloat16))
        tg.copy_(torch.from_numpy(ts[i]))

    load(0)
    launch(torch.cuda.current_stream(gpu).cuda_stream)        # eager warmup
    torch.cuda.synchronize(gpu)
    graph = torch.cuda.CUDAGraph()
    cap = torch.cuda.Stream(gpu)
    cap.wait_stream(torch.cuda.current_stream(gpu))
    with torch.cuda.graph(graph, stream=cap):
        launch(cap.cuda_stream)
    torch.cuda.synchronize(gpu)
    for i in range(REPLAYS):
        load(i)
        lp.fill_(0.0)
        gr.fill_(-7)
        torch.cuda.synchronize(gpu)
        graph.replay()
        torch.cuda.synchronize(gpu)
        got_lp, got_g = lp.cpu().numpy().copy(), gr.cpu().numpy().copy()
        elp, eg = llima_amd.lm_head_score(x, pk, tg)
        assert (got_lp.view(np.uint64) == elp.cpu().numpy().view(np.uint64)).all(), i
        assert (got_g == eg.cpu().numpy().astype(np.int32)).all(), i
        _, _, logits = llima_amd.lm_head_argmax(x, pk, return_logits=True)
        lg = logits.cpu().numpy()
        for r in range(B):
            olp, og = oracle.score_logits(lg[r], int(ts[i][r]))
            assert abs(got_lp[r] - olp) <= 1e-5 and bool(got_g[r]) == og, (i, r)


def test_lm_head_verify_greedy_graph_replays(gpu):
    """llima_lm_head_verify_greedy captured through the C ABI (the head's passes,
    lmh_finish and lmh_chain): each replay, on new hidden rows and drafts,
    equals an eager call."""
    import torch
    import llima_amd
    from llima_amd import _lib
    _say("graph replay llima_lm_head_verify_greedy")
    L = _lib.lib()
    rng = np.random.default_rng(78)
    B, D, H, V = 6, 4, 512, 9000
    xs = [wl.f32_to_bf16_bits(rng.normal(0, 1, (B * (D + 1), H)).astype(np.float32))
          for _ in range(REPLAYS)]
    wf = wl.f32_to_bf16_bits(rng.normal(0, 4.0 / np.sqrt(H), (V, H)).astype(np.float32))
    w = torch.from_numpy(wf.view(np.int16)).to(gpu).view(torch.bfloat16)
    x = torch.empty((B, D + 1, H), dtype=torch.bfloat16, device=gpu)
    dr = torch.empty((B, D), dtype=torch.int32, device=gpu)
    acc = torch.empty(B, dtype=torch.int32, device=gpu)
    em = torch.empty((B, D + 1), dtype=torch.int32, device=gpu)
    nws = L.llima_lm_head_verify_greedy_workspace_bytes(B, D, V)
    ws = torch.empty(nws, dtype=torch.uint8, device=gpu)

    def launch(stream):
        rc = L.llima_lm_head_verify_greedy(x.data_ptr(), w.data_ptr(), B, D, H, V, 0.0,
                                           _lib.LLIMA_BF16, dr.data_ptr(), acc.data_ptr(),
                                           em.data_ptr(), ws.data_ptr(), nws, stream)
        assert rc == 0

    drafts = []
    for i in range(REPLAYS):                     # drafts matching a prefix of the head's ids
        xi = torch.from_numpy(xs[i].view(np.int16)).to(gpu).view(torch.bfloat16)
        tok = llima_amd.lm_head_argmax(xi, w)[0].cpu().numpy().reshape(B, D + 1)
        d = rng.integers(0, V, (B, D)).astype(np.int32)
        for b in range(B):
            d[b, :b % (D + 1)] = tok[b, :b % (D + 1)]
        drafts.append(d)

    def load(i):
        x.copy_(torch.from_numpy(xs[i].view(np.int16)).view(torch.bfloat16).view(B, D + 1, H))
        dr.copy_(torch.from_numpy(drafts[i]))

    load(0)
    launch(torch.cuda.current_stream(gpu).cuda_stream)        # eager warmup
    torch.cuda.synchronize(gpu)
    graph = torch.cuda.CUDAGraph()
    cap = torch.cuda.Stream(gpu)
    cap.wait_stream(torch.cuda.current_stream(gpu))
    with torch.cuda.graph(graph, stream=cap):
        launch(cap.cuda_stream)
    torch.cuda.synchronize(gpu)
    for i in range(REPLAYS):
        load(i)
        acc.fill_(-7)
        em.fill_(-7)
        torch.cuda.synchronize(gpu)
        graph.replay()
        torch.cuda.synchronize(gpu)
        got_a, got_e = acc.cpu().numpy().copy(), em.cpu().numpy().copy()
        ea, ee = llima_amd.lm_head_verify_greedy(x, w, dr)
        assert (got_a == ea.cpu().numpy()).all() and (got_e == ee.cpu().numpy()).all(), i
        assert (got_a >= np.arange(B) % (D + 1)).all(), i      # the planted prefixes accepted
