"""GPU parity: every entry point of libllima_sampler.so (through the C ABI via
llima_amd) against the CPU oracle on identical inputs and uniforms.  Token ids,
index sets, kept-set bitmasks, accepted lengths are compared bit for bit; the
sampled token's probability is compared bit for bit as well (both sides compute
W/Z from the same integers)."""
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


def _np(t):
    return t.cpu().numpy()


# ----------------------------------------------------------------- argmax
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("B,V", [(1, 1), (3, 7), (1, 151936), (8, 128256), (5, 5003),
                                 (16, 262144), (64, 4096)])
def test_argmax_parity(gpu, oracle, dtype, B, V):
    import llima_amd
    _say("argmax", dtype, B, V)
    rng = np.random.default_rng(B * 1000 + V)
    x = rng.integers(-50, 51, size=(B, V)).astype(np.float32) * np.float32(0.25)  # ties
    if dtype == "bf16":
        x = wl.f32_to_bf16_bits(x)
    for mode, mname in [(0, "split_first"), (1, "neg_inf"), (2, "quarters"), (3, "lowest")]:
        ids, vals = llima_amd.argmax(_t(x, gpu), mode=mname)
        eids, evals = oracle.argmax(x, mode=mode)
        assert (_np(ids) == eids).all(), mname
        assert (_np(vals).view(np.uint32) == evals.view(np.uint32)).all()


def test_argmax_nan_split_rules(gpu, oracle):
    import llima_amd
    _say("argmax nan/splits")
    rng = np.random.default_rng(9)
    V = 20000
    x = rng.normal(0, 1, (12, V)).astype(np.float32)
    x[0, 0] = np.nan                        # NaN at index 0
    x[1, 5000] = np.nan; x[1, 4999] = 50    # NaN at a 5000-split start
    x[2, :] = -np.inf                       # all -inf
    x[3, :] = np.nan                        # all NaN
    x[4, V // 4] = np.nan; x[4, V // 4 + 3] = 99   # hidden quarter
    x[5, 7] = np.inf; x[5, 9] = np.inf
    x[6, 3] = np.nan; x[6, 10] = 1e30
    x[7, 10000] = np.nan; x[7, 12000] = 77         # NaN at the start of split 2
    x[8, :] = -1; x[8, 10] = -0.0; x[8, 20] = 0.0  # maximum -0 first: its sign is reported
    x[9, :] = -1; x[9, 10] = 0.0; x[9, 11] = -0.0
    for split in [0, 5000, 4096, 1]:
        for mode, mname in [(0, "split_first"), (1, "neg_inf"), (2, "quarters")]:
            ids, vals = llima_amd.argmax(_t(x, gpu), split_dim=split, mode=mname)
            eids, evals = oracle.argmax(x, split_dim=split, mode=mode)
            assert (_np(ids) == eids).all(), (split, mname, _np(ids), eids)
            g, e = _np(vals), evals
            assert ((g.view(np.uint32) == e.view(np.uint32)) | (np.isnan(g) & np.isnan(e))).all(), \
                (split, mname)


def test_argmax_strided_rows(gpu, oracle):
    import llima_amd
    _say("argmax strided")
    rng = np.random.default_rng(4)
    x = rng.normal(0, 1, (6, 1001)).astype(np.float32)
    xt = _t(x, gpu)[:, 3:1000]                 # row stride 1001, unaligned start
    ids, _ = llima_amd.argmax(xt)
    assert (_np(ids) == oracle.argmax(np.ascontiguousarray(x[:, 3:1000]))[0]).all()


# ----------------------------------------------------------------- sampler
def _cfg_obj(d, rows=None):
    import llima_amd
    return llima_amd.SamplerConfig(**d)


def _sample_both(gpu, oracle, logits, u, cfgd, history=None, hist_len=None, mask=None,
                 cfg_rows=None, want_keep=True):
    import llima_amd
    from oracle.oracle import SamplerConfig as OC
    if cfg_rows is None:
        gcfg = llima_amd.SamplerConfig(**cfgd)
        ocfg = OC(**cfgd)
    else:
        import torch
        gcfg = llima_amd.SamplerConfig(**{k: (torch.tensor(v) if isinstance(v, list) else v)
                                          for k, v in cfg_rows.items()})
        B = logits.shape[0]
        ocfg = [OC(**{k: (v[b] if isinstance(v, list) else v) for k, v in cfg_rows.items()
                      if k != "top_k_every_row"})     # a launch hint, not a setting
                for b in range(B)]
    # without the kept-set output the batch may take other paths (rows split
    # over several finish workgroups need none)
    out = llima_amd.sample(_t(logits, gpu), _t(u, gpu), gcfg, history=_t(history, gpu),
                           history_len=_t(hist_len, gpu), bitmask=_t(mask, gpu),
                           return_keep=want_keep)
    eout = oracle.sample(logits, u, ocfg, history=history, hist_len=hist_len, bitmask=mask,
                         want_keep=want_keep)
    eids, eprobs = eout[0], eout[1]
    gi, gp = _np(out[0]), _np(out[1])
    bad = np.flatnonzero(gi != eids)
    assert bad.size == 0, f"ids differ at rows {bad[:8]}: gpu {gi[bad[:8]]} oracle {eids[bad[:8]]}"
    assert (gp.view(np.uint32) == eprobs.view(np.uint32)).all()
    if want_keep:
        gk, ekeep = _np(out[2]).view(np.uint32), eout[2]
        assert (gk == ekeep).all(), np.flatnonzero((gk != ekeep).any(axis=1))[:8]
    return gi


WORKLOADS_SMALL = [
    ("single_row", dict()),
    ("batched_penalties", dict(B=16, V=128256, H=2048)),
    ("constrained", dict(B=8)),
    ("large_vocab_bf16", dict(B=16, V=262144, H=512)),
]


@pytest.mark.parametrize("name,kw", WORKLOADS_SMALL)
def test_sample_workloads(gpu, oracle, name, kw):
    _say("sample", name, kw)
    w = wl.WORKLOADS[name](**kw)
    _sample_both(gpu, oracle, w["logits"], w["uniforms"], w["cfg"], history=w["history"],
                 mask=w["bitmask"])


@pytest.mark.parametrize("name", ["batched_penalties", "constrained", "large_vocab_bf16", "top_p_only"])
def test_sample_workloads_full_size(gpu, oracle, name):
    _say("sample full", name)
    w = wl.WORKLOADS[name]()
    _sample_both(gpu, oracle, w["logits"], w["uniforms"], w["cfg"], history=w["history"],
                 mask=w["bitmask"])


def test_sample_greedy_variants_equal_argmax(gpu, oracle):
    """Greedy sampling without penalties or mask is the reference argmax."""
    import llima_amd
    _say("sample greedy == argmax")
    for name, kw in [("single_row", {}), ("large_vocab_bf16", dict(B=32, H=8))]:
        w = wl.WORKLOADS[name](**kw)
        ids, _ = llima_amd.sample(_t(w["logits"], gpu), _t(w["uniforms"], gpu),
                                  llima_amd.SamplerConfig(greedy=True))
        am, _ = llima_amd.argmax(_t(w["logits"], gpu))
        assert (_np(ids) == _np(am)).all()
        assert (_np(am) == oracle.argmax(w["logits"])[0]).all()


CONFIGS = [
    dict(temperature=0.7, top_k=40, top_p=0.9, repetition_penalty=1.1),
    dict(temperature=1.3, top_k=1),
    dict(temperature=0.5, top_k=257),                      # beyond the fast path's k
    dict(temperature=1.0, top_p=0.8),                      # no top-k, no mask: full-row path
    dict(temperature=1.0, top_p=0.0),
    dict(temperature=0.9, min_p=1.0, top_k=20),
    dict(temperature=1e-30, top_k=10),                     # overflowing quotients
    dict(temperature=2.0, top_k=100, top_p=0.99, min_p=0.01, presence_penalty=-0.7,
         frequency_penalty=0.2, repetition_penalty=0.9),
    dict(greedy=True, repetition_penalty=1.5, presence_penalty=1.0),
    dict(temperature=1.0),                                  # plain softmax sampling
]


@pytest.mark.parametrize("ci", range(len(CONFIGS)))
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_sample_configs(gpu, oracle, ci, dtype):
    cfgd = CONFIGS[ci]
    _say("sample config", ci, dtype, cfgd)
    rng = np.random.default_rng(ci * 7 + (dtype == "bf16"))
    B, V = 12, 50000
    x = rng.normal(0, 3, (B, V)).astype(np.float32)
    x[0] = np.round(x[0])                                  # heavy ties
    x[1, 100:200] = np.nan
    x[2, 5] = np.inf
    x[3, :] = -np.inf
    x[3, 77] = 1.0
    x[4, :] = 0.0                                          # all equal
    if dtype == "bf16":
        x = wl.f32_to_bf16_bits(x)
    hist = rng.integers(-5, V + 5, size=(B, 300)).astype(np.int32)
    hl = rng.integers(0, 301, size=B).astype(np.int32)
    u = rng.random(B).astype(np.float32)
    u[0] = 0.0
    u[1] = np.float32(1.0) - np.float32(2**-24)
    _sample_both(gpu, oracle, x, u, cfgd, history=hist, hist_len=hl)


def _random_cfg(rng):
    d = {}
    if rng.random() < 0.1:
        d["greedy"] = True
    d["temperature"] = float(rng.choice([1.0, 0.7, 1.3, 0.05, 3.0]))
    if rng.random() < 0.75:
        d["top_k"] = int(rng.choice([1, 5, 20, 40, 50, 64, 65, 100, 300]))
    if rng.random() < 0.6:
        d["top_p"] = float(rng.choice([0.5, 0.9, 0.95, 0.99]))
    if rng.random() < 0.3:
        d["min_p"] = float(rng.choice([0.01, 0.05, 0.2]))
    if rng.random() < 0.5:
        d["repetition_penalty"] = float(rng.choice([1.05, 1.15, 0.9]))
        d["presence_penalty"] = float(rng.choice([0.0, 0.5, -0.3]))
        d["frequency_penalty"] = float(rng.choice([0.0, 0.3]))
    return d


@pytest.mark.parametrize("seed", range(64))
def test_sample_random_configs(gpu, oracle, seed):
    """Seeded random shapes, dtypes, configs, histories and masks."""
    rng = np.random.default_rng(5000 + seed)
    B = int(rng.integers(1, 7))
    V = int(rng.choice([37, 1000, 4096, 8192, 30001, 65536, 128256]))
    dtype = "bf16" if rng.random() < 0.5 else "f32"
    sigma = float(rng.choice([1.0, 3.0, 5.0]))
    x = rng.normal(0, sigma, (B, V)).astype(np.float32)
    if rng.random() < 0.3:
        x = np.round(x * 2) / 2                              # ties
    if dtype == "bf16":
        x = wl.f32_to_bf16_bits(x)
    hist = hl = None
    if rng.random() < 0.6:
        H = int(rng.choice([16, 300, 2048]))
        hist = rng.integers(-3, V + 3, size=(B, H)).astype(np.int32)
        if rng.random() < 0.5:
            hist[:, : H // 4] = rng.integers(0, min(V, 64), size=(B, H // 4))   # hot ids
        hl = rng.integers(0, H + 1, size=B).astype(np.int32)
    mask = None
    if rng.random() < 0.3:
        nw = (V + 31) // 32
        mask = (rng.random((B, nw)) < rng.choice([0.02, 0.5, 0.98])).astype(np.uint32) * np.uint32(0xFFFFFFFF)
        mask ^= rng.integers(0, 2**32, size=(B, nw), dtype=np.uint64).astype(np.uint32) & np.uint32(0x0F0F0F0F)
    u = rng.random(B).astype(np.float32)
    cfgd = _random_cfg(rng)
    _say("sample random", seed, B, V, dtype, cfgd, "hist" if hist is not None else "", "mask" if mask is not None else "")
    _sample_both(gpu, oracle, x, u, cfgd, history=hist, hist_len=hl, mask=mask)


def _sparse_mask(rng, B, V, frac):
    nw = (V + 31) // 32
    keep = rng.random((B, V)) < frac
    bits = np.zeros((B, nw * 32), np.uint32)
    bits[:, :V] = keep
    return (bits.reshape(B, nw, 32) << np.arange(32, dtype=np.uint32)).sum(axis=2, dtype=np.uint64).astype(np.uint32)


@pytest.mark.parametrize("kind", ["normal", "integers", "fine_steps", "inf", "hot_history"])
def test_sample_gather_path_top_p(gpu, oracle, kind):
    """Rows whose candidates do not fit the finish's first round (a grammar mask
    with a few percent of the ids allowed, no top-k): the gather path, where
    the top-p boundary comes from value bins of 1/8 nat and a pairwise pass in
    one bin.  Integer-valued rows and rows in 1/64 steps put more than 64 tied
    or close values in the boundary bin (the radix rounds take over); an
    infinite value takes the radix rounds too."""
    _say("sample gather path", kind)
    rng = np.random.default_rng(["normal", "integers", "fine_steps", "inf", "hot_history"].index(kind) + 90)
    B, V = 8, 151936
    x = rng.normal(0, 3, (B, V)).astype(np.float32)
    if kind == "integers":
        x = np.round(x)
    elif kind == "fine_steps":
        x = np.round(rng.normal(0, 0.4, (B, V)) * 64).astype(np.float32) / 64
    elif kind == "inf":
        x[1, 1000:1010] = np.inf
    mask = _sparse_mask(rng, B, V, 0.02 if kind != "fine_steps" else 0.005)
    if kind == "inf":
        mask[1, 1000 >> 5] |= np.uint32(0xFFFFFFFF)          # the +inf ids are allowed
    hist = hl = None
    if kind == "hot_history":
        allowed = np.flatnonzero((mask[0, np.arange(V) >> 5] >> (np.arange(V) & 31).astype(np.uint32)) & 1)
        hist = np.tile(rng.choice(allowed, 300).astype(np.int32), (B, 1))
        hl = np.full(B, 300, np.int32)
    u = rng.random(B).astype(np.float32)
    for cfgd in [dict(temperature=1.0, top_p=0.9), dict(temperature=0.5, top_p=0.5, min_p=0.05),
                 dict(temperature=2.0, top_p=0.999),
                 dict(temperature=1.0, top_p=0.95, presence_penalty=-0.3, repetition_penalty=1.2)]:
        for dt in ("f32", "bf16"):
            xx = wl.f32_to_bf16_bits(x) if dt == "bf16" else x
            _sample_both(gpu, oracle, xx, u, cfgd, history=hist, hist_len=hl, mask=mask)


@pytest.mark.parametrize("V", [151936, 100000])
def test_sample_wide_dense_chunk(gpu, oracle, V):
    """A grammar mask allowing 1 % of the ids, plus 300 or 350 consecutive
    allowed ids inside one chunk (fewer than a region holds): that chunk's
    candidates exceed what the wide finish's first round of loads brings (127
    per chunk at 38 fp32 chunks, 255 at 25 fp32 or 19 bf16 chunks), so the
    rest come from its second round.  Each row has its dense block elsewhere."""
    _say("sample wide dense chunk", V)
    rng = np.random.default_rng(V + 7)
    B = 6
    x = rng.normal(0, 3, (B, V)).astype(np.float32)
    mask = _sparse_mask(rng, B, V, 0.01)
    nchunks = V // 8192
    for b in range(B):
        c0 = ((3 * b + 1) % nchunks) * 8192 + 100            # inside one fp32 and one bf16 chunk
        ids = np.arange(c0, c0 + (300 if b % 2 == 0 else 350))
        np.bitwise_or.at(mask[b], ids >> 5, (np.uint32(1) << (ids & 31).astype(np.uint32)))
    u = rng.random(B).astype(np.float32)
    for cfgd in [dict(temperature=1.0, top_p=0.9), dict(temperature=0.7, top_p=0.95, min_p=0.02)]:
        for dt in ("f32", "bf16"):
            xx = wl.f32_to_bf16_bits(x) if dt == "bf16" else x
            _sample_both(gpu, oracle, xx, u, cfgd, mask=mask)


DENSE_CONFIGS = [
    dict(temperature=1.0, top_p=0.9),
    dict(temperature=0.7, top_p=0.5, min_p=0.05),
    dict(temperature=1.5),                                  # plain sampling: every finite value kept
    dict(temperature=1.0, min_p=0.1),
    dict(temperature=1.0, top_p=0.95, repetition_penalty=1.2, presence_penalty=-0.4,
         frequency_penalty=0.1),
    dict(temperature=1.0, top_p=0.0),
    dict(temperature=3.0, top_p=0.999),
]
DENSE_KINDS = ["normal4", "normal1", "flat", "integers", "fine_steps", "specials", "small"]


def _dense_rows(kind, rng):
    if kind == "normal4":
        return rng.normal(0, 4, (4, 128256)).astype(np.float32)
    if kind == "normal1":                                    # V % 4 != 0: one value per load
        return rng.normal(0, 1, (4, 70001)).astype(np.float32)
    if kind == "flat":                                       # > 4096 values in the boundary bin
        return rng.normal(0, 0.05, (3, 50000)).astype(np.float32)
    if kind == "integers":
        return np.round(rng.normal(0, 3, (4, 128256))).astype(np.float32)
    if kind == "fine_steps":
        return (np.round(rng.normal(0, 0.4, (4, 128256)) * 64) / 64).astype(np.float32)
    if kind == "specials":
        x = rng.normal(0, 2, (6, 4099)).astype(np.float32)
        x[0, 10:300] = np.nan
        x[1, 4000:4010] = np.inf                             # infinite maximum
        x[2, :] = -np.inf                                    # no finite value: -1
        x[3, :] = -np.inf
        x[3, 4098] = 0.5                                     # one finite value, in the last chunk
        x[4, ::2] = -np.inf
        x[5, 7] = np.float32(3e38)
        x[5, 8] = np.float32(-3e38)
        return x
    return rng.normal(0, 2, (3, 37)).astype(np.float32)      # small: one partial chunk


@pytest.mark.parametrize("kind", DENSE_KINDS)
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_sample_dense_path(gpu, oracle, kind, dtype):
    """Rows without top-k or mask take the dense path: per-chunk statistics,
    chunk histograms of value bins (1/16 nat) merged by the row's last
    workgroup, the boundary bin's members ranked, the draw's chunk scanned.
    Flat rows put more than 4096 values into the boundary bin (the full-row
    path finishes them); integer rows and rows in 1/64 steps put many tied or
    close values there; an infinite maximum, NaN runs, rows without finite
    values and a single finite value in the last chunk are the edge cases."""
    _say("sample dense", kind, dtype)
    rng = np.random.default_rng(DENSE_KINDS.index(kind) * 2 + (dtype == "bf16") + 300)
    x = _dense_rows(kind, rng)
    B, V = x.shape
    if dtype == "bf16":
        x = wl.f32_to_bf16_bits(x)
    hist = rng.integers(-3, V + 3, size=(B, 500)).astype(np.int32)
    hist[:, :100] = rng.integers(0, min(V, 50), size=(B, 100))  # hot ids near the top
    hl = rng.integers(0, 501, size=B).astype(np.int32)
    u = rng.random(B).astype(np.float32)
    u[0] = 0.0
    u[-1] = np.float32(1.0) - np.float32(2**-24)
    for cfgd in DENSE_CONFIGS:
        _sample_both(gpu, oracle, x, u, cfgd, history=hist, hist_len=hl)


@pytest.mark.parametrize("seed", range(32))
def test_sample_dense_random(gpu, oracle, seed):
    """Seeded random rows and configurations without top-k or mask (the dense
    path): shapes with a ragged last chunk, both dtypes, narrow to wide value
    spreads, ties, histories, broadcast or per-row temperature / top-p / min-p
    (a zero temperature makes a greedy row)."""
    rng = np.random.default_rng(7000 + seed)
    B = int(rng.integers(1, 9))
    V = int(rng.choice([37, 4096, 4097, 30001, 128256, 151936]))
    dtype = "bf16" if rng.random() < 0.4 else "f32"
    sigma = float(rng.choice([0.3, 1.0, 3.0, 8.0]))
    x = rng.normal(0, sigma, (B, V)).astype(np.float32)
    if rng.random() < 0.25:
        x = np.round(x * 4) / 4
    if dtype == "bf16":
        x = wl.f32_to_bf16_bits(x)
    hist = hl = None
    if rng.random() < 0.5:
        H = int(rng.choice([8, 256, 2048]))
        hist = rng.integers(-2, V + 2, size=(B, H)).astype(np.int32)
        hl = rng.integers(0, H + 1, size=B).astype(np.int32)
    u = rng.random(B).astype(np.float32)
    base = dict(temperature=float(rng.choice([0.3, 0.7, 1.0, 1.6])),
                top_p=float(rng.choice([1.0, 0.5, 0.9, 0.99, 0.999])),
                min_p=float(rng.choice([0.0, 0.0, 0.01, 0.2])))
    if hist is not None and rng.random() < 0.7:
        base.update(repetition_penalty=float(rng.choice([1.1, 0.9])),
                    presence_penalty=float(rng.choice([0.0, 0.4, -0.2])),
                    frequency_penalty=float(rng.choice([0.0, 0.25])))
    _say("sample dense random", seed, B, V, dtype, sigma, base)
    if rng.random() < 0.3:
        rows = {k: v for k, v in base.items() if k not in ("temperature", "top_p")}
        rows["temperature"] = [float(v) for v in rng.choice([0.0, 0.5, 1.0, 2.0], size=B)]
        rows["top_p"] = [float(v) for v in rng.choice([1.0, 0.6, 0.95], size=B)]
        _sample_both(gpu, oracle, x, u, None, history=hist, hist_len=hl, cfg_rows=rows)
    else:
        _sample_both(gpu, oracle, x, u, base, history=hist, hist_len=hl)


def test_sample_dense_rows_config_and_strides(gpu, oracle):
    """The dense path with per-row temperatures and top-p (a zero temperature
    makes a greedy row) and on rows that start unaligned (a row stride of
    V + 3 and an offset of 3 values: one value per load)."""
    import llima_amd
    import torch
    from oracle.oracle import SamplerConfig as OC
    _say("sample dense per-row / strided")
    rng = np.random.default_rng(77)
    B, V = 8, 20000
    x = rng.normal(0, 3, (B, V)).astype(np.float32)
    u = rng.random(B).astype(np.float32)
    rows = dict(temperature=[1.0, 0.0, 0.7, 2.0, 1.0, 0.0, 0.3, 1.1],
                top_p=[0.9, 0.9, 1.0, 0.5, 0.99, 1.0, 0.0, 0.8],
                min_p=[0.0, 0.0, 0.05, 0.0, 0.2, 0.0, 0.0, 0.01])
    _sample_both(gpu, oracle, x, u, None, cfg_rows=rows)
    xs = np.zeros((B, V + 3), np.float32)
    xs[:, 3:] = x
    xt = _t(xs, gpu)[:, 3:]
    for cfgd in [dict(temperature=1.0, top_p=0.9), dict(temperature=0.8, min_p=0.05)]:
        ids, probs, keep = llima_amd.sample(xt, _t(u, gpu), llima_amd.SamplerConfig(**cfgd),
                                            return_keep=True)
        eids, eprobs, ekeep = oracle.sample(x, u, OC(**cfgd), want_keep=True)
        assert (_np(ids) == eids).all()
        assert (_np(probs).view(np.uint32) == eprobs.view(np.uint32)).all()
        assert (_np(keep).view(np.uint32) == ekeep).all()


FULL_ROW_CONFIGS = [
    dict(temperature=1.0, top_p=0.9),
    dict(temperature=0.7, top_p=0.6, min_p=0.02, repetition_penalty=1.2, presence_penalty=0.3),
    dict(temperature=1.3, min_p=0.05),
    dict(temperature=1.0),
    dict(temperature=1.0, top_p=0.0),
]


@pytest.mark.parametrize("density", [0.5, 0.98])
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_sample_full_row_path(gpu, oracle, density, dtype):
    """Rows whose grammar mask admits most ids and that have no top-k overflow
    the candidate regions and take the full-row path: value bins for top-p
    (the boundary bin's members ranked) and a one-segment scan for the draw;
    flat rows put more than 1024 values in the boundary bin and take the radix
    rounds instead; a row without an allowed id gives -1."""
    _say("sample full-row path", density, dtype)
    rng = np.random.default_rng(int(density * 100) + (dtype == "bf16") + 400)
    B, V = 6, 70001
    x = rng.normal(0, 3, (B, V)).astype(np.float32)
    x[1] = rng.normal(0, 0.02, V).astype(np.float32)        # flat: the radix rounds
    x[2] = np.round(x[2])                                    # ties
    x[3, 500:520] = np.inf
    if dtype == "bf16":
        x = wl.f32_to_bf16_bits(x)
    mask = _sparse_mask(rng, B, V, density)
    mask[4] = 0                                              # nothing allowed
    mask[3, 500 >> 5] |= np.uint32(0xFFFFFFFF)
    hist = rng.integers(0, V, size=(B, 400)).astype(np.int32)
    u = rng.random(B).astype(np.float32)
    for cfgd in FULL_ROW_CONFIGS:
        gi = _sample_both(gpu, oracle, x, u, cfgd, history=hist, mask=mask)
        assert gi[4] == -1


def test_sample_masks_and_edges(gpu, oracle):
    _say("sample masks/edges")
    rng = np.random.default_rng(21)
    for B, V in [(1, 1), (3, 33), (8, 1000), (9, 70001)]:
        x = rng.normal(0, 2, (B, V)).astype(np.float32)
        mask = rng.integers(0, 2**32, size=(B, (V + 31) // 32), dtype=np.uint64).astype(np.uint32)
        mask[0] = 0                                         # fully masked row -> -1
        u = rng.random(B).astype(np.float32)
        for cfgd in [dict(temperature=1.0, top_p=0.9), dict(temperature=0.8, top_k=5),
                     dict(greedy=True)]:
            gi = _sample_both(gpu, oracle, x, u, cfgd, mask=mask)
            assert gi[0] == -1


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_sample_sparse_waves(gpu, oracle, dtype):
    """Sweep waves with few lanes above the chunk bound take the sparse path
    (at most 12 lanes for fp32, 8 for bf16); with more candidates than a wave
    stages (those lanes' values all kept) it writes them to the region directly."""
    _say("sample sparse sweep waves", dtype)
    rng = np.random.default_rng(33)
    B, V = 4, 16384
    epl = 4 if dtype == "f32" else 8                              # values per 16-byte load
    ws = 1024 if dtype == "f32" else 2048                         # ids per wave slice
    x = np.full((B, V), -100.0, np.float32)
    lanes = 12 if dtype == "f32" else 8
    ids = np.array([j * 64 * epl + l * epl + e for j in range(4) for l in range(lanes)
                    for e in range(epl)])
    x[:, ids] = rng.normal(0, 1, (B, ids.size)).astype(np.float32)
    x[1, ids + ws] = rng.normal(0, 1, ids.size)                   # the next wave's slice too
    x[2, ids[:40]] = rng.normal(5, 1, 40)                         # a few lanes dominate
    if dtype == "bf16":
        x = wl.f32_to_bf16_bits(x)
    u = rng.random(B).astype(np.float32)
    for cfgd in [dict(temperature=1.0, top_p=0.9), dict(temperature=1.0, min_p=0.01),
                 dict(temperature=0.7, top_k=20, top_p=0.95), dict(temperature=1.0, top_k=3)]:
        _sample_both(gpu, oracle, x, u, cfgd)


def test_sample_per_row_configs(gpu, oracle):
    _say("sample per-row configs")
    rng = np.random.default_rng(5)
    B, V = 8, 30000
    x = rng.normal(0, 3, (B, V)).astype(np.float32)
    u = rng.random(B).astype(np.float32)
    rows = dict(temperature=[0.5, 1.0, 0.0, 2.0, 0.7, 1.0, 0.3, 1.5],
                top_k=[10, 0, 5, 300, 50, 1, 64, 0],
                top_p=[0.9, 0.5, 1.0, 0.95, 1.0, 0.9, 0.8, 1.0],
                min_p=[0.0, 0.1, 0.0, 0.0, 0.05, 0.0, 0.2, 0.0],
                repetition_penalty=1.2)
    hist = rng.integers(0, V, size=(B, 64)).astype(np.int32)
    _sample_both(gpu, oracle, x, u, None, history=hist, cfg_rows=rows)


def test_sample_per_row_lazy_and_eager_penalties(gpu, oracle):
    """Per-row settings decide per row where the penalties are applied: rows
    with top-k whose penalties only lower values take them in the finish, the
    others (a repetition penalty below 1, negative presence or frequency, no
    top-k, greedy) in the sweep.  One batch holds every kind, over the lazy
    hit patterns of the test below (history ids among the survivors, hot ids
    repeated), fp32 and bf16."""
    _say("sample per-row lazy and eager penalties")
    rng = np.random.default_rng(78)
    B, V, H = 8, 50000, 1500
    x = (rng.standard_normal((B, V), dtype=np.float32) * np.float32(4.0)).astype(np.float32)
    hist = rng.integers(0, V, size=(B, H)).astype(np.int32)
    for b in range(B):                                  # the row's top values, repeated
        top = np.argsort(-x[b])[:40]
        hist[b, :400] = np.resize(top, 400)
    u = rng.random(B).astype(np.float32)
    rows = dict(temperature=[0.8, 0.8, 1.0, 0.0, 0.7, 1.2, 0.8, 0.9],
                top_k=[50, 50, 40, 50, 0, 30, 64, 50],
                top_p=[0.95, 0.9, 1.0, 1.0, 0.9, 0.8, 0.95, 1.0],
                min_p=[0.05, 0.0, 0.02, 0.0, 0.0, 0.1, 0.05, 0.0],
                repetition_penalty=[1.15, 0.9, 1.0, 1.2, 1.3, 1.05, 1.15, 2.0],
                presence_penalty=[0.5, 0.5, -0.4, 0.0, 0.2, 0.0, 0.5, 1.0],
                frequency_penalty=[0.3, 0.3, 0.1, 0.0, 0.1, -0.2, 0.3, 0.5])
    _sample_both(gpu, oracle, x, u, None, history=hist, cfg_rows=rows)
    _sample_both(gpu, oracle, wl.f32_to_bf16_bits(x), u, None, history=hist, cfg_rows=rows)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_sample_split_rows(gpu, oracle, dtype):
    """Rows without top-k whose candidates overflow the sweep's regions, in a
    batch with per-row top-k: the finish splits each over ceil(S / 8)
    workgroups (bins per chunk, the last to arrive finishes the row).  Every
    kind of such row: top-p alone, min-p alone, both (either boundary the
    higher), plain temperature, penalties of either sign, T != 1, a flat row
    whose boundary bin holds more values than the split finish ranks (the
    full-row path), an all -inf row; beside top-k rows and a greedy row."""
    _say("sample split rows", dtype)
    rng = np.random.default_rng(91)
    B, V, H = 12, 128256, 700
    x = (rng.standard_normal((B, V), dtype=np.float32) * np.float32(4.0)).astype(np.float32)
    x[6] = np.float32(0.5) * np.round(rng.standard_normal(V).astype(np.float32) * 4)   # flat: few values
    x[7] = -np.inf
    x[8, :300] = np.nan
    hist = rng.integers(0, V, size=(B, H)).astype(np.int32)
    for b in range(B):
        hist[b, :200] = np.resize(np.argsort(-np.nan_to_num(x[b], nan=-1e30))[:50], 200)
    u = rng.random(B).astype(np.float32)
    rows = dict(temperature=[1.0, 0.8, 1.3, 1.0, 0.7, 1.0, 1.0, 1.0, 0.9, 1.0, 0.0, 1.0],
                top_k=[0, 0, 0, 0, 0, 0, 0, 0, 0, 50, 0, 40],
                top_p=[0.9, 1.0, 0.95, 0.5, 1.0, 0.9, 0.9, 0.9, 0.99, 0.95, 1.0, 1.0],
                min_p=[0.0, 0.1, 0.02, 0.3, 0.0, 0.0, 0.0, 0.0, 0.0, 0.05, 0.0, 0.0],
                repetition_penalty=[1.0, 1.0, 1.2, 1.0, 1.0, 0.8, 1.0, 1.0, 1.1, 1.15, 1.0, 1.0],
                presence_penalty=[0.0, 0.0, 0.5, 0.0, 0.0, -0.3, 0.0, 0.0, 0.2, 0.5, 0.0, 0.0],
                frequency_penalty=[0.0, 0.0, 0.3, 0.0, 0.0, 0.1, 0.0, 0.0, 0.0, 0.3, 0.0, 0.0])
    xx = x if dtype == "f32" else wl.f32_to_bf16_bits(x)
    _sample_both(gpu, oracle, xx, u, None, history=hist, cfg_rows=rows, want_keep=False)
    # the same rows again with other uniforms (other draw chunks)
    _sample_both(gpu, oracle, xx, rng.random(B).astype(np.float32), None, history=hist,
                 cfg_rows=rows, want_keep=False)
    # a wrong statement that every row has top-k: the rows without take the
    # full-row path, and the tokens stay the same
    _sample_both(gpu, oracle, xx, u, None, history=hist, cfg_rows=dict(rows, top_k_every_row=True),
                 want_keep=False)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_sample_split_masked_rows(gpu, oracle, dtype):
    """A grammar mask that allows about half of each row, top-p without
    top-k (the wide finish leaves these rows, whose regions overflow, to the
    split finish); also min-p, and a mask allowing 3 of every 4 ids."""
    _say("sample split masked rows", dtype)
    w = wl.constrained_half(B=8)
    x = w["logits"] if dtype == "f32" else wl.f32_to_bf16_bits(w["logits"])
    _sample_both(gpu, oracle, x, w["uniforms"], w["cfg"], mask=w["bitmask"], want_keep=False)
    _sample_both(gpu, oracle, x, w["uniforms"], dict(temperature=0.8, top_p=0.95, min_p=0.05),
                 mask=w["bitmask"], want_keep=False)
    m3 = w["bitmask"] | np.uint32(0x77777777)
    _sample_both(gpu, oracle, x, w["uniforms"], dict(temperature=1.0, min_p=0.2), mask=m3,
                 want_keep=False)


def test_sample_lazy_penalty_hits(gpu, oracle):
    """Penalties applied to the finish's survivors only (repetition >= 1,
    presence and frequency >= 0, broadcast top-k): history ids that are
    survivors, hot ids repeated hundreds of times, and survivors that share one
    bucket of the finish's 4-slot id hash (1024 buckets, Fibonacci hashing)."""
    _say("sample lazy penalty hits")
    rng = np.random.default_rng(77)
    B, V, H = 6, 128256, 2048
    x = (rng.standard_normal((B, V), dtype=np.float32) * np.float32(4.0)).astype(np.float32)
    ids = np.arange(V, dtype=np.uint64)
    bucket = (((ids * 2654435761) & 0xFFFFFFFF) >> 22).astype(np.int64)
    hist = rng.integers(0, V, size=(B, H)).astype(np.int32)
    # row 0: 14 survivors in one bucket (chains into the next buckets), each in the history
    same = np.flatnonzero(bucket == bucket[12345])[:14]
    x[0, same] = np.float32(18.0) + np.arange(14, dtype=np.float32) * np.float32(0.25)
    hist[0, :14 * 20] = np.repeat(same, 20)
    # row 1: the history is the row's 60 largest values, repeated
    top = np.argsort(-x[1])[:60]
    hist[1] = np.resize(top, H)
    # row 2: the row maximum repeated 2000 times
    hist[2, :2000] = int(np.argmax(x[2]))
    # row 3: two buckets' worth of survivors, counts 1..n
    b2 = np.flatnonzero(bucket == bucket[999])[:9]
    x[3, b2] = np.float32(17.0) + np.arange(9, dtype=np.float32) * np.float32(0.1)
    hist[3, :45] = np.concatenate([np.full(i + 1, v) for i, v in enumerate(b2)])
    # row 4: ids out of range and a short history length
    hist[4, :100] = -3
    hist[4, 100:200] = V + 7
    hl = np.full(B, H, dtype=np.int32)
    hl[4] = 700
    u = rng.random(B).astype(np.float32)
    cfg = dict(temperature=0.8, top_k=50, top_p=0.95, min_p=0.05, repetition_penalty=1.15,
               presence_penalty=0.5, frequency_penalty=0.3)
    _sample_both(gpu, oracle, x, u, cfg, history=hist, hist_len=hl)
    cfg2 = dict(temperature=1.1, top_k=20, repetition_penalty=3.0, frequency_penalty=2.0)
    _sample_both(gpu, oracle, x, u, cfg2, history=hist, hist_len=hl)


def test_sample_repeatable_and_workspace_reset(gpu, oracle):
    """Back-to-back calls sharing one workspace give identical results."""
    import llima_amd
    _say("sample repeat")
    w = wl.batched_penalties(B=24, V=40000, H=256)
    cfg = llima_amd.SamplerConfig(**w["cfg"])
    args = (_t(w["logits"], gpu), _t(w["uniforms"], gpu), cfg)
    first = _np(llima_amd.sample(*args, history=_t(w["history"], gpu))[0])
    for _ in range(5):
        again = _np(llima_amd.sample(*args, history=_t(w["history"], gpu))[0])
        assert (again == first).all()


# ----------------------------------------------------------------- verification
def test_verify_greedy_parity(gpu, oracle):
    import llima_amd
    _say("verify_greedy")
    rng = np.random.default_rng(8)
    for B, D, V, dt in [(16, 7, 128256, "f32"), (4, 6, 262144, "bf16"), (3, 0, 100, "f32")]:
        tgt = rng.integers(-20, 21, size=(B, D + 1, V)).astype(np.float32)
        am = tgt.argmax(axis=-1)
        drafts = np.where(rng.random((B, D)) < 0.8, am[:, :D], rng.integers(0, V, (B, D)))
        drafts = drafts.astype(np.int32)
        if dt == "bf16":
            tgt = wl.f32_to_bf16_bits(tgt)
        acc, em = llima_amd.verify_greedy(_t(tgt, gpu), _t(drafts, gpu))
        eacc, eem = oracle.verify_greedy(tgt, drafts)
        assert (_np(acc) == eacc).all() and (_np(em) == eem).all()


def test_verify_greedy_reference_vectors(gpu, oracle):
    import json, os
    import llima_amd
    _say("verify_greedy golden")
    with open(os.path.join(os.path.dirname(__file__), "golden", "reference_vectors.json")) as f:
        v = json.load(f)
    for case in v["resolve_draft_tokens"]:
        drafts, targets = case["drafts"], case["targets"]
        D = len(drafts)
        targets = targets + [0] * (D + 1 - len(targets))
        logits = np.zeros((1, D + 1, 64), np.float32)
        for k, t in enumerate(targets):
            logits[0, k, t] = 1.0
        acc, em = llima_amd.verify_greedy(_t(logits, gpu), _t(np.array(drafts, np.int32).reshape(1, D), gpu))
        exp = case["expected"]
        assert int(_np(acc)[0]) == sum(1 for _, a in exp if a)
        assert _np(em)[0, :len(exp)].tolist() == [t for t, _ in exp]


def test_verify_tree_parity(gpu, oracle):
    import llima_amd
    _say("verify_tree")
    rng = np.random.default_rng(12)
    K, V = 16, 128256
    for trial in range(4):
        logits = rng.normal(0, 2, (K, V)).astype(np.float32)
        row_tok = oracle.argmax(logits, mode=1)[0]
        P, L = 10, 5
        ri = rng.integers(-1, K, size=(P, L)).astype(np.int32)
        gathered = oracle.tree_gather(row_tok, ri)
        cand = rng.integers(0, V, size=(P, L)).astype(np.int32)
        # make some paths match the gathered target tokens
        for p in range(P):
            m = rng.integers(0, L)
            cand[p, 1:m + 1] = gathered[p, :m]
        cand[rng.random((P, L)) < 0.05] = -1
        exp = oracle.evaluate_posterior(gathered, cand)
        got = llima_amd.verify_tree(_t(logits, gpu), _t(ri, gpu), _t(cand, gpu))
        assert got == exp, (trial, got, exp)


@pytest.mark.parametrize("B,D,V", [(16, 7, 128256), (5, 3, 1000), (2, 0, 4096), (3, 6, 262144)])
def test_verify_rejection_parity(gpu, oracle, B, D, V):
    import llima_amd
    _say("verify_rejection", B, D, V)
    w = wl.speculative(B=B, D=D, V=V, seed=1004 + V)
    acc, em = llima_amd.verify_rejection(_t(w["target"], gpu), _t(w["draft"], gpu),
                                         _t(w["draft_ids"], gpu), _t(w["u_accept"], gpu),
                                         _t(w["u_resample"], gpu))
    eacc, eem = oracle.verify_rejection(w["target"], w["draft"], w["draft_ids"], w["u_accept"],
                                        w["u_resample"])
    assert (_np(acc) == eacc).all(), (_np(acc), eacc)
    assert (_np(em) == eem).all()


@pytest.mark.parametrize("seed", range(16))
def test_verify_rejection_random(gpu, oracle, seed):
    """Seeded random shapes; drafts either sampled, forced equal to the target
    argmax (long acceptance runs) or random ids (early rejection)."""
    import llima_amd
    rng = np.random.default_rng(7000 + seed)
    B = int(rng.integers(1, 9))
    D = int(rng.integers(0, 9))
    V = int(rng.choice([4, 100, 4096, 32000, 128256]))
    _say("verify_rejection random", seed, B, D, V)
    w = wl.speculative(B=B, D=D, V=V, seed=8000 + seed)
    ids = w["draft_ids"]
    mode = seed % 3
    if mode == 1 and D > 0:
        ids = w["target"][:, :D].argmax(-1).astype(np.int32)
    elif mode == 2 and D > 0:
        ids = rng.integers(0, V, size=(B, D)).astype(np.int32)
    acc, em = llima_amd.verify_rejection(_t(w["target"], gpu), _t(w["draft"], gpu), _t(ids, gpu),
                                         _t(w["u_accept"], gpu), _t(w["u_resample"], gpu))
    eacc, eem = oracle.verify_rejection(w["target"], w["draft"], ids, w["u_accept"],
                                        w["u_resample"])
    assert (_np(acc) == eacc).all(), (_np(acc), eacc)
    assert (_np(em) == eem).all()


def test_verify_rejection_edges(gpu, oracle):
    import llima_amd
    _say("verify_rejection edges")
    rng = np.random.default_rng(3)
    B, D, V = 6, 4, 3000
    tgt = rng.normal(0, 3, (B, D + 1, V)).astype(np.float32)
    drf = tgt[:, :D].copy()
    drf[1] += rng.normal(0, 3, (D, V)).astype(np.float32)
    drf[2, 0, :] = -np.inf; drf[2, 0, 5] = 0.0            # one-hot draft row
    tgt[3, 1, :] = -np.inf                                  # degenerate target row
    tgt[4, 0, 100:200] = np.nan
    tgt[0, 4, [7, 2999]] = np.inf                           # +inf maxima: W = 2^36 at each
    drf[5, 1, 11] = np.inf
    tgt[5, 1, 11] = np.inf
    ids = rng.integers(0, V, (B, D)).astype(np.int32)
    ids[5, 2] = V + 10                                      # out-of-range draft id
    ids[2, 0] = 5
    ua = rng.random((B, D)).astype(np.float32)
    ur = rng.random(B).astype(np.float32)
    acc, em = llima_amd.verify_rejection(_t(tgt, gpu), _t(drf, gpu), _t(ids, gpu), _t(ua, gpu),
                                         _t(ur, gpu))
    eacc, eem = oracle.verify_rejection(tgt, drf, ids, ua, ur)
    assert (_np(acc) == eacc).all() and (_np(em) == eem).all()
    assert eacc[0] == D                                     # identical rows accept every draft


def test_two_streams_use_separate_workspaces(gpu, oracle):
    """Two sampling calls on two streams with no synchronisation between them
    (each stream gets its own scratch), both checked against the oracle."""
    import torch
    import llima_amd
    _say("two streams")
    wa = wl.batched_penalties(B=32, V=128256, H=2048)
    wb = wl.large_vocab_bf16(B=32, V=262144, H=512)
    xa, ua, ha = _t(wa["logits"], gpu), _t(wa["uniforms"], gpu), _t(wa["history"], gpu)
    xb, ub, hb = _t(wb["logits"], gpu), _t(wb["uniforms"], gpu), _t(wb["history"], gpu)
    torch.cuda.synchronize(gpu)
    sa, sb = torch.cuda.Stream(gpu), torch.cuda.Stream(gpu)
    outs = {}
    for rep in range(3):
        with torch.cuda.stream(sa):
            outs["a"] = llima_amd.sample(xa, ua, llima_amd.SamplerConfig(**wa["cfg"]), history=ha)
        with torch.cuda.stream(sb):
            outs["b"] = llima_amd.sample(xb, ub, llima_amd.SamplerConfig(**wb["cfg"]), history=hb)
    torch.cuda.synchronize(gpu)
    from oracle.oracle import SamplerConfig as OC
    for k, w in (("a", wa), ("b", wb)):
        eids, eprobs = oracle.sample(w["logits"], w["uniforms"], OC(**w["cfg"]), history=w["history"])
        assert (_np(outs[k][0]) == eids).all(), k
        assert (_np(outs[k][1]).view(np.uint32) == eprobs.view(np.uint32)).all(), k


def test_empty_batches(gpu, oracle):
    """B = 0 rows (an empty server step) is a no-op on every entry point, with
    empty outputs; an empty row (V = 0) raises as the reference's argmax_bf16
    does (utils.hpp:85-87)."""
    import torch
    import llima_amd
    _say("empty batches")
    V = 1000
    x = torch.empty((0, V), dtype=torch.float32, device=gpu)
    ids, vals = llima_amd.argmax(x)
    assert ids.numel() == 0 and vals.numel() == 0
    ids, probs = llima_amd.sample(x, torch.empty(0, device=gpu),
                                  llima_amd.SamplerConfig(temperature=0.7, top_k=5),
                                  history=torch.empty((0, 4), dtype=torch.int32, device=gpu))
    assert ids.numel() == 0 and probs.numel() == 0
    t = torch.empty((0, 3, V), dtype=torch.float32, device=gpu)
    acc, em = llima_amd.verify_greedy(t, torch.empty((0, 2), dtype=torch.int32, device=gpu))
    assert acc.numel() == 0 and tuple(em.shape) == (0, 3)
    acc, em = llima_amd.verify_rejection(t, torch.empty((0, 2, V), device=gpu),
                                         torch.empty((0, 2), dtype=torch.int32, device=gpu),
                                         torch.empty((0, 2), device=gpu),
                                         torch.empty(0, device=gpu))
    assert acc.numel() == 0 and tuple(em.shape) == (0, 3)
    lp, g = llima_amd.score_logits(x, torch.empty(0, dtype=torch.int32))
    assert lp.numel() == 0 and g.numel() == 0
    cent = torch.empty((0, 8), dtype=torch.bfloat16, device=gpu)
    order = torch.arange(V, dtype=torch.int32, device=gpu)
    ids = llima_amd.argmax_gemma4_mtp_masked_rows(cent, order, 2,
                                                  torch.empty((0, V), dtype=torch.bfloat16,
                                                              device=gpu))
    assert ids.numel() == 0
    with pytest.raises(ValueError):
        llima_amd.argmax_bf16(torch.empty(0, dtype=torch.bfloat16, device=gpu))


def test_workspace_garbage(gpu, oracle):
    """Every entry point gives the same results on a workspace that holds
    arbitrary bytes (all ones, then random): nothing in it is read before the
    call wrote it."""
    import torch
    import llima_amd
    from llima_amd.sampler import Workspace
    _say("workspace garbage")
    rng = np.random.default_rng(99)
    x = rng.normal(0, 3, (4, 30000)).astype(np.float32)
    h = rng.integers(0, 30000, size=(4, 200)).astype(np.int32)
    u = rng.random(4).astype(np.float32)
    cw = wl.constrained(B=2, V=20000, runs=40, seed=5)
    xb = wl.f32_to_bf16_bits(rng.normal(0, 4, (3, 70000)).astype(np.float32))
    sp = wl.speculative(B=3, D=4, V=30000, seed=6)
    tr = rng.normal(0, 3, (6, 9000)).astype(np.float32)
    ri = np.array([[0, 1, 3], [0, 2, -1]], np.int32)
    cand = rng.integers(0, 9000, size=(2, 3)).astype(np.int32)
    cent = wl.f32_to_bf16_bits(rng.normal(0, 2, (2, 512)).astype(np.float32))
    order = rng.permutation(65536).astype(np.uint32)
    xm = wl.f32_to_bf16_bits(rng.normal(0, 2, (2, 65536)).astype(np.float32))
    xflat = rng.normal(0, 0.01, (4, 30000)).astype(np.float32)

    def run_all():
        out = []
        cfg = llima_amd.SamplerConfig(temperature=0.8, top_k=40, top_p=0.9, min_p=0.02,
                                      repetition_penalty=1.2, presence_penalty=0.3,
                                      frequency_penalty=0.2)
        out += [_np(t) for t in llima_amd.sample(_t(x, gpu), _t(u, gpu), cfg, history=_t(h, gpu))]
        out += [_np(t) for t in llima_amd.sample(_t(cw["logits"], gpu), _t(cw["uniforms"], gpu),
                                                  llima_amd.SamplerConfig(**cw["cfg"]),
                                                  bitmask=_t(cw["bitmask"], gpu))]
        for dcfg in (dict(temperature=0.9, top_p=0.9, min_p=0.01, repetition_penalty=1.1),
                     dict(temperature=1.0)):                   # the dense path
            out += [_np(t) for t in llima_amd.sample(_t(x, gpu), _t(u, gpu),
                                                      llima_amd.SamplerConfig(**dcfg),
                                                      history=_t(h, gpu), return_keep=True)]
        out += [_np(t) for t in llima_amd.sample(_t(xflat, gpu), _t(u, gpu),   # dense, then full-row
                                                  llima_amd.SamplerConfig(temperature=1.0, top_p=0.5))]
        out += [_np(t) for t in llima_amd.argmax(_t(xb, gpu))]
        out += [_np(t) for t in llima_amd.verify_greedy(_t(sp["target"], gpu),
                                                         _t(sp["draft_ids"], gpu))]
        out += [_np(t) for t in llima_amd.verify_rejection(
            _t(sp["target"], gpu), _t(sp["draft"], gpu), _t(sp["draft_ids"], gpu),
            _t(sp["u_accept"], gpu), _t(sp["u_resample"], gpu))]
        out += [np.array(llima_amd.verify_tree(_t(tr, gpu), _t(ri, gpu), _t(cand, gpu)))]
        out += [_np(t) for t in llima_amd.score_logits(
            _t(xb, gpu), torch.from_numpy(np.array([5, 7, 9], np.int32)))]
        out += [_np(llima_amd.argmax_gemma4_mtp_masked_rows(_t(cent, gpu), _t(order, gpu), 8,
                                                             _t(xm, gpu)))]
        return out

    ref = run_all()
    for fill in ("ones", "random"):
        for buf in Workspace._bufs.values():
            if fill == "ones":
                buf.fill_(255)
            else:
                buf.copy_(torch.randint(0, 256, buf.shape, dtype=torch.uint8, device=buf.device))
        got = run_all()
        for i, (a, b) in enumerate(zip(ref, got)):
            assert np.array_equal(a, b, equal_nan=True), (fill, i)


def test_workspace_reuse_across_shapes(gpu, oracle):
    """One workspace buffer per entry point serves calls of any shape, in any
    order (the kernels keep no state in the workspace between calls)."""
    import llima_amd
    _say("workspace reuse across shapes")
    rng = np.random.default_rng(77)
    for B, V in [(16, 30000), (4, 30000), (16, 9000), (1, 70000), (12, 30000)]:
        x = rng.normal(0, 2, (B, V)).astype(np.float32)
        h = rng.integers(0, V, size=(B, 100)).astype(np.int32)
        u = rng.random(B).astype(np.float32)
        _sample_both(gpu, oracle, x, u, dict(temperature=0.9, top_k=30, top_p=0.9,
                                             repetition_penalty=1.2), history=h)
    for B, D, V in [(6, 5, 3000), (2, 0, 4096), (3, 2, 9000), (6, 6, 3000)]:
        w = wl.speculative(B=B, D=D, V=V, seed=B + D)
        acc, em = llima_amd.verify_rejection(_t(w["target"], gpu), _t(w["draft"], gpu),
                                             _t(w["draft_ids"], gpu), _t(w["u_accept"], gpu),
                                             _t(w["u_resample"], gpu))
        eacc, eem = oracle.verify_rejection(w["target"], w["draft"], w["draft_ids"],
                                            w["u_accept"], w["u_resample"])
        assert (_np(acc) == eacc).all() and (_np(em) == eem).all()
        tgt = w["target"]
        dr = tgt[:, :D].argmax(-1).astype(np.int32)
        acc, em = llima_amd.verify_greedy(_t(tgt, gpu), _t(dr, gpu))
        eacc, eem = oracle.verify_greedy(tgt, dr)
        assert (_np(acc) == eacc).all() and (_np(em) == eem).all()


# ----------------------------------------------------------------- score_logits
# Tolerance: the reference sums exp(x - max) in double; the kernel's terms are
# fp32 exp2 values accumulated in double, so the log-probability agrees to about
# 1e-6 (asserted: 1e-5 absolute, the fp32 probability tolerance).  The argmax
# flag, NaN and infinity outcomes are exact.
SCORE_TOL = 1e-5


def _score_check(got_lp, got_g, x, targets, oracle):
    for r, t in enumerate(targets):
        elp, eg = oracle.score_logits(x[r], int(t))
        g = float(got_lp[r])
        if np.isnan(elp):
            assert np.isnan(g), (r, t, g)
        elif np.isinf(elp):
            assert g == elp, (r, t, g, elp)
        else:
            assert abs(g - elp) <= SCORE_TOL, (r, t, g, elp)
        assert bool(got_g[r]) == eg, (r, t)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("B,V", [(1, 1), (3, 7), (4, 5003), (8, 128256), (2, 262144)])
def test_score_logits_parity(gpu, oracle, dtype, B, V):
    import torch
    import llima_amd
    _say("score_logits", dtype, B, V)
    rng = np.random.default_rng(B * 7 + V)
    x = rng.normal(0, 3, (B, V)).astype(np.float32)
    x[:, rng.integers(0, V, size=3)] = x.max() + 1          # ties at the maximum
    if dtype == "bf16":
        x = wl.f32_to_bf16_bits(x)
    xf = x if dtype == "f32" else wl.bf16_bits_to_f32(x)
    am = np.argmax(xf, axis=1)
    for targets in [am, rng.integers(0, V, size=B)]:
        lp, g = llima_amd.score_logits(_t(x, gpu), torch.from_numpy(targets.astype(np.int32)))
        _score_check(_np(lp), _np(g), x, targets, oracle)


def test_score_logits_edges(gpu, oracle):
    import torch
    import llima_amd
    _say("score_logits edges")
    V = 10000
    rng = np.random.default_rng(5)
    x = rng.normal(0, 2, (8, V)).astype(np.float32)
    x[0, 77] = np.nan                      # any NaN -> NaN
    x[1, :] = -np.inf                      # all -inf -> NaN, argmax 0
    x[2, 5] = np.inf                       # infinite maximum -> NaN
    x[3, 9] = -np.inf                      # -inf target -> -inf
    x[4, :] = 1.5                          # all equal: argmax 0
    x[5, 4096:8192] = -np.inf              # a whole chunk of -inf
    x[6, :] = np.nan
    targets = np.array([3, 0, 5, 9, 0, 100, 1, 9999], np.int32)
    lp, g = llima_amd.score_logits(_t(x, gpu), torch.from_numpy(targets))
    _score_check(_np(lp), _np(g), x, targets, oracle)
    # strided rows
    xs = _t(x, gpu)[2:8, 7:9007]
    lp, g = llima_amd.score_logits(xs, torch.from_numpy(targets[2:8] % 9000))
    _score_check(_np(lp), _np(g), x[2:8, 7:9007], targets[2:8] % 9000, oracle)
    # one row, the reference's signature
    lp1, g1 = llima_amd.score_logits(_t(x[3], gpu), 9)
    assert lp1 == -np.inf and not g1
    with pytest.raises(RuntimeError):
        llima_amd.score_logits(_t(x[3], gpu), V)
    with pytest.raises(RuntimeError):
        llima_amd.score_logits(_t(x[:2], gpu), torch.tensor([0, V], dtype=torch.int32))


# ----------------------------------------------------------------- Gemma4 MTP masked argmax
def _mtp_expected(oracle, cent_bits, ordering, k, x):
    cand = oracle.select_candidate_tokens(cent_bits, ordering, k)
    return cand, oracle.masked_argmax(x, cand)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("B,C,V,k", [(4, 2048, 262144, 32), (3, 16, 64, 5), (2, 100, 1000, 100),
                                     (5, 8192, 65536, 7), (1, 1, 9, 1)])
def test_mtp_masked_argmax_parity(gpu, oracle, dtype, B, C, V, k):
    import llima_amd
    _say("mtp masked argmax", dtype, B, C, V, k)
    rng = np.random.default_rng(C + V + k)
    cent = wl.f32_to_bf16_bits(rng.integers(-20, 21, size=(B, C)).astype(np.float32) * 0.5)  # ties
    ordering = rng.permutation(V).astype(np.uint32)
    x = rng.integers(-40, 41, size=(B, V)).astype(np.float32) * np.float32(0.25)              # ties
    x[0, rng.integers(0, V, size=V // 3)] = -np.inf
    if dtype == "bf16":
        x = wl.f32_to_bf16_bits(x)
    ids = llima_amd.argmax_gemma4_mtp_masked_rows(_t(cent, gpu), _t(ordering, gpu), k, _t(x, gpu))
    cands = llima_amd.select_candidate_tokens(_t(cent, gpu), _t(ordering, gpu), k)
    for r in range(B):
        ec, eid = _mtp_expected(oracle, cent[r], ordering, k, x[r])
        assert _np(cands[r]).astype(np.uint32).tolist() == ec.tolist(), r
        assert int(_np(ids)[r]) == eid, r


def test_mtp_masked_argmax_reference_vectors_and_errors(gpu, oracle):
    import json
    import os
    import torch
    import llima_amd
    _say("mtp reference vectors")
    path = os.path.join(os.path.dirname(__file__), "golden", "reference_vectors.json")
    v = json.load(open(path))
    for case in v["select_candidate_tokens"]:
        c = wl.f32_to_bf16_bits(np.array(case["centroid_logits"], np.float32))
        got = llima_amd.select_candidate_tokens(_t(c, gpu), _t(np.array(case["token_ordering"],
                                                                        np.uint32), gpu),
                                                case["top_k"])
        assert got == case["expected"]
    for case in v["select_candidate_tokens_errors"]:
        c = wl.f32_to_bf16_bits(np.array(case["centroid_logits"], np.float32))
        with pytest.raises(RuntimeError):
            llima_amd.select_candidate_tokens(_t(c, gpu), _t(np.array(case["token_ordering"],
                                                                      np.uint32), gpu),
                                              case["top_k"])
    # no candidate with a number -> the reference's "selected no token"
    cent = wl.f32_to_bf16_bits(np.array([1, 3, 2, 0], np.float32))
    order = np.arange(8, dtype=np.uint32)
    x = np.zeros(8, np.float32)
    x[2:4] = np.nan
    with pytest.raises(RuntimeError):
        llima_amd.argmax_gemma4_mtp_masked_row(_t(cent, gpu), _t(order, gpu), 1, _t(x, gpu))
    x[3] = -np.inf                                           # -inf is a candidate value
    assert llima_amd.argmax_gemma4_mtp_masked_row(_t(cent, gpu), _t(order, gpu), 1,
                                                  _t(x, gpu)) == 3
    x[:] = 7.0                                               # equal values -> lowest token id
    assert llima_amd.argmax_gemma4_mtp_masked_row(_t(cent, gpu), _t(order, gpu), 4,
                                                  _t(x, gpu)) == 0
    bad = order.copy()
    bad[5] = 8                                               # out-of-range id in a selected run
    with pytest.raises(RuntimeError):
        llima_amd.argmax_gemma4_mtp_masked_row(_t(cent, gpu), _t(bad, gpu), 3, _t(x, gpu))
    bad = order.copy()
    bad[7] = 0xFFFFFFFF                                      # in an unselected run: ignored
    assert llima_amd.argmax_gemma4_mtp_masked_row(_t(cent, gpu), _t(bad, gpu), 3,
                                                  _t(x, gpu)) == 0
    with pytest.raises(RuntimeError):
        llima_amd.argmax_gemma4_mtp_masked_row(_t(cent, gpu), _t(order, gpu), 5, _t(x, gpu))


# ----------------------------------------------------------------- maximum sizes
def test_sample_maximum_sizes(gpu, oracle):
    """V = 2^24, the largest llima_sample takes: 4096 fp32 (2048 bf16) chunks a
    row, more than the finish gathers, so every row takes the exact full-row
    path; with a 65535-id history, the largest H_max."""
    _say("sample maximum sizes")
    rng = np.random.default_rng(11)
    V = 1 << 24
    x = rng.normal(0, 3, (2, V)).astype(np.float32)
    h = rng.integers(0, V, size=(2, 65535)).astype(np.int32)
    h[:, :4000] = np.argsort(x, axis=1)[:, -4000:]          # the top of each row repeated
    u = rng.random(2).astype(np.float32)
    _sample_both(gpu, oracle, x, u, dict(temperature=0.9, top_k=40, top_p=0.9,
                                         repetition_penalty=1.2, presence_penalty=0.2), history=h)
    xb = wl.f32_to_bf16_bits(x[:1])
    _sample_both(gpu, oracle, xb, u[:1], dict(temperature=1.0, top_k=64, top_p=0.95, min_p=0.01),
                 history=h[:1])


def test_argmax_and_verify_greedy_maximum_sizes(gpu, oracle):
    """Rows longer than 2^24 ids (argmax has no vocabulary limit): the index
    part of the 64-bit keys and the split arithmetic past 2^24."""
    import llima_amd
    _say("argmax maximum sizes")
    rng = np.random.default_rng(12)
    V = (1 << 24) + 1003
    x = rng.integers(-40, 41, size=(2, V)).astype(np.float32) * np.float32(0.25)
    x[0, V - 1] = 100.0                                      # the last id
    x[1, [(1 << 24) + 5, (1 << 24) + 7]] = 100.0             # ties past 2^24
    for mode, mname in [(0, "split_first"), (1, "neg_inf"), (2, "quarters")]:
        ids, vals = llima_amd.argmax(_t(x, gpu), split_dim=(1 << 22) + 1, mode=mname)
        eids, evals = oracle.argmax(x, split_dim=(1 << 22) + 1, mode=mode)
        assert (_np(ids) == eids).all(), (mname, _np(ids), eids)
        assert (_np(vals).view(np.uint32) == evals.view(np.uint32)).all()
    t = x.reshape(1, 2, V)
    dr = np.array([[V - 1]], np.int32)
    acc, em = llima_amd.verify_greedy(_t(t, gpu), _t(dr, gpu))
    eacc, eem = oracle.verify_greedy(t, dr)
    assert (_np(acc) == eacc).all() and (_np(em) == eem).all()


def test_verify_rejection_maximum_sizes(gpu, oracle):
    """V = 2^22, the largest llima_verify_rejection takes: 512 chunks a row
    (the row pass polls 8 slots a lane), 2048 draw workgroups per sequence."""
    import llima_amd
    _say("verify_rejection maximum sizes")
    w = wl.speculative(B=2, D=2, V=1 << 22, seed=13)
    for ids in [w["draft_ids"], w["target"][:, :2].argmax(-1).astype(np.int32)]:
        acc, em = llima_amd.verify_rejection(_t(w["target"], gpu), _t(w["draft"], gpu),
                                             _t(ids, gpu), _t(w["u_accept"], gpu),
                                             _t(w["u_resample"], gpu))
        eacc, eem = oracle.verify_rejection(w["target"], w["draft"], ids, w["u_accept"],
                                            w["u_resample"])
        assert (_np(acc) == eacc).all(), (_np(acc), eacc)
        assert (_np(em) == eem).all()


def test_score_and_mtp_maximum_sizes(gpu, oracle):
    """score_logits over rows longer than 2^24 ids; the MTP masked argmax at
    C = 8192 centroids and the largest V below 2^24 that C divides (65504
    candidates a row)."""
    import torch
    import llima_amd
    _say("score / mtp maximum sizes")
    rng = np.random.default_rng(14)
    V = (1 << 24) + 5
    x = rng.normal(0, 3, (2, V)).astype(np.float32)
    x[1, V - 2] = x[1].max() + 1
    targets = np.array([V - 1, V - 2], np.int32)
    lp, g = llima_amd.score_logits(_t(x, gpu), torch.from_numpy(targets))
    _score_check(_np(lp), _np(g), x, targets, oracle)
    C, k = 8192, 32
    Vm = (1 << 24) - C
    cent = wl.f32_to_bf16_bits(rng.integers(-20, 21, size=(1, C)).astype(np.float32) * 0.5)
    ordering = rng.permutation(Vm).astype(np.uint32)
    xm = wl.f32_to_bf16_bits(rng.normal(0, 2, (1, Vm)).astype(np.float32))
    ids = llima_amd.argmax_gemma4_mtp_masked_rows(_t(cent, gpu), _t(ordering, gpu), k, _t(xm, gpu))
    ec, eid = _mtp_expected(oracle, cent[0], ordering, k, xm[0])
    assert int(_np(ids)[0]) == eid


# ----------------------------------------------------------------- LM head
# Tolerance: each logit is a sum of H fp32 products of bf16 values (exact in
# fp32), in an order the float64 reference does not follow.  The longest
# sequential chain of fp32 additions is H/4 + 70 (the MFMA path adds 4-id
# products step after step; the GEMV path H/512 per lane, then a 64-lane tree),
# so |logit - ref| <= (H/4 + 70) 2^-24 sum_h |x_h w_h| + 1e-6, plus 4e-6 |ref|
# for the softcap's tanhf (x -> cap tanh(x / cap) is 1-Lipschitz).  The argmax is exact with respect to the
# kernel's own logits: the first index of their maximum, NaN never wins.
def _lm_head_check(ids, vals, logits, x, w, cap, bf16=True):
    """Logits against a float64 product of the same bf16 values: the fp32 sum's
    error bound, plus half a bf16 ulp (2^-8 relative) when the logits are
    rounded to bf16 (then they must be bf16 values); the argmax exact with
    respect to the logits returned (first index, NaN never wins), and against
    the float64 logits: the id's logit within the two error bounds of the
    float64 maximum, and the float64 argmax itself wherever it leads every
    other id by more than both bounds."""
    xf = wl.bf16_bits_to_f32(x).astype(np.float64)
    wf = wl.bf16_bits_to_f32(w).astype(np.float64)
    s = xf @ wf.T
    ref = cap * np.tanh(s / cap) if cap > 0 else s
    H = x.shape[1]
    bound = (H / 4 + 70) * 2.0**-24 * (np.abs(xf) @ np.abs(wf).T) + 1e-6 + 4e-6 * np.abs(ref)
    if bf16:
        bound = bound * (1 + 2.0**-8) + 2.0**-8 * np.abs(ref)
        assert ((logits.view(np.uint32) & 0xFFFF) == 0).all()
    fin = np.isfinite(ref)
    assert (np.abs(logits - ref)[fin] <= bound[fin]).all(), np.abs(logits - ref)[fin].max()
    for b in range(x.shape[0]):
        row = logits[b]
        ok = ~np.isnan(row)
        if not ok.any():
            assert ids[b] == 0 and np.isnan(vals[b])
            continue
        m = row[ok].max()
        assert ids[b] == int(np.flatnonzero(ok & (row == m))[0]), b
        assert vals[b] == m
        r, bd = ref[b], bound[b]
        if np.isfinite(r).all():
            top = int(np.argmax(r))
            assert r[ids[b]] >= r[top] - bd[ids[b]] - bd[top], (b, ids[b], top)
            rest = np.delete(r + bd, top)
            if rest.size == 0 or r[top] - bd[top] > rest.max():
                assert ids[b] == top, (b, ids[b], top)


@pytest.mark.parametrize("B,H,V,cap", [(1, 4096, 128256, 0.0), (3, 1536, 262144, 30.0),
                                       (8, 2048, 50000, 0.0), (11, 512, 1000, 30.0),
                                       (5, 8, 7, 0.0), (4, 4096, 3001, 0.0),
                                       (16, 4096, 128256, 0.0), (70, 1536, 3001, 30.0),
                                       (64, 2048, 50000, 0.0), (17, 512, 1000, 30.0),
                                       (20, 1000, 999, 0.0), (6, 4096, 70000, 30.0),
                                       (1, 8192, 5000, 0.0), (3, 16384, 1000, 30.0),
                                       (200, 512, 1000, 30.0), (300, 256, 777, 0.0),
                                       (128, 1024, 2049, 0.0)])
def test_lm_head_argmax_parity(gpu, B, H, V, cap):
    import llima_amd
    _say("lm head", B, H, V, cap)
    rng = np.random.default_rng(B * 31 + H + V)
    x = wl.f32_to_bf16_bits(rng.normal(0, 1, (B, H)).astype(np.float32))
    w = wl.f32_to_bf16_bits(rng.normal(0, 1.0 / np.sqrt(H), (V, H)).astype(np.float32))
    for ld in ("bf16", "f32"):
        ids, vals, logits = llima_amd.lm_head_argmax(_t(x, gpu), _t(w, gpu), softcap=cap,
                                                     return_logits=True, logit_dtype=ld)
        _lm_head_check(_np(ids), _np(vals), _np(logits), x, w, cap, bf16=ld == "bf16")
        ids2, vals2 = llima_amd.lm_head_argmax(_t(x, gpu), _t(w, gpu), softcap=cap, logit_dtype=ld)
        assert (_np(ids2) == _np(ids)).all()
        assert (_np(vals2).view(np.uint32) == _np(vals).view(np.uint32)).all()


def _lm_head_takes_mfma(B, H):
    """Whether llima_lm_head_argmax takes its MFMA tiles (more hidden rows than
    one matrix-vector pass stages, or rows wider than 4096)."""
    per = 16384 // H
    per = 8 if per >= 8 else 4 if per >= 4 else 2 if per >= 2 else 1
    return (B > per or H > 4096) and H % 64 == 0


@pytest.mark.parametrize("B,H,V,cap", [(1, 4096, 32768, 0.0), (64, 4096, 20000, 30.0),
                                       (33, 512, 1000, 30.0), (64, 2048, 50000, 0.0),
                                       (17, 256, 777, 0.0), (40, 1024, 70000, 30.0),
                                       (100, 512, 3001, 0.0), (5, 256, 31, 0.0),
                                       (32, 768, 4097, 0.0), (130, 256, 1000, 30.0),
                                       (8, 8192, 3000, 0.0)])
def test_lm_head_packed_parity(gpu, B, H, V, cap):
    """The packed weight (llima_lm_head_pack) gives logits within the fp32 sum's
    bound of the float64 product and, where the plain entry point takes its MFMA
    tiles (the same k order), the same logits and ids bit for bit."""
    import llima_amd
    _say("lm head packed", B, H, V, cap)
    rng = np.random.default_rng(B * 37 + H + V)
    x = wl.f32_to_bf16_bits(rng.normal(0, 1, (B, H)).astype(np.float32))
    w = wl.f32_to_bf16_bits(rng.normal(0, 1.0 / np.sqrt(H), (V, H)).astype(np.float32))
    pk = llima_amd.lm_head_pack(_t(w, gpu))
    assert pk.data.numel() == (V + 31) // 32 * 32 * H * 2
    for ld in ("bf16", "f32"):
        ids, vals, logits = llima_amd.lm_head_argmax(_t(x, gpu), pk, softcap=cap,
                                                     return_logits=True, logit_dtype=ld)
        _lm_head_check(_np(ids), _np(vals), _np(logits), x, w, cap, bf16=ld == "bf16")
        ids2, vals2 = llima_amd.lm_head_argmax(_t(x, gpu), pk, softcap=cap, logit_dtype=ld)
        assert (_np(ids2) == _np(ids)).all()
        assert (_np(vals2).view(np.uint32) == _np(vals).view(np.uint32)).all()
        if _lm_head_takes_mfma(B, H):
            ids3, vals3, logits3 = llima_amd.lm_head_argmax(_t(x, gpu), _t(w, gpu), softcap=cap,
                                                            return_logits=True, logit_dtype=ld)
            assert (_np(logits3).view(np.uint32) == _np(logits).view(np.uint32)).all()
            assert (_np(ids3) == _np(ids)).all()


def test_lm_head_packed_ties_and_nan(gpu):
    """The packed path's argmax rules: equal vocab rows tie and the lower index
    wins, a NaN logit never wins, an all-NaN row gives id 0 and a NaN value."""
    import llima_amd
    _say("lm head packed ties / nan")
    rng = np.random.default_rng(6)
    B, H, V = 3, 256, 5000
    x = wl.f32_to_bf16_bits(rng.normal(0, 1, (B, H)).astype(np.float32))
    wf = rng.normal(0, 0.05, (V, H)).astype(np.float32)
    wf[4000] = wl.bf16_bits_to_f32(x[0]) * 0.5
    wf[1234] = wf[4000]
    wf[17, 3] = np.nan
    w = wl.f32_to_bf16_bits(wf)
    xn = x.copy()
    xn[2] = wl.f32_to_bf16_bits(np.full(H, np.nan, np.float32))
    pk = llima_amd.lm_head_pack(_t(w, gpu))
    ids, vals, logits = llima_amd.lm_head_argmax(_t(xn, gpu), pk, return_logits=True)
    ids, vals, logits = _np(ids), _np(vals), _np(logits)
    assert ids[0] == 1234
    assert np.isnan(logits[1, 17]) and ids[1] != 17
    assert ids[2] == 0 and np.isnan(vals[2])
    _lm_head_check(ids[:2], vals[:2], logits[:2], x[:2], w, 0.0)


@pytest.mark.parametrize("ld,out", [("bf16", "f32"), ("f32", "f32"), ("bf16", "bf16")])
def test_lm_head_then_sample(gpu, oracle, ld, out):
    """A sampled decode step: the LM head's logits stay in device memory and feed
    llima_sample directly (fp32, or bf16 with half the bytes); ids,
    probabilities and kept sets equal the oracle's on the same logits (copied
    to the host), and the greedy sampler's ids equal the LM head's fused
    argmax."""
    import torch
    import llima_amd
    from oracle.oracle import SamplerConfig as OC
    _say("lm head -> sample", ld, out)
    rng = np.random.default_rng(31)
    B, H, V = 8, 1024, 50000
    x = wl.f32_to_bf16_bits(rng.normal(0, 1, (B, H)).astype(np.float32))
    w = wl.f32_to_bf16_bits(rng.normal(0, 4.0 / np.sqrt(H), (V, H)).astype(np.float32))
    ids_f, _, logits = llima_amd.lm_head_argmax(_t(x, gpu), _t(w, gpu), softcap=30.0,
                                                return_logits=True, logit_dtype=ld, logits_out=out)
    hist = rng.integers(0, V, size=(B, 256)).astype(np.int32)
    u = rng.random(B).astype(np.float32)
    cfgd = dict(temperature=0.8, top_k=50, top_p=0.95, min_p=0.05, repetition_penalty=1.15,
                presence_penalty=0.5, frequency_penalty=0.3)
    ids, probs, keep = llima_amd.sample(logits, _t(u, gpu), llima_amd.SamplerConfig(**cfgd),
                                        history=_t(hist, gpu), return_keep=True)
    host = _np(logits.view(torch.int16)).view(np.uint16) if out == "bf16" else _np(logits)
    eids, eprobs, ekeep = oracle.sample(host, u, OC(**cfgd), history=hist, want_keep=True)
    assert (_np(ids) == eids).all()
    assert (_np(probs).view(np.uint32) == eprobs.view(np.uint32)).all()
    assert (_np(keep).view(np.uint32) == ekeep).all()
    gids, _ = llima_amd.sample(logits, _t(u, gpu), llima_amd.SamplerConfig(greedy=True))
    assert (_np(gids) == _np(ids_f)).all()


@pytest.mark.parametrize("B,H,V,packed", [(2, 4096, 50000, False), (20, 1024, 30000, False),
                                           (40, 512, 20000, True), (3, 256, 777, True)])
def test_lm_head_bf16_logits_out(gpu, B, H, V, packed):
    """bf16 logits output (LLIMA_LOGITS_OUT_BF16) on the matrix-vector path,
    the MFMA tiles and the packed weight: every logit is the upper half of
    the fp32 output of the same bf16-rounded logits (NaN as a NaN), and the
    ids and values are unchanged."""
    import torch
    import llima_amd
    _say("lm head bf16 logits out", B, H, V, packed)
    rng = np.random.default_rng(B + H + V)
    x = wl.f32_to_bf16_bits(rng.normal(0, 1, (B, H)).astype(np.float32))
    wf = rng.normal(0, 3.0 / np.sqrt(H), (V, H)).astype(np.float32)
    wf[5, 0] = np.nan                                           # a NaN logit in every row
    w = _t(wl.f32_to_bf16_bits(wf), gpu)
    wt = llima_amd.lm_head_pack(w) if packed else w
    i32, v32, l32 = llima_amd.lm_head_argmax(_t(x, gpu), wt, softcap=30.0, return_logits=True)
    i16, v16, l16 = llima_amd.lm_head_argmax(_t(x, gpu), wt, softcap=30.0, return_logits=True,
                                             logits_out="bf16")
    assert l16.dtype == torch.bfloat16
    a = _np(l32).view(np.uint32)
    b = _np(l16.view(torch.int16)).view(np.uint16).astype(np.uint32)
    nan = np.isnan(_np(l32))
    assert (b[~nan] == (a[~nan] >> 16)).all()
    assert np.isnan(wl.bf16_bits_to_f32(b[nan].astype(np.uint16))).all() and nan[:, 5].all()
    assert (_np(i16) == _np(i32)).all()
    assert (_np(v16).view(np.uint32) == _np(v32).view(np.uint32)).all()
    with pytest.raises(ValueError):
        llima_amd.lm_head_argmax(_t(x, gpu), wt, return_logits=True, logit_dtype="f32",
                                 logits_out="bf16")


# LM head scoring: the (B, H, V, softcap, packed) cases cover the matrix-vector
# path (B up to 8), the MFMA tiles (wider batches, H > 4096, two 256-row passes)
# and the packed weight (32- and 64-row passes, two passes).
LM_SCORE_CASES = [(1, 4096, 32768, 0.0, False), (3, 1024, 50000, 30.0, False),
                  (8, 2048, 20000, 0.0, False), (17, 256, 777, 0.0, False),
                  (64, 4096, 20000, 30.0, False), (300, 256, 3001, 0.0, False),
                  (4, 8192, 3000, 0.0, False), (5, 256, 31, 0.0, True),
                  (40, 1024, 70000, 30.0, True), (64, 4096, 20000, 0.0, True),
                  (70, 512, 5000, 0.0, True)]


@pytest.mark.parametrize("B,H,V,cap,packed", LM_SCORE_CASES)
def test_lm_head_score(gpu, oracle, B, H, V, cap, packed):
    """llima_lm_head_score: the log-probability and greedy flag of score_logits
    over the logits lm_head_argmax writes for the same inputs (the oracle on
    those logits, SCORE_TOL; the flag exact), for bf16-rounded and fp32
    logits.  Half the targets are the row's argmax."""
    import llima_amd
    _say("lm head score", B, H, V, cap, packed)
    rng = np.random.default_rng(B * 7 + H + V)
    x = _t(wl.f32_to_bf16_bits(rng.normal(0, 1, (B, H)).astype(np.float32)), gpu)
    w = _t(wl.f32_to_bf16_bits(rng.normal(0, 4.0 / np.sqrt(H), (V, H)).astype(np.float32)), gpu)
    wt = llima_amd.lm_head_pack(w) if packed else w
    for ld in ("bf16", "f32"):
        ids, _, logits = llima_amd.lm_head_argmax(x, wt, softcap=cap, return_logits=True,
                                                  logit_dtype=ld)
        targets = rng.integers(0, V, B).astype(np.int32)
        targets[::2] = _np(ids)[::2]
        lp, g = llima_amd.lm_head_score(x, wt, torch_i32(targets, gpu), softcap=cap,
                                        logit_dtype=ld)
        _score_check(_np(lp), _np(g), _np(logits), targets, oracle)
        assert _np(g)[::2].all()


@pytest.mark.parametrize("seed", range(16))
def test_lm_head_random_configs(gpu, oracle, seed):
    """Seeded random LM head cases over every path (matrix-vector, MFMA tiles,
    packed; ragged batches and vocabularies, softcap on or off, bf16 or fp32
    logits): ids against the float64 product (_lm_head_check), and the scoring
    entry point against the oracle's score_logits on the head's logits."""
    import llima_amd
    rng = np.random.default_rng(9000 + seed)
    packed = bool(rng.integers(0, 2))
    H = int(rng.choice([256, 512, 1024, 4096] if packed else [8, 200, 256, 1000, 1536, 4096, 8192]))
    B = int(rng.choice([1, 3, 8, 9, 31, 33, 64, 65, 129, 257]))
    V = max(1, min(int(rng.integers(1, 40000)), int(1e9 // (B * H))))
    cap = float(rng.choice([0.0, 30.0]))
    ld = str(rng.choice(["bf16", "f32"]))
    _say("lm head random", seed, B, H, V, cap, ld, packed)
    x = wl.f32_to_bf16_bits(rng.normal(0, 1, (B, H)).astype(np.float32))
    w = wl.f32_to_bf16_bits(rng.normal(0, 4.0 / np.sqrt(H), (V, H)).astype(np.float32))
    wt = llima_amd.lm_head_pack(_t(w, gpu)) if packed else _t(w, gpu)
    ids, vals, logits = llima_amd.lm_head_argmax(_t(x, gpu), wt, softcap=cap, return_logits=True,
                                                 logit_dtype=ld)
    _lm_head_check(_np(ids), _np(vals), _np(logits), x, w, cap, bf16=ld == "bf16")
    targets = rng.integers(0, V, B).astype(np.int32)
    targets[::3] = _np(ids)[::3]
    lp, g = llima_amd.lm_head_score(_t(x, gpu), wt, torch_i32(targets, gpu), softcap=cap,
                                    logit_dtype=ld)
    _score_check(_np(lp), _np(g), _np(logits), targets, oracle)


@pytest.mark.parametrize("B,D,H,V,cap,packed", [(1, 0, 4096, 32000, 0.0, False),
                                                (4, 7, 4096, 128256, 0.0, True),
                                                (16, 7, 1024, 50000, 30.0, False),
                                                (9, 3, 256, 777, 0.0, True),
                                                (3, 15, 512, 5000, 30.0, True),
                                                (40, 5, 256, 3001, 0.0, False)])
def test_lm_head_verify_greedy(gpu, B, D, H, V, cap, packed):
    """llima_lm_head_verify_greedy: accepted lengths and emitted tokens equal the
    chain rule (resolve_draft_tokens) over the head's own argmax ids, and
    llima_verify_greedy over the logits the head writes; drafts built so that
    every acceptance length from 0 to D occurs."""
    import llima_amd
    _say("lm head verify greedy", B, D, H, V, cap, packed)
    rng = np.random.default_rng(B * 13 + D + H + V)
    x = wl.f32_to_bf16_bits(rng.normal(0, 1, (B * (D + 1), H)).astype(np.float32))
    w = wl.f32_to_bf16_bits(rng.normal(0, 4.0 / np.sqrt(H), (V, H)).astype(np.float32))
    wt = llima_amd.lm_head_pack(_t(w, gpu)) if packed else _t(w, gpu)
    for ld in ("bf16", "f32"):
        ids, _, logits = llima_amd.lm_head_argmax(_t(x, gpu), wt, softcap=cap, return_logits=True,
                                                  logit_dtype=ld)
        tok = _np(ids).reshape(B, D + 1)
        drafts = rng.integers(0, V, (B, D)).astype(np.int32)
        for b in range(B):
            L = b % (D + 1)
            drafts[b, :L] = tok[b, :L]
            if L < D and drafts[b, L] == tok[b, L]:
                drafts[b, L] = (tok[b, L] + 1) % V
        hid = _t(x, gpu).view(B, D + 1, H)
        acc, em = llima_amd.lm_head_verify_greedy(hid, wt, torch_i32(drafts, gpu), softcap=cap,
                                                  logit_dtype=ld)
        acc, em = _np(acc), _np(em)
        for b in range(B):
            want = llima_amd.resolve_draft_tokens(drafts[b], tok[b])
            assert acc[b] == len(want) - 1 == min(b % (D + 1), D), (b, acc[b])
            assert list(em[b, :acc[b] + 1]) == [t for t, _ in want], b
            assert (em[b, acc[b] + 1:] == -1).all(), b
        if D + 1 <= 64:
            acc2, em2 = llima_amd.verify_greedy(logits.reshape(B, D + 1, V), torch_i32(drafts, gpu))
            assert (_np(acc2) == acc).all() and (_np(em2) == em).all()


@pytest.mark.parametrize("K,H,V,packed", [(16, 4096, 128256, False), (16, 4096, 32000, True),
                                           (26, 512, 5000, True), (5, 256, 777, False)])
def test_lm_head_verify_tree(gpu, oracle, K, H, V, packed):
    """llima_lm_head_verify_tree: (best path, accept length, bonus) equal
    llima_verify_tree over the head's logits and the oracle's gather +
    evaluate_posterior over the head's argmax, with paths built to match."""
    import llima_amd
    _say("lm head verify tree", K, H, V, packed)
    rng = np.random.default_rng(K + H + V)
    xf = rng.normal(0, 1, (K, H)).astype(np.float32)
    xf[K // 2] = np.nan                         # a row with no logit above -inf: token 0
    x = wl.f32_to_bf16_bits(xf)
    w = wl.f32_to_bf16_bits(rng.normal(0, 4.0 / np.sqrt(H), (V, H)).astype(np.float32))
    wt = llima_amd.lm_head_pack(_t(w, gpu)) if packed else _t(w, gpu)
    ids, _, logits = llima_amd.lm_head_argmax(_t(x, gpu), wt, return_logits=True)
    row_tok = _np(ids)
    assert row_tok[K // 2] == 0 and np.isnan(_np(logits)[K // 2]).all()
    for trial in range(4):
        P, L = 10, 5
        ri = rng.integers(-1, K, size=(P, L)).astype(np.int32)
        gathered = oracle.tree_gather(row_tok, ri)
        cand = rng.integers(0, V, size=(P, L)).astype(np.int32)
        for p in range(P):
            m = rng.integers(0, L)
            cand[p, 1:m + 1] = gathered[p, :m]
        cand[rng.random((P, L)) < 0.05] = -1
        ri[0, :] = K // 2                       # one path through the NaN row (token 0)
        gathered = oracle.tree_gather(row_tok, ri)
        cand[0, 1:] = 0
        exp = oracle.evaluate_posterior(gathered, cand)
        got = llima_amd.lm_head_verify_tree(_t(x, gpu), wt, _t(ri, gpu), _t(cand, gpu))
        assert got == exp, (trial, got, exp)
        assert got == llima_amd.verify_tree(logits, _t(ri, gpu), _t(cand, gpu)), trial


def torch_i32(a, gpu):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.int32)).to(gpu)


@pytest.mark.parametrize("packed", [False, True])
def test_lm_head_score_edges(gpu, oracle, packed):
    """Scoring edge cases against the oracle on the written logits: equal
    vocab rows (the lower id is the greedy one), a NaN hidden row (NaN), a row
    with a +inf logit (NaN: infinite maximum), a -inf logit beside finite ones
    (the target's log-probability -inf, the others finite); a single row with
    an int target; a target outside the vocabulary raises (the C ABI's flag is
    LLIMA_E_RANGE)."""
    import torch
    import llima_amd
    from llima_amd import _lib
    _say("lm head score edges", packed)
    rng = np.random.default_rng(9)
    B, H, V = 6, 256, 5000
    xf = rng.normal(0, 1, (B, H)).astype(np.float32)
    wf = rng.normal(0, 0.1, (V, H)).astype(np.float32)
    wf[3000] = xf[0] * 0.5                                      # the maximum of row 0 ...
    wf[1234] = wf[3000]                                         # ... tied at a lower id
    xf[1] = np.nan                                              # all logits NaN
    wf[:, :2] = 0.0                                             # ids 0 and 1 of the hidden rows
    xf[:, :2] = 0.0                                             # reach only ids 7, 8 and 9
    xf[2] = 1e20                                                # +inf at id 7, -inf at id 8
    wf[7, 1] = 1e20
    wf[8, 1] = -1e20
    xf[3, 0] = 1e20                                             # -inf at id 9 only
    wf[9, 0] = -1e20
    x = _t(wl.f32_to_bf16_bits(xf), gpu)
    w = _t(wl.f32_to_bf16_bits(wf), gpu)
    wt = llima_amd.lm_head_pack(w) if packed else w
    targets = np.array([1234, 5, 7, 9, 3000, 0], np.int32)
    for ld in ("bf16", "f32"):
        _, _, logits = llima_amd.lm_head_argmax(x, wt, return_logits=True, logit_dtype=ld)
        lg = _np(logits)
        assert np.isinf(lg[3, 9]) and np.isfinite(np.delete(lg[3], 9)).all()
        for t4 in (9, 100):
            targets[3] = t4
            lp, g = llima_amd.lm_head_score(x, wt, torch_i32(targets, gpu), logit_dtype=ld)
            _score_check(_np(lp), _np(g), lg, targets, oracle)
        lp, g = _np(lp), _np(g)
        assert g[0] and np.isnan(lp[1]) and np.isnan(lp[2]) and np.isfinite(lp[3]), (
            ld, g, lp, lg[0, [1234, 3000]], np.argmax(lg[0]), np.nanmax(lg[0]))
        lp1, g1 = llima_amd.lm_head_score(x[0], wt, 3000, logit_dtype=ld)
        elp, eg = oracle.score_logits(lg[0], 3000)
        assert abs(lp1 - elp) <= SCORE_TOL and g1 == eg == False
    with pytest.raises(RuntimeError):
        llima_amd.lm_head_score(x[0], wt, V)
    with pytest.raises(RuntimeError):
        llima_amd.lm_head_score(x, wt, torch_i32([0, 1, V, 3, 4, 5], gpu))
    # through the C ABI: the flag of the out-of-range row, NaN beside it only there
    L = _lib.lib()
    tg = torch_i32([0, 1, -1, 3, 4, V + 5], gpu)
    lp = torch.empty(B, dtype=torch.float64, device=gpu)
    gr = torch.empty(B, dtype=torch.int32, device=gpu)
    if packed:
        n = L.llima_lm_head_score_packed_workspace_bytes(B, H, V)
        ws = torch.empty(n, dtype=torch.uint8, device=gpu)
        st = L.llima_lm_head_score_packed(x.data_ptr(), wt.data.data_ptr(), B, H, V, 0.0,
                                          _lib.LLIMA_BF16, tg.data_ptr(), lp.data_ptr(),
                                          gr.data_ptr(), ws.data_ptr(), n, None)
    else:
        n = L.llima_lm_head_score_workspace_bytes(B, V)
        ws = torch.empty(n, dtype=torch.uint8, device=gpu)
        st = L.llima_lm_head_score(x.data_ptr(), w.data_ptr(), B, H, V, 0.0, _lib.LLIMA_BF16,
                                   tg.data_ptr(), lp.data_ptr(), gr.data_ptr(), ws.data_ptr(), n,
                                   None)
    assert st == 0
    torch.cuda.synchronize()
    lp, gr = _np(lp), _np(gr)
    assert gr[2] == gr[5] == _lib.LLIMA_E_RANGE and np.isnan(lp[2]) and np.isnan(lp[5])
    assert np.isfinite(lp[[0, 3, 4]]).all() and (gr[[0, 1, 3, 4]] >= 0).all()


def test_lm_head_argmax_ties_and_nan(gpu):
    """Equal vocab rows tie: the lower index wins; a NaN logit never wins; a
    row whose logits are all NaN gives id 0 and a NaN value."""
    import llima_amd
    _say("lm head ties / nan")
    rng = np.random.default_rng(5)
    B, H, V = 3, 256, 5000
    x = wl.f32_to_bf16_bits(rng.normal(0, 1, (B, H)).astype(np.float32))
    wf = rng.normal(0, 0.05, (V, H)).astype(np.float32)
    wf[4000] = wl.bf16_bits_to_f32(x[0]) * 0.5               # the maximum of row 0 ...
    wf[1234] = wf[4000]                                      # ... tied at a lower index
    wf[17, 3] = np.nan                                       # a NaN logit in every row
    w = wl.f32_to_bf16_bits(wf)
    xn = x.copy()
    xn[2] = wl.f32_to_bf16_bits(np.full(H, np.nan, np.float32))   # row 2: all NaN
    ids, vals, logits = llima_amd.lm_head_argmax(_t(xn, gpu), _t(w, gpu), return_logits=True)
    ids, vals, logits = _np(ids), _np(vals), _np(logits)
    assert ids[0] == 1234
    assert np.isnan(logits[1, 17]) and ids[1] != 17
    assert ids[2] == 0 and np.isnan(vals[2])
    _lm_head_check(ids[:2], vals[:2], logits[:2], x[:2], w, 0.0)


def test_lm_head_argmax_bf16_ties(gpu):
    """Two vocab rows whose fp32 logits differ but round to the same bf16
    value: with bf16 logits (the reference's precision) the lower index wins;
    with fp32 logits the larger sum wins."""
    import llima_amd
    _say("lm head bf16 ties")
    rng = np.random.default_rng(8)
    B, H, V = 2, 512, 4096
    x = wl.f32_to_bf16_bits(rng.normal(0, 1, (B, H)).astype(np.float32))
    xf = wl.bf16_bits_to_f32(x).astype(np.float64)
    wf = wl.bf16_bits_to_f32(wl.f32_to_bf16_bits(rng.normal(0, 0.02, (V, H)).astype(np.float32)))
    top = wl.bf16_bits_to_f32(wl.f32_to_bf16_bits((wl.bf16_bits_to_f32(x[0]) * 0.05)))
    wf[3000] = top                                           # row 0's maximum ...
    wf[700] = top                                            # ... and a copy at a lower index
    j = int(np.argmax(np.abs(xf[0])))
    sign = 1.0 if xf[0, j] > 0 else -1.0
    bits = wl.f32_to_bf16_bits(wf[3000:3001])
    bits[0, j] = bits[0, j] + (1 if (sign > 0) == (wf[3000, j] >= 0) else -1)   # one bf16 ulp up
    wf[3000] = wl.bf16_bits_to_f32(bits)[0]
    w = wl.f32_to_bf16_bits(wf)
    s = xf @ wl.bf16_bits_to_f32(w).astype(np.float64).T
    assert s[0, 3000] > s[0, 700]
    r = wl.bf16_bits_to_f32(wl.f32_to_bf16_bits(s[0, [700, 3000]].astype(np.float32)))
    assert r[0] == r[1] and s[0].argmax() in (700, 3000)   # equal in bf16
    ids_b, _ = llima_amd.lm_head_argmax(_t(x, gpu), _t(w, gpu), logit_dtype="bf16")
    ids_f, _ = llima_amd.lm_head_argmax(_t(x, gpu), _t(w, gpu), logit_dtype="f32")
    assert int(_np(ids_b)[0]) == 700
    assert int(_np(ids_f)[0]) == 3000
