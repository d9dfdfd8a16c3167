"""GPU parity of the EAGLE3 draft-tree functions against the oracle: the heap
top-k (utils.hpp:216-281) -- indices and their order bit for bit, ties
included -- and the tree build (language_model_eagle3.cpp:808-1164) level by
level: input ids, parent rows, draft masks, then the final tokens, tree mask,
position ids and retrieve indices.  The log-softmax scores feed only index
decisions, so those are compared exactly; the oracle runs with the same
correctly rounded exp/log as the kernels (its C-library variant is checked
against this one on the CPU)."""
import numpy as np
import pytest

from llima_amd import workloads as wl

pytestmark = pytest.mark.gpu


def _say(*a):
    print("[gpu-case]", *a, flush=True)


def _t(a, dev):
    import torch
    if a.dtype == np.uint16:
        return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).to(dev).view(torch.bfloat16)
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _np(t):
    return t.cpu().numpy()


def _rows(kind, rows, cols, rng):
    if kind == "normal":
        return rng.normal(0, 3, (rows, cols)).astype(np.float32)
    if kind == "ties":                                   # a handful of distinct values
        return rng.integers(-6, 7, size=(rows, cols)).astype(np.float32)
    if kind == "ascending":                              # every value enters the heap
        return np.tile(np.arange(cols, dtype=np.float32), (rows, 1))
    if kind == "specials":
        x = rng.normal(0, 2, (rows, cols)).astype(np.float32)
        hit = rng.random((rows, cols)) < 0.01
        x[hit] = rng.choice(np.array([np.nan, -np.inf, np.inf, 0.0, -0.0], np.float32), hit.sum())
        x[0, 1] = np.nan                                 # a NaN among the first k: replay everything
        return x
    raise ValueError(kind)


CASES = [("normal", 5, 32000), ("ties", 5, 32000), ("normal", 1, 1000), ("ties", 15, 80),
         ("ties", 32, 5000), ("normal", 5, 128256), ("ties", 5, 70001), ("ascending", 5, 20000),
         ("specials", 5, 40000), ("specials", 3, 300), ("normal", 7, 7), ("ties", 16, 262144)]


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("kind,k,cols", CASES)
def test_topk_heap_order(gpu, oracle, dtype, kind, k, cols):
    import llima_amd
    _say("topk", kind, k, cols, dtype)
    rng = np.random.default_rng(k * 1000 + cols)
    x = _rows(kind, 4, cols, rng)
    if dtype == "bf16":
        x = wl.f32_to_bf16_bits(x)
    idx, val = llima_amd.topk(_t(x, gpu), k)
    eidx, evals = oracle.topk(x, k)
    assert (_np(idx) == eidx).all(), (_np(idx)[:2], eidx[:2])
    g = _np(val)
    assert ((g.view(np.uint32) == evals.view(np.uint32)) | (np.isnan(g) & np.isnan(evals))).all()


def test_topk_strided_rows(gpu, oracle):
    import llima_amd
    _say("topk strided")
    rng = np.random.default_rng(2)
    x = rng.integers(-5, 6, size=(3, 5003)).astype(np.float32)
    xt = _t(x, gpu)[:, 1:5000]
    idx, _ = llima_amd.topk(xt, 5)
    assert (_np(idx) == oracle.topk(np.ascontiguousarray(x[:, 1:5000]), 5)[0]).all()


def _run_tree(gpu, oracle, root, levels, d2t, K, depth, total, sample):
    import llima_amd
    tree = llima_amd.Eagle3DraftTree(_t(d2t, gpu), topk=K, depth=depth)
    e = oracle.eagle3_tree(root, levels, d2t, K, depth, total, sample, cr=True)
    ids = tree.begin(_t(root, gpu))
    assert (_np(ids) == e["inputs"][0]).all()
    for lv in range(1, depth):
        ids, prow, mask = tree.grow(_t(levels[lv - 1], gpu))
        assert (_np(ids) == e["inputs"][lv]).all(), lv
        assert (_np(prow) == e["parent_rows"][lv - 1]).all(), lv
        assert (_np(mask) == e["masks"][lv - 1][:, :K * (lv + 1)]).all(), lv
    # the node scores themselves (log-softmax plus the parent's score), to 1e-5
    # relative: the kernels and this oracle round exp/log the same way, so they
    # agree far closer than that
    ns = _np(tree.node_scores())
    assert ns.shape == e["node_scores"].shape
    assert np.allclose(ns, e["node_scores"], rtol=1e-5, atol=1e-6, equal_nan=True)
    out = tree.finish(total, sample)
    assert (_np(out["tokens"]) == e["tokens"]).all()
    assert (_np(out["tree_mask"]) == e["tree_mask"]).all()
    assert (_np(out["position_ids"]) == e["position_ids"]).all()
    assert _np(out["retrieve"]).tolist() == e["retrieve"].tolist()
    return e


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
@pytest.mark.parametrize("seed", range(3))
def test_eagle3_tree_llama3_draft(gpu, oracle, dtype, seed):
    """The reference's EAGLE3 shape: K = 5, depth 4, 15 draft tokens, a 32000-id
    draft vocabulary mapped to the 128256-id target vocabulary."""
    _say("eagle3 tree", dtype, seed)
    rng = np.random.default_rng(500 + seed)
    K, depth, total, Vd = 5, 4, 15, 32000
    root = rng.normal(0, 3, Vd).astype(np.float32)
    levels = rng.normal(0, 3, (depth - 1, K, Vd)).astype(np.float32)
    if dtype == "bf16":
        root, levels = wl.f32_to_bf16_bits(root), wl.f32_to_bf16_bits(levels)
    d2t = (np.sort(rng.choice(128256, Vd, replace=False)) - np.arange(Vd)).astype(np.int32)
    _run_tree(gpu, oracle, root, levels, d2t, K, depth, total, sample=int(rng.integers(0, 128256)))


def test_eagle3_tree_ties_and_shapes(gpu, oracle):
    """Integer-valued logits (ties in the heaps and in the cumulative scores),
    identical rows, and other (K, depth, total) shapes."""
    rng = np.random.default_rng(77)
    for K, depth, total, Vd in [(5, 4, 15, 32000), (2, 2, 3, 64), (8, 5, 32, 9000), (1, 3, 2, 100),
                                (5, 1, 4, 500), (32, 2, 32, 4096)]:
        _say("eagle3 tree ties", K, depth, total, Vd)
        root = rng.integers(-3, 4, Vd).astype(np.float32)
        levels = rng.integers(-3, 4, (max(depth - 1, 1), K, Vd)).astype(np.float32)[:depth - 1]
        if depth > 1 and K > 1:
            levels[0, 1] = levels[0, 0]                  # identical rows
        d2t = rng.integers(0, 1000, Vd).astype(np.int32)
        _run_tree(gpu, oracle, wl.f32_to_bf16_bits(root), wl.f32_to_bf16_bits(levels)
                  if depth > 1 else np.zeros((0, K, Vd), np.uint16), d2t, K, depth, total, 3)
