"""CPU tests that pin the oracle's EAGLE3 draft-tree functions: the heap top-k
(utils.hpp:216-281) on hand-traced tie cases and against a textbook top-k on
tie-free rows, log-softmax (utils.hpp:283-301) against scipy and its closed
forms, and the tree build (language_model_eagle3.cpp:808-1164) on a
hand-derived case and on the invariants every tree must satisfy."""
import math

import numpy as np
import pytest
import scipy.special

from llima_amd import workloads as wl


# ----------------------------------------------------------------- heap top-k
# Each expected output was traced by hand through the reference's heap:
# heapify of the first k, replacement only on a strictly greater value,
# sift-down to the smaller child (the left one on ties), selection sort.
HAND_TRACED = [
    # (row, k, expected indices): a plausible mistake in each rule changes the answer
    ([2, 2, 0, 5], 2, [3, 1]),        # the tie kept is index 1: index 0 was the root when 5 came
    ([1, 3, 3], 1, [1]),              # replacement needs '>': with '>=' the answer is [2]
    ([5, 4, 4, 9], 3, [3, 0, 2]),     # heapify takes the left child on a tie: the right gives [3, 0, 1]
    ([3, 1, 2, 2, 5], 3, [4, 0, 2]),  # index 3 entered and was evicted again
    ([1, 1, 1, 1, 1, 1], 3, [0, 1, 2]),
    ([7], 1, [0]),
]


@pytest.mark.parametrize("row,k,expected", HAND_TRACED)
def test_topk_hand_traced(oracle, row, k, expected):
    idx, val = oracle.topk(np.array([row], np.float32), k)
    assert list(idx[0]) == expected
    assert list(val[0]) == [row[i] for i in expected]


def test_topk_tie_free_rows_are_the_sorted_top_k(oracle):
    rng = np.random.default_rng(3)
    for cols, k in [(5, 5), (40, 1), (1000, 5), (32000, 5), (80, 15), (25, 5), (4096, 32)]:
        x = rng.permutation(cols).astype(np.float32) * np.float32(0.5) - 100
        idx, val = oracle.topk(x[None], k)
        ref = np.argsort(-x, kind="stable")[:k]
        assert list(idx[0]) == list(ref)
        assert (val[0] == x[ref]).all()


def test_topk_values_are_the_top_k_multiset(oracle):
    """With heavy ties the chosen indices are heap-order dependent, but the
    values are always the k largest (with multiplicity), descending, and the
    indices are distinct positions holding those values."""
    rng = np.random.default_rng(4)
    for trial in range(200):
        cols = int(rng.integers(1, 60))
        k = int(rng.integers(1, min(cols, 32) + 1))
        x = rng.integers(-3, 4, size=cols).astype(np.float32)
        if trial % 3 == 0:
            x = wl.bf16_bits_to_f32(wl.f32_to_bf16_bits(x * np.float32(1.37)))
        idx, val = oracle.topk(x[None], k)
        assert len(set(idx[0])) == k
        assert (x[idx[0]] == val[0]).all()
        assert (val[0] == np.sort(x)[::-1][:k]).all()


def test_topk_bf16_rows(oracle):
    rng = np.random.default_rng(5)
    x = rng.normal(0, 3, (3, 5000)).astype(np.float32)
    xb = wl.f32_to_bf16_bits(x)
    i1, v1 = oracle.topk(xb, 5)
    i2, v2 = oracle.topk(wl.bf16_bits_to_f32(xb), 5)
    assert (i1 == i2).all() and (v1 == v2).all()


# ----------------------------------------------------------------- log-softmax
def test_logsoftmax_against_scipy(oracle):
    rng = np.random.default_rng(6)
    for n in [1, 2, 5, 15, 80]:
        for scale in [0.5, 3.0, 20.0]:
            v = (rng.normal(0, scale, n)).astype(np.float32)
            ref = scipy.special.log_softmax(v.astype(np.float64))
            for cr in (False, True):
                got = oracle.logsoftmax(v, cr=cr).astype(np.float64)
                assert np.allclose(got, ref, rtol=1e-6, atol=2e-6), (n, scale, cr)


def test_logsoftmax_closed_forms(oracle):
    for n in [1, 2, 5, 32]:
        v = np.full(n, 3.25, np.float32)
        for cr in (False, True):
            got = oracle.logsoftmax(v, cr=cr)
            assert np.allclose(got, -math.log(n), rtol=1e-7, atol=1e-7)
    # one dominant value: its log-probability is -log(1 + sum exp(others - max))
    v = np.array([10.0, 0.0, 0.0], np.float32)
    assert abs(float(oracle.logsoftmax(v)[0]) + math.log1p(2 * math.exp(-10))) < 1e-6


def test_logsoftmax_libm_and_correctly_rounded_agree(oracle):
    """The C library's expf/logf (the reference's) and exp/log rounded once
    from double (the HIP path's) give shifts log(sum) + max within one ulp of
    each other, so each v - shift differs by at most that ulp plus one ulp of
    the result's rounding (near the maximum the result is small and the
    shift's ulp spans several of its own ulps)."""
    rng = np.random.default_rng(7)
    differ = 0
    for _ in range(3000):
        v = wl.bf16_bits_to_f32(wl.f32_to_bf16_bits(rng.normal(0, 4, 5).astype(np.float32)))
        a = oracle.logsoftmax(v, cr=False).astype(np.float64)
        b = oracle.logsoftmax(v, cr=True).astype(np.float64)
        shift = float(v.max()) + math.log(float(np.exp(v.astype(np.float64) - v.max()).sum()))
        bound = np.spacing(np.float32(abs(shift))) + np.spacing(np.abs(a).astype(np.float32))
        assert (np.abs(a - b) <= bound * 1.0001).all()
        differ += int((a != b).any())
    assert differ < 300          # the two agree bit for bit on most rows


# ----------------------------------------------------------------- tree build
def test_eagle3_tree_hand_derived(oracle):
    """K=2, depth=2, 3 surviving tokens: every step traced by hand."""
    root = np.array([0, 1, 3, 2], np.float32)
    levels = np.array([[[5, 0, 0, 4], [0, 7, 6, 0]]], np.float32)
    d2t = np.zeros(4, np.int32)
    t = oracle.eagle3_tree(root, levels, d2t, K=2, depth=2, total_tokens=3, sample_token=99)
    assert list(t["inputs"][0]) == [2, 3]          # root top-2
    # cumulative scores: [-0.63, -1.63 | -1.63, -2.63]; the tie stays at flat index 1
    assert list(t["parent_rows"][0]) == [0, 0]
    assert list(t["inputs"][1]) == [0, 3]
    assert list(t["tokens"]) == [99, 2, 3, 0]
    assert list(t["position_ids"]) == [0, 1, 1, 2]
    assert t["tree_mask"].tolist() == [[1, 0, 0, 0], [1, 1, 0, 0], [1, 0, 1, 0], [1, 1, 0, 1]]
    assert t["retrieve"].tolist() == [[0, 2, -1], [0, 1, 3]]
    # the draft mask after the level: the parent rows of the old mask plus an identity block
    assert t["masks"][0][:, :4].tolist() == [[1, 0, 1, 0], [1, 0, 0, 1]]


def _tree_invariants(t, K, depth, total):
    N = total + 1
    m = t["tree_mask"].astype(int)
    pos = t["position_ids"]
    assert (np.diag(m) == 1).all() and (m[:, 0] == 1).all()
    assert (np.triu(m, 1) == 0).all()                 # a node's ancestors come before it
    assert (m.sum(1) - 1 == pos).all()
    assert pos.max() <= depth
    ret = t["retrieve"]
    leaves = [r for r in range(N) if not any(m[c, r] for c in range(N) if c != r)]
    assert len(ret) == len(leaves)
    for row, leaf in zip(ret, leaves):
        path = [c for c in row if c >= 0]
        assert path[0] == 0 and path[-1] == leaf
        assert len(path) == pos[leaf] + 1
        assert list(np.flatnonzero(m[leaf])) == path  # the walk back is the ancestor set


@pytest.mark.parametrize("seed", range(6))
def test_eagle3_tree_invariants_random(oracle, seed):
    rng = np.random.default_rng(100 + seed)
    K, depth, total, Vd = 5, 4, 15, 2000
    root = wl.f32_to_bf16_bits(rng.normal(0, 2, Vd).astype(np.float32))
    levels = wl.f32_to_bf16_bits(rng.normal(0, 2, (depth - 1, K, Vd)).astype(np.float32))
    d2t = rng.integers(0, 50000, Vd).astype(np.int32)
    for cr in (True, False):
        t = oracle.eagle3_tree(root, levels, d2t, K, depth, total, 7, cr=cr)
        _tree_invariants(t, K, depth, total)
        # tokens are d2t-mapped draft ids of the nodes, behind the sample token
        assert t["tokens"][0] == 7
        mapped = set(int(i) + int(d2t[i]) for i in range(Vd))
        assert all(int(x) in mapped for x in t["tokens"][1:])
    # the C library's and the correctly rounded exp/log build the same tree here
    a = oracle.eagle3_tree(root, levels, d2t, K, depth, total, 7, cr=True)
    b = oracle.eagle3_tree(root, levels, d2t, K, depth, total, 7, cr=False)
    for key in a:
        assert (a[key] == b[key]).all(), key


# ----------------------------------------------------------------- tree build, literally
# A plain-loop restatement of topk_generate (language_model_eagle3.cpp:808-1164),
# kept in the reference's own shape -- nested lists, the same variable roles, one
# statement per reference step -- as a checker of orc_eagle3_tree.  In particular
# the parent groups of every level come from the topk_cs_index declared before
# the depth loop and filled with 0 .. K-1 (:867-868, :903-909): the selection
# made inside the loop is a new variable of the same name (:953) that hides it,
# so it never reaches the parent groups.  `textbook=True` instead takes them from
# the previous level's selection (EAGLE's published rule), only to show that the
# comparison tells the two apart.
def _heap_topk(row, k):
    """topk<T> (utils.hpp:225-271) for one row, in plain loops."""
    hv = [row[j] for j in range(k)]
    hi = list(range(k))

    def sift_down(root):
        while 2 * root + 1 < k:
            child = 2 * root + 1
            if child + 1 < k and hv[child] > hv[child + 1]:
                child += 1
            if not hv[root] > hv[child]:
                return
            hv[root], hv[child] = hv[child], hv[root]
            hi[root], hi[child] = hi[child], hi[root]
            root = child

    for j in range(k // 2 - 1, -1, -1):
        sift_down(j)
    for j in range(k, len(row)):
        if row[j] > hv[0]:
            hv[0] = row[j]
            hi[0] = j
            sift_down(0)
    vals, idx = [], []
    for a in range(k):
        max_i = a
        for b in range(a + 1, k):
            if hv[b] > hv[max_i]:
                max_i = b
        vals.append(hv[max_i])
        idx.append(hi[max_i])
        hv[max_i] = hv[a]
        hi[max_i] = hi[a]
    return idx, vals


def _logsoftmax_f32(values):
    """logsoftmax<T> (utils.hpp:283-301) in float32 steps, exp and log of the
    float argument evaluated in double and rounded once (the kernels' choice)."""
    f = np.float32
    max_v = f(-np.inf)
    for v in values:
        max_v = max(max_v, f(v))
    s = f(0.0)
    for v in values:
        s = f(s + f(math.exp(float(f(f(v) - max_v)))))
    log_sum = f(f(math.log(float(s))) + max_v)
    return [f(f(v) - log_sum) for v in values]


def _literal_topk_generate(root, levels, d2t, K, depth, total_tokens, sample_token,
                           textbook=False):
    f = np.float32
    topk_index, topk_p_raw = _heap_topk([f(x) for x in root], K)
    scores = _logsoftmax_f32(topk_p_raw)                                       # :820-829
    scores_list = [[scores]]
    parents_list = [[0]]
    ss_token = [[[int(i) + int(d2t[i]) for i in topk_index]]]                   # :834-841
    topk_cs_index = list(range(K))                                             # :867-868
    prev_selection = list(range(K))
    for i in range(depth - 1):
        bias1 = K if i > 0 else 0                                              # :903-909
        bias2 = max(0, i - 1)
        bias = 1 + K * K * bias2 + bias1
        src = prev_selection if textbook else topk_cs_index
        parents_list.append([c + bias for c in src])
        topk_index_d, topk_p_d = [], []
        for r in range(K):                                                     # :914-927
            ix, vals = _heap_topk([f(x) for x in levels[i][r]], K)
            topk_index_d.append(ix)
            topk_p_d.append(_logsoftmax_f32(vals))
        cu_scores = [[f(topk_p_d[r][k] + scores[r]) for k in range(K)] for r in range(K)]
        flat_cu = [cu_scores[r][k] for r in range(K) for k in range(K)]        # :940-945
        inner_topk_cs_index, topk_cs_p = _heap_topk(flat_cu, K)                # :946-954: the
        scores = topk_cs_p                                                     # new variable
        prev_selection = inner_topk_cs_index
        ss_token.append([[int(x) + int(d2t[x]) for x in row] for row in topk_index_d])
        scores_list.append(cu_scores)
    scores_list_flat = [v for entry in scores_list for row in entry for v in row]   # :1040-1048
    ss_token_list = [t for entry in ss_token for row in entry for t in row]
    top_scores_index, _ = _heap_topk(scores_list_flat, total_tokens)          # :1051-1059
    top_scores_index = sorted(top_scores_index)
    draft_tokens = [sample_token] + [ss_token_list[q] for q in top_scores_index]
    draft_parents_flat = [p for entry in parents_list for p in entry]          # :1072-1077
    draft_parents = [draft_parents_flat[q // K] for q in top_scores_index]
    mask_index = []
    for p in draft_parents:                                                    # :1088-1104
        pos = int(np.searchsorted(np.array(top_scores_index), p - 1, side="left"))
        mask_index.append((-1 if p == 0 else pos) + 1)
    N = total_tokens + 1
    tm = [[0] * N for _ in range(N)]
    for r in range(N):
        tm[r][r] = 1
        tm[r][0] = 1
    for q in range(total_tokens):                                              # :1111-1116
        for j in range(N):
            tm[q + 1][j] |= tm[mask_index[q]][j]
    pos_ids = [sum(row) - 1 for row in tm]
    max_depth = max(pos_ids) + 1
    noleaf = set(mask_index)
    leaf_num = total_tokens - (len(noleaf) - 1)
    retrieve = [[-1] * max_depth for _ in range(leaf_num)]
    rid = 0
    for node in range(N):                                                      # :1147-1157
        if node in noleaf:
            continue
        cid = node
        for j in range(pos_ids[node], -1, -1):
            retrieve[rid][j] = cid
            if cid > 0:
                cid = mask_index[cid - 1]
        rid += 1
    return dict(tokens=draft_tokens, tree_mask=tm, position_ids=pos_ids, retrieve=retrieve,
                node_scores=scores_list_flat)


def _as_f32(x):
    return wl.bf16_bits_to_f32(x) if x.dtype == np.uint16 else x


def _same_tree(t, lit):
    return (list(t["tokens"]) == lit["tokens"] and t["tree_mask"].astype(int).tolist() == lit["tree_mask"]
            and list(t["position_ids"]) == lit["position_ids"]
            and t["retrieve"].tolist() == lit["retrieve"])


def test_eagle3_tree_matches_literal_restatement(oracle):
    """orc_eagle3_tree against the plain-loop restatement at the reference's
    shape (K = 5, depth 4, 15 tokens) on 60 random trees, bf16 draft logits.
    The textbook parent rule builds a different tree on a large share of the
    same trees, so this comparison pins the reference's rule."""
    rng = np.random.default_rng(900)
    K, depth, total, Vd = 5, 4, 15, 400
    differs = 0
    for trial in range(60):
        root = wl.f32_to_bf16_bits(rng.normal(0, 2, Vd).astype(np.float32))
        levels = wl.f32_to_bf16_bits(rng.normal(0, 2, (depth - 1, K, Vd)).astype(np.float32))
        d2t = rng.integers(0, 50000, Vd).astype(np.int32)
        t = oracle.eagle3_tree(root, levels, d2t, K, depth, total, 11, cr=True)
        lit = _literal_topk_generate(_as_f32(root), _as_f32(levels), d2t, K, depth, total, 11)
        assert _same_tree(t, lit), trial
        assert (t["node_scores"] == np.array(lit["node_scores"], np.float32)).all(), trial
        txt = _literal_topk_generate(_as_f32(root), _as_f32(levels), d2t, K, depth, total, 11,
                                     textbook=True)
        differs += int(not _same_tree(t, txt))
    assert differs >= 10, differs


def test_eagle3_tree_hand_derived_depth3(oracle):
    """K = 2, depth 3, 6 surviving tokens, traced by hand.  The level-1
    selection is flat (2, 1), not (0, 1), so the two parent rules part at
    level 2: the node of level-2 row 0 hangs, by the reference's rule, off
    parent group entry 0 + 3 (flat node 2), not off the selected continuation
    2 + 3 (flat node 4).
      root [0, 1, 3, 3]: top-2 ids (3, 2) -- the tie keeps heap order -- and
        scores (-ln 2, -ln 2): nodes n0, n1.
      level 1, rows [0, 0, 0, 0] and [0, 10, 0, 0]: ids (0, 1) and (1, 0);
        cumulative n2 = n3 = -2 ln 2, n4 = -ln 2 - 4.54e-5, n5 ~ -10.69;
        the best two are flat 2 then 1: parent rows (1, 0), inputs (1, 1).
      level 2, rows [7, 0, 0, 0] and [0, 0, 0, 0] over scores (n4, n3):
        n6 = n4 - 9.11e-4, n7 ~ -7.69, n8 = n9 = -3 ln 2; best flat (0, 2).
      finish: the top 6 are {n0, n1, n4, n6, n2, n3} (every tie inside);
        parents: n0, n1 -> root; n2, n3 -> n0; n4 -> n1; n6 -> group entry
        3 = flat node 2 -> tree row 3 (the textbook rule: flat node 4 ->
        tree row 5)."""
    root = np.array([0, 1, 3, 3], np.float32)
    levels = np.array([[[0, 0, 0, 0], [0, 10, 0, 0]],
                       [[7, 0, 0, 0], [0, 0, 0, 0]]], np.float32)
    d2t = np.zeros(4, np.int32)
    t = oracle.eagle3_tree(root, levels, d2t, K=2, depth=3, total_tokens=6, sample_token=99)
    assert t["inputs"].tolist() == [[3, 2], [1, 1], [0, 0]]
    assert t["parent_rows"].tolist() == [[1, 0], [0, 1]]
    assert t["masks"][0][:, :4].tolist() == [[0, 1, 1, 0], [1, 0, 0, 1]]
    assert t["masks"][1][:, :6].tolist() == [[0, 1, 1, 0, 1, 0], [1, 0, 0, 1, 0, 1]]
    assert list(t["tokens"]) == [99, 3, 2, 0, 1, 1, 0]
    assert t["tree_mask"].astype(int).tolist() == [
        [1, 0, 0, 0, 0, 0, 0],
        [1, 1, 0, 0, 0, 0, 0],
        [1, 0, 1, 0, 0, 0, 0],
        [1, 1, 0, 1, 0, 0, 0],
        [1, 1, 0, 0, 1, 0, 0],
        [1, 0, 1, 0, 0, 1, 0],
        [1, 1, 0, 1, 0, 0, 1]]
    assert list(t["position_ids"]) == [0, 1, 1, 2, 2, 2, 3]
    assert t["retrieve"].tolist() == [[0, 1, 4, -1], [0, 2, 5, -1], [0, 1, 3, 6]]
    ln2 = math.log(2.0)
    ns = t["node_scores"].astype(np.float64)
    assert np.allclose(ns[[0, 1, 2, 3, 8, 9]], [-ln2, -ln2, -2 * ln2, -2 * ln2, -3 * ln2, -3 * ln2],
                       rtol=0, atol=1e-6)
    assert abs(ns[4] - (-ln2 - math.log1p(math.exp(-10)))) < 1e-6
    assert abs(ns[6] - (ns[4] - math.log1p(math.exp(-7)))) < 1e-6
    # the literal restatement agrees, and the textbook rule does not
    lit = _literal_topk_generate(root, levels, d2t, 2, 3, 6, 99)
    assert _same_tree(t, lit)
    txt = _literal_topk_generate(root, levels, d2t, 2, 3, 6, 99, textbook=True)
    assert txt["tree_mask"][6] == [1, 0, 1, 0, 0, 1, 1]


def _libm_vs_cr_trees(args):
    seed, n = args
    from oracle import oracle as orc
    rng = np.random.default_rng(seed)
    K, depth, total, Vd = 5, 4, 15, 32000
    d2t = np.zeros(Vd, np.int32)
    differ = 0
    for _ in range(n):
        x = (rng.standard_normal((1 + (depth - 1) * K) * Vd, dtype=np.float32) * np.float32(3))
        b = (x.view(np.uint32) >> 16).astype(np.uint16)          # bf16 draft logits
        root, lv = b[:Vd], b[Vd:].reshape(depth - 1, K, Vd)
        a = orc.eagle3_tree(root, lv, d2t, K, depth, total, 7, cr=True)
        c = orc.eagle3_tree(root, lv, d2t, K, depth, total, 7, cr=False)
        differ += int(not all((a[k] == c[k]).all() for k in a if k != "node_scores"))
    return differ


def test_eagle3_tree_libm_and_cr_build_the_same_trees():
    """The reference calls the C library's expf/logf; the kernels round exp
    and log from double.  The scores differ by an ulp now and then; over 10^4
    trees of the reference's shape (K = 5, depth 4, 15 tokens, 32000 bf16 draft
    logits ~ N(0, 3^2), whose top values tie often) count how many trees --
    tokens, masks, positions, retrieve paths, per-level inputs -- differ."""
    from concurrent.futures import ProcessPoolExecutor
    jobs = [(4000 + i, 1250) for i in range(8)]
    with ProcessPoolExecutor(max_workers=8) as ex:
        differ = sum(ex.map(_libm_vs_cr_trees, jobs))
    print(f"trees that differ between libm and correctly rounded exp/log: {differ} of 10000")
    assert differ <= 10
