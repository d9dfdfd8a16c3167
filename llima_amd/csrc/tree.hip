// tree.hip -- EAGLE3 draft-tree construction (gfx950).
//
// Restates on device memory the selection side of the reference's EAGLE3
// drafting (sima-neat/llima, paths relative to that repository):
//   topk<T>          sima_lmm/devkit/cpp/utils.hpp:216-281   heap top-k, its exact output order
//   logsoftmax<T>    sima_lmm/devkit/cpp/utils.hpp:283-301
//   topk_generate    sima_lmm/devkit/cpp/language_model_eagle3.cpp:808-1164
//   searchsorted     sima_lmm/devkit/cpp/eagle_helpers.hpp:197-214
// The draft model's forward passes between tree levels are the caller's.
//
// Heap top-k.  The reference keeps a min-heap of k values; its output order,
// and which of several values equal to the k-th it keeps, depend on the order
// of its insertions.  So the heap is replayed exactly: lane i of wavefront 0
// holds heap slot i, and each insertion and sift-down runs as the reference's
// does (uniform control flow, readlane/writelane).  What runs in parallel is
// finding the few values that can enter the heap.  Value j >= k enters iff it
// exceeds the root, which is then the k-th largest of values 0..j-1 (NaN never
// enters; a NaN among the first k values switches to replaying every value).
// The row is read in tiles of 16384 values; thread t of 1024 holds 16
// consecutive values of a tile.  The k-th largest of the 16 values of each
// earlier thread, and the root after the previous tile, are each at most that
// root, so a value not above their maximum cannot enter and is skipped.  The
// rest (a few hundred of a 32000-value row) are compacted in index order and
// replayed 64 at a time: a ballot finds the next one above the root.
//
// log-softmax.  The reference's float arithmetic (maximum, float sum of exp in
// index order, log(sum) + max, subtraction) with exp and log evaluated in
// double and rounded once to float: the correctly rounded values, which the C
// library's expf/logf return on all but a few arguments.
#include "common.hpp"
#include "../../include/llima_sampler.h"

namespace llima {

#define TK_WG 1024                        // threads of a top-k workgroup
#define TK_WAVES (TK_WG / 64)
#define TK_EPT 16                         // consecutive values per thread and tile
#define TK_TILE (TK_WG * TK_EPT)          // values per tile
#define TK_PAD(e) ((e) + ((e) >> 4))      // LDS slot of tile element e (conflict-free rows)
#define TK_CAP 4096                       // candidates of a tile held for the replay
#define TK_MAXK 32                        // the reference's limit on k
#define TREE_WG 256
#define TREE_MAX_NODES 16384              // node scores the finish stages in LDS

// ------------------------------------------------------------------ tree state layout
// A caller-owned device buffer that persists from begin to finish: the current
// level's scores, the parent groups, every node's score and token, the draft
// attention mask, and the per-row top-k of the level being grown.
struct TreeLayout {
    size_t score, parent, node_score, node_tok, mask, row_idx, row_val, total;
};

__host__ __device__ inline size_t tree_take(size_t* o, size_t bytes) {
    const size_t r = *o;
    *o += (bytes + 255) & ~(size_t)255;
    return r;
}

__host__ __device__ inline TreeLayout tree_layout(int K, int depth) {
    TreeLayout L;
    size_t o = 0;
    const size_t nodes = (size_t)K + (size_t)(depth - 1) * K * K;
    L.score = tree_take(&o, 4 * (size_t)K);
    L.parent = tree_take(&o, 4 * (1 + (size_t)(depth - 1) * K));
    L.node_score = tree_take(&o, 4 * nodes);
    L.node_tok = tree_take(&o, 4 * nodes);
    L.mask = tree_take(&o, 4 * (size_t)K * K * depth);
    L.row_idx = tree_take(&o, 4 * (size_t)K * K);
    L.row_val = tree_take(&o, 4 * (size_t)K * K);
    L.total = o;
    return L;
}

struct TreeParams {
    const void* x;           // top-k rows / level logits / root row
    int64_t row_stride;
    int32_t rows, cols, k;
    int32_t vec;             // rows 16-byte aligned: the fast top-k reads them with 16-byte loads
    int32_t* out_idx;        // [rows][k]
    float* out_val;          // [rows][k]
    const int32_t* d2t;
    char* state;
    int32_t K, depth, level, total, sample_token;
    int32_t* out_inputs;     // [K]
    int32_t* out_prow;       // [K]
    float* out_mask;         // [K][K * (level + 1)]
    int32_t* out_tokens;     // [N]
    float* out_tree_mask;    // [N][N]
    int32_t* out_pos;        // [N]
    int32_t* out_retrieve;   // [N][N]
    int32_t* out_dims;       // [2]
};

template <typename T>
__device__ __forceinline__ T* st(const TreeParams& P, size_t off) { return (T*)(P.state + off); }

// ------------------------------------------------------------------ helpers
template <typename TL>
__device__ __forceinline__ float tk_load(const TL* p, int64_t i);
template <>
__device__ __forceinline__ float tk_load<float>(const float* p, int64_t i) { return p[i]; }
template <>
__device__ __forceinline__ float tk_load<uint16_t>(const uint16_t* p, int64_t i) {
    return bf16_bits_to_f32(p[i]);
}

__device__ __forceinline__ float rdl_f(float v, int l) {
    return __uint_as_float((uint32_t)__builtin_amdgcn_readlane((int)__float_as_uint(v), l));
}
// Lane l of v replaced by the uniform x (a compare and a select).
__device__ __forceinline__ float wrl_f(float v, float x, int l) {
    return (int)lane_id() == l ? x : v;
}
__device__ __forceinline__ int32_t rdl_i(int32_t v, int l) { return __builtin_amdgcn_readlane(v, l); }
__device__ __forceinline__ int32_t wrl_i(int32_t v, int32_t x, int l) {
    return (int)lane_id() == l ? x : v;
}

__device__ __forceinline__ float exp_cr(float x) { return (float)exp((double)x); }
__device__ __forceinline__ float log_cr(float x) { return (float)log((double)x); }

// Inclusive maximum over lanes 0..l (keys; 0 is the identity).
__device__ __forceinline__ uint32_t wave_incl_max_u32(uint32_t v) {
    auto mx = [](uint32_t a, uint32_t b) { return a > b ? a : b; };
    v = mx(v, dpp32<DPP_ROW_SHR(1), 0xF, true>(0u, v));
    v = mx(v, dpp32<DPP_ROW_SHR(2), 0xF, true>(0u, v));
    v = mx(v, dpp32<DPP_ROW_SHR(4), 0xF, true>(0u, v));
    v = mx(v, dpp32<DPP_ROW_SHR(8), 0xF, true>(0u, v));
    v = mx(v, dpp32<DPP_ROW_BCAST15, 0xA, false>(0u, v));
    v = mx(v, dpp32<DPP_ROW_BCAST31, 0xC, false>(0u, v));
    return v;
}

// The k-th largest key (NaN: 0) of 16 values (k <= 16; 0 otherwise): a
// bitonic sorting network (descending) and a select.
__device__ __forceinline__ uint32_t kth_of_16(const float* vals, int k) {
    uint32_t v[TK_EPT];
#pragma unroll
    for (int i = 0; i < TK_EPT; ++i) v[i] = vals[i] == vals[i] ? f32_key(vals[i]) : 0u;
#pragma unroll
    for (int size = 2; size <= TK_EPT; size <<= 1) {
#pragma unroll
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
#pragma unroll
            for (int i = 0; i < TK_EPT; ++i) {
                const int j = i ^ stride;
                if (j > i) {
                    const bool desc = (i & size) == 0;
                    const uint32_t hi = v[i] > v[j] ? v[i] : v[j], lo = v[i] > v[j] ? v[j] : v[i];
                    v[i] = desc ? hi : lo;
                    v[j] = desc ? lo : hi;
                }
            }
        }
    }
    uint32_t r = 0;
#pragma unroll
    for (int i = 0; i < TK_EPT; ++i) r = i == k - 1 ? v[i] : r;
    return r;
}

struct TopkShared {
    float tile[TK_PAD(TK_TILE)];
    float cv[TK_CAP];
    int32_t ci[TK_CAP];
    uint32_t wpart[TK_WAVES + 1];          // + the fast path's heap root
    uint32_t init_k[TK_MAXK];
    uint32_t wcnt[TK_WAVES];
    float carry;             // the heap root after the previous tile
    uint32_t nan_init;       // a NaN among the first k values: replay every value
    float res_v[TK_MAXK];
    int32_t res_i[TK_MAXK];
};

template <typename TL>
__device__ __forceinline__ void tk_fetch(const TL* rowp, int base, int cols, float (&r)[TK_EPT]) {
#pragma unroll
    for (int i = 0; i < TK_EPT; ++i) {
        const int j = base + i * TK_WG + (int)threadIdx.x;
        r[i] = j < cols ? tk_load<TL>(rowp, j) : __builtin_nanf("");
    }
}

// Sift-down from slot `node` of the heap held by this wavefront (slot i in lane i).
__device__ __forceinline__ void heap_sift(float& hv, int32_t& hi, int node, int k) {
    for (;;) {
        int c = 2 * node + 1;
        if (c >= k) return;
        float vc = rdl_f(hv, c);
        if (c + 1 < k) {
            const float vr = rdl_f(hv, c + 1);
            if (vc > vr) { ++c; vc = vr; }
        }
        const float vn = rdl_f(hv, node);
        if (!(vn > vc)) return;
        const int32_t in_ = rdl_i(hi, node), ic = rdl_i(hi, c);
        hv = wrl_f(hv, vc, node);
        hv = wrl_f(hv, vn, c);
        hi = wrl_i(hi, ic, node);
        hi = wrl_i(hi, in_, c);
        node = c;
    }
}

// topk<T> of one row (utils.hpp:225-281) -> sh.res_v / sh.res_i [k], in the
// reference's output order, for any k <= 32 (readlane heap).  Every thread of
// the 1024 calls it.
template <typename TL>
__device__ __forceinline__ void topk_row_generic(const TL* rowp, int cols, int k, TopkShared& sh) {
    const int t = (int)threadIdx.x, lane = t & 63, wave = t >> 6;
    const int ntiles = (cols + TK_TILE - 1) / TK_TILE;
    if (t == 0) sh.nan_init = 0;
    __syncthreads();
    if (t < k) {
        const float v = tk_load<TL>(rowp, t);
        if (v != v) sh.nan_init = 1u;
    }
    float nxt[TK_EPT];
    tk_fetch<TL>(rowp, 0, cols, nxt);
    __syncthreads();
    const bool every = sh.nan_init != 0;
    float hv = 0.0f;                     // wavefront 0: heap slot `lane`
    int32_t hi = 0;
    for (int ti = 0; ti < ntiles; ++ti) {
        const int base = ti * TK_TILE;
#pragma unroll
        for (int i = 0; i < TK_EPT; ++i) sh.tile[TK_PAD(i * TK_WG + t)] = nxt[i];
        __syncthreads();
        if (ti + 1 < ntiles) tk_fetch<TL>(rowp, base + TK_TILE, cols, nxt);   // in flight meanwhile
        // ---- the candidates of this tile (thread t: values t*16 .. t*16+15, read
        //      from LDS each time they are needed, which keeps registers free)
        const float* seg = sh.tile + t * (TK_EPT + 1);                 // = TK_PAD(t * 16)
        uint32_t kk = kth_of_16(seg, k);
        uint32_t inc = wave_incl_max_u32(kk);
        uint32_t exc = (uint32_t)__shfl_up((int)inc, 1);
        exc = lane == 0 ? 0u : exc;
        if (lane == 63) sh.wpart[wave] = inc;
        __syncthreads();
        uint32_t lk = exc;
        for (int w = 0; w < wave; ++w) lk = sh.wpart[w] > lk ? sh.wpart[w] : lk;
        if (ti > 0) {
            const uint32_t ck = f32_key(sh.carry);
            lk = ck > lk ? ck : lk;
        }
        lk = lk > LLIMA_KEY_NEG_INF ? lk : LLIMA_KEY_NEG_INF;
        const float bound = key_f32(lk);
        uint32_t mine = 0;
#pragma unroll
        for (int q = 0; q < TK_EPT; ++q) {
            const int j = base + t * TK_EPT + q;
            mine += (j >= k && j < cols && seg[q] > bound) ? 1u : 0u;
        }
        const uint32_t winc = wave_incl_scan_u32(mine);
        if (lane == 63) sh.wcnt[wave] = winc;
        __syncthreads();
        uint32_t off = winc - mine, total = 0;
        for (int w = 0; w < TK_WAVES; ++w) {
            off += w < wave ? sh.wcnt[w] : 0u;
            total += sh.wcnt[w];
        }
        const bool all_values = every || total > TK_CAP;
        if (!all_values) {
#pragma unroll
            for (int q = 0; q < TK_EPT; ++q) {
                const int j = base + t * TK_EPT + q;
                if (j >= k && j < cols && seg[q] > bound) {
                    sh.cv[off] = seg[q];
                    sh.ci[off] = j;
                    ++off;
                }
            }
        }
        __syncthreads();
        // ---- the replay (wavefront 0)
        if (wave == 0) {
            if (ti == 0) {
                hv = lane < k ? sh.tile[TK_PAD(lane)] : 0.0f;
                hi = lane;
                for (int j = k / 2 - 1; j >= 0; --j) heap_sift(hv, hi, j, k);
            }
            const int n = all_values ? (cols - base < TK_TILE ? cols - base : TK_TILE) : (int)total;
            const int start = all_values && ti == 0 ? k : 0;
            float root = rdl_f(hv, 0);
            for (int g = start; g < n; g += 64) {
                const int e = g + lane;
                float x = __builtin_nanf("");
                int32_t xj = 0;
                if (e < n) {
                    x = all_values ? sh.tile[TK_PAD(e)] : sh.cv[e];
                    xj = all_values ? base + e : sh.ci[e];
                }
                uint64_t m = ballot(x > root);
                while (m) {
                    const int L = __builtin_ctzll(m);
                    const float xv = rdl_f(x, L);
                    hv = wrl_f(hv, xv, 0);
                    hi = wrl_i(hi, rdl_i(xj, L), 0);
                    heap_sift(hv, hi, 0, k);
                    root = rdl_f(hv, 0);
                    const uint64_t after = L == 63 ? 0ull : (~0ull << (L + 1));
                    m = ballot(x > root) & after;
                }
            }
            if (lane == 0) sh.carry = root;
        }
        __syncthreads();
    }
    // ---- output: the reference's selection sort over the heap slots
    if (wave == 0) {
        float rv = 0.0f;
        int32_t ri = 0;
        for (int a = 0; a < k; ++a) {
            int m = a;
            float vm = rdl_f(hv, a);
            for (int b = a + 1; b < k; ++b) {
                const float vb = rdl_f(hv, b);
                if (vb > vm) { m = b; vm = vb; }
            }
            rv = wrl_f(rv, vm, a);
            ri = wrl_i(ri, rdl_i(hi, m), a);
            hv = wrl_f(hv, rdl_f(hv, a), m);
            hi = wrl_i(hi, rdl_i(hi, a), m);
        }
        if (lane < k) { sh.res_v[lane] = rv; sh.res_i[lane] = ri; }
    }
    __syncthreads();
}

// ------------------------------------------------------------------ fast heap top-k (k <= 8)
// The same replay with the heap in registers: every lane of wavefront 0 holds
// the same copy (keys and ids, uniform control flow, uniform indices), so a
// sift-down step is a few register moves and compares instead of readlane
// round trips.  Keys compare as the floats do (order-preserving, -0 folded
// onto +0; no NaN is ever in the heap on this path).  Each thread's k-th
// largest key comes from a sorted list of its TK_FAST_K largest (one max/min
// pair per list entry and value).
#define TK_FAST_K 8
#define TK_VPT 16
#define TK_FTILE (TK_WG * TK_VPT)

// Sift-down from slot NODE of a heap of KC keys: indices are compile-time
// constants, so the heap stays in registers.
template <int KC, int NODE>
__device__ __forceinline__ void uheap_sift(uint32_t (&hk)[TK_FAST_K], int32_t (&hi)[TK_FAST_K]) {
    constexpr int C = 2 * NODE + 1;
    if constexpr (C < KC) {
        bool right = false;
        uint32_t vc = hk[C];
        if constexpr (C + 1 < KC) {
            right = hk[C] > hk[C + 1];
            vc = right ? hk[C + 1] : vc;
        }
        const uint32_t vn = hk[NODE];
        if (vn > vc) {
            const int32_t in_ = hi[NODE];
            if constexpr (C + 1 < KC) {
                if (right) {
                    hk[NODE] = vc; hi[NODE] = hi[C + 1]; hk[C + 1] = vn; hi[C + 1] = in_;
                    uheap_sift<KC, C + 1>(hk, hi);
                    return;
                }
            }
            hk[NODE] = vc; hi[NODE] = hi[C]; hk[C] = vn; hi[C] = in_;
            uheap_sift<KC, C>(hk, hi);
        }
    }
}

// The reference's heapify of the first KC values: sift-down from KC/2 - 1 to 0.
template <int KC, int J>
__device__ __forceinline__ void uheap_build(uint32_t (&hk)[TK_FAST_K], int32_t (&hi)[TK_FAST_K]) {
    if constexpr (J >= 0) {
        uheap_sift<KC, J>(hk, hi);
        uheap_build<KC, J - 1>(hk, hi);
    }
}

// The raw bits of TK_VPT values from id i0 (ids at or past cols: a NaN
// pattern, which has no key), 16-byte loads when vec and the block lies in
// the row, else one value per load.
template <typename TL>
__device__ __forceinline__ void tk_raw(const TL* rowp, int i0, int cols, bool vec,
                                       llima_u32x4 (&q)[TK_VPT * sizeof(TL) / 16]) {
    constexpr int EPL = 16 / sizeof(TL);
    constexpr int NQ = TK_VPT / EPL;
    if (vec && i0 + TK_VPT <= cols) {
#pragma unroll
        for (int j = 0; j < NQ; ++j) q[j] = __builtin_nontemporal_load((const llima_u32x4*)(rowp + i0 + j * EPL));
    } else {
#pragma unroll
        for (int j = 0; j < NQ; ++j) {
            uint32_t w[4] = {0u, 0u, 0u, 0u};
#pragma unroll
            for (int e = 0; e < EPL; ++e) {
                const int i = i0 + j * EPL + e;
                uint32_t b;
                if constexpr (sizeof(TL) == 4) b = i < cols ? __float_as_uint(tk_load<TL>(rowp, i)) : 0x7FC00000u;
                else b = i < cols ? (uint32_t)((const uint16_t*)rowp)[i] : 0x7FC0u;
                if constexpr (sizeof(TL) == 4) w[e] = b;
                else w[e >> 1] |= b << ((e & 1) * 16);
            }
            q[j] = llima_u32x4{w[0], w[1], w[2], w[3]};
        }
    }
}

// The keys of a block's raw bits (a NaN: key 0, never a candidate).
template <typename TL>
__device__ __forceinline__ void tk_keys(const llima_u32x4 (&q)[TK_VPT * sizeof(TL) / 16],
                                        uint32_t (&kk)[TK_VPT]) {
    constexpr int EPL = 16 / sizeof(TL);
#pragma unroll
    for (int j = 0; j < TK_VPT / EPL; ++j) {
        const uint32_t w4[4] = {q[j].x, q[j].y, q[j].z, q[j].w};
#pragma unroll
        for (int e = 0; e < EPL; ++e) {
            const float f = sizeof(TL) == 4 ? __uint_as_float(w4[e])
                                            : __uint_as_float((e & 1) ? (w4[e >> 1] & 0xFFFF0000u)
                                                                      : (w4[e >> 1] << 16));
            kk[j * EPL + e] = f == f ? f32_key(f) : 0u;
        }
    }
}

// v into the descending list L[0, KC) of the KC largest keys (with multiplicity).
template <int KC>
__device__ __forceinline__ void tk_list_put(uint32_t (&L)[TK_FAST_K], uint32_t v) {
#pragma unroll
    for (int i = KC - 1; i > 0; --i) {
        const uint32_t lo = L[i - 1] < v ? L[i - 1] : v;
        L[i] = L[i] > lo ? L[i] : lo;
    }
    L[0] = L[0] > v ? L[0] : v;
}

// Rows are taken in tiles of TK_FTILE values; thread t holds the block of
// TK_VPT values at t TK_VPT.  A value after the first k is a candidate when it
// exceeds every earlier block's k-th largest key, the heap root after the
// earlier tiles, and the k-th largest key of its own block before it: each is
// at most the heap root when the value arrives.  The candidates, in id order,
// are replayed by wavefront 0.
template <typename TL, int KC>
__device__ __forceinline__ void topk_row_fast(const TL* rowp, int cols, bool vec, TopkShared& sh) {
    constexpr int k = KC;
    constexpr int NQ = TK_VPT * (int)sizeof(TL) / 16;
    const int t = (int)threadIdx.x, lane = t & 63, wave = t >> 6;
    uint32_t hk[TK_FAST_K];                // wavefront 0: the heap, every lane alike
    int32_t hi[TK_FAST_K];
#pragma unroll
    for (int i = 0; i < TK_FAST_K; ++i) { hk[i] = 0u; hi[i] = 0; }
    uint32_t carry = 0u;                   // the heap root after the earlier tiles
    for (int base = 0; base < cols; base += TK_FTILE) {
        const int ib = base + t * TK_VPT;
        llima_u32x4 q[NQ];
        tk_raw<TL>(rowp, ib, cols, vec, q);
        // ---- the block's k-th largest key, the bound from the earlier blocks
        uint32_t kth;
        {
            uint32_t kk[TK_VPT], L[TK_FAST_K];
            tk_keys<TL>(q, kk);
#pragma unroll
            for (int i = 0; i < TK_FAST_K; ++i) L[i] = 0u;
#pragma unroll
            for (int e = 0; e < TK_VPT; ++e) tk_list_put<KC>(L, kk[e]);
            kth = L[k - 1];
        }
        const uint32_t inc = wave_incl_max_u32(kth);
        uint32_t bound = (uint32_t)__shfl_up((int)inc, 1);
        bound = lane == 0 ? 0u : bound;
        bound = bound > carry ? bound : carry;
        if (lane == 63) sh.wpart[wave] = inc;
        __syncthreads();
        for (int w = 0; w < TK_WAVES; ++w) bound = w < wave && sh.wpart[w] > bound ? sh.wpart[w] : bound;
        // ---- candidates: above the bound and the block's own running k-th key
        uint32_t cmask = 0;
        {
            uint32_t kk[TK_VPT], L[TK_FAST_K];
            tk_keys<TL>(q, kk);
#pragma unroll
            for (int i = 0; i < TK_FAST_K; ++i) L[i] = 0u;
#pragma unroll
            for (int e = 0; e < TK_VPT; ++e) {
                const uint32_t thr = L[k - 1] > bound ? L[k - 1] : bound;
                cmask |= (ib + e >= k && kk[e] > thr) ? (1u << e) : 0u;
                tk_list_put<KC>(L, kk[e]);
            }
        }
        const uint32_t cnt = (uint32_t)__popc(cmask);
        const uint32_t ci = wave_incl_scan_u32(cnt);
        if (lane == 63) sh.wcnt[wave] = ci;
        if (base == 0 && t == 0) {                          // the first k values start the heap
            uint32_t kk[TK_VPT];
            tk_keys<TL>(q, kk);
#pragma unroll
            for (int e = 0; e < TK_FAST_K; ++e)
                if (e < k) sh.init_k[e] = kk[e];
        }
        __syncthreads();
        uint32_t off = ci - cnt, total = 0;
        for (int w = 0; w < TK_WAVES; ++w) {
            off += w < wave ? sh.wcnt[w] : 0u;
            total += sh.wcnt[w];
        }
        if (wave == 0 && base == 0) {
            // readfirstlane: the heap is uniform, so the compiler keeps it in
            // scalar registers and sifts with scalar compares and branches
#pragma unroll
            for (int i = 0; i < k; ++i) {
                hk[i] = (uint32_t)__builtin_amdgcn_readfirstlane((int)sh.init_k[i]);
                hi[i] = i;
            }
            uheap_build<KC, KC / 2 - 1>(hk, hi);
        }
        // ---- rounds of TK_CAP candidates: staged in LDS, replayed by wavefront 0
        for (uint32_t r0 = 0; r0 < total; r0 += TK_CAP) {
            if (r0) __syncthreads();                        // wavefront 0 read the LDS
            {
                uint32_t kk[TK_VPT];
                tk_keys<TL>(q, kk);
                uint32_t o = off;
#pragma unroll
                for (int e = 0; e < TK_VPT; ++e) {
                    const bool c = (cmask >> e) & 1u;
                    if (c && o >= r0 && o < r0 + TK_CAP) {
                        sh.cv[o - r0] = __uint_as_float(kk[e]);    // the key's bits
                        sh.ci[o - r0] = ib + e;
                    }
                    o += c ? 1u : 0u;
                }
            }
            __syncthreads();
            if (wave == 0) {
                const uint32_t n = total - r0 < TK_CAP ? total - r0 : TK_CAP;
                uint32_t root = hk[0];
                for (uint32_t g = 0; g < n; g += 64) {
                    const uint32_t e = g + (uint32_t)lane;
                    const uint32_t x = e < n ? __float_as_uint(sh.cv[e]) : 0u;
                    const int32_t xj = e < n ? sh.ci[e] : 0;
                    uint64_t m = ballot(x > root);
                    while (m) {
                        const int Ln = __builtin_ctzll(m);
                        hk[0] = (uint32_t)__builtin_amdgcn_readlane((int)x, Ln);
                        hi[0] = __builtin_amdgcn_readlane(xj, Ln);
                        uheap_sift<KC, 0>(hk, hi);
                        root = hk[0];
                        const uint64_t after = Ln == 63 ? 0ull : (~0ull << (Ln + 1));
                        m = ballot(x > root) & after;
                    }
                }
            }
        }
        if (base + TK_FTILE < cols) {
            if (wave == 0 && lane == 0) sh.wpart[TK_WAVES] = hk[0];
            __syncthreads();
            carry = sh.wpart[TK_WAVES];                     // the k-th largest key so far
        }
    }
    // output: the reference's selection sort over the heap slots; the values
    // are the row's own (their bits, -0 included)
    if (wave == 0) {
        int32_t ri = 0;
#pragma unroll
        for (int a = 0; a < k; ++a) {
            // the first slot holding the largest of slots a .. k-1, then slot a's
            // entry moved into it (every index a select over the fixed slots)
            uint32_t vm = hk[a];
            int32_t im = hi[a];
            int m = a;
#pragma unroll
            for (int b = a + 1; b < k; ++b) {
                const bool gt = hk[b] > vm;
                vm = gt ? hk[b] : vm;
                im = gt ? hi[b] : im;
                m = gt ? b : m;
            }
            ri = lane == a ? im : ri;
#pragma unroll
            for (int b = a + 1; b < k; ++b) {
                hk[b] = m == b ? hk[a] : hk[b];
                hi[b] = m == b ? hi[a] : hi[b];
            }
        }
        if (lane < k) {
            sh.res_i[lane] = ri;
            sh.res_v[lane] = tk_load<TL>(rowp, ri);
        }
    }
    __syncthreads();
}

// topk<T> of one row (utils.hpp:225-281) -> sh.res_v / sh.res_i [k], in the
// reference's output order.  Every thread of the 1024 calls it.  k <= 8 with
// no NaN among the first k values takes the register heap.
template <typename TL>
__device__ __forceinline__ void topk_row(const TL* rowp, int cols, int k, bool vec, TopkShared& sh) {
    if (threadIdx.x == 0) sh.nan_init = 0;
    __syncthreads();
    if ((int)threadIdx.x < k) {
        const float v = tk_load<TL>(rowp, threadIdx.x);
        if (v != v) sh.nan_init = 1u;
    }
    __syncthreads();
    if (!sh.nan_init) {
        switch (k) {
            case 1: topk_row_fast<TL, 1>(rowp, cols, vec, sh); return;
            case 2: topk_row_fast<TL, 2>(rowp, cols, vec, sh); return;
            case 3: topk_row_fast<TL, 3>(rowp, cols, vec, sh); return;
            case 4: topk_row_fast<TL, 4>(rowp, cols, vec, sh); return;
            case 5: topk_row_fast<TL, 5>(rowp, cols, vec, sh); return;
            case 6: topk_row_fast<TL, 6>(rowp, cols, vec, sh); return;
            case 7: topk_row_fast<TL, 7>(rowp, cols, vec, sh); return;
            case 8: topk_row_fast<TL, 8>(rowp, cols, vec, sh); return;
            default: break;
        }
    }
    topk_row_generic<TL>(rowp, cols, k, sh);
}

// ------------------------------------------------------------------ kernels
template <typename TL>
__global__ __launch_bounds__(TK_WG) void topk_rows_kernel(TreeParams P) {
    __shared__ TopkShared sh;
    const int r = (int)blockIdx.x;
    topk_row<TL>((const TL*)P.x + (size_t)r * P.row_stride, P.cols, P.k, P.vec != 0, sh);
    if ((int)threadIdx.x < P.k) {
        P.out_idx[(size_t)r * P.k + threadIdx.x] = sh.res_i[threadIdx.x];
        P.out_val[(size_t)r * P.k + threadIdx.x] = sh.res_v[threadIdx.x];
    }
}

// topk<float> of n values in LDS by one thread (the reference's heap, in LDS
// slots hv/hi), into out_i / out_v.
__device__ void heap_topk_serial(const float* x, int n, int k, float* hv, int32_t* hi,
                                 int32_t* out_i, float* out_v) {
    for (int j = 0; j < k; ++j) { hv[j] = x[j]; hi[j] = j; }
    auto sift = [&](int node) {
        for (;;) {
            int c = 2 * node + 1;
            if (c >= k) return;
            if (c + 1 < k && hv[c] > hv[c + 1]) ++c;
            if (!(hv[node] > hv[c])) return;
            const float tv = hv[node]; hv[node] = hv[c]; hv[c] = tv;
            const int32_t ti = hi[node]; hi[node] = hi[c]; hi[c] = ti;
            node = c;
        }
    };
    for (int j = k / 2 - 1; j >= 0; --j) sift(j);
    for (int j = k; j < n; ++j)
        if (x[j] > hv[0]) { hv[0] = x[j]; hi[0] = j; sift(0); }
    for (int a = 0; a < k; ++a) {
        int m = a;
        for (int b = a + 1; b < k; ++b)
            if (hv[b] > hv[m]) m = b;
        out_v[a] = hv[m];
        out_i[a] = hi[m];
        hv[m] = hv[a];
        hi[m] = hi[a];
    }
}

// logsoftmax<float> of `rows` rows of n values in LDS (v, row-major) into out,
// by every thread of the workgroup: the row maximum (std::max order: a NaN
// never replaces it) and exp(v - max) per value in parallel, then per row the
// float sum of those terms in index order and log(sum) + max (one thread per
// row), then v - shift.  ex and shift are LDS scratch of rows * n and rows
// floats.  Contains two barriers; every thread calls it.
__device__ __forceinline__ void logsoftmax_rows(const float* v, int rows, int n, float* ex,
                                                float* shift, float* out) {
    const int t = (int)threadIdx.x;
    for (int q = t; q < rows * n; q += (int)blockDim.x) {
        const float* rv = v + (q / n) * n;
        float mx = -__builtin_inff();
        for (int i = 0; i < n; ++i) mx = mx < rv[i] ? rv[i] : mx;
        ex[q] = exp_cr(v[q] - mx);
    }
    __syncthreads();
    for (int r = t; r < rows; r += (int)blockDim.x) {
        const float* rv = v + r * n;
        float mx = -__builtin_inff(), sum = 0.0f;
        for (int i = 0; i < n; ++i) mx = mx < rv[i] ? rv[i] : mx;
        for (int i = 0; i < n; ++i) sum += ex[r * n + i];
        shift[r] = log_cr(sum) + mx;
    }
    __syncthreads();
    for (int q = t; q < rows * n; q += (int)blockDim.x) out[q] = v[q] - shift[q / n];
}

// topk<float> (the reference's heap) of n values in LDS, k = KC <= TK_FAST_K,
// by wavefront 0 (every lane alike) with the heap in scalar registers: the
// first KC values heapified, then every value above the root in index order
// (a ballot per 64 values finds them), then the selection sort.  Returns false
// (writing nothing) when a NaN is among the first KC values: the caller then
// takes heap_topk_serial.
template <int KC>
__device__ __forceinline__ bool heap_small(const float* x, int n, int32_t* out_i, float* out_v) {
    const int lane = (int)lane_id();
    uint32_t hk[TK_FAST_K];
    int32_t hi[TK_FAST_K];
    bool nan0 = false;
#pragma unroll
    for (int i = 0; i < TK_FAST_K; ++i) {
        hk[i] = 0u;
        hi[i] = 0;
        if (i < KC) {
            const float f = x[i];
            nan0 = nan0 || f != f;
            hk[i] = (uint32_t)__builtin_amdgcn_readfirstlane((int)f32_key(f));
            hi[i] = i;
        }
    }
    if (nan0) return false;
    uheap_build<KC, KC / 2 - 1>(hk, hi);
    uint32_t root = hk[0];
    for (int g = KC; g < n; g += 64) {
        const int e = g + lane;
        const float f = e < n ? x[e] : __builtin_nanf("");
        const uint32_t key = f == f ? f32_key(f) : 0u;         // a NaN never enters
        uint64_t m = ballot(key > root);
        while (m) {
            const int Ln = __builtin_ctzll(m);
            hk[0] = (uint32_t)__builtin_amdgcn_readlane((int)key, Ln);
            hi[0] = g + Ln;
            uheap_sift<KC, 0>(hk, hi);
            root = hk[0];
            const uint64_t after = Ln == 63 ? 0ull : (~0ull << (Ln + 1));
            m = ballot(key > root) & after;
        }
    }
    int32_t ri = 0;
#pragma unroll
    for (int a = 0; a < KC; ++a) {
        uint32_t vm = hk[a];
        int32_t im = hi[a];
        int m = a;
#pragma unroll
        for (int b = a + 1; b < KC; ++b) {
            const bool gt = hk[b] > vm;
            vm = gt ? hk[b] : vm;
            im = gt ? hi[b] : im;
            m = gt ? b : m;
        }
        ri = lane == a ? im : ri;
#pragma unroll
        for (int b = a + 1; b < KC; ++b) {
            hk[b] = m == b ? hk[a] : hk[b];
            hi[b] = m == b ? hi[a] : hi[b];
        }
    }
    if (lane < KC) {
        out_i[lane] = ri;
        out_v[lane] = x[ri];
    }
    return true;
}

// heap_small for a run-time k (wavefront 0); false when k > TK_FAST_K or a
// NaN is among the first k values.
__device__ __forceinline__ bool heap_small_k(const float* x, int n, int k, int32_t* out_i,
                                             float* out_v) {
    switch (k) {
        case 1: return heap_small<1>(x, n, out_i, out_v);
        case 2: return heap_small<2>(x, n, out_i, out_v);
        case 3: return heap_small<3>(x, n, out_i, out_v);
        case 4: return heap_small<4>(x, n, out_i, out_v);
        case 5: return heap_small<5>(x, n, out_i, out_v);
        case 6: return heap_small<6>(x, n, out_i, out_v);
        case 7: return heap_small<7>(x, n, out_i, out_v);
        case 8: return heap_small<8>(x, n, out_i, out_v);
        default: return false;
    }
}

// Level 0: the root row's top K, their log-softmax as the scores, their
// mapped tokens; parent group 0; the draft mask starts as the K x K identity.
template <typename TL>
__global__ __launch_bounds__(TK_WG) void eagle3_begin_kernel(TreeParams P) {
    __shared__ TopkShared sh;
    __shared__ float lp[TK_MAXK], ex[TK_MAXK], shift[1];
    const TreeLayout L = tree_layout(P.K, P.depth);
    const int K = P.K, t = (int)threadIdx.x;
    topk_row<TL>((const TL*)P.x, P.cols, K, P.vec != 0, sh);
    logsoftmax_rows(sh.res_v, 1, K, ex, shift, lp);
    if (t < K) {
        const int32_t id = sh.res_i[t];
        const int32_t tok = id + P.d2t[id];
        st<float>(P, L.score)[t] = lp[t];
        st<float>(P, L.node_score)[t] = lp[t];
        st<int32_t>(P, L.node_tok)[t] = tok;
        P.out_inputs[t] = tok;
    }
    if (t == 0) st<int32_t>(P, L.parent)[0] = 0;
    const int mc = K * P.depth;
    for (int e = t; e < K * mc; e += TK_WG) st<float>(P, L.mask)[e] = (e % mc) == e / mc ? 1.0f : 0.0f;
}

// The top K of each of the K rows of a level, into the state.
template <typename TL>
__global__ __launch_bounds__(TK_WG) void eagle3_rows_kernel(TreeParams P) {
    __shared__ TopkShared sh;
    const TreeLayout L = tree_layout(P.K, P.depth);
    const int K = P.K, r = (int)blockIdx.x;
    topk_row<TL>((const TL*)P.x + (size_t)r * P.row_stride, P.cols, K, P.vec != 0, sh);
    if ((int)threadIdx.x < K) {
        st<int32_t>(P, L.row_idx)[r * K + threadIdx.x] = sh.res_i[threadIdx.x];
        st<float>(P, L.row_val)[r * K + threadIdx.x] = sh.res_v[threadIdx.x];
    }
}

// Level `level` (1 .. depth-1) from the rows' top K: cumulative scores, the
// best K of them, parent rows, next input ids, node lists, parent group, mask.
__global__ __launch_bounds__(TREE_WG) void eagle3_combine_kernel(TreeParams P) {
    __shared__ float cu[TK_MAXK * TK_MAXK];
    __shared__ int32_t tok[TK_MAXK * TK_MAXK];
    __shared__ float rv[TK_MAXK * TK_MAXK];
    __shared__ float score[TK_MAXK], hv[TK_MAXK], bestv[TK_MAXK], shift[TK_MAXK];
    __shared__ float ex[TK_MAXK * TK_MAXK];
    __shared__ int32_t hi[TK_MAXK], best[TK_MAXK];
    __shared__ uint32_t fast;
    __shared__ float oldm[TK_MAXK * TK_MAXK * 16];
    const TreeLayout L = tree_layout(P.K, P.depth);
    const int K = P.K, KK = K * K, t = (int)threadIdx.x;
    const int i = P.level - 1;                    // the reference's loop counter
    const int mc = K * P.depth, acols = K * P.level;
    for (int q = t; q < KK; q += TREE_WG) {
        const int32_t id = st<int32_t>(P, L.row_idx)[q];
        tok[q] = id + P.d2t[id];
        rv[q] = st<float>(P, L.row_val)[q];
    }
    if (t < K) score[t] = st<float>(P, L.score)[t];
    for (int e = t; e < K * acols; e += TREE_WG)
        oldm[e] = st<float>(P, L.mask)[(e / acols) * mc + e % acols];
    __syncthreads();
    // each row's log-softmax plus the row's score (the reference's float steps)
    logsoftmax_rows(rv, K, K, ex, shift, cu);
    for (int q = t; q < KK; q += TREE_WG) cu[q] = cu[q] + score[q / K];
    __syncthreads();
    // the best K of the K*K cumulative scores (the reference's heap)
    if (t < 64) {
        const bool ok = heap_small_k(cu, KK, K, best, bestv);
        if (t == 0) fast = ok ? 1u : 0u;
    }
    __syncthreads();
    if (!fast) {
        if (t == 0) heap_topk_serial(cu, KK, K, hv, hi, best, bestv);
        __syncthreads();
    }
    const size_t nbase = (size_t)K + (size_t)i * KK;
    for (int q = t; q < KK; q += TREE_WG) {
        st<float>(P, L.node_score)[nbase + q] = cu[q];
        st<int32_t>(P, L.node_tok)[nbase + q] = tok[q];
    }
    if (t < K) {
        const int32_t gbase = 1 + KK * (i - 1 > 0 ? i - 1 : 0) + (i > 0 ? K : 0);
        st<int32_t>(P, L.parent)[1 + i * K + t] = t + gbase;
        st<float>(P, L.score)[t] = bestv[t];
        P.out_inputs[t] = tok[best[t]];
        if (P.out_prow) P.out_prow[t] = best[t] / K;
    }
    // the mask: row r = old row of its parent, then an identity block
    const int ncols = acols + K;
    for (int e = t; e < K * ncols; e += TREE_WG) {
        const int r = e / ncols, c = e % ncols;
        const float v = c < acols ? oldm[(best[r] / K) * acols + c] : (c - acols == r ? 1.0f : 0.0f);
        st<float>(P, L.mask)[r * mc + c] = v;
        if (P.out_mask) P.out_mask[e] = v;
    }
}

// The final tree: best `total` node scores, tokens, parents located among the
// survivors, tree mask, position ids, retrieve indices.  Only the set of the
// best `total` nodes matters (the reference sorts their positions), so it is
// found by ranking: node i is in when fewer than `total` nodes score above
// it; when the nodes equal to the boundary score are not all in, which of
// them the reference's heap keeps depends on its history, and one thread
// replays it (heap_topk_serial), as it does for NaN scores or more than
// TREE_RANK_MAX nodes.  The rest runs in parallel: positions by a scan of the
// membership flags, each survivor's parent by a binary search, each tree
// row's ancestors by walking up, leaves and their retrieve paths.
#define TREE_RANK_MAX 1024
__global__ __launch_bounds__(TREE_WG) void eagle3_finish_kernel(TreeParams P) {
    __shared__ float ns[TREE_MAX_NODES];
    __shared__ int32_t par[1 + TREE_MAX_NODES / TK_MAXK];
    __shared__ float hv[TK_MAXK], selv[TK_MAXK];
    __shared__ int32_t hi[TK_MAXK], sel[TK_MAXK], up[TK_MAXK];
    __shared__ uint64_t rowbits[TK_MAXK + 1];
    __shared__ uint32_t flag[TREE_RANK_MAX / 32];
    __shared__ uint32_t wsum[LLIMA_WAVES];
    __shared__ uint32_t slow, nan_any, bad_tie, parents_lo, parents_hi, maxpos_s;
    const TreeLayout L = tree_layout(P.K, P.depth);
    const int K = P.K, T = P.total, N = T + 1, t = (int)threadIdx.x;
    const int nodes = K + (P.depth - 1) * K * K, ngroups = 1 + (P.depth - 1) * K;
    const int rc = N;                        // a leaf path has at most N nodes
    if (t == 0) { nan_any = 0; bad_tie = 0; parents_lo = 0; parents_hi = 0; maxpos_s = 0; }
    for (int q = t; q < TREE_RANK_MAX / 32; q += TREE_WG) flag[q] = 0;
    for (int q = t; q < nodes; q += TREE_WG) ns[q] = st<float>(P, L.node_score)[q];
    for (int q = t; q < ngroups; q += TREE_WG) par[q] = st<int32_t>(P, L.parent)[q];
    for (int e = t; e < N * rc; e += TREE_WG) P.out_retrieve[e] = -1;
    __syncthreads();
    // ---- the set: rank every node against every node
    if (nodes <= TREE_RANK_MAX) {
        for (int i = t; i < nodes; i += TREE_WG) {
            const float v = ns[i];
            if (v != v) { nan_any = 1u; continue; }
            int gt = 0, eq = 0;
            for (int j = 0; j < nodes; ++j) {
                const float u = ns[j];
                gt += u > v ? 1 : 0;
                eq += u == v ? 1 : 0;
            }
            if (gt < T) {
                atomicOr(&flag[i >> 5], 1u << (i & 31));
                if (gt + eq > T) bad_tie = 1u;      // equal nodes straddle the boundary
            }
        }
    }
    __syncthreads();
    if (t == 0) slow = (nodes > TREE_RANK_MAX || nan_any || bad_tie) ? 1u : 0u;
    __syncthreads();
    if (slow) {
        if (t == 0) {
            heap_topk_serial(ns, nodes, T, hv, hi, sel, selv);
            for (int a = 1; a < T; ++a) {                       // ascending positions
                const int32_t v = sel[a];
                int b = a - 1;
                while (b >= 0 && sel[b] > v) { sel[b + 1] = sel[b]; --b; }
                sel[b + 1] = v;
            }
        }
    } else {
        // positions: a scan of the membership flags (thread t: nodes 4t .. 4t+3)
        const int i0 = 4 * t;
        uint32_t f4 = 0, c = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int i = i0 + e;
            const uint32_t b = i < nodes ? (flag[i >> 5] >> (i & 31)) & 1u : 0u;
            f4 |= b << e;
            c += b;
        }
        const uint32_t inc = wave_incl_scan_u32(c);
        if (lane_id() == 63) wsum[wave_id()] = inc;
        __syncthreads();
        uint32_t o = inc - c;
        for (uint32_t w = 0; w < wave_id(); ++w) o += wsum[w];
#pragma unroll
        for (int e = 0; e < 4; ++e)
            if ((f4 >> e) & 1u) sel[o++] = i0 + e;
    }
    __syncthreads();
    // ---- each survivor's parent: its group's entry minus 1 located among the
    //      sorted positions (eagle_helpers.hpp:197-214, lower bound), + 1
    if (t < T) {
        const int32_t pg = par[sel[t] / K];
        int lo = 0, hi2 = T;
        while (lo < hi2) {
            const int mid = (lo + hi2) >> 1;
            if (sel[mid] < pg - 1) lo = mid + 1; else hi2 = mid;
        }
        const int u = (pg == 0 ? -1 : lo) + 1;
        up[t] = u;
        if (u < 32) atomicOr(&parents_lo, 1u << u);
        else atomicOr(&parents_hi, 1u << (u - 32));
    }
    __syncthreads();
    // ---- tree rows: identity, column 0, and the ancestors (walk up)
    if (t < N) {
        uint64_t b = (1ull << t) | 1ull;
        int a = t;
        while (a > 0) {
            a = up[a - 1];
            b |= 1ull << a;
        }
        rowbits[t] = b;
        atomicMax(&maxpos_s, (uint32_t)(__popcll(b) - 1));
    }
    __syncthreads();
    const uint64_t parents = ((uint64_t)parents_hi << 32) | parents_lo;
    const int leaves = T - (__popcll(parents) - 1);
    // ---- retrieve: leaf r (the r-th node that is nobody's parent) walked
    //      back to the root
    if (t < N && !((parents >> t) & 1ull)) {
        const int row = t - __popcll(parents & ((1ull << t) - 1ull));   // nodes before t that are leaves
        if (row < leaves) {
            int at = t;
            for (int j = __popcll(rowbits[t]) - 1; j >= 0; --j) {
                P.out_retrieve[row * rc + j] = at;
                if (at > 0) at = up[at - 1];
            }
        }
    }
    for (int e = t; e < N * N; e += TREE_WG) {
        const int r = e / N, c = e % N;
        P.out_tree_mask[e] = (float)((rowbits[r] >> c) & 1ull);
    }
    if (t < N) {
        P.out_pos[t] = __popcll(rowbits[t]) - 1;
        P.out_tokens[t] = t == 0 ? P.sample_token : st<int32_t>(P, L.node_tok)[sel[t - 1]];
    }
    if (t == 0) {
        P.out_dims[0] = leaves;
        P.out_dims[1] = (int)maxpos_s + 1;
    }
}

}  // namespace llima

using namespace llima;

// Rows start on 16-byte boundaries (the row stride in bytes is a multiple of 16).
static int32_t rows_vec(const void* x, int64_t row_stride, int32_t dtype) {
    const int64_t esz = dtype == LLIMA_F32 ? 4 : 2;
    return ((uintptr_t)x % 16 == 0) && ((row_stride * esz) % 16 == 0) ? 1 : 0;
}

static bool tree_dims_ok(int32_t K, int32_t depth) {
    if (K < 1 || K > TK_MAXK || depth < 1 || depth > 16) return false;
    const int64_t nodes = (int64_t)K + (int64_t)(depth - 1) * K * K;
    return nodes <= TREE_MAX_NODES && (int64_t)K * K * (depth > 1 ? depth - 1 : 1) <= 16384;
}

extern "C" int llima_topk(const void* x, int32_t dtype, int32_t rows, int32_t cols,
                          int64_t row_stride, int32_t k, int32_t* out_idx, float* out_vals,
                          void* stream) {
    if (dtype != LLIMA_F32 && dtype != LLIMA_BF16) return LLIMA_E_INVAL;
    if (rows < 0 || k < 1 || k > TK_MAXK || cols < k || row_stride < cols) return LLIMA_E_INVAL;
    if (rows == 0) return LLIMA_OK;
    if (!x || !out_idx || !out_vals) return LLIMA_E_INVAL;
    TreeParams P = {};
    P.x = x; P.row_stride = row_stride; P.rows = rows; P.cols = cols; P.k = k;
    P.out_idx = out_idx; P.out_val = out_vals;
    P.vec = rows_vec(x, row_stride, dtype);
    hipStream_t st = (hipStream_t)stream;
    if (dtype == LLIMA_F32)
        hipLaunchKernelGGL(topk_rows_kernel<float>, dim3(rows), dim3(TK_WG), 0, st, P);
    else
        hipLaunchKernelGGL(topk_rows_kernel<uint16_t>, dim3(rows), dim3(TK_WG), 0, st, P);
    return hipGetLastError() == hipSuccess ? LLIMA_OK : LLIMA_E_HIP;
}

extern "C" size_t llima_eagle3_tree_bytes(int32_t K, int32_t depth) {
    if (!tree_dims_ok(K, depth)) return 0;
    return tree_layout(K, depth).total;
}

extern "C" int llima_eagle3_tree_begin(const void* logits, int32_t dtype, int32_t Vd,
                                       const int32_t* d2t, int32_t K, int32_t depth, void* tree,
                                       size_t tree_bytes, int32_t* out_input_ids, void* stream) {
    if (dtype != LLIMA_F32 && dtype != LLIMA_BF16) return LLIMA_E_INVAL;
    if (!tree_dims_ok(K, depth) || Vd < K || !logits || !d2t || !out_input_ids) return LLIMA_E_INVAL;
    if (!tree || tree_bytes < tree_layout(K, depth).total) return LLIMA_E_WORKSPACE;
    TreeParams P = {};
    P.x = logits; P.cols = Vd; P.k = K; P.d2t = d2t; P.state = (char*)tree;
    P.K = K; P.depth = depth; P.out_inputs = out_input_ids;
    P.vec = rows_vec(logits, Vd, dtype);
    hipStream_t st = (hipStream_t)stream;
    if (dtype == LLIMA_F32)
        hipLaunchKernelGGL(eagle3_begin_kernel<float>, dim3(1), dim3(TK_WG), 0, st, P);
    else
        hipLaunchKernelGGL(eagle3_begin_kernel<uint16_t>, dim3(1), dim3(TK_WG), 0, st, P);
    return hipGetLastError() == hipSuccess ? LLIMA_OK : LLIMA_E_HIP;
}

extern "C" int llima_eagle3_tree_grow(const void* logits, int32_t dtype, int32_t Vd,
                                      int64_t row_stride, const int32_t* d2t, int32_t K,
                                      int32_t depth, int32_t level, void* tree, size_t tree_bytes,
                                      int32_t* out_input_ids, int32_t* out_parent_rows,
                                      float* out_mask, void* stream) {
    if (dtype != LLIMA_F32 && dtype != LLIMA_BF16) return LLIMA_E_INVAL;
    if (!tree_dims_ok(K, depth) || Vd < K || row_stride < Vd || level < 1 || level >= depth)
        return LLIMA_E_INVAL;
    if (!logits || !d2t || !out_input_ids) return LLIMA_E_INVAL;
    if (!tree || tree_bytes < tree_layout(K, depth).total) return LLIMA_E_WORKSPACE;
    TreeParams P = {};
    P.x = logits; P.row_stride = row_stride; P.cols = Vd; P.k = K; P.d2t = d2t;
    P.state = (char*)tree; P.K = K; P.depth = depth; P.level = level;
    P.out_inputs = out_input_ids; P.out_prow = out_parent_rows; P.out_mask = out_mask;
    P.vec = rows_vec(logits, row_stride, dtype);
    hipStream_t st = (hipStream_t)stream;
    if (dtype == LLIMA_F32)
        hipLaunchKernelGGL(eagle3_rows_kernel<float>, dim3(K), dim3(TK_WG), 0, st, P);
    else
        hipLaunchKernelGGL(eagle3_rows_kernel<uint16_t>, dim3(K), dim3(TK_WG), 0, st, P);
    hipLaunchKernelGGL(eagle3_combine_kernel, dim3(1), dim3(TREE_WG), 0, st, P);
    return hipGetLastError() == hipSuccess ? LLIMA_OK : LLIMA_E_HIP;
}

extern "C" int llima_eagle3_tree_finish(void* tree, size_t tree_bytes, int32_t K, int32_t depth,
                                        int32_t total_tokens, int32_t sample_token,
                                        int32_t* out_tokens, float* out_tree_mask,
                                        int32_t* out_position_ids, int32_t* out_retrieve,
                                        int32_t* out_dims, void* stream) {
    if (!tree_dims_ok(K, depth) || total_tokens < 1 || total_tokens > TK_MAXK) return LLIMA_E_INVAL;
    if (total_tokens > K + (depth - 1) * K * K) return LLIMA_E_INVAL;
    if (!out_tokens || !out_tree_mask || !out_position_ids || !out_retrieve || !out_dims)
        return LLIMA_E_INVAL;
    if (!tree || tree_bytes < tree_layout(K, depth).total) return LLIMA_E_WORKSPACE;
    TreeParams P = {};
    P.state = (char*)tree; P.K = K; P.depth = depth; P.total = total_tokens;
    P.sample_token = sample_token;
    P.out_tokens = out_tokens; P.out_tree_mask = out_tree_mask; P.out_pos = out_position_ids;
    P.out_retrieve = out_retrieve; P.out_dims = out_dims;
    hipLaunchKernelGGL(eagle3_finish_kernel, dim3(1), dim3(TREE_WG), 0, (hipStream_t)stream, P);
    return hipGetLastError() == hipSuccess ? LLIMA_OK : LLIMA_E_HIP;
}
