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
    uint32_t wpart[TK_WAVES];
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
// reference's output order.  Every thread of the 1024 calls it.
template <typename TL>
__device__ void topk_row(const TL* rowp, int cols, int k, TopkShared& sh) {
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

// ------------------------------------------------------------------ kernels
template <typename TL>
__global__ __launch_bounds__(TK_WG) void topk_rows_kernel(TreeParams P) {
    __shared__ TopkShared sh;
    const int r = (int)blockIdx.x;
    topk_row<TL>((const TL*)P.x + (size_t)r * P.row_stride, P.cols, P.k, sh);
    if ((int)threadIdx.x < P.k) {
        P.out_idx[(size_t)r * P.k + threadIdx.x] = sh.res_i[threadIdx.x];
        P.out_val[(size_t)r * P.k + threadIdx.x] = sh.res_v[threadIdx.x];
    }
}

// logsoftmax<float> of n values in LDS (one thread), into out.
__device__ __forceinline__ void logsoftmax_serial(const float* v, int n, float* out) {
    float mx = -__builtin_inff();
    for (int i = 0; i < n; ++i) mx = mx < v[i] ? v[i] : mx;    // std::max(mx, v)
    float sum = 0.0f;
    for (int i = 0; i < n; ++i) sum += exp_cr(v[i] - mx);
    const float shift = log_cr(sum) + mx;
    for (int i = 0; i < n; ++i) out[i] = v[i] - shift;
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

// Level 0: the root row's top K, their log-softmax as the scores, their
// mapped tokens; parent group 0; the draft mask starts as the K x K identity.
template <typename TL>
__global__ __launch_bounds__(TK_WG) void eagle3_begin_kernel(TreeParams P) {
    __shared__ TopkShared sh;
    __shared__ float lp[TK_MAXK];
    const TreeLayout L = tree_layout(P.K, P.depth);
    const int K = P.K, t = (int)threadIdx.x;
    topk_row<TL>((const TL*)P.x, P.cols, K, sh);
    if (t == 0) logsoftmax_serial(sh.res_v, K, lp);
    __syncthreads();
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
    topk_row<TL>((const TL*)P.x + (size_t)r * P.row_stride, P.cols, K, sh);
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
    __shared__ float score[TK_MAXK], lpv[TK_MAXK], hv[TK_MAXK], bestv[TK_MAXK];
    __shared__ int32_t hi[TK_MAXK], best[TK_MAXK];
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
    if (t == 0) {
        for (int r = 0; r < K; ++r) {
            logsoftmax_serial(rv + r * K, K, lpv);
            for (int j = 0; j < K; ++j) cu[r * K + j] = lpv[j] + score[r];
        }
        heap_topk_serial(cu, KK, K, hv, hi, best, bestv);
    }
    __syncthreads();
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
// survivors, tree mask, position ids, retrieve indices.  The choices are made
// by one thread on LDS copies (a few dozen values); the outputs are written by
// all.
__global__ __launch_bounds__(TREE_WG) void eagle3_finish_kernel(TreeParams P) {
    __shared__ float ns[TREE_MAX_NODES];
    __shared__ int32_t par[1 + TREE_MAX_NODES / TK_MAXK];
    __shared__ float hv[TK_MAXK], selv[TK_MAXK];
    __shared__ int32_t hi[TK_MAXK], sel[TK_MAXK], up[TK_MAXK];
    __shared__ uint64_t rowbits[TK_MAXK + 1];
    __shared__ int32_t leaves_s, rcols_s;
    const TreeLayout L = tree_layout(P.K, P.depth);
    const int K = P.K, T = P.total, N = T + 1, t = (int)threadIdx.x;
    const int nodes = K + (P.depth - 1) * K * K, ngroups = 1 + (P.depth - 1) * K;
    const int rc = N;                        // a leaf path has at most N nodes
    for (int q = t; q < nodes; q += TREE_WG) ns[q] = st<float>(P, L.node_score)[q];
    for (int q = t; q < ngroups; q += TREE_WG) par[q] = st<int32_t>(P, L.parent)[q];
    for (int e = t; e < N * rc; e += TREE_WG) P.out_retrieve[e] = -1;
    __syncthreads();
    if (t == 0) {
        heap_topk_serial(ns, nodes, T, hv, hi, sel, selv);
        for (int a = 1; a < T; ++a) {                       // ascending positions
            const int32_t v = sel[a];
            int b = a - 1;
            while (b >= 0 && sel[b] > v) { sel[b + 1] = sel[b]; --b; }
            sel[b + 1] = v;
        }
        for (int q = 0; q < T; ++q) {
            const int32_t pg = par[sel[q] / K];
            int lo = 0, hi2 = T;                            // lower_bound of pg - 1
            while (lo < hi2) {
                const int mid = (lo + hi2) >> 1;
                if (sel[mid] < pg - 1) lo = mid + 1; else hi2 = mid;
            }
            up[q] = (pg == 0 ? -1 : lo) + 1;
        }
        for (int r = 0; r < N; ++r) rowbits[r] = (1ull << r) | 1ull;
        for (int q = 0; q < T; ++q) rowbits[q + 1] |= rowbits[up[q]];
        uint64_t parents = 0;
        for (int q = 0; q < T; ++q) parents |= 1ull << up[q];
        int maxpos = 0;
        for (int r = 0; r < N; ++r) {
            const int p = __popcll(rowbits[r]) - 1;
            maxpos = p > maxpos ? p : maxpos;
        }
        const int leaves = T - (__popcll(parents) - 1);
        int row = 0;
        for (int node = 0; node < N && row < leaves; ++node) {
            if ((parents >> node) & 1ull) continue;
            int at = node;
            for (int j = __popcll(rowbits[node]) - 1; j >= 0; --j) {
                P.out_retrieve[row * rc + j] = at;
                if (at > 0) at = up[at - 1];
            }
            ++row;
        }
        leaves_s = leaves;
        rcols_s = maxpos + 1;
    }
    __syncthreads();
    for (int e = t; e < N * N; e += TREE_WG) {
        const int r = e / N, c = e % N;
        P.out_tree_mask[e] = (float)((rowbits[r] >> c) & 1ull);
    }
    if (t < N) {
        P.out_pos[t] = __popcll(rowbits[t]) - 1;
        P.out_tokens[t] = t == 0 ? P.sample_token : st<int32_t>(P, L.node_tok)[sel[t - 1]];
    }
    if (t == 0) {
        P.out_dims[0] = leaves_s;
        P.out_dims[1] = rcols_s;
    }
}

}  // namespace llima

using namespace llima;

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
