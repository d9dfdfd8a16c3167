// argmax.hip -- greedy token selection and greedy draft verification (gfx950).
//
// Restates on device memory the reference's host-side argmax family:
//   argmax_bf16                 sima_lmm/devkit/cpp/utils.hpp:80-152
//   _calc_next_token_id         sima_lmm/devkit/cpp/language_model.cpp:3689-3714
//   _argmax_lm_head_row(s)      sima_lmm/devkit/cpp/language_model.cpp:3616-3687
//   EAGLE3 verify argmax        sima_lmm/devkit/cpp/language_model_eagle3.cpp:486-522
// and the verification epilogues
//   resolve_draft_tokens        sima_lmm/devkit/cpp/gemma4_mtp_helpers.cpp:81-111
//   tree gather + evaluate_posterior
//                               sima_lmm/devkit/cpp/language_model_eagle3.cpp:551-567,
//                               sima_lmm/devkit/cpp/eagle_helpers.hpp:153-195
//
// Layout: a [rows][V] logits matrix is cut into B x S workgroups of 256*E
// values; each workgroup streams its chunk with 16-byte loads, keeps a running
// (value, first index) per thread with a strict '>' (so NaN never wins and the
// first maximum is kept, as the reference's scalar loop), reduces the chunk to a
// 64-bit key (value key << 32 | ~index) and merges it into the row with one
// device-scope atomicMax.  The last workgroup of a row (completion counter)
// writes the result; with the verification epilogues the last row of a
// sequence (or of the tree) also resolves the drafts.  The reference's early
// exit after the first mismatching row (language_model.cpp:3679-3684) is a host
// latency optimisation; every row is computed here and the emitted tokens are
// identical.
#include "common.hpp"
#include "../../include/llima_sampler.h"

namespace llima {

// Workspace: one 32-byte slot per row index; the completion counter of
// verification group g lives in slot g, so the layout never depends on the
// call's shape and a workspace can be reused for any shape.
struct ArgmaxRowWs {
    uint64_t best;
    uint32_t done;
    int32_t token;
    uint32_t group_done;
    uint32_t pad[3];
};

enum { EPI_NONE = 0, EPI_CHAIN = 1, EPI_TREE = 2 };

struct ArgmaxParams {
    const void* logits;
    int64_t row_stride;
    int32_t* out_ids;
    float* out_vals;
    ArgmaxRowWs* ws;
    int32_t B, V, S, split_dim, mode, vec_ok;
    // epilogues
    int32_t epi, D;                // chain: rows per sequence = D + 1
    const int32_t* draft_ids;      // chain [nseq][D]
    int32_t* accepted_len;         // chain [nseq]
    int32_t* emitted;              // chain [nseq][D+1]
    const int32_t* retrieve;       // tree [n_paths][L]
    const int32_t* candidates;     // tree [n_paths][L]
    int32_t n_paths, L;
    int32_t* tree_out;             // tree [3]
};

template <typename TL>
__device__ __forceinline__ float ld1(const TL* p, int64_t i);
template <>
__device__ __forceinline__ float ld1<float>(const float* p, int64_t i) { return p[i]; }
template <>
__device__ __forceinline__ float ld1<uint16_t>(const uint16_t* p, int64_t i) {
    return bf16_bits_to_f32(p[i]);
}

__device__ __forceinline__ uint64_t pack_best(float v, uint32_t idx) {
    // A thread that saw no value above -inf contributes nothing.
    if (!(v > -__builtin_inff())) return 0;
    return ((uint64_t)f32_key(v) << 32) | (uint64_t)(~idx);
}

// Split of index i (mode SPLIT_FIRST: uniform split_dim; QUARTERS: V*p/4).
__device__ __forceinline__ int split_of(int64_t i, int V, int sd, int mode) {
    if (mode == LLIMA_ARGMAX_QUARTERS) {
        int p = 0;
        while (p < 3 && i >= (int64_t)V * (p + 1) / 4) ++p;
        return p;
    }
    return (int)(i / sd);
}
__device__ __forceinline__ int64_t split_begin(int s, int V, int sd, int mode) {
    return mode == LLIMA_ARGMAX_QUARTERS ? (int64_t)V * s / 4 : (int64_t)s * sd;
}

template <typename TL, int E>
__global__ __launch_bounds__(LLIMA_WG) void argmax_kernel(ArgmaxParams P) {
    constexpr int EPL = 16 / sizeof(TL);
    constexpr int NL = E / EPL;
    constexpr int CHUNK = LLIMA_WG * E;
    __shared__ BlockScratch bs;
    __shared__ uint32_t flag, bad_splits;

    uint32_t row, chunk;
    map_row_chunk(blockIdx.x, (uint32_t)P.B, (uint32_t)P.S, &row, &chunk);
    if (row >= (uint32_t)P.B) return;
    const TL* rowp = (const TL*)P.logits + (size_t)row * P.row_stride;
    const int V = P.V;
    const int c0 = (int)chunk * CHUNK;
    const int c1 = c0 + CHUNK < V ? c0 + CHUNK : V;
    const int sd = (P.split_dim <= 0 || P.split_dim >= V) ? V : P.split_dim;

    // Splits whose first value is NaN are invisible (argmax_bf16 starts its
    // running maximum at values[0]).  Rare: detected per chunk, handled slowly.
    if (threadIdx.x == 0) bad_splits = 0;
    __syncthreads();
    if (P.mode != LLIMA_ARGMAX_NEG_INF) {
        const int s_lo = split_of(c0, V, sd, P.mode), s_hi = split_of(c1 - 1, V, sd, P.mode);
        for (int s = s_lo + (int)threadIdx.x; s <= s_hi; s += LLIMA_WG) {
            const float f = ld1<TL>(rowp, split_begin(s, V, sd, P.mode));
            if (f != f) bad_splits = 1u;
        }
    }
    __syncthreads();
    const uint32_t bad = bad_splits;

    float best = -__builtin_inff();
    uint32_t bidx = 0xFFFFFFFFu;
    if (bad == 0) {
#pragma unroll
        for (int j = 0; j < NL; ++j) {
            const int i0 = c0 + j * (LLIMA_WG * EPL) + (int)threadIdx.x * EPL;
            float t[EPL];
            if (P.vec_ok && i0 + EPL <= c1) {
                if constexpr (sizeof(TL) == 4) {
                    float4 q = *(const float4*)(rowp + i0);
                    t[0] = q.x; t[1] = q.y; t[2] = q.z; t[3] = q.w;
                } else {
                    uint4 q = *(const uint4*)(rowp + i0);
                    const uint32_t w4[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        t[2 * e] = __uint_as_float(w4[e] << 16);
                        t[2 * e + 1] = __uint_as_float(w4[e] & 0xFFFF0000u);
                    }
                }
            } else {
#pragma unroll
                for (int e = 0; e < EPL; ++e)
                    t[e] = (i0 + e < c1) ? ld1<TL>(rowp, i0 + e) : -__builtin_inff();
            }
#pragma unroll
            for (int e = 0; e < EPL; ++e)
                if (t[e] > best) { best = t[e]; bidx = (uint32_t)(i0 + e); }
        }
    } else {
        // element-wise: skip values whose split starts with NaN
        for (int i = c0 + (int)threadIdx.x; i < c1; i += LLIMA_WG) {
            const float f = ld1<TL>(rowp, split_begin(split_of(i, V, sd, P.mode), V, sd, P.mode));
            if (f != f) continue;
            const float x = ld1<TL>(rowp, i);
            if (x > best) { best = x; bidx = (uint32_t)i; }
        }
    }
    uint64_t key = block_max_u64(pack_best(best, bidx), bs);
    ArgmaxRowWs* rw = P.ws + row;
    if (threadIdx.x == 0 && key) atomicMax((unsigned long long*)&rw->best, (unsigned long long)key);
    if (!arrive_last(&rw->done, (uint32_t)P.S, &flag)) return;

    // ---- row result
    if (threadIdx.x == 0) {
        const uint64_t k = load_coherent(&rw->best);
        rw->best = 0;
        int32_t id = 0;
        float val = -__builtin_inff();
        if (k) { id = (int32_t)(~(uint32_t)k); val = ld1<TL>(rowp, id); }
        if (P.mode == LLIMA_ARGMAX_QUARTERS) {
            const float v0 = ld1<TL>(rowp, 0);
            if (v0 != v0) { id = 0; val = v0; }
        }
        if (P.out_ids) P.out_ids[row] = id;
        if (P.out_vals) P.out_vals[row] = val;
        rw->token = id;
    }
    if (P.epi == EPI_NONE) return;

    // ---- verification epilogues: the last row of the group resolves it
    const uint32_t grp = P.epi == EPI_CHAIN ? row / (uint32_t)(P.D + 1) : 0u;
    const uint32_t grp_rows = P.epi == EPI_CHAIN ? (uint32_t)(P.D + 1) : (uint32_t)P.B;
    if (!arrive_last(&P.ws[grp].group_done, grp_rows, &flag)) return;
    if (threadIdx.x != 0) return;
    if (P.epi == EPI_CHAIN) {
        const int D = P.D;
        const ArgmaxRowWs* g = P.ws + (size_t)grp * (D + 1);
        const int32_t* dr = P.draft_ids + (size_t)grp * D;
        int32_t* em = P.emitted + (size_t)grp * (D + 1);
        int acc = 0;
        while (acc < D && dr[acc] == load_coherent(&g[acc].token)) { em[acc] = dr[acc]; ++acc; }
        em[acc] = load_coherent(&g[acc].token);
        for (int j = acc + 1; j <= D; ++j) em[j] = -1;
        P.accepted_len[grp] = acc;
    } else {
        // gather target tokens along each path (-1 -> last tree row), then the
        // first path with the strictly longest accepted prefix wins.
        const int K = P.B, L = P.L;
        int32_t best_c = 0, max_acc = 0;
        for (int p = 0; p < P.n_paths; ++p) {
            int32_t acc = 0;
            for (int i = 0; i + 1 < L; ++i) {
                int32_t idx = P.retrieve[p * L + i];
                if (idx < 0) idx = K - 1;
                const int32_t arg = load_coherent(&P.ws[idx < K ? idx : K - 1].token);
                const int32_t nxt = P.candidates[p * L + i + 1];
                if (nxt < 0 || arg != nxt) break;
                ++acc;
            }
            if (acc > max_acc) { max_acc = acc; best_c = p; }
        }
        int32_t idx = P.retrieve[best_c * L + max_acc];
        if (idx < 0) idx = K - 1;
        P.tree_out[0] = best_c;
        P.tree_out[1] = max_acc;
        P.tree_out[2] = load_coherent(&P.ws[idx < K ? idx : K - 1].token);
    }
}

struct ATile { int E, S; };
static ATile argmax_tile(int B, int V, int dtype) {
    int E = dtype == LLIMA_F32 ? 32 : 64;
    auto S_of = [&](int e) { return (V + LLIMA_WG * e - 1) / (LLIMA_WG * e); };
    while (E > 8 && (int64_t)B * S_of(E) < 1024) E /= 2;
    return {E, S_of(E)};
}

template <typename TL, int E>
static hipError_t launch_argmax(const ArgmaxParams& P, hipStream_t st) {
    hipLaunchKernelGGL((argmax_kernel<TL, E>), dim3((uint32_t)P.B * (uint32_t)P.S), dim3(LLIMA_WG),
                       0, st, P);
    return hipGetLastError();
}

static int run_argmax(ArgmaxParams& P, int dtype, hipStream_t st) {
    const ATile t = argmax_tile(P.B, P.V, dtype);
    P.S = t.S;
    const size_t esz = dtype == LLIMA_F32 ? 4 : 2;
    P.vec_ok = ((uintptr_t)P.logits % 16 == 0) && ((P.row_stride * (int64_t)esz) % 16 == 0);
    hipError_t e;
    if (dtype == LLIMA_F32) {
        switch (t.E) {
            case 8: e = launch_argmax<float, 8>(P, st); break;
            case 16: e = launch_argmax<float, 16>(P, st); break;
            default: e = launch_argmax<float, 32>(P, st); break;
        }
    } else {
        switch (t.E) {
            case 8: e = launch_argmax<uint16_t, 8>(P, st); break;
            case 16: e = launch_argmax<uint16_t, 16>(P, st); break;
            case 32: e = launch_argmax<uint16_t, 32>(P, st); break;
            default: e = launch_argmax<uint16_t, 64>(P, st); break;
        }
    }
    return e == hipSuccess ? LLIMA_OK : LLIMA_E_HIP;
}

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

}  // namespace llima

using namespace llima;

extern "C" size_t llima_argmax_workspace_bytes(int32_t B, int32_t V, int32_t dtype) {
    (void)V; (void)dtype;
    return B > 0 ? align256((size_t)B * sizeof(ArgmaxRowWs)) : 0;
}

extern "C" int llima_argmax(const void* logits, int32_t dtype, int32_t B, int32_t V,
                            int64_t row_stride, int32_t split_dim, int32_t mode,
                            int32_t* out_ids, float* out_vals, void* workspace,
                            size_t workspace_bytes, void* stream) {
    if (!logits || !out_ids) return LLIMA_E_INVAL;
    if (dtype != LLIMA_F32 && dtype != LLIMA_BF16) return LLIMA_E_INVAL;
    if (B < 0 || V <= 0 || row_stride < V) return LLIMA_E_INVAL;
    if (mode < LLIMA_ARGMAX_SPLIT_FIRST || mode > LLIMA_ARGMAX_QUARTERS) return LLIMA_E_INVAL;
    if (B == 0) return LLIMA_OK;
    if (!workspace || workspace_bytes < llima_argmax_workspace_bytes(B, V, dtype))
        return LLIMA_E_WORKSPACE;
    ArgmaxParams P = {};
    P.logits = logits;
    P.row_stride = row_stride;
    P.out_ids = out_ids;
    P.out_vals = out_vals;
    P.ws = (ArgmaxRowWs*)workspace;
    P.B = B; P.V = V; P.split_dim = split_dim; P.mode = mode;
    P.epi = EPI_NONE;
    return run_argmax(P, dtype, (hipStream_t)stream);
}

extern "C" size_t llima_verify_greedy_workspace_bytes(int32_t B, int32_t D, int32_t V,
                                                      int32_t dtype) {
    if (B <= 0 || D < 0) return 0;
    return llima_argmax_workspace_bytes(B * (D + 1), V, dtype);
}

extern "C" int llima_verify_greedy(const void* target_logits, int32_t dtype, int32_t B, int32_t D,
                                   int32_t V, const int32_t* draft_ids, int32_t* accepted_len,
                                   int32_t* emitted, void* workspace, size_t workspace_bytes,
                                   void* stream) {
    if (!target_logits || !accepted_len || !emitted || (D > 0 && !draft_ids)) return LLIMA_E_INVAL;
    if (dtype != LLIMA_F32 && dtype != LLIMA_BF16) return LLIMA_E_INVAL;
    if (B < 0 || D < 0 || V <= 0) return LLIMA_E_INVAL;
    if (B == 0) return LLIMA_OK;
    if (!workspace || workspace_bytes < llima_verify_greedy_workspace_bytes(B, D, V, dtype))
        return LLIMA_E_WORKSPACE;
    ArgmaxParams P = {};
    P.logits = target_logits;
    P.row_stride = V;
    P.ws = (ArgmaxRowWs*)workspace;
    P.B = B * (D + 1); P.V = V; P.split_dim = 0; P.mode = LLIMA_ARGMAX_SPLIT_FIRST;
    P.epi = EPI_CHAIN; P.D = D;
    P.draft_ids = draft_ids; P.accepted_len = accepted_len; P.emitted = emitted;
    return run_argmax(P, dtype, (hipStream_t)stream);
}

extern "C" size_t llima_verify_tree_workspace_bytes(int32_t K, int32_t V, int32_t dtype) {
    if (K <= 0) return 0;
    return llima_argmax_workspace_bytes(K, V, dtype);
}

extern "C" int llima_verify_tree(const void* tree_logits, int32_t dtype, int32_t K, int32_t V,
                                 const int32_t* retrieve_indices, const int32_t* candidates,
                                 int32_t n_paths, int32_t L, int32_t* out, void* workspace,
                                 size_t workspace_bytes, void* stream) {
    if (!tree_logits || !retrieve_indices || !candidates || !out) return LLIMA_E_INVAL;
    if (dtype != LLIMA_F32 && dtype != LLIMA_BF16) return LLIMA_E_INVAL;
    if (K <= 0 || V <= 0 || n_paths <= 0 || L <= 0) return LLIMA_E_INVAL;
    if (!workspace || workspace_bytes < llima_verify_tree_workspace_bytes(K, V, dtype))
        return LLIMA_E_WORKSPACE;
    ArgmaxParams P = {};
    P.logits = tree_logits;
    P.row_stride = V;
    P.ws = (ArgmaxRowWs*)workspace;
    // The EAGLE3 verify argmax starts from -inf (language_model_eagle3.cpp:491-521).
    P.B = K; P.V = V; P.split_dim = 0; P.mode = LLIMA_ARGMAX_NEG_INF;
    P.epi = EPI_TREE;
    P.retrieve = retrieve_indices; P.candidates = candidates; P.n_paths = n_paths; P.L = L;
    P.tree_out = out;
    return run_argmax(P, dtype, (hipStream_t)stream);
}

extern "C" int llima_workspace_init(void* workspace, size_t workspace_bytes, void* stream) {
    if (!workspace && workspace_bytes) return LLIMA_E_INVAL;
    if (!workspace_bytes) return LLIMA_OK;
    return hipMemsetAsync(workspace, 0, workspace_bytes, (hipStream_t)stream) == hipSuccess
               ? LLIMA_OK : LLIMA_E_HIP;
}

extern "C" const char* llima_status_string(int status) {
    switch (status) {
        case LLIMA_OK: return "ok";
        case LLIMA_E_INVAL: return "invalid argument";
        case LLIMA_E_RANGE: return "value out of range";
        case LLIMA_E_HIP: return "HIP launch error";
        case LLIMA_E_WORKSPACE: return "workspace missing or too small";
        default: return "unknown status";
    }
}

extern "C" int llima_abi_version(void) { return 1; }
