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
// Two launches, no atomics or fences between workgroups.  argmax_sweep cuts a
// [rows][V] logits matrix into rows x S workgroups of 256*E values; each streams
// its chunk with 16-byte loads, keeps a running (value, first index) per thread
// with a strict '>' (so NaN never wins and the first maximum is kept, as the
// reference's scalar loop) and writes the chunk's 64-bit key
// (value key << 32 | ~index) to its own workspace slot.  argmax_finish reduces
// the S keys of each row with one wavefront per row and writes the result; with
// the verification epilogues one workgroup takes a whole sequence (or the whole
// tree) and resolves its drafts.  The reference's early exit after the first
// mismatching row (language_model.cpp:3679-3684) is a host latency
// optimisation; every row is computed here and the emitted tokens are identical.
//
// A row is one contiguous buffer, or up to 16 split buffers holding consecutive
// vocabulary ranges (the reference's n{N}_lm_split{i} buffers,
// language_model.cpp:3584-3613); chunks never straddle two buffers.
#include "common.hpp"
#include "../../include/llima_sampler.h"

namespace llima {

// Workspace: [rows][S] chunk keys (uint64) then [rows][S] flags (uint32).
// Nothing persists between calls.
#define ARGMAX_MIN_CHUNK 2048
#define ARGMAX_MAX_GROUP 1024       // rows of one sequence / of one tree
#define ARGMAX_MAX_SEGS 16          // split buffers of one row

// bf16 lowest() = -(2 - 2^-7) * 2^127, the start of the spec-path multi-split scan
#define LLIMA_BF16_LOWEST (-3.38953139e38f)

enum { EPI_NONE = 0, EPI_CHAIN = 1, EPI_TREE = 2 };

struct ArgmaxParams {
    // the row's segments: one contiguous buffer, or split buffers (split_segs)
    const void* seg_ptr[ARGMAX_MAX_SEGS];     // row 0 of each segment
    int64_t seg_stride[ARGMAX_MAX_SEGS];      // row stride of each segment, elements
    int32_t seg_begin[ARGMAX_MAX_SEGS + 1];   // vocabulary id of each segment's first value; [nseg] = V
    int32_t seg_chunk0[ARGMAX_MAX_SEGS + 1];  // first chunk of each segment; [nseg] = S
    int32_t nseg, split_segs;                 // split_segs: SPLIT_FIRST splits are the segments
    int32_t* out_ids;
    float* out_vals;
    uint64_t* keys;                // [rows][S]
    uint32_t* flags;               // [rows][S]: chunk meets a split led by NaN
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

// Row `row` of segment sg, indexed from the segment's first vocabulary id.
template <typename TL>
__device__ __forceinline__ const TL* seg_row(const ArgmaxParams& P, int sg, uint32_t row) {
    return (const TL*)P.seg_ptr[sg] + (size_t)row * P.seg_stride[sg];
}

// The value of vocabulary id i in row `row` (any segment; slow paths only).
template <typename TL>
__device__ __forceinline__ float ld_id(const ArgmaxParams& P, uint32_t row, int64_t i) {
    int sg = 0;
    while (sg + 1 < P.nseg && i >= P.seg_begin[sg + 1]) ++sg;
    return ld1<TL>(seg_row<TL>(P, sg, row), i - P.seg_begin[sg]);
}

// Values at or below this never win: -inf, or bf16 lowest() for LOWEST.
__device__ __forceinline__ float start_value(int mode) {
    return mode == LLIMA_ARGMAX_LOWEST ? LLIMA_BF16_LOWEST : -__builtin_inff();
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

// VEC: rows 16-byte aligned and V a multiple of the values per load: every
// chunk is read with 16-byte loads from clamped, always-valid addresses, the
// out-of-row values are masked in registers, and all loads are in flight
// before the first compare.
template <typename TL, int E, bool VEC>
__global__ __launch_bounds__(LLIMA_WG) void argmax_sweep(ArgmaxParams P) {
    constexpr int EPL = 16 / sizeof(TL);
    constexpr int NL = E / EPL;
    constexpr int CHUNK = LLIMA_WG * E;
    __shared__ uint32_t bad_splits;
    __shared__ uint32_t wmax[LLIMA_WAVES], wfi[LLIMA_WAVES];

    uint32_t row, chunk;
    map_row_chunk(blockIdx.x, (uint32_t)P.B, (uint32_t)P.S, &row, &chunk);
    if (row >= (uint32_t)P.B) return;
    int sg = 0;                                   // the chunk's segment (uniform)
    while (sg + 1 < P.nseg && (int)chunk >= P.seg_chunk0[sg + 1]) ++sg;
    const int sb = P.seg_begin[sg], se = P.seg_begin[sg + 1];
    const TL* segp = seg_row<TL>(P, sg, row);     // segp[i - sb] holds vocabulary id i
    const int V = P.V;
    const int c0 = sb + ((int)chunk - P.seg_chunk0[sg]) * CHUNK;
    const int c1 = c0 + CHUNK < se ? c0 + CHUNK : se;

    llima_u32x4 q[NL];
#pragma unroll
    for (int j = 0; j < NL; ++j) {
        const int i0 = c0 + j * (LLIMA_WG * EPL) + (int)threadIdx.x * EPL;
        if constexpr (VEC) {
            const int ia = i0 < se ? i0 : se - EPL;
            q[j] = __builtin_nontemporal_load((const llima_u32x4*)(segp + (ia - sb)));
        } else {
            uint32_t w[4] = {0, 0, 0, 0};
#pragma unroll
            for (int e = 0; e < EPL; ++e) {
                const int ia = i0 + e < se ? i0 + e : se - 1;
                const float f = ld1<TL>(segp, ia - sb);
                if constexpr (sizeof(TL) == 4) w[e] = __float_as_uint(f);
                else w[e >> 1] |= (__float_as_uint(f) >> 16) << ((e & 1) * 16);
            }
            q[j] = llima_u32x4{w[0], w[1], w[2], w[3]};
        }
    }
    // Splits whose first value is NaN are invisible (argmax_bf16 starts its
    // running maximum at values[0]).  Rare: flagged here, the row is then
    // redone exactly by the finish kernel.
    if (threadIdx.x == 0) bad_splits = 0;
    __syncthreads();
    if (P.mode == LLIMA_ARGMAX_SPLIT_FIRST && P.split_segs) {
        if (threadIdx.x == 0 && c0 == sb) {
            const float f = ld1<TL>(segp, 0);
            if (f != f) bad_splits = 1u;
        }
    } else if (P.mode == LLIMA_ARGMAX_SPLIT_FIRST || P.mode == LLIMA_ARGMAX_QUARTERS) {
        // one contiguous segment: splits of split_dim values, or the quarters
        const int sd = (P.split_dim <= 0 || P.split_dim >= V) ? V : P.split_dim;
        const int s_lo = split_of(c0, V, sd, P.mode), s_hi = split_of(c1 - 1, V, sd, P.mode);
        for (int s = s_lo + (int)threadIdx.x; s <= s_hi; s += LLIMA_WG) {
            const float f = ld1<TL>(segp, split_begin(s, V, sd, P.mode));
            if (f != f) bad_splits = 1u;
        }
    }

    // the chunk maximum first (one max per value; values past the row are
    // -inf), then its first index, searched only by the threads that hold it
    float t[NL * EPL];
    const bool full = c1 - c0 == CHUNK;
#pragma unroll
    for (int j = 0; j < NL; ++j) {
        const int i0 = c0 + j * (LLIMA_WG * EPL) + (int)threadIdx.x * EPL;
        const uint32_t w4[4] = {q[j].x, q[j].y, q[j].z, q[j].w};
#pragma unroll
        for (int e = 0; e < EPL; ++e) {
            float f;
            if constexpr (sizeof(TL) == 4) f = __uint_as_float(w4[e]);
            else f = __uint_as_float((e & 1) ? (w4[e >> 1] & 0xFFFF0000u) : (w4[e >> 1] << 16));
            t[j * EPL + e] = full || i0 + e < c1 ? f : -__builtin_inff();
        }
    }
    float mt = -__builtin_inff();                  // fmaxf ignores NaN: a NaN never wins
#pragma unroll
    for (int e = 0; e < NL * EPL; ++e) mt = __builtin_fmaxf(mt, t[e]);
    const uint32_t km = wave_max_u32(mt > start_value(P.mode) ? f32_key(mt) : 0u);
    if (lane_id() == 0) wmax[threadIdx.x >> 6] = km;
    __syncthreads();                               // also: bad_splits final
    uint32_t kc = 0;
#pragma unroll
    for (int w = 0; w < LLIMA_WAVES; ++w) kc = wmax[w] > kc ? wmax[w] : kc;
    const float mc = kc ? key_f32(kc) : -__builtin_inff();
    uint32_t fi = 0xFFFFFFFFu;
    if (kc && mt == mc) {
#pragma unroll
        for (int j = NL - 1; j >= 0; --j) {
            const int i0 = c0 + j * (LLIMA_WG * EPL) + (int)threadIdx.x * EPL;
#pragma unroll
            for (int e = EPL - 1; e >= 0; --e) fi = t[j * EPL + e] == mc ? (uint32_t)(i0 + e) : fi;
        }
    }
    fi = wave_min_u32(fi);
    if (lane_id() == 0) wfi[threadIdx.x >> 6] = fi;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t first = 0xFFFFFFFFu;
#pragma unroll
        for (int w = 0; w < LLIMA_WAVES; ++w) first = wfi[w] < first ? wfi[w] : first;
        P.keys[(size_t)row * P.S + chunk] = kc ? (((uint64_t)kc << 32) | (uint32_t)~first) : 0ull;
        P.flags[(size_t)row * P.S + chunk] = bad_splits;
    }
}

// Row result from its S chunk keys (one wavefront).  A row with nothing above
// the start value gives id 0.  A row with a NaN-led split is rescanned exactly
// by the wavefront.
template <typename TL>
__device__ __forceinline__ int32_t row_result(const ArgmaxParams& P, int row, float* val) {
    const uint64_t* k = P.keys + (size_t)row * P.S;
    const uint32_t* fl = P.flags + (size_t)row * P.S;
    // QUARTERS (one segment): merged from (values[0], 0), read now (independent of the keys)
    const float v0 = P.mode == LLIMA_ARGMAX_QUARTERS ? ld1<TL>(seg_row<TL>(P, 0, row), 0) : 0.0f;
    uint64_t best = 0;
    uint32_t bad = 0;
    for (int i = (int)lane_id(); i < P.S; i += 64) {
        best = k[i] > best ? k[i] : best;
        bad |= fl[i];
    }
    best = wave_max_u64(best);
    bad = wave_max_u32(bad);
    // the value is the key's; the key maps -0 to +0, so a zero is read back
    float v = best ? key_f32((uint32_t)(best >> 32)) : start_value(P.mode);
    if (best && v == 0.0f) v = ld_id<TL>(P, row, (int64_t)(~(uint32_t)best));
    if (bad) {
        float bv = -__builtin_inff();
        uint32_t bi = 0xFFFFFFFFu;
        if (P.split_segs) {
            for (int sg = 0; sg < P.nseg; ++sg) {      // each split buffer is a split
                const TL* sp = seg_row<TL>(P, sg, row);
                const float f0 = ld1<TL>(sp, 0);
                if (f0 != f0) continue;
                const int w = P.seg_begin[sg + 1] - P.seg_begin[sg];
                for (int i = (int)lane_id(); i < w; i += 64) {
                    const float x = ld1<TL>(sp, i);
                    if (x > bv) { bv = x; bi = (uint32_t)(P.seg_begin[sg] + i); }
                }
            }
        } else {
            const TL* rowp = seg_row<TL>(P, 0, row);
            const int V = P.V;
            const int sd = (P.split_dim <= 0 || P.split_dim >= V) ? V : P.split_dim;
            for (int i = (int)lane_id(); i < V; i += 64) {
                const float f = ld1<TL>(rowp, split_begin(split_of(i, V, sd, P.mode), V, sd, P.mode));
                if (f != f) continue;
                const float x = ld1<TL>(rowp, i);
                if (x > bv) { bv = x; bi = (uint32_t)i; }
            }
        }
        best = wave_max_u64(pack_best(bv, bi));
        v = best ? ld_id<TL>(P, row, (int64_t)(~(uint32_t)best)) : -__builtin_inff();
    }
    int32_t id = best ? (int32_t)(~(uint32_t)best) : 0;
    if (P.mode == LLIMA_ARGMAX_QUARTERS && v0 != v0) { id = 0; v = v0; }   // a NaN there is kept
    *val = v;
    return id;
}

template <typename TL>
__global__ __launch_bounds__(LLIMA_WG) void argmax_finish(ArgmaxParams P) {
    __shared__ int32_t tok[ARGMAX_MAX_GROUP];
    const int wave = (int)(threadIdx.x >> 6);
    if (P.epi == EPI_NONE) {
        const int row = finish_row(blockIdx.x, (uint32_t)wave, (uint32_t)P.B);
        if (row < 0) return;
        float v;
        const int32_t id = row_result<TL>(P, row, &v);
        if (lane_id() == 0) {
            if (P.out_ids) P.out_ids[row] = id;
            if (P.out_vals) P.out_vals[row] = v;
        }
        return;
    }
    // one workgroup per sequence (chain) or for the whole tree
    const int nrows = P.epi == EPI_CHAIN ? P.D + 1 : P.B;
    const int row0 = P.epi == EPI_CHAIN ? (int)blockIdx.x * nrows : 0;
    for (int r = wave; r < nrows; r += LLIMA_WAVES) {
        float v;
        const int32_t id = row_result<TL>(P, row0 + r, &v);
        if (lane_id() == 0) tok[r] = id;
    }
    __syncthreads();
    if (threadIdx.x != 0) return;
    if (P.epi == EPI_CHAIN) {
        // resolve_draft_tokens: accept while the draft equals the target argmax,
        // then emit the target token at the first mismatch (or the bonus).
        const int D = P.D, g = (int)blockIdx.x;
        const int32_t* dr = P.draft_ids + (size_t)g * D;
        int32_t* em = P.emitted + (size_t)g * (D + 1);
        int acc = 0;
        while (acc < D && dr[acc] == tok[acc]) { em[acc] = dr[acc]; ++acc; }
        em[acc] = tok[acc];
        for (int j = acc + 1; j <= D; ++j) em[j] = -1;
        P.accepted_len[g] = acc;
    } else {
        // gather target tokens along each path (-1 -> last tree row), then the
        // first path with the strictly longest accepted prefix wins.
        const int K = P.B, L = P.L;
        int32_t best_c = 0, max_acc = 0;
        for (int p = 0; p < P.n_paths; ++p) {
            int32_t acc = 0;
            for (int i = 0; i + 1 < L; ++i) {
                int32_t idx = P.retrieve[p * L + i];
                if (idx < 0 || idx >= K) idx = K - 1;
                const int32_t nxt = P.candidates[p * L + i + 1];
                if (nxt < 0 || tok[idx] != nxt) break;
                ++acc;
            }
            if (acc > max_acc) { max_acc = acc; best_c = p; }
        }
        int32_t idx = P.retrieve[best_c * L + max_acc];
        if (idx < 0 || idx >= K) idx = K - 1;
        P.tree_out[0] = best_c;
        P.tree_out[1] = max_acc;
        P.tree_out[2] = tok[idx];
    }
}

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

struct ATile { int E, S; };
static ATile argmax_tile(int B, int V, int dtype) {
    // 16 KB per workgroup streams best on MI355X; smaller when the grid is small.
    int E = dtype == LLIMA_F32 ? 16 : 32;
    auto S_of = [&](int e) { return (V + LLIMA_WG * e - 1) / (LLIMA_WG * e); };
    while (E > 8 && (int64_t)B * S_of(E) < 1024) E /= 2;
    return {E, S_of(E)};
}

template <typename TL, int E>
static hipError_t launch_argmax(const ArgmaxParams& P, hipStream_t st) {
    const dim3 g((uint32_t)P.B * (uint32_t)P.S), b(LLIMA_WG);
    if (P.vec_ok) hipLaunchKernelGGL((argmax_sweep<TL, E, true>), g, b, 0, st, P);
    else hipLaunchKernelGGL((argmax_sweep<TL, E, false>), g, b, 0, st, P);
    const uint32_t nfin = P.epi == EPI_NONE ? finish_row_blocks((uint32_t)P.B)
                        : P.epi == EPI_CHAIN ? (uint32_t)(P.B / (P.D + 1)) : 1u;
    hipLaunchKernelGGL((argmax_finish<TL>), dim3(nfin), dim3(LLIMA_WG), 0, st, P);
    return hipGetLastError();
}

static int run_argmax(ArgmaxParams& P, int dtype, hipStream_t st) {
    const ATile t = argmax_tile(P.B, P.V, dtype);
    const int chunk = LLIMA_WG * t.E;
    const size_t esz = dtype == LLIMA_F32 ? 4 : 2;
    const int epl = (int)(16 / esz);
    int S = 0;
    P.vec_ok = 1;
    for (int sg = 0; sg < P.nseg; ++sg) {
        const int w = P.seg_begin[sg + 1] - P.seg_begin[sg];
        P.seg_chunk0[sg] = S;
        S += (w + chunk - 1) / chunk;
        P.vec_ok &= ((uintptr_t)P.seg_ptr[sg] % 16 == 0) &&
                    ((P.seg_stride[sg] * (int64_t)esz) % 16 == 0) && (w % epl == 0);
    }
    P.seg_chunk0[P.nseg] = S;
    P.S = S;
    P.flags = (uint32_t*)((char*)P.keys + align256((size_t)P.B * S * sizeof(uint64_t)));
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

// One contiguous buffer: a single segment.
static void one_segment(ArgmaxParams& P, const void* logits, int64_t row_stride, int V) {
    P.nseg = 1;
    P.split_segs = 0;
    P.seg_ptr[0] = logits;
    P.seg_stride[0] = row_stride;
    P.seg_begin[0] = 0;
    P.seg_begin[1] = V;
}

// Split buffers: buffer i holds vocabulary ids [sum of widths before i, + width i),
// rows at strides[i] elements (widths[i] when strides is null).  Returns V, or
// -1 for an invalid description.
static int64_t split_segments(ArgmaxParams& P, const void* const* splits, const int32_t* widths,
                              const int64_t* strides, int32_t n, int32_t B) {
    if (!widths || n < 1 || n > ARGMAX_MAX_SEGS || (B > 0 && !splits)) return -1;
    int64_t V = 0;
    P.nseg = n;
    P.split_segs = 1;
    for (int i = 0; i < n; ++i) {
        const int64_t st = strides ? strides[i] : widths[i];
        if (widths[i] <= 0 || st < widths[i] || (B > 0 && !splits[i])) return -1;
        P.seg_ptr[i] = B > 0 ? splits[i] : nullptr;
        P.seg_stride[i] = st;
        P.seg_begin[i] = (int32_t)V;
        V += widths[i];
        if (V > INT32_MAX) return -1;
    }
    P.seg_begin[n] = (int32_t)V;
    return V;
}

static bool valid_mode(int32_t mode) {
    return mode >= LLIMA_ARGMAX_SPLIT_FIRST && mode <= LLIMA_ARGMAX_LOWEST;
}

static int run_verify_greedy(ArgmaxParams& P, int32_t dtype, int32_t B, int32_t D,
                             const int32_t* draft_ids, int32_t* accepted_len, int32_t* emitted,
                             void* workspace, size_t workspace_bytes, hipStream_t st) {
    if (!workspace || workspace_bytes < llima_verify_greedy_workspace_bytes(B, D, P.V, dtype))
        return LLIMA_E_WORKSPACE;
    P.keys = (uint64_t*)workspace;
    P.B = B * (D + 1);
    P.epi = EPI_CHAIN; P.D = D;
    P.draft_ids = draft_ids; P.accepted_len = accepted_len; P.emitted = emitted;
    return run_argmax(P, dtype, st);
}

}  // namespace llima

using namespace llima;

extern "C" size_t llima_argmax_workspace_bytes(int32_t B, int32_t V, int32_t dtype) {
    (void)dtype;
    if (B <= 0 || V <= 0) return 0;
    // every split buffer adds at most one partial chunk to a row
    const size_t n = (size_t)B * ((V + ARGMAX_MIN_CHUNK - 1) / ARGMAX_MIN_CHUNK + ARGMAX_MAX_SEGS);
    return align256(n * sizeof(uint64_t)) + align256(n * sizeof(uint32_t));
}

extern "C" int llima_argmax(const void* logits, int32_t dtype, int32_t B, int32_t V,
                            int64_t row_stride, int32_t split_dim, int32_t mode,
                            int32_t* out_ids, float* out_vals, void* workspace,
                            size_t workspace_bytes, void* stream) {
    if (B > 0 && (!logits || !out_ids)) return LLIMA_E_INVAL;   // B = 0: empty buffers may be null
    if (dtype != LLIMA_F32 && dtype != LLIMA_BF16) return LLIMA_E_INVAL;
    if (B < 0 || V <= 0 || row_stride < V || !valid_mode(mode)) return LLIMA_E_INVAL;
    if (B == 0) return LLIMA_OK;
    if (!workspace || workspace_bytes < llima_argmax_workspace_bytes(B, V, dtype))
        return LLIMA_E_WORKSPACE;
    ArgmaxParams P = {};
    one_segment(P, logits, row_stride, V);
    P.out_ids = out_ids;
    P.out_vals = out_vals;
    P.keys = (uint64_t*)workspace;
    P.B = B; P.V = V; P.split_dim = split_dim; P.mode = mode;
    P.epi = EPI_NONE;
    return run_argmax(P, dtype, (hipStream_t)stream);
}

extern "C" int llima_argmax_splits(const void* const* splits, const int32_t* split_widths,
                                   const int64_t* split_row_strides, int32_t n_splits,
                                   int32_t dtype, int32_t B, int32_t mode, int32_t* out_ids,
                                   float* out_vals, void* workspace, size_t workspace_bytes,
                                   void* stream) {
    if (B > 0 && !out_ids) return LLIMA_E_INVAL;
    if (dtype != LLIMA_F32 && dtype != LLIMA_BF16) return LLIMA_E_INVAL;
    if (B < 0 || !valid_mode(mode) || mode == LLIMA_ARGMAX_QUARTERS) return LLIMA_E_INVAL;
    ArgmaxParams P = {};
    const int64_t V = split_segments(P, splits, split_widths, split_row_strides, n_splits, B);
    if (V <= 0) return LLIMA_E_INVAL;
    if (B == 0) return LLIMA_OK;
    if (!workspace || workspace_bytes < llima_argmax_workspace_bytes(B, (int32_t)V, dtype))
        return LLIMA_E_WORKSPACE;
    P.out_ids = out_ids;
    P.out_vals = out_vals;
    P.keys = (uint64_t*)workspace;
    P.B = B; P.V = (int32_t)V; P.split_dim = 0; P.mode = mode;
    P.epi = EPI_NONE;
    return run_argmax(P, dtype, (hipStream_t)stream);
}

extern "C" size_t llima_verify_greedy_workspace_bytes(int32_t B, int32_t D, int32_t V,
                                                      int32_t dtype) {
    if (B <= 0 || D < 0) return 0;
    return llima_argmax_workspace_bytes(B * (D + 1), V, dtype);
}

extern "C" int llima_verify_greedy(const void* target_logits, int32_t dtype, int32_t B, int32_t D,
                                   int32_t V, int32_t split_dim, int32_t mode,
                                   const int32_t* draft_ids, int32_t* accepted_len,
                                   int32_t* emitted, void* workspace, size_t workspace_bytes,
                                   void* stream) {
    if (B > 0 && (!target_logits || !accepted_len || !emitted || (D > 0 && !draft_ids)))
        return LLIMA_E_INVAL;
    if (dtype != LLIMA_F32 && dtype != LLIMA_BF16) return LLIMA_E_INVAL;
    if (B < 0 || D < 0 || D + 1 > ARGMAX_MAX_GROUP || V <= 0 || !valid_mode(mode))
        return LLIMA_E_INVAL;
    if (B == 0) return LLIMA_OK;
    ArgmaxParams P = {};
    one_segment(P, target_logits, V, V);
    P.V = V; P.split_dim = split_dim; P.mode = mode;
    return run_verify_greedy(P, dtype, B, D, draft_ids, accepted_len, emitted, workspace,
                             workspace_bytes, (hipStream_t)stream);
}

extern "C" int llima_verify_greedy_splits(const void* const* splits, const int32_t* split_widths,
                                          const int64_t* split_row_strides, int32_t n_splits,
                                          int32_t dtype, int32_t B, int32_t D, int32_t mode,
                                          const int32_t* draft_ids, int32_t* accepted_len,
                                          int32_t* emitted, void* workspace,
                                          size_t workspace_bytes, void* stream) {
    if (B > 0 && (!accepted_len || !emitted || (D > 0 && !draft_ids))) return LLIMA_E_INVAL;
    if (dtype != LLIMA_F32 && dtype != LLIMA_BF16) return LLIMA_E_INVAL;
    if (B < 0 || D < 0 || D + 1 > ARGMAX_MAX_GROUP || !valid_mode(mode) ||
        mode == LLIMA_ARGMAX_QUARTERS)
        return LLIMA_E_INVAL;
    ArgmaxParams P = {};
    const int64_t V = split_segments(P, splits, split_widths, split_row_strides, n_splits, B);
    if (V <= 0) return LLIMA_E_INVAL;
    if (B == 0) return LLIMA_OK;
    P.V = (int32_t)V; P.split_dim = 0; P.mode = mode;
    return run_verify_greedy(P, dtype, B, D, draft_ids, accepted_len, emitted, workspace,
                             workspace_bytes, (hipStream_t)stream);
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
    if (K <= 0 || K > ARGMAX_MAX_GROUP || V <= 0 || n_paths <= 0 || L <= 0) return LLIMA_E_INVAL;
    if (!workspace || workspace_bytes < llima_verify_tree_workspace_bytes(K, V, dtype))
        return LLIMA_E_WORKSPACE;
    ArgmaxParams P = {};
    one_segment(P, tree_logits, V, V);
    P.keys = (uint64_t*)workspace;
    // The EAGLE3 verify argmax starts from -inf (language_model_eagle3.cpp:491-521).
    P.B = K; P.V = V; P.split_dim = 0; P.mode = LLIMA_ARGMAX_NEG_INF;
    P.epi = EPI_TREE;
    P.retrieve = retrieve_indices; P.candidates = candidates; P.n_paths = n_paths; P.L = L;
    P.tree_out = out;
    return run_argmax(P, dtype, (hipStream_t)stream);
}

extern "C" const char* llima_status_string(int status) {
    switch (status) {
        case LLIMA_OK: return "ok";
        case LLIMA_E_INVAL: return "invalid argument";
        case LLIMA_E_RANGE: return "value out of range";
        case LLIMA_E_HIP: return "HIP launch error";
        case LLIMA_E_WORKSPACE: return "workspace missing or too small";
        case LLIMA_E_SCRATCH: return "call exceeds the library's static scratch";
        case LLIMA_E_CAPTURE: return "first call on this device made under stream capture";
        default: return "unknown status";
    }
}

extern "C" int llima_abi_version(void) { return 2; }
