// lmhead.hip -- LM-head matrix-vector product with a fused softcap and argmax
// epilogue for decode-sized batches on MI355X (gfx950).
//
//   logits[b][v] = cap * tanh(s / cap) (s when cap <= 0),  s = sum_h hidden[b][h] * weight[v][h]
//
// hidden [B][H] bf16, weight [V][H] bf16 (the nn.Linear layout: one vocab row
// contiguous), fp32 products and sums; then the first index of each row's
// maximum (NaN never wins).  The reference computes the LM head on the NPU and,
// with one split, takes its argmax in-graph after Gemma's softcap
// (sima_lmm/model/language_part_base.py:171-180, sima_lmm/model/model_graph.py:601,
// 868-870); the host reads back one int32 (sima_lmm/devkit/cpp/language_model.cpp:1607-1609).
//
// At decode batch sizes the product is bound by reading the weights (V H 2
// bytes, read once per pass of up to 8 hidden rows); batches that would need
// more than one such pass take the MFMA tiling further down (one pass per 256
// rows).
//
// lmh_rows: 512-thread workgroups; the pass's hidden rows (NB of them) are
// staged in LDS as fp32; each wave streams whole vocab rows (lane l holds ids
// h = 8 l + 512 j of a row, 16-byte loads, the next row's loads issued before
// the current row is summed), sums each hidden row's products in fp32 (per
// lane in h order, then across the wave), applies the softcap, optionally
// writes the logits, and keeps per hidden row the 64-bit key
// (value key << 32 | ~v) of its best vocab row.  lmh_finish: one workgroup per
// hidden row reduces the waves' keys.
//
// Scoring epilogue (every path, a compile-time flag): beside its key, each key
// slot (a wave's vocab rows of one hidden row) keeps s_w = sum of
// exp(logit - m_w) over its logits, m_w its greatest non-NaN logit (the key's
// value), and the wave holding the target id stores the target's logit;
// lmh_score_finish combines the slots in double into the log-softmax at the
// target and the first-maximum flag of score_logits
// (sima_lmm/devkit/cpp/language_model.cpp:29-62) over the logits as the
// argmax sees them, so scoring never writes or reads the [B][V] logits.
//
// Verification through the head: the argmax of every draft row, then
// lmh_chain (greedy chains, one thread per sequence) or lmh_tree (the EAGLE3
// tree, one thread) applies the rule of llima_verify_greedy / llima_verify_tree
// to the ids, again with no logits written.
#include "common.hpp"
#include "../../include/llima_sampler.h"

namespace llima {

#define LMH_WG 512
#define LMH_WAVES (LMH_WG / 64)
#define LMH_MAX_H 4096                 // 8 load rounds of 512 ids per vocab row
#define LMH_R (LMH_MAX_H / 512)
#define LMH_LDS_FLOATS 16384           // 64 KB of staged hidden values

struct LmhParams {
    const uint16_t* hidden;            // [B][H]
    const uint16_t* weight;            // [V][H]
    float* out_logits;                 // [B][V] or null
    uint64_t* keys;                    // [B][NW]
    int32_t* out_ids;
    float* out_vals;                   // or null
    int32_t B, H, V, NW;
    float cap;
    int32_t round_bf16;                // logits rounded to bf16 before the argmax
    int32_t logits_bf16;               // out_logits holds bf16 [B][V] (LLIMA_LOGITS_OUT_BF16)
    // scoring epilogue
    float* sums;                       // [B][NW] s_w of each key slot (NaN: a NaN logit)
    float* tval;                       // [B] the target's logit
    const int32_t* targets;            // [B]
    double* out_logprob;               // [B]
    int32_t* out_greedy;               // [B]
};

// The logit as the argmax sees it: softcapped, then (round_bf16) rounded to
// the nearest bf16, ties to even (NaN stays NaN), the precision of the
// reference's executed graphs (model_graph.py:30-45), in which equal bf16
// logits tie and the lower index wins.
__device__ __forceinline__ float lmh_logit(float s, const LmhParams& P) {
    if (P.cap > 0.0f) s = P.cap * tanhf(s / P.cap);
    if (P.round_bf16 && s == s) {
        const uint32_t u = __float_as_uint(s);
        s = __uint_as_float((u + 0x7FFFu + ((u >> 16) & 1u)) & 0xFFFF0000u);
    }
    return s;
}

// lmh_logit over a tile's values, its two decisions taken once for the tile;
// the rounding selects NaN through unchanged rather than branching.
template <int WR>
__device__ __forceinline__ void lmh_logit_tile(float (&v)[16][WR], const LmhParams& P) {
    if (P.cap > 0.0f) {                                      // uniform
#pragma unroll
        for (int i = 0; i < 16; ++i)
#pragma unroll
            for (int j = 0; j < WR; ++j) v[i][j] = P.cap * tanhf(v[i][j] / P.cap);
    }
    if (P.round_bf16) {                                      // uniform
#pragma unroll
        for (int i = 0; i < 16; ++i)
#pragma unroll
            for (int j = 0; j < WR; ++j) {
                const float s = v[i][j];
                const uint32_t u = __float_as_uint(s);
                const float q = __uint_as_float((u + 0x7FFFu + ((u >> 16) & 1u)) & 0xFFFF0000u);
                v[i][j] = s == s ? q : s;
            }
    }
}

// Writes logit i of the [B][V] output: fp32, or the bf16 it was rounded to
// (its upper 16 bits; a NaN as the quiet NaN).
__device__ __forceinline__ void lmh_store_logit(const LmhParams& P, size_t i, float v) {
    if (P.logits_bf16)
        ((uint16_t*)P.out_logits)[i] = v == v ? (uint16_t)(__float_as_uint(v) >> 16) : (uint16_t)0x7FC0u;
    else
        P.out_logits[i] = v;
}

#define LMH_LOG2E 1.44269504088896340736f

// Scoring statistics of one key slot, one logit at a time: m the greatest
// non-NaN logit so far, s the sum of exp(v - m) over its logits above -inf
// (rescaled when m grows).  A NaN logit makes s NaN for good (s * 0 keeps it),
// and so does a second +inf: the row's result is NaN either way.
__device__ __forceinline__ void lmh_stat_push(float& m, float& s, float v) {
    if (v != v) {
        s = __builtin_nanf("");
    } else if (v > m) {
        s = s * (m > -__builtin_inff() ? __builtin_amdgcn_exp2f((m - v) * LMH_LOG2E) : 0.0f) + 1.0f;
        m = v;
    } else if (v > -__builtin_inff()) {
        s += __builtin_amdgcn_exp2f((v - m) * LMH_LOG2E);
    }
}

// One logit's term of its key slot's sum, mw the slot's greatest non-NaN logit:
// exp(v - mw); 0 past the vocabulary (in false) and for -inf, NaN for NaN.
__device__ __forceinline__ float lmh_term(float v, float mw, bool in) {
    const float e = v > -__builtin_inff() ? __builtin_amdgcn_exp2f((v - mw) * LMH_LOG2E) : 0.0f;
    return !in ? 0.0f : v != v ? __builtin_nanf("") : e;
}

__device__ __forceinline__ float wave_sum_f32(float v) {
    return __uint_as_float(wave_reduce<uint32_t>(
        __float_as_uint(v), 0u,
        [](uint32_t a, uint32_t b) { return __float_as_uint(__uint_as_float(a) + __uint_as_float(b)); }));
}

// One vocab row's 8 rounds of 16-byte loads (8 bf16 each) for this lane;
// rounds past H, and every round when v < 0, read the weights' first 16 bytes.
__device__ __forceinline__ void issue_row(const LmhParams& P, int v, llima_u32x4 (&w)[LMH_R]) {
    const uint16_t* row = P.weight + (size_t)(v < 0 ? 0 : v) * P.H;
#pragma unroll
    for (int j = 0; j < LMH_R; ++j) {
        const int h0 = (int)lane_id() * 8 + j * 512;
        const int ho = v >= 0 && h0 < P.H ? h0 : 0;
        w[j] = __builtin_nontemporal_load((const llima_u32x4*)(row + ho));
    }
}

template <int NB, bool SC>
__global__ __launch_bounds__(LMH_WG) void lmh_rows(LmhParams P, int b0, int nb) {
    __shared__ __align__(16) float xs[LMH_LDS_FLOATS];
    const int H = P.H;
    // stage hidden rows b0 .. b0 + nb - 1 as fp32 (rows nb .. NB - 1 are zero)
    for (int i = (int)threadIdx.x * 8; i < NB * H; i += LMH_WG * 8) {
        const int b = i / H, h = i - b * H;                  // H % 8 == 0: one row per group
        llima_u32x4 q = {0u, 0u, 0u, 0u};
        if (b < nb) q = *(const llima_u32x4*)(P.hidden + (size_t)(b0 + b) * H + h);
        const uint32_t u[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            xs[i + 2 * e] = __uint_as_float(u[e] << 16);
            xs[i + 2 * e + 1] = __uint_as_float(u[e] & 0xFFFF0000u);
        }
    }
    __syncthreads();
    const uint32_t lane = lane_id();
    const int wg = (int)blockIdx.x * LMH_WAVES + (int)(threadIdx.x >> 6);
    uint64_t best[NB];
    float sm[NB], ss[NB];                                    // scoring: m and s of this slot
    int32_t tg[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        best[b] = 0;
        sm[b] = -__builtin_inff();
        ss[b] = 0.0f;
        tg[b] = SC && b < nb ? P.targets[b0 + b] : -1;
    }
    llima_u32x4 wc[LMH_R], wn[LMH_R];
    int v = wg;
    issue_row(P, v < P.V ? v : -1, wc);
    while (v < P.V) {
        const int vn = v + P.NW;
        issue_row(P, vn < P.V ? vn : -1, wn);                // in flight while this row is summed
        float acc[NB];
#pragma unroll
        for (int b = 0; b < NB; ++b) acc[b] = 0.0f;
#pragma unroll
        for (int j = 0; j < LMH_R; ++j) {
            const int h0 = (int)lane * 8 + j * 512;
            if (h0 < H) {
                const uint32_t u[4] = {wc[j].x, wc[j].y, wc[j].z, wc[j].w};
                float wf[8];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    wf[2 * e] = __uint_as_float(u[e] << 16);
                    wf[2 * e + 1] = __uint_as_float(u[e] & 0xFFFF0000u);
                }
#pragma unroll
                for (int b = 0; b < NB; ++b) {
                    const float* xr = xs + b * H + h0;
                    const float4 x0 = *(const float4*)xr, x1 = *(const float4*)(xr + 4);
                    float a = acc[b];
                    a = __builtin_fmaf(wf[0], x0.x, a); a = __builtin_fmaf(wf[1], x0.y, a);
                    a = __builtin_fmaf(wf[2], x0.z, a); a = __builtin_fmaf(wf[3], x0.w, a);
                    a = __builtin_fmaf(wf[4], x1.x, a); a = __builtin_fmaf(wf[5], x1.y, a);
                    a = __builtin_fmaf(wf[6], x1.z, a); a = __builtin_fmaf(wf[7], x1.w, a);
                    acc[b] = a;
                }
            }
        }
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            const float s = lmh_logit(wave_sum_f32(acc[b]), P);
            if (b < nb && P.out_logits && lane == 0) lmh_store_logit(P, (size_t)(b0 + b) * P.V + v, s);
            const uint64_t key = s == s ? ((uint64_t)f32_key(s) << 32) | (uint32_t)~(uint32_t)v : 0ull;
            best[b] = key > best[b] ? key : best[b];
            if constexpr (SC) {
                lmh_stat_push(sm[b], ss[b], s);
                if (lane == 0 && b < nb && v == tg[b]) P.tval[b0 + b] = s;
            }
        }
#pragma unroll
        for (int j = 0; j < LMH_R; ++j) wc[j] = wn[j];
        v = vn;
    }
    if (lane == 0) {
#pragma unroll
        for (int b = 0; b < NB; ++b)
            if (b < nb) {
                P.keys[(size_t)(b0 + b) * P.NW + wg] = best[b];
                if constexpr (SC) P.sums[(size_t)(b0 + b) * P.NW + wg] = ss[b];
            }
    }
}

// ------------------------------------------------------------------ MFMA path
// Batches wider than one GEMV pass: gfx950's v_mfma_f32_32x32x16_bf16 tiles,
// the weight read once per pass of up to 256 hidden rows.  Lane l supplies row
// (A: a hidden row) or column (B: a vocab row) l % 32 and 8 consecutive values
// of k; the k assignment only has to be the same for both operands, and step s
// of a 64-id chunk gives lane half g the ids 16 s + 8 g .. 16 s + 8 g + 7, so
// every id of the chunk is used once.  Accumulator element i of lane l is
// C[i % 4 + 8 (i / 4) + 4 (l / 32)][l % 32].  The order of the fp32 sum over k
// is not the GEMV path's.
typedef __bf16 lmh_b8 __attribute__((ext_vector_type(8)));
typedef float lmh_acc __attribute__((ext_vector_type(16)));
#define LMH_MB 256                     // hidden rows per pass at most

__device__ __forceinline__ uint64_t lmh_key(float s, int n, int V) {
    return s == s && n < V ? ((uint64_t)f32_key(s) << 32) | (uint32_t)~(uint32_t)n : 0ull;
}

// Sum over the 32 lanes of this lane's half-wave.
__device__ __forceinline__ float half_sum_f32(float v) {
#pragma unroll
    for (int o = 16; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// Half-wave collectives over the 16 rows of a 32 x 32 accumulator tile, whose
// lane (r, g) holds rows i % 4 + 8 (i / 4) + 4 g (i < 16).  The reduce-scatter
// exchanges with lanes r ^ 16, r ^ 8, r ^ 4, r ^ 2 (each time keeping the half
// of its rows the lane's bit selects and combining them with the partner's)
// and r ^ 1, leaving lanes r and r ^ 1 with row (r >> 1) % 16's result over
// the half-wave: 16 shuffles for 16 rows, where a reduction per row takes 80.
// The all-gather returns every row's value to every lane (15 shuffles).
__device__ __forceinline__ uint64_t shfl_xor_t(uint64_t v, int m) {
    const uint32_t lo = (uint32_t)__shfl_xor((int)(uint32_t)v, m, 64);
    const uint32_t hi = (uint32_t)__shfl_xor((int)(uint32_t)(v >> 32), m, 64);
    return ((uint64_t)hi << 32) | lo;
}
__device__ __forceinline__ uint32_t shfl_xor_t(uint32_t v, int m) {
    return (uint32_t)__shfl_xor((int)v, m, 64);
}
__device__ __forceinline__ float shfl_xor_t(float v, int m) { return __shfl_xor(v, m, 64); }

template <class T, int N>
__device__ __forceinline__ void half_rs_step(const T (&a)[2 * N], T (&b)[N], int r, int bit,
                                             T (*op)(T, T)) {
    const bool hi = (r & bit) != 0;
#pragma unroll
    for (int k = 0; k < N; ++k) {
        const T send = hi ? a[k] : a[k + N], keep = hi ? a[k + N] : a[k];
        b[k] = op(keep, shfl_xor_t(send, bit));
    }
}

template <class T>
__device__ __forceinline__ T half_reduce_scatter16(const T (&a)[16], int r, T (*op)(T, T)) {
    T b8[8], b4[4], b2[2], b1[1];
    half_rs_step<T, 8>(a, b8, r, 16, op);
    half_rs_step<T, 4>(b8, b4, r, 8, op);
    half_rs_step<T, 2>(b4, b2, r, 4, op);
    half_rs_step<T, 1>(b2, b1, r, 2, op);
    return op(b1[0], shfl_xor_t(b1[0], 1));
}

__device__ __forceinline__ void half_all_gather16(uint32_t own, int r, uint32_t (&h)[16]) {
    const int ir = (r >> 1) & 15;
    h[0] = own;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        const bool mine = ((ir >> s) & 1) != 0;
#pragma unroll
        for (int k = 0; k < (1 << s); ++k) {
            const uint32_t cur = h[k], recv = shfl_xor_t(cur, 2 << s);
            h[k] = mine ? recv : cur;
            h[k + (1 << s)] = mine ? cur : recv;
        }
    }
}

__device__ __forceinline__ uint64_t lmh_max_u64(uint64_t a, uint64_t b) { return a > b ? a : b; }
__device__ __forceinline__ float lmh_add_f32(float a, float b) { return a + b; }

// The epilogue of one 32 x 32 accumulator tile over WR column blocks: lane
// (r, g) holds v[i][j], the logit of tile row i % 4 + 8 (i / 4) + 4 g (pass row
// mbase + that) and column ncol[j].  Writes the logits (when asked) and each
// row's greatest key over the wave's 32 WR columns into key slot wv; with SC
// also the slot's sum of exp(logit - its maximum) and the target's logit (tg[i]:
// row i's target, -1 for rows past nb).
template <int WR, bool SC>
__device__ __forceinline__ void lmh_tile_out(const LmhParams& P, const float (&v)[16][WR],
                                             const int (&ncol)[WR], int mbase, int b0, int nb,
                                             int wv, int r, int g, const int32_t (&tg)[16]) {
    const int V = P.V;
    if (P.out_logits) {                                      // uniform
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int m = mbase + (i & 3) + 8 * (i >> 2) + 4 * g;
#pragma unroll
            for (int j = 0; j < WR; ++j)
                if (m < nb && ncol[j] < V) lmh_store_logit(P, (size_t)(b0 + m) * V + ncol[j], v[i][j]);
        }
    }
    uint64_t k[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        k[i] = 0;
#pragma unroll
        for (int j = 0; j < WR; ++j) k[i] = lmh_max_u64(k[i], lmh_key(v[i][j], ncol[j], V));
    }
    const uint64_t best = half_reduce_scatter16<uint64_t>(k, r, lmh_max_u64);
    const int ir = (r >> 1) & 15, mr = mbase + (ir & 3) + 8 * (ir >> 2) + 4 * g;
    const bool st = (r & 1) == 0 && mr < nb;                 // one lane per row stores
    if (st) P.keys[(size_t)(b0 + mr) * P.NW + wv] = best;
    if constexpr (SC) {
        uint32_t hv[16];                                     // each row's maximum key
        half_all_gather16((uint32_t)(best >> 32), r, hv);
        float e[16];
        bool hit = false;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const float mw = hv[i] ? key_f32(hv[i]) : -__builtin_inff();
            e[i] = 0.0f;
#pragma unroll
            for (int j = 0; j < WR; ++j) {
                e[i] += lmh_term(v[i][j], mw, ncol[j] < V);
                hit |= ncol[j] < V && ncol[j] == tg[i];
            }
        }
        const float sw = half_reduce_scatter16<float>(e, r, lmh_add_f32);
        if (st) P.sums[(size_t)(b0 + mr) * P.NW + wv] = sw;
        if (hit) {                                           // one lane of the grid per row
#pragma unroll
            for (int i = 0; i < 16; ++i)
#pragma unroll
                for (int j = 0; j < WR; ++j)
                    if (ncol[j] < V && ncol[j] == tg[i])
                        P.tval[b0 + mbase + (i & 3) + 8 * (i >> 2) + 4 * g] = v[i][j];
        }
    }
}

// Workgroup tile: 32 NWN vocab rows x 64 WM hidden rows, 64 NWN WM threads.
// Wave w computes vocab rows 32 (w % NWN) .. + 31 against hidden rows
// 64 (w / NWN) .. + 63 (two 32 x 32 accumulators); the WM groups of waves share
// the staged weights, the NWN vocab tiles the staged hidden rows.  k in chunks of 64 ids (128 bytes of a row), each read with
// coalesced 16-byte loads (8 threads per row: whole 128-byte lines) and taken
// global -> registers -> LDS (rows padded by 16 bytes, double-buffered,
// one barrier per chunk).  The registers form a ring of R chunks, so R chunks
// are in flight while one feeds the MFMAs: a chunk's loads are requested R
// iterations before it is staged.
#define LMH_KC 64                      // the H multiple the MFMA path needs

template <int NWN, int WM, int R, int KC, bool SC>
__global__ __launch_bounds__(64 * NWN * WM) void lmh_mfma(LmhParams P, int b0, int nb) {
    constexpr int NT = 64 * NWN * WM;                        // threads
    constexpr int WR = 32 * NWN;                             // vocab rows of the workgroup
    constexpr int M = 64 * WM;                               // hidden rows of the pass
    constexpr int PPR = KC / 8;                              // 16-byte pieces per row per chunk
    constexpr int LDSR = 2 * KC + 16;                        // bytes per staged row (16-byte aligned)
    constexpr int WQ = WR * PPR / NT;                        // weight pieces per thread per chunk
    constexpr int XQ = M * PPR / NT;                         // hidden pieces per thread per chunk
    static_assert(WQ * NT == WR * PPR && XQ * NT == M * PPR, "pieces split evenly");
    __shared__ __align__(16) uint8_t lw[2][WR * LDSR];
    __shared__ __align__(16) uint8_t lx[2][M * LDSR];
    const int t = (int)threadIdx.x, lane = t & 63, wave = t >> 6, g = lane >> 5, r = lane & 31;
    const int wn = wave % NWN, wm = wave / NWN;              // vocab tile, hidden group
    const int n0 = (int)blockIdx.x * WR;
    const int H = P.H, V = P.V, nch = H / KC;
    // global -> LDS mapping: piece p = t + NT q is row p / PPR, 16-byte column p % PPR
    const int pc = t % PPR;
    const uint16_t* gw[WQ];
#pragma unroll
    for (int q = 0; q < WQ; ++q) {
        const int n = n0 + (t + NT * q) / PPR;               // rows past V read row V - 1
        gw[q] = P.weight + (size_t)(n < V ? n : V - 1) * H + pc * 8;
    }
    const uint16_t* gx[XQ];
#pragma unroll
    for (int q = 0; q < XQ; ++q) {
        const int m = (t + NT * q) / PPR;                    // rows past nb read row b0
        gx[q] = P.hidden + (size_t)(b0 + (m < nb ? m : 0)) * H + pc * 8;
    }
    llima_u32x4 rw[R][WQ], rx[R][XQ];
    auto fetch = [&](int c, llima_u32x4 (&fw)[WQ], llima_u32x4 (&fx)[XQ]) {
#pragma unroll
        for (int q = 0; q < WQ; ++q) fw[q] = __builtin_nontemporal_load((const llima_u32x4*)(gw[q] + c * KC));
#pragma unroll
        for (int q = 0; q < XQ; ++q) fx[q] = *(const llima_u32x4*)(gx[q] + c * KC);
    };
    auto stage = [&](const llima_u32x4 (&fw)[WQ], const llima_u32x4 (&fx)[XQ], int buf) {
#pragma unroll
        for (int q = 0; q < WQ; ++q)
            *(llima_u32x4*)(lw[buf] + (t + NT * q) / PPR * LDSR + pc * 16) = fw[q];
#pragma unroll
        for (int q = 0; q < XQ; ++q)
            *(llima_u32x4*)(lx[buf] + (t + NT * q) / PPR * LDSR + pc * 16) = fx[q];
    };
    lmh_acc acc[2];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[mt][i] = 0.0f;
    // prologue: chunks 0 .. R-1 requested, chunk 0 staged
#pragma unroll
    for (int i = 0; i < R; ++i) fetch(i < nch ? i : 0, rw[i], rx[i]);
    stage(rw[0], rx[0], 0);
    __syncthreads();
    // Loads and stages are unconditional (a chunk index past the last reads
    // the last chunk again, a stage past it fills a buffer nobody reads), so
    // the loop body is straight-line code for the wait counters: staging chunk
    // c + 1 waits only for its own loads, not for the R - 1 chunks behind it.
    for (int c0 = 0; c0 < nch; c0 += R) {
#pragma unroll
        for (int i = 0; i < R; ++i) {
            const int c = c0 + i;                            // in LDS buffer c & 1
            // ring slot i held chunk c (staged): it now receives chunk c + R
            fetch(c + R < nch ? c + R : nch - 1, rw[i], rx[i]);
            const int buf = c & 1;
            if (c < nch) {                                   // uniform
                const uint8_t* wrow = lw[buf] + (wn * 32 + r) * LDSR + 16 * g;
                const uint8_t* xrow = lx[buf] + (wm * 64 + r) * LDSR + 16 * g;
#pragma unroll
                for (int s = 0; s < KC / 16; ++s) {
                    const lmh_b8 bo = *(const lmh_b8*)(wrow + 32 * s);
                    const lmh_b8 a0 = *(const lmh_b8*)(xrow + 32 * s);
                    const lmh_b8 a1 = *(const lmh_b8*)(xrow + 32 * LDSR + 32 * s);
                    acc[0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, bo, acc[0], 0, 0, 0);
                    acc[1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, bo, acc[1], 0, 0, 0);
                }
            }
            // chunk c + 1 (ring slot (i + 1) % R) into the other buffer, whose
            // last readers passed the previous barrier
            stage(rw[(i + 1) % R], rx[(i + 1) % R], buf ^ 1);
            __syncthreads();
        }
    }
    // key slots past this grid's waves (a grid of 128-row tiles can leave up
    // to 4 of the P.NW slots, counted in 256-row tiles): no logit
    if (blockIdx.x == gridDim.x - 1) {
        const int w0 = (int)gridDim.x * NWN, nx = P.NW - w0;
        for (int e = t; e < nx * nb; e += NT) {
            P.keys[(size_t)(b0 + e / nx) * P.NW + w0 + e % nx] = 0;
            if constexpr (SC) P.sums[(size_t)(b0 + e / nx) * P.NW + w0 + e % nx] = 0.0f;
        }
    }
    // epilogue: softcap, logits, and per hidden row the greatest key of the wave's 32 columns
    const int wv = (int)blockIdx.x * NWN + wn;
    const int ncol[1] = {n0 + wn * 32 + r};
    int32_t tgv[2][16];                                      // scoring: the lane's rows' targets,
#pragma unroll                                               // requested together (-1: no row)
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int m = wm * 64 + mt * 32 + (i & 3) + 8 * (i >> 2) + 4 * g;
            tgv[mt][i] = SC && m < nb ? P.targets[b0 + m] : -1;
        }
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
        float v[16][1];
#pragma unroll
        for (int i = 0; i < 16; ++i) v[i][0] = acc[mt][i];
        lmh_logit_tile<1>(v, P);
        lmh_tile_out<1, SC>(P, v, ncol, wm * 64 + mt * 32, b0, nb, wv, r, g, tgv[mt]);
    }
}

// One workgroup per hidden row: the greatest key over the waves (16 loads per
// thread in flight at a time).  A row with no non-NaN logit gives id 0 and a
// NaN value.
__global__ __launch_bounds__(LLIMA_WG) void lmh_finish(LmhParams P) {
    __shared__ BlockScratch bs;
    const int b = (int)blockIdx.x;
    const uint64_t* k = P.keys + (size_t)b * P.NW;
    uint64_t best = 0;
    for (int i0 = 0; i0 < P.NW; i0 += LLIMA_WG * 16) {
        uint64_t kv[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const int i = i0 + j * LLIMA_WG + (int)threadIdx.x;
            kv[j] = k[i < P.NW ? i : 0];
        }
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const bool in = i0 + j * LLIMA_WG + (int)threadIdx.x < P.NW;
            best = in && kv[j] > best ? kv[j] : best;
        }
    }
    best = block_max_u64(best, bs);
    if (threadIdx.x == 0) {
        P.out_ids[b] = best ? (int32_t)~(uint32_t)best : 0;
        if (P.out_vals) P.out_vals[b] = best ? key_f32((uint32_t)(best >> 32)) : __builtin_nanf("");
    }
}

// One workgroup per hidden row of a scoring call: the first maximum M (the
// greatest key), S = sum over the key slots of exp(m_w - M) s_w in double, and
// the target's log-probability x_t - (M + log S): NaN when a logit is NaN or M
// is infinite (as the reference's double sum), a NaN and LLIMA_E_RANGE for a
// target outside [0, V).  The flag is 1 when the target is the first maximum
// (a row with no non-NaN logit has maximum id 0).  Slots are read 16 per
// thread at a time (maximum, then sum; rows of at most 16 slots per thread
// stay in registers between the two).
__global__ __launch_bounds__(LLIMA_WG) void lmh_score_finish(LmhParams P) {
    constexpr int SPAN = LLIMA_WG * 16;
    __shared__ BlockScratch bs;
    const int b = (int)blockIdx.x, t = (int)threadIdx.x;
    const uint64_t* k = P.keys + (size_t)b * P.NW;
    const float* sm = P.sums + (size_t)b * P.NW;
    uint64_t kv[16];
    float sv[16];
    auto load = [&](int i0) {
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const int i = i0 + j * LLIMA_WG + t, ic = i < P.NW ? i : 0;
            kv[j] = k[ic];
            sv[j] = sm[ic];
        }
    };
    uint64_t best = 0;
    uint32_t nan = 0;
    for (int i0 = 0; i0 < P.NW; i0 += SPAN) {
        load(i0);
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const bool in = i0 + j * LLIMA_WG + t < P.NW;
            best = in && kv[j] > best ? kv[j] : best;
            nan |= in && sv[j] != sv[j] ? 1u : 0u;
        }
    }
    best = block_max_u64(best, bs);
    nan = block_max_u32(nan, bs);
    const float M = best ? key_f32((uint32_t)(best >> 32)) : -__builtin_inff();
    const bool finite = M > -__builtin_inff() && M < __builtin_inff();
    double S = 0.0;
    if (finite && !nan) {                                    // uniform
        for (int i0 = 0; i0 < P.NW; i0 += SPAN) {
            if (P.NW > SPAN) load(i0);                       // one span: still in registers
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const bool in = i0 + j * LLIMA_WG + t < P.NW;
                const float mc = kv[j] ? key_f32((uint32_t)(kv[j] >> 32)) : -__builtin_inff();
                if (in && mc > -__builtin_inff()) S += exp((double)mc - (double)M) * (double)sv[j];
            }
        }
    }
    S = block_sum_f64(S, bs);
    if (t != 0) return;
    const int32_t tg = P.targets[b];
    if (tg < 0 || tg >= P.V) {
        P.out_logprob[b] = __builtin_nan("");
        P.out_greedy[b] = LLIMA_E_RANGE;
        return;
    }
    const uint32_t am = best ? ~(uint32_t)best : 0u;
    P.out_logprob[b] = (nan || !finite) ? __builtin_nan("") : (double)P.tval[b] - ((double)M + log(S));
    P.out_greedy[b] = am == (uint32_t)tg ? 1 : 0;
}

// Greedy chain verification from the head's ids, one thread per sequence
// (resolve_draft_tokens, sima_lmm/devkit/cpp/gemma4_mtp_helpers.cpp:81-111):
// accept while the draft equals the target row's argmax, then emit the
// target's token at the first mismatch (or the bonus token), then -1.
__global__ __launch_bounds__(LLIMA_WG) void lmh_chain(const int32_t* ids, const int32_t* draft_ids,
                                                      int32_t* accepted_len, int32_t* emitted,
                                                      int nseq, int D) {
    const int g = (int)(blockIdx.x * LLIMA_WG + threadIdx.x);
    if (g >= nseq) return;
    const int32_t* tok = ids + (size_t)g * (D + 1);
    const int32_t* dr = draft_ids + (size_t)g * D;
    int32_t* em = emitted + (size_t)g * (D + 1);
    int acc = 0;
    while (acc < D && dr[acc] == tok[acc]) { em[acc] = dr[acc]; ++acc; }
    em[acc] = tok[acc];
    for (int j = acc + 1; j <= D; ++j) em[j] = -1;
    accepted_len[g] = acc;
}

// EAGLE3 tree verification from the head's ids, one thread: each row's token
// is its argmax when the row's maximum exceeds -inf, else 0 (the reference's
// scan starts from -inf with a strict >, sima_lmm/devkit/cpp/language_model_eagle3.cpp:486-522);
// the targets gathered along each path (-1 -> the last row), the first path
// with the strictly longest accepted prefix, its bonus token
// (sima_lmm/devkit/cpp/eagle_helpers.hpp:153-195).
__global__ void lmh_tree(const int32_t* ids, const float* vals, int K, const int32_t* retrieve,
                         const int32_t* candidates, int n_paths, int L, int32_t* out) {
    if (blockIdx.x != 0 || threadIdx.x != 0) return;
    auto tok = [&](int r) { return vals[r] > -__builtin_inff() ? ids[r] : 0; };
    int32_t best_c = 0, max_acc = 0;
    for (int p = 0; p < n_paths; ++p) {
        int32_t acc = 0;
        for (int i = 0; i + 1 < L; ++i) {
            int32_t idx = retrieve[p * L + i];
            if (idx < 0 || idx >= K) idx = K - 1;
            const int32_t nxt = candidates[p * L + i + 1];
            if (nxt < 0 || tok(idx) != nxt) break;
            ++acc;
        }
        if (acc > max_acc) { max_acc = acc; best_c = p; }
    }
    int32_t idx = retrieve[best_c * L + max_acc];
    if (idx < 0 || idx >= K) idx = K - 1;
    out[0] = best_c;
    out[1] = max_acc;
    out[2] = tok(idx);
}

// ------------------------------------------------------------------ packed weights
// A weight prepacked once (at model load) in the order the MFMA reads it:
// fragment (rb, s) is 1 KB, lane l's 16 bytes being
//   weight[32 rb + l % 32][16 s + 8 (l / 32) .. + 7]
// (rows past V zero), at offset ((s / 8) 8 NRB + 8 rb + s % 8) KB: a row
// block's 8 k-steps of a group are 8 KB of contiguous memory, and the NRB row
// blocks' groups follow each other.  A wave reads its row block as 1 KB loads
// straight into the MFMA's B operand (no weight staging, no LDS for the
// weight), 8 KB contiguous per group, and the waves, which take consecutive
// row blocks and advance through k together, read adjacent groups: the device
// reads a sliding window of the packed weight, as the matrix-vector path reads
// whole rows of the plain one.
//
// lmh_packed: 256-thread workgroups; each wave takes WR consecutive row
// blocks of 32 vocab rows (adjacent in the packed layout) against the pass's
// 32 NMT hidden rows.  Those are staged in LDS per range of KR ids, once per
// workgroup, in the same fragment order (1 KB per 16 ids and 32 rows, a
// 16-byte LDS read per lane), double-buffered with one barrier per range;
// the next range's hidden values are requested before the current range's
// MFMAs.  A wave's weight fragments form a ring of R k-steps, requested R
// k-steps ahead in straight-line code.  The k order of the sums is the one of
// lmh_mfma (k-step s, lane half g: ids 16 s + 8 g .. + 7), so the two give the
// same logits.
#define LMP_WG 256
#define LMP_WAVES (LMP_WG / 64)
#define LMP_SG 8                       // k-steps per contiguous group of a row block
#define LMP_MB 64                      // hidden rows per pass
#define LMP_HM 256                     // the H multiple of the packed layout

template <int NMT, int WR, int R, int KR, bool SC>
__global__ __launch_bounds__(LMP_WG) void lmh_packed(LmhParams P, const uint8_t* packed, int b0,
                                                     int nb) {
    constexpr int SPR = KR / 16;                             // k-steps per range
    constexpr int XB = SPR * NMT * 1024;                     // bytes of a staged range
    constexpr int XQ = XB / 16 / LMP_WG;                     // 16-byte pieces per thread
    static_assert(XQ * 16 * LMP_WG == XB && SPR % R == 0 && KR % LMP_HM == 0, "even split");
    __shared__ __align__(16) uint8_t lx[2][XB];
    const int t = (int)threadIdx.x, lane = t & 63, wave = t >> 6, g = lane >> 5, r = lane & 31;
    const int H = P.H, V = P.V, NS = H / 16, NRB = (V + 31) / 32, nkr = H / KR;
    const int wv = (int)blockIdx.x * LMP_WAVES + wave;       // key slot
    const int rb0 = wv * WR;                                 // >= NRB: spare row blocks
    const size_t gstride = (size_t)NRB * LMP_SG * 1024;      // bytes between groups
    const uint8_t* wp[WR];
#pragma unroll
    for (int j = 0; j < WR; ++j)
        wp[j] = packed + (size_t)(rb0 + j < NRB ? rb0 + j : NRB - 1) * LMP_SG * 1024 + lane * 16;
    auto wfrag = [&](int j, int f) {
        return __builtin_nontemporal_load(
            (const lmh_b8*)(wp[j] + (size_t)(f / LMP_SG) * gstride + (f % LMP_SG) * 1024));
    };
    // staging: piece p = t + LMP_WG q is lane p % 64 of fragment (s, mt) =
    // (p / 64 / NMT, p / 64 % NMT) of the range: 16 bytes of hidden row
    // 32 mt + p % 32 (rows past nb read row b0; their sums are not used) at ids
    // 16 s + 8 (p % 64 / 32) of the range
    const uint16_t* gx[XQ];
#pragma unroll
    for (int q = 0; q < XQ; ++q) {
        const int p = t + LMP_WG * q, fr = p >> 6, mt = fr % NMT, s = fr / NMT;
        const int m = 32 * mt + (p & 31);
        gx[q] = P.hidden + (size_t)(b0 + (m < nb ? m : 0)) * H + 16 * s + 8 * ((p & 63) >> 5);
    }
    llima_u32x4 rx[XQ];
    auto fetch_x = [&](int kr) {
#pragma unroll
        for (int q = 0; q < XQ; ++q) rx[q] = *(const llima_u32x4*)(gx[q] + kr * KR);
    };
    auto stage_x = [&](int buf) {
#pragma unroll
        for (int q = 0; q < XQ; ++q) *(llima_u32x4*)(lx[buf] + (t + LMP_WG * q) * 16) = rx[q];
    };
    lmh_b8 rw[R][WR];
#pragma unroll
    for (int i = 0; i < R; ++i)                              // NS >= 16 >= R
#pragma unroll
        for (int j = 0; j < WR; ++j) rw[i][j] = wfrag(j, i);
    lmh_acc acc[WR][NMT];
#pragma unroll
    for (int j = 0; j < WR; ++j)
#pragma unroll
        for (int mt = 0; mt < NMT; ++mt)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[j][mt][i] = 0.0f;
    fetch_x(0);
    stage_x(0);
    __syncthreads();
    for (int kr = 0; kr < nkr; ++kr) {
        fetch_x(kr + 1 < nkr ? kr + 1 : nkr - 1);            // the next range, in flight
        const uint8_t* xb = lx[kr & 1] + lane * 16;
#pragma unroll
        for (int s = 0; s < SPR; ++s) {
            const int f = kr * SPR + s, i = s % R;           // ring slot i holds k-step f
            lmh_b8 bo[WR], a[NMT];
#pragma unroll
            for (int j = 0; j < WR; ++j) bo[j] = rw[i][j];
            const int fn = f + R < NS ? f + R : NS - 1;
#pragma unroll
            for (int j = 0; j < WR; ++j) rw[i][j] = wfrag(j, fn);
#pragma unroll
            for (int mt = 0; mt < NMT; ++mt) a[mt] = *(const lmh_b8*)(xb + (s * NMT + mt) * 1024);
#pragma unroll
            for (int j = 0; j < WR; ++j)
#pragma unroll
                for (int mt = 0; mt < NMT; ++mt)
                    acc[j][mt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[mt], bo[j], acc[j][mt], 0, 0, 0);
        }
        stage_x((kr + 1) & 1);                               // its last readers passed the last barrier
        __syncthreads();
    }
    // key slots past this grid's waves (a pass with more row blocks per wave
    // than another uses fewer of the P.NW slots): no logit, spread over the grid
    {
        const int w0 = (int)gridDim.x * LMP_WAVES, nx = P.NW - w0;
        for (int e = (int)blockIdx.x * LMP_WG + t; e < nx * nb; e += (int)gridDim.x * LMP_WG) {
            P.keys[(size_t)(b0 + e / nx) * P.NW + w0 + e % nx] = 0;
            if constexpr (SC) P.sums[(size_t)(b0 + e / nx) * P.NW + w0 + e % nx] = 0.0f;
        }
    }
    // epilogue: softcap, logits, per hidden row the greatest key of the wave's
    // 32 WR vocab rows
    int ncol[WR];
#pragma unroll
    for (int j = 0; j < WR; ++j) ncol[j] = 32 * (rb0 + j) + r;   // >= V for a spare row block
    int32_t tgv[NMT][16];                                    // scoring: the lane's rows' targets,
#pragma unroll                                               // requested together (-1: no row)
    for (int mt = 0; mt < NMT; ++mt)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int m = mt * 32 + (i & 3) + 8 * (i >> 2) + 4 * g;
            tgv[mt][i] = SC && m < nb ? P.targets[b0 + m] : -1;
        }
#pragma unroll
    for (int mt = 0; mt < NMT; ++mt) {
        float v[16][WR];
#pragma unroll
        for (int i = 0; i < 16; ++i)
#pragma unroll
            for (int j = 0; j < WR; ++j) v[i][j] = acc[j][mt][i];
        lmh_logit_tile<WR>(v, P);
        lmh_tile_out<WR, SC>(P, v, ncol, mt * 32, b0, nb, wv, r, g, tgv[mt]);
    }
}

__global__ __launch_bounds__(LLIMA_WG) void lmh_pack(const uint16_t* weight, uint8_t* packed,
                                                     int V, int H, size_t npieces) {
    const size_t p = (size_t)blockIdx.x * LLIMA_WG + threadIdx.x;
    if (p >= npieces) return;
    const int l = (int)(p & 63);
    const size_t fr = p >> 6, nrb = (size_t)(V + 31) / 32, gs = nrb * LMP_SG;
    const size_t rem = fr % gs, rb = rem / LMP_SG;           // group fr / gs, step rem % 8
    const int s = (int)(fr / gs) * LMP_SG + (int)(rem % LMP_SG);
    const size_t row = 32 * rb + (size_t)(l & 31);
    llima_u32x4 v = {0u, 0u, 0u, 0u};
    if (row < (size_t)V) v = *(const llima_u32x4*)(weight + row * H + 16 * s + 8 * (l >> 5));
    *(llima_u32x4*)(packed + p * 16) = v;
}

static size_t lmh_align256(size_t x) { return (x + 255) & ~(size_t)255; }

// Waves of the rows kernel (a whole number of workgroups): two 512-thread
// workgroups per CU (64 KB of LDS each), fewer for a short vocabulary.
static int lmh_waves(int V) {
    const int nw = 256 * 2 * LMH_WAVES;
    const int need = (V + LMH_WAVES - 1) / LMH_WAVES * LMH_WAVES;
    return need < nw ? need : nw;
}

// Hidden rows per pass: as many as fit the staging buffer, at most 8.
static int lmh_rows_per_pass(int H) {
    int nb = LMH_LDS_FLOATS / H;
    nb = nb >= 8 ? 8 : nb >= 4 ? 4 : nb >= 2 ? 2 : 1;
    return nb;
}

}  // namespace llima

using namespace llima;

// Key slots per hidden row of the MFMA kernel: one per 32 vocab rows, in
// whole 256-row tiles (a grid of 128-row tiles writes 0 to the up to 4 slots
// it leaves).
static int lmh_mfma_waves(int V) {
    return (V + 255) / 256 * 8;
}

static int lmh_plain_slots(int V) {
    return lmh_waves(V) > lmh_mfma_waves(V) ? lmh_waves(V) : lmh_mfma_waves(V);
}

// Workspace of B rows with nw key slots each: the keys, then (scoring) the
// slots' sums and the targets' logits.
static size_t lmh_ws_bytes(int32_t B, int nw, bool sc) {
    const size_t keys = lmh_align256((size_t)B * nw * sizeof(uint64_t));
    return sc ? keys + lmh_align256((size_t)B * nw * sizeof(float)) + lmh_align256((size_t)B * sizeof(float))
              : keys;
}

static void lmh_ws_split(LmhParams& P, void* workspace, int nw) {
    uint8_t* w = (uint8_t*)workspace;
    P.keys = (uint64_t*)w;
    w += lmh_align256((size_t)P.B * nw * sizeof(uint64_t));
    P.sums = (float*)w;
    w += lmh_align256((size_t)P.B * nw * sizeof(float));
    P.tval = (float*)w;
}

// The softcap and logit dtype checks shared by the entry points; clears
// LLIMA_LOGITS_OUT_BF16 from *logit_dtype into *out_bf16.
static int lmh_check_dtype(float softcap, int32_t* logit_dtype, int32_t* out_bf16) {
    if (!(softcap == softcap) || __builtin_isinf(softcap)) return LLIMA_E_INVAL;
    *out_bf16 = (*logit_dtype & LLIMA_LOGITS_OUT_BF16) != 0;
    *logit_dtype &= ~LLIMA_LOGITS_OUT_BF16;
    if (*logit_dtype != LLIMA_F32 && *logit_dtype != LLIMA_BF16) return LLIMA_E_INVAL;
    if (*out_bf16 && *logit_dtype != LLIMA_BF16) return LLIMA_E_INVAL;   // bf16 output of bf16 logits
    return LLIMA_OK;
}

static int lmh_check_plain(const void* hidden, const void* weight, int32_t B, int32_t H,
                           int32_t V) {
    if (B < 0 || H <= 0 || V <= 0 || H % 8 != 0) return LLIMA_E_INVAL;
    if (H > LMH_MAX_H && (H > 65536 || H % LMH_KC != 0)) return LLIMA_E_INVAL;   // MFMA path only
    if (!weight || (B > 0 && !hidden)) return LLIMA_E_INVAL;
    if ((uintptr_t)weight % 16 || (B > 0 && (uintptr_t)hidden % 16)) return LLIMA_E_INVAL;
    return LLIMA_OK;
}

// The passes over the plain weight (MFMA tiles, or the matrix-vector rows
// kernel) and the finish: lmh_finish, or lmh_score_finish with SC.
template <bool SC>
static int lmh_run_plain(LmhParams& P, hipStream_t st) {
    const int B = P.B, H = P.H, V = P.V;
    if ((B > lmh_rows_per_pass(H) || H > LMH_MAX_H) && H % LMH_KC == 0) {   // MFMA tiles
        P.NW = lmh_mfma_waves(V);
        const dim3 g128((uint32_t)((V + 127) / 128));
        for (int b0 = 0; b0 < B; b0 += LMH_MB) {
            const int nb = B - b0 < LMH_MB ? B - b0 : LMH_MB;
            // 128 vocab rows per workgroup; the narrowest tile that holds the
            // pass: 64, 128 or 256 hidden rows
            if (nb <= 64) hipLaunchKernelGGL((lmh_mfma<4, 1, 4, LMH_KC, SC>), g128, dim3(256), 0, st, P, b0, nb);
            else if (nb <= 128) hipLaunchKernelGGL((lmh_mfma<4, 2, 2, LMH_KC, SC>), g128, dim3(512), 0, st, P, b0, nb);
            else hipLaunchKernelGGL((lmh_mfma<4, 4, 2, LMH_KC, SC>), g128, dim3(1024), 0, st, P, b0, nb);
        }
    } else {
        P.NW = lmh_waves(V);
        // rows per pass: what H allows, but no more than the batch fills
        int nbp = lmh_rows_per_pass(H);
        while (nbp > 1 && nbp / 2 >= B) nbp /= 2;
        const dim3 g((uint32_t)((P.NW + LMH_WAVES - 1) / LMH_WAVES)), blk(LMH_WG);
        for (int b0 = 0; b0 < B; b0 += nbp) {
            const int nb = B - b0 < nbp ? B - b0 : nbp;
            switch (nbp) {
                case 8: hipLaunchKernelGGL((lmh_rows<8, SC>), g, blk, 0, st, P, b0, nb); break;
                case 4: hipLaunchKernelGGL((lmh_rows<4, SC>), g, blk, 0, st, P, b0, nb); break;
                case 2: hipLaunchKernelGGL((lmh_rows<2, SC>), g, blk, 0, st, P, b0, nb); break;
                default: hipLaunchKernelGGL((lmh_rows<1, SC>), g, blk, 0, st, P, b0, nb); break;
            }
        }
    }
    if (SC) hipLaunchKernelGGL(lmh_score_finish, dim3((uint32_t)B), dim3(LLIMA_WG), 0, st, P);
    else hipLaunchKernelGGL(lmh_finish, dim3((uint32_t)B), dim3(LLIMA_WG), 0, st, P);
    return hipGetLastError() == hipSuccess ? LLIMA_OK : LLIMA_E_HIP;
}

extern "C" size_t llima_lm_head_argmax_workspace_bytes(int32_t B, int32_t V) {
    if (B <= 0 || V <= 0) return 0;
    return lmh_ws_bytes(B, lmh_plain_slots(V), false);
}

extern "C" int llima_lm_head_argmax(const void* hidden, const void* weight, int32_t B, int32_t H,
                                    int32_t V, float softcap, int32_t logit_dtype,
                                    int32_t* out_ids, float* out_vals, float* out_logits,
                                    void* workspace, size_t workspace_bytes, void* stream) {
    int st0 = lmh_check_plain(hidden, weight, B, H, V);
    if (st0 != LLIMA_OK) return st0;
    if (B > 0 && !out_ids) return LLIMA_E_INVAL;
    int32_t logits_bf16 = 0;
    if ((st0 = lmh_check_dtype(softcap, &logit_dtype, &logits_bf16)) != LLIMA_OK) return st0;
    if (B == 0) return LLIMA_OK;
    if (!workspace || workspace_bytes < llima_lm_head_argmax_workspace_bytes(B, V))
        return LLIMA_E_WORKSPACE;
    LmhParams P = {};
    P.hidden = (const uint16_t*)hidden;
    P.weight = (const uint16_t*)weight;
    P.out_logits = out_logits;
    P.keys = (uint64_t*)workspace;
    P.out_ids = out_ids;
    P.out_vals = out_vals;
    P.B = B; P.H = H; P.V = V;
    P.cap = softcap;
    P.round_bf16 = logit_dtype == LLIMA_BF16;
    P.logits_bf16 = logits_bf16;
    return lmh_run_plain<false>(P, (hipStream_t)stream);
}

// Workspace of the verification entry points: the head's own, then the ids
// of the B (D + 1) target rows.
static size_t lmh_verify_ws(size_t head, int64_t rows) {
    return head == 0 ? 0 : head + lmh_align256((size_t)rows * sizeof(int32_t));
}

static int lmh_verify_check(int32_t B, int32_t D, const int32_t* draft_ids,
                            const int32_t* accepted_len, const int32_t* emitted) {
    if (B < 0 || D < 0 || (int64_t)B * (D + 1) > (int64_t)INT32_MAX) return LLIMA_E_INVAL;
    if (B > 0 && (!accepted_len || !emitted || (D > 0 && !draft_ids))) return LLIMA_E_INVAL;
    return LLIMA_OK;
}

static int lmh_launch_chain(const int32_t* ids, const int32_t* draft_ids, int32_t* accepted_len,
                            int32_t* emitted, int32_t B, int32_t D, hipStream_t st) {
    hipLaunchKernelGGL(lmh_chain, dim3((uint32_t)((B + LLIMA_WG - 1) / LLIMA_WG)), dim3(LLIMA_WG),
                       0, st, ids, draft_ids, accepted_len, emitted, (int)B, (int)D);
    return hipGetLastError() == hipSuccess ? LLIMA_OK : LLIMA_E_HIP;
}

extern "C" size_t llima_lm_head_verify_greedy_workspace_bytes(int32_t B, int32_t D, int32_t V) {
    if (B <= 0 || D < 0 || (int64_t)B * (D + 1) > (int64_t)INT32_MAX) return 0;
    const int32_t rows = B * (D + 1);
    return lmh_verify_ws(llima_lm_head_argmax_workspace_bytes(rows, V), rows);
}

extern "C" int llima_lm_head_verify_greedy(const void* hidden, const void* weight, int32_t B,
                                           int32_t D, int32_t H, int32_t V, float softcap,
                                           int32_t logit_dtype, const int32_t* draft_ids,
                                           int32_t* accepted_len, int32_t* emitted,
                                           void* workspace, size_t workspace_bytes,
                                           void* stream) {
    int st0 = lmh_verify_check(B, D, draft_ids, accepted_len, emitted);
    if (st0 != LLIMA_OK) return st0;
    if (logit_dtype & LLIMA_LOGITS_OUT_BF16) return LLIMA_E_INVAL;       // no logits output
    const int32_t rows = B * (D + 1);
    if ((st0 = lmh_check_plain(hidden, weight, rows, H, V)) != LLIMA_OK) return st0;
    int32_t logits_bf16 = 0;
    if ((st0 = lmh_check_dtype(softcap, &logit_dtype, &logits_bf16)) != LLIMA_OK) return st0;
    if (B == 0) return LLIMA_OK;
    if (!workspace || workspace_bytes < llima_lm_head_verify_greedy_workspace_bytes(B, D, V))
        return LLIMA_E_WORKSPACE;
    const size_t head = llima_lm_head_argmax_workspace_bytes(rows, V);
    int32_t* ids = (int32_t*)((uint8_t*)workspace + head);
    LmhParams P = {};
    P.hidden = (const uint16_t*)hidden;
    P.weight = (const uint16_t*)weight;
    P.keys = (uint64_t*)workspace;
    P.out_ids = ids;
    P.B = rows; P.H = H; P.V = V;
    P.cap = softcap;
    P.round_bf16 = logit_dtype == LLIMA_BF16;
    hipStream_t st = (hipStream_t)stream;
    if ((st0 = lmh_run_plain<false>(P, st)) != LLIMA_OK) return st0;
    return lmh_launch_chain(ids, draft_ids, accepted_len, emitted, B, D, st);
}

// Workspace of the tree entry points: the head's own, then the K rows' ids
// and values.
static size_t lmh_tree_ws(size_t head, int K) {
    return head == 0 ? 0 : head + 2 * lmh_align256((size_t)K * 4);
}

static int lmh_tree_check(int32_t K, const int32_t* retrieve, const int32_t* candidates,
                          int32_t n_paths, int32_t L, const int32_t* out) {
    if (K <= 0 || n_paths <= 0 || L <= 0 || !retrieve || !candidates || !out) return LLIMA_E_INVAL;
    if ((int64_t)n_paths * L > (int64_t)INT32_MAX) return LLIMA_E_INVAL;
    return LLIMA_OK;
}

static int lmh_launch_tree(const LmhParams& P, const int32_t* retrieve, const int32_t* candidates,
                           int32_t n_paths, int32_t L, int32_t* out, hipStream_t st) {
    hipLaunchKernelGGL(lmh_tree, dim3(1), dim3(64), 0, st, (const int32_t*)P.out_ids,
                       (const float*)P.out_vals, P.B, retrieve, candidates, (int)n_paths, (int)L,
                       out);
    return hipGetLastError() == hipSuccess ? LLIMA_OK : LLIMA_E_HIP;
}

extern "C" size_t llima_lm_head_verify_tree_workspace_bytes(int32_t K, int32_t V) {
    if (K <= 0) return 0;
    return lmh_tree_ws(llima_lm_head_argmax_workspace_bytes(K, V), K);
}

extern "C" int llima_lm_head_verify_tree(const void* hidden, const void* weight, int32_t K,
                                         int32_t H, int32_t V, float softcap, int32_t logit_dtype,
                                         const int32_t* retrieve_indices, const int32_t* candidates,
                                         int32_t n_paths, int32_t L, int32_t* out, void* workspace,
                                         size_t workspace_bytes, void* stream) {
    int st0 = lmh_tree_check(K, retrieve_indices, candidates, n_paths, L, out);
    if (st0 != LLIMA_OK) return st0;
    if (logit_dtype & LLIMA_LOGITS_OUT_BF16) return LLIMA_E_INVAL;       // no logits output
    if ((st0 = lmh_check_plain(hidden, weight, K, H, V)) != LLIMA_OK) return st0;
    int32_t logits_bf16 = 0;
    if ((st0 = lmh_check_dtype(softcap, &logit_dtype, &logits_bf16)) != LLIMA_OK) return st0;
    if (!workspace || workspace_bytes < llima_lm_head_verify_tree_workspace_bytes(K, V))
        return LLIMA_E_WORKSPACE;
    uint8_t* rest = (uint8_t*)workspace + llima_lm_head_argmax_workspace_bytes(K, V);
    LmhParams P = {};
    P.hidden = (const uint16_t*)hidden;
    P.weight = (const uint16_t*)weight;
    P.keys = (uint64_t*)workspace;
    P.out_ids = (int32_t*)rest;
    P.out_vals = (float*)(rest + lmh_align256((size_t)K * 4));
    P.B = K; P.H = H; P.V = V;
    P.cap = softcap;
    P.round_bf16 = logit_dtype == LLIMA_BF16;
    hipStream_t st = (hipStream_t)stream;
    if ((st0 = lmh_run_plain<false>(P, st)) != LLIMA_OK) return st0;
    return lmh_launch_tree(P, retrieve_indices, candidates, n_paths, L, out, st);
}

extern "C" size_t llima_lm_head_score_workspace_bytes(int32_t B, int32_t V) {
    if (B <= 0 || V <= 0) return 0;
    return lmh_ws_bytes(B, lmh_plain_slots(V), true);
}

extern "C" int llima_lm_head_score(const void* hidden, const void* weight, int32_t B, int32_t H,
                                   int32_t V, float softcap, int32_t logit_dtype,
                                   const int32_t* targets, double* out_logprob,
                                   int32_t* out_is_greedy, void* workspace,
                                   size_t workspace_bytes, void* stream) {
    int st0 = lmh_check_plain(hidden, weight, B, H, V);
    if (st0 != LLIMA_OK) return st0;
    if (B > 0 && (!targets || !out_logprob || !out_is_greedy)) return LLIMA_E_INVAL;
    if (logit_dtype & LLIMA_LOGITS_OUT_BF16) return LLIMA_E_INVAL;       // no logits output
    int32_t logits_bf16 = 0;
    if ((st0 = lmh_check_dtype(softcap, &logit_dtype, &logits_bf16)) != LLIMA_OK) return st0;
    if (B == 0) return LLIMA_OK;
    if (!workspace || workspace_bytes < llima_lm_head_score_workspace_bytes(B, V))
        return LLIMA_E_WORKSPACE;
    LmhParams P = {};
    P.hidden = (const uint16_t*)hidden;
    P.weight = (const uint16_t*)weight;
    P.B = B; P.H = H; P.V = V;
    P.cap = softcap;
    P.round_bf16 = logit_dtype == LLIMA_BF16;
    P.targets = targets;
    P.out_logprob = out_logprob;
    P.out_greedy = out_is_greedy;
    lmh_ws_split(P, workspace, lmh_plain_slots(V));
    return lmh_run_plain<true>(P, (hipStream_t)stream);
}

// Row blocks per wave, and ring depth, of lmh_packed passes of 32 and of 64
// hidden rows.
#define LMP_WR1 2
#define LMP_R1 8
#define LMP_WR2 2
#define LMP_R2 4
#define LMP_KR 256                     // hidden ids per LDS-staged range

// Workgroups of lmh_packed for WR row blocks per wave; its key slots per
// hidden row are one per wave.
static int lmp_groups(int V, int wr) {
    return ((V + 31) / 32 + LMP_WAVES * wr - 1) / (LMP_WAVES * wr);
}

extern "C" size_t llima_lm_head_packed_bytes(int32_t V, int32_t H) {
    if (V <= 0 || H <= 0 || H % LMP_HM != 0 || H > 65536) return 0;
    return (size_t)((V + 31) / 32) * 32 * (size_t)H * 2;
}

static int lmp_slots(int V) {
    const int g1 = lmp_groups(V, LMP_WR1), g2 = lmp_groups(V, LMP_WR2);
    return (g1 > g2 ? g1 : g2) * LMP_WAVES;
}

extern "C" size_t llima_lm_head_argmax_packed_workspace_bytes(int32_t B, int32_t H, int32_t V) {
    if (B <= 0 || llima_lm_head_packed_bytes(V, H) == 0) return 0;
    return lmh_ws_bytes(B, lmp_slots(V), false);
}

extern "C" size_t llima_lm_head_score_packed_workspace_bytes(int32_t B, int32_t H, int32_t V) {
    if (B <= 0 || llima_lm_head_packed_bytes(V, H) == 0) return 0;
    return lmh_ws_bytes(B, lmp_slots(V), true);
}

extern "C" int llima_lm_head_pack(const void* weight, int32_t V, int32_t H, void* packed,
                                  size_t packed_bytes, void* stream) {
    const size_t need = llima_lm_head_packed_bytes(V, H);
    if (need == 0 || !weight || !packed) return LLIMA_E_INVAL;
    if ((uintptr_t)weight % 16 || (uintptr_t)packed % 16) return LLIMA_E_INVAL;
    if (packed_bytes < need) return LLIMA_E_WORKSPACE;
    const size_t npieces = need / 16;
    hipLaunchKernelGGL(lmh_pack, dim3((uint32_t)((npieces + LLIMA_WG - 1) / LLIMA_WG)),
                       dim3(LLIMA_WG), 0, (hipStream_t)stream, (const uint16_t*)weight,
                       (uint8_t*)packed, V, H, npieces);
    return hipGetLastError() == hipSuccess ? LLIMA_OK : LLIMA_E_HIP;
}

// The passes over a packed weight and the finish (lmh_score_finish with SC).
template <bool SC>
static int lmh_run_packed(LmhParams& P, const uint8_t* packed, hipStream_t st) {
    const int B = P.B, V = P.V;
    const int ng1 = lmp_groups(V, LMP_WR1), ng2 = lmp_groups(V, LMP_WR2);
    P.NW = lmp_slots(V);
    for (int b0 = 0; b0 < B; b0 += LMP_MB) {
        const int nb = B - b0 < LMP_MB ? B - b0 : LMP_MB;
        if (nb <= 32)
            hipLaunchKernelGGL((lmh_packed<1, LMP_WR1, LMP_R1, LMP_KR, SC>), dim3(ng1), dim3(LMP_WG), 0,
                               st, P, packed, b0, nb);
        else
            hipLaunchKernelGGL((lmh_packed<2, LMP_WR2, LMP_R2, LMP_KR, SC>), dim3(ng2), dim3(LMP_WG), 0,
                               st, P, packed, b0, nb);
    }
    if (SC) hipLaunchKernelGGL(lmh_score_finish, dim3((uint32_t)B), dim3(LLIMA_WG), 0, st, P);
    else hipLaunchKernelGGL(lmh_finish, dim3((uint32_t)B), dim3(LLIMA_WG), 0, st, P);
    return hipGetLastError() == hipSuccess ? LLIMA_OK : LLIMA_E_HIP;
}

extern "C" int llima_lm_head_argmax_packed(const void* hidden, const void* packed, int32_t B,
                                           int32_t H, int32_t V, float softcap,
                                           int32_t logit_dtype, int32_t* out_ids, float* out_vals,
                                           float* out_logits, void* workspace,
                                           size_t workspace_bytes, void* stream) {
    if (B < 0 || llima_lm_head_packed_bytes(V, H) == 0) return LLIMA_E_INVAL;
    if (!packed || (B > 0 && (!hidden || !out_ids))) return LLIMA_E_INVAL;
    int32_t logits_bf16 = 0;
    const int st0 = lmh_check_dtype(softcap, &logit_dtype, &logits_bf16);
    if (st0 != LLIMA_OK) return st0;
    if ((uintptr_t)packed % 16 || (B > 0 && (uintptr_t)hidden % 16)) return LLIMA_E_INVAL;
    if (B == 0) return LLIMA_OK;
    if (!workspace || workspace_bytes < llima_lm_head_argmax_packed_workspace_bytes(B, H, V))
        return LLIMA_E_WORKSPACE;
    LmhParams P = {};
    P.hidden = (const uint16_t*)hidden;
    P.out_logits = out_logits;
    P.keys = (uint64_t*)workspace;
    P.out_ids = out_ids;
    P.out_vals = out_vals;
    P.B = B; P.H = H; P.V = V;
    P.cap = softcap;
    P.round_bf16 = logit_dtype == LLIMA_BF16;
    P.logits_bf16 = logits_bf16;
    return lmh_run_packed<false>(P, (const uint8_t*)packed, (hipStream_t)stream);
}

extern "C" int llima_lm_head_score_packed(const void* hidden, const void* packed, int32_t B,
                                          int32_t H, int32_t V, float softcap,
                                          int32_t logit_dtype, const int32_t* targets,
                                          double* out_logprob, int32_t* out_is_greedy,
                                          void* workspace, size_t workspace_bytes, void* stream) {
    if (B < 0 || llima_lm_head_packed_bytes(V, H) == 0) return LLIMA_E_INVAL;
    if (!packed || (B > 0 && (!hidden || !targets || !out_logprob || !out_is_greedy)))
        return LLIMA_E_INVAL;
    if (logit_dtype & LLIMA_LOGITS_OUT_BF16) return LLIMA_E_INVAL;       // no logits output
    int32_t logits_bf16 = 0;
    const int st0 = lmh_check_dtype(softcap, &logit_dtype, &logits_bf16);
    if (st0 != LLIMA_OK) return st0;
    if ((uintptr_t)packed % 16 || (B > 0 && (uintptr_t)hidden % 16)) return LLIMA_E_INVAL;
    if (B == 0) return LLIMA_OK;
    if (!workspace || workspace_bytes < llima_lm_head_score_packed_workspace_bytes(B, H, V))
        return LLIMA_E_WORKSPACE;
    LmhParams P = {};
    P.hidden = (const uint16_t*)hidden;
    P.B = B; P.H = H; P.V = V;
    P.cap = softcap;
    P.round_bf16 = logit_dtype == LLIMA_BF16;
    P.targets = targets;
    P.out_logprob = out_logprob;
    P.out_greedy = out_is_greedy;
    lmh_ws_split(P, workspace, lmp_slots(V));
    return lmh_run_packed<true>(P, (const uint8_t*)packed, (hipStream_t)stream);
}

extern "C" size_t llima_lm_head_verify_greedy_packed_workspace_bytes(int32_t B, int32_t D,
                                                                    int32_t H, int32_t V) {
    if (B <= 0 || D < 0 || (int64_t)B * (D + 1) > (int64_t)INT32_MAX) return 0;
    const int32_t rows = B * (D + 1);
    return lmh_verify_ws(llima_lm_head_argmax_packed_workspace_bytes(rows, H, V), rows);
}

extern "C" int llima_lm_head_verify_greedy_packed(const void* hidden, const void* packed,
                                                  int32_t B, int32_t D, int32_t H, int32_t V,
                                                  float softcap, int32_t logit_dtype,
                                                  const int32_t* draft_ids, int32_t* accepted_len,
                                                  int32_t* emitted, void* workspace,
                                                  size_t workspace_bytes, void* stream) {
    int st0 = lmh_verify_check(B, D, draft_ids, accepted_len, emitted);
    if (st0 != LLIMA_OK) return st0;
    if (llima_lm_head_packed_bytes(V, H) == 0 || !packed || (B > 0 && !hidden)) return LLIMA_E_INVAL;
    if (logit_dtype & LLIMA_LOGITS_OUT_BF16) return LLIMA_E_INVAL;       // no logits output
    int32_t logits_bf16 = 0;
    if ((st0 = lmh_check_dtype(softcap, &logit_dtype, &logits_bf16)) != LLIMA_OK) return st0;
    if ((uintptr_t)packed % 16 || (B > 0 && (uintptr_t)hidden % 16)) return LLIMA_E_INVAL;
    if (B == 0) return LLIMA_OK;
    if (!workspace || workspace_bytes < llima_lm_head_verify_greedy_packed_workspace_bytes(B, D, H, V))
        return LLIMA_E_WORKSPACE;
    const int32_t rows = B * (D + 1);
    const size_t head = llima_lm_head_argmax_packed_workspace_bytes(rows, H, V);
    int32_t* ids = (int32_t*)((uint8_t*)workspace + head);
    LmhParams P = {};
    P.hidden = (const uint16_t*)hidden;
    P.keys = (uint64_t*)workspace;
    P.out_ids = ids;
    P.B = rows; P.H = H; P.V = V;
    P.cap = softcap;
    P.round_bf16 = logit_dtype == LLIMA_BF16;
    hipStream_t st = (hipStream_t)stream;
    if ((st0 = lmh_run_packed<false>(P, (const uint8_t*)packed, st)) != LLIMA_OK) return st0;
    return lmh_launch_chain(ids, draft_ids, accepted_len, emitted, B, D, st);
}

extern "C" size_t llima_lm_head_verify_tree_packed_workspace_bytes(int32_t K, int32_t H, int32_t V) {
    if (K <= 0) return 0;
    return lmh_tree_ws(llima_lm_head_argmax_packed_workspace_bytes(K, H, V), K);
}

extern "C" int llima_lm_head_verify_tree_packed(const void* hidden, const void* packed, int32_t K,
                                                int32_t H, int32_t V, float softcap,
                                                int32_t logit_dtype,
                                                const int32_t* retrieve_indices,
                                                const int32_t* candidates, int32_t n_paths,
                                                int32_t L, int32_t* out, void* workspace,
                                                size_t workspace_bytes, void* stream) {
    int st0 = lmh_tree_check(K, retrieve_indices, candidates, n_paths, L, out);
    if (st0 != LLIMA_OK) return st0;
    if (llima_lm_head_packed_bytes(V, H) == 0 || !packed || !hidden) return LLIMA_E_INVAL;
    if (logit_dtype & LLIMA_LOGITS_OUT_BF16) return LLIMA_E_INVAL;       // no logits output
    int32_t logits_bf16 = 0;
    if ((st0 = lmh_check_dtype(softcap, &logit_dtype, &logits_bf16)) != LLIMA_OK) return st0;
    if ((uintptr_t)packed % 16 || (uintptr_t)hidden % 16) return LLIMA_E_INVAL;
    if (!workspace || workspace_bytes < llima_lm_head_verify_tree_packed_workspace_bytes(K, H, V))
        return LLIMA_E_WORKSPACE;
    uint8_t* rest = (uint8_t*)workspace + llima_lm_head_argmax_packed_workspace_bytes(K, H, V);
    LmhParams P = {};
    P.hidden = (const uint16_t*)hidden;
    P.keys = (uint64_t*)workspace;
    P.out_ids = (int32_t*)rest;
    P.out_vals = (float*)(rest + lmh_align256((size_t)K * 4));
    P.B = K; P.H = H; P.V = V;
    P.cap = softcap;
    P.round_bf16 = logit_dtype == LLIMA_BF16;
    hipStream_t st = (hipStream_t)stream;
    if ((st0 = lmh_run_packed<false>(P, (const uint8_t*)packed, st)) != LLIMA_OK) return st0;
    return lmh_launch_tree(P, retrieve_indices, candidates, n_paths, L, out, st);
}
