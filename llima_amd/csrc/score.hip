// score.hip -- log-likelihood scoring and the centroid-masked argmax (gfx950).
//
// Restates on device memory:
//   score_logits                    sima_lmm/devkit/cpp/language_model.cpp:29-62
//   select_candidate_tokens         sima_lmm/devkit/cpp/gemma4_mtp_helpers.cpp:113-167
//   _argmax_gemma4_mtp_masked_row   sima_lmm/devkit/cpp/language_model_gemma4_mtp.cpp:31-97
//
// score_logits: two launches.  score_sweep cuts [rows][V] into rows x S
// workgroups; each streams its chunk once with 16-byte loads and produces the
// chunk's first-maximum key (value key << 32 | ~index, as the argmax sweep), a
// NaN flag and s_c = sum of exp(x - m_c) over its values, m_c the chunk
// maximum: the values stay in registers between the maximum and the sum, so
// the row crosses HBM once.  score_finish (one wavefront per row) combines
// S = sum_c exp(m_c - M) s_c in double and writes x_t - (M + log S).
// Precision: the reference sums exp in double; here each term is an fp32
// exp2 of (x - m_c) log2(e) (relative error about 1e-7 times |x - m_c|, so the
// terms that dominate S are nearly exact), the per-thread sums are fp32 over
// at most 32 terms and everything after that is double.  The log-probability
// agrees to about 1e-6 absolute; the argmax, the greedy flag and every NaN /
// infinity outcome are exact.
//
// Masked argmax: G workgroups per row, then one wavefront per row combines
// their maxima.  The top_k centroids by (value desc,
// index asc) are found as a set by an 8-bit radix select on the value keys in
// LDS (plus an index-order scan of the ties at the boundary when only some of
// them are in); their tokens (the token_ordering runs of the selected
// centroids) are gathered and reduced to the greatest value, lowest token id
// on equal values.  The reference visits
// the candidates in rank order; the result does not depend on that order.
#include "common.hpp"
#include "../../include/llima_sampler.h"

namespace llima {

// ================================================================ score_logits
struct ScoreParams {
    const void* logits;
    int64_t row_stride;
    const int32_t* targets;        // [B]
    double* out_logprob;           // [B]
    int32_t* out_greedy;           // [B]: 1 / 0, LLIMA_E_RANGE for a target outside [0, V)
    uint64_t* keys;                // [B][S] chunk first-maximum key (0: no value above -inf)
    double* sums;                  // [B][S] sum of exp(x - m_c)
    uint32_t* flags;               // [B][S] 1: the chunk holds a NaN
    int32_t B, V, S, vec_ok;
};

template <typename TL>
__device__ __forceinline__ float sc_ld1(const TL* p, int64_t i);
template <>
__device__ __forceinline__ float sc_ld1<float>(const float* p, int64_t i) { return p[i]; }
template <>
__device__ __forceinline__ float sc_ld1<uint16_t>(const uint16_t* p, int64_t i) {
    return bf16_bits_to_f32(p[i]);
}

template <typename TL, int E, bool VEC>
__global__ __launch_bounds__(LLIMA_WG) void score_sweep(ScoreParams P) {
    constexpr int EPL = 16 / sizeof(TL);
    constexpr int NL = E / EPL;
    constexpr int CHUNK = LLIMA_WG * E;
    constexpr float LOG2E = 1.44269504088896340736f;
    __shared__ double wsum[LLIMA_WAVES];
    __shared__ uint32_t wmax[LLIMA_WAVES], wfi[LLIMA_WAVES], wnan[LLIMA_WAVES];

    uint32_t row, chunk;
    map_row_chunk(blockIdx.x, (uint32_t)P.B, (uint32_t)P.S, &row, &chunk);
    if (row >= (uint32_t)P.B) return;
    const TL* rowp = (const TL*)P.logits + (size_t)row * P.row_stride;
    const int V = P.V;
    const int c0 = (int)chunk * CHUNK;
    const int c1 = c0 + CHUNK < V ? c0 + CHUNK : V;

    llima_u32x4 q[NL];
#pragma unroll
    for (int j = 0; j < NL; ++j) {
        const int i0 = c0 + j * (LLIMA_WG * EPL) + (int)threadIdx.x * EPL;
        if constexpr (VEC) {
            const int ia = i0 < V ? i0 : V - EPL;
            q[j] = __builtin_nontemporal_load((const llima_u32x4*)(rowp + ia));
        } else {
            uint32_t w[4] = {0, 0, 0, 0};
#pragma unroll
            for (int e = 0; e < EPL; ++e) {
                const int ia = i0 + e < V ? i0 + e : V - 1;
                const float f = sc_ld1<TL>(rowp, ia);
                if constexpr (sizeof(TL) == 4) w[e] = __float_as_uint(f);
                else w[e >> 1] |= (__float_as_uint(f) >> 16) << ((e & 1) * 16);
            }
            q[j] = llima_u32x4{w[0], w[1], w[2], w[3]};
        }
    }
    // values past the row are -inf (no maximum, no NaN, weight 0)
    float x[E];
#pragma unroll
    for (int j = 0; j < NL; ++j) {
        const int i0 = c0 + j * (LLIMA_WG * EPL) + (int)threadIdx.x * EPL;
        const uint32_t w4[4] = {q[j].x, q[j].y, q[j].z, q[j].w};
#pragma unroll
        for (int e = 0; e < EPL; ++e) {
            float f;
            if constexpr (sizeof(TL) == 4) f = __uint_as_float(w4[e]);
            else f = __uint_as_float((e & 1) ? (w4[e >> 1] & 0xFFFF0000u) : (w4[e >> 1] << 16));
            x[j * EPL + e] = i0 + e < c1 ? f : -__builtin_inff();
        }
    }
    // per thread: its maximum m_t (fmaxf ignores NaN) and s_t = sum of
    // exp(x - m_t) (NaN when a value is NaN or m_t = +inf)
    float mt = -__builtin_inff();
#pragma unroll
    for (int e = 0; e < E; ++e) mt = __builtin_fmaxf(mt, x[e]);
    float s = 0.0f;
    uint32_t nan = 0;
    if (mt > -__builtin_inff()) {
#pragma unroll
        for (int e = 0; e < E; ++e) s += __builtin_amdgcn_exp2f((x[e] - mt) * LOG2E);
    } else {
#pragma unroll
        for (int e = 0; e < E; ++e) nan |= x[e] != x[e] ? 1u : 0u;    // NaN beside -inf only
    }
    // the chunk maximum m_c (one barrier: every thread reads the four waves')
    const uint32_t km = wave_max_u32(mt > -__builtin_inff() ? f32_key(mt) : 0u);
    if (lane_id() == 0) wmax[wave_id()] = km;
    __syncthreads();
    uint32_t kc = 0;
#pragma unroll
    for (int w = 0; w < LLIMA_WAVES; ++w) kc = wmax[w] > kc ? wmax[w] : kc;
    const float mc = kc ? key_f32(kc) : -__builtin_inff();
    // its first index: only threads whose maximum is m_c search their values
    uint32_t fi = 0xFFFFFFFFu;
    if (kc && mt == mc) {
#pragma unroll
        for (int j = NL - 1; j >= 0; --j) {
            const int i0 = c0 + j * (LLIMA_WG * EPL) + (int)threadIdx.x * EPL;
#pragma unroll
            for (int e = EPL - 1; e >= 0; --e) fi = x[j * EPL + e] == mc ? (uint32_t)(i0 + e) : fi;
        }
    }
    // s_c = sum_t s_t exp(m_t - m_c); a NaN s_t (a NaN value, or an infinite
    // maximum) makes s_c NaN, which the finish reads as "NaN result"
    const float f = mt > -__builtin_inff() ? s * __builtin_amdgcn_exp2f((mt - mc) * LOG2E) : 0.0f;
    const double ws = wave_sum_f64((double)f);
    fi = wave_min_u32(fi);
    nan = wave_max_u32(nan);
    if (lane_id() == 0) { wsum[wave_id()] = ws; wfi[wave_id()] = fi; wnan[wave_id()] = nan; }
    __syncthreads();
    if (threadIdx.x == 0) {
        double tot = 0.0;
        uint32_t n = 0, first = 0xFFFFFFFFu;
#pragma unroll
        for (int w = 0; w < LLIMA_WAVES; ++w) {
            tot += wsum[w];
            n |= wnan[w];
            first = wfi[w] < first ? wfi[w] : first;
        }
        n |= tot != tot ? 1u : 0u;
        const size_t o = (size_t)row * P.S + chunk;
        P.keys[o] = kc ? (((uint64_t)kc << 32) | (uint32_t)~first) : 0ull;
        P.sums[o] = tot;
        P.flags[o] = n;
    }
}

// One wavefront per row: M, S and the log-probability at the target.
template <typename TL>
__global__ __launch_bounds__(LLIMA_WG) void score_finish(ScoreParams P) {
    const int row = finish_row(blockIdx.x, wave_id(), (uint32_t)P.B);
    if (row < 0) return;
    const uint32_t lane = lane_id();
    const uint64_t* k = P.keys + (size_t)row * P.S;
    const double* sm = P.sums + (size_t)row * P.S;
    const uint32_t* fl = P.flags + (size_t)row * P.S;
    uint64_t best = 0;
    uint32_t nan = 0;
    for (int i = (int)lane; i < P.S; i += 64) {
        best = k[i] > best ? k[i] : best;
        nan |= fl[i];
    }
    best = wave_max_u64(best);
    nan = wave_max_u32(nan);
    const float M = best ? key_f32((uint32_t)(best >> 32)) : -__builtin_inff();
    const bool finite = M > -__builtin_inff() && M < __builtin_inff();
    double S = 0.0;
    if (finite) {
        for (int i = (int)lane; i < P.S; i += 64) {
            const uint64_t ki = k[i];
            const float mc = ki ? key_f32((uint32_t)(ki >> 32)) : -__builtin_inff();
            if (mc > -__builtin_inff()) S += exp((double)mc - (double)M) * sm[i];
        }
        S = wave_sum_f64(S);
    }
    if (lane != 0) return;
    const int32_t tg = P.targets[row];
    if (tg < 0 || tg >= P.V) {
        P.out_logprob[row] = __builtin_nan("");
        P.out_greedy[row] = LLIMA_E_RANGE;
        return;
    }
    const TL* rowp = (const TL*)P.logits + (size_t)row * P.row_stride;
    const double xt = (double)sc_ld1<TL>(rowp, tg);
    // the reference's double sum is NaN with a NaN value, and with an infinite
    // maximum (exp(inf - inf) / exp(-inf + inf))
    const double lp = (nan || !finite) ? __builtin_nan("") : xt - ((double)M + log(S));
    const uint32_t am = best ? ~(uint32_t)best : 0u;
    P.out_logprob[row] = lp;
    P.out_greedy[row] = am == (uint32_t)tg ? 1 : 0;
}

static size_t sc_align256(size_t x) { return (x + 255) & ~(size_t)255; }

struct STile { int E, S; };
static STile score_tile(int B, int V, int dtype) {
    int E = dtype == LLIMA_F32 ? 16 : 32;
    auto S_of = [&](int e) { return (V + LLIMA_WG * e - 1) / (LLIMA_WG * e); };
    while (E > 8 && (int64_t)B * S_of(E) < 1024) E /= 2;
    return {E, S_of(E)};
}

template <typename TL, int E>
static hipError_t launch_score(const ScoreParams& P, hipStream_t st) {
    const dim3 g((uint32_t)P.B * (uint32_t)P.S), b(LLIMA_WG);
    if (P.vec_ok) hipLaunchKernelGGL((score_sweep<TL, E, true>), g, b, 0, st, P);
    else hipLaunchKernelGGL((score_sweep<TL, E, false>), g, b, 0, st, P);
    hipLaunchKernelGGL((score_finish<TL>), dim3(finish_row_blocks((uint32_t)P.B)),
                       dim3(LLIMA_WG), 0, st, P);
    return hipGetLastError();
}

// ============================================================ masked argmax
#define MTP_MAX_C 8192             // centroids per row held in LDS
#define MTP_GB 16                  // candidates per thread with loads in flight together
#define MTP_MAX_G 16               // workgroups sharing one row's candidates
#define MTP_SHARE 256              // candidates per workgroup (at least)

struct MtpParams {
    const uint16_t* centroids;     // bf16 [B][c_stride]
    int64_t c_stride;
    const uint32_t* ordering;      // [V]
    const void* logits;            // [B][row_stride] or null (selection only)
    int64_t row_stride;
    int32_t* out_ids;              // [B] or null
    int32_t* out_status;           // [B] or null
    uint32_t* out_cand;            // [B][k * per] or null
    uint64_t* pkeys;               // [B][G] best (value key, ~token) of each share
    uint32_t* pbad;                // [B][G] 1: an ordering entry >= V in the share
    int32_t B, V, C, k, per, G;
};

struct MtpShared {
    uint32_t ck[MTP_MAX_C];        // centroid value keys (16 bits), NaN -> 0
    uint32_t sel[MTP_MAX_C];       // selected centroids, index order
    uint32_t hist[256];
    uint32_t digit, need, ties, bad;
    BlockScratch bs;
};

// Workgroup (row, part): the centroid selection of the row (every part of the
// row repeats it: a few microseconds of latency, no traffic to speak of), then
// share `part` of the row's candidates: the gathers of one row are spread over
// G workgroups, since one CU pulls one scattered cache line per candidate.
template <typename TL>
__global__ __launch_bounds__(LLIMA_WG) void mtp_select_gather(MtpParams P) {
    __shared__ MtpShared sh;
    const int row = (int)blockIdx.x / P.G, part = (int)blockIdx.x % P.G;
    const uint32_t t = threadIdx.x, lane = lane_id(), wave = wave_id();
    const int C = P.C;
    const uint16_t* crow = P.centroids + (size_t)row * P.c_stride;
    for (int i0 = 0; i0 < C; i0 += 8 * LLIMA_WG) {     // 8 loads in flight per thread
        uint32_t h[8];
#pragma unroll
        for (int m = 0; m < 8; ++m) {
            const int i = i0 + m * LLIMA_WG + (int)t;
            h[m] = crow[i < C ? i : 0];
        }
#pragma unroll
        for (int m = 0; m < 8; ++m) {
            const int i = i0 + m * LLIMA_WG + (int)t;
            const float v = bf16_bits_to_f32(h[m]);
            if (i < C) sh.ck[i] = v == v ? f32_key(v) >> 16 : 0u;   // bf16: the low half is constant
        }
    }
    if (t == 0) sh.bad = 0;
    // ---- the k-th largest value key tau, 8 bits per round, and how many of
    //      the centroids with key tau belong to the top k (need)
    uint32_t prefix = 0, pmask = 0, need = (uint32_t)P.k;
    for (int shift = 8; shift >= 0; shift -= 8) {
        sh.hist[t] = 0;
        __syncthreads();
        for (int i = (int)t; i < C; i += LLIMA_WG) {
            const uint32_t kk = sh.ck[i];
            if ((kk & pmask) == prefix) atomicAdd(&sh.hist[(kk >> shift) & 255u], 1u);
        }
        __syncthreads();
        if (wave == 0) {
            // lane l: bins 255 - 4l .. 252 - 4l (descending)
            uint32_t cn[4], s4 = 0;
#pragma unroll
            for (int i = 0; i < 4; ++i) { cn[i] = sh.hist[255u - 4u * lane - (uint32_t)i]; s4 += cn[i]; }
            const uint32_t inc = wave_incl_scan_u32(s4);
            uint32_t run = inc - s4;                   // keys in higher bins
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                if (run < need && need <= run + cn[i]) {
                    sh.digit = 255u - 4u * lane - (uint32_t)i;
                    sh.need = need - run;
                    sh.ties = cn[i];
                }
                run += cn[i];
            }
        }
        __syncthreads();
        prefix |= sh.digit << shift;
        pmask |= 0xFFu << shift;
        need = sh.need;
    }
    const uint32_t tau = prefix;
    // ---- the selected centroids (keys above tau, then the first `need` with
    //      key tau by index) into sh.sel in index order: every workgroup of
    //      the row builds the same list, and each takes its share of it
    const int per_t = (C + LLIMA_WG - 1) / LLIMA_WG;           // thread t: a contiguous index range
    const int i0 = (int)t * per_t, i1 = i0 + per_t < C ? i0 + per_t : C;
    uint32_t neq = 0, nsl = 0;
    for (int i = i0; i < i1; ++i) {
        const uint32_t kk = sh.ck[i];
        neq += kk == tau ? 1u : 0u;
        nsl += kk > tau ? 1u : 0u;
    }
    const bool all_ties = need == sh.ties;                      // the usual case
    uint32_t teq = 0, tsel;
    uint32_t eqb = all_ties ? 0u : block_excl_scan_u32(neq, &teq, sh.bs);   // ties before this range
    uint32_t ns2 = nsl;
    if (!all_ties) {
        uint32_t e2 = eqb;
        for (int i = i0; i < i1; ++i) {
            const bool tie = sh.ck[i] == tau;
            ns2 += tie && e2 < need ? 1u : 0u;
            e2 += tie ? 1u : 0u;
        }
    } else {
        ns2 += neq;
    }
    uint32_t o = block_excl_scan_u32(ns2, &tsel, sh.bs);          // tsel == k
    for (int i = i0; i < i1; ++i) {
        const uint32_t kk = sh.ck[i];
        if (kk > tau || (kk == tau && (all_ties || eqb < need))) sh.sel[o++] = (uint32_t)i;
        eqb += kk == tau ? 1u : 0u;
    }
    __syncthreads();
    // ---- candidates: the ordering runs of the selected centroids; their rank
    //      (for the candidate list) is the number of selected centroids ahead
    //      by (value desc, index asc)
    const int per = P.per, k = P.k;
    const int ncand = k * per;
    const TL* rowp = P.logits ? (const TL*)P.logits + (size_t)row * P.row_stride : nullptr;
    uint32_t* cand = P.out_cand ? P.out_cand + (size_t)row * ncand : nullptr;
    const float inv_per = 1.0f / (float)per;
    const int share = (ncand + P.G - 1) / P.G;
    const int jlo = part * share, jhi = jlo + share < ncand ? jlo + share : ncand;
    uint64_t best = 0;
    uint32_t bad = 0;
    // candidate j = jlo + t + 256 m of a batch: centroid rank r = j / per (fp32
    // quotient, exact after one correction since j < 2^24), position off
    for (int j0 = jlo; j0 < jhi; j0 += MTP_GB * LLIMA_WG) {
        uint32_t tok[MTP_GB], cr[MTP_GB], co[MTP_GB];
        bool ok[MTP_GB];
#pragma unroll
        for (int m = 0; m < MTP_GB; ++m) {             // every ordering load first
            const int j = j0 + m * LLIMA_WG + (int)t;
            ok[m] = j < jhi;
            int r = (int)((float)j * inv_per);
            int off = j - r * per;
            r = off < 0 ? r - 1 : (off >= per ? r + 1 : r);
            off = j - r * per;
            const uint32_t c = sh.sel[ok[m] ? r : 0];
            cr[m] = (uint32_t)r; co[m] = (uint32_t)off;
            tok[m] = P.ordering[ok[m] ? (size_t)c * per + off : 0];
        }
        float v[MTP_GB];
        if (rowp) {
#pragma unroll
            for (int m = 0; m < MTP_GB; ++m)              // then every logit load
                v[m] = sc_ld1<TL>(rowp, ok[m] && tok[m] < (uint32_t)P.V ? tok[m] : 0u);
        }
#pragma unroll
        for (int m = 0; m < MTP_GB; ++m) {
            if (!ok[m]) continue;
            if (tok[m] >= (uint32_t)P.V) { bad = 1; continue; }
            if (cand) {
                const uint32_t c = sh.sel[cr[m]], kc = sh.ck[c];
                uint32_t rank = 0;
                for (int q = 0; q < k; ++q) {
                    const uint32_t cq = sh.sel[q], kq = sh.ck[cq];
                    rank += (kq > kc || (kq == kc && cq < c)) ? 1u : 0u;
                }
                cand[(size_t)rank * per + co[m]] = tok[m];
            }
            if (rowp) {
                const uint64_t kv = v[m] == v[m] ? (((uint64_t)f32_key(v[m]) << 32) | (uint32_t)~tok[m])
                                                 : 0ull;
                best = kv > best ? kv : best;
            }
        }
    }
    if (bad) sh.bad = 1;                              // benign race: every writer stores 1
    best = block_max_u64(best, sh.bs);                // barrier: sh.bad final
    if (t != 0) return;
    P.pkeys[(size_t)row * P.G + part] = best;
    P.pbad[(size_t)row * P.G + part] = sh.bad;
}

// One wavefront per row: the shares' maxima and error flags combined.
__global__ __launch_bounds__(LLIMA_WG) void mtp_combine(MtpParams P) {
    const int row = (int)blockIdx.x * LLIMA_WAVES + (int)wave_id();
    if (row >= P.B) return;
    const uint32_t lane = lane_id();
    const bool in = (int)lane < P.G;
    const uint64_t kb = wave_max_u64(in ? P.pkeys[(size_t)row * P.G + lane] : 0ull);
    const uint32_t bad = wave_max_u32(in ? P.pbad[(size_t)row * P.G + lane] : 0u);
    if (lane != 0) return;
    int32_t id = -1, st = LLIMA_OK;
    if (bad) st = LLIMA_E_RANGE;                      // out-of-range token id in the ordering
    else if (P.logits && kb == 0) st = LLIMA_E_INVAL; // no candidate value (all NaN)
    else if (P.logits) id = (int32_t)~(uint32_t)kb;
    if (P.out_ids) P.out_ids[row] = id;
    if (P.out_status) P.out_status[row] = st;
}

}  // namespace llima

using namespace llima;

extern "C" size_t llima_score_logits_workspace_bytes(int32_t B, int32_t V, int32_t dtype) {
    (void)dtype;
    if (B <= 0 || V <= 0) return 0;
    const size_t n = (size_t)B * ((V + 2047) / 2048);        // chunks of at least 2048 values
    return sc_align256(n * sizeof(uint64_t)) + sc_align256(n * sizeof(double)) +
           sc_align256(n * sizeof(uint32_t));
}

extern "C" int llima_score_logits(const void* logits, int32_t dtype, int32_t B, int32_t V,
                                  int64_t row_stride, const int32_t* targets, double* out_logprob,
                                  int32_t* out_is_greedy, void* workspace, size_t workspace_bytes,
                                  void* stream) {
    if (B > 0 && (!logits || !targets || !out_logprob || !out_is_greedy)) return LLIMA_E_INVAL;
    if (dtype != LLIMA_F32 && dtype != LLIMA_BF16) return LLIMA_E_INVAL;
    if (B < 0 || V <= 0 || row_stride < V) return LLIMA_E_INVAL;
    if (B == 0) return LLIMA_OK;
    if (!workspace || workspace_bytes < llima_score_logits_workspace_bytes(B, V, dtype))
        return LLIMA_E_WORKSPACE;
    const STile tl = score_tile(B, V, dtype);
    ScoreParams P = {};
    P.logits = logits;
    P.row_stride = row_stride;
    P.targets = targets;
    P.out_logprob = out_logprob;
    P.out_greedy = out_is_greedy;
    P.B = B; P.V = V; P.S = tl.S;
    const size_t n = (size_t)B * tl.S;
    P.keys = (uint64_t*)workspace;
    P.sums = (double*)((char*)workspace + sc_align256(n * sizeof(uint64_t)));
    P.flags = (uint32_t*)((char*)P.sums + sc_align256(n * sizeof(double)));
    const size_t esz = dtype == LLIMA_F32 ? 4 : 2;
    P.vec_ok = ((uintptr_t)logits % 16 == 0) && ((row_stride * (int64_t)esz) % 16 == 0) &&
               (V % (int32_t)(16 / esz) == 0);
    const hipStream_t st = (hipStream_t)stream;
    hipError_t e;
    if (dtype == LLIMA_F32) {
        switch (tl.E) {
            case 8: e = launch_score<float, 8>(P, st); break;
            default: e = launch_score<float, 16>(P, st); break;
        }
    } else {
        switch (tl.E) {
            case 8: e = launch_score<uint16_t, 8>(P, st); break;
            case 16: e = launch_score<uint16_t, 16>(P, st); break;
            default: e = launch_score<uint16_t, 32>(P, st); break;
        }
    }
    return e == hipSuccess ? LLIMA_OK : LLIMA_E_HIP;
}

extern "C" size_t llima_mtp_masked_argmax_workspace_bytes(int32_t B) {
    if (B <= 0) return 0;
    return sc_align256((size_t)B * MTP_MAX_G * sizeof(uint64_t)) +
           sc_align256((size_t)B * MTP_MAX_G * sizeof(uint32_t));
}

extern "C" int llima_mtp_masked_argmax(const uint16_t* centroid_logits, int64_t centroid_stride,
                                       int32_t C, const uint32_t* token_ordering, int32_t top_k,
                                       const void* logits, int32_t dtype, int32_t B, int32_t V,
                                       int64_t row_stride, int32_t* out_ids, int32_t* out_status,
                                       uint32_t* out_candidates, void* workspace,
                                       size_t workspace_bytes, void* stream) {
    if (!token_ordering || (B > 0 && !centroid_logits)) return LLIMA_E_INVAL;
    if (B < 0 || V <= 0 || C <= 0 || C > MTP_MAX_C || centroid_stride < C) return LLIMA_E_INVAL;
    if (V % C != 0) return LLIMA_E_INVAL;                 // gemma4_mtp_helpers.cpp:118-125
    if (V >= (1 << 24)) return LLIMA_E_INVAL;             // candidate indices stay exact in fp32
    if (top_k <= 0 || top_k > C) return LLIMA_E_INVAL;    // gemma4_mtp_helpers.cpp:126-128
    if (logits) {
        if (dtype != LLIMA_F32 && dtype != LLIMA_BF16) return LLIMA_E_INVAL;
        if (row_stride < V || (B > 0 && !out_ids)) return LLIMA_E_INVAL;
    } else if (!out_candidates && B > 0) {
        return LLIMA_E_INVAL;                             // nothing to compute
    }
    if (B == 0) return LLIMA_OK;
    if (!workspace || workspace_bytes < llima_mtp_masked_argmax_workspace_bytes(B))
        return LLIMA_E_WORKSPACE;
    MtpParams P = {};
    P.centroids = centroid_logits;
    P.c_stride = centroid_stride;
    P.ordering = token_ordering;
    P.logits = logits;
    P.row_stride = row_stride;
    P.out_ids = out_ids;
    P.out_status = out_status;
    P.out_cand = out_candidates;
    P.B = B; P.V = V; P.C = C; P.k = top_k; P.per = V / C;
    const int64_t ncand = (int64_t)top_k * (V / C);
    const int64_t g = (ncand + MTP_SHARE - 1) / MTP_SHARE;
    P.G = (int32_t)(g < 1 ? 1 : (g > MTP_MAX_G ? MTP_MAX_G : g));
    P.pkeys = (uint64_t*)workspace;
    P.pbad = (uint32_t*)((char*)workspace + sc_align256((size_t)B * MTP_MAX_G * sizeof(uint64_t)));
    const hipStream_t st = (hipStream_t)stream;
    const dim3 grid((uint32_t)B * (uint32_t)P.G), blk(LLIMA_WG);
    if (logits && dtype == LLIMA_F32) hipLaunchKernelGGL(mtp_select_gather<float>, grid, blk, 0, st, P);
    else hipLaunchKernelGGL(mtp_select_gather<uint16_t>, grid, blk, 0, st, P);
    hipLaunchKernelGGL(mtp_combine, dim3((uint32_t)(B + LLIMA_WAVES - 1) / LLIMA_WAVES), blk, 0, st, P);
    return hipGetLastError() == hipSuccess ? LLIMA_OK : LLIMA_E_HIP;
}
