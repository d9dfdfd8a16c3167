// sample.hip -- fused penalty / temperature / mask / top-k / top-p / min-p /
// inverse-CDF sampling over [B, V] logits rows on MI355X (gfx950).
//
// Two launches per step, with no atomics or fences between workgroups (on
// this part, device-scope cache maintenance and same-address atomics cost far
// more than the whole sweep):
//
// sample_sweep: B x S workgroups; workgroup (row, chunk) streams a 16 KB chunk
//   of its row with 16-byte loads, all issued before anything waits, and keeps
//   it in registers.  It counts the row's history ids that fall in the chunk in
//   an LDS table (packed u16), then computes every value in registers: masked
//   (packed-uint32 grammar bitmask, LSB first), NaN and out-of-row values become
//   -inf and history values take the repetition / frequency / presence
//   penalties.  A lower bound g of the chunk's k-th largest value comes from the
//   lane maxima (a ballot search per wave for the ceil(k/4)-th largest, min over
//   the 4 waves), and every value >= g - |g| 2^-20 is written, with its id, to
//   the chunk's own workspace slot at offsets taken from ballots (no atomics),
//   together with a small header.  The LDS footprint (8 KB for fp32) lets all
//   workgroups of a B=64, V=128256 step be resident at once.
//
// sample_finish: one workgroup per row loads the headers and the candidates
//   straight into registers (16 slots per thread), divides them by the
//   temperature, drops those below the largest chunk bound, proves that no
//   member of the top-k set can be missing (else falls back), and selects with
//   LDS radix histograms whose scans use DPP: the top-k threshold (count), then,
//   for up to 64 survivors, top-p / min-p / the draw by pairwise sums spread
//   over the 4 waves, or otherwise the top-p threshold (fixed-point mass) and
//   the draw (mass by ascending id).  Rows that the candidates cannot serve
//   (overflow, top-k disabled without a mask, degenerate temperatures) are
//   finished by the same workgroup with a full-row multi-pass version.
//
// The sampling semantics have no counterpart in the reference runtime, which
// only ever takes the argmax (sima_lmm/devkit/cpp/utils.hpp:80-152,
// sima_lmm/devkit/cpp/language_model.cpp:3689-3714); greedy rows follow that
// argmax (first index of the maximum) over the masked, penalised row.
#include "common.hpp"
#include "../../include/llima_sampler.h"

namespace llima {

#define SAMPLE_SLOTS 16                            // candidates per finishing thread
#define SAMPLE_FIN_CAP (SAMPLE_SLOTS * LLIMA_WG)   // 4096
#define SAMPLE_ROW_CAND 16384                      // candidate slots per row (all chunks)
#define SAMPLE_MIN_CHUNK 4096                      // smallest chunk (fp32: 256 threads x 16)
#define SAMPLE_SEG 8192                            // full-row path segment
#define SAMPLE_HBATCH 8                            // history ids per thread loaded up front
#define SAMPLE_K_BOUND 256                         // largest top-k the sweep bounds
#define SAMPLE_BOUND_LOWBIT 12                     // key bits below this are not searched
#define SAMPLE_SMALL 64                            // survivors handled one per lane

#define HDR_OVERFLOW 1u
#define HDR_FILTERED 2u

// Written by every sweep workgroup (no state survives a call).
struct ChunkHdr {
    uint32_t count;      // candidates in this chunk's slot
    uint32_t flags;      // HDR_*
    uint32_t bound;      // key of the chunk bound (when FILTERED)
    uint32_t pad;
    uint32_t w[8];       // sampling rows: keys of the two largest lane maxima of
                         // each wave (0: none); greedy rows: w[1]:w[0] =
                         // (key << 32 | ~index) of the chunk maximum
};

struct SampleParams {
    const void* logits;
    int64_t row_stride;
    const int32_t* hist;
    const int32_t* hist_len;
    const uint32_t* bitmask;
    const float* uniforms;
    llima_sampler_config cfg;
    int32_t* out_ids;
    float* out_probs;
    uint32_t* out_keep;
    ChunkHdr* hdr;       // [B][S]
    uint64_t* cand;      // [B][S][share]  (value bits << 32 | id)
    int32_t B, V, H_max, S, share;
    int32_t vec_ok;
    int32_t lp, ls;      // log2 of pre (candidate slots per chunk the finish loads
                         // up front) and of share (slots per chunk)
};

// Pads a chunk's first `pre` candidate slots behind its candidates: value -inf,
// which no bound admits.
#define SAMPLE_SENTINEL (0xFF800000ull << 32)

struct RowCfg {
    float T, p, m, R, alpha, beta;
    int32_t k;
    bool greedy, pen;
    int32_t hlen;
};

__device__ __forceinline__ RowCfg load_cfg(const SampleParams& P, int row) {
    const llima_sampler_config& c = P.cfg;
    RowCfg r;
    r.T = c.temperature_rows ? c.temperature_rows[row] : c.temperature;
    r.k = c.top_k_rows ? c.top_k_rows[row] : c.top_k;
    r.p = c.top_p_rows ? c.top_p_rows[row] : c.top_p;
    r.m = c.min_p_rows ? c.min_p_rows[row] : c.min_p;
    r.R = c.repetition_penalty_rows ? c.repetition_penalty_rows[row] : c.repetition_penalty;
    r.alpha = c.presence_penalty_rows ? c.presence_penalty_rows[row] : c.presence_penalty;
    r.beta = c.frequency_penalty_rows ? c.frequency_penalty_rows[row] : c.frequency_penalty;
    r.greedy = (c.greedy != 0) || !(r.T > 0.0f);
    int h = 0;
    if (P.H_max > 0) {
        h = P.hist_len ? P.hist_len[row] : P.H_max;
        h = h < 0 ? 0 : (h > P.H_max ? P.H_max : h);
    }
    r.hlen = h;
    r.pen = h > 0 && (r.R != 1.0f || r.alpha != 0.0f || r.beta != 0.0f);
    if (!(r.k > 0 && r.k < P.V)) r.k = 0;             // disabled
    return r;
}

// HF RepetitionPenalty (score < 0 ? score * p : score / p), then OpenAI
// frequency and presence, each one IEEE operation (no contraction).
__device__ __forceinline__ float penalize(float l, uint32_t c, const RowCfg& cfg) {
    l = (l < 0.0f) ? l * cfg.R : l / cfg.R;
    return (l - cfg.beta * (float)c) - cfg.alpha;
}

// The pre-filter bound lowered by a relative 2^-20, so that no value whose
// quotient by T can round onto the bound's quotient is filtered out.
__device__ __forceinline__ float lower_bound_margin(float t) {
    return t - __builtin_fabsf(t) * 0x1p-20f;
}

__device__ __forceinline__ uint32_t table_count(const uint32_t* table, uint32_t off) {
    return (table[off >> 1] >> ((off & 1u) * 16u)) & 0xFFFFu;
}

template <typename TL>
__device__ __forceinline__ float load_one(const TL* rowp, int i);
template <>
__device__ __forceinline__ float load_one<float>(const float* rowp, int i) { return rowp[i]; }
template <>
__device__ __forceinline__ float load_one<uint16_t>(const uint16_t* rowp, int i) {
    return bf16_bits_to_f32(rowp[i]);
}

// Counts the row's history ids in [lo, hi) into an LDS table of packed u16
// counts (full-row path).
__device__ __forceinline__ void count_history(const SampleParams& P, int row, int hlen, int lo,
                                              int hi, uint32_t* table, int nwords) {
    for (int i = threadIdx.x; i < nwords; i += LLIMA_WG) table[i] = 0;
    __syncthreads();
    const int32_t* h = P.hist + (size_t)row * P.H_max;
    for (int j = threadIdx.x; j < hlen; j += LLIMA_WG) {
        const int32_t id = h[j];
        if (id >= lo && id < hi) {
            const uint32_t off = (uint32_t)(id - lo);
            atomicAdd(&table[off >> 1], 1u << ((off & 1u) * 16u));
        }
    }
    __syncthreads();
}

// ================================================================== sweep
// VEC: rows are 16-byte aligned and V is a multiple of the values per load, so
// every chunk (also a row's partial last one) is read with 16-byte loads from
// clamped, always-valid addresses and the out-of-row values masked in registers.
template <bool B>
struct Flag { static constexpr bool value = B; };

// MASK: a grammar bitmask is given.  NaN values are never turned into -inf
// here: every later use is an ordered comparison (x > best, x > lane max,
// x >= bound), which a NaN fails, so a NaN is never selected.
template <typename TL, int E, bool VEC, bool MASK>
__global__ __launch_bounds__(LLIMA_WG) void sample_sweep(SampleParams P) {
    constexpr int EPL = 16 / sizeof(TL);       // values per 16-byte load
    constexpr int NL = E / EPL;                // loads per thread
    constexpr int CHUNK = LLIMA_WG * E;
    constexpr int CW = CHUNK / 2;              // history count words
    __shared__ __align__(16) uint32_t cnt[CW];
    __shared__ uint32_t xw[4][LLIMA_WAVES];
    __shared__ uint64_t xg[LLIMA_WAVES];
    const float NEG_INF = -__builtin_inff();

    uint32_t row, chunk;
    map_row_chunk(blockIdx.x, (uint32_t)P.B, (uint32_t)P.S, &row, &chunk);
    if (row >= (uint32_t)P.B) return;
    const int t = (int)threadIdx.x;
    const uint32_t lane = lane_id(), wave = wave_id();
    const TL* rowp = (const TL*)P.logits + (size_t)row * P.row_stride;
    const int V = P.V;
    const int c0 = (int)chunk * CHUNK;
    const int c1 = c0 + CHUNK < V ? c0 + CHUNK : V;
    const int H = P.H_max;
    const int32_t* hrow = P.hist + (size_t)row * H;
    const uint32_t* mrow = P.bitmask ? P.bitmask + (size_t)row * ((V + 31) >> 5) : nullptr;

    // ---- 1. every load, issued before anything waits and in the order the
    //         data is consumed: history ids, mask words, the chunk.  Only
    //         kernel arguments decide them (the row's configuration is still
    //         in flight); every address is valid.
    int32_t hid[SAMPLE_HBATCH];
#pragma unroll
    for (int b = 0; b < SAMPLE_HBATCH; ++b) {
        const int j = t + b * LLIMA_WG;
        hid[b] = (b * LLIMA_WG < H) ? hrow[j < H ? j : H - 1] : -1;
    }
    uint32_t mword[NL];
    if constexpr (MASK) {
#pragma unroll
        for (int j = 0; j < NL; ++j) {
            const int i0 = c0 + j * (LLIMA_WG * EPL) + t * EPL;
            mword[j] = mrow[(i0 < V ? i0 : V - 1) >> 5];
        }
    }
    llima_u32x4 raw[NL];
#pragma unroll
    for (int j = 0; j < NL; ++j) {
        const int i0 = c0 + j * (LLIMA_WG * EPL) + t * EPL;
        if constexpr (VEC) {
            const int ia = i0 < V ? i0 : V - EPL;
            raw[j] = __builtin_nontemporal_load((const llima_u32x4*)(rowp + ia));
        } else {
            uint32_t w[4] = {0, 0, 0, 0};
#pragma unroll
            for (int e = 0; e < EPL; ++e) {
                const int ia = i0 + e < V ? i0 + e : V - 1;
                const float f = load_one<TL>(rowp, ia);
                if constexpr (sizeof(TL) == 4) w[e] = __float_as_uint(f);
                else w[e >> 1] |= (__float_as_uint(f) >> 16) << ((e & 1) * 16);
            }
            raw[j] = llima_u32x4{w[0], w[1], w[2], w[3]};
        }
    }
    const RowCfg c = load_cfg(P, row);

    // ---- 2. history counts of the chunk
    if (c.pen) {
        for (int i = t; i < CW / 4; i += LLIMA_WG) ((llima_u32x4*)cnt)[i] = llima_u32x4{0, 0, 0, 0};
        __syncthreads();
#pragma unroll
        for (int b = 0; b < SAMPLE_HBATCH; ++b) {
            const int32_t id = hid[b];
            if (t + b * LLIMA_WG < c.hlen && id >= c0 && id < c1) {
                const uint32_t off = (uint32_t)(id - c0);
                atomicAdd(&cnt[off >> 1], 1u << ((off & 1u) * 16u));
            }
        }
        for (int j = t + SAMPLE_HBATCH * LLIMA_WG; j < c.hlen; j += LLIMA_WG) {
            const int32_t id = hrow[j];
            if (id >= c0 && id < c1) {
                const uint32_t off = (uint32_t)(id - c0);
                atomicAdd(&cnt[off >> 1], 1u << ((off & 1u) * 16u));
            }
        }
        __syncthreads();
    }

    // ---- 3. values: masked and out-of-row -> -inf, history values penalised
    float v[E];
    auto convert = [&](auto pen_tag) {
        constexpr bool PEN = decltype(pen_tag)::value;
#pragma unroll
        for (int j = 0; j < NL; ++j) {
            const int i0 = c0 + j * (LLIMA_WG * EPL) + t * EPL;
            float xs[EPL];
            const uint32_t w4[4] = {raw[j].x, raw[j].y, raw[j].z, raw[j].w};
            if constexpr (sizeof(TL) == 4) {
#pragma unroll
                for (int e = 0; e < 4; ++e) xs[e] = __uint_as_float(w4[e]);
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    xs[2 * e] = __uint_as_float(w4[e] << 16);
                    xs[2 * e + 1] = __uint_as_float(w4[e] & 0xFFFF0000u);
                }
            }
            if constexpr (MASK) {
                const uint32_t mb = mword[j] >> (i0 & 31);
#pragma unroll
                for (int e = 0; e < EPL; ++e) xs[e] = ((mb >> e) & 1u) ? xs[e] : NEG_INF;
            }
            if constexpr (PEN) {
                uint32_t cw[EPL / 2];
                const uint32_t* cp = cnt + ((i0 - c0) >> 1);
                if constexpr (EPL == 4) {
                    const uint2 w2 = *(const uint2*)cp;
                    cw[0] = w2.x; cw[1] = w2.y;
                } else {
                    const llima_u32x4 wq = *(const llima_u32x4*)cp;
                    cw[0] = wq.x; cw[1] = wq.y; cw[2] = wq.z; cw[3] = wq.w;
                }
#pragma unroll
                for (int h = 0; h < EPL / 2; ++h) {
                    if (cw[h]) {
                        const uint32_t lo = cw[h] & 0xFFFFu, hi = cw[h] >> 16;
                        if (lo) xs[2 * h] = penalize(xs[2 * h], lo, c);
                        if (hi) xs[2 * h + 1] = penalize(xs[2 * h + 1], hi, c);
                    }
                }
            }
#pragma unroll
            for (int e = 0; e < EPL; ++e) v[j * EPL + e] = xs[e];
        }
    };
    if (c.pen) convert(Flag<true>{});
    else convert(Flag<false>{});
    if (c1 - c0 < CHUNK) {                         // the row's last, partial chunk
#pragma unroll
        for (int j = 0; j < NL; ++j) {
            const int i0 = c0 + j * (LLIMA_WG * EPL) + t * EPL;
#pragma unroll
            for (int e = 0; e < EPL; ++e)
                if (i0 + e >= c1) v[j * EPL + e] = NEG_INF;
        }
    }

    ChunkHdr* hdr = P.hdr + (size_t)row * P.S + chunk;
    if (c.greedy) {
        // ---- argmax: first index of the maximum (values visited in index order)
        float best = NEG_INF;
        uint32_t bidx = 0xFFFFFFFFu;
#pragma unroll
        for (int j = 0; j < NL; ++j) {
            const int i0 = c0 + j * (LLIMA_WG * EPL) + t * EPL;
#pragma unroll
            for (int e = 0; e < EPL; ++e)
                if (v[j * EPL + e] > best) { best = v[j * EPL + e]; bidx = (uint32_t)(i0 + e); }
        }
        const uint32_t kb = best > NEG_INF ? f32_key(best) : 0u;
        const uint32_t wk = wave_max_u32(kb);
        const uint32_t wi = wave_max_u32((wk != 0 && kb == wk) ? ~bidx : 0u);
        if (lane == 0) xg[wave] = wk ? (((uint64_t)wk << 32) | wi) : 0ull;
        __syncthreads();
        if (t == 0) {
            uint64_t g = 0;
#pragma unroll
            for (int w = 0; w < LLIMA_WAVES; ++w) g = xg[w] > g ? xg[w] : g;
            *(llima_u32x4*)hdr = llima_u32x4{0u, 0u, 0u, 0u};
            *(llima_u32x4*)hdr->w = llima_u32x4{(uint32_t)g, (uint32_t)(g >> 32), 0u, 0u};
            *(llima_u32x4*)(hdr->w + 4) = llima_u32x4{0u, 0u, 0u, 0u};
        }
        return;
    }

    // ---- 4. chunk bound: every wave has >= r = ceil(k/4) lanes whose maximum
    //         is >= its bound, so the chunk has >= 4r >= k values >= their min
    uint32_t gkey = 0;
    if (c.k > 0 && c.k <= SAMPLE_K_BOUND) {
        float lm = NEG_INF;
#pragma unroll
        for (int e = 0; e < E; ++e) lm = v[e] > lm ? v[e] : lm;
        const uint32_t lk = lm > NEG_INF ? f32_key(lm) : 0u;
        const uint32_t r = ((uint32_t)c.k + 3u) >> 2;
        const uint32_t tw = wave_rth_largest(lk, r, SAMPLE_BOUND_LOWBIT);
        const uint32_t wm = wave_max_u32(lk);
        const uint32_t wm2 = wave_max_u32(lk < wm ? lk : 0u);   // a lane other than the maximum's
        if (lane == 0) { xw[0][wave] = tw; xw[2][wave] = wm; xw[3][wave] = wm2; }
        __syncthreads();
        gkey = xw[0][0];
#pragma unroll
        for (int w = 1; w < LLIMA_WAVES; ++w) gkey = xw[0][w] < gkey ? xw[0][w] : gkey;
    }
    float g = -__FLT_MAX__;                       // keeps every finite value
    if (gkey) {
        const float m = lower_bound_margin(key_f32(gkey));
        g = m > -__FLT_MAX__ ? m : -__FLT_MAX__;
    }

    // ---- 5. write the values >= g: count per wave, then ballot offsets
    uint32_t wcount = 0;
#pragma unroll
    for (int e = 0; e < E; ++e) wcount += (uint32_t)__popcll(ballot(v[e] >= g));
    if (lane == 0) xw[1][wave] = wcount;
    __syncthreads();
    uint32_t base = 0, total = 0;
#pragma unroll
    for (int w = 0; w < LLIMA_WAVES; ++w) {
        const uint32_t n = xw[1][w];
        base += (uint32_t)w < wave ? n : 0u;
        total += n;
    }
    const uint32_t cap = 1u << P.ls;
    if (total <= cap) {
        uint64_t* dst = P.cand + (((size_t)row * P.S + chunk) << P.ls);
        uint32_t o = base;
#pragma unroll
        for (int j = 0; j < NL; ++j) {
            const int i0 = c0 + j * (LLIMA_WG * EPL) + t * EPL;
#pragma unroll
            for (int e = 0; e < EPL; ++e) {
                const float x = v[j * EPL + e];
                const bool pr = x >= g;
                const uint64_t m = ballot(pr);
                if (m) {
                    if (pr) dst[mbcnt_add(m, o)] = ((uint64_t)__float_as_uint(x) << 32) | (uint32_t)(i0 + e);
                    o += (uint32_t)__popcll(m);
                }
            }
        }
        for (uint32_t i = total + (uint32_t)t; i < (1u << P.lp); i += LLIMA_WG) dst[i] = SAMPLE_SENTINEL;
    }
    if (t == 0) {
        *(llima_u32x4*)hdr = llima_u32x4{total <= cap ? total : 0u,
                                         (total > cap ? HDR_OVERFLOW : 0u) | (gkey ? HDR_FILTERED : 0u),
                                         gkey, 0u};
        *(llima_u32x4*)hdr->w = gkey ? llima_u32x4{xw[2][0], xw[2][1], xw[2][2], xw[2][3]}
                                     : llima_u32x4{0u, 0u, 0u, 0u};
        *(llima_u32x4*)(hdr->w + 4) = gkey ? llima_u32x4{xw[3][0], xw[3][1], xw[3][2], xw[3][3]}
                                           : llima_u32x4{0u, 0u, 0u, 0u};
    }
}

// ================================================================== finish
struct FinishShared {
    union {
        uint64_t cbuf[SAMPLE_FIN_CAP];         // candidates gathered in chunk order
        uint32_t table[SAMPLE_SEG / 2];        // full-row path history counts
    } u;
    uint32_t wcnt[LLIMA_WAVES][LLIMA_WG];      // each wave's own copy of the chunk counts
    uint32_t coff[LLIMA_WG];                   // chunk offsets (gather path)
    uint64_t stage[LLIMA_WAVES][SAMPLE_SMALL]; // survivors of the bound, per wave
    uint32_t hcnt[2][256];                     // radix histograms (double-buffered)
    uint64_t hmass[2][256];
    uint64_t above[256];
    uint64_t part[2][LLIMA_WAVES][64];
    llima_u32x4 sv[LLIMA_WAVES][64];           // each wave's copy of the survivors
    uint32_t bh[LLIMA_WAVES][256];             // each wave's histogram of header values
    uint32_t pc[LLIMA_WAVES][64];
    uint32_t r32[8][LLIMA_WAVES];
    uint64_t r64[2][LLIMA_WAVES];
    uint32_t sel[2];
    uint64_t sel64[2];
    BlockScratch bs;
};

// ------------------------------------------------------------------ radix selects
// Each select runs over register-resident elements (SAMPLE_SLOTS per thread,
// key 0 = absent).  Digits are 8 bits wide and start at the highest bit in
// which the keys differ (the bits above it are common to all of them).
// hcnt[buf] and hmass[buf] are zero on entry and on return; every round clears
// the other buffer for the next one, so a round needs three barriers.
struct Digits {
    uint32_t prefix, pmask;   // fixed high bits of the selected key
    int top;                  // top bit of the next digit (-1: done)
};

__device__ __forceinline__ Digits digits_init(uint32_t kmin, uint32_t kmax) {
    Digits d;
    const uint32_t diff = kmax ^ kmin;
    if (diff == 0) { d.prefix = kmax; d.pmask = 0xFFFFFFFFu; d.top = -1; return d; }
    d.top = 31 - __builtin_clz(diff);
    d.pmask = d.top == 31 ? 0u : ~((2u << d.top) - 1u);
    d.prefix = kmax & d.pmask;
    return d;
}

// Exclusive prefix of v over the workgroup in thread order, given this wave's
// inclusive scan inc; r is a per-wave LDS slot array.  Contains one barrier.
__device__ __forceinline__ uint64_t wg_prefix_u64(uint64_t inc, uint64_t v, uint64_t* r) {
    const uint32_t wave = wave_id();
    if (lane_id() == 63) r[wave] = inc;
    __syncthreads();
    uint64_t before = 0;
#pragma unroll
    for (int w = 0; w < LLIMA_WAVES; ++w) before += (uint32_t)w < wave ? r[w] : 0ull;
    return before + inc - v;
}

// k-th largest key (with multiplicity) among the elements, all of whose keys
// lie in [kmin, kmax].
__device__ __forceinline__ uint32_t fin_kth_desc(const uint32_t (&key)[SAMPLE_SLOTS], uint32_t k,
                                                 uint32_t kmin, uint32_t kmax, FinishShared& sh,
                                                 int& buf) {
    Digits d = digits_init(kmin, kmax);
    uint32_t rem = k;
    const uint32_t t = threadIdx.x;
    while (d.top >= 0) {
        const int lo = d.top - 7 > 0 ? d.top - 7 : 0;
        const uint32_t bmask = (1u << (d.top - lo + 1)) - 1u;
        uint32_t* hc = sh.hcnt[buf];
#pragma unroll
        for (int j = 0; j < SAMPLE_SLOTS; ++j)
            if (key[j] && (key[j] & d.pmask) == d.prefix) atomicAdd(&hc[(key[j] >> lo) & bmask], 1u);
        __syncthreads();
        const uint32_t bin = 255u - t;                 // thread 0 <-> top bin
        const uint32_t cn = hc[bin];
        sh.hcnt[buf ^ 1][t] = 0;
        sh.hmass[buf ^ 1][t] = 0;
        const uint32_t inc = wave_incl_scan_u32(cn);
        const uint32_t above = (uint32_t)wg_prefix_u64(inc, cn, sh.r64[0]);
        if (above < rem && above + cn >= rem) { sh.sel[0] = bin; sh.sel[1] = rem - above; }
        __syncthreads();
        d.prefix |= sh.sel[0] << lo;
        d.pmask |= bmask << lo;
        d.top = lo - 1;
        rem = sh.sel[1];
        buf ^= 1;
    }
    return d.prefix;
}

// Top-p boundary: the smallest key theta such that an element with key theta has
// (mass strictly above) * 2^32 < PZ; when none has (PZ == 0) the top key.
__device__ __forceinline__ uint32_t fin_topp_desc(const uint32_t (&key)[SAMPLE_SLOTS],
                                                  const uint64_t (&w)[SAMPLE_SLOTS],
                                                  llima_u128 PZ, uint32_t kmin, uint32_t kmax,
                                                  FinishShared& sh, int& buf) {
    Digits d = digits_init(kmin, kmax);
    uint64_t acc = 0;
    const uint32_t t = threadIdx.x, lane = lane_id(), wave = wave_id();
    while (d.top >= 0) {
        const int lo = d.top - 7 > 0 ? d.top - 7 : 0;
        const uint32_t bmask = (1u << (d.top - lo + 1)) - 1u;
        uint32_t* hc = sh.hcnt[buf];
        uint64_t* hm = sh.hmass[buf];
#pragma unroll
        for (int j = 0; j < SAMPLE_SLOTS; ++j) {
            if (key[j] && (key[j] & d.pmask) == d.prefix) {
                const uint32_t b = (key[j] >> lo) & bmask;
                atomicAdd(&hc[b], 1u);
                if (w[j]) atomicAdd((unsigned long long*)&hm[b], (unsigned long long)w[j]);
            }
        }
        __syncthreads();
        const uint32_t bin = 255u - t;
        const uint32_t cn = hc[bin];
        const uint64_t m = hm[bin];
        sh.hcnt[buf ^ 1][t] = 0;
        sh.hmass[buf ^ 1][t] = 0;
        const uint64_t inc = wave_incl_scan_u64(m);
        const uint64_t above = acc + wg_prefix_u64(inc, m, sh.r64[0]);
        const bool cond = cn > 0 && (((llima_u128)above << 32) < PZ);
        sh.above[t] = above;
        const uint64_t bc = ballot(cond), bn = ballot(cn > 0);
        if (lane == 0) {
            sh.r32[1][wave] = bc ? 64u - (uint32_t)__builtin_clzll(bc) : 0u;    // highest lane + 1
            sh.r32[2][wave] = bn ? (uint32_t)__builtin_ffsll((long long)bn) : 0u;   // lowest lane + 1
        }
        __syncthreads();
        // the lowest qualifying bin (highest t); else the top non-empty bin (lowest t)
        int sel_t = -1;
#pragma unroll
        for (int w2 = LLIMA_WAVES - 1; w2 >= 0; --w2)
            if (sel_t < 0 && sh.r32[1][w2]) sel_t = w2 * 64 + (int)sh.r32[1][w2] - 1;
        if (sel_t < 0) {
#pragma unroll
            for (int w2 = 0; w2 < LLIMA_WAVES; ++w2)
                if (sel_t < 0 && sh.r32[2][w2]) sel_t = w2 * 64 + (int)sh.r32[2][w2] - 1;
        }
        if (sel_t < 0) sel_t = 0;
        d.prefix |= (255u - (uint32_t)sel_t) << lo;
        d.pmask |= bmask << lo;
        d.top = lo - 1;
        acc = sh.above[sel_t];
        buf ^= 1;
    }
    return d.prefix;
}

// Draw: the smallest id whose ascending-id prefix mass exceeds target (< the
// total mass); also returns that element's weight.  Ids are < V <= 2^24.
__device__ __forceinline__ uint32_t fin_draw_asc(const uint32_t (&id)[SAMPLE_SLOTS],
                                                 const uint64_t (&w)[SAMPLE_SLOTS], uint64_t target,
                                                 uint32_t V, uint64_t* w_out, FinishShared& sh,
                                                 int& buf) {
    Digits d = digits_init(0u, V > 1 ? V - 1 : 1u);
    uint64_t acc = 0;
    const uint32_t t = threadIdx.x;
    while (d.top >= 0) {
        const int lo = d.top - 7 > 0 ? d.top - 7 : 0;
        const uint32_t bmask = (1u << (d.top - lo + 1)) - 1u;
        uint64_t* hm = sh.hmass[buf];
#pragma unroll
        for (int j = 0; j < SAMPLE_SLOTS; ++j)
            if (w[j] && (id[j] & d.pmask) == d.prefix)
                atomicAdd((unsigned long long*)&hm[(id[j] >> lo) & bmask], (unsigned long long)w[j]);
        __syncthreads();
        const uint32_t bin = t;
        const uint64_t m = hm[bin];
        sh.hcnt[buf ^ 1][t] = 0;
        sh.hmass[buf ^ 1][t] = 0;
        const uint64_t inc = wave_incl_scan_u64(m);
        const uint64_t below = acc + wg_prefix_u64(inc, m, sh.r64[0]);
        if (m > 0 && below <= target && target < below + m) {
            sh.sel[0] = bin; sh.sel64[0] = below; sh.sel64[1] = m;
        }
        __syncthreads();
        d.prefix |= sh.sel[0] << lo;
        d.pmask |= bmask << lo;
        d.top = lo - 1;
        acc = sh.sel64[0];
        *w_out = sh.sel64[1];
        buf ^= 1;
    }
    return d.prefix;
}

__device__ __forceinline__ void write_result(const SampleParams& P, int row, int32_t id, float prob) {
    P.out_ids[row] = id;
    if (P.out_probs) P.out_probs[row] = prob;
}

// Writes the kept set of a row as a bitmask (zero-filled first).
template <class Visit>
__device__ __forceinline__ void write_keep(const SampleParams& P, int row, Visit visit) {
    const int nw = (P.V + 31) >> 5;
    uint32_t* km = P.out_keep + (size_t)row * nw;
    for (int i = threadIdx.x; i < nw; i += LLIMA_WG) km[i] = 0;
    __threadfence_block();
    __syncthreads();
    visit([&](uint32_t id) {
        if (id < (uint32_t)P.V) atomicOr(&km[id >> 5], 1u << (id & 31u));
    });
    __syncthreads();
}

// ------------------------------------------------------------------ full-row path
// Exact multi-pass selection by one workgroup; recomputes x for the whole row on
// every pass (history table rebuilt per segment).
template <typename TL>
__device__ __forceinline__ void finish_full_row(const SampleParams& P, int row, const RowCfg& c,
                                             FinishShared& sh) {
    const TL* rowp = (const TL*)P.logits + (size_t)row * P.row_stride;
    const int V = P.V;
    const int nw = (V + 31) >> 5;
    const uint32_t* mrow = P.bitmask ? P.bitmask + (size_t)row * nw : nullptr;
    uint32_t* table = sh.u.table;
    __syncthreads();
    // fn(x, id) for every element of the row.
    auto for_each_x = [&](auto fn) {
        for (int lo = 0; lo < V; lo += SAMPLE_SEG) {
            const int hi = lo + SAMPLE_SEG < V ? lo + SAMPLE_SEG : V;
            if (c.pen) count_history(P, row, c.hlen, lo, hi, table, SAMPLE_SEG / 2);
            for (int i = lo + threadIdx.x; i < hi; i += LLIMA_WG) {
                float l = load_one<TL>(rowp, i);
                if (l != l) l = -__builtin_inff();
                if (mrow && !((mrow[i >> 5] >> (i & 31)) & 1u)) l = -__builtin_inff();
                if (c.pen) {
                    const uint32_t cnt = table_count(table, (uint32_t)(i - lo));
                    if (cnt) l = penalize(l, cnt, c);
                }
                fn(c.greedy ? l : l / c.T, (uint32_t)i);
            }
            __syncthreads();
        }
    };
    // Radix select over the row: histogram rounds that visit every element.
    auto radix = [&](auto elem, uint32_t kmin, uint32_t kmax, auto pick) {
        // elem(x, id, fn): calls fn(key, weight) for elements taking part
        Digits d = digits_init(kmin, kmax);
        uint64_t acc = 0;
        uint32_t rem = 0;
        while (d.top >= 0) {
            const int lo = d.top - 7 > 0 ? d.top - 7 : 0;
            const uint32_t bmask = (1u << (d.top - lo + 1)) - 1u;
            sh.hcnt[0][threadIdx.x] = 0;
            sh.hmass[0][threadIdx.x] = 0;
            __syncthreads();
            const uint32_t prefix = d.prefix, pmask = d.pmask;
            for_each_x([&](float x, uint32_t id) {
                elem(x, id, [&](uint32_t key, uint64_t w) {
                    if ((key & pmask) == prefix) {
                        const uint32_t b = (key >> lo) & bmask;
                        atomicAdd(&sh.hcnt[0][b], 1u);
                        if (w) atomicAdd((unsigned long long*)&sh.hmass[0][b], (unsigned long long)w);
                    }
                });
            });
            __syncthreads();
            const uint32_t sel = pick(lo, acc, rem);
            d.prefix |= sel << lo;
            d.pmask |= bmask << lo;
            d.top = lo - 1;
            __syncthreads();
        }
        return d.prefix;
    };

    if (c.greedy) {
        uint64_t best = 0;
        for_each_x([&](float x, uint32_t id) {
            const uint64_t kk = ((uint64_t)f32_key(x) << 32) | (uint64_t)(~id);
            best = kk > best ? kk : best;
        });
        best = block_max_u64(best, sh.bs);
        const bool ok = (uint32_t)(best >> 32) > LLIMA_KEY_NEG_INF;
        const uint32_t tok = ok ? ~(uint32_t)best : 0xFFFFFFFFu;
        if (threadIdx.x == 0) write_result(P, row, ok ? (int32_t)tok : -1, ok ? 1.0f : 0.0f);
        if (P.out_keep)
            write_keep(P, row, [&](auto set) { if (threadIdx.x == 0 && ok) set(tok); });
        return;
    }

    // Pass: maximum, minimum and number of finite values.
    uint32_t kmax = 0, nkmin = 0, nfin = 0;
    for_each_x([&](float x, uint32_t) {
        const uint32_t k = f32_key(x);
        if (k > LLIMA_KEY_NEG_INF) {
            nfin++;
            kmax = k > kmax ? k : kmax;
            nkmin = ~k > nkmin ? ~k : nkmin;
        }
    });
    kmax = block_max_u32(kmax, sh.bs);
    const uint32_t kmin = ~block_max_u32(nkmin, sh.bs);
    nfin = block_sum_u32(nfin, sh.bs);
    if (nfin == 0) {
        if (threadIdx.x == 0) write_result(P, row, -1, 0.0f);
        if (P.out_keep) write_keep(P, row, [&](auto) {});
        return;
    }
    const float xmax = key_f32(kmax);

    // top-k threshold
    uint32_t tau = LLIMA_KEY_NEG_INF + 1u;
    if (c.k > 0 && (uint32_t)c.k <= nfin) {
        uint32_t rem = (uint32_t)c.k;
        tau = radix(
            [&](float x, uint32_t, auto fn) {
                const uint32_t k = f32_key(x);
                if (k > LLIMA_KEY_NEG_INF) fn(k, 0ull);
            },
            kmin, kmax,
            [&](int, uint64_t&, uint32_t&) {
                const uint32_t bin = 255u - threadIdx.x;
                const uint32_t cn = sh.hcnt[0][bin];
                uint32_t tot;
                const uint32_t above = block_excl_scan_u32(cn, &tot, sh.bs);
                if (above < rem && above + cn >= rem) { sh.sel[0] = bin; sh.sel[1] = rem - above; }
                __syncthreads();
                rem = sh.sel[1];
                return sh.sel[0];
            });
    }
    const uint32_t kmin_k = tau > kmin ? tau : kmin;
    auto elem_k = [&](float x, uint32_t id, auto fn) {
        const uint32_t k = f32_key(x);
        if (k >= tau) fn(k, weight(x, xmax));
        (void)id;
    };

    // top-p threshold
    uint32_t theta = 0;
    if (c.p < 1.0f) {
        uint64_t Z = 0;
        for_each_x([&](float x, uint32_t id) { elem_k(x, id, [&](uint32_t, uint64_t w) { Z += w; }); });
        Z = block_sum_u64(Z, sh.bs);
        const llima_u128 PZ = (llima_u128)frac32(c.p) * Z;
        uint64_t acc = 0;
        theta = radix(elem_k, kmin_k, kmax, [&](int, uint64_t&, uint32_t&) {
            const uint32_t t = threadIdx.x, bin = 255u - t;
            const uint32_t cn = sh.hcnt[0][bin];
            uint64_t m = sh.hmass[0][bin], tot;
            const uint64_t above = acc + block_excl_scan_u64(m, &tot, sh.bs);
            const bool cond = cn > 0 && (((llima_u128)above << 32) < PZ);
            const uint32_t best_cond = block_max_u32(cond ? t + 1u : 0u, sh.bs);
            const uint32_t top_nonempty = 255u - block_max_u32(cn > 0 ? 255u - t : 0u, sh.bs);
            const uint32_t sel_t = best_cond ? best_cond - 1u : top_nonempty;
            if (t == sel_t) { sh.sel[0] = bin; sh.sel64[0] = above; }
            __syncthreads();
            acc = sh.sel64[0];
            return sh.sel[0];
        });
    }
    const uint64_t mthr = c.m > 0.0f ? frac32(c.m) << 4 : 0;
    auto fin_elem = [&](float x, uint32_t id, auto fn) {
        const uint32_t k = f32_key(x);
        if (k >= tau && k >= theta) {
            const uint64_t w = weight(x, xmax);
            if (w >= mthr) fn(id, w);
        }
    };
    uint64_t Zf = 0;
    for_each_x([&](float x, uint32_t id) { fin_elem(x, id, [&](uint32_t, uint64_t w) { Zf += w; }); });
    Zf = block_sum_u64(Zf, sh.bs);
    int32_t tok = -1;
    float prob = 0.0f;
    if (Zf > 0) {
        const uint64_t target = (uint64_t)(((llima_u128)uniform32(P.uniforms[row]) * Zf) >> 32);
        uint64_t acc = 0, wtok = 0;
        tok = (int32_t)radix(
            [&](float x, uint32_t id, auto fn) {
                fin_elem(x, id, [&](uint32_t i, uint64_t w) { if (w) fn(i, w); });
            },
            0u, (uint32_t)(V > 1 ? V - 1 : 1),
            [&](int, uint64_t&, uint32_t&) {
                const uint32_t bin = threadIdx.x;
                uint64_t m = sh.hmass[0][bin], tot;
                const uint64_t below = acc + block_excl_scan_u64(m, &tot, sh.bs);
                if (m > 0 && below <= target && target < below + m) {
                    sh.sel[0] = bin; sh.sel64[0] = below; sh.sel64[1] = m;
                }
                __syncthreads();
                acc = sh.sel64[0];
                wtok = sh.sel64[1];
                return sh.sel[0];
            });
        prob = (float)((double)wtok / (double)Zf);
    }
    if (threadIdx.x == 0) write_result(P, row, tok, prob);
    if (P.out_keep)
        write_keep(P, row, [&](auto set) {
            for_each_x([&](float x, uint32_t id) { fin_elem(x, id, [&](uint32_t i, uint64_t) { set(i); }); });
        });
}

// ------------------------------------------------------------------ fast path
// At most 64 candidates left by the bound, one per lane in every wave (lanes
// >= nk and candidates that are -inf after the temperature hold key 0).  One
// pairwise pass, split over the 4 waves by the candidate it reads (broadcast
// LDS reads of the wave's own copy), gives each lane the number of keys above
// and equal to its own and the mass above it: the top-k threshold is the key
// of a lane with (above < k <= above + equal), and the top-p test uses the
// mass above, which for a kept lane only counts kept lanes.  A second pass
// gives the mass of final ids up to each id for the draw.  False when the
// bound cannot be proven to keep the top-k set (full-row path).
__device__ __forceinline__ bool fin_small(const SampleParams& P, int row, const RowCfg& c,
                                          uint32_t key, uint32_t id, uint32_t nk, uint32_t nfin,
                                          uint32_t kmin, uint32_t kmax, uint32_t gthr,
                                          FinishShared& sh) {
    const uint32_t lane = lane_id(), wave = wave_id();
    const uint64_t w = key ? weight(key_f32(key), key_f32(kmax)) : 0ull;
    const uint32_t j0 = wave * 16u;
    sh.sv[wave][lane] = llima_u32x4{key, id, (uint32_t)w, (uint32_t)(w >> 32)};
    uint32_t gt = 0, eq = 0;
    uint64_t above = 0;
    // lanes >= nk hold key 0, weight 0: reading them changes nothing
#pragma unroll
    for (uint32_t jj = 0; jj < 16; ++jj) {
        const llima_u32x4 o = sh.sv[wave][j0 + jj];
        const uint64_t wj = ((uint64_t)o.w << 32) | o.z;
        gt += o.x > key ? 1u : 0u;
        eq += o.x == key ? 1u : 0u;
        above += o.x > key ? wj : 0ull;
    }
    sh.part[0][wave][lane] = above;
    sh.pc[wave][lane] = gt | (eq << 16);
    __syncthreads();
    above = 0; gt = 0; eq = 0;
#pragma unroll
    for (int w2 = 0; w2 < LLIMA_WAVES; ++w2) {
        above += sh.part[0][w2][lane];
        const uint32_t g2 = sh.pc[w2][lane];
        gt += g2 & 0xFFFFu;
        eq += g2 >> 16;
    }
    uint32_t tau = kmin;
    if (c.k > 0 && (uint32_t)c.k < nfin) {
        const bool at = key != 0 && gt < (uint32_t)c.k && gt + eq >= (uint32_t)c.k;
        tau = wave_max_u32(at ? key : 0u);
    } else if (c.k > 0 && (uint32_t)c.k > nfin && gthr) {
        return false;
    }
    // the proof that the bound dropped no member of the top-k set: a value
    // below it has x <= fl(g / T) < tau
    if (gthr && !(lower_bound_margin(key_f32(gthr)) / c.T < key_f32(tau))) return false;

    const bool mine = key != 0 && key >= tau;
    bool fin = mine;
    if (c.p < 1.0f) {
        // (above << 32) < frac32(p) * Z  <=>  above < ceil(frac32(p) * Z / 2^32)
        const uint64_t Z = wave_sum_u64(mine ? w : 0ull);
        const llima_u128 PZ = (llima_u128)frac32(c.p) * Z;
        const uint64_t plim = (uint64_t)((PZ + 0xFFFFFFFFull) >> 32);
        fin = fin && (above < plim || key == kmax);
    }
    if (c.m > 0.0f) fin = fin && w >= (frac32(c.m) << 4);
    const uint64_t wf = fin ? w : 0ull;
    const uint64_t Zf = wave_sum_u64(wf);            // the same in every wave
    if (Zf == 0) {
        if (threadIdx.x == 0) write_result(P, row, -1, 0.0f);
    } else {
        const uint64_t target = (uint64_t)(((llima_u128)uniform32(P.uniforms[row]) * Zf) >> 32);
        sh.sv[wave][lane] = llima_u32x4{id, 0u, (uint32_t)wf, (uint32_t)(wf >> 32)};
        uint64_t upto = 0;                            // mass of final ids <= this id
#pragma unroll
        for (uint32_t jj = 0; jj < 16; ++jj) {
            const llima_u32x4 o = sh.sv[wave][j0 + jj];
            upto += o.x <= id ? (((uint64_t)o.w << 32) | o.z) : 0ull;
        }
        sh.part[1][wave][lane] = upto;
        __syncthreads();
        upto = 0;
#pragma unroll
        for (int w2 = 0; w2 < LLIMA_WAVES; ++w2) upto += sh.part[1][w2][lane];
        if (wave == 0 && wf > 0 && upto - wf <= target && target < upto)
            write_result(P, row, (int32_t)id, (float)((double)wf / (double)Zf));
    }
    if (P.out_keep)
        write_keep(P, row, [&](auto set) { if (wave == 0 && fin) set(id); });
    return true;
}

// Many survivors (top-k disabled, ties, k > 64): radix selects over the
// register-resident candidates.
__device__ __forceinline__ void fin_large(const SampleParams& P, int row, const RowCfg& c,
                                          uint32_t (&key)[SAMPLE_SLOTS],
                                          const uint32_t (&id)[SAMPLE_SLOTS], uint32_t tau,
                                          uint32_t kmax, FinishShared& sh, int& buf) {
    uint64_t w[SAMPLE_SLOTS];
    const float xmax = key_f32(kmax);
    uint64_t Z = 0;
#pragma unroll
    for (int j = 0; j < SAMPLE_SLOTS; ++j) {
        if (key[j] < tau) key[j] = 0;
        w[j] = key[j] ? weight(key_f32(key[j]), xmax) : 0ull;
        Z += w[j];
    }
    uint32_t theta = 0;
    if (c.p < 1.0f) {
        Z = block_sum_u64(Z, sh.bs);
        const llima_u128 PZ = (llima_u128)frac32(c.p) * Z;
        theta = fin_topp_desc(key, w, PZ, tau, kmax, sh, buf);
    }
    const uint64_t mthr = c.m > 0.0f ? frac32(c.m) << 4 : 0;
    uint32_t fmask = 0;
    uint64_t Zf = 0;
#pragma unroll
    for (int j = 0; j < SAMPLE_SLOTS; ++j) {
        const bool f = key[j] && key[j] >= theta && w[j] >= mthr;
        fmask |= f ? (1u << j) : 0u;
        w[j] = f ? w[j] : 0ull;
        Zf += w[j];
    }
    Zf = block_sum_u64(Zf, sh.bs);
    int32_t tok = -1;
    float prob = 0.0f;
    if (Zf > 0) {
        const uint64_t target = (uint64_t)(((llima_u128)uniform32(P.uniforms[row]) * Zf) >> 32);
        uint64_t wtok = 0;
        tok = (int32_t)fin_draw_asc(id, w, target, (uint32_t)P.V, &wtok, sh, buf);
        prob = (float)((double)wtok / (double)Zf);
    }
    if (threadIdx.x == 0) write_result(P, row, tok, prob);
    if (P.out_keep)
        write_keep(P, row, [&](auto set) {
#pragma unroll
            for (int j = 0; j < SAMPLE_SLOTS; ++j)
                if ((fmask >> j) & 1u) set(id[j]);
        });
}

// The row from the sweep's candidates; false when it needs the full-row path.
__device__ __forceinline__ bool fin_fast(const SampleParams& P, int row, const RowCfg& c,
                                         FinishShared& sh) {
    constexpr int HPL = 2;                           // chunk headers per lane (S <= 128)
    const uint32_t t = threadIdx.x, lane = lane_id(), wave = wave_id();
    const int S = P.S;
    if (S > 64 * HPL) return false;
    const ChunkHdr* hdr = P.hdr + (size_t)row * S;

    // ---- 1. loads, all issued before any is used: this thread's candidate
    //         slots (the first `pre` slots of every chunk, whatever their
    //         counts), then every header, read by every wave (lane l: chunks l
    //         and l + 64)
    uint64_t q[SAMPLE_SLOTS];
    const uint64_t* crow = P.cand + ((size_t)row * S << P.ls);
    const uint32_t pmask = (1u << P.lp) - 1u;
#pragma unroll
    for (int j = 0; j < SAMPLE_SLOTS; ++j) {
        const uint32_t f = t + (uint32_t)j * LLIMA_WG;   // chunk f >> lp, slot f & pmask
        const uint32_t ch = f >> P.lp;
        q[j] = crow[ch < (uint32_t)S ? (ch << P.ls) + (f & pmask) : 0u];
    }
    llima_u32x4 ha[HPL], hb[HPL], hc[HPL];
#pragma unroll
    for (int i = 0; i < HPL; ++i) {
        const int ch = (int)lane + 64 * i;
        const llima_u32x4* hp = (const llima_u32x4*)(hdr + (ch < S ? ch : 0));
        ha[i] = hp[0];
        hb[i] = hp[1];
        hc[i] = hp[2];
    }
    sh.hcnt[0][t] = 0; sh.hcnt[1][t] = 0;
    sh.hmass[0][t] = 0; sh.hmass[1][t] = 0;

    // ---- 2. header summary, computed by every wave (no barrier)
    uint32_t fl = 0, bstar = 0, n = 0, spill = 0;
    uint64_t greedy = 0;
#pragma unroll
    for (int i = 0; i < HPL; ++i) {
        if (i * 64 < S) {
            const int ch = (int)lane + 64 * i;
            if (ch < S) {
                fl |= ha[i].y;
                if (ha[i].y & HDR_FILTERED) bstar = ha[i].z > bstar ? ha[i].z : bstar;
                n += ha[i].x;
                spill |= ha[i].x > (1u << P.lp) ? 1u : 0u;
                const uint64_t g = ((uint64_t)hb[i].y << 32) | hb[i].x;
                greedy = g > greedy ? g : greedy;
                sh.wcnt[wave][ch] = ha[i].x;
            }
        }
    }
    fl = wave_or_u32(fl);
    bstar = wave_max_u32(bstar);
    n = wave_sum_u32(n);
    spill = wave_max_u32(spill);
    greedy = wave_max_u64(greedy);

    if (c.greedy) {
        if (fl & HDR_OVERFLOW) return false;
        const bool ok = (uint32_t)(greedy >> 32) > LLIMA_KEY_NEG_INF;
        const uint32_t tok = ok ? ~(uint32_t)greedy : 0xFFFFFFFFu;
        if (t == 0) write_result(P, row, ok ? (int32_t)tok : -1, ok ? 1.0f : 0.0f);
        if (P.out_keep)
            write_keep(P, row, [&](auto set) { if (t == 0 && ok) set(tok); });
        return true;
    }
    if ((fl & HDR_OVERFLOW) || n > SAMPLE_FIN_CAP) return false;

    // ---- 3. bound on the top-k threshold: the largest chunk bound (that chunk
    //         has k values at or above it), or the k-th largest of the lane
    //         maxima in the headers (distinct values of the row), whichever is larger
    uint32_t gthr = bstar;
    if (c.k > 0 && 8 * S >= c.k) {
        constexpr int NV = 8 * HPL;
        uint32_t hv[NV];
        uint32_t vmax = 0, vmin = 0xFFFFFFFFu, nz = 0;
#pragma unroll
        for (int i = 0; i < HPL; ++i) {
            const bool in = (int)lane + 64 * i < S;
            const uint32_t a[8] = {hb[i].x, hb[i].y, hb[i].z, hb[i].w,
                                   hc[i].x, hc[i].y, hc[i].z, hc[i].w};
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const uint32_t x = in ? a[u] : 0u;
                hv[i * 8 + u] = x;
                vmax = x > vmax ? x : vmax;
                vmin = x && x < vmin ? x : vmin;
                nz += x ? 1u : 0u;
            }
        }
        vmax = wave_max_u32(vmax);
        vmin = wave_min_u32(vmin);
        nz = wave_sum_u32(nz);
        if (nz >= (uint32_t)c.k) {
            // The lower edge of the histogram bin holding the k-th largest
            // value (8-bit bins below the bits all the values share), with a
            // histogram of its own in every wave: no barrier.
            const uint32_t diff = vmax ^ vmin;
            uint32_t tb = vmax;
            if (diff) {
                const int top = 31 - __builtin_clz(diff);
                const int lo = top - 7 > 0 ? top - 7 : 0;
                const uint32_t bmask = (2u << (top - lo)) - 1u;
                const uint32_t prefix = top == 31 ? 0u : (vmax & ~((2u << top) - 1u));
                uint32_t* bh = sh.bh[wave];
                *(llima_u32x4*)(bh + 4 * lane) = llima_u32x4{0u, 0u, 0u, 0u};
#pragma unroll
                for (int u = 0; u < NV; ++u)
                    if (hv[u]) atomicAdd(&bh[(hv[u] >> lo) & bmask], 1u);
                // lane l holds bins 255 - 4l (top) down to 252 - 4l
                const llima_u32x4 b4 = *(const llima_u32x4*)(bh + 252 - 4 * lane);
                const uint32_t s4 = b4.x + b4.y + b4.z + b4.w;
                const uint32_t inc = wave_incl_scan_u32(s4);   // values in bins >= 252 - 4l
                const uint64_t hit = ballot(inc >= (uint32_t)c.k);
                const uint32_t L = (uint32_t)__builtin_ffsll((long long)hit) - 1u;
                uint32_t acc = readlane(inc - s4, L);
                const uint32_t q3 = readlane(b4.w, L), q2 = readlane(b4.z, L), q1 = readlane(b4.y, L);
                uint32_t bin = 252u - 4u * L;
                if (acc + q3 >= (uint32_t)c.k) bin = 255u - 4u * L;
                else if (acc + q3 + q2 >= (uint32_t)c.k) bin = 254u - 4u * L;
                else if (acc + q3 + q2 + q1 >= (uint32_t)c.k) bin = 253u - 4u * L;
                tb = prefix | (bin << lo);
            }
            gthr = tb > gthr ? tb : gthr;
        }
    }
    float gr = -__FLT_MAX__;
    if (gthr) {
        const float m = lower_bound_margin(key_f32(gthr));
        gr = m > -__FLT_MAX__ ? m : -__FLT_MAX__;
    }

    // ---- 4. slots f < lim hold a candidate or the padding; a chunk with more
    //         than `pre` candidates sends every candidate of the row through
    //         LDS in chunk order
    uint32_t lim = (uint32_t)S << P.lp;
    if (spill) {
        lim = SAMPLE_FIN_CAP;
        const uint32_t cn = (int)t < S ? sh.wcnt[wave][t] : 0u;
        const uint32_t inc = wave_incl_scan_u32(cn);
        const uint32_t off = (uint32_t)wg_prefix_u64(inc, cn, sh.r64[0]);
        if ((int)t < S) sh.coff[t] = off;
        __syncthreads();
        for (int ch = (int)wave; ch < S; ch += LLIMA_WAVES) {
            const uint32_t o = sh.coff[ch];
            const uint32_t m = sh.wcnt[wave][ch];
            const uint64_t* src = crow + ((size_t)ch << P.ls);
            for (uint32_t i = lane; i < m; i += 64) sh.u.cbuf[o + i] = src[i];
        }
        __syncthreads();
#pragma unroll
        for (int j = 0; j < SAMPLE_SLOTS; ++j) {
            const uint32_t f = t + (uint32_t)j * LLIMA_WG;
            q[j] = f < n ? sh.u.cbuf[f] : SAMPLE_SENTINEL;
        }
    }

    // ---- 5. candidates at or above the bound, staged per wave
    uint32_t o = 0;
#pragma unroll
    for (int j = 0; j < SAMPLE_SLOTS; ++j) {
        const bool pass = t + (uint32_t)j * LLIMA_WG < lim &&
                          __uint_as_float((uint32_t)(q[j] >> 32)) >= gr;
        const uint64_t m = ballot(pass);
        if (m) {
            const uint32_t s2 = mbcnt_add(m, o);
            if (pass && s2 < SAMPLE_SMALL) sh.stage[wave][s2] = q[j];
            o += (uint32_t)__popcll(m);
        }
    }
    if (lane == 0) sh.r32[0][wave] = o;
    __syncthreads();
    uint32_t wc[LLIMA_WAVES], nk0 = 0;
#pragma unroll
    for (int w = 0; w < LLIMA_WAVES; ++w) { wc[w] = sh.r32[0][w]; nk0 += wc[w]; }

    if (nk0 <= SAMPLE_SMALL) {
        // ---- 6a. every wave holds all survivors, one per lane
        uint32_t key = 0, id = 0;
        if (lane < nk0) {
            uint32_t w = 0, idx = lane;
            while (w < LLIMA_WAVES - 1 && idx >= wc[w]) { idx -= wc[w]; ++w; }
            const uint64_t qq = sh.stage[w][idx];
            const uint32_t k = f32_key(__uint_as_float((uint32_t)(qq >> 32)) / c.T);
            key = k > LLIMA_KEY_NEG_INF ? k : 0u;
            id = (uint32_t)qq;
        }
        const uint32_t nfin = (uint32_t)__popcll(ballot(key != 0));
        if (nfin == 0) {
            if (gthr) return false;
            if (t == 0) write_result(P, row, -1, 0.0f);
            if (P.out_keep) write_keep(P, row, [&](auto) {});
            return true;
        }
        const uint32_t kmax = wave_max_u32(key);
        const uint32_t kmin = wave_min_u32(key ? key : 0xFFFFFFFFu);
        return fin_small(P, row, c, key, id, nk0, nfin, kmin, kmax, gthr, sh);
    }

    // ---- 6b. many survivors: keys in registers, radix selects
    uint32_t key[SAMPLE_SLOTS], id[SAMPLE_SLOTS];
    uint32_t kmax = 0, nkmin = 0, nkeep = 0;
#pragma unroll
    for (int j = 0; j < SAMPLE_SLOTS; ++j) {
        const float x = __uint_as_float((uint32_t)(q[j] >> 32));
        const uint32_t k = f32_key(x / c.T);
        const bool keep = t + (uint32_t)j * LLIMA_WG < lim && x >= gr && k > LLIMA_KEY_NEG_INF;
        key[j] = keep ? k : 0u;
        id[j] = (uint32_t)q[j];
        nkeep += keep ? 1u : 0u;
        kmax = keep && k > kmax ? k : kmax;
        nkmin = keep && ~k > nkmin ? ~k : nkmin;
    }
    {
        const uint32_t a = wave_max_u32(kmax), b = wave_max_u32(nkmin), s2 = wave_sum_u32(nkeep);
        if (lane == 0) { sh.r32[4][wave] = a; sh.r32[5][wave] = b; sh.r32[6][wave] = s2; }
        __syncthreads();
        kmax = 0; nkmin = 0; nkeep = 0;
#pragma unroll
        for (int w = 0; w < LLIMA_WAVES; ++w) {
            kmax = sh.r32[4][w] > kmax ? sh.r32[4][w] : kmax;
            nkmin = sh.r32[5][w] > nkmin ? sh.r32[5][w] : nkmin;
            nkeep += sh.r32[6][w];
        }
    }
    if (nkeep == 0) return false;                    // cannot happen with nk0 > 64 finite
    const uint32_t kmin = ~nkmin;
    int buf = 0;
    uint32_t tau = kmin;
    if (c.k > 0 && (uint32_t)c.k < nkeep) tau = fin_kth_desc(key, (uint32_t)c.k, kmin, kmax, sh, buf);
    else if (c.k > 0 && (uint32_t)c.k > nkeep && gthr) return false;
    if (gthr && !(lower_bound_margin(key_f32(gthr)) / c.T < key_f32(tau))) return false;
    fin_large(P, row, c, key, id, tau, kmax, sh, buf);
    return true;
}

template <typename TL>
__global__ __launch_bounds__(LLIMA_WG) void sample_finish(SampleParams P) {
    __shared__ FinishShared sh;
    const int row = blockIdx.x;
    const RowCfg c = load_cfg(P, row);
    if (!fin_fast(P, row, c, sh)) finish_full_row<TL>(P, row, c, sh);
}

// ================================================================== host side
static size_t al256(size_t x) { return (x + 255) & ~(size_t)255; }
static int max_chunks(int V) { return (V + SAMPLE_MIN_CHUNK - 1) / SAMPLE_MIN_CHUNK; }

template <typename TL, int E>
static void launch_sweep(const SampleParams& P, hipStream_t st) {
    const dim3 g((uint32_t)P.B * (uint32_t)P.S), b(LLIMA_WG);
    if (P.bitmask) {
        if (P.vec_ok) hipLaunchKernelGGL((sample_sweep<TL, E, true, true>), g, b, 0, st, P);
        else hipLaunchKernelGGL((sample_sweep<TL, E, false, true>), g, b, 0, st, P);
    } else {
        if (P.vec_ok) hipLaunchKernelGGL((sample_sweep<TL, E, true, false>), g, b, 0, st, P);
        else hipLaunchKernelGGL((sample_sweep<TL, E, false, false>), g, b, 0, st, P);
    }
}

}  // namespace llima

using namespace llima;

extern "C" size_t llima_sample_workspace_bytes(int32_t B, int32_t V, int32_t dtype) {
    (void)dtype;
    if (B <= 0 || V <= 0) return 0;
    return al256((size_t)B * max_chunks(V) * sizeof(ChunkHdr)) +
           (size_t)B * SAMPLE_ROW_CAND * sizeof(uint64_t);
}

extern "C" int llima_sample(const void* logits, int32_t dtype, int32_t B, int32_t V,
                            int64_t row_stride, const int32_t* history,
                            const int32_t* history_len, int32_t H_max, const uint32_t* bitmask,
                            const float* uniforms, const llima_sampler_config* cfg,
                            int32_t* out_ids, float* out_probs, uint32_t* out_keep,
                            void* workspace, size_t workspace_bytes, void* stream) {
    if (!logits || !cfg || !out_ids || !uniforms) return LLIMA_E_INVAL;
    if (dtype != LLIMA_F32 && dtype != LLIMA_BF16) return LLIMA_E_INVAL;
    if (B < 0 || V <= 0 || V > (1 << 24) || row_stride < V) return LLIMA_E_INVAL;
    if (history && (H_max < 0 || H_max >= 65536)) return LLIMA_E_INVAL;
    if (B == 0) return LLIMA_OK;
    if (!workspace || workspace_bytes < llima_sample_workspace_bytes(B, V, dtype))
        return LLIMA_E_WORKSPACE;
    if (!cfg->greedy && !cfg->temperature_rows) {
        if (!(cfg->temperature >= 0.0f) || __builtin_isinf(cfg->temperature)) return LLIMA_E_INVAL;
    }
    if (!cfg->repetition_penalty_rows &&
        (!(cfg->repetition_penalty > 0.0f) || __builtin_isinf(cfg->repetition_penalty)))
        return LLIMA_E_INVAL;
    if (!__builtin_isfinite(cfg->presence_penalty) || !__builtin_isfinite(cfg->frequency_penalty))
        return LLIMA_E_INVAL;

    SampleParams P;
    P.logits = logits;
    P.row_stride = row_stride;
    P.hist = history;
    P.hist_len = history_len;
    P.bitmask = bitmask;
    P.uniforms = uniforms;
    P.cfg = *cfg;
    P.out_ids = out_ids;
    P.out_probs = out_probs;
    P.out_keep = out_keep;
    P.B = B;
    P.V = V;
    P.H_max = history ? H_max : 0;
    const size_t esz = dtype == LLIMA_F32 ? 4 : 2;
    P.vec_ok = ((uintptr_t)logits % 16 == 0) && ((row_stride * (int64_t)esz) % 16 == 0) &&
               (V % (int32_t)(16 / esz) == 0);
    // 16 KB of logits per workgroup: 4096 fp32 or 8192 bf16 values.
    const int chunk = dtype == LLIMA_F32 ? 4096 : 8192;
    P.S = (V + chunk - 1) / chunk;
    // powers of two: share = slots per chunk, pre = slots per chunk the finish
    // reads up front (S * pre <= 4096 = one slot per finishing thread x 16)
    auto floor_log2 = [](int x) { int l = 0; while ((2 << l) <= x) ++l; return l; };
    P.ls = floor_log2(SAMPLE_ROW_CAND / P.S);
    P.lp = floor_log2(SAMPLE_FIN_CAP / P.S);
    P.hdr = (ChunkHdr*)workspace;
    P.cand = (uint64_t*)((char*)workspace + al256((size_t)B * max_chunks(V) * sizeof(ChunkHdr)));
    hipStream_t st = (hipStream_t)stream;
    if (dtype == LLIMA_F32) {
        launch_sweep<float, 16>(P, st);
        hipLaunchKernelGGL(sample_finish<float>, dim3(B), dim3(LLIMA_WG), 0, st, P);
    } else {
        launch_sweep<uint16_t, 32>(P, st);
        hipLaunchKernelGGL(sample_finish<uint16_t>, dim3(B), dim3(LLIMA_WG), 0, st, P);
    }
    return hipGetLastError() == hipSuccess ? LLIMA_OK : LLIMA_E_HIP;
}
