// sample.hip -- fused penalty / temperature / mask / top-k / top-p / min-p /
// inverse-CDF sampling over [B, V] logits rows on MI355X (gfx950).
//
// Two launches per step, with no atomics or fences between workgroups (on
// this part, device-scope cache maintenance and same-address atomics cost far
// more than the whole sweep):
//
// sample_sweep: B x S workgroups; workgroup (row, chunk) streams a 256*E chunk
//   of its row from HBM with 16-byte loads, issued before anything else, and
//   keeps it in registers.  While the loads are in flight it counts the row's
//   history ids that fall in the chunk in an LDS table (packed u16 counts);
//   distinct ids become "exceptions" whose penalised value is computed apart, so
//   the per-element work is a count != 0 test (no division in the stream).
//   Masked (packed-uint32 grammar bitmask, LSB first), NaN and history values
//   become -inf.  A lower bound t of the chunk's k-th largest value comes from
//   the lane maxima (wavefront bitonic sort, min over the 4 waves) and every
//   value >= t - |t| 2^-20 is written, with its id, to the chunk's own slot of
//   the workspace together with a small header.
//
// sample_finish: one workgroup per row gathers the candidates into LDS, divides
//   them by the temperature, proves that the bound could not have dropped a
//   member of the top-k set (else falls back), and runs three radix selects over
//   LDS histograms on register-resident candidates: top-k threshold (count),
//   top-p threshold (fixed-point mass) and the draw (mass by ascending id).
//   Rows that the candidates cannot serve (overflow, k beyond the fast path,
//   top-k disabled without a mask, degenerate temperatures) are finished by the
//   same workgroup with a full-row multi-pass version of the same selects.
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
#define SAMPLE_PRECAP 1024                         // candidates staged in LDS per chunk
#define SAMPLE_EXC_CAP 512                         // distinct history ids per chunk
#define SAMPLE_MIN_CHUNK 2048                      // 256 threads x E = 8
#define SAMPLE_SEG 8192                            // full-row path segment
#define SAMPLE_HBATCH 8                            // history ids per thread loaded up front

#define HDR_OVERFLOW 1u
#define HDR_FILTERED 2u

// Written by every sweep workgroup (no state survives a call).
struct ChunkHdr {
    uint32_t count;      // candidates in this chunk's slot
    uint32_t flags;      // HDR_*
    uint32_t bound;      // key of the pre-filter bound (when FILTERED)
    uint32_t pad;
    uint64_t greedy;     // (key << 32 | ~index) of the chunk maximum
    uint64_t pad2;
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
};

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
    if (P.hist) {
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
// counts.  With exc_id, lists the distinct ids (first occurrence wins the slot)
// with their raw logits, fetched here so that the load overlaps the scan.
template <typename TL>
__device__ __forceinline__ void count_history(const SampleParams& P, int row, int hlen, int lo,
                                              int hi, uint32_t* table, int nwords,
                                              int32_t* exc_id, float* exc_raw, uint32_t* n_exc,
                                              const TL* rowp) {
    for (int i = threadIdx.x; i < nwords; i += LLIMA_WG) table[i] = 0;
    __syncthreads();
    const int32_t* h = P.hist + (size_t)row * P.H_max;
    for (int j = threadIdx.x; j < hlen; j += LLIMA_WG) {
        const int32_t id = h[j];
        if (id >= lo && id < hi) {
            const uint32_t off = (uint32_t)(id - lo);
            const uint32_t sh16 = (off & 1u) * 16u;
            const uint32_t old = atomicAdd(&table[off >> 1], 1u << sh16);
            if (exc_id && ((old >> sh16) & 0xFFFFu) == 0) {
                const uint32_t slot = atomicAdd(n_exc, 1u);
                if (slot < SAMPLE_EXC_CAP) {
                    exc_id[slot] = id;
                    exc_raw[slot] = load_one<TL>(rowp, id);
                }
            }
        }
    }
    __syncthreads();
}

// ================================================================== sweep
template <int CHUNK>
struct SweepShared {
    uint32_t cnt[CHUNK / 2];
    int32_t exc_id[SAMPLE_EXC_CAP];
    float exc_val[SAMPLE_EXC_CAP];           // raw, then penalised value
    uint64_t pre[SAMPLE_PRECAP];
    uint32_t n_exc, n_pre;
    uint32_t wave_bound[LLIMA_WAVES];
    BlockScratch bs;
};

// VEC: rows are 16-byte aligned and V is a multiple of the values per load, so
// every chunk (also a row's partial last one) is read with 16-byte loads from
// clamped, always-valid addresses and the out-of-row values masked in registers.
template <typename TL, int E, bool VEC>
__global__ __launch_bounds__(LLIMA_WG) void sample_sweep(SampleParams P) {
    constexpr int EPL = 16 / sizeof(TL);       // values per 16-byte load
    constexpr int NL = E / EPL;                // loads per thread
    constexpr int CHUNK = LLIMA_WG * E;
    __shared__ SweepShared<CHUNK> sh;
    const float NEG_INF = -__builtin_inff();

    uint32_t row, chunk;
    map_row_chunk(blockIdx.x, (uint32_t)P.B, (uint32_t)P.S, &row, &chunk);
    if (row >= (uint32_t)P.B) return;
    const TL* rowp = (const TL*)P.logits + (size_t)row * P.row_stride;
    const int V = P.V;
    const int c0 = (int)chunk * CHUNK;
    const int c1 = c0 + CHUNK < V ? c0 + CHUNK : V;
    const int nw = (V + 31) >> 5;
    const uint32_t* mrow = P.bitmask ? P.bitmask + (size_t)row * nw : nullptr;

    const RowCfg c = load_cfg(P, row);
    const int32_t* hrow = P.hist + (size_t)row * P.H_max;

    // ---- 0. clear the chunk's history table
    if (c.pen)
        for (int i = threadIdx.x; i < CHUNK / 2; i += LLIMA_WG) sh.cnt[i] = 0;
    if (threadIdx.x == 0) { sh.n_exc = 0; sh.n_pre = 0; }
    __syncthreads();

    // ---- 1. issue the loads, oldest first in the order they are consumed:
    //         mask words, the first batch of history ids, then the chunk itself.
    //         Every address is valid; nothing waits until all are in flight.
    uint32_t mword[NL];
    if (mrow) {
#pragma unroll
        for (int j = 0; j < NL; ++j) {
            const int i0 = c0 + j * (LLIMA_WG * EPL) + (int)threadIdx.x * EPL;
            mword[j] = mrow[(i0 < V ? i0 : V - 1) >> 5];
        }
    } else {
#pragma unroll
        for (int j = 0; j < NL; ++j) mword[j] = 0xFFFFFFFFu;
    }
    // history ids: whether slot b holds a real id (j < hlen) is decided only
    // when it is counted
    int32_t hid[SAMPLE_HBATCH];
    if (c.pen) {
#pragma unroll
        for (int b = 0; b < SAMPLE_HBATCH; ++b) {
            const int j = (int)threadIdx.x + b * LLIMA_WG;
            hid[b] = hrow[j < c.hlen ? j : 0];
        }
    }
    llima_u32x4 raw[NL];
#pragma unroll
    for (int j = 0; j < NL; ++j) {
        const int i0 = c0 + j * (LLIMA_WG * EPL) + (int)threadIdx.x * EPL;
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

    // ---- 2. while the chunk is in flight: count the history ids of the chunk
    if (c.pen) {
#pragma unroll
        for (int b = 0; b < SAMPLE_HBATCH; ++b) {
            const int32_t id = hid[b];
            if ((int)threadIdx.x + b * LLIMA_WG < c.hlen && id >= c0 && id < c1) {
                const uint32_t off = (uint32_t)(id - c0);
                atomicAdd(&sh.cnt[off >> 1], 1u << ((off & 1u) * 16u));
            }
        }
        for (int j = (int)threadIdx.x + SAMPLE_HBATCH * LLIMA_WG; j < c.hlen; j += LLIMA_WG) {
            const int32_t id = hrow[j];
            if (id >= c0 && id < c1) {
                const uint32_t off = (uint32_t)(id - c0);
                atomicAdd(&sh.cnt[off >> 1], 1u << ((off & 1u) * 16u));
            }
        }
    }
    __syncthreads();

    // ---- 3. values after mask / NaN; history values leave the stream as
    //         exceptions (owner thread appends id and raw value), so that the
    //         stream needs no division
    float v[E];
#pragma unroll
    for (int j = 0; j < NL; ++j) {
        const int i0 = c0 + j * (LLIMA_WG * EPL) + (int)threadIdx.x * EPL;
        const uint32_t mb = mword[j] >> (i0 & 31);
        float t[EPL];
        const uint32_t w4[4] = {raw[j].x, raw[j].y, raw[j].z, raw[j].w};
        if constexpr (sizeof(TL) == 4) {
#pragma unroll
            for (int e = 0; e < 4; ++e) t[e] = __uint_as_float(w4[e]);
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                t[2 * e] = __uint_as_float(w4[e] << 16);
                t[2 * e + 1] = __uint_as_float(w4[e] & 0xFFFF0000u);
            }
        }
        uint32_t cw[EPL / 2];
#pragma unroll
        for (int e = 0; e < EPL / 2; ++e) cw[e] = 0;
        if (c.pen && i0 < c1) {
            const uint32_t off = (uint32_t)(i0 - c0);
#pragma unroll
            for (int e = 0; e < EPL / 2; ++e) cw[e] = sh.cnt[(off >> 1) + e];
        }
#pragma unroll
        for (int e = 0; e < EPL; ++e) {
            float x = t[e];
            if (x != x || !((mb >> e) & 1u) || i0 + e >= c1) x = NEG_INF;
            const uint32_t cnt = (cw[e >> 1] >> ((e & 1) * 16)) & 0xFFFFu;
            if (cnt) {
                const uint32_t slot = atomicAdd(&sh.n_exc, 1u);
                if (slot < SAMPLE_EXC_CAP) {
                    sh.exc_id[slot] = i0 + e;
                    sh.exc_val[slot] = x;
                }
                x = NEG_INF;
            }
            v[j * EPL + e] = x;
        }
    }
    __syncthreads();

    // ---- 4. exceptions: distinct history ids of this chunk, penalised exactly
    const uint32_t n_exc = c.pen ? sh.n_exc : 0u;
    const uint32_t n_exc_c = n_exc < SAMPLE_EXC_CAP ? n_exc : SAMPLE_EXC_CAP;
    uint32_t flags = n_exc > SAMPLE_EXC_CAP ? HDR_OVERFLOW : 0u;
    float tmax = NEG_INF;
    for (uint32_t j = threadIdx.x; j < n_exc_c; j += LLIMA_WG) {
        const int id = sh.exc_id[j];
        const float l = penalize(sh.exc_val[j], table_count(sh.cnt, (uint32_t)(id - c0)), c);
        sh.exc_val[j] = l;
        tmax = l > tmax ? l : tmax;
    }

    ChunkHdr* hdr = P.hdr + (size_t)row * P.S + chunk;
    if (c.greedy) {
        // ---- argmax: first index of the maximum (values visited in index order)
        float best = NEG_INF;
        uint32_t bidx = 0xFFFFFFFFu;
#pragma unroll
        for (int j = 0; j < NL; ++j) {
            const int i0 = c0 + j * (LLIMA_WG * EPL) + (int)threadIdx.x * EPL;
#pragma unroll
            for (int e = 0; e < EPL; ++e)
                if (v[j * EPL + e] > best) { best = v[j * EPL + e]; bidx = (uint32_t)(i0 + e); }
        }
        uint64_t kb = best > NEG_INF ? (((uint64_t)f32_key(best) << 32) | (uint64_t)(~bidx)) : 0ull;
        for (uint32_t j = threadIdx.x; j < n_exc_c; j += LLIMA_WG) {
            const float x = sh.exc_val[j];
            const uint64_t kk = x > NEG_INF ? (((uint64_t)f32_key(x) << 32) |
                                               (uint64_t)(~(uint32_t)sh.exc_id[j])) : 0ull;
            kb = kk > kb ? kk : kb;
        }
        kb = block_max_u64(kb, sh.bs);
        if (threadIdx.x == 0) {
            hdr->count = 0;
            hdr->flags = flags;
            hdr->bound = 0;
            hdr->greedy = kb;
        }
        return;
    }

    // ---- 5. pre-filter bound from lane maxima: every wave has >= r lanes whose
    //         maximum is >= its bound, so the chunk has >= 4r >= k values >= t
    float g = NEG_INF;
    if (c.k > 0 && c.k <= 4 * 64) {
#pragma unroll
        for (int e = 0; e < E; ++e) tmax = v[e] > tmax ? v[e] : tmax;
        const uint32_t r = (uint32_t)(c.k + 3) >> 2;          // ceil(k/4) <= 64
        const uint32_t sorted = wave_sort_desc(f32_key(tmax));
        const uint32_t wb = __shfl(sorted, (int)r - 1, 64);
        if (lane_id() == 0) sh.wave_bound[threadIdx.x >> 6] = wb;
        __syncthreads();
        uint32_t tb = sh.wave_bound[0];
#pragma unroll
        for (int w = 1; w < LLIMA_WAVES; ++w) tb = sh.wave_bound[w] < tb ? sh.wave_bound[w] : tb;
        if (tb > LLIMA_KEY_NEG_INF) g = lower_bound_margin(key_f32(tb));
    }
    // ---- 6. stage the values >= g in LDS
#pragma unroll
    for (int j = 0; j < NL; ++j) {
        const int i0 = c0 + j * (LLIMA_WG * EPL) + (int)threadIdx.x * EPL;
#pragma unroll
        for (int e = 0; e < EPL; ++e) {
            const float x = v[j * EPL + e];
            if (x > NEG_INF && x >= g) {
                const uint32_t s2 = atomicAdd(&sh.n_pre, 1u);
                if (s2 < SAMPLE_PRECAP)
                    sh.pre[s2] = ((uint64_t)__float_as_uint(x) << 32) | (uint32_t)(i0 + e);
            }
        }
    }
    for (uint32_t j = threadIdx.x; j < n_exc_c; j += LLIMA_WG) {
        const float x = sh.exc_val[j];
        if (x > NEG_INF && x >= g) {
            const uint32_t s2 = atomicAdd(&sh.n_pre, 1u);
            if (s2 < SAMPLE_PRECAP)
                sh.pre[s2] = ((uint64_t)__float_as_uint(x) << 32) | (uint32_t)sh.exc_id[j];
        }
    }
    __syncthreads();
    const uint32_t n_pre = sh.n_pre;
    if (n_pre > SAMPLE_PRECAP) flags |= HDR_OVERFLOW;
    const uint32_t n_st = n_pre < SAMPLE_PRECAP ? n_pre : SAMPLE_PRECAP;

    // ---- 7. the chunk's exact k-th largest value tau_c among the staged ones
    //         (they hold every value >= g, hence the chunk's top k) by rank counting
    float gout = NEG_INF;
    uint32_t bound = 0;
    if (c.k > 0 && n_st >= (uint32_t)c.k && !(flags & HDR_OVERFLOW)) {
        uint32_t kt = 0;                                      // key of a tau_c candidate
        for (uint32_t i = threadIdx.x; i < n_st; i += LLIMA_WG) {
            const float xi = __uint_as_float((uint32_t)(sh.pre[i] >> 32));
            uint32_t ge = 0;
            for (uint32_t jj = 0; jj < n_st; ++jj)
                ge += __uint_as_float((uint32_t)(sh.pre[jj] >> 32)) >= xi;
            if (ge >= (uint32_t)c.k) { const uint32_t kk = f32_key(xi); kt = kk > kt ? kk : kt; }
        }
        bound = block_max_u32(kt, sh.bs);
        gout = lower_bound_margin(key_f32(bound));
        flags |= HDR_FILTERED;
    }
    // ---- 8. write the chunk's candidates (values >= gout) and its header
    if (threadIdx.x == 0) sh.n_exc = 0;                      // reused as the output count
    __syncthreads();
    const uint32_t cap = (uint32_t)P.share;
    uint64_t* dst = P.cand + ((size_t)row * P.S + chunk) * P.share;
    if (!(flags & HDR_OVERFLOW)) {
        for (uint32_t i = threadIdx.x; i < n_st; i += LLIMA_WG) {
            const uint64_t q = sh.pre[i];
            if (__uint_as_float((uint32_t)(q >> 32)) >= gout) {
                const uint32_t o = atomicAdd(&sh.n_exc, 1u);
                if (o < cap) dst[o] = q;
            }
        }
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t n_out = sh.n_exc;
        if (n_out > cap) { flags |= HDR_OVERFLOW; }
        if (flags & HDR_OVERFLOW) n_out = 0;
        hdr->count = n_out;
        hdr->flags = flags;
        hdr->bound = bound;
        hdr->greedy = 0;
    }
}

// ================================================================== finish
#define SMALL_K 256                                // brute-force path: one element per thread

struct FinishShared {
    union {
        uint64_t cbuf[SAMPLE_FIN_CAP];         // gathered candidates
        uint32_t table[SAMPLE_SEG / 2];        // full-row path history counts
    } u;
    uint32_t hcnt[256];
    uint64_t hmass[256];
    uint32_t off[LLIMA_WG];
    uint8_t cid[SAMPLE_FIN_CAP];               // candidate position -> chunk (S <= 256)
    uint32_t kkey[SMALL_K], kid[SMALL_K];      // the top-k survivors (small path)
    uint64_t kw[SMALL_K], kwf[SMALL_K];
    uint32_t nk;
    uint32_t sel;
    uint64_t sel64, sel64b;
    BlockScratch bs;
};

// ------------------------------------------------------------------ radix selects
// Each select runs over a set of (key, id, weight) elements presented by a
// visitor; every thread visits its own elements.  Digits are 8 bits wide and
// start at the highest bit in which the visited keys differ (the bits above it
// are common to all of them), so the first histogram already spreads the keys.
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

// k-th largest key (with multiplicity) among visited elements, all of whose
// keys lie in [kmin, kmax].
template <class Visit>
__device__ __forceinline__ uint32_t select_kth_desc(Visit visit, uint32_t k, uint32_t kmin,
                                                    uint32_t kmax, FinishShared& sh) {
    Digits d = digits_init(kmin, kmax);
    uint32_t rem = k;
    while (d.top >= 0) {
        const int lo = d.top - 7 > 0 ? d.top - 7 : 0;
        const uint32_t bmask = (1u << (d.top - lo + 1)) - 1u;
        sh.hcnt[threadIdx.x] = 0;
        __syncthreads();
        const uint32_t prefix = d.prefix, pmask = d.pmask;
        visit([&](uint32_t key, uint32_t, uint64_t) {
            if ((key & pmask) == prefix) atomicAdd(&sh.hcnt[(key >> lo) & bmask], 1u);
        });
        __syncthreads();
        const uint32_t bin = 255u - threadIdx.x;          // thread 0 <-> top bin
        const uint32_t c = sh.hcnt[bin];
        uint32_t tot;
        const uint32_t above = block_excl_scan_u32(c, &tot, sh.bs);
        if (above < rem && above + c >= rem) { sh.sel = bin; sh.sel64 = rem - above; }
        __syncthreads();
        d.prefix |= sh.sel << lo;
        d.pmask |= bmask << lo;
        d.top = lo - 1;
        rem = (uint32_t)sh.sel64;
        __syncthreads();
    }
    return d.prefix;
}

// Top-p boundary: the smallest key theta such that an element with key theta has
// (mass strictly above) * 2^32 < PZ; when none has (PZ == 0) the top key.
template <class Visit>
__device__ __forceinline__ uint32_t select_topp_desc(Visit visit, llima_u128 PZ, uint32_t kmin,
                                                     uint32_t kmax, FinishShared& sh) {
    Digits d = digits_init(kmin, kmax);
    uint64_t acc = 0;
    while (d.top >= 0) {
        const int lo = d.top - 7 > 0 ? d.top - 7 : 0;
        const uint32_t bmask = (1u << (d.top - lo + 1)) - 1u;
        sh.hcnt[threadIdx.x] = 0;
        sh.hmass[threadIdx.x] = 0;
        __syncthreads();
        const uint32_t prefix = d.prefix, pmask = d.pmask;
        visit([&](uint32_t key, uint32_t, uint64_t w) {
            if ((key & pmask) == prefix) {
                const uint32_t b = (key >> lo) & bmask;
                atomicAdd(&sh.hcnt[b], 1u);
                if (w) atomicAdd((unsigned long long*)&sh.hmass[b], (unsigned long long)w);
            }
        });
        __syncthreads();
        const uint32_t t = threadIdx.x, bin = 255u - t;
        const uint32_t c = sh.hcnt[bin];
        uint64_t m = sh.hmass[bin], tot;
        const uint64_t above = acc + block_excl_scan_u64(m, &tot, sh.bs);
        const bool cond = c > 0 && (((llima_u128)above << 32) < PZ);
        // lowest qualifying bin = highest t; else the top non-empty bin = lowest t
        const uint32_t best_cond = block_max_u32(cond ? t + 1u : 0u, sh.bs);
        const uint32_t top_nonempty = 255u - block_max_u32(c > 0 ? 255u - t : 0u, sh.bs);
        const uint32_t sel_t = best_cond ? best_cond - 1u : top_nonempty;
        if (t == sel_t) { sh.sel = bin; sh.sel64 = above; }
        __syncthreads();
        d.prefix |= sh.sel << lo;
        d.pmask |= bmask << lo;
        d.top = lo - 1;
        acc = sh.sel64;
        __syncthreads();
    }
    return d.prefix;
}

// Draw: the smallest id whose ascending-id prefix mass exceeds target; also
// returns that element's weight.  Ids are < V <= 2^24.
template <class Visit>
__device__ __forceinline__ uint32_t select_draw_asc(Visit visit, uint64_t target, uint32_t V,
                                                    uint64_t* w_out, FinishShared& sh) {
    Digits d = digits_init(0u, V > 1 ? V - 1 : 1u);
    uint64_t acc = 0;
    while (d.top >= 0) {
        const int lo = d.top - 7 > 0 ? d.top - 7 : 0;
        const uint32_t bmask = (1u << (d.top - lo + 1)) - 1u;
        sh.hmass[threadIdx.x] = 0;
        __syncthreads();
        const uint32_t prefix = d.prefix, pmask = d.pmask;
        visit([&](uint32_t, uint32_t id, uint64_t w) {
            if (w && (id & pmask) == prefix)
                atomicAdd((unsigned long long*)&sh.hmass[(id >> lo) & bmask], (unsigned long long)w);
        });
        __syncthreads();
        const uint32_t bin = threadIdx.x;
        uint64_t m = sh.hmass[bin], tot;
        const uint64_t below = acc + block_excl_scan_u64(m, &tot, sh.bs);
        if (m > 0 && below <= target && target < below + m) {
            sh.sel = bin; sh.sel64 = below; sh.sel64b = m;
        }
        __syncthreads();
        d.prefix |= sh.sel << lo;
        d.pmask |= bmask << lo;
        d.top = lo - 1;
        acc = sh.sel64;
        *w_out = sh.sel64b;
        __syncthreads();
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
            if (c.pen)
                count_history<TL>(P, row, c.hlen, lo, hi, table, SAMPLE_SEG / 2, nullptr, nullptr,
                                  nullptr, rowp);
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
    auto visit_fin = [&](auto fn) {
        for_each_x([&](float x, uint32_t id) {
            const uint32_t k = f32_key(x);
            if (k > LLIMA_KEY_NEG_INF) fn(k, id, 0ull);
        });
    };
    uint32_t tau = LLIMA_KEY_NEG_INF + 1u;
    if (c.k > 0 && (uint32_t)c.k <= nfin) tau = select_kth_desc(visit_fin, (uint32_t)c.k, kmin, kmax, sh);
    const uint32_t kmin_k = tau > kmin ? tau : kmin;

    auto visit_k = [&](auto fn) {
        for_each_x([&](float x, uint32_t id) {
            const uint32_t k = f32_key(x);
            if (k >= tau) fn(k, id, weight(x, xmax));
        });
    };
    uint32_t theta = 0;
    if (c.p < 1.0f) {
        uint64_t Z = 0;
        visit_k([&](uint32_t, uint32_t, uint64_t w) { Z += w; });
        Z = block_sum_u64(Z, sh.bs);
        const llima_u128 PZ = (llima_u128)frac32(c.p) * Z;
        theta = select_topp_desc(visit_k, PZ, kmin_k, kmax, sh);
    }
    const uint64_t mthr = c.m > 0.0f ? frac32(c.m) << 4 : 0;
    auto visit_final = [&](auto fn) {
        visit_k([&](uint32_t k, uint32_t id, uint64_t w) {
            if (k >= theta && w >= mthr) fn(k, id, w);
        });
    };
    uint64_t Zf = 0;
    visit_final([&](uint32_t, uint32_t, uint64_t w) { Zf += w; });
    Zf = block_sum_u64(Zf, sh.bs);
    int32_t tok = -1;
    float prob = 0.0f;
    if (Zf > 0) {
        const uint64_t target = (uint64_t)(((llima_u128)uniform32(P.uniforms[row]) * Zf) >> 32);
        uint64_t wtok = 0;
        tok = (int32_t)select_draw_asc(visit_final, target, (uint32_t)V, &wtok, sh);
        prob = (float)((double)wtok / (double)Zf);
    }
    if (threadIdx.x == 0) write_result(P, row, tok, prob);
    if (P.out_keep)
        write_keep(P, row, [&](auto set) {
            visit_final([&](uint32_t, uint32_t id, uint64_t) { set(id); });
        });
}

// ------------------------------------------------------------------ fast path
// The survivors of top-k held one per thread (at most SMALL_K): top-p, min-p
// and the draw by direct sums over the LDS copy of the survivors.
__device__ __forceinline__ void finish_small(const SampleParams& P, int row, const RowCfg& c,
                                             uint32_t nk, uint32_t kmax, FinishShared& sh) {
    const uint32_t t = threadIdx.x;
    const bool mine = t < nk;
    const uint32_t key = mine ? sh.kkey[t] : 0u;
    const uint32_t id = mine ? sh.kid[t] : 0u;
    const uint64_t w = mine ? sh.kw[t] : 0ull;
    bool fin = mine;
    if (c.p < 1.0f) {
        const uint64_t Z = block_sum_u64(w, sh.bs);
        const llima_u128 PZ = (llima_u128)frac32(c.p) * Z;
        uint64_t above = 0;                       // mass strictly above this key
        for (uint32_t j = 0; j < nk; ++j) above += sh.kkey[j] > key ? sh.kw[j] : 0ull;
        fin = fin && ((((llima_u128)above << 32) < PZ) || key == kmax);
    }
    if (c.m > 0.0f) fin = fin && w >= (frac32(c.m) << 4);
    if (mine) sh.kwf[t] = fin ? w : 0ull;
    const uint64_t Zf = block_sum_u64(fin ? w : 0ull, sh.bs);   // barrier also publishes kwf
    int32_t tok = -1;
    if (Zf > 0 && fin && w > 0) {
        const uint64_t target = (uint64_t)(((llima_u128)uniform32(P.uniforms[row]) * Zf) >> 32);
        uint64_t upto = 0;                        // mass of final ids <= this id
        for (uint32_t j = 0; j < nk; ++j) upto += sh.kid[j] <= id ? sh.kwf[j] : 0ull;
        if (upto - w <= target && target < upto) {
            tok = (int32_t)id;
            write_result(P, row, tok, (float)((double)w / (double)Zf));
        }
    }
    if (Zf == 0 && t == 0) write_result(P, row, -1, 0.0f);
    if (P.out_keep)
        write_keep(P, row, [&](auto set) { if (fin) set(id); });
}

// Many survivors (top-k disabled, ties, k > SMALL_K): register-resident
// candidates (slot j of thread t is candidate t + 256 j) and radix selects.
__device__ __forceinline__ void finish_large(const SampleParams& P, int row, const RowCfg& c,
                                             uint32_t n, uint32_t tau, uint32_t kmax,
                                             FinishShared& sh) {
    uint32_t key[SAMPLE_SLOTS], id[SAMPLE_SLOTS];
    uint64_t w[SAMPLE_SLOTS];
    const float xmax = key_f32(kmax);
#pragma unroll
    for (int j = 0; j < SAMPLE_SLOTS; ++j) {
        const uint32_t s = threadIdx.x + j * LLIMA_WG;
        key[j] = 0; id[j] = 0; w[j] = 0;
        if (s < n) {
            const uint64_t q = sh.u.cbuf[s];
            key[j] = (uint32_t)(q >> 32);
            id[j] = (uint32_t)q;
            if (key[j] >= tau) w[j] = weight(key_f32(key[j]), xmax);
        }
    }
    auto visit_k = [&](auto fn) {
#pragma unroll
        for (int j = 0; j < SAMPLE_SLOTS; ++j)
            if (key[j] >= tau) fn(key[j], id[j], w[j]);
    };
    uint32_t theta = 0;
    if (c.p < 1.0f) {
        uint64_t Z = 0;
#pragma unroll
        for (int j = 0; j < SAMPLE_SLOTS; ++j) Z += w[j];
        Z = block_sum_u64(Z, sh.bs);
        const llima_u128 PZ = (llima_u128)frac32(c.p) * Z;
        theta = select_topp_desc(visit_k, PZ, tau, kmax, sh);
    }
    const uint64_t mthr = c.m > 0.0f ? frac32(c.m) << 4 : 0;
    auto visit_final = [&](auto fn) {
        visit_k([&](uint32_t k, uint32_t i, uint64_t ww) {
            if (k >= theta && ww >= mthr) fn(k, i, ww);
        });
    };
    uint64_t Zf = 0;
    visit_final([&](uint32_t, uint32_t, uint64_t ww) { Zf += ww; });
    Zf = block_sum_u64(Zf, sh.bs);
    int32_t tok = -1;
    float prob = 0.0f;
    if (Zf > 0) {
        const uint64_t target = (uint64_t)(((llima_u128)uniform32(P.uniforms[row]) * Zf) >> 32);
        uint64_t wtok = 0;
        tok = (int32_t)select_draw_asc(visit_final, target, (uint32_t)P.V, &wtok, sh);
        prob = (float)((double)wtok / (double)Zf);
    }
    if (threadIdx.x == 0) write_result(P, row, tok, prob);
    if (P.out_keep)
        write_keep(P, row, [&](auto set) {
            visit_final([&](uint32_t, uint32_t i, uint64_t) { set(i); });
        });
}

// Sampling from the gathered candidates (n of them in sh.u.cbuf).  Returns false
// when they cannot be proven to contain the kept set (the caller then runs the
// full-row path).
__device__ __forceinline__ bool finish_fast(const SampleParams& P, int row, const RowCfg& c,
                                            uint32_t n, uint32_t flags, uint32_t bound_key,
                                            FinishShared& sh) {
    // ---- values after the temperature, as keys, in place: (key << 32 | id)
    uint32_t kmax = 0, nkmin = 0, nfin = 0;
    for (uint32_t s = threadIdx.x; s < n; s += LLIMA_WG) {
        const uint64_t q = sh.u.cbuf[s];
        const uint32_t k = f32_key(__uint_as_float((uint32_t)(q >> 32)) / c.T);
        sh.u.cbuf[s] = ((uint64_t)k << 32) | (uint32_t)q;
        if (k > LLIMA_KEY_NEG_INF) {
            nfin++;
            kmax = k > kmax ? k : kmax;
            nkmin = ~k > nkmin ? ~k : nkmin;
        }
    }
    kmax = block_max_u32(kmax, sh.bs);
    const uint32_t kmin = ~block_max_u32(nkmin, sh.bs);
    nfin = block_sum_u32(nfin, sh.bs);
    if (nfin == 0) {
        // Every candidate is -inf after the temperature (or there are none).
        if (flags & HDR_FILTERED) return false;
        if (threadIdx.x == 0) write_result(P, row, -1, 0.0f);
        if (P.out_keep) write_keep(P, row, [&](auto) {});
        return true;
    }

    // ---- top-k threshold, then the proof that the pre-filter kept every member:
    // a value below a chunk's lowered bound g has x <= fl(g / T) < tau.
    uint32_t tau = LLIMA_KEY_NEG_INF + 1u;
    if (c.k > 0) {
        auto visit_fin = [&](auto fn) {
            for (uint32_t s = threadIdx.x; s < n; s += LLIMA_WG) {
                const uint32_t k = (uint32_t)(sh.u.cbuf[s] >> 32);
                if (k > LLIMA_KEY_NEG_INF) fn(k, 0u, 0ull);
            }
        };
        if ((uint32_t)c.k <= nfin) tau = select_kth_desc(visit_fin, (uint32_t)c.k, kmin, kmax, sh);
        else if (flags & HDR_FILTERED) return false;
        if (flags & HDR_FILTERED) {
            const float gq = lower_bound_margin(key_f32(bound_key)) / c.T;
            if (!(gq < key_f32(tau))) return false;
        }
    }

    // ---- survivors of top-k: one per thread when few
    uint32_t cnt = 0;
    for (uint32_t s = threadIdx.x; s < n; s += LLIMA_WG) cnt += (uint32_t)(sh.u.cbuf[s] >> 32) >= tau;
    const uint32_t nk = block_sum_u32(cnt, sh.bs);
    if (nk > SMALL_K) {
        finish_large(P, row, c, n, tau, kmax, sh);
        return true;
    }
    if (threadIdx.x == 0) sh.nk = 0;
    __syncthreads();
    const float xmax = key_f32(kmax);
    for (uint32_t s = threadIdx.x; s < n; s += LLIMA_WG) {
        const uint64_t q = sh.u.cbuf[s];
        const uint32_t k = (uint32_t)(q >> 32);
        if (k >= tau) {
            const uint32_t slot = atomicAdd(&sh.nk, 1u);
            sh.kkey[slot] = k;
            sh.kid[slot] = (uint32_t)q;
            sh.kw[slot] = weight(key_f32(k), xmax);
        }
    }
    __syncthreads();
    finish_small(P, row, c, nk, kmax, sh);
    return true;
}

template <typename TL>
__global__ __launch_bounds__(LLIMA_WG) void sample_finish(SampleParams P) {
    __shared__ FinishShared sh;
    const int row = blockIdx.x;
    const RowCfg c = load_cfg(P, row);
    const ChunkHdr* hdr = P.hdr + (size_t)row * P.S;

    // ---- merge the chunk headers
    uint32_t flags = 0, bound = 0, n = 0;
    uint64_t greedy = 0;
    for (int ch = threadIdx.x; ch < P.S; ch += LLIMA_WG) {
        const ChunkHdr h = hdr[ch];
        flags |= h.flags;
        n += h.count;
        if (h.flags & HDR_FILTERED) bound = h.bound > bound ? h.bound : bound;
        greedy = h.greedy > greedy ? h.greedy : greedy;
    }
    // OR of flags through a max of the two flag bits
    const uint32_t fl = block_max_u32(flags & HDR_OVERFLOW, sh.bs) |
                        block_max_u32(flags & HDR_FILTERED, sh.bs);
    bound = block_max_u32(bound, sh.bs);
    n = block_sum_u32(n, sh.bs);

    bool done = false;
    if (c.greedy) {
        greedy = block_max_u64(greedy, sh.bs);
        if (!(fl & HDR_OVERFLOW)) {
            const bool ok = (uint32_t)(greedy >> 32) > LLIMA_KEY_NEG_INF;
            const uint32_t tok = ok ? ~(uint32_t)greedy : 0xFFFFFFFFu;
            if (threadIdx.x == 0) write_result(P, row, ok ? (int32_t)tok : -1, ok ? 1.0f : 0.0f);
            if (P.out_keep)
                write_keep(P, row, [&](auto set) { if (threadIdx.x == 0 && ok) set(tok); });
            done = true;
        }
    } else if (!(fl & HDR_OVERFLOW) && n <= SAMPLE_FIN_CAP) {
        // ---- gather the candidates into LDS
        if (P.S <= LLIMA_WG) {
            // chunk offsets by one block scan, a position -> chunk table, then
            // every thread issues all of its loads before storing any
            const int ch = (int)threadIdx.x;
            const uint32_t cnt = ch < P.S ? hdr[ch].count : 0u;
            uint32_t tot;
            const uint32_t ex = block_excl_scan_u32(cnt, &tot, sh.bs);
            sh.off[threadIdx.x] = ex;
            for (uint32_t i = 0; i < cnt; ++i) sh.cid[ex + i] = (uint8_t)ch;
            __syncthreads();
            uint64_t q[SAMPLE_SLOTS];
#pragma unroll
            for (int j = 0; j < SAMPLE_SLOTS; ++j) {
                const uint32_t f = threadIdx.x + j * LLIMA_WG;
                const uint32_t cc = f < n ? sh.cid[f] : 0u;
                const uint32_t o = f < n ? f - sh.off[cc] : 0u;
                q[j] = P.cand[((size_t)row * P.S + cc) * P.share + o];
            }
#pragma unroll
            for (int j = 0; j < SAMPLE_SLOTS; ++j) {
                const uint32_t f = threadIdx.x + j * LLIMA_WG;
                if (f < n) sh.u.cbuf[f] = q[j];
            }
            __syncthreads();
        } else {
            uint32_t base = 0;
            for (int g0 = 0; g0 < P.S; g0 += LLIMA_WG) {
                const int ch = g0 + (int)threadIdx.x;
                const uint32_t cnt = ch < P.S ? hdr[ch].count : 0u;
                uint32_t tot;
                const uint32_t ex = block_excl_scan_u32(cnt, &tot, sh.bs);
                sh.off[threadIdx.x] = base + ex;
                __syncthreads();
                const int nch = P.S - g0 < LLIMA_WG ? P.S - g0 : LLIMA_WG;
                for (int k = (int)(threadIdx.x >> 6); k < nch; k += LLIMA_WAVES) {
                    const uint32_t o = sh.off[k];
                    const uint32_t m = hdr[g0 + k].count;
                    const uint64_t* src = P.cand + ((size_t)row * P.S + g0 + k) * P.share;
                    for (uint32_t i = lane_id(); i < m; i += 64) sh.u.cbuf[o + i] = src[i];
                }
                base += tot;
                __syncthreads();
            }
        }
        done = finish_fast(P, row, c, n, fl, bound, sh);
    }
    if (!done) finish_full_row<TL>(P, row, c, sh);
}

// ================================================================== host side
struct Tile { int E; int S; };

static Tile choose_tile(int B, int V, int dtype, int k) {
    // 16 KB of logits per workgroup; smaller chunks while the grid is small, as
    // long as the row's candidates (about k per chunk) fit the finish.
    int E = dtype == LLIMA_F32 ? 16 : 32;
    auto S_of = [&](int e) { return (V + LLIMA_WG * e - 1) / (LLIMA_WG * e); };
    while (E > 8) {
        if ((int64_t)B * S_of(E) >= 1024) break;
        if (k > 0 && (int64_t)S_of(E / 2) * k > SAMPLE_FIN_CAP / 2) break;
        E /= 2;
    }
    return {E, S_of(E)};
}

static size_t al256(size_t x) { return (x + 255) & ~(size_t)255; }
static int max_chunks(int V) { return (V + SAMPLE_MIN_CHUNK - 1) / SAMPLE_MIN_CHUNK; }

template <typename TL, int E>
static void launch_sweep(const SampleParams& P, hipStream_t st) {
    const dim3 g((uint32_t)P.B * (uint32_t)P.S), b(LLIMA_WG);
    if (P.vec_ok) hipLaunchKernelGGL((sample_sweep<TL, E, true>), g, b, 0, st, P);
    else hipLaunchKernelGGL((sample_sweep<TL, E, false>), g, b, 0, st, P);
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
    const int k_hint = cfg->top_k_rows ? 0 : cfg->top_k;
    const Tile t = choose_tile(B, V, dtype, (k_hint > 0 && k_hint < V) ? k_hint : 0);
    P.S = t.S;
    P.share = SAMPLE_ROW_CAND / t.S;
    P.hdr = (ChunkHdr*)workspace;
    P.cand = (uint64_t*)((char*)workspace + al256((size_t)B * max_chunks(V) * sizeof(ChunkHdr)));
    hipStream_t st = (hipStream_t)stream;
    if (dtype == LLIMA_F32) {
        if (t.E == 8) launch_sweep<float, 8>(P, st);
        else launch_sweep<float, 16>(P, st);
        hipLaunchKernelGGL(sample_finish<float>, dim3(B), dim3(LLIMA_WG), 0, st, P);
    } else {
        if (t.E == 8) launch_sweep<uint16_t, 8>(P, st);
        else if (t.E == 16) launch_sweep<uint16_t, 16>(P, st);
        else launch_sweep<uint16_t, 32>(P, st);
        hipLaunchKernelGGL(sample_finish<uint16_t>, dim3(B), dim3(LLIMA_WG), 0, st, P);
    }
    return hipGetLastError() == hipSuccess ? LLIMA_OK : LLIMA_E_HIP;
}
