// sample.hip -- fused penalty / temperature / mask / top-k / top-p / min-p /
// inverse-CDF sampling over [B, V] logits rows on MI355X (gfx950).
//
// Rows with top-k (or a grammar mask) take two launches per step, with no
// atomics or fences between workgroups (a device-scope release costs an L2
// write-back per workgroup on this part, and same-address atomics from
// thousands of workgroups serialise); masked batches without top-k add
// sample_finish_wide between them (further down); rows without top-k or mask
// take the dense path (five launches, every chunk's workgroup in each):
//
// sample_sweep: B x S workgroups; workgroup (row, chunk) owns 16 KB of one row
//   (4096 fp32 or 8192 bf16 values).  At 5 TB/s an fp32 value arrives every
//   ~0.8 ps, which leaves a few VALU operations per value: the sweep does one
//   max per value (the lane maxima), picks the chunk bound g from them with a
//   per-wave ballot search, and tests values against g only in the few lanes
//   whose maximum reaches it.  Values >= g are written, with their ids and in
//   id order, to the chunk's own workspace region behind a 16-byte header:
//     top-k rows    g = the largest of the four waves' r-th largest lane
//                   maxima (r ~ 8): about 20-30 values pass it;
//     other rows    g = chunk max - 27 T when values of zero weight cannot
//                   matter, else every finite value;
//     greedy rows   only the chunk's (maximum, first index) in the header.
//   Penalties: when they can only lower a value (repetition >= 1, presence
//   and frequency >= 0) on top-k rows, the sweep selects on the raw values
//   (a penalised value never exceeds its raw value, so the bound argument
//   holds) and the finish penalises the candidates only.  Otherwise the sweep
//   builds the chunk's history counts in LDS, with the history ids loaded
//   ahead of the chunk so that they are counted while it is in flight, and
//   penalises in registers.
//
// sample_finish: one workgroup per row.  One round of 16-byte loads covers the
//   header and the first slots of every chunk region; the candidates are
//   gathered into LDS in id order and spread over the threads (4 or 16 per
//   thread).  Lazy penalties count the row's history ids against an LDS hash
//   of the candidate ids.  After division by T, histogram rounds narrow the
//   top-k boundary until at most 64 values remain above it; those are ranked
//   pairwise (exact tau, top-p mass, min-p, the draw) split over the 4 waves.
//   The result stands only if the bounds provably lost nothing: tau must
//   exceed every chunk's fl(g / T), or, without top-k, every skipped value
//   must have weight 0.  Otherwise an exact multi-pass scan of the whole row
//   finishes it.
//
// The sampling semantics have no counterpart in the reference runtime, which
// only ever takes the argmax (sima_lmm/devkit/cpp/utils.hpp:80-152,
// sima_lmm/devkit/cpp/language_model.cpp:3689-3714); greedy rows follow that
// argmax (first index of the maximum) over the masked, penalised row.
#include <mutex>
#include <type_traits>

#include "common.hpp"
#include "../../include/llima_sampler.h"

namespace llima {

#define SMP_REGION 512                             // u64 slots per chunk region (4 KB)
#define SMP_HDR 1                                  // header slots at the start of a region
#define SMP_CAP (SMP_REGION - SMP_HDR)             // candidates a chunk can hand over
#define SMP_FIN_CAP 4096                           // candidates per row the finish holds
#define SMP_MAX_S 256                              // chunks per row the finish can gather
#define SMP_HBATCH 8                               // history ids per thread loaded up front
#define SMP_BOUND_LOWBIT 16                        // key bits below this are not searched
#define SMP_SMALL 64                               // survivors handled one per lane
#define SMP_WCAP 128                               // candidates a sweep wave can stage
#define SMP_SPARSE 12                              // lanes above the bound for a sparse sweep wave
#define SMP_SEG 8192                               // full-row path segment
#define SMP_HASH 4096                              // lazy-penalty hash slots
#define SMP_RCNT 16                                // split-row arrival counter stride (u32: 64 bytes)
#define SMP_XSTG 128                               // staging slots per chunk beyond its region
#define SMP_DSTG 64                                // of which the dense path's window uses
static_assert(SMP_DSTG <= 64 && SMP_DSTG <= SMP_XSTG, "one wave reads a dense window");
#define SMP_PBINS 256                              // top-p value bins: floor(8 (xmax - x)), the last open
#define SMP_PBIN_SCALE 8.0f
#define SMP_PBIN_SLOTS (SMP_PBINS + 64)            // + a spare bin per lane

#define HF_OVERFLOW 1u
#define SMP_PENDING ((int32_t)0x80000000)          // out_ids of a row sample_finish_wide left

// Chunk region: slot 0 is the header, low 32 bits: candidates written |
// flags << 16; high 32 bits (float bits): on top-k rows the bound g, every
// finite value >= g was written (-inf: all); on other rows the chunk maximum M,
// the bound being nontopk_bound(M).  Candidates follow from slot 1 as (key << 32 | id)
// in id order (the key of a finite value is never 0); the slots the finish
// reads in its first round (pre_slots) that hold no candidate carry
// SMP_SENTINEL, key 0.  Greedy rows: slot 1 holds (key << 32 | ~index) of the
// chunk maximum.
#define SMP_SENTINEL 0ull                          // key 0: no candidate

// Phase trace of sample_finish, compiled in only with -DLLIMA_FINISH_TRACE:
// thread 0 of each of the first SMP_TRACE_ROWS workgroups clears its row of
// fin_trace, then stores the wall clock (100 MHz) at each mark it passes
// (marks 14 and 15 hold counts); llima_finish_trace_read copies the table to
// the host.
#define SMP_TRACE_ROWS 512
#define SMP_TRACE_MARKS 16
#ifdef LLIMA_FINISH_TRACE
__device__ unsigned long long fin_trace[SMP_TRACE_ROWS][SMP_TRACE_MARKS];
#define FIN_MARK(i) do { if (threadIdx.x == 0 && blockIdx.y == 0 && blockIdx.x < SMP_TRACE_ROWS) fin_trace[blockIdx.x][i] = wall_clock64(); } while (0)
#define FIN_NOTE(i, v) do { if (threadIdx.x == 0 && blockIdx.y == 0 && blockIdx.x < SMP_TRACE_ROWS) fin_trace[blockIdx.x][i] = (v); } while (0)
// any part of a split row (the one that finishes it)
#define FIN_MARK_ANY(i) do { if (threadIdx.x == 0 && blockIdx.x < SMP_TRACE_ROWS) fin_trace[blockIdx.x][i] = wall_clock64(); } while (0)
#define FIN_BEGIN() do { if (threadIdx.x == 0 && blockIdx.y == 0 && blockIdx.x < SMP_TRACE_ROWS) { \
        for (int m_ = 1; m_ < SMP_TRACE_MARKS; ++m_) fin_trace[blockIdx.x][m_] = 0; } FIN_MARK(0); } while (0)
#else
#define FIN_BEGIN() do { } while (0)
#define FIN_MARK(i) do { } while (0)
#define FIN_MARK_ANY(i) do { } while (0)
#define FIN_NOTE(i, v) do { } while (0)
#endif
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
    uint64_t* ws;        // [B][S][SMP_REGION]
    int32_t B, V, H_max, S;
    int32_t lgs;         // log2 of S rounded up to a power of two (finish gather)
    int32_t vec_ok;
    int32_t lazy;        // rows may take their penalties in the finish (row_lazy decides per row)
    int32_t eager;       // rows may take their penalties in the sweep (its history count table)
    int32_t rank;        // bound_rank of the broadcast top-k (per-row k: computed per row)
    int32_t wide;        // sample_finish_wide ran first: finish only the rows it left pending
    int32_t fsplit;      // sample_finish workgroups per row (> 1: rows without top-k may be split)
    int32_t rcpw;        // chunks per part of a split row (at most SMP_RCPW)
    int32_t scap;        // values a split row's chunk stages (at most SMP_STG_CAP)
    uint64_t* xstg;      // [B][S][SMP_XSTG] split-row staging beyond the regions
    uint32_t* rcnt;      // [B][SMP_RCNT] split-row arrival counters, zeroed by the sweep
};

struct RowCfg {
    float T, p, m, R, alpha, beta;
    float u;             // the row's uniform (loaded up front: it ends the finish)
    int32_t k;           // 0: top-k disabled
    bool greedy, pen;
    int32_t hlen;
};

// The per-row value when the array is given, else the broadcast scalar (passed
// by value: selecting between a pointer into the kernel arguments and one
// into global memory would force the arguments into private memory).
template <typename T>
__device__ __forceinline__ T row_or(const T* rows, T scalar, int row) {
    return rows ? __builtin_nontemporal_load(rows + row) : scalar;
}

__device__ __forceinline__ RowCfg load_cfg(const SampleParams& P, int row) {
    const llima_sampler_config& c = P.cfg;
    RowCfg r;
    r.T = row_or(c.temperature_rows, c.temperature, row);
    r.k = row_or(c.top_k_rows, c.top_k, row);
    r.p = row_or(c.top_p_rows, c.top_p, row);
    r.m = row_or(c.min_p_rows, c.min_p, row);
    r.R = row_or(c.repetition_penalty_rows, c.repetition_penalty, row);
    r.alpha = row_or(c.presence_penalty_rows, c.presence_penalty, row);
    r.beta = row_or(c.frequency_penalty_rows, c.frequency_penalty, row);
    r.u = P.uniforms[row];
    r.greedy = (c.greedy != 0) || !(r.T > 0.0f);
    int h = 0;
    if (P.H_max > 0) {
        h = row_or(P.hist_len, (int32_t)P.H_max, row);
        h = h < 0 ? 0 : (h > P.H_max ? P.H_max : h);
    }
    r.hlen = h;
    r.pen = h > 0 && (r.R != 1.0f || r.alpha != 0.0f || r.beta != 0.0f);
    if (!(r.k > 0 && r.k < P.V)) r.k = 0;
    return r;
}

// A row's penalties are applied by the finish, to its candidates only, when
// they can only lower a value (repetition >= 1, presence and frequency >= 0)
// and the row samples with top-k: a penalised value never exceeds its raw
// value, so the sweep's bound on the raw values still holds.  Otherwise the
// sweep applies them to every value of the row.
__device__ __forceinline__ bool row_lazy(const SampleParams& P, const RowCfg& c) {
    return P.lazy && c.pen && !c.greedy && c.k > 0 && c.R >= 1.0f && c.alpha >= 0.0f &&
           c.beta >= 0.0f;
}

// Values of weight 0 can be left out of the candidates when they cannot be in
// the reported kept set: top-p drops them (all positive mass lies above them),
// min-p with a positive threshold drops them, and without a kept-set output
// they never affect the draw.
__device__ __forceinline__ bool zero_weight_irrelevant(const SampleParams& P, const RowCfg& c) {
    return P.out_keep == nullptr || c.p < 1.0f || (c.m > 0.0f && frac32(c.m) > 0);
}

// The sweep's chunk bound on a row without top-k, from the chunk maximum M
// (penalised and masked, before / T; -inf when the chunk has no value above
// -inf): M - 27 T when values of zero weight cannot matter, else -inf (every
// finite value is a candidate).  The sweep and the finish evaluate it with the
// same operations, so the header holds M and both derive the same bound.
__device__ __forceinline__ float nontopk_bound(const SampleParams& P, const RowCfg& c, float M) {
    if (!(M > -__builtin_inff()) || !zero_weight_irrelevant(P, c)) return -__builtin_inff();
    const float gm = M - 27.0f * c.T;
    return gm == gm ? gm : -__builtin_inff();
}

// Lane maxima ranked, per wave, for the top-k chunk bound: a wave (1024 fp32
// or 2048 bf16 values) rarely holds this many of the row's top-k values (about
// k / (4 S) on average).  Also used on the host for a broadcast top-k.
__host__ __device__ inline uint32_t bound_rank(int k, int S) {
    int r = (k + S - 1) / S + 6;
    r = r < 8 ? 8 : (r > 64 ? 64 : r);
    return (uint32_t)(k < r ? k : r);
}

// HF RepetitionPenalty (score < 0 ? score * p : score / p), then OpenAI
// frequency and presence, each one IEEE operation (no contraction).
__device__ __forceinline__ float penalize(float l, uint32_t c, const RowCfg& cfg) {
    l = (l < 0.0f) ? l * cfg.R : l / cfg.R;
    return (l - cfg.beta * (float)c) - cfg.alpha;
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

__device__ __forceinline__ uint64_t* region_of(const SampleParams& P, uint32_t row, uint32_t chunk) {
    return P.ws + ((size_t)row * (uint32_t)P.S + chunk) * SMP_REGION;
}

// Slots of every region the finish reads in its first round: 8 per thread,
// 256 >> lgs threads per chunk.
__device__ __forceinline__ uint32_t pre_slots(const SampleParams& P) {
    const uint32_t n = (uint32_t)(LLIMA_WG >> P.lgs) * 8u;
    return n < SMP_REGION ? n : SMP_REGION;
}

// ================================================================== sweep
// VEC: rows are 16-byte aligned and V is a multiple of the values per load, so
// every chunk (also a row's partial last one) is read with 16-byte loads from
// clamped, always-valid addresses and the out-of-row values masked in registers.
// MASK: a grammar bitmask is given.  NaN values stay NaN here: every later use
// is an ordered comparison or a max that ignores NaN, so a NaN is never selected.
// SC: chunks per workgroup (consecutive chunks of one row).  Chunk cc + 1 is
// requested once chunk cc has arrived and before it is processed, so the
// processing overlaps the next transfer (with every load of the grid issued at
// once, each chunk completes only when the last of all requests does).
template <typename TL, bool VEC, bool MASK, int SC>
__global__ __launch_bounds__(LLIMA_WG) void sample_sweep(SampleParams P) {
    constexpr int EPL = 16 / sizeof(TL);       // values per 16-byte load
    constexpr int NL = 4;                      // 16-byte loads per thread and chunk
    constexpr int E = NL * EPL;                // values per thread and chunk
    constexpr int CHUNK = LLIMA_WG * E;
    constexpr int CW = SC * CHUNK / 2;         // history count words (the group)
    constexpr int WS = CHUNK / LLIMA_WAVES;    // ids per wave and chunk
    // lanes of a sparse wave: 8 for bf16 (64 parked values per load: one step), 12 for fp32
    constexpr int SPL = sizeof(TL) == 2 ? 8 : SMP_SPARSE;
    // history counts of the group, two 16-bit counts per word: dynamic LDS,
    // sized by the launch only when the sweep applies the penalties itself
    // (otherwise 0 bytes, which keeps the workgroups' LDS small)
    extern __shared__ __align__(16) uint32_t cnt[];
    __shared__ uint32_t xa[SC][LLIMA_WAVES];
    __shared__ uint32_t xn[SC][LLIMA_WAVES];              // candidates per wave
    // a wave's staged candidates (+ a spare slot per lane) or, for a sparse
    // wave, first its parked values: the same 1.5 KB (the sweep's LDS size
    // sets how fast its workgroups are dispatched)
    __shared__ __align__(16) uint64_t xst[SC][LLIMA_WAVES][SMP_WCAP + 64];
    __shared__ uint32_t xl[SC][LLIMA_WAVES][SMP_SPARSE];     // a sparse wave's parking lanes
    static_assert(NL * SMP_SPARSE * EPL * 4 <= (SMP_WCAP + 64) * 8, "parked values exceed the staging");
    __shared__ uint64_t xg[SC][LLIMA_WAVES];
    const float NEG_INF = -__builtin_inff();

    const uint32_t G = ((uint32_t)P.S + SC - 1) / SC;   // chunk groups per row
    uint32_t row, grp;
    map_row_chunk(blockIdx.x, (uint32_t)P.B, G, &row, &grp);
    if (row >= (uint32_t)P.B) return;
    const int t = (int)threadIdx.x;
    const uint32_t lane = lane_id(), wave = wave_id();
    // wave w of a chunk owns its ids [w WS, (w + 1) WS); load j of lane l covers
    // EPL ids at j 64 EPL + l EPL of that slice (1 KB contiguous per wave load)
    const int lofs = (int)wave * WS + (int)lane * EPL;
    const TL* rowp = (const TL*)P.logits + (size_t)row * P.row_stride;
    const int V = P.V;
    const int g0 = (int)grp * SC * CHUNK;                      // first id of the group
    const int g1 = g0 + SC * CHUNK < V ? g0 + SC * CHUNK : V;
    const uint32_t* mrow = P.bitmask ? P.bitmask + (size_t)row * ((V + 31) >> 5) : nullptr;
    const int H = P.H_max;
    const bool eager = H > 0 && P.eager;
    if (P.fsplit > 1 && grp == 0 && t == 0) P.rcnt[(size_t)row * SMP_RCNT] = 0u;   // split-row arrivals

    // ---- 1. loads, in the order their data is used, all before the first
    //         wait: the row's settings (per-row arrays: loaded first, since the
    //         history count waits for them and a wait covers every older
    //         load), history ids (rows penalised here), mask words, the chunks
    const RowCfg c = load_cfg(P, row);
    int32_t hid[SMP_HBATCH];
    if (eager) {
        const int32_t* hrow = P.hist + (size_t)row * H;
#pragma unroll
        for (int b = 0; b < SMP_HBATCH; ++b) {
            const int j = t + b * LLIMA_WG;
            hid[b] = hrow[j < H ? j : H - 1];
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    uint32_t mword[SC][NL];
    llima_u32x4 raw[SC][NL];
    auto issue = [&](int cc) {                  // mask words and values of chunk cc
        if constexpr (MASK) {
#pragma unroll
            for (int j = 0; j < NL; ++j) {
                const int i0 = g0 + cc * CHUNK + j * (64 * EPL) + lofs;
                mword[cc][j] = mrow[(i0 < V ? i0 : V - 1) >> 5];
            }
        }
#pragma unroll
        for (int j = 0; j < NL; ++j) {
            const int i0 = g0 + cc * CHUNK + j * (64 * EPL) + lofs;
            if constexpr (VEC) {
                const int ia = i0 < V ? i0 : V - EPL;
                raw[cc][j] = __builtin_nontemporal_load((const llima_u32x4*)(rowp + ia));
            } else {
                uint32_t w[4] = {0, 0, 0, 0};
#pragma unroll
                for (int e = 0; e < EPL; ++e) {
                    const int ia = i0 + e < V ? i0 + e : V - 1;
                    const float f = load_one<TL>(rowp, ia);
                    if constexpr (sizeof(TL) == 4) w[e] = __float_as_uint(f);
                    else w[e >> 1] |= (__float_as_uint(f) >> 16) << ((e & 1) * 16);
                }
                raw[cc][j] = llima_u32x4{w[0], w[1], w[2], w[3]};
            }
        }
    };
    issue(0);
    __builtin_amdgcn_sched_barrier(0);
    const bool pen_here = eager && c.pen && !row_lazy(P, c);

    // ---- 2. history counts of the group (waits for the history ids only)
    if (pen_here) {
#pragma unroll
        for (int i = t; i < CW / 4; i += LLIMA_WG) ((llima_u32x4*)cnt)[i] = llima_u32x4{0, 0, 0, 0};
        __syncthreads();
#pragma unroll
        for (int b = 0; b < SMP_HBATCH; ++b) {
            const int32_t id = hid[b];
            if (t + b * LLIMA_WG < c.hlen && id >= g0 && id < g1) {
                const uint32_t off = (uint32_t)(id - g0);
                atomicAdd(&cnt[off >> 1], 1u << ((off & 1u) * 16u));
            }
        }
        const int32_t* hrow = P.hist + (size_t)row * H;
        for (int j = t + SMP_HBATCH * LLIMA_WG; j < c.hlen; j += LLIMA_WG) {
            const int32_t id = hrow[j];
            if (id >= g0 && id < g1) {
                const uint32_t off = (uint32_t)(id - g0);
                atomicAdd(&cnt[off >> 1], 1u << ((off & 1u) * 16u));
            }
        }
        __syncthreads();
    }
    const uint32_t rank = P.cfg.top_k_rows ? bound_rank(c.k, P.S) : (uint32_t)P.rank;

#pragma unroll
    for (int cc = 0; cc < SC; ++cc) {
        const uint32_t chunk = grp * SC + (uint32_t)cc;
        if (chunk >= (uint32_t)P.S) break;
        const int c0 = g0 + cc * CHUNK;
        const int c1 = c0 + CHUNK < V ? c0 + CHUNK : V;

        // ---- 3. values: masked -> -inf, history values penalised (here),
        //         values past the row -> -inf (the last chunk only)
        float v[E];
#pragma unroll
        for (int j = 0; j < NL; ++j) {
            const int i0 = c0 + j * (64 * EPL) + lofs;
            float xv[EPL];
            const uint32_t w4[4] = {raw[cc][j].x, raw[cc][j].y, raw[cc][j].z, raw[cc][j].w};
            if constexpr (sizeof(TL) == 4) {
#pragma unroll
                for (int e = 0; e < 4; ++e) xv[e] = __uint_as_float(w4[e]);
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    xv[2 * e] = __uint_as_float(w4[e] << 16);
                    xv[2 * e + 1] = __uint_as_float(w4[e] & 0xFFFF0000u);
                }
            }
            if constexpr (MASK) {
                const uint32_t mb = mword[cc][j] >> (i0 & 31);
#pragma unroll
                for (int e = 0; e < EPL; ++e) xv[e] = ((mb >> e) & 1u) ? xv[e] : NEG_INF;
            }
            if (pen_here) {
                uint32_t cw[EPL / 2];
                const uint32_t* cp = cnt + ((i0 - g0) >> 1);
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
                        if (lo) xv[2 * h] = penalize(xv[2 * h], lo, c);
                        if (hi) xv[2 * h + 1] = penalize(xv[2 * h + 1], hi, c);
                    }
                }
            }
#pragma unroll
            for (int e = 0; e < EPL; ++e) v[j * EPL + e] = xv[e];
        }
        if (c1 - c0 < CHUNK) {
#pragma unroll
            for (int j = 0; j < NL; ++j) {
                const int i0 = c0 + j * (64 * EPL) + lofs;
#pragma unroll
                for (int e = 0; e < EPL; ++e)
                    if (i0 + e >= c1) v[j * EPL + e] = NEG_INF;
            }
        }
        // lane maximum (a NaN is ignored by the max): it reads every value, so
        // chunk cc is in when it is done; then the next chunk is requested
        // before this one is worked on (unconditionally: addresses past the row
        // are clamped, and loads behind a branch make the next use wait)
        float lm = v[0];
#pragma unroll
        for (int e = 1; e < E; ++e) lm = __builtin_fmaxf(lm, v[e]);
        if (cc + 1 < SC) {
            asm volatile("" ::"v"(lm) : "memory");   // lm computed here, loads stay below
            issue(cc + 1);
        }

        uint64_t* reg = region_of(P, row, chunk);
        if (c.greedy) {
            // ---- argmax: first index of the maximum (values visited in index order)
            float best = NEG_INF;
            uint32_t bidx = 0;
#pragma unroll
            for (int j = 0; j < NL; ++j) {
                const int i0 = c0 + j * (64 * EPL) + lofs;
#pragma unroll
                for (int e = 0; e < EPL; ++e)
                    if (v[j * EPL + e] > best) { best = v[j * EPL + e]; bidx = (uint32_t)(i0 + e); }
            }
            const uint64_t kk = best > NEG_INF ? (((uint64_t)f32_key(best) << 32) | (uint32_t)~bidx) : 0ull;
            const uint64_t wk = wave_max_u64(kk);
            if (lane == 0) xg[cc][wave] = wk;
            __syncthreads();
            if (t == 0) {
                uint64_t g = 0;
#pragma unroll
                for (int w = 0; w < LLIMA_WAVES; ++w) g = xg[cc][w] > g ? xg[cc][w] : g;
                *(llima_u32x4*)reg = llima_u32x4{0u, __float_as_uint(NEG_INF), (uint32_t)g,
                                                 (uint32_t)(g >> 32)};
            }
            continue;
        }

        // ---- 4. the chunk bound g
        const uint32_t lk = lm > NEG_INF ? f32_key(lm) : 0u;
        float g = NEG_INF, cmax = NEG_INF;
        if (c.k > 0) {
            // g = the largest of the four waves' r-th largest lane maxima (low
            // key bits cleared: a lower value).  Any g is correct, since every
            // value >= g is written and the finish checks that its top-k
            // boundary lies above g; a smaller g costs candidates, a larger
            // one the finish's fast path (when one wave holds r of the row's
            // top-k values).  One wave-level search, no second pass: this runs
            // after the chunk's data arrived, on the kernel's critical path.
            const uint32_t bw = wave_rth_largest_exp(lk, rank, SMP_BOUND_LOWBIT);
            if (lane == 0) xa[cc][wave] = bw;
            __syncthreads();
            uint32_t gk = 0;
#pragma unroll
            for (int w = 0; w < LLIMA_WAVES; ++w) gk = xa[cc][w] > gk ? xa[cc][w] : gk;
            if (gk) g = key_f32(gk);
        } else {
            // the chunk maximum (the header keeps it for the finish), and the
            // bound below which values have weight 0 (checked exactly by the
            // finish against the row maximum)
            const uint32_t wm = wave_max_u32(lk);
            if (lane == 0) xa[cc][wave] = wm;
            __syncthreads();
            uint32_t mk = 0;
#pragma unroll
            for (int w = 0; w < LLIMA_WAVES; ++w) mk = xa[cc][w] > mk ? xa[cc][w] : mk;
            if (mk) cmax = key_f32(mk);
            g = nontopk_bound(P, c, cmax);
        }
        // the smallest finite float stands for -inf: -inf and NaN never pass
        const float g2 = g > NEG_INF ? g : -__FLT_MAX__;

        // ---- 5. the values >= g in id order (load j, lane, value: id order
        //         inside the wave's slice).  Each wave stages its own in LDS,
        //         then, after the one barrier, copies its run to the region
        //         behind the runs of the waves before it.
        //         Sparse waves (at most SPL lanes hold a value >= g: every top-k
        //         row): those lanes park their values in LDS in id order and
        //         all 64 lanes then test 64 of them per step (ballot + mbcnt
        //         place them), so the cost follows the lanes that matter.
        //         Dense waves: per-lane bit masks, two packed wave scans for
        //         the offsets, writes to a spare slot per lane instead of
        //         branches.
        uint64_t* stg = xst[cc][wave];
        const uint64_t qm = ballot(lm >= g2);
        const uint32_t nq = (uint32_t)__popcll(qm);
        const bool sparse = nq <= (uint32_t)SPL;              // uniform in the wave
        float* xw = (float*)stg;                              // parked values
        constexpr int SR = (SPL * EPL + 63) / 64;             // steps per load
        // staging: writes only when the wave's candidates fit (its parked
        // values, all read by then, are overwritten); else nothing, and the
        // pass runs again after the barrier with the region as destination
        auto sparse_pass = [&](auto put, bool staging) {
            // every LDS read first (one latency), then the tests and writes
            float f[NL][SR];
            uint32_t L[NL][SR];
#pragma unroll
            for (int j = 0; j < NL; ++j)
#pragma unroll
                for (int r = 0; r < SR; ++r) {
                    const uint32_t k = (uint32_t)r * 64u + lane;     // value k % EPL of rank k / EPL
                    const bool valid = k < nq * EPL;
                    f[j][r] = xw[j * SPL * EPL + (valid ? k : 0u)];
                    L[j][r] = xl[cc][wave][valid ? k / EPL : 0u];
                }
            uint64_t b[NL][SR];
            uint32_t tot = 0;
#pragma unroll
            for (int j = 0; j < NL; ++j)
#pragma unroll
                for (int r = 0; r < SR; ++r) {
                    b[j][r] = ballot((uint32_t)r * 64u + lane < nq * EPL && f[j][r] >= g2);
                    tot += (uint32_t)__popcll(b[j][r]);
                }
            if (!staging || tot <= SMP_WCAP) {
                uint32_t base = 0;
#pragma unroll
                for (int j = 0; j < NL; ++j)
#pragma unroll
                    for (int r = 0; r < SR; ++r) {
                        if ((b[j][r] >> lane) & 1ull) {
                            const uint32_t k = (uint32_t)r * 64u + lane;
                            const uint32_t id = (uint32_t)(c0 + j * (64 * EPL) + (int)wave * WS) + L[j][r] * EPL + k % EPL;
                            put(base + mbcnt(b[j][r]), ((uint64_t)__float_as_uint(f[j][r]) << 32) | id);
                        }
                        base += (uint32_t)__popcll(b[j][r]);
                    }
            }
            return tot;
        };
        uint32_t pm[NL] = {0, 0, 0, 0}, start[NL] = {0, 0, 0, 0};
        uint32_t nw;
        if (sparse) {
            if (lm >= g2) {
                const uint32_t qr = mbcnt(qm);
#pragma unroll
                for (int j = 0; j < NL; ++j) {
#pragma unroll
                    for (int h = 0; h < EPL / 4; ++h)
                        *(llima_u32x4*)&xw[j * SPL * EPL + qr * EPL + 4 * h] =
                            llima_u32x4{__float_as_uint(v[j * EPL + 4 * h]), __float_as_uint(v[j * EPL + 4 * h + 1]),
                                        __float_as_uint(v[j * EPL + 4 * h + 2]), __float_as_uint(v[j * EPL + 4 * h + 3])};
                }
                xl[cc][wave][qr] = lane;
            }
            __builtin_amdgcn_wave_barrier();                  // the wave's LDS writes precede its reads
            nw = sparse_pass([&](uint32_t pos, uint64_t val) { stg[pos] = val; }, true);
        } else {
            if (lm >= g2) {
#pragma unroll
                for (int j = 0; j < NL; ++j) {
                    uint32_t m = 0;
#pragma unroll
                    for (int e = 0; e < EPL; ++e) m |= v[j * EPL + e] >= g2 ? (1u << e) : 0u;
                    pm[j] = m;
                }
            }
            const uint32_t a01 = (uint32_t)__popc(pm[0]) | ((uint32_t)__popc(pm[1]) << 16);
            const uint32_t a23 = (uint32_t)__popc(pm[2]) | ((uint32_t)__popc(pm[3]) << 16);
            const uint32_t i01 = wave_incl_scan_u32(a01), i23 = wave_incl_scan_u32(a23);
            const uint32_t t01 = readlane63(i01), t23 = readlane63(i23);
            const uint32_t T0 = t01 & 0xFFFFu, T1 = t01 >> 16, T2 = t23 & 0xFFFFu, T3 = t23 >> 16;
            nw = T0 + T1 + T2 + T3;
            const uint32_t e01 = i01 - a01, e23 = i23 - a23;
            start[0] = e01 & 0xFFFFu;                          // this lane's first slot per load
            start[1] = T0 + (e01 >> 16);
            start[2] = T0 + T1 + (e23 & 0xFFFFu);
            start[3] = T0 + T1 + T2 + (e23 >> 16);
            if (nw <= SMP_WCAP && lm >= g2) {
#pragma unroll
                for (int j = 0; j < NL; ++j) {
                    const int i0 = c0 + j * (64 * EPL) + lofs;
                    uint32_t o = start[j];
#pragma unroll
                    for (int e = 0; e < EPL; ++e) {
                        const bool in = (pm[j] >> e) & 1u;
                        stg[in ? o : SMP_WCAP + lane] =
                            ((uint64_t)__float_as_uint(v[j * EPL + e]) << 32) | (uint32_t)(i0 + e);
                        o += in ? 1u : 0u;
                    }
                }
            }
        }
        if (lane == 0) xn[cc][wave] = nw;
        __syncthreads();
        uint32_t off = 0, total = 0;
#pragma unroll
        for (int w = 0; w < LLIMA_WAVES; ++w) {
            const uint32_t n = xn[cc][w];
            off += (uint32_t)w < wave ? n : 0u;
            total += n;
        }
        const bool fits = total <= SMP_CAP;
        if (fits) {
            if (nw <= SMP_WCAP) {
                for (uint32_t i = lane; i < nw; i += 64) {     // staged as value bits, written as keys
                    const uint64_t sv = stg[i];
                    reg[SMP_HDR + off + i] =
                        ((uint64_t)f32_key(__uint_as_float((uint32_t)(sv >> 32))) << 32) | (uint32_t)sv;
                }
            } else if (sparse) {
                // more than the staging holds: the sparse pass again, to the region
                sparse_pass([&](uint32_t pos, uint64_t val) {
                    reg[SMP_HDR + off + pos] =
                        ((uint64_t)f32_key(__uint_as_float((uint32_t)(val >> 32))) << 32) | (uint32_t)val;
                }, false);
            } else if (lm >= g2) {
                // more than the staging holds (dense rows such as grammar-masked
                // ones without top-k): straight from the registers
#pragma unroll
                for (int j = 0; j < NL; ++j) {
                    const int i0 = c0 + j * (64 * EPL) + lofs;
                    uint32_t o = SMP_HDR + off + start[j];
#pragma unroll
                    for (int e = 0; e < EPL; ++e) {
                        if ((pm[j] >> e) & 1u) {
                            reg[o] = ((uint64_t)f32_key(v[j * EPL + e]) << 32) | (uint32_t)(i0 + e);
                            ++o;
                        }
                    }
                }
            }
            const uint32_t pre = pre_slots(P);
            for (uint32_t i = SMP_HDR + total + (uint32_t)t; i < pre; i += LLIMA_WG) reg[i] = SMP_SENTINEL;
        }
        if (t == 0)
            *(uint64_t*)reg = ((uint64_t)__float_as_uint(c.k > 0 ? g : cmax) << 32) |
                              (fits ? total : (HF_OVERFLOW << 16));
    }
}

// ================================================================== finish
struct FinShared {
    union {
        uint64_t cand[SMP_FIN_CAP + SMP_FIN_CAP / 16];   // element f at f + f / 16
        uint32_t table[SMP_SEG / 2];                     // full-row path history counts
        struct {
            uint32_t key[SMP_HASH];                      // candidate id + 1, 0 = empty
            uint32_t cnt[SMP_HASH];                      // history occurrences
        } hash;
    } u;
    uint32_t ccount[SMP_MAX_S];
    uint32_t coff[SMP_MAX_S];
    uint32_t hcnt[3][256 + 64];                      // + a spare bin per lane
    uint64_t hmass[3][256 + 64];                     // + a spare bin per lane
    llima_u32x4 sv[2 * SMP_SMALL + 64];              // + a spare slot per lane
    llima_u32x4 sv2[LLIMA_WAVES][2 * SMP_SMALL];
    uint32_t pc[2][LLIMA_WAVES][64];
    uint64_t part[2][LLIMA_WAVES][64];
    uint64_t part2[2][LLIMA_WAVES][64];
    uint64_t r64[4][LLIMA_WAVES];
    uint32_t r32[8][LLIMA_WAVES];
    uint32_t sel[4];
    uint64_t sel64[2];
    uint32_t hflags, hgkey, hn, lcount;
    uint64_t hgreedy;
    uint32_t hc[LLIMA_WG];                           // survivors' history occurrences
    BlockScratch bs;
};

// ------------------------------------------------------------------ radix helpers
// Digits are 8 bits wide and start at the highest bit in which the keys differ.
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

// Top-p boundary: the smallest key theta such that an element with key theta
// has (mass strictly above) * 2^32 < p32 * Z, Z the mass of every element
// (every nonzero key lies in [kmin, kmax]); when none has (p32 == 0) the top
// key.  Radix rounds over 8-bit digits with one barrier each: round r counts
// into buffer r % 3 (buffers 0 and 1 zero on entry; non-members count into a
// spare bin per lane), then every wave scans all 256 bins itself and zeroes
// buffer (r + 2) % 3.  Round 0 holds every element, so its total is Z.  Stops
// early when the selected bin holds one key.  With pz_given the elements are
// the part of a larger set below a mass `above`, and PZ0 = p32 * Z of that set.
template <int EPT>
__device__ __forceinline__ uint32_t fin_topp_desc(const uint32_t (&key)[EPT], const uint64_t (&w)[EPT],
                                  uint64_t p32, uint32_t kmin, uint32_t kmax, FinShared& sh,
                                  uint64_t above = 0, llima_u128 PZ0 = 0, bool pz_given = false) {
    Digits d = digits_init(kmin, kmax);
    uint64_t acc = above;
    llima_u128 PZ = 0;
    bool first = true;
    const uint32_t t = threadIdx.x, lane = lane_id();
    uint32_t buf = 0;
    while (d.top >= 0) {
        const int lo = d.top - 7 > 0 ? d.top - 7 : 0;
        const uint32_t bmask = (1u << (d.top - lo + 1)) - 1u;
        uint64_t* hm = sh.hmass[buf];
        // one 64-bit atomic per value: (mass << 13) + count (W <= 2^36 and at
        // most 4096 values: mass < 2^49, count < 2^13)
#pragma unroll
        for (int j = 0; j < EPT; ++j) {
            const bool in = (key[j] != 0u) & ((key[j] & d.pmask) == d.prefix);
            const uint32_t b = in ? (key[j] >> lo) & bmask : 256u + lane;
            atomicAdd((unsigned long long*)&hm[b], (unsigned long long)((w[j] << 13) | 1ull));
        }
        __syncthreads();
        // lane l: bins 255 - 4l down to 252 - 4l
        uint32_t cs[4];
        uint64_t ms[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint64_t v = hm[255u - 4u * lane - (uint32_t)i];
            cs[i] = (uint32_t)(v & 0x1FFFu);
            ms[i] = v >> 13;
        }
        const uint32_t nxt = buf == 0u ? 2u : buf - 1u;
        sh.hmass[nxt][t] = 0;
        const uint64_t m4 = ms[0] + ms[1] + ms[2] + ms[3];
        const uint64_t inc = wave_incl_scan_u64(m4);
        if (first) PZ = pz_given ? PZ0 : (llima_u128)p32 * readlane63(inc);   // p32 * Z
        first = false;
        uint64_t ab = acc + inc - m4;                               // mass above the lane's top bin
        // last qualifying bin of the lane (lowest key), first non-empty bin
        int qi = -1, ni = -1;
        uint64_t qab = 0, nab = 0;
        uint32_t qcn = 0, ncn = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const bool ne = cs[i] > 0u;
            const bool q = ne && (((llima_u128)ab << 32) < PZ);
            qi = q ? i : qi; qab = q ? ab : qab; qcn = q ? cs[i] : qcn;
            const bool first = ne && ni < 0;
            ni = first ? i : ni; nab = first ? ab : nab; ncn = first ? cs[i] : ncn;
            ab += ms[i];
        }
        const uint64_t bq = ballot(qi >= 0), bn = ballot(ni >= 0);
        uint32_t L, sel;
        uint64_t sab;
        uint32_t scn;
        if (bq) {                                   // the lowest qualifying bin: highest lane
            L = 63u - (uint32_t)__builtin_clzll(bq);
            sel = 255u - 4u * L - (uint32_t)readlane((uint32_t)qi, L);
            sab = readlane64(qab, L);
            scn = readlane(qcn, L);
        } else {                                    // else the top non-empty bin: lowest lane
            L = bn ? (uint32_t)__builtin_ffsll((long long)bn) - 1u : 0u;
            sel = bn ? 255u - 4u * L - (uint32_t)readlane((uint32_t)ni, L) : 255u;
            sab = bn ? readlane64(nab, L) : acc;
            scn = bn ? readlane(ncn, L) : 0u;
        }
        d.prefix |= sel << lo;
        d.pmask |= bmask << lo;
        d.top = lo - 1;
        acc = sab;
        buf = buf == 2u ? 0u : buf + 1u;
        if (scn == 1u && d.top >= 0) {
            // one key left in the selected bin: later rounds would select it
            // digit by digit (its mass above is the same at every level), so it
            // is theta
            uint32_t kk = 0;
#pragma unroll
            for (int j = 0; j < EPT; ++j) {
                const bool in = (key[j] != 0u) & ((key[j] & d.pmask) == d.prefix);
                kk = in && key[j] > kk ? key[j] : kk;
            }
            return block_max_u32(kk, sh.bs);
        }
    }
    __syncthreads();
    return d.prefix;
}

// Top-p boundary over value bins: the key fin_topp_desc returns, found with one
// round of 64-bit LDS atomics ((mass << 13) + count) into bins of 1/8 nat below
// the maximum (bin floor(8 (xmax - x)), a monotone function of the key, the
// last bin open), then inside the one bin that holds the boundary: the last
// non-empty bin whose mass above, times 2^32, is below p32 Z.  Its members (at
// most 64) are ranked pairwise in every wave.  bins: SMP_PBIN_SLOTS zeroed
// slots (a spare per lane), sh.lcount zero on entry.  Returns 0, with every
// wave taking the same branch, when the maximum is infinite or the boundary
// bin holds more than 64 values: the caller then runs fin_topp_desc.
template <int EPT, class SH>
__device__ __forceinline__ uint32_t fin_topp_bins(const uint32_t (&key)[EPT], const uint64_t (&w)[EPT],
                                                  uint64_t p32, uint32_t kmax, uint64_t* bins,
                                                  SH& sh) {
    const uint32_t lane = lane_id();
    const float xmax = key_f32(kmax);
    if (!(xmax < __builtin_inff())) return 0u;      // uniform
    uint32_t bn[EPT];
#pragma unroll
    for (int j = 0; j < EPT; ++j) {
        const float d = __builtin_fminf((xmax - key_f32(key[j])) * SMP_PBIN_SCALE, (float)(SMP_PBINS - 1));
        const uint32_t b = (uint32_t)d;                 // d in [0, SMP_PBINS - 1] for a present key
        bn[j] = key[j] ? b : 0xFFFFFFFFu;
        atomicAdd((unsigned long long*)&bins[key[j] ? b : SMP_PBINS + lane],
                  (unsigned long long)((w[j] << 13) | 1ull));
    }
    __syncthreads();
    // every wave reads every bin: lane l holds bins 4 l .. 4 l + 3
    uint64_t m[4];
    uint32_t cn[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint64_t v = bins[4u * lane + (uint32_t)i];
        m[i] = v >> 13;
        cn[i] = (uint32_t)(v & 0x1FFFu);
    }
    const uint64_t ms = m[0] + m[1] + m[2] + m[3];
    const uint64_t inc = wave_incl_scan_u64(ms);
    // a * 2^32 < p32 Z  <=>  a < ceil(p32 Z / 2^32)
    const llima_u128 PZ = (llima_u128)p32 * readlane63(inc);
    const uint64_t lim = (uint64_t)((PZ + 0xFFFFFFFFull) >> 32);
    uint64_t a = inc - ms;                           // mass of the bins before this lane's
    int qb = -1;
    uint64_t qa = 0;
    uint32_t qc = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const bool q = cn[i] > 0u && a < lim;
        qb = q ? (int)(4u * lane) + i : qb;
        qa = q ? a : qa;
        qc = q ? cn[i] : qc;
        a += m[i];
    }
    const uint64_t bq = ballot(qb >= 0);
    if (bq == 0) return kmax;                        // none qualifies (p32 Z < 2^32)
    const uint32_t L = 63u - (uint32_t)__builtin_clzll(bq);
    const uint32_t bstar = (uint32_t)readlane((uint32_t)qb, L), nb = readlane(qc, L);
    const uint64_t above = readlane64(qa, L);
    if (nb > 64u) return 0u;                         // uniform: every wave read the same bins
    // the boundary bin's members -> sh.sv[0, nb): one atomic per thread
    uint32_t mine = 0;
#pragma unroll
    for (int j = 0; j < EPT; ++j) mine += bn[j] == bstar ? 1u : 0u;
    if (mine) {
        uint32_t o = atomicAdd(&sh.lcount, mine);
#pragma unroll
        for (int j = 0; j < EPT; ++j)
            if (bn[j] == bstar) sh.sv[o++] = llima_u32x4{key[j], 0u, (uint32_t)w[j], (uint32_t)(w[j] >> 32)};
    }
    __syncthreads();
    const llima_u32x4 me = lane < nb ? sh.sv[lane] : llima_u32x4{0u, 0u, 0u, 0u};
    uint64_t ab = above;
    for (uint32_t i = 0; i < nb; ++i) {
        const llima_u32x4 o = sh.sv[i];
        ab += o.x > me.x ? (((uint64_t)o.w << 32) | o.z) : 0ull;
    }
    const bool q = lane < nb && ab < lim;
    // the top member always qualifies (its mass above is the bin's); the
    // boundary is the smallest qualifying key
    return ~wave_max_u32(q ? ~me.x : 0u);
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

// ------------------------------------------------------------------ value bins
// Used by the full-row path and the dense path: bins of 1/16 nat below the
// row maximum, exact weights in their float form.
#define SMP_DBINS 448                              // value bins, 1/16 nat (28 nats; the last open)
#define SMP_DBIN_SCALE 16.0f

// 16 (xmax - x) clamped to the last bin, 0 at x == xmax (also when both are
// +inf): the value bin of x (x <= xmax, not NaN) is its integral part, so
// bin < b exactly when it is below b, and bin == b when it lies in [b, b + 1).
__device__ __forceinline__ float dense_d16(float x, float xmax) {
    return x == xmax ? 0.0f : __builtin_fminf((xmax - x) * SMP_DBIN_SCALE, (float)(SMP_DBINS - 1));
}

// weight(x, xmax) as an integral float: weight_f, and 2^36 at x == xmax also
// when the maximum is +inf (every other value then weighs 0, as weight_f's
// clamp at -26 gives).
__device__ __forceinline__ float dense_wf(float x, float xmax) {
    return weight_fd(x == xmax ? 0.0f : x - xmax);      // a select, not a branch per value
}

// The min-p threshold frac32(m) 2^4 rounded up to a float: an integral float
// weight W has W >= threshold exactly when W >= this.
__device__ __forceinline__ float dense_mthr(const RowCfg& c) {
    const uint64_t m = c.m > 0.0f ? frac32(c.m) << 4 : 0ull;
    float f = (float)m;
    if (f32_integral_to_u64(f) < m) f = __uint_as_float(__float_as_uint(f) + 1u);
    return f;
}

// ------------------------------------------------------------------ full-row path
#define SMP_FE 16                                  // values per thread per full-row step
#define SMP_FRMCAP 1024                            // boundary-bin members the full-row path ranks

// SMP_FE consecutive values from id i0 of a row, ids at or past hi (a multiple
// of the values per 16-byte load when vec) read from clamped addresses: 16-byte
// loads when vec (the row 16-byte aligned), else one value per load, every
// load issued before the first value is used.
template <typename TL>
__device__ __forceinline__ void load_fe(const TL* rowp, int i0, int hi, bool vec, float (&xs)[SMP_FE]) {
    constexpr int EPL = 16 / sizeof(TL);             // values per 16-byte load
    if (vec) {
        llima_u32x4 q[SMP_FE / EPL];
#pragma unroll
        for (int j = 0; j < SMP_FE / EPL; ++j) {
            const int ia = i0 + j * EPL < hi ? i0 + j * EPL : hi - EPL;
            q[j] = *(const llima_u32x4*)(rowp + ia);
        }
#pragma unroll
        for (int j = 0; j < SMP_FE / EPL; ++j) {
            const uint32_t w4[4] = {q[j].x, q[j].y, q[j].z, q[j].w};
#pragma unroll
            for (int e = 0; e < EPL; ++e) {
                if constexpr (sizeof(TL) == 4) xs[j * EPL + e] = __uint_as_float(w4[e]);
                else xs[j * EPL + e] = __uint_as_float((e & 1) ? (w4[e >> 1] & 0xFFFF0000u) : (w4[e >> 1] << 16));
            }
        }
    } else {
#pragma unroll
        for (int e = 0; e < SMP_FE; ++e) xs[e] = load_one<TL>(rowp, i0 + e < hi ? i0 + e : hi - 1);
    }
}
// The full-row path's step: FE consecutive ids per thread (16-byte loads when
// the rows allow), NB steps in flight per thread.
template <typename TL>
struct FrGeom {
    static constexpr int EPL = 16 / (int)sizeof(TL);   // values per 16-byte load
    static constexpr int FE = 16;                      // ids per thread and step
    static constexpr int NL = FE / EPL;                // 16-byte loads per thread and step
    static constexpr int STEP = LLIMA_WG * FE;         // 4096 ids
    static constexpr int NB = 2;                       // steps in flight
    static constexpr int CHUNK = LLIMA_WG * 64 / (int)sizeof(TL);   // the sweep's chunk
};
static_assert(SMP_SEG % FrGeom<float>::STEP == 0 && SMP_SEG % FrGeom<uint16_t>::STEP == 0,
              "full-row steps tile a segment");

// Requests FE consecutive values from id i0 (ids at or past V from clamped
// addresses; V a multiple of EPL when VEC), packed as they lie in memory.  VEC
// is a template argument so that every path issues the same loads: the
// compiler's wait counts then let later steps' loads stay in flight.
template <typename TL, bool VEC>
__device__ __forceinline__ void fr_issue(const TL* rowp, int i0, int V, llima_u32x4 (&q)[FrGeom<TL>::NL]) {
    constexpr int EPL = FrGeom<TL>::EPL;
    if constexpr (VEC) {
#pragma unroll
        for (int j = 0; j < FrGeom<TL>::NL; ++j) {
            const int ia = i0 + j * EPL < V ? i0 + j * EPL : V - EPL;
            q[j] = *(const llima_u32x4*)(rowp + ia);
        }
    } else {
#pragma unroll
        for (int j = 0; j < FrGeom<TL>::NL; ++j) {
            uint32_t w[4] = {0, 0, 0, 0};
#pragma unroll
            for (int e = 0; e < EPL; ++e) {
                const int ia = i0 + j * EPL + e < V ? i0 + j * EPL + e : V - 1;
                const float f = load_one<TL>(rowp, ia);
                if constexpr (sizeof(TL) == 4) w[e] = __float_as_uint(f);
                else w[e >> 1] |= (__float_as_uint(f) >> 16) << ((e & 1) * 16);
            }
            q[j] = llima_u32x4{w[0], w[1], w[2], w[3]};
        }
    }
}

// Value e of a step fr_issue requested.
template <typename TL>
__device__ __forceinline__ float fr_value(const llima_u32x4 (&q)[FrGeom<TL>::NL], int e) {
    constexpr int EPL = FrGeom<TL>::EPL;
    const llima_u32x4 v = q[e / EPL];
    const int d = sizeof(TL) == 4 ? e % 4 : (e % EPL) / 2;
    const uint32_t w = d == 0 ? v.x : d == 1 ? v.y : d == 2 ? v.z : v.w;
    if constexpr (sizeof(TL) == 4) return __uint_as_float(w);
    else return __uint_as_float((e & 1) ? (w & 0xFFFF0000u) : (w << 16));
}

// The value transform of one step, ids from i0 (NaN -> -inf, mask, penalties,
// / T unless greedy; ids past the row -inf); lo: the segment table's first id.
template <typename TL, bool PEN>
__device__ __forceinline__ void fr_transform(const SampleParams& P, const RowCfg& c,
                                             const llima_u32x4 (&qq)[FrGeom<TL>::NL], uint32_t m,
                                             const uint32_t* mrow, int i0, int lo, const uint32_t* table,
                                             float (&x)[FrGeom<TL>::FE]) {
#pragma unroll
    for (int e = 0; e < FrGeom<TL>::FE; ++e) {
        const int i = i0 + e;
        float l = i < P.V ? fr_value<TL>(qq, e) : -__builtin_inff();
        if (l != l) l = -__builtin_inff();
        if (mrow && !((m >> (i & 31)) & 1u)) l = -__builtin_inff();
        if (PEN && i < P.V) {
            const uint32_t cnt = table_count(table, (uint32_t)(i - lo));
            if (cnt) l = penalize(l, cnt, c);
        }
        x[e] = l;
    }
    if (!c.greedy && c.T != 1.0f) {
#pragma unroll
        for (int e = 0; e < FrGeom<TL>::FE; ++e) x[e] = x[e] / c.T;
    }
}

// Streams steps [s_begin, s_end) of a row through fn(x, i0): x[e] is the value
// of id i0 + e after the row's transform (NaN -> -inf, mask, penalties, / T
// unless greedy; -inf past the row), a whole step's values at once so that
// fn can work on them without a branch per value; step_end(s, x, i0) after
// it, with the same values: step s
// covers the FrGeom::STEP ids from step_base(s) (a multiple of FrGeom::FE),
// thread t taking FE consecutive ids (within one mask word).  The loads of step
// s + NB - 1 are requested before step s is worked on, so NB steps (64 KB of
// fp32 per workgroup) are in flight instead of one; barriers do not wait for
// outstanding global loads.  step_end(s) is called by every thread after step
// s.  table holds the history counts of the SMP_SEG segment in use (rows with
// penalties), rebuilt when a step enters another segment.
template <typename TL, int NB, bool VEC, bool PEN, class Base, class Fn, class StepEnd>
__device__ __forceinline__ void fr_stream(const SampleParams& P, int row, const RowCfg& c, uint32_t* table,
                                          int s_begin, int s_end, Base step_base, Fn fn, StepEnd step_end) {
    using FG = FrGeom<TL>;
    if (s_end <= s_begin) {                                   // uniform
        __syncthreads();
        return;
    }
    const TL* rowp = (const TL*)P.logits + (size_t)row * P.row_stride;
    const int V = P.V;
    const uint32_t* mrow = P.bitmask ? P.bitmask + (size_t)row * ((V + 31) >> 5) : nullptr;
    // the mask word is loaded on every row (from the uniforms when there is no
    // mask) so that every step issues the same loads
    const uint32_t* mload = mrow ? mrow : (const uint32_t*)P.uniforms;
    const int mlast = mrow ? (V - 1) >> 5 : 0;
    int seg = -1;                                             // the segment table holds
    llima_u32x4 q[NB][FG::NL];
    uint32_t mw[NB] = {};
    auto issue = [&](llima_u32x4 (&qq)[FG::NL], uint32_t& m, int s) __attribute__((always_inline)) {
        // past the range: the last step again (cache hits, no new traffic)
        const int i0 = step_base(s < s_end ? s : s_end - 1) + (int)threadIdx.x * FG::FE;
        const int mi = i0 >> 5;
        m = mload[mi < mlast ? mi : mlast];
        fr_issue<TL, VEC>(rowp, i0, V, qq);
    };
    auto work = [&](const llima_u32x4 (&qq)[FG::NL], uint32_t m, int s) __attribute__((always_inline)) {
        const int base = step_base(s);
        const int lo = base & ~(SMP_SEG - 1);
        if constexpr (PEN) {
            if (lo != seg) {                                  // uniform
                if (seg >= 0) __syncthreads();                // every thread is done with the old table
                count_history(P, row, c.hlen, lo, lo + SMP_SEG < V ? lo + SMP_SEG : V, table, SMP_SEG / 2);
                seg = lo;
            }
        }
        const int i0 = base + (int)threadIdx.x * FG::FE;
        float x[FG::FE];
        fr_transform<TL, PEN>(P, c, qq, m, mrow, i0, lo, table, x);
        fn(x, i0);                                            // ids past the row: -inf
        step_end(s, x, i0);
    };
    // the scheduling barriers keep the loads in step order (waiting for one
    // step's data then waits for no later step's)
#pragma unroll
    for (int b = 0; b < NB - 1; ++b) {
        issue(q[b], mw[b], s_begin + b);
        __builtin_amdgcn_sched_barrier(0);
    }
    // the step loop stays rolled: its body is executed from the instruction
    // cache after the first round (fully unrolled, every step would be code
    // fetched once)
#pragma clang loop unroll(disable)
    for (int s0 = s_begin; s0 < s_end; s0 += NB) {
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            const int nb = (b + NB - 1) % NB;                 // the slot worked on last
            issue(q[nb], mw[nb], s0 + b + NB - 1);
            __builtin_amdgcn_sched_barrier(0);
            if (s0 + b < s_end) work(q[b], mw[b], s0 + b);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    __syncthreads();
}

// fr_stream with the row's load width and penalties as template arguments.
template <typename TL, int NB, class Base, class Fn, class StepEnd>
__device__ __forceinline__ void fr_stream_row(const SampleParams& P, int row, const RowCfg& c, uint32_t* table,
                                              int s_begin, int s_end, Base step_base, Fn fn, StepEnd step_end) {
    if (P.vec_ok) {
        if (c.pen) fr_stream<TL, NB, true, true>(P, row, c, table, s_begin, s_end, step_base, fn, step_end);
        else fr_stream<TL, NB, true, false>(P, row, c, table, s_begin, s_end, step_base, fn, step_end);
    } else {
        if (c.pen) fr_stream<TL, NB, false, true>(P, row, c, table, s_begin, s_end, step_base, fn, step_end);
        else fr_stream<TL, NB, false, false>(P, row, c, table, s_begin, s_end, step_base, fn, step_end);
    }
}

// Exact multi-pass selection by one workgroup; recomputes x for the whole row on
// every pass (history table rebuilt per segment).
template <typename TL>
__device__ __forceinline__ void finish_full_row(const SampleParams& P, int row, const RowCfg& c, FinShared& sh) {
    const TL* rowp = (const TL*)P.logits + (size_t)row * P.row_stride;
    const int V = P.V;
    const int nw = (V + 31) >> 5;
    const uint32_t* mrow = P.bitmask ? P.bitmask + (size_t)row * nw : nullptr;
    uint32_t* table = sh.u.table;
    __syncthreads();
    // Every pass visits the row in steps of LLIMA_WG * SMP_FE ids: thread t
    // takes SMP_FE consecutive ids and requests all of them (16-byte loads when
    // the rows allow) before the first is used, so a step costs one memory
    // round trip instead of one per value.
    const bool vec = P.vec_ok != 0;
    auto for_each_x = [&](auto fn) {
        for (int lo = 0; lo < V; lo += SMP_SEG) {
            const int hi = lo + SMP_SEG < V ? lo + SMP_SEG : V;
            if (c.pen) count_history(P, row, c.hlen, lo, hi, table, SMP_SEG / 2);
            for (int b0 = lo; b0 < hi; b0 += LLIMA_WG * SMP_FE) {
                const int i0 = b0 + (int)threadIdx.x * SMP_FE;
                float xs[SMP_FE];
                load_fe<TL>(rowp, i0, hi, vec, xs);
#pragma unroll
                for (int e = 0; e < SMP_FE; ++e) {
                    const int i = i0 + e;
                    if (i < hi) {
                        float l = xs[e];
                        if (l != l) l = -__builtin_inff();
                        if (mrow && !((mrow[i >> 5] >> (i & 31)) & 1u)) l = -__builtin_inff();
                        if (c.pen) {
                            const uint32_t cnt = table_count(table, (uint32_t)(i - lo));
                            if (cnt) l = penalize(l, cnt, c);
                        }
                        fn(c.greedy ? l : l / c.T, (uint32_t)i);
                    }
                }
            }
            __syncthreads();
        }
    };
    // for_each_x with seg_end(lo) called by every thread after the SMP_SEG ids
    // from lo, before the barrier that ends them.
    auto for_each_x_seg = [&](auto fn, auto seg_end) {
        for (int lo = 0; lo < V; lo += SMP_SEG) {
            const int hi = lo + SMP_SEG < V ? lo + SMP_SEG : V;
            if (c.pen) count_history(P, row, c.hlen, lo, hi, table, SMP_SEG / 2);
            for (int b0 = lo; b0 < hi; b0 += LLIMA_WG * SMP_FE) {
                const int i0 = b0 + (int)threadIdx.x * SMP_FE;
                float xs[SMP_FE];
                load_fe<TL>(rowp, i0, hi, vec, xs);
#pragma unroll
                for (int e = 0; e < SMP_FE; ++e) {
                    const int i = i0 + e;
                    if (i < hi) {
                        float l = xs[e];
                        if (l != l) l = -__builtin_inff();
                        if (mrow && !((mrow[i >> 5] >> (i & 31)) & 1u)) l = -__builtin_inff();
                        if (c.pen) {
                            const uint32_t cnt = table_count(table, (uint32_t)(i - lo));
                            if (cnt) l = penalize(l, cnt, c);
                        }
                        fn(c.greedy ? l : l / c.T, (uint32_t)i);
                    }
                }
            }
            seg_end(lo);
            __syncthreads();
        }
    };
    // Radix select over the row: histogram rounds that visit every element.
    auto radix = [&](auto elem, uint32_t kmin, uint32_t kmax, auto pick) {
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

    // Top-p, min-p and the draw over value bins of 1/16 nat below the maximum.
    // One pass counts the top-k set's mass into the bins: Z, and the bin b*
    // holding the top-p boundary (the last non-empty bin whose mass above,
    // times 2^32, is below p32 Z; the top non-empty bin when none is), which is
    // where the radix rounds below would find it.  A second pass collects b*'s
    // members and each segment's kept mass above b*; the members, ranked from
    // the mass above b*, give theta; the draw scans the one segment that holds
    // its target, in id order.  When b* has more members than the LDS holds,
    // the radix rounds below run instead.
    const uint64_t mthr = c.m > 0.0f ? frac32(c.m) << 4 : 0;
    uint32_t theta = 0;
    int32_t tok = -1;
    float prob = 0.0f;
    bool binned = false;
    auto fin_elem = [&](float x, uint32_t id, auto fn) {
        const uint32_t k = f32_key(x);
        if (k >= tau && k >= theta) {
            const uint64_t w = weight(x, xmax);
            if (w >= mthr) fn(id, w);
        }
    };
    {
        int segw = SMP_SEG;
        while ((V + segw - 1) / segw > LLIMA_WG) segw <<= 1;
        const int nseg = (V + segw - 1) / segw;
        uint64_t* seg = &sh.part[0][0][0];                     // nseg <= LLIMA_WG slots
        uint64_t* mem = (uint64_t*)&sh.sv2[0][0];             // SMP_FRMCAP members
        uint64_t* bins = &sh.hmass[0][0];                     // SMP_DBINS slots
        const uint32_t t = threadIdx.x;
        const bool topp = c.p < 1.0f;
        const float mthr_f = dense_mthr(c);
        uint32_t bstar = SMP_DBINS;
        uint64_t above = 0, Zb = 0;
        if (topp) {
            for (uint32_t i = t; i < SMP_DBINS; i += LLIMA_WG) bins[i] = 0;
            __syncthreads();
            for_each_x([&](float x, uint32_t) {
                if (f32_key(x) >= tau)
                    atomicAdd((unsigned long long*)&bins[(uint32_t)dense_d16(x, xmax)],
                              (unsigned long long)wf_u64(dense_wf(x, xmax)));
            });
            // a bin's mass is 0 only when it is empty or every value in it weighs
            // 0, and such a bin never qualifies (its mass above is Z)
            const uint64_t m0 = t < SMP_DBINS / 2 ? bins[2u * t] : 0ull;
            const uint64_t m1 = t < SMP_DBINS / 2 ? bins[2u * t + 1u] : 0ull;
            const uint64_t ab = block_excl_scan_u64(m0 + m1, &Zb, sh.bs);
            const llima_u128 PZ = (llima_u128)frac32(c.p) * Zb;
            const bool q0 = m0 > 0 && (((llima_u128)ab << 32) < PZ);
            const bool q1 = m1 > 0 && (((llima_u128)(ab + m0) << 32) < PZ);
            const uint32_t qb = block_max_u32(q1 ? 2u * t + 2u : (q0 ? 2u * t + 1u : 0u), sh.bs);
            const uint32_t ne = m0 ? 2u * t : (m1 ? 2u * t + 1u : 0xFFFFFFFFu);
            const uint32_t top = ~block_max_u32(~ne, sh.bs);
            bstar = qb ? qb - 1u : top;
            if ((bstar >> 1) == t) sh.sel64[0] = (bstar & 1u) ? ab + m0 : ab;
            __syncthreads();
            above = sh.sel64[0];
        }
        for (int i = (int)t; i < nseg; i += LLIMA_WG) seg[i] = 0;
        if (t == 0) sh.lcount = 0;
        __syncthreads();
        const float blo = (float)bstar, bhi = (float)bstar + 1.0f;
        uint64_t acc = 0;
        for_each_x_seg(
            [&](float x, uint32_t id) {
                const uint32_t k = f32_key(x);
                if (k >= tau) {
                    const float d16 = dense_d16(x, xmax);
                    if (d16 < blo) {
                        const float wf = dense_wf(x, xmax);
                        if (wf >= mthr_f) acc += wf_u64(wf);
                    } else if (d16 < bhi) {
                        const uint32_t o = atomicAdd(&sh.lcount, 1u);
                        if (o < SMP_FRMCAP) mem[o] = ((uint64_t)k << 32) | id;
                    }
                }
            },
            [&](int lo) {
                const uint64_t v = wave_sum_u64(acc);
                if (lane_id() == 0 && v)
                    atomicAdd((unsigned long long*)&seg[lo / segw], (unsigned long long)v);
                acc = 0;
            });
        const uint32_t nmem = sh.lcount;
        if (nmem <= SMP_FRMCAP && (!topp || nmem > 0)) {         // uniform
            binned = true;
            if (topp) {
                constexpr int EPT = SMP_FRMCAP / LLIMA_WG;
                uint32_t key[EPT], mid[EPT];
                uint64_t w[EPT];
                uint32_t mk = 0, nmk = 0;
#pragma unroll
                for (int e = 0; e < EPT; ++e) {
                    const uint32_t j = t + (uint32_t)e * LLIMA_WG;
                    const uint64_t v = j < nmem ? mem[j] : 0ull;
                    key[e] = (uint32_t)(v >> 32);
                    mid[e] = (uint32_t)v;
                    w[e] = key[e] ? wf_u64(dense_wf(key_f32(key[e]), xmax)) : 0ull;
                    mk = key[e] > mk ? key[e] : mk;
                    nmk = key[e] && ~key[e] > nmk ? ~key[e] : nmk;
                }
                sh.hmass[0][t] = 0;                                // the bins are no longer needed
                sh.hmass[1][t] = 0;
                mk = block_max_u32(mk, sh.bs);
                const uint32_t mkmin = ~block_max_u32(nmk, sh.bs);
                const uint64_t p32 = frac32(c.p);
                theta = fin_topp_desc<EPT>(key, w, p32, mkmin, mk, sh, above, (llima_u128)p32 * Zb, true);
#pragma unroll
                for (int e = 0; e < EPT; ++e)
                    if (key[e] && key[e] >= theta && w[e] >= mthr)
                        atomicAdd((unsigned long long*)&seg[mid[e] / (uint32_t)segw], (unsigned long long)w[e]);
            }
            if (t == 0) {
                sh.sel[0] = 0;
                sh.sel64[0] = 0;
            }
            __syncthreads();
            const uint64_t m = (int)t < nseg ? seg[t] : 0ull;
            uint64_t Zf;
            const uint64_t below = block_excl_scan_u64(m, &Zf, sh.bs);
            if (Zf > 0) {
                const uint64_t target = (uint64_t)(((llima_u128)uniform32(c.u) * Zf) >> 32);
                if (m > 0 && below <= target && target < below + m) {
                    sh.sel[0] = t;
                    sh.sel64[0] = target - below;
                }
                __syncthreads();
                const int sg = (int)sh.sel[0];
                uint64_t rel = sh.sel64[0];
                // the segment in blocks of SMP_SEG ids, each in id order: thread t
                // holds SMP_SEG / LLIMA_WG consecutive ids of the block
                constexpr int EPS = SMP_SEG / LLIMA_WG;
                const int s1 = (sg + 1) * segw < V ? (sg + 1) * segw : V;
                for (int lo = sg * segw; lo < s1; lo += SMP_SEG) {
                    const int hi = lo + SMP_SEG < V ? lo + SMP_SEG : V;
                    if (c.pen) count_history(P, row, c.hlen, lo, hi, table, SMP_SEG / 2);
                    const int i0 = lo + (int)t * EPS;
                    // the kept weight of id i (0 when not kept)
                    auto kept_w = [&](float l, int i) -> uint64_t {
                        if (l != l) l = -__builtin_inff();
                        if (mrow && !((mrow[i >> 5] >> (i & 31)) & 1u)) l = -__builtin_inff();
                        if (c.pen) {
                            const uint32_t cnt = table_count(table, (uint32_t)(i - lo));
                            if (cnt) l = penalize(l, cnt, c);
                        }
                        const float x = l / c.T;
                        const uint32_t k = f32_key(x);
                        if (!(k >= tau && k >= theta)) return 0ull;
                        const float wf = dense_wf(x, xmax);
                        return wf >= mthr_f ? wf_u64(wf) : 0ull;
                    };
                    uint64_t sum = 0;
                    for (int g = 0; g < EPS; g += SMP_FE) {
                        float xs[SMP_FE];
                        load_fe<TL>(rowp, i0 + g, hi, vec, xs);   // ids past hi: clamped addresses
#pragma unroll
                        for (int e = 0; e < SMP_FE; ++e)
                            if (i0 + g + e < hi) sum += kept_w(xs[e], i0 + g + e);
                    }
                    uint64_t tot;
                    const uint64_t bl = block_excl_scan_u64(sum, &tot, sh.bs);
                    if (rel < tot) {                                   // uniform
                        if (sum > 0 && bl <= rel && rel < bl + sum) {
                            uint64_t a = bl, wtok = 0;
                            for (int g = 0; g < EPS; g += SMP_FE) {
                                float xs[SMP_FE];
                                load_fe<TL>(rowp, i0 + g, hi, vec, xs);
#pragma unroll
                                for (int e = 0; e < SMP_FE; ++e) {
                                    const int i = i0 + g + e;
                                    const uint64_t w = i < hi ? kept_w(xs[e], i) : 0ull;
                                    const bool hit = tok < 0 && w > 0 && rel < a + w;
                                    tok = hit ? i : tok;
                                    wtok = hit ? w : wtok;
                                    a += w;
                                }
                            }
                            prob = (float)((double)wtok / (double)Zf);
                            write_result(P, row, tok, prob);
                        }
                        break;
                    }
                    rel -= tot;
                    __syncthreads();
                }
            } else if (t == 0) {
                write_result(P, row, -1, 0.0f);
            }
        }
    }
    if (!binned) {
        // radix rounds over the keys: theta, then the draw over the ids
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
        uint64_t Zf = 0;
        for_each_x([&](float x, uint32_t id) { fin_elem(x, id, [&](uint32_t, uint64_t w) { Zf += w; }); });
        Zf = block_sum_u64(Zf, sh.bs);
        if (Zf > 0) {
            const uint64_t target = (uint64_t)(((llima_u128)uniform32(c.u) * Zf) >> 32);
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
    }
    if (P.out_keep)
        write_keep(P, row, [&](auto set) {
            for_each_x([&](float x, uint32_t id) { fin_elem(x, id, [&](uint32_t i, uint64_t) { set(i); }); });
        });
}

// ------------------------------------------------------------------ split rows
// Rows without top-k whose candidates overflow the sweep's regions (ordinary
// logits under top-p alone, or a grammar mask that allows much of the row) in
// a batch whose other rows keep the two-launch path (per-row settings, or a
// mask): sample_finish then runs with P.fsplit workgroups per row, and such a
// row is binned by all of them in parallel instead of by one workgroup's
// full-row passes.  Part f takes chunks [f P.rcpw, (f + 1) P.rcpw): every
// value's exact weight into the full-row path's SMP_DBINS value bins below the
// row maximum (fl(max M / T) from the sweep's headers), written per chunk to
// the chunk's region as the mass above each bin and the bin's count, with the
// chunk's mass and the first bin holding a value below the min-p threshold.
// The stores are write-through (agent scope) and complete before the part is
// counted on the row's arrival counter; the last part to arrive reads them
// back (agent-scope loads miss stale lines) and finishes the row: the
// boundary bin bb (the top-p boundary bin b* or the min-p bin, the higher of
// the two), the members of bb from a pass over the chunks holding any, theta
// among them, each chunk's kept mass, the chunk of the draw target and a scan
// of it in id order.  Every weight, bin and test is the full-row path's, so
// the kept set, the token and its probability are the same; a row whose
// boundary bin holds more than SMP_FRMCAP values takes the full-row path.
//
// Region use (slot 0, the sweep's header, is kept; the candidate slots are
// not read on such rows):
//   SMP_RCUM + b, b < SMP_DBINS  (mass of the chunk above bin b) << 14 | count of b
//   SMP_RCUM + SMP_DBINS         the chunk's mass << 14
//   SMP_RBMF                     the chunk's first bin with a value below min-p
//   SMP_RSTGI, SMP_RSTG          staged values: every value of the chunk in bins
//                                [lo, hi] (at most P.scap <= SMP_STG_CAP: the
//                                first SMP_RSTG_CAP here, the rest in the
//                                chunk's SMP_XSTG slots after the regions); the last
//                                part reads a chunk again only when the row's
//                                boundary bin lies outside the window
// The window: the part's own chunks (those binned so far, for fp32) give an
// estimate bh of the row's boundary bin.  The row's mass is dominated by its
// highest values, so bh misses both ways; when the chunk's highest bins
// [0, hi] that fit the staging reach bh, they are the window, else the widest
// [bh - 4w, bh + w] that fits (the miss is more often upward).
#define SMP_RCUM 1
#define SMP_RBMF (SMP_RCUM + SMP_DBINS + 1)
#define SMP_RSTGI (SMP_RBMF + 1)                   // staged bins lo | hi << 16 | count << 32
#define SMP_RSTG (SMP_RSTGI + 1)                   // staged values (key << 32 | id)
#define SMP_RSTG_CAP (SMP_REGION - SMP_RSTG)       // 60
#define SMP_STG_CAP (SMP_RSTG_CAP + SMP_XSTG)      // 188
#define SMP_RCPW 4                                 // chunks per part, at most
static_assert(SMP_RBMF < SMP_REGION, "split-row region layout");
static_assert(SMP_STG_CAP <= 192, "a wave reads a chunk's staging in three loads per lane");

// Staged value j of a chunk: in its region, then beyond the regions.
__device__ __forceinline__ uint64_t* stg_slot(const SampleParams& P, uint32_t row, uint32_t chunk, uint32_t j) {
    return j < SMP_RSTG_CAP ? region_of(P, row, chunk) + SMP_RSTG + j
                            : P.xstg + ((size_t)row * (uint32_t)P.S + chunk) * SMP_XSTG + (j - SMP_RSTG_CAP);
}

// Whether the row is split (every part of it decides alike, from the sweep's
// headers): no top-k, not greedy, a finite T, a region that overflowed or
// more candidates than the finish gathers, and a value above -inf.  Returns
// the row's maximum key, or 0.
__device__ __forceinline__ uint32_t split_row(const SampleParams& P, int row, const RowCfg& c, FinShared& sh) {
    if (P.fsplit <= 1 || c.greedy || c.k > 0 || !(c.T < __builtin_inff()) || P.S > SMP_MAX_S) return 0u;
    const uint32_t t = threadIdx.x;
    uint32_t ov = 0, cnt = 0, mk = 0;
    if ((int)t < P.S) {
        const uint64_t h = *region_of(P, (uint32_t)row, t);
        const uint32_t lo = (uint32_t)h;
        ov = (lo >> 16) & HF_OVERFLOW;
        cnt = ov ? 0u : (lo & 0xFFFFu);
        const float M = __uint_as_float((uint32_t)(h >> 32));
        mk = M > -__builtin_inff() ? f32_key(M / c.T) : 0u;
    }
    ov = block_max_u32(ov, sh.bs);
    cnt = block_sum_u32(cnt, sh.bs);
    mk = block_max_u32(mk, sh.bs);
    return ((ov != 0u || cnt > SMP_FIN_CAP) && mk > LLIMA_KEY_NEG_INF) ? mk : 0u;
}

// The last part of a split row to arrive: the chunks' bins merged, the
// boundary, its members, theta, the kept masses and the draw.
template <typename TL>
__device__ __forceinline__ void split_final(const SampleParams& P, int row, const RowCfg& c, uint32_t kmax, FinShared& sh) {
    using FG = FrGeom<TL>;
    constexpr int CV = FG::CHUNK;
    constexpr int SPC = CV / FG::STEP;
    const int S = P.S, V = P.V;
    const uint32_t t = threadIdx.x;
    const float xmax = key_f32(kmax);
    uint64_t* r0 = region_of(P, (uint32_t)row, 0);
    // ---- the chunks merged: mass above bins 2t and 2t + 1 and their counts;
    //      Z; the first bin below min-p
    uint64_t a0 = 0, a1 = 0;
    uint32_t n0 = 0, n1 = 0;
    if (t < SMP_DBINS / 2) {
        constexpr int NB = 20;                               // 38 chunks: two rounds
        for (int b0 = 0; b0 < S; b0 += NB) {
            uint64_t v0[NB], v1[NB];
#pragma unroll
            for (int i = 0; i < NB; ++i) {
                const int ci = b0 + i < S ? b0 + i : S - 1;
                uint64_t* q = r0 + (size_t)ci * SMP_REGION + SMP_RCUM + 2u * t;
                v0[i] = load_agent(q);
                v1[i] = load_agent(q + 1);
            }
#pragma unroll
            for (int i = 0; i < NB; ++i) {
                const bool in = b0 + i < S;
                a0 += in ? v0[i] >> 14 : 0ull;
                n0 += in ? (uint32_t)(v0[i] & 0x3FFFu) : 0u;
                a1 += in ? v1[i] >> 14 : 0ull;
                n1 += in ? (uint32_t)(v1[i] & 0x3FFFu) : 0u;
            }
        }
    }
    uint64_t zc = 0;
    uint32_t bmc = SMP_DBINS;
    if ((int)t < S) {
        uint64_t* reg = r0 + (size_t)t * SMP_REGION;
        zc = load_agent(reg + SMP_RCUM + SMP_DBINS) >> 14;
        bmc = (uint32_t)load_agent(reg + SMP_RBMF);
    }
    const uint64_t Z = block_sum_u64(zc, sh.bs);
    const uint32_t bmf = ~block_max_u32(~bmc, sh.bs);
    FIN_MARK_ANY(8);
    // ---- the top-p boundary bin b*: the last non-empty bin whose mass above,
    //      times 2^32, is below p32 Z; the top non-empty bin when none is
    const bool topp = c.p < 1.0f;
    uint32_t bstar = SMP_DBINS;
    if (topp) {                                              // uniform
        const llima_u128 PZ = (llima_u128)frac32(c.p) * Z;
        const bool q0 = n0 > 0u && (((llima_u128)a0 << 32) < PZ);
        const bool q1 = n1 > 0u && (((llima_u128)a1 << 32) < PZ);
        const uint32_t qb = block_max_u32(q1 ? 2u * t + 2u : (q0 ? 2u * t + 1u : 0u), sh.bs);
        const uint32_t ne = n0 ? 2u * t : (n1 ? 2u * t + 1u : 0xFFFFFFFFu);
        const uint32_t top = ~block_max_u32(~ne, sh.bs);
        bstar = qb ? qb - 1u : top;
    }
    // the boundary: values in bins below bb are kept, above it not
    const uint32_t bb = bstar < bmf ? bstar : bmf;
    if ((bb >> 1) == t) sh.sel64[0] = (bb & 1u) ? a1 : a0;   // mass above bb (when bb < SMP_DBINS)
    // ---- each chunk's mass above bb and its members of bb: from the chunk's
    //      staging when bb lies in its window, else from a read of the chunk
    uint64_t* kc = &sh.part[0][0][0];                        // kept mass per chunk (SMP_MAX_S)
    uint32_t mc = 0, sn = 0;
    bool staged = false;
    if ((int)t < S) {
        uint64_t* reg = r0 + (size_t)t * SMP_REGION;
        const uint64_t v = load_agent(reg + SMP_RCUM + bb);
        const uint64_t si = load_agent(reg + SMP_RSTGI);
        kc[t] = v >> 14;
        mc = bb < SMP_DBINS ? (uint32_t)(v & 0x3FFFu) : 0u;
        const uint32_t lo = (uint32_t)si & 0xFFFFu, hi = ((uint32_t)si >> 16) & 0xFFFFu;
        sn = (uint32_t)(si >> 32);
        staged = mc > 0u && lo <= bb && bb <= hi;
    }
    uint32_t nlist, nstg;
    const uint32_t li = block_excl_scan_u32(mc > 0u && !staged ? 1u : 0u, &nlist, sh.bs);
    if (mc > 0u && !staged) sh.ccount[li] = t;               // the chunks read again
    const uint32_t ls = block_excl_scan_u32(staged ? 1u : 0u, &nstg, sh.bs);
    if (staged) sh.coff[ls] = t | (sn << 16);                // the chunks whose staging holds them
    const uint32_t nm = block_sum_u32(mc, sh.bs);            // its barriers publish the lists
    const uint64_t above = sh.sel64[0];
    FIN_MARK_ANY(9);
    if (nm > SMP_FRMCAP) {                                   // uniform: a nearly flat row
        finish_full_row<TL>(P, row, c, sh);
        return;
    }
    // ---- the members of bb: from the staging (a wave per chunk), then a pass
    //      over the chunks whose staging does not hold them
    uint64_t* mem = (uint64_t*)&sh.sv2[0][0];                // SMP_FRMCAP members
    if (t == 0) sh.lcount = 0;
    __syncthreads();
    const uint32_t lane = lane_id();
    // a wave takes chunks k, k + 4, k + 8 per round: their staging (three
    // slots per lane each) requested together, one memory wait per round
    constexpr int SQ = 3;
    for (uint32_t k0 = wave_id(); k0 < nstg; k0 += SQ * LLIMA_WAVES) {
        uint64_t v[SQ][3];
        uint32_t ns[SQ];
#pragma unroll
        for (int q = 0; q < SQ; ++q) {
            const uint32_t k = k0 + (uint32_t)q * LLIMA_WAVES;
            const uint32_t e = k < nstg ? sh.coff[k] : 0u;
            const uint32_t ch = e & 0xFFFFu;
            ns[q] = e >> 16;
#pragma unroll
            for (int h = 0; h < 3; ++h) {
                const uint32_t j = lane + 64u * (uint32_t)h;
                v[q][h] = j < ns[q] ? load_agent(stg_slot(P, (uint32_t)row, ch, j)) : 0ull;
            }
        }
#pragma unroll
        for (int q = 0; q < SQ; ++q) {
            bool m[3];
            uint32_t nmh = 0;
#pragma unroll
            for (int h = 0; h < 3; ++h) {
                m[h] = lane + 64u * (uint32_t)h < ns[q] &&
                       (uint32_t)dense_d16(key_f32((uint32_t)(v[q][h] >> 32)), xmax) == bb;
                nmh += m[h] ? 1u : 0u;
            }
            if (nmh) {
                uint32_t o = atomicAdd(&sh.lcount, nmh);
#pragma unroll
                for (int h = 0; h < 3; ++h)
                    if (m[h]) {
                        if (o < SMP_FRMCAP) mem[o] = v[q][h];
                        ++o;
                    }
            }
        }
    }
    auto listed = [&](int s) { return (int)sh.ccount[s / SPC] * CV + (s % SPC) * FG::STEP; };
    auto member = [&](const float (&x)[FG::FE], int i0) {
        uint32_t hm = 0;
#pragma unroll
        for (int e = 0; e < FG::FE; ++e)
            hm |= x[e] > -__builtin_inff() && (uint32_t)dense_d16(x[e], xmax) == bb ? 1u << e : 0u;
        const uint32_t n = (uint32_t)__popc(hm);
        if (ballot(n != 0u)) {                               // uniform in the wave
            const uint32_t inc = wave_incl_scan_u32(n);
            uint32_t base = 0;
            if (lane == 63) base = atomicAdd(&sh.lcount, inc);
            uint32_t o = readlane(base, 63) + inc - n;
            while (hm) {
                const int e = __builtin_ctz(hm);
                hm &= hm - 1u;
                if (o < SMP_FRMCAP) mem[o] = ((uint64_t)f32_key(x[e]) << 32) | (uint32_t)(i0 + e);
                ++o;
            }
        }
    };
    fr_stream_row<TL, FG::NB>(P, row, c, sh.u.table, 0, (int)nlist * SPC, listed, member, [](int, const auto&, int) {});
    if (sh.lcount != nm) {                                   // uniform: never (the counts are the bins')
        finish_full_row<TL>(P, row, c, sh);
        return;
    }
    const uint32_t nmem = nm;
    FIN_MARK_ANY(10);
    // ---- theta among the members (top-p boundary), the kept members' weights
    //      added to their chunks
    constexpr int EPT = SMP_FRMCAP / LLIMA_WG;
    uint32_t key[EPT], mid[EPT];
    uint64_t w[EPT];
    uint32_t mk = 0, nmk = 0;
#pragma unroll
    for (int e = 0; e < EPT; ++e) {
        const uint32_t j = t + (uint32_t)e * LLIMA_WG;
        const uint64_t v = j < nmem ? mem[j] : 0ull;
        key[e] = (uint32_t)(v >> 32);
        mid[e] = (uint32_t)v;
        w[e] = key[e] ? wf_u64(dense_wf(key_f32(key[e]), xmax)) : 0ull;
        mk = key[e] > mk ? key[e] : mk;
        nmk = key[e] && ~key[e] > nmk ? ~key[e] : nmk;
    }
    uint32_t theta = 0;
    if (topp && bb == bstar && nmem > 0u) {                  // uniform
        sh.hmass[0][t] = 0;
        sh.hmass[1][t] = 0;
        mk = block_max_u32(mk, sh.bs);
        const uint32_t mkmin = ~block_max_u32(nmk, sh.bs);
        const uint64_t p32 = frac32(c.p);
        theta = fin_topp_desc<EPT>(key, w, p32, mkmin, mk, sh, above, (llima_u128)p32 * Z, true);
    }
    const uint64_t mthr = c.m > 0.0f ? frac32(c.m) << 4 : 0ull;
    const bool tb = bb == bstar, mb = bb == bmf;
#pragma unroll
    for (int e = 0; e < EPT; ++e)
        if (key[e] && (!tb || key[e] >= theta) && (!mb || w[e] >= mthr))
            atomicAdd((unsigned long long*)&kc[mid[e] / (uint32_t)CV], (unsigned long long)w[e]);
    if (t == 0) {             // overwritten by the thread whose chunk holds the target
        sh.sel[0] = 0;
        sh.sel64[1] = 0;
    }
    __syncthreads();
    FIN_MARK_ANY(11);
    // ---- the chunk of the draw target, then that chunk in id order
    const uint64_t m = (int)t < S ? kc[t] : 0ull;
    uint64_t Zf;
    const uint64_t below = block_excl_scan_u64(m, &Zf, sh.bs);
    if (Zf == 0) {
        if (t == 0) write_result(P, row, -1, 0.0f);
        return;
    }
    const uint64_t target = (uint64_t)(((llima_u128)uniform32(c.u) * Zf) >> 32);
    if (m > 0 && below <= target && target < below + m) {
        sh.sel[0] = t;
        sh.sel64[1] = target - below;
    }
    __syncthreads();
    const int cs = (int)sh.sel[0];
    uint64_t rel = sh.sel64[1];
    const float mthr_f = dense_mthr(c);
    const TL* rowp = (const TL*)P.logits + (size_t)row * P.row_stride;
    const uint32_t* mrow = P.bitmask ? P.bitmask + (size_t)row * ((V + 31) >> 5) : nullptr;
    const int c0 = cs * CV;
    const int lo = c0 & ~(SMP_SEG - 1);
    llima_u32x4 qd[SPC][FG::NL];
    uint32_t mw[SPC] = {};
#pragma unroll
    for (int j = 0; j < SPC; ++j) {
        const int i0 = c0 + j * FG::STEP + (int)t * FG::FE;
        if (mrow) mw[j] = mrow[(i0 < V ? i0 : V - 1) >> 5];
        if (P.vec_ok) fr_issue<TL, true>(rowp, i0, V, qd[j]);
        else fr_issue<TL, false>(rowp, i0, V, qd[j]);
    }
    if (c.pen) count_history(P, row, c.hlen, lo, lo + SMP_SEG < V ? lo + SMP_SEG : V, sh.u.table, SMP_SEG / 2);
    const float blo = (float)bb;
#pragma unroll
    for (int j = 0; j < SPC; ++j) {
        const int i0 = c0 + j * FG::STEP + (int)t * FG::FE;
        float x[FG::FE];
        if (c.pen) fr_transform<TL, true>(P, c, qd[j], mw[j], mrow, i0, lo, sh.u.table, x);
        else fr_transform<TL, false>(P, c, qd[j], mw[j], mrow, i0, lo, sh.u.table, x);
        uint64_t wv[FG::FE], sum = 0;
#pragma unroll
        for (int e = 0; e < FG::FE; ++e) {
            uint64_t we = 0;
            if (i0 + e < V && x[e] > -__builtin_inff()) {
                const float d16 = dense_d16(x[e], xmax);
                const float wf = dense_wf(x[e], xmax);
                const bool kept = d16 < blo ||
                                  ((uint32_t)d16 == bb && (!tb || f32_key(x[e]) >= theta) && (!mb || wf >= mthr_f));
                we = kept ? wf_u64(wf) : 0ull;
            }
            wv[e] = we;
            sum += we;
        }
        uint64_t tot;
        const uint64_t bl = block_excl_scan_u64(sum, &tot, sh.bs);
        if (rel < tot) {                                     // uniform
            if (sum > 0 && bl <= rel && rel < bl + sum) {
                uint64_t a = bl, wtok = 0;
                int32_t tok = -1;
#pragma unroll
                for (int e = 0; e < FG::FE; ++e) {
                    const bool hit = tok < 0 && wv[e] > 0 && rel < a + wv[e];
                    tok = hit ? i0 + e : tok;
                    wtok = hit ? wv[e] : wtok;
                    a += wv[e];
                }
                write_result(P, row, tok, (float)((double)wtok / (double)Zf));
            }
            FIN_MARK_ANY(12);
            return;
        }
        rel -= tot;
    }
}

// Part `part` of a split row: its chunks' bins (kept in LDS); the staging of
// each chunk's values in a window chosen for the boundary bin that the part's
// own chunks give (fp32: at each chunk's end, from the chunks binned so far,
// while the chunk's values are in registers; bf16: after the pass, from all of
// them, by a second read of the chunks from the cache); the cumulative bins
// and staging written to the workspace (a wave per chunk), then the arrival;
// the last part finishes the row.
template <typename TL>
__device__ __forceinline__ void split_part(const SampleParams& P, int row, const RowCfg& c, uint32_t kmax,
                                           int part, FinShared& sh) {
    using FG = FrGeom<TL>;
    constexpr int CV = FG::CHUNK;
    constexpr int SPC = CV / FG::STEP;                       // steps per chunk
    static_assert(SPC * FG::STEP == CV, "steps tile a chunk");
    static_assert(SMP_SEG / 2 * sizeof(uint32_t) + (SMP_RCPW * SMP_DBINS + 64) * sizeof(uint64_t) <=
                      sizeof(FinShared::u),
                  "the part's chunk bins fit beside the history table");
    static_assert(SMP_RCPW <= LLIMA_WAVES, "one wave per chunk of a part");
    const int S = P.S;
    const int ch0 = part * P.rcpw, ch1 = ch0 + P.rcpw < S ? ch0 + P.rcpw : S;
    const int nch = ch1 - ch0;
    const float xmax = key_f32(kmax);
    const float mthr_f = dense_mthr(c);
    const uint32_t t = threadIdx.x, lane = lane_id(), wave = wave_id();
    // [SMP_RCPW][SMP_DBINS] chunk bins, then a spare bin per lane (-inf values)
    uint64_t* cb = (uint64_t*)(sh.u.table + SMP_SEG / 2);
    for (uint32_t i = t; i < (uint32_t)nch * SMP_DBINS; i += LLIMA_WG) cb[i] = 0;
    // staged values gather in LDS (a global store inside a pass would make
    // every step wait for all loads), then go to the workspace
    static_assert(SMP_RCPW * SMP_STG_CAP * sizeof(uint64_t) <= sizeof(FinShared::sv2), "staging in LDS");
    uint64_t* stg = (uint64_t*)&sh.sv2[0][0];                // [SMP_RCPW][SMP_STG_CAP]
    uint32_t* bmfc = sh.hcnt[0];                             // per chunk: its first bin below min-p
    if (t < (uint32_t)SMP_RCPW) {
        sh.ccount[t] = 1u;                                   // windows: empty (lo 1, hi 0)
        sh.coff[t] = 0;
        bmfc[t] = SMP_DBINS;
    }
    __syncthreads();
    FIN_MARK(5);
    uint32_t bmf = SMP_DBINS;                                // this thread's, in the current chunk
    static_assert(SMP_DBINS % 64 == 0, "bins tile the lanes");
    constexpr int BPL = SMP_DBINS / 64;                      // bins per lane
    // chunk cl's window (by one wave) for the estimate bbh
    auto window = [&](int cl, uint32_t bbh) {
        if (bbh >= SMP_DBINS) {                              // uniform: no estimate, nothing staged
            if (lane == 0) sh.ccount[cl] = 1u;
            return;
        }
        const uint64_t* bins = cb + (size_t)cl * SMP_DBINS;
        // the highest bins: lane d holds bins [BPL d, BPL d + BPL); the
        // deepest bin hi_top with bins [0, hi_top] fitting (-1: none)
        uint32_t bc[BPL], lsum = 0;
#pragma unroll
        for (int i = 0; i < BPL; ++i) {
            bc[i] = (uint32_t)(bins[BPL * lane + i] & 0x3FFFu);
            lsum += bc[i];
        }
        const uint32_t cum = wave_incl_scan_u32(lsum);
        const uint32_t scap = (uint32_t)P.scap;
        const uint64_t full = ballot(cum <= scap);           // a prefix of the lanes
        const int j = __builtin_popcountll(full);            // the first lane that does not fit
        int hi_top = SMP_DBINS - 1;
        if (j < 64) {                                        // uniform
            uint32_t run = cum - lsum, nf = 0;
#pragma unroll
            for (int i = 0; i < BPL; ++i) {
                run += bc[i];
                nf += run <= scap && nf == (uint32_t)i ? 1u : 0u;
            }
            hi_top = BPL * j + (int)readlane(nf, (uint32_t)j) - 1;
        }
        uint32_t lo, hi;
        if (hi_top >= (int)bbh) {                            // uniform
            lo = 0;
            hi = (uint32_t)hi_top;
        } else {
            // lane w adds bins [bbh - 4w, bbh - 4w + 3] and bbh + w: window
            // w is [bbh - 4w, bbh + w]
            const int b0 = (int)bbh - 4 * (int)lane, bu = (int)bbh + (int)lane;
            uint32_t cnt = 0;
            if (lane == 0) cnt = (uint32_t)(bins[bbh] & 0x3FFFu);
            else {
#pragma unroll
                for (int i = 0; i < 4; ++i) cnt += b0 + i >= 0 ? (uint32_t)(bins[b0 + i] & 0x3FFFu) : 0u;
                cnt += bu < SMP_DBINS ? (uint32_t)(bins[bu] & 0x3FFFu) : 0u;
            }
            const uint32_t inc = wave_incl_scan_u32(cnt);
            const uint64_t fits = ballot(inc <= scap);          // a prefix of the lanes
            const int w = fits ? 63 - __builtin_clzll(fits) : -1;  // the widest window
            lo = w < 0 ? 1u : (uint32_t)((int)bbh - 4 * w > 0 ? (int)bbh - 4 * w : 0);
            hi = w < 0 ? 0u : (uint32_t)((int)bbh + w < SMP_DBINS - 1 ? (int)bbh + w : SMP_DBINS - 1);
        }
        if (lane == 0) sh.ccount[cl] = lo | (hi << 16);
    };
    // by one wave: the boundary bin of the part's chunks [0, ne) (top-p and
    // min-p over their own masses), an estimate of the row's, and chunk cl's
    // window for it
    auto plan = [&](int cl, int ne) {
        uint64_t m[BPL];
        uint32_t n[BPL];
#pragma unroll
        for (int i = 0; i < BPL; ++i) {
            m[i] = 0;
            n[i] = 0;
        }
        uint32_t bbh = SMP_DBINS;
        for (int k = 0; k < ne; ++k) {
            const uint64_t* bins = cb + (size_t)k * SMP_DBINS + BPL * lane;
#pragma unroll
            for (int i = 0; i < BPL; ++i) {
                const uint64_t v = bins[i];
                m[i] += v >> 14;
                n[i] += (uint32_t)(v & 0x3FFFu);
            }
            bbh = bmfc[k] < bbh ? bmfc[k] : bbh;
        }
        if (c.p < 1.0f) {                                    // uniform
            uint64_t lm = 0;
#pragma unroll
            for (int i = 0; i < BPL; ++i) lm += m[i];
            const uint64_t incl = wave_incl_scan_u64(lm);
            const llima_u128 PZ = (llima_u128)frac32(c.p) * readlane63(incl);
            uint64_t above = incl - lm;
            uint32_t qb = 0, top = 0xFFFFFFFFu;
#pragma unroll
            for (int i = 0; i < BPL; ++i) {
                const uint32_t b = BPL * lane + (uint32_t)i;
                qb = n[i] > 0u && ((llima_u128)above << 32) < PZ ? b + 1u : qb;
                top = n[i] > 0u && top == 0xFFFFFFFFu ? b : top;
                above += m[i];
            }
            qb = wave_max_u32(qb);
            top = wave_min_u32(top);
            const uint32_t bhat = qb ? qb - 1u : (top < SMP_DBINS ? top : SMP_DBINS);
            bbh = bhat < bbh ? bhat : bbh;
        }
        window(cl, bbh);
    };
    // one step's values of chunk cl inside window wc to the chunk's staging:
    // a bit mask per thread, one LDS atomic per wave for their places
    auto stage_step = [&](const float (&x)[FG::FE], int i0, uint32_t cl, uint32_t wc) {
        uint32_t hm = 0;
#pragma unroll
        for (int e = 0; e < FG::FE; ++e) {
            const uint32_t b = (uint32_t)dense_d16(x[e], xmax);
            hm |= x[e] > -__builtin_inff() && b >= (wc & 0xFFFFu) && b <= (wc >> 16) ? 1u << e : 0u;
        }
        const uint32_t n = (uint32_t)__popc(hm);
        if (ballot(n != 0u)) {                               // uniform in the wave
            const uint32_t inc = wave_incl_scan_u32(n);
            uint32_t base = 0;
            if (lane == 63) base = atomicAdd(&sh.coff[cl], inc);
            uint32_t o = readlane(base, 63) + inc - n;
            while (hm) {
                const int e = __builtin_ctz(hm);
                hm &= hm - 1u;
                if (o < SMP_STG_CAP) stg[cl * SMP_STG_CAP + o] = ((uint64_t)f32_key(x[e]) << 32) | (uint32_t)(i0 + e);
                ++o;
            }
        }
    };
    auto bin = [&](const float (&x)[FG::FE], int i0) {
        // every weight first (independent chains), then the LDS atomics, -inf
        // values into the lane's spare bin: no branch per value
        const uint32_t cbase = (uint32_t)(i0 / CV - ch0) * SMP_DBINS;
        uint32_t slot[FG::FE];
        uint64_t add[FG::FE];
#pragma unroll
        for (int e = 0; e < FG::FE; ++e) {
            const bool fin = x[e] > -__builtin_inff();
            const float wf = dense_wf(x[e], xmax);
            const uint32_t b = (uint32_t)dense_d16(x[e], xmax);
            slot[e] = fin ? cbase + b : SMP_RCPW * SMP_DBINS + lane;
            add[e] = fin ? (wf_u64(wf) << 14) | 1ull : 0ull;
            bmf = fin && wf < mthr_f && b < bmf ? b : bmf;
        }
#pragma unroll
        for (int e = 0; e < FG::FE; ++e) atomicAdd((unsigned long long*)&cb[slot[e]], (unsigned long long)add[e]);
    };
    auto chunk_end = [&](int s, const float (&x)[FG::FE], int i0) {
        if (s % SPC != SPC - 1) return;                      // uniform: not the chunk's last step
        const int cl = s / SPC - ch0;
        const uint32_t wbm = wave_min_u32(bmf);
        if (lane == 0) atomicMin(&bmfc[cl], wbm);
        bmf = SMP_DBINS;
        if constexpr (SPC == 1) {
            // the chunk's values are this step's, still in registers: its
            // window from the part's chunks binned so far, and the staging now
            __syncthreads();                                 // the chunk's bins are complete
            if (wave == 0) plan(cl, cl + 1);
            __syncthreads();
            const uint32_t wc = sh.ccount[cl];
            if ((wc & 0xFFFFu) <= (wc >> 16)) stage_step(x, i0, (uint32_t)cl, wc);   // uniform
        }
    };
    auto by_step = [](int s) { return s * FG::STEP; };
    fr_stream_row<TL, FG::NB>(P, row, c, sh.u.table, ch0 * SPC, ch1 * SPC, by_step, bin, chunk_end);
    FIN_MARK(6);
    if constexpr (SPC != 1) {
        // chunks of two steps: the estimate from all of the part's chunks,
        // each chunk's window, and a second read of the chunks for the staging
        if ((int)wave < nch) plan((int)wave, nch);
        __syncthreads();
        uint32_t win[SMP_RCPW];
        bool any = false;
#pragma unroll
        for (int cl = 0; cl < SMP_RCPW; ++cl) {
            win[cl] = cl < nch ? sh.ccount[cl] : 1u;
            any = any || (win[cl] & 0xFFFFu) <= (win[cl] >> 16);
        }
        FIN_MARK(13);
        if (any) {                                           // uniform
            auto stage = [&](const float (&x)[FG::FE], int i0) {
                const uint32_t cl = (uint32_t)(i0 / CV - ch0);   // the step lies in one chunk
                uint32_t wc = win[0];
#pragma unroll
                for (int k = 1; k < SMP_RCPW; ++k) wc = cl == (uint32_t)k ? win[k] : wc;
                stage_step(x, i0, cl, wc);
            };
            fr_stream_row<TL, FG::NB>(P, row, c, sh.u.table, ch0 * SPC, ch1 * SPC, by_step, stage,
                                      [](int, const auto&, int) {});
        }
    }
    FIN_MARK(14);
    // each chunk's cumulative bins, first bin below min-p and staging to the
    // workspace, a wave per chunk
    for (int cl = (int)wave; cl < nch; cl += LLIMA_WAVES) {
        const uint32_t ch = (uint32_t)(ch0 + cl);
        uint64_t* reg = region_of(P, (uint32_t)row, ch);
        const uint64_t* bins = cb + (size_t)cl * SMP_DBINS;
        uint64_t above = 0;                                  // the chunk's mass above bin 64 i
#pragma unroll
        for (int i = 0; i < BPL; ++i) {
            const uint64_t v = bins[64 * i + lane];
            const uint64_t mv = v >> 14;
            const uint64_t inc = wave_incl_scan_u64(mv);
            store_agent(reg + SMP_RCUM + 64 * i + lane, ((above + inc - mv) << 14) | (v & 0x3FFFu));
            above += readlane63(inc);
        }
        if (lane == 0) {
            store_agent(reg + SMP_RCUM + SMP_DBINS, above << 14);
            store_agent(reg + SMP_RBMF, (uint64_t)bmfc[cl]);
        }
        const uint32_t n = sh.coff[cl] < SMP_STG_CAP ? sh.coff[cl] : SMP_STG_CAP;
#pragma unroll
        for (uint32_t j = lane; j < SMP_STG_CAP; j += 64u)
            if (j < n) store_agent(stg_slot(P, (uint32_t)row, ch, j), stg[cl * SMP_STG_CAP + j]);
        if (lane == 0) store_agent(reg + SMP_RSTGI, ((uint64_t)n << 32) | sh.ccount[cl]);
    }
    // every store of the part completes before its arrival is counted
    __builtin_amdgcn_s_waitcnt(LLIMA_WAITCNT_VM0);
    __syncthreads();
    FIN_MARK(15);
    if (t == 0) sh.sel[3] = arrive_agent(P.rcnt + (size_t)row * SMP_RCNT, 1u) + 1u == (uint32_t)P.fsplit;
    __syncthreads();
    FIN_MARK(7);
    if (sh.sel[3]) split_final<TL>(P, row, c, kmax, sh);
}

// ------------------------------------------------------------------ small path
// At most 64 NPL candidates, staged in sv[0, ns) as {key, id, w lo, w hi},
// that contain every value of the top-k set (all values >= tau, ties
// included).  Every wave holds all of them (lane l: candidates l and, with
// NPL = 2, l + 64); pairwise passes split over the 4 waves by the candidate
// they read (broadcast LDS reads) rank them: tau is the key of the candidate
// with (above < k <= above + equal), and the top-p test uses the mass strictly
// above.  The draw is a scan when sv is in id order (id_sorted), else a second
// pairwise pass (mass of final ids up to each id).  Returns false, before
// writing anything, when tau does not exceed tcut (a key no value left out of
// sv can reach).
template <int NPL, bool padded>
__device__ __forceinline__ bool fin_small(const SampleParams& P, int row, const RowCfg& c, uint32_t ns,
                          uint32_t kmax, uint32_t tcut, llima_u32x4* sv, bool id_sorted,
                          FinShared& sh) {
    constexpr uint32_t PER = 16u * NPL;              // candidates each wave reads
    const uint32_t lane = lane_id(), wave = wave_id();
    uint32_t key[NPL], id[NPL];
    uint64_t w[NPL];
#pragma unroll
    for (int e = 0; e < NPL; ++e) {
        const uint32_t i = (uint32_t)e * 64u + lane;
        const llima_u32x4 me = i < ns ? sv[i] : llima_u32x4{0u, 0u, 0u, 0u};
        key[e] = me.x; id[e] = me.y;
        w[e] = ((uint64_t)me.w << 32) | me.z;
    }
    const uint32_t j0 = wave * PER;
    uint32_t gt[NPL], eq[NPL];
    uint64_t above[NPL], same[NPL];
#pragma unroll
    for (int e = 0; e < NPL; ++e) { gt[e] = 0; eq[e] = 0; above[e] = 0; same[e] = 0; }
    // every read first (one LDS latency), then the comparisons.  Entries past
    // ns are zero (key 0, weight 0) when padded, and then need no bound check.
    llima_u32x4 ov[PER];
#pragma unroll
    for (uint32_t jj = 0; jj < PER; ++jj) ov[jj] = sv[j0 + jj];
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (uint32_t jj = 0; jj < PER; ++jj) {
        const llima_u32x4 o = ov[jj];
        const bool in = padded || j0 + jj < ns;
        const uint64_t wj = ((uint64_t)o.w << 32) | o.z;
#pragma unroll
        for (int e = 0; e < NPL; ++e) {
            const bool g = in && o.x > key[e], q = in && o.x == key[e];
            gt[e] += g ? 1u : 0u;
            eq[e] += q ? 1u : 0u;
            above[e] += g ? wj : 0ull;
            same[e] += q ? wj : 0ull;
        }
    }
#pragma unroll
    for (int e = 0; e < NPL; ++e) {
        sh.part[e][wave][lane] = above[e];
        sh.part2[e][wave][lane] = same[e];
        sh.pc[e][wave][lane] = gt[e] | (eq[e] << 16);
    }
    __syncthreads();
    FIN_MARK(10);
    // tau: the key of a candidate with gt < k <= gt + eq; Z (the mass kept by
    // top-k) = mass above tau + mass equal to it, read off that candidate
    uint32_t tk = 0;
    uint64_t zt = 0;
    const bool has_k = c.k > 0 && (uint32_t)c.k <= ns;
#pragma unroll
    for (int e = 0; e < NPL; ++e) {
        above[e] = 0; same[e] = 0; gt[e] = 0; eq[e] = 0;
#pragma unroll
        for (int w2 = 0; w2 < LLIMA_WAVES; ++w2) {
            above[e] += sh.part[e][w2][lane];
            same[e] += sh.part2[e][w2][lane];
            const uint32_t g2 = sh.pc[e][w2][lane];
            gt[e] += g2 & 0xFFFFu;
            eq[e] += g2 >> 16;
        }
        const uint32_t i = (uint32_t)e * 64u + lane;
        const bool at = has_k && i < ns && gt[e] < (uint32_t)c.k && gt[e] + eq[e] >= (uint32_t)c.k;
        if (at && key[e] > tk) { tk = key[e]; zt = above[e] + same[e]; }
    }
    uint32_t tau = 1u;
    uint64_t Zk = 0;                                  // valid when has_k
    if (has_k) {
        tau = wave_max_u32(tk);
        const uint64_t hit = ballot(tk == tau && tau != 0u);
        const uint32_t L = hit ? (uint32_t)__builtin_ffsll((long long)hit) - 1u : 0u;
        Zk = readlane64(zt, L);
    }
    if (c.k > 0 && tcut && !(tau > tcut)) return false;   // uniform: every wave has tau
    FIN_MARK(11);

    bool fin[NPL];
    uint64_t zk = 0;
#pragma unroll
    for (int e = 0; e < NPL; ++e) {
        fin[e] = (uint32_t)e * 64u + lane < ns && key[e] != 0u && key[e] >= tau;
        zk += fin[e] ? w[e] : 0ull;
    }
    if (c.p < 1.0f) {
        // (above << 32) < frac32(p) * Z  <=>  above < ceil(frac32(p) * Z / 2^32)
        const uint64_t Z = has_k ? Zk : wave_sum_u64(zk);
        const llima_u128 PZ = (llima_u128)frac32(c.p) * Z;
        const uint64_t plim = (uint64_t)((PZ + 0xFFFFFFFFull) >> 32);
#pragma unroll
        for (int e = 0; e < NPL; ++e) fin[e] = fin[e] && (above[e] < plim || key[e] == kmax);
    }
    if (c.m > 0.0f) {
        const uint64_t mthr = frac32(c.m) << 4;
#pragma unroll
        for (int e = 0; e < NPL; ++e) fin[e] = fin[e] && w[e] >= mthr;
    }
    uint64_t wf[NPL];
#pragma unroll
    for (int e = 0; e < NPL; ++e) wf[e] = fin[e] ? w[e] : 0ull;
    if (id_sorted) {
        // element order (e, lane) is id order: the draw is a scan
        uint64_t upto[NPL], Zf = 0;
#pragma unroll
        for (int e = 0; e < NPL; ++e) {
            upto[e] = wave_incl_scan_u64(wf[e]) + Zf;
            Zf = readlane63(upto[e]);
        }
        if (Zf == 0) {
            if (threadIdx.x == 0) write_result(P, row, -1, 0.0f);
        } else {
            const uint64_t target = (uint64_t)(((llima_u128)uniform32(c.u) * Zf) >> 32);
#pragma unroll
            for (int e = 0; e < NPL; ++e)
                if (wave == 0 && wf[e] > 0 && upto[e] - wf[e] <= target && target < upto[e])
                    write_result(P, row, (int32_t)id[e], (float)((double)wf[e] / (double)Zf));
        }
    } else {
        uint64_t zl = 0;
#pragma unroll
        for (int e = 0; e < NPL; ++e) zl += wf[e];
        const uint64_t Zf = wave_sum_u64(zl);        // the same in every wave
        __syncthreads();                              // every wave has read sv and part
        if (Zf == 0) {
            if (threadIdx.x == 0) write_result(P, row, -1, 0.0f);
        } else {
            const uint64_t target = (uint64_t)(((llima_u128)uniform32(c.u) * Zf) >> 32);
            if (wave == 0) {
#pragma unroll
                for (int e = 0; e < NPL; ++e)
                    sv[(uint32_t)e * 64u + lane] = llima_u32x4{id[e], 0u, (uint32_t)wf[e], (uint32_t)(wf[e] >> 32)};
            }
            __syncthreads();
            uint64_t upto[NPL];
#pragma unroll
            for (int e = 0; e < NPL; ++e) upto[e] = 0;
#pragma unroll
            for (uint32_t jj = 0; jj < PER; ++jj) {
                const llima_u32x4 o = sv[j0 + jj];
                const uint64_t wj = ((uint64_t)o.w << 32) | o.z;
#pragma unroll
                for (int e = 0; e < NPL; ++e) upto[e] += o.x <= id[e] ? wj : 0ull;   // wf 0 past ns
            }
#pragma unroll
            for (int e = 0; e < NPL; ++e) sh.part[e][wave][lane] = upto[e];
            __syncthreads();
#pragma unroll
            for (int e = 0; e < NPL; ++e) {
                uint64_t u = 0;
#pragma unroll
                for (int w2 = 0; w2 < LLIMA_WAVES; ++w2) u += sh.part[e][w2][lane];
                if (wave == 0 && wf[e] > 0 && u - wf[e] <= target && target < u)
                    write_result(P, row, (int32_t)id[e], (float)((double)wf[e] / (double)Zf));
            }
        }
    }
    FIN_MARK(12);
    if (P.out_keep)
        write_keep(P, row, [&](auto set) {
#pragma unroll
            for (int e = 0; e < NPL; ++e)
                if (wave == 0 && fin[e]) set(id[e]);
        });
    return true;
}

// ------------------------------------------------------------------ fast path
__device__ __forceinline__ uint32_t hash_slot(uint32_t id) {
    return (id * 2654435761u) >> (32 - 12);         // SMP_HASH = 4096 slots
}

// Candidates f = EPT t + j (j < EPT) of the N gathered in sh.u.cand (id
// order), so a thread's candidates are consecutive and (thread, j) order is id
// order.  False when the row needs the full-row path (nothing written yet).
template <int EPT>
__device__ __forceinline__ bool fin_elems(const SampleParams& P, int row, const RowCfg& c, uint32_t N,
                          uint32_t gkey, const int32_t (&hid)[SMP_HBATCH], FinShared& sh) {
    const uint32_t t = threadIdx.x, lane = lane_id(), wave = wave_id();
    float x[EPT];
    uint32_t id[EPT];
    // every read at once from a clamped slot, the element past N made -inf
#pragma unroll
    for (int j = 0; j < EPT; ++j) {
        const uint32_t f = t * EPT + (uint32_t)j;
        const uint32_t fc = f < N ? f : 0u;
        const uint64_t q = sh.u.cand[fc + (fc >> 4)];
        x[j] = f < N ? key_f32((uint32_t)(q >> 32)) : -__builtin_inff();
        id[j] = (uint32_t)q;
    }

    // ---- lazy penalties: history ids counted against a hash of the candidate ids
    if (row_lazy(P, c)) {
        if (N > SMP_HASH / 2) return false;
        __syncthreads();                              // sh.u.cand is read
        for (uint32_t i = t; i < SMP_HASH / 4; i += LLIMA_WG) {
            ((llima_u32x4*)sh.u.hash.key)[i] = llima_u32x4{0u, 0u, 0u, 0u};
            ((llima_u32x4*)sh.u.hash.cnt)[i] = llima_u32x4{0u, 0u, 0u, 0u};
        }
        __syncthreads();
        uint32_t slot[EPT];
#pragma unroll
        for (int j = 0; j < EPT; ++j) {
            slot[j] = 0;
            if (t * EPT + (uint32_t)j < N) {
                uint32_t h = hash_slot(id[j]);
                for (int p = 0; p < SMP_HASH; ++p) {
                    const uint32_t prev = atomicCAS(&sh.u.hash.key[h], 0u, id[j] + 1u);
                    if (prev == 0u) break;
                    h = (h + 1u) & (SMP_HASH - 1u);
                }
                slot[j] = h;
            }
        }
        __syncthreads();
        auto count_id = [&](int32_t hv) {
            if (hv < 0 || hv >= P.V) return;
            uint32_t h = hash_slot((uint32_t)hv);
            for (int p = 0; p < SMP_HASH; ++p) {
                const uint32_t kk = sh.u.hash.key[h];
                if (kk == (uint32_t)hv + 1u) { atomicAdd(&sh.u.hash.cnt[h], 1u); return; }
                if (kk == 0u) return;
                h = (h + 1u) & (SMP_HASH - 1u);
            }
        };
#pragma unroll
        for (int b = 0; b < SMP_HBATCH; ++b)
            if ((int)t + b * LLIMA_WG < c.hlen) count_id(hid[b]);
        const int32_t* hrow = P.hist + (size_t)row * P.H_max;
        for (int i = (int)t + SMP_HBATCH * LLIMA_WG; i < c.hlen; i += LLIMA_WG) count_id(hrow[i]);
        __syncthreads();
#pragma unroll
        for (int j = 0; j < EPT; ++j) {
            if (t * EPT + (uint32_t)j < N) {
                const uint32_t cn = sh.u.hash.cnt[slot[j]];
                if (cn) x[j] = penalize(x[j], cn, c);
            }
        }
    }

    // ---- keys of x / T (0: absent or -inf; past N x is -inf), row maximum
    //      and minimum, count.  x / 1 is x: no division at temperature 1.
    uint32_t key[EPT];
    uint32_t kmx = 0, nkmn = 0, nf = 0;
    if (c.T == 1.0f) {
#pragma unroll
        for (int j = 0; j < EPT; ++j) key[j] = f32_key(x[j]);
    } else {
#pragma unroll
        for (int j = 0; j < EPT; ++j) key[j] = f32_key(x[j] / c.T);
    }
#pragma unroll
    for (int j = 0; j < EPT; ++j) {
        key[j] = key[j] > LLIMA_KEY_NEG_INF ? key[j] : 0u;
        kmx = key[j] > kmx ? key[j] : kmx;
        nkmn = key[j] && ~key[j] > nkmn ? ~key[j] : nkmn;
        nf += key[j] ? 1u : 0u;
    }
    {
        const uint32_t a = wave_max_u32(kmx), b = wave_max_u32(nkmn), s2 = wave_sum_u32(nf);
        if (lane == 0) { sh.r32[0][wave] = a; sh.r32[1][wave] = b; sh.r32[2][wave] = s2; }
        sh.hcnt[0][t] = 0; sh.hcnt[1][t] = 0;
        sh.hmass[0][t] = 0; sh.hmass[1][t] = 0;
        __syncthreads();
        kmx = 0; nkmn = 0; nf = 0;
#pragma unroll
        for (int w = 0; w < LLIMA_WAVES; ++w) {
            kmx = sh.r32[0][w] > kmx ? sh.r32[0][w] : kmx;
            nkmn = sh.r32[1][w] > nkmn ? sh.r32[1][w] : nkmn;
            nf += sh.r32[2][w];
        }
        // the candidates are in registers: sh.u holds the top-p bins from here
        for (uint32_t i = t; i < SMP_PBIN_SLOTS; i += LLIMA_WG) sh.u.cand[i] = 0;
        if (t == 0) sh.lcount = 0;
        __syncthreads();
    }
    FIN_MARK(5);
    const uint32_t kmax = kmx, kmin = ~nkmn;
    if (nf == 0) {
        if (gkey) return false;                      // skipped values may be finite
        if (t == 0) write_result(P, row, -1, 0.0f);
        if (P.out_keep) write_keep(P, row, [&](auto) {});
        return true;
    }
    const float xmax = key_f32(kmax);

    // ---- lower edge of the top-k boundary: histogram rounds until at most 64
    //      values are at or above it (or the k-th largest key itself is known)
    uint32_t lowkey = 1u;
    bool exact = true;                               // lowkey is tau itself
    if (c.k > 0) {
        if (nf < (uint32_t)c.k) {
            if (gkey) return false;                  // values left out could count
        } else {
            Digits d = digits_init(kmin, kmax);
            uint32_t rem = (uint32_t)c.k, above_all = 0;
            lowkey = d.prefix;
            exact = d.top < 0;
            int buf = 0;
            while (d.top >= 0) {
                const int lo = d.top - 7 > 0 ? d.top - 7 : 0;
                const uint32_t bmask = (1u << (d.top - lo + 1)) - 1u;
                uint32_t* hc = sh.hcnt[buf];
#pragma unroll
                for (int j = 0; j < EPT; ++j)
                    if (key[j] && (key[j] & d.pmask) == d.prefix) atomicAdd(&hc[(key[j] >> lo) & bmask], 1u);
                __syncthreads();
                const uint32_t bin = 255u - t;                 // thread 0 <-> top bin
                const uint32_t cn = hc[bin];
                sh.hcnt[buf ^ 1][t] = 0;
                const uint32_t inc = wave_incl_scan_u32(cn);
                const uint32_t ab = (uint32_t)wg_prefix_u64(inc, cn, sh.r64[0]);
                if (ab < rem && ab + cn >= rem) { sh.sel[0] = bin; sh.sel[1] = ab; sh.sel[2] = cn; }
                __syncthreads();
                const uint32_t sb = sh.sel[0], sab = sh.sel[1], scn = sh.sel[2];
                hc[t] = 0;
                buf ^= 1;
                d.prefix |= sb << lo;
                d.pmask |= bmask << lo;
                d.top = lo - 1;
                rem -= sab;
                above_all += sab;
                lowkey = d.prefix;
                exact = d.top < 0;
                if (above_all + scn <= SMP_SMALL) break;
            }
            __syncthreads();
        }
    } else if (gkey) {
        // without top-k every skipped value must have weight 0 (and not matter)
        const float dg = key_f32(gkey) - xmax;
        if (dg >= -26.0f || !zero_weight_irrelevant(P, c)) return false;
    }
    if (c.k > 0 && exact && gkey && !(lowkey > gkey)) return false;
    FIN_MARK(6);

    // ---- values at or above lowkey: at most 64 -> pairwise small path
    uint32_t ns = 0;
#pragma unroll
    for (int j = 0; j < EPT; ++j) ns += key[j] && key[j] >= lowkey ? 1u : 0u;
    uint32_t nst;
    const uint32_t so = block_excl_scan_u32(ns, &nst, sh.bs);
    FIN_MARK(7);
    if (nst <= SMP_SMALL) {
        uint32_t o = so;
#pragma unroll
        for (int j = 0; j < EPT; ++j) {
            if (key[j] && key[j] >= lowkey) {
                const uint64_t w = weight(key_f32(key[j]), xmax);
                sh.sv[o] = llima_u32x4{key[j], id[j], (uint32_t)w, (uint32_t)(w >> 32)};
                ++o;
            }
        }
        __syncthreads();
        return fin_small<1, false>(P, row, c, nst, kmax, c.k > 0 ? gkey : 0u, sh.sv, true, sh);
    }
    // more than 64 remain only when lowkey is tau (ties) or there is no top-k

    // ---- many survivors: weights, top-p radix, min-p, draw by a scan in id order
    const uint32_t tau = lowkey;
    uint64_t w[EPT];
#pragma unroll
    for (int j = 0; j < EPT; ++j) key[j] = key[j] < tau ? 0u : key[j];
    if (xmax < __builtin_inff()) {                   // uniform; key 0 decodes to NaN, weight 0
#pragma unroll
        for (int j = 0; j < EPT; ++j) {
            const uint64_t wj = wf_u64(weight_f(key_f32(key[j]), xmax));
            w[j] = key[j] ? wj : 0ull;
        }
    } else {
#pragma unroll
        for (int j = 0; j < EPT; ++j) {
            const uint64_t wj = weight(key_f32(key[j]), xmax);
            w[j] = key[j] ? wj : 0ull;
        }
    }
    FIN_MARK(8);
    uint32_t theta = 0;
    if (c.p < 1.0f) {
        theta = fin_topp_bins<EPT>(key, w, frac32(c.p), kmax, sh.u.cand, sh);
        if (theta == 0u)                             // an infinite maximum or a crowded bin
            theta = fin_topp_desc<EPT>(key, w, frac32(c.p), tau > kmin ? tau : kmin, kmax, sh);
    }
    FIN_MARK(9);
    const uint64_t mthr = c.m > 0.0f ? frac32(c.m) << 4 : 0;
    uint32_t fmask = 0;
#pragma unroll
    for (int j = 0; j < EPT; ++j) {
        const bool f = key[j] && key[j] >= theta && w[j] >= mthr;
        fmask |= f ? (1u << j) : 0u;
        w[j] = f ? w[j] : 0ull;
    }
    // the draw: a thread's candidates are consecutive ids, so one scan of the
    // per-thread sums orders the whole row
    uint64_t mysum = 0;
#pragma unroll
    for (int j = 0; j < EPT; ++j) mysum += w[j];
    FIN_MARK(10);
    uint64_t Zf;
    const uint64_t before = block_excl_scan_u64(mysum, &Zf, sh.bs);
    FIN_MARK(11);
    if (Zf == 0) {
        if (t == 0) write_result(P, row, -1, 0.0f);
    } else {
        const uint64_t target = (uint64_t)(((llima_u128)uniform32(c.u) * Zf) >> 32);
        if (mysum > 0 && before <= target && target < before + mysum) {
            uint64_t acc = before;
            bool hit = false;
#pragma unroll
            for (int j = 0; j < EPT; ++j) {
                if (!hit && w[j] && acc <= target && target < acc + w[j]) {
                    write_result(P, row, (int32_t)id[j], (float)((double)w[j] / (double)Zf));
                    hit = true;
                }
                acc += w[j];
            }
        }
    }
    FIN_MARK(12);
    if (P.out_keep)
        write_keep(P, row, [&](auto set) {
#pragma unroll
            for (int j = 0; j < EPT; ++j)
                if ((fmask >> j) & 1u) set(id[j]);
        });
    return true;
}

// ------------------------------------------------------------------ direct path
// Survivors (at most 64 NPL), in id order as {raw key, id} (me): the
// candidates at or above the raw key lowkey (1: every candidate).  Every wave
// holds all of them (element e of lane l: survivor 64 e + l).  Lazy rows take
// their penalties here (history ids counted against a bitmap of the survivor
// ids, two barriers); then every wave computes the same x / T, keys, row
// maximum and weights, ranks the survivors against its quarter of them (ge:
// keys at or above, above: the mass strictly above), and after one barrier
// adds the quarters: tau = the largest key with ge >= k, the top-p and min-p
// cuts and the draw as a scan in id order (wave 0 writes).  Returns false
// (every wave alike), before writing anything, when the result cannot be
// proven: tau must exceed the chunk bounds (gkey) and, when lowkey cut
// candidates off, fl(lowkey / T) (a value below lowkey, penalised or not, is
// at most that).
template <int NPL>
__device__ __forceinline__ bool fin_tail(const SampleParams& P, int row, const RowCfg& c,
                                         const llima_u32x4 (&me)[2], uint32_t ns, uint32_t lowkey,
                                         uint32_t gkey, const int32_t (&hid)[SMP_HBATCH],
                                         FinShared& sh) {
    const uint32_t t = threadIdx.x, lane = lane_id(), wave = wave_id();
    float x[NPL];
    uint32_t id[NPL];
#pragma unroll
    for (int e = 0; e < NPL; ++e) {
        const uint32_t i = (uint32_t)e * 64u + lane;
        x[e] = i < ns ? key_f32(me[e].x) : -__builtin_inff();
        id[e] = i < ns ? me[e].y : 0xFFFFFFFFu;         // matches no history id
    }
    if (row_lazy(P, c)) {
        // A bitmap of the survivor ids (2^16 bits in sh.u.hash.key, cleared
        // by fin_direct) passes a history id with one LDS read; the few that
        // pass (the survivors' own occurrences and about 0.1 % false hits) are
        // broadcast one distinct id per wave at a time and counted by the lanes
        // holding the survivors, together with the wave's other copies of that
        // id; the waves' counts are added in sh.hc (zeroed by fin_direct).
        uint32_t* bm = sh.u.hash.key;
        auto bit_of = [](uint32_t v) { return (v * 2654435761u) >> 16; };
        if (wave == 0) {
#pragma unroll
            for (int e = 0; e < NPL; ++e) {
                const uint32_t h = bit_of(id[e]);
                if ((uint32_t)e * 64u + lane < ns) atomicOr(&bm[h >> 5], 1u << (h & 31u));
            }
        }
        __syncthreads();
        FIN_MARK(6);
        uint32_t cn[NPL];
#pragma unroll
        for (int e = 0; e < NPL; ++e) cn[e] = 0u;
        // hv: this lane's history id; m: the lanes whose id passed; inlen:
        // the lanes whose entry lies before hlen
        auto count_pass = [&](uint32_t hv, uint64_t m, uint64_t inlen) {
            while (m) {
                const uint32_t L = (uint32_t)__builtin_ctzll(m);
                const uint32_t u = readlane(hv, L);
                const uint64_t same = ballot(hv == u) & inlen;
                m &= ~same;
                const uint32_t k = (uint32_t)__popcll(same);
#pragma unroll
                for (int e = 0; e < NPL; ++e) cn[e] += id[e] == u ? k : 0u;
            }
        };
        uint32_t bw[SMP_HBATCH];                         // every bitmap read first
#pragma unroll
        for (int b = 0; b < SMP_HBATCH; ++b) bw[b] = bm[bit_of((uint32_t)hid[b]) >> 5];
#pragma unroll
        for (int b = 0; b < SMP_HBATCH; ++b) {
            const uint64_t inlen = ballot((int)t + b * LLIMA_WG < c.hlen);
            const uint64_t m = ballot((bw[b] >> (bit_of((uint32_t)hid[b]) & 31u)) & 1u) & inlen;
            count_pass((uint32_t)hid[b], m, inlen);
        }
        const int32_t* hrow = P.hist + (size_t)row * P.H_max;
        for (int base = SMP_HBATCH * LLIMA_WG; base < c.hlen; base += LLIMA_WG) {
            const int i = base + (int)t;
            const uint32_t hv = i < c.hlen ? (uint32_t)hrow[i] : 0u;
            const uint32_t h = bit_of(hv);
            const uint64_t inlen = ballot(i < c.hlen);
            count_pass(hv, ballot((bm[h >> 5] >> (h & 31u)) & 1u) & inlen, inlen);
        }
        FIN_MARK(7);
        // ids outside [0, V) match no survivor
#pragma unroll
        for (int e = 0; e < NPL; ++e)
            if (cn[e]) atomicAdd(&sh.hc[(uint32_t)e * 64u + lane], cn[e]);
        __syncthreads();
#pragma unroll
        for (int e = 0; e < NPL; ++e) {
            const uint32_t n = sh.hc[(uint32_t)e * 64u + lane];    // 0 past ns
            x[e] = n ? penalize(x[e], n, c) : x[e];
        }
    }
    FIN_MARK(8);
    uint32_t key[NPL], kmax = 0;
#pragma unroll
    for (int e = 0; e < NPL; ++e) {
        const float xt = x[e] / c.T;
        key[e] = (uint32_t)e * 64u + lane < ns && xt > -__builtin_inff() ? f32_key(xt) : 0u;
        kmax = key[e] > kmax ? key[e] : kmax;
    }
    kmax = wave_max_u32(kmax);
    if (kmax == 0u) {                                 // uniform: every wave holds every survivor
        if (gkey || lowkey > 1u) return false;
        if (t == 0) write_result(P, row, -1, 0.0f);
        if (P.out_keep) write_keep(P, row, [&](auto) {});
        return true;
    }
    uint64_t w[NPL];
    llima_u32x4* sv = sh.sv2[wave];
#pragma unroll
    for (int e = 0; e < NPL; ++e) {
        const uint64_t w0 = weight(key_f32(key[e]), key_f32(kmax));
        w[e] = key[e] ? w0 : 0ull;
        sv[(uint32_t)e * 64u + lane] = llima_u32x4{key[e], 0u, (uint32_t)w[e], (uint32_t)(w[e] >> 32)};
    }
    __builtin_amdgcn_wave_barrier();                 // the wave's LDS writes precede its reads
    FIN_MARK(9);
    // this wave's quarter of the survivors against every survivor (entries
    // past ns hold key 0 and weight 0: they count for no present key)
    constexpr uint32_t PER = 16u * NPL;
    const uint32_t j0 = wave * PER;
    uint32_t ge[NPL];
    uint64_t above[NPL];
#pragma unroll
    for (int e = 0; e < NPL; ++e) { ge[e] = 0; above[e] = 0; }
    llima_u32x4 ov[PER];
#pragma unroll
    for (uint32_t jj = 0; jj < PER; ++jj) ov[jj] = sv[j0 + jj];
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (uint32_t jj = 0; jj < PER; ++jj) {
        const llima_u32x4 o = ov[jj];
        const uint64_t wj = ((uint64_t)o.w << 32) | o.z;
#pragma unroll
        for (int e = 0; e < NPL; ++e) {
            ge[e] += o.x >= key[e] ? 1u : 0u;
            above[e] += o.x > key[e] ? wj : 0ull;
        }
    }
#pragma unroll
    for (int e = 0; e < NPL; ++e) {
        sh.part[e][wave][lane] = above[e];
        sh.pc[e][wave][lane] = ge[e];
    }
    __syncthreads();
    FIN_MARK(10);
#pragma unroll
    for (int e = 0; e < NPL; ++e) {
        above[e] = 0; ge[e] = 0;
#pragma unroll
        for (int w2 = 0; w2 < LLIMA_WAVES; ++w2) {
            above[e] += sh.part[e][w2][lane];
            ge[e] += sh.pc[e][w2][lane];
        }
    }
    // tau: the k-th largest key counted with multiplicity, the largest key
    // with at least k keys at or above it
    const bool has_k = c.k > 0 && (uint32_t)c.k <= ns;
    uint32_t tau = 1u;
    if (has_k) {
        uint32_t tk = 0;
#pragma unroll
        for (int e = 0; e < NPL; ++e) tk = key[e] && ge[e] >= (uint32_t)c.k && key[e] > tk ? key[e] : tk;
        tau = wave_max_u32(tk);
    }
    uint32_t tcut = 0;
    if (c.k > 0) {
        tcut = gkey;
        if (lowkey > 1u) {
            const uint32_t kl = f32_key(key_f32(lowkey) / c.T);
            tcut = kl > tcut ? kl : tcut;
        }
    }
    if (c.k > 0 && tcut && !(tau > tcut)) return false;   // uniform: every wave has tau
    FIN_MARK(11);
    bool fin[NPL];
    uint64_t zk = 0;
#pragma unroll
    for (int e = 0; e < NPL; ++e) {
        fin[e] = key[e] != 0u && key[e] >= tau;
        zk += fin[e] ? w[e] : 0ull;
    }
    if (c.p < 1.0f) {
        // (above << 32) < frac32(p) * Z  <=>  above < ceil(frac32(p) * Z / 2^32),
        // Z the mass top-k keeps
        const uint64_t Z = wave_sum_u64(zk);
        const llima_u128 PZ = (llima_u128)frac32(c.p) * Z;
        const uint64_t plim = (uint64_t)((PZ + 0xFFFFFFFFull) >> 32);
#pragma unroll
        for (int e = 0; e < NPL; ++e) fin[e] = fin[e] && (above[e] < plim || key[e] == kmax);
    }
    if (c.m > 0.0f) {
        const uint64_t mthr = frac32(c.m) << 4;
#pragma unroll
        for (int e = 0; e < NPL; ++e) fin[e] = fin[e] && w[e] >= mthr;
    }
    // element order (e, lane) is id order: the draw is a scan
    uint64_t wf[NPL], upto[NPL], Zf = 0;
#pragma unroll
    for (int e = 0; e < NPL; ++e) {
        wf[e] = fin[e] ? w[e] : 0ull;
        upto[e] = wave_incl_scan_u64(wf[e]) + Zf;
        Zf = readlane63(upto[e]);
    }
    if (Zf == 0) {
        if (t == 0) write_result(P, row, -1, 0.0f);
    } else {
        const uint64_t target = (uint64_t)(((llima_u128)uniform32(c.u) * Zf) >> 32);
#pragma unroll
        for (int e = 0; e < NPL; ++e)
            if (wave == 0 && wf[e] > 0 && upto[e] - wf[e] <= target && target < upto[e])
                write_result(P, row, (int32_t)id[e], (float)((double)wf[e] / (double)Zf));
    }
    FIN_MARK(12);
    if (P.out_keep)
        write_keep(P, row, [&](auto set) {
#pragma unroll
            for (int e = 0; e < NPL; ++e)
                if (wave == 0 && fin[e]) set(id[e]);
        });
    return true;
}

// Candidates straight from the first-round loads: thread t holds the 8 slots
// [8 part, 8 part + 8) of its chunk's region, so slot order over the threads
// is id order.  kr: raw keys (0 = no candidate), idv: ids.  Finds the lower
// edge lowkey of the top-k boundary on the raw values with histogram rounds
// until at most 64 candidates remain at or above it, stages them and hands
// over to fin_survivors.  False when the row needs another path.
__device__ __forceinline__ bool fin_direct(const SampleParams& P, int row, const RowCfg& c, const uint32_t (&kr)[8],
                           const uint32_t (&idv)[8], uint32_t N, uint32_t kmin, uint32_t kmax,
                           uint32_t gkey, const int32_t (&hid)[SMP_HBATCH], FinShared& sh) {
    const uint32_t t = threadIdx.x;
    if (N == 0) {
        if (gkey) return false;
        if (t == 0) write_result(P, row, -1, 0.0f);
        if (P.out_keep) write_keep(P, row, [&](auto) {});
        return true;
    }
    if (row_lazy(P, c)) {
#pragma unroll
        for (int i = 0; i < 2; ++i)                          // the 2^16-bit survivor-id bitmap
            ((llima_u32x4*)sh.u.hash.key)[t + i * LLIMA_WG] = llima_u32x4{0u, 0u, 0u, 0u};
    }
    FIN_MARK(3);
    uint32_t lowkey = 1u;
    if (c.k > 0) {
        if (N < (uint32_t)c.k) {
            if (gkey) return false;                  // values left out could count
        } else {
            Digits d = digits_init(kmin, kmax);
            // lazy penalties can push values of the top-k below their raw rank:
            // keep a margin of candidates below the k-th largest raw value (the
            // row falls back when more survivors than that drop below the rest;
            // a random history holds about one in a thousand ids, and a wider
            // margin narrows the window the first round can stop in)
            const uint32_t kk = (uint32_t)c.k;
            const uint32_t margin = !row_lazy(P, c) ? 0u
                                  : kk + 6u <= SMP_SMALL ? 6u
                                  : kk < 2u * SMP_SMALL ? min(32u, 2u * SMP_SMALL - kk) : 0u;
            uint32_t rem = min(N, (uint32_t)c.k + margin), above_all = 0;
            // survivors wanted: at least rem, at most cap (one per lane when
            // rem allows it: the pairwise ranking costs the square)
            const uint32_t cap = rem <= SMP_SMALL ? SMP_SMALL : 2u * SMP_SMALL;
            lowkey = d.prefix;
            // round r counts into hcnt[r % 3] (rounds 0 and 1 zeroed by the
            // caller); after its barrier every wave scans all 256 bins itself
            // and zeroes hcnt[(r + 2) % 3], which every wave has finished
            // reading (round r - 1) and nobody counts into before round r + 2
            uint32_t buf = 0;
            while (d.top >= 0) {
                const int lo = d.top - 7 > 0 ? d.top - 7 : 0;
                const uint32_t bmask = (1u << (d.top - lo + 1)) - 1u;
                uint32_t* hc = sh.hcnt[buf];
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const bool in = (kr[j] != 0u) & ((kr[j] & d.pmask) == d.prefix);
                    atomicAdd(&hc[in ? (kr[j] >> lo) & bmask : 256u + lane_id()], 1u);
                }
                __syncthreads();
                // lane l: bins 255 - 4l down to 252 - 4l (.w .z .y .x)
                const llima_u32x4 c4 = ((const llima_u32x4*)hc)[63u - lane_id()];
                const uint32_t nxt = buf == 0u ? 2u : buf - 1u;
                sh.hcnt[nxt][t] = 0;
                const uint32_t s4 = c4.x + c4.y + c4.z + c4.w;
                uint32_t ab = wave_incl_scan_u32(s4) - s4;
                const uint32_t top = 255u - 4u * lane_id();
                const uint32_t cs[4] = {c4.w, c4.z, c4.y, c4.x};
                // mb: the bin holding the rem-th key; fb: the lowest bin such
                // that it and the bins above hold at most cap - above_all keys
                uint32_t mb = 0, mab = 0, mcn = 0, fb = 0, fcum = 0;
                bool hit = false, fit = false;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const bool h = ab < rem && ab + cs[i] >= rem;
                    mb = h ? top - (uint32_t)i : mb;
                    mab = h ? ab : mab;
                    mcn = h ? cs[i] : mcn;
                    hit = hit || h;
                    const bool f = above_all + ab + cs[i] <= cap;
                    fb = f ? top - (uint32_t)i : fb;
                    fcum = f ? ab + cs[i] : fcum;
                    fit = fit || f;
                    ab += cs[i];
                }
                const uint64_t hm = ballot(hit), fm = ballot(fit);
                if (hm == 0) return false;               // cannot happen: the bins hold rem
                buf = buf == 2u ? 0u : buf + 1u;
                if (fm) {
                    const uint32_t F = 63u - (uint32_t)__builtin_clzll(fm);
                    if (readlane(fcum, F) >= rem) {      // cap keys or fewer, rem or more
                        lowkey = d.prefix | (readlane(fb, F) << lo);
                        break;
                    }
                }
                const uint32_t L = (uint32_t)__builtin_ffsll((long long)hm) - 1u;
                const uint32_t sb = readlane(mb, L), sab = readlane(mab, L), scn = readlane(mcn, L);
                d.prefix |= sb << lo;
                d.pmask |= bmask << lo;
                d.top = lo - 1;
                rem -= sab;
                above_all += sab;
                lowkey = d.prefix;
                if (cap > SMP_SMALL && above_all + scn <= cap) break;
            }
        }
    } else if (gkey) {
        // without top-k every skipped value must have weight 0 (and not matter)
        const float dg = key_f32(gkey) - key_f32(kmax) / c.T;
        if (dg >= -26.0f || !zero_weight_irrelevant(P, c)) return false;
    }
    FIN_MARK(4);
    uint32_t ns = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) ns += kr[j] && kr[j] >= lowkey ? 1u : 0u;
    // exclusive scan of the counts over the workgroup (sh.bs.w32 is not
    // written again before the barrier below)
    const uint32_t inc = wave_incl_scan_u32(ns);
    const uint32_t wave = wave_id(), lane = lane_id();
    if (lane == 63) sh.bs.w32[wave] = inc;
    __syncthreads();
    uint32_t nst = 0, before = 0;
#pragma unroll
    for (int w = 0; w < LLIMA_WAVES; ++w) {
        const uint32_t n = sh.bs.w32[w];
        before += (uint32_t)w < wave ? n : 0u;
        nst += n;
    }
    if (nst > 2 * SMP_SMALL) return false;
    uint32_t o = before + inc - ns;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const bool in = (kr[j] != 0u) & (kr[j] >= lowkey);
        sh.sv[in ? o : 2u * SMP_SMALL + lane] = llima_u32x4{kr[j], idv[j], 0u, 0u};
        o += in ? 1u : 0u;
    }
    sh.hc[t] = 0;
    __syncthreads();
    FIN_MARK(5);
    FIN_NOTE(15, 1);
    llima_u32x4 me[2];
#pragma unroll
    for (int e = 0; e < 2; ++e) me[e] = sh.sv[(uint32_t)e * 64u + lane];
    return nst <= SMP_SMALL ? fin_tail<1>(P, row, c, me, nst, lowkey, gkey, hid, sh)
                            : fin_tail<2>(P, row, c, me, nst, lowkey, gkey, hid, sh);
}

// SPLIT: the instantiation launched when rows may be split (P.fsplit > 1); the
// split code stays out of the other one, whose registers it would crowd.
template <typename TL, bool SPLIT>
__global__ __launch_bounds__(LLIMA_WG) void sample_finish(SampleParams P) {
    __shared__ FinShared sh;
    FIN_BEGIN();
    const int row = blockIdx.x;
    if (P.wide && P.out_ids[row] != SMP_PENDING) return;     // uniform: finished by the wide kernel
    const RowCfg c = load_cfg(P, row);
    if constexpr (SPLIT) {
        if (!c.greedy && c.k == 0) {                          // uniform: the row may be split
            const uint32_t kx = split_row(P, row, c, sh);
            if (kx) {
                split_part<TL>(P, row, c, kx, (int)blockIdx.y, sh);
                return;
            }
        }
        if (blockIdx.y > 0) return;                           // the other parts serve split rows only
    }
    const uint32_t t = threadIdx.x, lane = lane_id(), wave = wave_id();
    const int S = P.S;
    bool done = false;
    if (S <= SMP_MAX_S) {
        // ---- 1. one round of loads: thread t reads 64 bytes (8 slots) of chunk
        //         t >> (8 - lgs), part t & (tpc - 1) (part 0 starts with the
        //         header); then the history ids when the penalties are applied here
        const int sh8 = 8 - P.lgs;
        const uint32_t tpc = 1u << sh8;
        const uint32_t ch = t >> sh8, pt = t & (tpc - 1u);
        const bool mine = (int)ch < S && pt * 8u < SMP_REGION;
        const uint64_t* reg = P.ws + ((size_t)row * S + (mine ? ch : 0u)) * SMP_REGION + (mine ? pt * 8u : 0u);
        llima_u32x4 q[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) q[i] = ((const llima_u32x4*)reg)[i];
        // issued on every row (from the workspace when unused): loads behind a
        // branch would make the first use of q wait for them as well
        int32_t hid[SMP_HBATCH];
        {
            const bool lp = row_lazy(P, c);
            // unused: every load reads the workspace's first word
            const int32_t* hrow = lp ? P.hist + (size_t)row * P.H_max : (const int32_t*)P.ws;
            const int hl = lp ? c.hlen : 1;
#pragma unroll
            for (int b = 0; b < SMP_HBATCH; ++b) {
                const int j = (int)t + b * LLIMA_WG;
                hid[b] = hrow[j < hl ? j : hl - 1];
            }
        }

        // ---- 2. this thread's slots as candidates (raw keys; padding and the
        //         header are none) and the header facts, reduced over the row
        // (selects and bitwise logic throughout: one wave per SIMD runs this,
        // so every branch is paid in full)
        const uint32_t pre = pre_slots(P);
        const bool hdr = mine & (pt == 0u);
        const bool live = mine & !c.greedy;
        uint32_t kr[8], idv[8];
        uint32_t kmx = 0, nkmn = 0, n = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const uint32_t hi = h ? q[i].w : q[i].y, lo = h ? q[i].z : q[i].x;
                const bool valid = live & ((i | h) != 0 || !hdr);   // slot 0 of a region is the header
                const uint32_t k = valid ? hi : 0u;                  // sentinels hold key 0
                kr[2 * i + h] = k;
                idv[2 * i + h] = lo;
                kmx = k > kmx ? k : kmx;
                const uint32_t nk = k ? ~k : 0u;
                nkmn = nk > nkmn ? nk : nkmn;
                n += k ? 1u : 0u;
            }
        }
        const uint32_t flags = q[0].x >> 16;
        const uint32_t count = (flags & HF_OVERFLOW) ? 0u : (q[0].x & 0xFFFFu);
        const uint32_t ovf = !hdr ? 0u : (flags & HF_OVERFLOW) ? 2u : (SMP_HDR + count > pre ? 1u : 0u);
        const float h0 = __uint_as_float(q[0].y);
        const float g0 = c.k > 0 ? h0 : nontopk_bound(P, c, h0);
        const float gt0 = g0 / c.T;
        const uint32_t gk = (hdr & !c.greedy & (g0 > -__builtin_inff())) ? (gt0 == gt0 ? f32_key(gt0) : 0xFFFFFFFFu) : 0u;
        const uint64_t gr = hdr ? ((uint64_t)q[0].w << 32) | q[0].z : 0ull;
        FIN_MARK(1);
        if (hdr) sh.ccount[ch] = count;
        {
            const uint32_t a = wave_max_u32(kmx), b = wave_max_u32(nkmn), s2 = wave_sum_u32(n);
            const uint32_t o2 = wave_max_u32(ovf), g2 = wave_max_u32(gk);
            const uint64_t gg = c.greedy ? wave_max_u64(gr) : 0ull;
            if (lane == 0) {
                sh.r32[0][wave] = a; sh.r32[1][wave] = b; sh.r32[2][wave] = s2;
                sh.r32[3][wave] = o2; sh.r32[4][wave] = g2; sh.r64[1][wave] = gg;
            }
            sh.hcnt[0][t] = 0; sh.hcnt[1][t] = 0;
            sh.hmass[0][t] = 0; sh.hmass[1][t] = 0;
            __syncthreads();
        }
        uint32_t kmax = 0, nkmin = 0, N = 0, ov = 0, gkey = 0;
        uint64_t best = 0;
#pragma unroll
        for (int w = 0; w < LLIMA_WAVES; ++w) {
            kmax = sh.r32[0][w] > kmax ? sh.r32[0][w] : kmax;
            nkmin = sh.r32[1][w] > nkmin ? sh.r32[1][w] : nkmin;
            N += sh.r32[2][w];
            ov = sh.r32[3][w] > ov ? sh.r32[3][w] : ov;
            gkey = sh.r32[4][w] > gkey ? sh.r32[4][w] : gkey;
            best = sh.r64[1][w] > best ? sh.r64[1][w] : best;
        }

        FIN_MARK(2);
        FIN_NOTE(14, N);
        if (c.greedy) {
            const bool ok = (uint32_t)(best >> 32) > LLIMA_KEY_NEG_INF;
            const uint32_t tok = ok ? ~(uint32_t)best : 0xFFFFFFFFu;
            if (t == 0) write_result(P, row, ok ? (int32_t)tok : -1, ok ? 1.0f : 0.0f);
            if (P.out_keep)
                write_keep(P, row, [&](auto set) { if (t == 0 && ok) set(tok); });
            done = true;
        } else if (ov == 0u) {
            done = fin_direct(P, row, c, kr, idv, N, ~nkmin, kmax, gkey, hid, sh);
        }
        // the gather and full-row paths are cold: their code is placed after
        // the direct path's, which then streams through the instruction cache
        if (__builtin_expect(!done && ov < 2u, 0)) {
            // ---- 3. gather: candidates into LDS in id order (element f at f + f / 16)
            __syncthreads();
            if (wave == 0) {
                // exclusive scan of the counts: lane l owns chunks 4l .. 4l+3
                uint32_t cc[4], s4 = 0;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int cix = (int)lane * 4 + i;
                    cc[i] = cix < S ? sh.ccount[cix] : 0u;
                    s4 += cc[i];
                }
                const uint32_t inc = wave_incl_scan_u32(s4);
                uint32_t o = inc - s4;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int cix = (int)lane * 4 + i;
                    if (cix < S) sh.coff[cix] = o;
                    o += cc[i];
                }
                if (lane == 63) sh.hn = inc;
            }
            __syncthreads();
            FIN_MARK(3);
            FIN_NOTE(15, 2);
            const uint32_t NG = sh.hn;
            if (NG <= SMP_FIN_CAP) {
                if (mine) {
                    const uint32_t n_c = sh.ccount[ch], o_c = sh.coff[ch];
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
#pragma unroll
                        for (int h = 0; h < 2; ++h) {
                            const int s = (int)(pt * 8u) + 2 * i + h - SMP_HDR;   // candidate index
                            if (s >= 0 && (uint32_t)s < n_c) {
                                const uint32_t f = o_c + (uint32_t)s;
                                const uint64_t val = h ? (((uint64_t)q[i].w << 32) | q[i].z)
                                                       : (((uint64_t)q[i].y << 32) | q[i].x);
                                sh.u.cand[f + (f >> 4)] = val;
                            }
                        }
                    }
                }
                // chunks with more candidates than the first round covered
                const uint32_t pre_c = pre - SMP_HDR;
                for (int cc = (int)wave; cc < S; cc += LLIMA_WAVES) {
                    const uint32_t n_c = sh.ccount[cc];
                    if (n_c > pre_c) {
                        const uint32_t o_c = sh.coff[cc];
                        const uint64_t* src = P.ws + ((size_t)row * S + cc) * SMP_REGION + SMP_HDR;
                        for (uint32_t s = pre_c + lane; s < n_c; s += 64) {
                            const uint32_t f = o_c + s;
                            sh.u.cand[f + (f >> 4)] = src[s];
                        }
                    }
                }
                sh.hcnt[0][t] = 0; sh.hcnt[1][t] = 0;
                sh.hmass[0][t] = 0; sh.hmass[1][t] = 0;
                __syncthreads();
                FIN_MARK(4);
                done = NG <= 4u * LLIMA_WG ? fin_elems<4>(P, row, c, NG, gkey, hid, sh)
                                           : fin_elems<16>(P, row, c, NG, gkey, hid, sh);
            }
        }
    }
    if (__builtin_expect(!done, 0)) finish_full_row<TL>(P, row, c, sh);
    FIN_MARK(13);
}

// ================================================================== wide finish
// The rows of a grammar-masked batch without top-k hold a few thousand
// candidates each (every allowed value within the weight window), which one
// 256-thread workgroup per row takes through its gather path at one wave per
// SIMD.  This kernel runs before sample_finish on such batches and takes each
// row with 1024 threads, 4 candidates each: the gather (one round of loads
// brings every chunk's header and its first 8 tpc - 1 candidates, tpc =
// 1024 / 2^lgs threads per chunk; only chunks with more are read again),
// keys, weights, the top-p boundary over value bins (fin_topp_bins),
// min-p and the draw as one block scan in id order: fin_elems' steps for rows
// without top-k.  A row it does not finish (greedy, an overflowed region,
// more than SMP_FIN_CAP candidates, a bound the exactness check rejects, an
// infinite maximum or a boundary bin of more than 64 values) gets out_ids =
// SMP_PENDING, and sample_finish finishes exactly those rows.
#define SMP_WIDE 1024
#define SMP_WIDE_WAVES (SMP_WIDE / 64)
#define SMP_WEPT (SMP_FIN_CAP / SMP_WIDE)          // candidates per thread
#define SMP_WPAD 3                                 // candidate f at f + f / 8 (no bank conflicts at 4 per thread)

template <int NW>
struct BlockScratchN {
    uint64_t w64[NW];
    uint32_t w32[NW];
};

template <int NW>
__device__ __forceinline__ uint64_t blk_excl_scan_u64(uint64_t v, uint64_t* total, BlockScratchN<NW>& s) {
    const uint64_t inc = wave_incl_scan_u64(v);
    const uint32_t w = threadIdx.x >> 6;
    if (lane_id() == 63) s.w64[w] = inc;
    __syncthreads();
    uint64_t before = 0, tt = 0;
#pragma unroll
    for (int i = 0; i < NW; ++i) {
        before += (uint32_t)i < w ? s.w64[i] : 0ull;
        tt += s.w64[i];
    }
    __syncthreads();
    *total = tt;
    return before + inc - v;
}

struct WideShared {
    uint64_t cand[SMP_FIN_CAP + (SMP_FIN_CAP >> SMP_WPAD)];   // candidates, then the top-p bins
    uint32_t ccount[SMP_MAX_S];                               // chunk candidate counts
    uint32_t coff[SMP_MAX_S];                                 // chunk offsets of the candidates
    llima_u32x4 sv[2 * SMP_SMALL + 64];                       // fin_topp_bins's boundary members
    uint32_t lcount;
    uint32_t r[3][SMP_WIDE_WAVES];                            // per-wave facts
    BlockScratchN<SMP_WIDE_WAVES> bs;
};
static_assert(SMP_PBIN_SLOTS <= SMP_FIN_CAP, "the top-p bins reuse the candidate array");

template <typename TL>
__global__ __launch_bounds__(SMP_WIDE) void sample_finish_wide(SampleParams P) {
    constexpr int NW = SMP_WIDE_WAVES, EPT = SMP_WEPT;
    __shared__ WideShared sh;
    const int row = blockIdx.x;
    const RowCfg c = load_cfg(P, row);
    const uint32_t t = threadIdx.x;
    const int S = P.S;
    if (c.greedy) {                                              // uniform
        if (t == 0) P.out_ids[row] = SMP_PENDING;
        return;
    }
    // ---- one round of loads: thread t reads 8 slots (64 bytes) of chunk
    //      t >> sh8, part t & (tpc - 1), so up to pre - 1 candidates of every
    //      chunk arrive with its header (slot 0 of part 0)
    const uint32_t wv = t >> 6, lane = lane_id();
    const int sh8 = 10 - P.lgs;                                  // S <= 2^lgs, lgs <= 8
    const uint32_t tpc = 1u << sh8;
    const uint32_t ch = t >> sh8, pt = t & (tpc - 1u);
    const bool mine = (int)ch < S && pt * 8u < SMP_REGION;
    const uint32_t pre = 8u * tpc < SMP_REGION ? 8u * tpc : SMP_REGION;   // first-round slots per chunk
    const uint64_t* reg = P.ws + ((size_t)row * S + (mine ? ch : 0u)) * SMP_REGION + (mine ? pt * 8u : 0u);
    llima_u32x4 q[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) q[i] = ((const llima_u32x4*)reg)[i];
    // the header facts: candidate count, overflow, the largest bound g / T
    const bool hdr = mine && pt == 0u;
    uint32_t cnt = 0, ovf = 0, gk = 0;
    if (hdr) {
        const uint32_t lo = q[0].x;
        ovf = (lo >> 16) & HF_OVERFLOW;
        cnt = ovf ? 0u : (lo & 0xFFFFu);
        const float g0 = nontopk_bound(P, c, __uint_as_float(q[0].y));   // no top-k here
        const float gt0 = g0 / c.T;
        gk = g0 > -__builtin_inff() ? (gt0 == gt0 ? f32_key(gt0) : 0xFFFFFFFFu) : 0u;
        sh.ccount[ch] = cnt;
    }
    // one exchange: the count, any overflow, the largest bound
    uint32_t NG = 0, anyov = 0, gkey = 0;
    {
        const uint32_t sc = wave_sum_u32(cnt), wov = wave_max_u32(ovf), wgk = wave_max_u32(gk);
        if (lane == 63) { sh.r[0][wv] = sc; sh.r[1][wv] = wov; sh.r[2][wv] = wgk; }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < NW; ++i) {
            NG += sh.r[0][i];
            anyov = sh.r[1][i] > anyov ? sh.r[1][i] : anyov;
            gkey = sh.r[2][i] > gkey ? sh.r[2][i] : gkey;
        }
    }
    if (anyov || NG > SMP_FIN_CAP) {                             // uniform
        if (t == 0) P.out_ids[row] = SMP_PENDING;
        return;
    }
    // the chunks' offsets in id order: wave 0, lane l owns chunks 4l .. 4l+3
    if (wv == 0) {
        uint32_t cc[4], s4 = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int cix = (int)lane * 4 + i;
            cc[i] = cix < S ? sh.ccount[cix] : 0u;
            s4 += cc[i];
        }
        const uint32_t inc = wave_incl_scan_u32(s4);
        uint32_t o = inc - s4;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int cix = (int)lane * 4 + i;
            if (cix < S) sh.coff[cix] = o;
            o += cc[i];
        }
    }
    __syncthreads();
    // ---- the candidates into LDS in id order (candidate f at f + f / 8):
    //      this thread's first-round slots, then the rest of any chunk with
    //      more than the first round covered
    if (mine) {
        const uint32_t n_c = sh.ccount[ch], o_c = sh.coff[ch];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int sl = (int)(pt * 8u) + 2 * i + h - SMP_HDR;   // candidate index
                if (sl >= 0 && (uint32_t)sl < n_c) {
                    const uint32_t f = o_c + (uint32_t)sl;
                    sh.cand[f + (f >> SMP_WPAD)] = h ? (((uint64_t)q[i].w << 32) | q[i].z)
                                                     : (((uint64_t)q[i].y << 32) | q[i].x);
                }
            }
        }
    }
    const uint32_t pre_c = pre - SMP_HDR;
    for (int cc = (int)wv; cc < S; cc += NW) {
        const uint32_t n_c = sh.ccount[cc];
        if (n_c > pre_c) {                                       // uniform in the wave
            const uint32_t o_c = sh.coff[cc];
            const uint64_t* src = P.ws + ((size_t)row * S + cc) * SMP_REGION + SMP_HDR;
            for (uint32_t sl = pre_c + lane; sl < n_c; sl += 64) {
                const uint32_t f = o_c + sl;
                sh.cand[f + (f >> SMP_WPAD)] = src[sl];
            }
        }
    }
    __syncthreads();
    // ---- this thread's candidates 4t .. 4t+3, their keys of x / T
    uint32_t key[EPT], id[EPT];
    uint32_t kmx = 0, nf = 0;
#pragma unroll
    for (int j = 0; j < EPT; ++j) {
        const uint32_t f = t * EPT + (uint32_t)j;
        const uint32_t fc = f < NG ? f : 0u;
        const uint64_t v = sh.cand[fc + (fc >> SMP_WPAD)];
        const float x = f < NG ? key_f32((uint32_t)(v >> 32)) : -__builtin_inff();
        id[j] = (uint32_t)v;
        const uint32_t k = f32_key(c.T == 1.0f ? x : x / c.T);
        key[j] = k > LLIMA_KEY_NEG_INF ? k : 0u;
        kmx = key[j] > kmx ? key[j] : kmx;
        nf += key[j] ? 1u : 0u;
    }
    uint32_t kmax = 0, nft = 0;
    {
        const uint32_t a = wave_max_u32(kmx), b = wave_sum_u32(nf);
        if (lane == 0) { sh.r[0][wv] = a; sh.r[1][wv] = b; }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < NW; ++i) {
            kmax = sh.r[0][i] > kmax ? sh.r[0][i] : kmax;
            nft += sh.r[1][i];
        }
    }
    const float xmax = key_f32(kmax);
    // rows the standard finish takes: no finite candidate with values left
    // out, a bound above the weight window, an infinite maximum
    bool pend = nft == 0 && gkey != 0u;
    if (nft > 0 && gkey) {
        const float dg = key_f32(gkey) - xmax;
        pend = dg >= -26.0f || !zero_weight_irrelevant(P, c);
    }
    pend = pend || (nft > 0 && !(xmax < __builtin_inff()));
    if (pend) {                                                  // uniform
        if (t == 0) P.out_ids[row] = SMP_PENDING;
        return;
    }
    uint64_t w[EPT];
    uint32_t theta = 0;
    if (nft > 0) {
#pragma unroll
        for (int j = 0; j < EPT; ++j) w[j] = key[j] ? wf_u64(weight_f(key_f32(key[j]), xmax)) : 0ull;
        if (c.p < 1.0f) {
            // the candidates are in registers: the array holds the top-p bins from here
            for (uint32_t i = t; i < SMP_PBIN_SLOTS; i += SMP_WIDE) sh.cand[i] = 0;
            if (t == 0) sh.lcount = 0;
            __syncthreads();
            theta = fin_topp_bins<EPT>(key, w, frac32(c.p), kmax, sh.cand, sh);
            if (theta == 0u) {                                   // uniform: a crowded bin
                if (t == 0) P.out_ids[row] = SMP_PENDING;
                return;
            }
        }
    } else {
#pragma unroll
        for (int j = 0; j < EPT; ++j) w[j] = 0;
    }
    const uint64_t mthr = c.m > 0.0f ? frac32(c.m) << 4 : 0;
    uint32_t fmask = 0;
    uint64_t mysum = 0;
#pragma unroll
    for (int j = 0; j < EPT; ++j) {
        const bool f = key[j] && key[j] >= theta && w[j] >= mthr;
        fmask |= f ? (1u << j) : 0u;
        w[j] = f ? w[j] : 0ull;
        mysum += w[j];
    }
    // ---- the draw: a thread's candidates are consecutive ids, so one scan of
    //      the per-thread sums orders the whole row
    uint64_t Zf;
    const uint64_t before = blk_excl_scan_u64<NW>(mysum, &Zf, sh.bs);
    if (Zf == 0) {
        if (t == 0) write_result(P, row, -1, 0.0f);
    } else {
        const uint64_t target = (uint64_t)(((llima_u128)uniform32(c.u) * Zf) >> 32);
        if (mysum > 0 && before <= target && target < before + mysum) {
            uint64_t acc = before;
            bool hit = false;
#pragma unroll
            for (int j = 0; j < EPT; ++j) {
                if (!hit && w[j] && acc <= target && target < acc + w[j]) {
                    write_result(P, row, (int32_t)id[j], (float)((double)w[j] / (double)Zf));
                    hit = true;
                }
                acc += w[j];
            }
        }
    }
    if (P.out_keep) {
        const int nw = (P.V + 31) >> 5;
        uint32_t* km = P.out_keep + (size_t)row * nw;
        for (int i = (int)t; i < nw; i += SMP_WIDE) km[i] = 0;
        __threadfence_block();
        __syncthreads();
#pragma unroll
        for (int j = 0; j < EPT; ++j)
            if ((fmask >> j) & 1u) atomicOr(&km[id[j] >> 5], 1u << (id[j] & 31u));
    }
}

// ================================================================== dense path
// Rows without top-k and without a grammar mask: top-p, min-p or plain
// temperature over the whole row.  The sweep's bound for such rows is the
// chunk maximum - 27 T (a weight is nonzero down to 25.6 nats below the row
// maximum), which on ordinary logits admits nearly every value: every region
// would overflow and one workgroup per row would make the full-row passes.
// These rows are selected instead by the workgroups of all their chunks in
// parallel (one 16 KB chunk per workgroup, the sweep's lane layout), over
// three reads of the row:
//   dense_stats  the chunk's maximum key and finite count, or on greedy rows
//                its (key, first id) maximum;
//   dense_hist   rows with top-p: the chunk's exact weights counted into
//                SMP_DBINS value bins of 1/16 nat below the row maximum (bin
//                floor(16 (xmax - x)), monotone in the key, the last open) as
//                (mass << 14) + count;
//   dense_bound  one workgroup per row with top-p: the chunks' bins merged,
//                and the bin holding the top-p boundary: the last non-empty
//                bin whose mass above, times 2^32, is below p32 Z (the top
//                non-empty bin when none is);
//   dense_keep   the chunk's kept mass strictly above that bin (min-p
//                applied), its words of the kept-set mask, and the bin's
//                members (key, id), staged in LDS and appended to the row's
//                member list;
//   dense_final  one workgroup per row: the members ranked by radix rounds
//                over their keys, starting from the mass above the bin, give
//                theta (the full-row path's boundary: the smallest key whose
//                mass strictly above, times 2^32, is below p32 Z); the kept
//                members' weights are added to their chunks, a scan over the
//                chunks' kept masses finds the chunk of the draw target and a
//                scan of that chunk in id order the token.
// Every weight, bin and test is the full-row path's arithmetic on the same
// values, so the kept set, the token and its probability are the same.  A row
// whose boundary bin holds more members than dense_final ranks (more than
// 4096 values within 1/16 nat, or more than 512 in one chunk: a nearly flat
// row) is finished there by the full-row path.
//
// Region use per row (the row's S regions of SMP_REGION slots):
//   region c, slots [0, SMP_DBINS)  dense_hist's bins of chunk c, then the
//                                   boundary members (member j at region
//                                   j / SMP_DBINS, slot j % SMP_DBINS)
//   region c, SMP_DSTAT / SMP_DBEST  dense_stats's results for chunk c
//   region c, SMP_DKEPT             the kept mass of chunk c (dense_bound or dense_keep)
//   region c, SMP_DMCNT             dense_bound: chunk c's count in the boundary bin
//   region c, SMP_DSWIN             dense_hist: the chunk's highest bins [0, hi]
//                                   holding at most SMP_DSTG values, staged in
//                                   the chunk's slots after the regions
//                                   (hi + 1, 0 for none | the count << 32)
//   region 0, SMP_DINFO..+2         dense_bound's boundary bin, mass above it, Z
//   region 0, SMP_DMEM              members appended (a 128-byte line of its
//                                   own), zeroed by dense_stats
#define SMP_DSTAT 448                              // chunk max key << 32 | finite count
#define SMP_DBEST 449                              // greedy: key << 32 | ~id of the chunk maximum
#define SMP_DKEPT 450                              // kept mass strictly above the boundary bin
#define SMP_DMCNT 451                              // the chunk's members of the boundary bin
#define SMP_DSWIN 452                              // the chunk's staged top window
#define SMP_DINFO 456                              // region 0: boundary bin, mass above it, Z
#define SMP_DMEM 496                               // region 0: boundary members appended
#define SMP_DMCAP 4096                             // members dense_final ranks (16 per thread)
#define SMP_DMWG 512                               // members a dense_keep workgroup stages
static_assert(SMP_DBINS <= SMP_DSTAT && SMP_DMEM + 16 <= SMP_REGION, "dense region layout");
static_assert(SMP_DMCAP == 16 * LLIMA_WG, "dense_final holds 16 members per thread");

template <typename TL>
struct DenseGeom {
    static constexpr int EPL = 16 / (int)sizeof(TL);   // values per 16-byte load
    static constexpr int NL = 4;                       // loads per thread and chunk
    static constexpr int E = NL * EPL;                 // values per thread
    static constexpr int CHUNK = LLIMA_WG * E;         // 4096 fp32 / 8192 bf16 (the sweep's chunk)
    static constexpr int WS = CHUNK / LLIMA_WAVES;     // ids per wave
};
static_assert(DenseGeom<float>::CHUNK == FrGeom<float>::CHUNK &&
              DenseGeom<uint16_t>::CHUNK == FrGeom<uint16_t>::CHUNK, "one chunk size");

__device__ __forceinline__ uint64_t* dense_member(uint64_t* r0, uint32_t j) {
    return r0 + (size_t)(j / SMP_DBINS) * SMP_REGION + (j % SMP_DBINS);
}

__device__ __forceinline__ uint32_t dense_member_cap(int S) {
    const uint32_t n = (uint32_t)S * SMP_DBINS;
    return n < SMP_DMCAP ? n : SMP_DMCAP;
}

// A value after the row's transform, in the full-row path's order: NaN ->
// -inf, the penalties (cnt occurrences in the history), / T unless greedy.
__device__ __forceinline__ float dense_x(float l, uint32_t cnt, const RowCfg& c) {
    if (l != l) l = -__builtin_inff();
    if (cnt) l = penalize(l, cnt, c);
    return c.greedy || c.T == 1.0f ? l : l / c.T;      // l / 1 is l, exactly
}

// The loads of the row's first SMP_HBATCH * LLIMA_WG history ids (clamped to
// H_max; the count checks the row's own length).
__device__ __forceinline__ void dense_hist_ids(const SampleParams& P, int row, int32_t (&hid)[SMP_HBATCH]) {
    const int32_t* hrow = P.hist + (size_t)row * P.H_max;
#pragma unroll
    for (int b = 0; b < SMP_HBATCH; ++b) {
        const int j = (int)threadIdx.x + b * LLIMA_WG;
        hid[b] = hrow[j < P.H_max ? j : P.H_max - 1];
    }
}

// Counts the row's history ids in [lo, lo + n) into table (n / 2 words, two
// 16-bit counts each); the first batch of ids from hid.
__device__ __forceinline__ void dense_count(const SampleParams& P, int row, const RowCfg& c,
                                            const int32_t (&hid)[SMP_HBATCH], int lo, int n,
                                            uint32_t* table) {
    const int t = (int)threadIdx.x;
    for (int i = t; i < n / 8; i += LLIMA_WG) ((llima_u32x4*)table)[i] = llima_u32x4{0, 0, 0, 0};
    __syncthreads();
#pragma unroll
    for (int b = 0; b < SMP_HBATCH; ++b) {
        const int32_t id = hid[b];
        if (t + b * LLIMA_WG < c.hlen && id >= lo && id < lo + n) {
            const uint32_t off = (uint32_t)(id - lo);
            atomicAdd(&table[off >> 1], 1u << ((off & 1u) * 16u));
        }
    }
    const int32_t* hrow = P.hist + (size_t)row * P.H_max;
    for (int j = t + SMP_HBATCH * LLIMA_WG; j < c.hlen; j += LLIMA_WG) {
        const int32_t id = hrow[j];
        if (id >= lo && id < lo + n) {
            const uint32_t off = (uint32_t)(id - lo);
            atomicAdd(&table[off >> 1], 1u << ((off & 1u) * 16u));
        }
    }
    __syncthreads();
}

// Id of value (j, e) of this lane in the chunk from c0: wave w owns ids
// [w WS, (w + 1) WS), load j of lane l covers EPL ids at j 64 EPL + l EPL.
template <typename TL>
__device__ __forceinline__ int dense_id(int c0, int j, int e) {
    using G = DenseGeom<TL>;
    return c0 + (int)wave_id() * G::WS + j * 64 * G::EPL + (int)lane_id() * G::EPL + e;
}

// The chunk's 16-byte loads (clamped, always-valid addresses), issued before
// any use.
template <typename TL>
__device__ __forceinline__ void dense_issue(const SampleParams& P, int row, int c0,
                                            llima_u32x4 (&raw)[DenseGeom<TL>::NL]) {
    using G = DenseGeom<TL>;
    const TL* rowp = (const TL*)P.logits + (size_t)row * P.row_stride;
    const int V = P.V;
    if (P.vec_ok) {
#pragma unroll
        for (int j = 0; j < G::NL; ++j) {
            const int i0 = dense_id<TL>(c0, j, 0);
            const int ia = i0 < V ? i0 : V - G::EPL;
            raw[j] = __builtin_nontemporal_load((const llima_u32x4*)(rowp + ia));
        }
    } else {
#pragma unroll
        for (int j = 0; j < G::NL; ++j) {
            const int i0 = dense_id<TL>(c0, j, 0);
            uint32_t w[4] = {0, 0, 0, 0};
#pragma unroll
            for (int e = 0; e < G::EPL; ++e) {
                const int ia = i0 + e < V ? i0 + e : V - 1;
                const float f = load_one<TL>(rowp, ia);
                if constexpr (sizeof(TL) == 4) w[e] = __float_as_uint(f);
                else w[e >> 1] |= (__float_as_uint(f) >> 16) << ((e & 1) * 16);
            }
            raw[j] = llima_u32x4{w[0], w[1], w[2], w[3]};
        }
    }
}

// The chunk's values after NaN -> -inf and the penalties (not yet divided by
// T); ids past the row are -inf.
template <typename TL>
__device__ __forceinline__ void dense_unpack(const SampleParams& P, const RowCfg& c, int c0,
                                             const llima_u32x4 (&raw)[DenseGeom<TL>::NL],
                                             const uint32_t* table, float (&x)[DenseGeom<TL>::E]) {
    using G = DenseGeom<TL>;
#pragma unroll
    for (int j = 0; j < G::NL; ++j) {
        const uint32_t w4[4] = {raw[j].x, raw[j].y, raw[j].z, raw[j].w};
#pragma unroll
        for (int e = 0; e < G::EPL; ++e) {
            const int i = dense_id<TL>(c0, j, e);
            uint32_t bits;
            if constexpr (sizeof(TL) == 4) bits = w4[e];
            else bits = (e & 1) ? (w4[e >> 1] & 0xFFFF0000u) : (w4[e >> 1] << 16);
            float l = i < P.V ? __uint_as_float(bits) : -__builtin_inff();
            if (l != l) l = -__builtin_inff();
            const uint32_t cnt = c.pen ? table_count(table, (uint32_t)(i - c0)) : 0u;
            x[j * G::EPL + e] = cnt ? penalize(l, cnt, c) : l;
        }
    }
}

// x / T, skipped (a uniform branch) on greedy rows and at T == 1, where it is x.
template <int E>
__device__ __forceinline__ void dense_div(float (&x)[E], const RowCfg& c) {
    if (!c.greedy && c.T != 1.0f) {
#pragma unroll
        for (int i = 0; i < E; ++i) x[i] = x[i] / c.T;
    }
}

// The row's maximum key and finite count from the chunks' statistics, read
// by every wave (lane i: chunks i, i + 64, ...) and reduced with DPP.
__device__ __forceinline__ void dense_row_stats(const SampleParams& P, int row, uint32_t* kmax,
                                                uint32_t* nfin) {
    const uint64_t* r0 = region_of(P, (uint32_t)row, 0);
    uint32_t km = 0, nf = 0;
    for (int i = (int)lane_id(); i < P.S; i += 64) {
        const uint64_t v = r0[(size_t)i * SMP_REGION + SMP_DSTAT];
        const uint32_t k = (uint32_t)(v >> 32);
        km = k > km ? k : km;
        nf += (uint32_t)v;
    }
    *kmax = wave_max_u32(km);
    *nfin = wave_sum_u32(nf);
}

template <typename TL>
__global__ __launch_bounds__(LLIMA_WG) __attribute__((amdgpu_waves_per_eu(8, 8))) void dense_stats(SampleParams P) {
    using G = DenseGeom<TL>;
    extern __shared__ __align__(16) uint32_t table[];   // history counts (rows with penalties)
    __shared__ BlockScratch bs;
    uint32_t row, chunk;
    map_row_chunk(blockIdx.x, (uint32_t)P.B, (uint32_t)P.S, &row, &chunk);
    if (row >= (uint32_t)P.B) return;
    const int c0 = (int)chunk * G::CHUNK;
    int32_t hid[SMP_HBATCH];
    if (P.H_max > 0) dense_hist_ids(P, (int)row, hid);
    llima_u32x4 raw[G::NL];
    dense_issue<TL>(P, (int)row, c0, raw);
    const RowCfg c = load_cfg(P, (int)row);
    if (c.pen) dense_count(P, (int)row, c, hid, c0, G::CHUNK, table);
    float x[G::E];
    dense_unpack<TL>(P, c, c0, raw, table, x);
    uint64_t* reg = region_of(P, row, chunk);
    if (c.greedy) {
        uint64_t best = 0;
#pragma unroll
        for (int j = 0; j < G::NL; ++j)
#pragma unroll
            for (int e = 0; e < G::EPL; ++e) {
                const uint32_t id = (uint32_t)dense_id<TL>(c0, j, e);
                const uint64_t kk = ((uint64_t)f32_key(x[j * G::EPL + e]) << 32) | (uint64_t)(~id);
                best = kk > best ? kk : best;
            }
        best = block_max_u64(best, bs);
        if (threadIdx.x == 0) reg[SMP_DBEST] = best;
    } else {
        // no division: l / T is monotone in l, so the largest quotient is the
        // quotient of the largest l, and l / T rounds to -inf exactly when
        // l <= -T (2^128 - 2^103) (exact in double), so both follow from l
        const double thr = -(double)c.T * 3.4028235677973366e38;
        float lm = -__builtin_inff();
        uint32_t nf = 0;
#pragma unroll
        for (int i = 0; i < G::E; ++i) {
            lm = __builtin_fmaxf(lm, x[i]);
            nf += (double)x[i] > thr ? 1u : 0u;
        }
        uint32_t km = f32_key(lm);
        km = block_max_u32(km, bs);
        nf = block_sum_u32(nf, bs);
        if (threadIdx.x == 0) {
            const float xm = key_f32(km) / c.T;
            reg[SMP_DSTAT] = ((uint64_t)(nf ? f32_key(xm) : 0u) << 32) | nf;
        }
    }
    if (chunk == 0 && threadIdx.x == 0) reg[SMP_DMEM] = 0;
}

// The top-p boundary bin of each row from its chunks' bins, one workgroup per
// row: thread t merges bins 2t and 2t + 1 over the chunks (16-byte loads of up
// to 32 chunks issued before any is used), then a block scan gives each bin's
// mass above.
__global__ __launch_bounds__(LLIMA_WG) void dense_bound(SampleParams P) {
    __shared__ BlockScratch bs;
    const int row = blockIdx.x;
    const RowCfg c = load_cfg(P, row);
    if (c.greedy || !(c.p < 1.0f)) return;              // uniform: no top-p on this row
    uint32_t kmax, nfin;
    dense_row_stats(P, row, &kmax, &nfin);
    if (nfin == 0) return;
    const uint32_t t = threadIdx.x;
    uint64_t* r0 = region_of(P, (uint32_t)row, 0);
    uint32_t cn0 = 0, cn1 = 0;
    uint64_t m0 = 0, m1 = 0;
    if (t < SMP_DBINS / 2) {
        constexpr int NB = 32;
        for (int b0 = 0; b0 < P.S; b0 += NB) {
            llima_u32x4 q[NB];
#pragma unroll
            for (int i = 0; i < NB; ++i) {
                const int ci = b0 + i < P.S ? b0 + i : P.S - 1;
                q[i] = *(const llima_u32x4*)(r0 + (size_t)ci * SMP_REGION + 2u * t);
            }
#pragma unroll
            for (int i = 0; i < NB; ++i) {
                const bool in = b0 + i < P.S;
                const uint64_t h0 = in ? ((uint64_t)q[i].y << 32) | q[i].x : 0ull;
                const uint64_t h1 = in ? ((uint64_t)q[i].w << 32) | q[i].z : 0ull;
                cn0 += (uint32_t)(h0 & 0x3FFFu);
                m0 += h0 >> 14;
                cn1 += (uint32_t)(h1 & 0x3FFFu);
                m1 += h1 >> 14;
            }
        }
    }
    uint64_t Z;
    const uint64_t ab = block_excl_scan_u64(m0 + m1, &Z, bs);   // mass above bin 2t
    const llima_u128 PZ = (llima_u128)frac32(c.p) * Z;
    const bool q0 = cn0 > 0u && (((llima_u128)ab << 32) < PZ);
    const bool q1 = cn1 > 0u && (((llima_u128)(ab + m0) << 32) < PZ);
    const uint32_t qb = block_max_u32(q1 ? 2u * t + 2u : (q0 ? 2u * t + 1u : 0u), bs);
    const uint32_t ne = cn0 ? 2u * t : (cn1 ? 2u * t + 1u : 0xFFFFFFFFu);
    const uint32_t top = ~block_max_u32(~ne, bs);               // top non-empty bin
    const uint32_t bstar = qb ? qb - 1u : top;
    if ((bstar >> 1) == t) {
        r0[SMP_DINFO] = bstar;
        r0[SMP_DINFO + 1] = (bstar & 1u) ? ab + m0 : ab;
        r0[SMP_DINFO + 2] = Z;
    }
    // each chunk's count in b*, so that dense_keep skips the chunks without members
    for (int i = (int)t; i < P.S; i += LLIMA_WG) {
        uint64_t* reg = r0 + (size_t)i * SMP_REGION;
        reg[SMP_DMCNT] = reg[bstar] & 0x3FFFu;
    }
    if (!(c.m > 0.0f)) {
        // Without min-p every value above b* is kept, so each chunk's kept
        // mass is the sum of its bins before b*: 8 threads per chunk (32
        // chunks per round), thread part p summing bin pairs p, p + 8, ...
        // (4 loads in flight), then a reduction over the 8 lanes.
        const uint32_t part = t & 7u, npairs = (bstar + 1u) >> 1;
        for (int cb = 0; cb < P.S; cb += LLIMA_WG / 8) {
            const int ci = cb + (int)(t >> 3);
            const uint64_t* reg = r0 + (size_t)(ci < P.S ? ci : 0) * SMP_REGION;
            uint64_t acc = 0;
            for (uint32_t q0 = part; q0 < npairs; q0 += 32u) {
                llima_u32x4 h[4];
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const uint32_t q = q0 + 8u * (uint32_t)k;
                    h[k] = *(const llima_u32x4*)(reg + 2u * (q < npairs ? q : 0u));
                }
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const uint32_t q = q0 + 8u * (uint32_t)k;
                    const uint64_t a = ((uint64_t)h[k].y << 32) | h[k].x, b = ((uint64_t)h[k].w << 32) | h[k].z;
                    acc += q < npairs ? (a >> 14) + (2u * q + 1u < bstar ? b >> 14 : 0ull) : 0ull;
                }
            }
#pragma unroll
            for (int sft = 1; sft < 8; sft <<= 1) {
                const uint32_t lo = (uint32_t)__shfl_xor((int)(uint32_t)acc, sft);
                const uint32_t hi = (uint32_t)__shfl_xor((int)(uint32_t)(acc >> 32), sft);
                acc += ((uint64_t)hi << 32) | lo;
            }
            if (part == 0 && ci < P.S) r0[(size_t)ci * SMP_REGION + SMP_DKEPT] = acc;
        }
    }
}

template <typename TL>
__global__ __launch_bounds__(LLIMA_WG) __attribute__((amdgpu_waves_per_eu(8, 8))) void dense_hist(SampleParams P) {
    using G = DenseGeom<TL>;
    extern __shared__ __align__(16) uint32_t table[];
    __shared__ uint64_t hist[SMP_DBINS + 64];           // + a spare bin per lane
    __shared__ uint32_t swin_n;                         // values staged so far
    uint32_t row, chunk;
    map_row_chunk(blockIdx.x, (uint32_t)P.B, (uint32_t)P.S, &row, &chunk);
    if (row >= (uint32_t)P.B) return;
    const int c0 = (int)chunk * G::CHUNK;
    int32_t hid[SMP_HBATCH];
    if (P.H_max > 0) dense_hist_ids(P, (int)row, hid);
    llima_u32x4 raw[G::NL];
    dense_issue<TL>(P, (int)row, c0, raw);
    const RowCfg c = load_cfg(P, (int)row);
    if (c.greedy || !(c.p < 1.0f)) return;              // uniform: no top-p on this row
    uint32_t kmax, nfin;
    dense_row_stats(P, (int)row, &kmax, &nfin);
    if (nfin == 0) return;
    const uint32_t t = threadIdx.x, lane = lane_id();
    for (uint32_t i = t; i < SMP_DBINS + 64; i += LLIMA_WG) hist[i] = 0;
    if (t == 0) swin_n = 0;
    if (c.pen) dense_count(P, (int)row, c, hid, c0, G::CHUNK, table);
    __syncthreads();
    float x[G::E];
    dense_unpack<TL>(P, c, c0, raw, table, x);
    dense_div(x, c);
    const float xmax = key_f32(kmax);
    uint32_t bin[G::E];                                 // kept for the staging (fp32)
#pragma unroll
    for (int i = 0; i < G::E; ++i) {
        const bool fin = x[i] > -__builtin_inff();
        const float wf = dense_wf(x[i], xmax);
        const uint32_t b = fin ? (uint32_t)dense_d16(x[i], xmax) : SMP_DBINS + lane;
        bin[i] = b;
        // (W << 14) + 1: W 2^14 < 2^51 is an exact integral float
        atomicAdd((unsigned long long*)&hist[b], (unsigned long long)(wf_u64(wf * 16384.0f) | 1ull));
    }
    __syncthreads();
    uint64_t* reg = region_of(P, row, chunk);
    if (t < SMP_DBINS / 2) {
        const uint64_t h0 = hist[2u * t], h1 = hist[2u * t + 1u];
        ((llima_u32x4*)reg)[t] = llima_u32x4{(uint32_t)h0, (uint32_t)(h0 >> 32), (uint32_t)h1,
                                             (uint32_t)(h1 >> 32)};
    }
    // the chunk's highest values: bins [0, hi] with at most SMP_DSTG values
    // (BPL bins per lane), staged so that dense_keep takes the
    // boundary bin's members from them instead of reading the chunk again.
    // fp32 only: a bf16 thread's 32 values kept live past the binning would
    // not fit the 64 registers of eight waves per SIMD.
    if constexpr (sizeof(TL) != 4) {
        if (t == 0) reg[SMP_DSWIN] = 0;                  // no window
        return;
    }
    // Every wave finds the window itself from the same bins, and stores its
    // own staged values at places from one LDS atomic: no barrier.
    static_assert(SMP_DBINS % 64 == 0, "bins tile the lanes");
    constexpr int BPL = SMP_DBINS / 64;
    uint32_t bc[BPL], lsum = 0;
#pragma unroll
    for (int i = 0; i < BPL; ++i) {
        bc[i] = (uint32_t)(hist[BPL * lane + i] & 0x3FFFu);
        lsum += bc[i];
    }
    const uint32_t cum = wave_incl_scan_u32(lsum);
    const int jl = __builtin_popcountll(ballot(cum <= SMP_DSTG));   // the first lane that does not fit
    int hi = SMP_DBINS - 1;
    uint32_t n = readlane(cum, 63);                          // the window's count
    if (jl < 64) {                                           // uniform
        uint32_t run = cum - lsum, nf = 0, fit = run;
#pragma unroll
        for (int i = 0; i < BPL; ++i) {
            run += bc[i];
            const bool in = run <= SMP_DSTG && nf == (uint32_t)i;
            nf += in ? 1u : 0u;
            fit = in ? run : fit;
        }
        hi = BPL * jl + (int)readlane(nf, (uint32_t)jl) - 1;
        n = readlane(fit, (uint32_t)jl);
    }
    if (t == 0) reg[SMP_DSWIN] = (uint64_t)(uint32_t)(hi + 1) | ((uint64_t)n << 32);
    if (hi >= 0) {                                           // uniform
        uint32_t sm = 0;
#pragma unroll
        for (int i = 0; i < G::E; ++i)
            sm |= (int)bin[i] <= hi ? 1u << i : 0u;          // -inf: a spare bin, above hi
        if (ballot(sm != 0u)) {                              // uniform in the wave
            const uint32_t cnt = (uint32_t)__popc(sm);
            const uint32_t inc = wave_incl_scan_u32(cnt);
            uint32_t base = 0;
            if (lane == 63) base = atomicAdd(&swin_n, inc);
            base = readlane(base, 63) + inc - cnt;
            uint64_t* dst = P.xstg + ((size_t)row * (uint32_t)P.S + chunk) * SMP_XSTG;
#pragma unroll
            for (int j = 0; j < G::NL; ++j)
#pragma unroll
                for (int e = 0; e < G::EPL; ++e)
                    if ((sm >> (j * G::EPL + e)) & 1u) {
                        if (base < SMP_DSTG)                 // always: the window's count
                            dst[base] = ((uint64_t)f32_key(x[j * G::EPL + e]) << 32) |
                                        (uint32_t)dense_id<TL>(c0, j, e);
                        ++base;
                    }
        }
    }
}

template <typename TL>
__global__ __launch_bounds__(LLIMA_WG) __attribute__((amdgpu_waves_per_eu(sizeof(TL) == 4 ? 8 : 1))) void dense_keep(SampleParams P) {
    using G = DenseGeom<TL>;
    extern __shared__ __align__(16) uint32_t table[];
    __shared__ BlockScratch bs;
    __shared__ uint64_t mbuf[SMP_DMWG];                 // the chunk's boundary members
    __shared__ uint32_t mcount, mbase;
    uint32_t row, chunk;
    map_row_chunk(blockIdx.x, (uint32_t)P.B, (uint32_t)P.S, &row, &chunk);
    if (row >= (uint32_t)P.B) return;
    const int c0 = (int)chunk * G::CHUNK;
    const RowCfg c = load_cfg(P, (int)row);
    if (c.greedy) return;                               // dense_final writes greedy rows
    const bool topp = c.p < 1.0f;
    // top-p rows without min-p or a kept-set output need this pass only for
    // the boundary bin's members: chunks without any leave before loading,
    // and chunks whose staged top window holds the boundary bin take them
    // from it (wave 0) instead of reading the chunk
    if (topp && !(c.m > 0.0f) && !P.out_keep) {         // uniform
        const uint64_t* creg = region_of(P, row, chunk);
        uint64_t* r0s = region_of(P, row, 0);
        const uint32_t lane = lane_id();
        // the staged path's loads, all requested before any is used (a lane
        // past the window's count reads an unused slot)
        const uint64_t mv = creg[SMP_DMCNT], win = creg[SMP_DSWIN], binfo = r0s[SMP_DINFO];
        const uint64_t v = P.xstg[((size_t)row * (uint32_t)P.S + chunk) * SMP_XSTG + lane];
        uint32_t kmax, nfin;
        dense_row_stats(P, (int)row, &kmax, &nfin);
        const uint32_t mcnt = (uint32_t)mv;
        if (mcnt == 0u) return;                          // uniform
        const uint32_t bs_ = (uint32_t)binfo;
        if ((uint32_t)win > bs_) {                       // uniform: bins [0, hi] hold b*
            if (wave_id() != 0 || nfin == 0) return;     // (nfin == 0: dense_bound did not run)
            const float xmax = key_f32(kmax);
            const uint32_t n = (uint32_t)(win >> 32);
            const bool mem = lane < n && (uint32_t)dense_d16(key_f32((uint32_t)(v >> 32)), xmax) == bs_;
            const uint64_t bm = ballot(mem);
            const uint32_t nm = (uint32_t)__popcll(bm);
            const uint32_t cap = dense_member_cap(P.S);
            // the bin's count from dense_bound: a mismatch (never) leaves the
            // row's member count above the cap, so dense_final takes the full-row path
            uint32_t base = 0;
            if (lane == 0) base = arrive_agent((uint32_t*)(r0s + SMP_DMEM), nm == mcnt ? nm : cap + 1u);
            base = readlane(base, 0);
            const uint32_t o = base + (uint32_t)__popcll(bm & ((1ull << lane) - 1ull));
            if (mem && nm == mcnt && o < cap) *dense_member(r0s, o) = v;
            return;
        }
    }
    int32_t hid[SMP_HBATCH];
    if (P.H_max > 0) dense_hist_ids(P, (int)row, hid);
    llima_u32x4 raw[G::NL];
    dense_issue<TL>(P, (int)row, c0, raw);
    uint64_t* r0 = region_of(P, row, 0);
    // the boundary bin requested with the statistics (both written by earlier launches)
    const uint64_t binfo = r0[SMP_DINFO];
    uint32_t kmax, nfin;
    dense_row_stats(P, (int)row, &kmax, &nfin);
    if (nfin == 0) return;
    const uint32_t bstar = topp ? (uint32_t)binfo : (uint32_t)SMP_DBINS;
    if (threadIdx.x == 0) mcount = 0;
    if (c.pen) dense_count(P, (int)row, c, hid, c0, G::CHUNK, table);
    else __syncthreads();
    float x[G::E];
    dense_unpack<TL>(P, c, c0, raw, table, x);
    dense_div(x, c);
    const float xmax = key_f32(kmax);
    const float mthr = dense_mthr(c);
    const float blo = (float)bstar, bhi = (float)bstar + 1.0f;   // bin b*: d16 in [blo, bhi)
    const uint32_t lane = lane_id();
    const int nw = (P.V + 31) >> 5;
    uint32_t* kw = P.out_keep + (size_t)row * nw;
    // top-p rows without min-p: dense_bound summed each chunk's kept mass from
    // its bins, and no weight is needed here
    const bool need_w = !topp || c.m > 0.0f;
    double kmd = 0.0;                                   // at most 32 weights below 2^37: exact
    uint32_t mb = 0;                                    // this thread's boundary members
#pragma unroll
    for (int j = 0; j < G::NL; ++j) {
        uint32_t kb = 0;
#pragma unroll
        for (int e = 0; e < G::EPL; ++e) {
            const float xv = x[j * G::EPL + e];
            const bool fin = xv > -__builtin_inff();
            const float d16 = dense_d16(xv, xmax);
            bool kept = fin && d16 < blo;
            if (need_w && ballot(kept)) {               // uniform: weights only where some lane keeps
                const float wf = dense_wf(xv, xmax);
                kept = kept && wf >= mthr;
                kmd += kept ? (double)wf : 0.0;
            }
            kb |= kept ? 1u << e : 0u;
            mb |= fin && d16 >= blo && d16 < bhi ? 1u << (j * G::EPL + e) : 0u;
        }
        if (P.out_keep) {
            // lanes sharing a 32-id word: 32 / EPL of them (the chunk starts on a word)
            constexpr int LPW = 32 / G::EPL;
            uint32_t word = kb << ((lane * G::EPL) & 31u);
#pragma unroll
            for (int s = 1; s < LPW; s <<= 1) word |= (uint32_t)__shfl_xor((int)word, s);
            const int i0 = dense_id<TL>(c0, j, 0);
            if ((lane & (LPW - 1)) == 0 && i0 < P.V) kw[i0 >> 5] = word;
        }
    }
    // boundary members, staged in LDS (one LDS atomic per wave that has any)
    if (ballot(mb != 0u)) {                              // uniform
        const uint32_t cnt = (uint32_t)__popc(mb);
        const uint32_t inc = wave_incl_scan_u32(cnt);
        uint32_t base = 0;
        if (lane == 63) base = atomicAdd(&mcount, inc);
        base = readlane(base, 63) + inc - cnt;
#pragma unroll
        for (int j = 0; j < G::NL; ++j)
#pragma unroll
            for (int e = 0; e < G::EPL; ++e)
                if ((mb >> (j * G::EPL + e)) & 1u) {
                    if (base < SMP_DMWG)
                        mbuf[base] = ((uint64_t)f32_key(x[j * G::EPL + e]) << 32) |
                                     (uint32_t)dense_id<TL>(c0, j, e);
                    ++base;
                }
    }
    const uint64_t km = block_sum_u64((uint64_t)kmd, bs);   // its barriers also settle mcount
    if (threadIdx.x == 0 && need_w) region_of(P, row, chunk)[SMP_DKEPT] = km;
    const uint32_t n = mcount;
    if (n) {                                             // uniform
        // a workgroup with more members than it stages makes the row's count
        // exceed what dense_final ranks (that row then takes the full-row path)
        const uint32_t cap = dense_member_cap(P.S);
        if (threadIdx.x == 0)
            mbase = arrive_agent((uint32_t*)(r0 + SMP_DMEM), n <= SMP_DMWG ? n : cap + 1u);
        __syncthreads();
        const uint32_t o = mbase;
        if (n <= SMP_DMWG)
            for (uint32_t i = threadIdx.x; i < n; i += LLIMA_WG)
                if (o + i < cap) *dense_member(r0, o + i) = mbuf[i];
    }
}

template <typename TL>
__global__ __launch_bounds__(LLIMA_WG) void dense_final(SampleParams P) {
    using G = DenseGeom<TL>;
    constexpr int EPT = SMP_DMCAP / LLIMA_WG;
    __shared__ FinShared sh;
    __shared__ uint64_t cmass[SMP_MAX_S];
    __shared__ uint32_t dsel;
    __shared__ uint64_t drel;
    const int row = blockIdx.x;
    const RowCfg c = load_cfg(P, row);
    const uint32_t t = threadIdx.x;
    const int S = P.S;
    uint64_t* r0 = region_of(P, (uint32_t)row, 0);
    if (t == 0) {             // overwritten by the thread whose chunk holds the target
        dsel = 0;
        drel = 0;
    }
    if (c.greedy) {
        uint64_t best = 0;
        for (int i = (int)t; i < S; i += LLIMA_WG) {
            const uint64_t v = r0[(size_t)i * SMP_REGION + SMP_DBEST];
            best = v > best ? v : best;
        }
        best = block_max_u64(best, sh.bs);
        const bool ok = (uint32_t)(best >> 32) > LLIMA_KEY_NEG_INF;
        const uint32_t tok = ok ? ~(uint32_t)best : 0xFFFFFFFFu;
        if (t == 0) write_result(P, row, ok ? (int32_t)tok : -1, ok ? 1.0f : 0.0f);
        if (P.out_keep)
            write_keep(P, row, [&](auto set) { if (t == 0 && ok) set(tok); });
        return;
    }
    // requested together, before the statistics are reduced: the member
    // count, the boundary's mass above and Z, the chunks' kept masses and the
    // first LLIMA_WG member slots (always inside region 0's member slots)
    const bool topp = c.p < 1.0f;
    const uint32_t nmem = topp ? *(const uint32_t*)(r0 + SMP_DMEM) : 0u;
    const uint64_t above = r0[SMP_DINFO + 1], Z = r0[SMP_DINFO + 2];
    const uint64_t v0 = topp ? *dense_member(r0, t) : 0ull;
    const uint64_t cm = (int)t < S ? r0[(size_t)t * SMP_REGION + SMP_DKEPT] : 0ull;
    uint32_t kmax, nfin;
    dense_row_stats(P, row, &kmax, &nfin);
    if (nfin == 0) {
        if (t == 0) write_result(P, row, -1, 0.0f);
        if (P.out_keep) write_keep(P, row, [&](auto) {});
        return;
    }
    const float xmax = key_f32(kmax);
    if (topp && (nmem == 0u || nmem > dense_member_cap(S))) {   // uniform
        finish_full_row<TL>(P, row, c, sh);
        return;
    }
    const float mthr = dense_mthr(c);
    if ((int)t < S) cmass[t] = cm;
    uint32_t theta = 0;
    const int nw = (P.V + 31) >> 5;
    if (topp && nmem <= 64u) {
        // at most 64 members: ranked pairwise in every wave (lane l holds
        // member l); theta is the smallest key whose mass strictly above,
        // counted from the bin's, times 2^32, is below p32 Z (the largest key
        // when none is: p32 Z < 2^32)
        const uint32_t mk = (uint32_t)(v0 >> 32), mi = (uint32_t)v0;
        const uint64_t mw = t < nmem ? wf_u64(dense_wf(key_f32(mk), xmax)) : 0ull;
        if (t < nmem) sh.sv[t] = llima_u32x4{mk, mi, (uint32_t)mw, (uint32_t)(mw >> 32)};
        __syncthreads();
        const uint32_t lane = lane_id();
        const llima_u32x4 me = lane < nmem ? sh.sv[lane] : llima_u32x4{0u, 0u, 0u, 0u};
        uint64_t ab = above;
        for (uint32_t i = 0; i < nmem; ++i) {
            const llima_u32x4 o = sh.sv[i];
            ab += o.x > me.x ? (((uint64_t)o.w << 32) | o.z) : 0ull;
        }
        const llima_u128 PZ = (llima_u128)frac32(c.p) * Z;
        const uint64_t lim = (uint64_t)((PZ + 0xFFFFFFFFull) >> 32);   // a 2^32 < PZ  <=>  a < lim
        const bool q = lane < nmem && ab < lim;
        theta = ballot(q) ? ~wave_max_u32(q ? ~me.x : 0u) : wave_max_u32(me.x);
        if (t < nmem && mk >= theta && (float)mw >= mthr) {
            atomicAdd((unsigned long long*)&cmass[mi / (uint32_t)G::CHUNK], (unsigned long long)mw);
            if (P.out_keep) atomicOr(P.out_keep + (size_t)row * nw + (mi >> 5), 1u << (mi & 31u));
        }
    } else if (topp) {
        uint32_t key[EPT], mid[EPT];
        uint64_t w[EPT];
#pragma unroll
        for (int e = 0; e < EPT; ++e) {
            const uint32_t j = t + (uint32_t)e * LLIMA_WG;
            const uint64_t v = j < nmem ? *dense_member(r0, j) : 0ull;
            key[e] = (uint32_t)(v >> 32);
            mid[e] = (uint32_t)v;
        }
        uint32_t mk = 0, nmk = 0;
#pragma unroll
        for (int e = 0; e < EPT; ++e) {
            w[e] = key[e] ? wf_u64(dense_wf(key_f32(key[e]), xmax)) : 0ull;
            mk = key[e] > mk ? key[e] : mk;
            nmk = key[e] && ~key[e] > nmk ? ~key[e] : nmk;
        }
        sh.hmass[0][t] = 0;
        sh.hmass[1][t] = 0;
        mk = block_max_u32(mk, sh.bs);
        const uint32_t mkmin = ~block_max_u32(nmk, sh.bs);
        const uint64_t p32 = frac32(c.p);
        theta = fin_topp_desc<EPT>(key, w, p32, mkmin, mk, sh, above, (llima_u128)p32 * Z, true);
#pragma unroll
        for (int e = 0; e < EPT; ++e) {
            if (key[e] && key[e] >= theta && (float)w[e] >= mthr) {
                atomicAdd((unsigned long long*)&cmass[mid[e] / (uint32_t)G::CHUNK], (unsigned long long)w[e]);
                if (P.out_keep)
                    atomicOr(P.out_keep + (size_t)row * nw + (mid[e] >> 5), 1u << (mid[e] & 31u));
            }
        }
    }
    __syncthreads();
    // the chunk holding the draw target
    const uint64_t m = (int)t < S ? cmass[t] : 0ull;
    uint64_t Zf;
    const uint64_t below = block_excl_scan_u64(m, &Zf, sh.bs);
    if (Zf == 0) {
        if (t == 0) write_result(P, row, -1, 0.0f);
        return;
    }
    const uint64_t target = (uint64_t)(((llima_u128)uniform32(c.u) * Zf) >> 32);
    if (m > 0 && below <= target && target < below + m) {
        dsel = t;
        drel = target - below;
    }
    __syncthreads();
    const int cs = (int)dsel;
    const uint64_t rel = drel;
    // that chunk in id order: thread t holds ids c0 + E t .. c0 + E t + E - 1
    const int c0 = cs * G::CHUNK;
    const int c1 = c0 + G::CHUNK < P.V ? c0 + G::CHUNK : P.V;
    if (c.pen) count_history(P, row, c.hlen, c0, c1, sh.u.table, G::CHUNK / 2);
    const TL* rowp = (const TL*)P.logits + (size_t)row * P.row_stride;
    const int i0 = c0 + (int)t * G::E;
    float xs[G::E];
#pragma unroll
    for (int g = 0; g < G::E; g += SMP_FE) {
        float sub[SMP_FE];
        load_fe<TL>(rowp, i0 + g, c1, P.vec_ok != 0, sub);
#pragma unroll
        for (int e = 0; e < SMP_FE; ++e) xs[g + e] = sub[e];
    }
    uint64_t wk[G::E];
    uint64_t s = 0;
#pragma unroll
    for (int e = 0; e < G::E; ++e) {
        const int i = i0 + e;
        const float l = i < c1 ? xs[e] : -__builtin_inff();
        const uint32_t cnt = c.pen && i < c1 ? table_count(sh.u.table, (uint32_t)(i - c0)) : 0u;
        const float xv = dense_x(l, cnt, c);
        const uint32_t k = f32_key(xv);
        const float wf = dense_wf(xv, xmax);
        const bool kept = k > LLIMA_KEY_NEG_INF && k >= theta && wf >= mthr;
        wk[e] = kept ? wf_u64(wf) : 0ull;
        s += wk[e];
    }
    uint64_t tot;
    const uint64_t bl = block_excl_scan_u64(s, &tot, sh.bs);
    if (s > 0 && bl <= rel && rel < bl + s) {
        uint64_t acc = bl;
        int32_t tok = -1;
        uint64_t wtok = 0;
#pragma unroll
        for (int e = 0; e < G::E; ++e) {
            const bool hit = tok < 0 && wk[e] > 0 && rel < acc + wk[e];
            tok = hit ? i0 + e : tok;
            wtok = hit ? wk[e] : wtok;
            acc += wk[e];
        }
        write_result(P, row, tok, (float)((double)wtok / (double)Zf));
    }
}

// ================================================================== host side
static int chunk_values(int dtype) { return dtype == LLIMA_F32 ? 4096 : 8192; }

#define SMP_SWEEP_SC 1                             // chunks per sweep workgroup

template <typename TL>
static void launch_sweep(const SampleParams& P, hipStream_t st) {
    constexpr int SC = SMP_SWEEP_SC;
    const dim3 g((uint32_t)P.B * (uint32_t)((P.S + SC - 1) / SC)), b(LLIMA_WG);
    // the history count table (dynamic LDS) only when the sweep penalises
    const size_t cnt_bytes = (P.H_max > 0 && P.eager) ? (size_t)SC * (16 / sizeof(TL)) * 4 * LLIMA_WG / 2 * 4 : 0;
    if (P.bitmask) {
        if (P.vec_ok) hipLaunchKernelGGL((sample_sweep<TL, true, true, SC>), g, b, cnt_bytes, st, P);
        else hipLaunchKernelGGL((sample_sweep<TL, false, true, SC>), g, b, cnt_bytes, st, P);
    } else {
        if (P.vec_ok) hipLaunchKernelGGL((sample_sweep<TL, true, false, SC>), g, b, cnt_bytes, st, P);
        else hipLaunchKernelGGL((sample_sweep<TL, false, false, SC>), g, b, cnt_bytes, st, P);
    }
}

// The dense path's launches: three reads of the rows by B x S workgroups
// (dense_hist and dense_bound only when some row has top-p), then one
// workgroup per row.
template <typename TL>
static void launch_dense(const SampleParams& P, bool topp, hipStream_t st) {
    const dim3 g((uint32_t)P.B * (uint32_t)P.S), b(LLIMA_WG);
    const size_t tb = P.H_max > 0 ? (size_t)DenseGeom<TL>::CHUNK / 2 * sizeof(uint32_t) : 0;
    hipLaunchKernelGGL(dense_stats<TL>, g, b, tb, st, P);
    if (topp) {
        hipLaunchKernelGGL(dense_hist<TL>, g, b, tb, st, P);
        hipLaunchKernelGGL(dense_bound, dim3((uint32_t)P.B), b, 0, st, P);
    }
    hipLaunchKernelGGL(dense_keep<TL>, g, b, tb, st, P);
    hipLaunchKernelGGL(dense_final<TL>, dim3((uint32_t)P.B), b, 0, st, P);
}

}  // namespace llima

using namespace llima;

extern "C" size_t llima_sample_workspace_bytes(int32_t B, int32_t V, int32_t dtype) {
    if (B <= 0 || V <= 0 || (dtype != LLIMA_F32 && dtype != LLIMA_BF16)) return 0;
    const size_t S = (size_t)((V + chunk_values(dtype) - 1) / chunk_values(dtype));
    // the chunk regions, the split-row staging of every chunk, then one
    // split-row arrival counter (64 bytes) per row
    return (size_t)B * S * (SMP_REGION + SMP_XSTG) * sizeof(uint64_t) + (size_t)B * SMP_RCNT * sizeof(uint32_t);
}

#ifdef LLIMA_FINISH_TRACE
// Copies the phase-trace table ([SMP_TRACE_ROWS][SMP_TRACE_MARKS] uint64) of
// the current device to host memory (traced builds only).
extern "C" int llima_finish_trace_read(unsigned long long* host) {
    return hipMemcpyFromSymbol(host, HIP_SYMBOL(llima::fin_trace), sizeof(llima::fin_trace)) == hipSuccess
               ? LLIMA_OK : LLIMA_E_HIP;
}
#endif

extern "C" int llima_sample(const void* logits, int32_t dtype, int32_t B, int32_t V,
                            int64_t row_stride, const int32_t* history,
                            const int32_t* history_len, int32_t H_max, const uint32_t* bitmask,
                            const float* uniforms, const llima_sampler_config* cfg,
                            int32_t* out_ids, float* out_probs, uint32_t* out_keep,
                            void* workspace, size_t workspace_bytes, void* stream) {
    if (!cfg || (B > 0 && (!logits || !out_ids || !uniforms))) return LLIMA_E_INVAL;
    if (dtype != LLIMA_F32 && dtype != LLIMA_BF16) return LLIMA_E_INVAL;
    if (B < 0 || V <= 0 || V > (1 << 24) || row_stride < V) return LLIMA_E_INVAL;
    if (history && (H_max < 0 || H_max >= 65536)) return LLIMA_E_INVAL;
    if (B == 0) return LLIMA_OK;
    if (!workspace || workspace_bytes < llima_sample_workspace_bytes(B, V, dtype) ||
        ((uintptr_t)workspace & 15u))
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
    P.ws = (uint64_t*)workspace;
    P.B = B;
    P.V = V;
    P.H_max = history ? H_max : 0;
    const int chunk = chunk_values(dtype);
    P.S = (V + chunk - 1) / chunk;
    int lgs = 0;
    while ((1 << lgs) < P.S && lgs < 8) ++lgs;
    P.lgs = lgs;
    {
        const int k = cfg->top_k;
        P.rank = (k > 0 && k < V) ? (int32_t)bound_rank(k, P.S) : 0;
    }
    const size_t esz = dtype == LLIMA_F32 ? 4 : 2;
    P.vec_ok = ((uintptr_t)logits % 16 == 0) && ((row_stride * (int64_t)esz) % 16 == 0) &&
               (V % (int32_t)(16 / esz) == 0);
    // Penalties: a row takes them in the finish, to its candidates only, when
    // it samples with top-k and they can only lower a value (row_lazy, decided
    // per row on the device); otherwise in the sweep.  With one broadcast
    // configuration every row decides alike, and the sweep's history count
    // table is allocated only when they are applied there.
    const bool rows_cfg = cfg->temperature_rows || cfg->top_k_rows || cfg->repetition_penalty_rows ||
                          cfg->presence_penalty_rows || cfg->frequency_penalty_rows;
    const bool all_lazy = !rows_cfg && !cfg->greedy && cfg->temperature > 0.0f &&
                          cfg->top_k > 0 && cfg->top_k < V && cfg->repetition_penalty >= 1.0f &&
                          cfg->presence_penalty >= 0.0f && cfg->frequency_penalty >= 0.0f;
    P.lazy = P.H_max > 0 && !cfg->greedy && (rows_cfg || all_lazy);
    P.eager = P.H_max > 0 && !all_lazy;
    hipStream_t st = (hipStream_t)stream;
    // Masked batches without top-k: the wide finish first (sample_finish then
    // takes only the rows it left)
    P.wide = bitmask && !cfg->greedy && !cfg->top_k_rows && !(cfg->top_k > 0 && cfg->top_k < V) &&
             P.S <= SMP_MAX_S;
    // Rows without top-k whose candidates overflow are split over
    // ceil(S / P.rcpw) finish workgroups in batches that keep the two-launch
    // path: per-row top-k (rows of either kind), or a mask without top-k.  With
    // per-row top-k, a scalar top_k in (0, V) is the caller's word that every
    // row has top-k (a row without then takes the full-row path: slower, not
    // wrong), and the lean finish is launched.
    const bool rows_may_lack_topk = cfg->top_k_rows && !(cfg->top_k > 0 && cfg->top_k < V);
    P.xstg = P.ws + (size_t)B * P.S * SMP_REGION;
    P.rcnt = (uint32_t*)(P.xstg + (size_t)B * P.S * SMP_XSTG);
    // Chunks per part: three under a mask (every row of such a batch may be
    // split, and the finish's two workgroups per CU still hold all the parts
    // of 32 rows of 38 chunks), four with per-row top-k (the rows with top-k
    // finish beside the parts; three measured slower there).
    P.rcpw = P.wide ? 3 : SMP_RCPW;
    // Staged values per chunk: masked rows need more of them for a window that
    // holds the row's boundary bin (about 135 values of a half-masked chunk lie
    // at or above it) than unmasked ones, whose extra staging only costs time.
    P.scap = P.wide ? SMP_STG_CAP : 124;
    P.fsplit = (!cfg->greedy && !out_keep && P.S <= SMP_MAX_S && (rows_may_lack_topk || P.wide))
                   ? (P.S + P.rcpw - 1) / P.rcpw : 1;
    // Rows without top-k (and without a mask) take the dense path: their sweep
    // bound would admit nearly every value of ordinary logits.
    const bool dense = !bitmask && !cfg->greedy && !cfg->top_k_rows &&
                       !(cfg->top_k > 0 && cfg->top_k < V) &&
                       (cfg->temperature_rows || cfg->temperature > 0.0f) && P.S <= SMP_MAX_S;
    if (dense) {
        const bool topp = cfg->top_p_rows || cfg->top_p < 1.0f;
        if (dtype == LLIMA_F32) launch_dense<float>(P, topp, st);
        else launch_dense<uint16_t>(P, topp, st);
    } else if (dtype == LLIMA_F32) {
        launch_sweep<float>(P, st);
        if (P.wide) hipLaunchKernelGGL(sample_finish_wide<float>, dim3(B), dim3(SMP_WIDE), 0, st, P);
        if (P.fsplit > 1) hipLaunchKernelGGL((sample_finish<float, true>), dim3(B, P.fsplit), dim3(LLIMA_WG), 0, st, P);
        else hipLaunchKernelGGL((sample_finish<float, false>), dim3(B), dim3(LLIMA_WG), 0, st, P);
    } else {
        launch_sweep<uint16_t>(P, st);
        if (P.wide) hipLaunchKernelGGL(sample_finish_wide<uint16_t>, dim3(B), dim3(SMP_WIDE), 0, st, P);
        if (P.fsplit > 1) hipLaunchKernelGGL((sample_finish<uint16_t, true>), dim3(B, P.fsplit), dim3(LLIMA_WG), 0, st, P);
        else hipLaunchKernelGGL((sample_finish<uint16_t, false>), dim3(B), dim3(LLIMA_WG), 0, st, P);
    }
    return hipGetLastError() == hipSuccess ? LLIMA_OK : LLIMA_E_HIP;
}

// ================================================================== no-alloc variant
// llima_sample_noalloc: llima_sample with its workspace in a static device
// array instead of a caller buffer, for callers that cannot allocate (code under
// HIP graph capture, serving loops that forbid hipMalloc).  The array is
// allocated on each GPU when the library's code object is loaded there and is
// held until the process ends.  Its name is a host-side stand-in, not a device
// address: host code uses only the address hipGetSymbolAddress returns, looked
// up once per device with that device current and kept in g_scratch_dev.
// The sampler keeps no state in its workspace between calls (every slot a call
// reads is written earlier in the same call), so nothing needs clearing; calls
// that overlap on one GPU share the array and race.
#define LLIMA_SAMPLE_SCRATCH_BYTES ((size_t)48 << 20)
#define LLIMA_SCRATCH_MAX_DEVICES 64

static __device__ __align__(256) uint64_t scratch[LLIMA_SAMPLE_SCRATCH_BYTES / sizeof(uint64_t)];

static std::mutex g_scratch_mu;
static void* g_scratch_dev[LLIMA_SCRATCH_MAX_DEVICES];   // guarded by g_scratch_mu

static int scratch_of_current_device(hipStream_t stream, void** out) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= LLIMA_SCRATCH_MAX_DEVICES)
        return LLIMA_E_HIP;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_dev[dev]) {
        // the lookup may load the library's code object on this device, which
        // is no stream operation a capture could record: the first call on a
        // device must come before any capture
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        if (hipStreamIsCapturing(stream, &cs) != hipSuccess) return LLIMA_E_HIP;
        if (cs != hipStreamCaptureStatusNone) return LLIMA_E_CAPTURE;
        void* p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return LLIMA_E_HIP;
        g_scratch_dev[dev] = p;
    }
    *out = g_scratch_dev[dev];
    return LLIMA_OK;
}

extern "C" size_t llima_sample_noalloc_max_bytes(void) { return LLIMA_SAMPLE_SCRATCH_BYTES; }

extern "C" int llima_sample_noalloc(const void* logits, int32_t dtype, int32_t B, int32_t V,
                                    int64_t row_stride, const int32_t* history,
                                    const int32_t* history_len, int32_t H_max,
                                    const uint32_t* bitmask, const float* uniforms,
                                    const llima_sampler_config* cfg, int32_t* out_ids,
                                    float* out_probs, uint32_t* out_keep, void* stream) {
    const size_t need = llima_sample_workspace_bytes(B, V, dtype);
    if (B <= 0 || need == 0)   // an empty call, or sizes llima_sample rejects: nothing is launched
        return llima_sample(logits, dtype, B, V, row_stride, history, history_len, H_max, bitmask,
                            uniforms, cfg, out_ids, out_probs, out_keep, nullptr, 0, stream);
    if (need > LLIMA_SAMPLE_SCRATCH_BYTES) return LLIMA_E_SCRATCH;
    void* ws = nullptr;
    const int rc = scratch_of_current_device((hipStream_t)stream, &ws);
    if (rc != LLIMA_OK) return rc;
    return llima_sample(logits, dtype, B, V, row_stride, history, history_len, H_max, bitmask,
                        uniforms, cfg, out_ids, out_probs, out_keep, ws,
                        LLIMA_SAMPLE_SCRATCH_BYTES, stream);
}
