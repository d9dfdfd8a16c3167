// sample.hip -- fused penalty / temperature / mask / top-k / top-p / min-p /
// inverse-CDF sampling over [B, V] logits rows on MI355X (gfx950).
//
// One launch per step.  The grid is B x S workgroups; workgroup (row, chunk)
// streams a 256*E-element chunk of its row once from HBM with 16-byte loads
// and keeps it in registers:
//   1. history ids of the row that fall in the chunk are counted in an LDS
//      table (packed u16 counts); distinct ids become "exceptions" whose
//      penalised value is computed separately, so the streaming loop only
//      tests a count != 0 per element (no division in the hot loop);
//   2. masked (packed-uint32 grammar bitmask, LSB first), NaN and history
//      elements are set to -inf in registers;
//   3. a lower bound t of the chunk's k-th largest value is found from the
//      lane maxima (wavefront bitonic sort, min over the 4 waves) and every
//      element >= t - |t|*2^-20 is appended to the row's candidate list;
//   4. the last workgroup of the row to finish (device-scope counter) divides
//      the candidates by the temperature, verifies that the bound could not
//      have dropped a member of the top-k set, and runs three radix selects
//      over LDS histograms on register-resident candidates: top-k threshold
//      (count), top-p threshold (fixed-point mass), and the draw (mass by id).
// Rows the fast path cannot prove complete (candidate overflow, very large k,
// top-k disabled without a mask, degenerate temperatures) are finished by the
// same last workgroup with a full-row multi-pass version of the same selects.
//
// The sampling semantics have no counterpart in the reference runtime, which
// only ever takes the argmax (sima_lmm/devkit/cpp/utils.hpp:80-152,
// sima_lmm/devkit/cpp/language_model.cpp:3689-3714); greedy rows here follow
// that argmax (first index of the maximum) over the masked, penalised row.
#include "common.hpp"
#include "../../include/llima_sampler.h"

namespace llima {

#define SAMPLE_RCAP 4096          // candidates per row (finish holds 16 per thread)
#define SAMPLE_SLOTS (SAMPLE_RCAP / LLIMA_WG)
#define SAMPLE_PRECAP 1024        // candidates per chunk staged in LDS
#define SAMPLE_EXC_CAP 512        // distinct history ids per chunk

#define CTL_OVERFLOW 1u
#define CTL_FILTERED 2u

struct RowCtl {
    uint32_t done;       // workgroups of the row that have finished the sweep
    uint32_t count;      // candidates appended
    uint32_t flags;      // CTL_*
    uint32_t tmax_key;   // max over chunks of the filter bound's key
    uint64_t greedy;     // max over chunks of (key << 32 | ~index)
    uint64_t pad;
};

// Workspace: one fixed-size slot per row index, [RowCtl | SAMPLE_RCAP candidates],
// so the position of a row's control words never depends on B or V and a
// workspace can be reused for any shape (control words are left zero).
#define SAMPLE_CTL_BYTES 256
#define SAMPLE_SLOT_BYTES (SAMPLE_CTL_BYTES + SAMPLE_RCAP * 8)

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
    char* ws;            // B slots of SAMPLE_SLOT_BYTES
    int32_t B, V, H_max, S;
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

__device__ __forceinline__ float penalize(float l, uint32_t c, const RowCfg& cfg) {
    l = (l < 0.0f) ? l * cfg.R : l / cfg.R;
    return (l - cfg.beta * (float)c) - cfg.alpha;
}

// The pre-filter bound lowered by a relative 2^-20, so that no value whose
// quotient by T can round onto the bound's quotient is filtered out.
__device__ __forceinline__ float lower_bound_margin(float t) {
    return t - __builtin_fabsf(t) * 0x1p-20f;
}

template <int CHUNK>
struct SampleShared {
    struct {
        uint32_t cnt[CHUNK / 2];              // packed u16 history counts
        int32_t exc_id[SAMPLE_EXC_CAP];
        float exc_val[SAMPLE_EXC_CAP];
        uint64_t pre[SAMPLE_PRECAP];
    } s;
    struct {
        uint32_t hcnt[256];
        uint64_t hmass[256];
    } f;
    uint32_t n_exc, n_pre, flags, base;
    uint32_t sel, wave_bound[LLIMA_WAVES];
    uint64_t sel64, sel64b;
    uint32_t last;
    BlockScratch bs;
};

// Builds the history count table for [lo, hi) (requires hi - lo <= CHUNK).
// When exc is set the distinct ids are listed (first occurrence wins the slot).
template <int CHUNK>
__device__ __forceinline__ void build_hist_table(const SampleParams& P, int row, const RowCfg& c, int lo, int hi,
                                 uint32_t* table, SampleShared<CHUNK>& sh, bool exc) {
    for (int i = threadIdx.x; i < CHUNK / 2; i += LLIMA_WG) table[i] = 0;
    if (threadIdx.x == 0) sh.n_exc = 0;
    __syncthreads();
    const int32_t* h = P.hist + (size_t)row * P.H_max;
    for (int j = threadIdx.x; j < c.hlen; j += LLIMA_WG) {
        int32_t id = h[j];
        if (id >= lo && id < hi) {
            uint32_t off = (uint32_t)(id - lo);
            uint32_t sh16 = (off & 1u) * 16u;
            uint32_t old = atomicAdd(&table[off >> 1], 1u << sh16);
            if (exc && ((old >> sh16) & 0xFFFFu) == 0) {
                uint32_t slot = atomicAdd(&sh.n_exc, 1u);
                if (slot < SAMPLE_EXC_CAP) sh.s.exc_id[slot] = id;
            }
        }
    }
    __syncthreads();
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

// ------------------------------------------------------------------ radix selects
// Each select runs over a set of (key, id, weight) elements presented by a
// visitor; every thread visits its own elements.  Histograms live in LDS; the
// boundary bin of each 8-bit digit is found with one workgroup scan.

// k-th largest key (with multiplicity) among visited elements.
template <int CHUNK, class Visit>
__device__ __forceinline__ uint32_t select_kth_desc(Visit visit, uint32_t k, SampleShared<CHUNK>& sh) {
    uint32_t prefix = 0, pmask = 0, rem = k;
    for (int shift = 24; shift >= 0; shift -= 8) {
        sh.f.hcnt[threadIdx.x] = 0;
        __syncthreads();
        visit([&](uint32_t key, uint32_t, uint64_t) {
            if ((key & pmask) == prefix) atomicAdd(&sh.f.hcnt[(key >> shift) & 255u], 1u);
        });
        __syncthreads();
        const uint32_t bin = 255u - threadIdx.x;          // thread 0 <-> top bin
        uint32_t c = sh.f.hcnt[bin], tot;
        uint32_t above = block_excl_scan_u32(c, &tot, sh.bs);
        if (above < rem && above + c >= rem) { sh.sel = bin; sh.sel64 = rem - above; }
        __syncthreads();
        prefix |= sh.sel << shift;
        pmask |= 255u << shift;
        rem = (uint32_t)sh.sel64;
        __syncthreads();
    }
    return prefix;
}

// Top-p boundary: the smallest key theta such that an element with key theta has
// (mass strictly above) * 2^32 < PZ; when none has (PZ == 0) the top key.
template <int CHUNK, class Visit>
__device__ __forceinline__ uint32_t select_topp_desc(Visit visit, llima_u128 PZ, SampleShared<CHUNK>& sh) {
    uint32_t prefix = 0, pmask = 0;
    uint64_t acc = 0;
    for (int shift = 24; shift >= 0; shift -= 8) {
        sh.f.hcnt[threadIdx.x] = 0;
        sh.f.hmass[threadIdx.x] = 0;
        __syncthreads();
        visit([&](uint32_t key, uint32_t, uint64_t w) {
            if ((key & pmask) == prefix) {
                uint32_t b = (key >> shift) & 255u;
                atomicAdd(&sh.f.hcnt[b], 1u);
                if (w) atomicAdd((unsigned long long*)&sh.f.hmass[b], (unsigned long long)w);
            }
        });
        __syncthreads();
        const uint32_t t = threadIdx.x, bin = 255u - t;
        uint32_t c = sh.f.hcnt[bin];
        uint64_t m = sh.f.hmass[bin], tot;
        uint64_t above = acc + block_excl_scan_u64(m, &tot, sh.bs);
        bool cond = c > 0 && (((llima_u128)above << 32) < PZ);
        // lowest qualifying bin = highest t; else the top non-empty bin = lowest t
        uint32_t best_cond = block_max_u32(cond ? t + 1u : 0u, sh.bs);
        uint32_t top_nonempty = 255u - block_max_u32(c > 0 ? 255u - t : 0u, sh.bs);
        uint32_t sel_t = best_cond ? best_cond - 1u : top_nonempty;
        if (t == sel_t) { sh.sel = bin; sh.sel64 = above; }
        __syncthreads();
        prefix |= sh.sel << shift;
        pmask |= 255u << shift;
        acc = sh.sel64;
        __syncthreads();
    }
    return prefix;
}

// Draw: the smallest id whose ascending-id prefix mass exceeds target.  Also
// returns that element's weight.
template <int CHUNK, class Visit>
__device__ __forceinline__ uint32_t select_draw_asc(Visit visit, uint64_t target, uint64_t* w_out,
                                    SampleShared<CHUNK>& sh) {
    uint32_t prefix = 0, pmask = 0;
    uint64_t acc = 0;
    for (int shift = 16; shift >= 0; shift -= 8) {
        sh.f.hmass[threadIdx.x] = 0;
        __syncthreads();
        visit([&](uint32_t, uint32_t id, uint64_t w) {
            if (w && (id & pmask) == prefix)
                atomicAdd((unsigned long long*)&sh.f.hmass[(id >> shift) & 255u],
                          (unsigned long long)w);
        });
        __syncthreads();
        const uint32_t bin = threadIdx.x;
        uint64_t m = sh.f.hmass[bin], tot;
        uint64_t below = acc + block_excl_scan_u64(m, &tot, sh.bs);
        if (m > 0 && below <= target && target < below + m) {
            sh.sel = bin; sh.sel64 = below; sh.sel64b = m;
        }
        __syncthreads();
        prefix |= sh.sel << shift;
        pmask |= 255u << shift;
        acc = sh.sel64;
        *w_out = sh.sel64b;
        __syncthreads();
    }
    return prefix;
}

__device__ __forceinline__ void write_result(const SampleParams& P, int row, int32_t id,
                                             float prob) {
    P.out_ids[row] = id;
    if (P.out_probs) P.out_probs[row] = prob;
}

__device__ __forceinline__ void reset_ctl(RowCtl* ctl) {
    ctl->count = 0;
    ctl->flags = 0;
    ctl->tmax_key = 0;
    ctl->greedy = 0;
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
// every pass (history table rebuilt per CHUNK segment).
template <typename TL, int CHUNK>
__device__ __forceinline__ void finish_full_row(const SampleParams& P, int row, const RowCfg& c,
                                SampleShared<CHUNK>& sh) {
    const TL* rowp = (const TL*)P.logits + (size_t)row * P.row_stride;
    const int V = P.V;
    const int nw = (V + 31) >> 5;
    const uint32_t* mrow = P.bitmask ? P.bitmask + (size_t)row * nw : nullptr;
    uint32_t* table = sh.s.cnt;
    // fn(x, id) for every element of the row.
    auto for_each_x = [&](auto fn) {
        for (int lo = 0; lo < V; lo += CHUNK) {
            const int hi = lo + CHUNK < V ? lo + CHUNK : V;
            if (c.pen) build_hist_table<CHUNK>(P, row, c, lo, hi, table, sh, false);
            for (int i = lo + threadIdx.x; i < hi; i += LLIMA_WG) {
                float l = load_one<TL>(rowp, i);
                if (l != l) l = -__builtin_inff();
                if (mrow && !((mrow[i >> 5] >> (i & 31)) & 1u)) l = -__builtin_inff();
                if (c.pen) {
                    uint32_t cnt = table_count(table, (uint32_t)(i - lo));
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
            uint64_t kk = ((uint64_t)f32_key(x) << 32) | (uint64_t)(~id);
            best = kk > best ? kk : best;
        });
        best = block_max_u64(best, sh.bs);
        if (threadIdx.x == 0) {
            bool ok = (uint32_t)(best >> 32) > LLIMA_KEY_NEG_INF;
            write_result(P, row, ok ? (int32_t)(~(uint32_t)best) : -1, ok ? 1.0f : 0.0f);
        }
        if (P.out_keep) {
            const uint32_t tok = (uint32_t)(best >> 32) > LLIMA_KEY_NEG_INF ? ~(uint32_t)best : 0xFFFFFFFFu;
            write_keep(P, row, [&](auto set) { if (threadIdx.x == 0 && tok != 0xFFFFFFFFu) set(tok); });
        }
        return;
    }

    // Pass: maximum and number of finite values.
    uint32_t kmax = 0, nfin = 0;
    for_each_x([&](float x, uint32_t) {
        uint32_t k = f32_key(x);
        if (k > LLIMA_KEY_NEG_INF) { nfin++; kmax = k > kmax ? k : kmax; }
    });
    kmax = block_max_u32(kmax, sh.bs);
    nfin = block_sum_u32(nfin, sh.bs);
    if (nfin == 0) {
        if (threadIdx.x == 0) write_result(P, row, -1, 0.0f);
        if (P.out_keep) write_keep(P, row, [&](auto) {});
        return;
    }
    const float xmax = key_f32(kmax);
    auto visit_fin = [&](auto fn) {   // finite elements, weights not needed
        for_each_x([&](float x, uint32_t id) {
            uint32_t k = f32_key(x);
            if (k > LLIMA_KEY_NEG_INF) fn(k, id, 0ull);
        });
    };
    uint32_t tau = LLIMA_KEY_NEG_INF + 1u;
    if (c.k > 0 && (uint32_t)c.k <= nfin) tau = select_kth_desc<CHUNK>(visit_fin, (uint32_t)c.k, sh);

    auto visit_k = [&](auto fn) {     // top-k survivors with weights
        for_each_x([&](float x, uint32_t id) {
            uint32_t k = f32_key(x);
            if (k >= tau) fn(k, id, weight(x, xmax));
        });
    };
    uint32_t theta = 0;
    if (c.p < 1.0f) {
        uint64_t Z = 0;
        visit_k([&](uint32_t, uint32_t, uint64_t w) { Z += w; });
        Z = block_sum_u64(Z, sh.bs);
        llima_u128 PZ = (llima_u128)frac32(c.p) * Z;
        theta = select_topp_desc<CHUNK>(visit_k, PZ, sh);
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
        tok = (int32_t)select_draw_asc<CHUNK>(visit_final, target, &wtok, sh);
        prob = (float)((double)wtok / (double)Zf);
    }
    if (threadIdx.x == 0) write_result(P, row, tok, prob);
    if (P.out_keep)
        write_keep(P, row, [&](auto set) {
            visit_final([&](uint32_t, uint32_t id, uint64_t) { set(id); });
        });
}

// Greedy rows: the row's best (key, index) was merged by atomicMax.  Returns
// false when the row must be redone by the full-row path.
template <typename TL, int CHUNK>
__device__ __forceinline__ bool finish_greedy(const SampleParams& P, int row, const RowCfg& c,
                                              RowCtl* ctl, SampleShared<CHUNK>& sh) {
    (void)c;
    // More distinct history ids in a chunk than the exception list holds.
    const bool ovf = (load_coherent(&ctl->flags) & CTL_OVERFLOW) != 0;
    __syncthreads();
    if (ovf) {
        if (threadIdx.x == 0) reset_ctl(ctl);
        return false;
    }
    if (threadIdx.x == 0) {
        const uint64_t best = load_coherent(&ctl->greedy);
        const bool ok = (uint32_t)(best >> 32) > LLIMA_KEY_NEG_INF;
        write_result(P, row, ok ? (int32_t)(~(uint32_t)best) : -1, ok ? 1.0f : 0.0f);
        sh.sel = ok ? ~(uint32_t)best : 0xFFFFFFFFu;
        reset_ctl(ctl);
    }
    if (P.out_keep) {
        __syncthreads();
        const uint32_t tok = sh.sel;
        write_keep(P, row, [&](auto set) { if (threadIdx.x == 0 && tok != 0xFFFFFFFFu) set(tok); });
    }
    return true;
}

// Sampling rows from the candidate list.  Returns false when the candidates
// cannot be proven to contain the kept set (the full-row path then runs).
template <typename TL, int CHUNK>
__device__ __forceinline__ bool finish_fast(const SampleParams& P, int row, const RowCfg& c,
                                            RowCtl* ctl, SampleShared<CHUNK>& sh) {
    const float NEG_INF = -__builtin_inff();
    const uint32_t flags = load_coherent(&ctl->flags);
    const uint32_t n = load_coherent(&ctl->count);
    const uint32_t tmax_key = load_coherent(&ctl->tmax_key);
    __syncthreads();
    if (threadIdx.x == 0) reset_ctl(ctl);
    if ((flags & CTL_OVERFLOW) || n > SAMPLE_RCAP) return false;

    // ---- load candidates into registers: slot j of thread t is candidate t + 256 j
    uint32_t key[SAMPLE_SLOTS], id[SAMPLE_SLOTS];
    float xs[SAMPLE_SLOTS];
    const uint64_t* src = (const uint64_t*)(P.ws + (size_t)row * SAMPLE_SLOT_BYTES + SAMPLE_CTL_BYTES);
    uint32_t kmax = 0;
#pragma unroll
    for (int j = 0; j < SAMPLE_SLOTS; ++j) {
        const uint32_t s = threadIdx.x + j * LLIMA_WG;
        key[j] = 0; id[j] = 0; xs[j] = NEG_INF;
        if (s < n) {
            const uint64_t q = src[s];
            const float x = __uint_as_float((uint32_t)(q >> 32)) / c.T;
            xs[j] = x;
            key[j] = f32_key(x);
            id[j] = (uint32_t)q;
            kmax = key[j] > kmax ? key[j] : kmax;
        }
    }
    kmax = block_max_u32(kmax, sh.bs);
    if (kmax <= LLIMA_KEY_NEG_INF) {
        // Every candidate is -inf after the temperature (or there are none).
        if (flags & CTL_FILTERED) return false;
        if (threadIdx.x == 0) write_result(P, row, -1, 0.0f);
        if (P.out_keep) write_keep(P, row, [&](auto) {});
        return true;
    }
    const float xmax = key_f32(kmax);
    auto visit_all = [&](auto fn) {
#pragma unroll
        for (int j = 0; j < SAMPLE_SLOTS; ++j)
            if (key[j] > LLIMA_KEY_NEG_INF) fn(key[j], id[j], 0ull);
    };

    // ---- top-k threshold, then proof that the pre-filter kept every member
    uint32_t tau = LLIMA_KEY_NEG_INF + 1u;
    if (c.k > 0) {
        uint32_t nfin = 0;
#pragma unroll
        for (int j = 0; j < SAMPLE_SLOTS; ++j) nfin += key[j] > LLIMA_KEY_NEG_INF;
        nfin = block_sum_u32(nfin, sh.bs);
        if ((uint32_t)c.k <= nfin) tau = select_kth_desc<CHUNK>(visit_all, (uint32_t)c.k, sh);
        else if (flags & CTL_FILTERED) return false;
        if (flags & CTL_FILTERED) {
            const float gq = lower_bound_margin(key_f32(tmax_key)) / c.T;
            if (!(gq < key_f32(tau))) return false;
        }
    }

    // ---- weights of the top-k survivors
    uint64_t w[SAMPLE_SLOTS];
#pragma unroll
    for (int j = 0; j < SAMPLE_SLOTS; ++j)
        w[j] = (key[j] > LLIMA_KEY_NEG_INF && key[j] >= tau) ? weight(xs[j], xmax) : 0ull;
    auto visit_k = [&](auto fn) {
#pragma unroll
        for (int j = 0; j < SAMPLE_SLOTS; ++j)
            if (key[j] > LLIMA_KEY_NEG_INF && key[j] >= tau) fn(key[j], id[j], w[j]);
    };

    uint32_t theta = 0;
    if (c.p < 1.0f) {
        uint64_t Z = 0;
#pragma unroll
        for (int j = 0; j < SAMPLE_SLOTS; ++j) Z += w[j];
        Z = block_sum_u64(Z, sh.bs);
        const llima_u128 PZ = (llima_u128)frac32(c.p) * Z;
        theta = select_topp_desc<CHUNK>(visit_k, PZ, sh);
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
        tok = (int32_t)select_draw_asc<CHUNK>(visit_final, target, &wtok, sh);
        prob = (float)((double)wtok / (double)Zf);
    }
    if (threadIdx.x == 0) write_result(P, row, tok, prob);
    if (P.out_keep)
        write_keep(P, row, [&](auto set) {
            visit_final([&](uint32_t, uint32_t i, uint64_t) { set(i); });
        });
    return true;
}

// ------------------------------------------------------------------ the kernel
template <typename TL, int E>
__global__ __launch_bounds__(LLIMA_WG) void sample_kernel(SampleParams P) {
    constexpr int EPL = 16 / sizeof(TL);       // elements per 16-byte load
    constexpr int NL = E / EPL;                // loads per thread
    constexpr int CHUNK = LLIMA_WG * E;
    __shared__ SampleShared<CHUNK> sh;

    uint32_t row, chunk;
    map_row_chunk(blockIdx.x, (uint32_t)P.B, (uint32_t)P.S, &row, &chunk);
    if (row >= (uint32_t)P.B) return;
    const RowCfg c = load_cfg(P, row);
    const TL* rowp = (const TL*)P.logits + (size_t)row * P.row_stride;
    const int V = P.V;
    const int c0 = (int)chunk * CHUNK;
    const int c1 = c0 + CHUNK < V ? c0 + CHUNK : V;
    const int nw = (V + 31) >> 5;
    const uint32_t* mrow = P.bitmask ? P.bitmask + (size_t)row * nw : nullptr;
    RowCtl* ctl = (RowCtl*)(P.ws + (size_t)row * SAMPLE_SLOT_BYTES);
    const float NEG_INF = -__builtin_inff();

    if (threadIdx.x == 0) { sh.n_pre = 0; sh.flags = 0; sh.n_exc = 0; }
    if (c.pen) build_hist_table<CHUNK>(P, row, c, c0, c1, sh.s.cnt, sh, true);
    else __syncthreads();

    // ---- stream the chunk into registers (value after mask / NaN / history exclusion)
    float v[E];
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
            for (int e = 0; e < EPL; ++e) t[e] = (i0 + e < c1) ? load_one<TL>(rowp, i0 + e) : NEG_INF;
        }
        uint32_t mbits = 0xFFFFFFFFu;
        if (mrow && i0 < c1) mbits = mrow[i0 >> 5] >> (i0 & 31);
        uint32_t cw[EPL / 2];
        if (c.pen && i0 < c1) {
            const uint32_t off = (uint32_t)(i0 - c0);
#pragma unroll
            for (int e = 0; e < EPL / 2; ++e) cw[e] = sh.s.cnt[(off >> 1) + e];
        } else {
#pragma unroll
            for (int e = 0; e < EPL / 2; ++e) cw[e] = 0;
        }
#pragma unroll
        for (int e = 0; e < EPL; ++e) {
            float x = t[e];
            const bool hist_hit = ((cw[e >> 1] >> ((e & 1) * 16)) & 0xFFFFu) != 0;
            if (x != x || !((mbits >> e) & 1u) || hist_hit) x = NEG_INF;
            v[j * EPL + e] = x;
        }
    }

    // ---- exceptions: distinct history ids of this chunk, penalised exactly
    const uint32_t n_exc = c.pen ? sh.n_exc : 0u;
    if (n_exc > SAMPLE_EXC_CAP) {
        if (threadIdx.x == 0) atomicOr(&ctl->flags, CTL_OVERFLOW);
    }
    const uint32_t n_exc_c = n_exc < SAMPLE_EXC_CAP ? n_exc : SAMPLE_EXC_CAP;
    float tmax = NEG_INF;
    for (uint32_t j = threadIdx.x; j < n_exc_c; j += LLIMA_WG) {
        const int id = sh.s.exc_id[j];
        float l = load_one<TL>(rowp, id);
        if (l != l) l = NEG_INF;
        if (mrow && !((mrow[id >> 5] >> (id & 31)) & 1u)) l = NEG_INF;
        l = penalize(l, table_count(sh.s.cnt, (uint32_t)(id - c0)), c);
        sh.s.exc_val[j] = l;
        tmax = l > tmax ? l : tmax;
    }

    if (c.greedy) {
        // ---- argmax: first index of the maximum
        uint64_t best = 0;
#pragma unroll
        for (int j = 0; j < NL; ++j) {
            const int i0 = c0 + j * (LLIMA_WG * EPL) + (int)threadIdx.x * EPL;
#pragma unroll
            for (int e = 0; e < EPL; ++e) {
                uint64_t kk = ((uint64_t)f32_key(v[j * EPL + e]) << 32) | (uint64_t)(~(uint32_t)(i0 + e));
                best = kk > best ? kk : best;
            }
        }
        for (uint32_t j = threadIdx.x; j < n_exc_c; j += LLIMA_WG) {
            uint64_t kk = ((uint64_t)f32_key(sh.s.exc_val[j]) << 32) |
                          (uint64_t)(~(uint32_t)sh.s.exc_id[j]);
            best = kk > best ? kk : best;
        }
        best = block_max_u64(best, sh.bs);
        if (threadIdx.x == 0) atomicMax((unsigned long long*)&ctl->greedy, (unsigned long long)best);
    } else {
        // ---- pre-filter bound from lane maxima
        float g = NEG_INF;
        if (c.k > 0 && c.k <= 4 * 64) {
#pragma unroll
            for (int e = 0; e < E; ++e) tmax = v[e] > tmax ? v[e] : tmax;
            const uint32_t r = (uint32_t)(c.k + 3) >> 2;          // ceil(k/4) <= 64
            uint32_t sorted = wave_sort_desc(f32_key(tmax));
            uint32_t wb = __shfl(sorted, (int)r - 1, 64);
            if (lane_id() == 0) sh.wave_bound[threadIdx.x >> 6] = wb;
            __syncthreads();
            uint32_t tb = sh.wave_bound[0];
#pragma unroll
            for (int w = 1; w < LLIMA_WAVES; ++w) tb = sh.wave_bound[w] < tb ? sh.wave_bound[w] : tb;
            if (tb > LLIMA_KEY_NEG_INF) {
                g = lower_bound_margin(key_f32(tb));
                if (threadIdx.x == 0) {
                    atomicMax(&ctl->tmax_key, tb);
                    atomicOr(&ctl->flags, CTL_FILTERED);
                }
            }
        }
        // ---- stage candidates in LDS
#pragma unroll
        for (int j = 0; j < NL; ++j) {
            const int i0 = c0 + j * (LLIMA_WG * EPL) + (int)threadIdx.x * EPL;
#pragma unroll
            for (int e = 0; e < EPL; ++e) {
                const float x = v[j * EPL + e];
                if (x > NEG_INF && x >= g) {
                    uint32_t s = atomicAdd(&sh.n_pre, 1u);
                    if (s < SAMPLE_PRECAP)
                        sh.s.pre[s] = ((uint64_t)__float_as_uint(x) << 32) | (uint32_t)(i0 + e);
                }
            }
        }
        for (uint32_t j = threadIdx.x; j < n_exc_c; j += LLIMA_WG) {
            const float x = sh.s.exc_val[j];
            if (x > NEG_INF && x >= g) {
                uint32_t s = atomicAdd(&sh.n_pre, 1u);
                if (s < SAMPLE_PRECAP)
                    sh.s.pre[s] = ((uint64_t)__float_as_uint(x) << 32) | (uint32_t)sh.s.exc_id[j];
            }
        }
        __syncthreads();
        const uint32_t n_pre = sh.n_pre;
        if (threadIdx.x == 0) {
            uint32_t base = 0xFFFFFFFFu;
            if (n_pre > SAMPLE_PRECAP) atomicOr(&ctl->flags, CTL_OVERFLOW);
            else if (n_pre) {
                base = atomicAdd(&ctl->count, n_pre);
                if (base + n_pre > SAMPLE_RCAP) { atomicOr(&ctl->flags, CTL_OVERFLOW); base = 0xFFFFFFFFu; }
            }
            sh.base = base;
        }
        __syncthreads();
        const uint32_t base = sh.base;
        if (base != 0xFFFFFFFFu) {
            uint64_t* dst = (uint64_t*)(P.ws + (size_t)row * SAMPLE_SLOT_BYTES + SAMPLE_CTL_BYTES) + base;
            for (uint32_t j = threadIdx.x; j < n_pre; j += LLIMA_WG) dst[j] = sh.s.pre[j];
        }
    }

    // ---- the last workgroup of the row finishes it
    if (!arrive_last(&ctl->done, (uint32_t)P.S, &sh.last)) return;

    bool done;
    if (c.greedy) done = finish_greedy<TL, CHUNK>(P, row, c, ctl, sh);
    else done = finish_fast<TL, CHUNK>(P, row, c, ctl, sh);
    if (!done) finish_full_row<TL, CHUNK>(P, row, c, sh);
}

// ------------------------------------------------------------------ host side
struct Tile { int E; int S; };

static Tile choose_tile(int B, int V, int dtype, int k) {
    // Largest E first; shrink while the grid is small, but keep the row's
    // candidate count (about 2k per chunk) well inside SAMPLE_RCAP.
    const int emax = dtype == LLIMA_F32 ? 32 : 64;
    int E = emax;
    auto S_of = [&](int e) { return (V + LLIMA_WG * e - 1) / (LLIMA_WG * e); };
    while (E > 8) {
        const int S2 = S_of(E / 2);
        if ((int64_t)B * S_of(E) >= 1024) break;
        if (k > 0 && (int64_t)S2 * 2 * k > SAMPLE_RCAP / 2) break;
        E /= 2;
        (void)S2;
    }
    return {E, S_of(E)};
}

template <typename TL, int E>
static hipError_t launch(const SampleParams& P, hipStream_t st) {
    const uint32_t nblk = (uint32_t)P.B * (uint32_t)P.S;
    hipLaunchKernelGGL((sample_kernel<TL, E>), dim3(nblk), dim3(LLIMA_WG), 0, st, P);
    return hipGetLastError();
}

}  // namespace llima

using namespace llima;

extern "C" size_t llima_sample_workspace_bytes(int32_t B, int32_t V, int32_t dtype) {
    (void)V; (void)dtype;
    if (B <= 0) return 0;
    return (size_t)B * SAMPLE_SLOT_BYTES;
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
    P.ws = (char*)workspace;
    P.B = B;
    P.V = V;
    P.H_max = history ? H_max : 0;
    const size_t esz = dtype == LLIMA_F32 ? 4 : 2;
    P.vec_ok = ((uintptr_t)logits % 16 == 0) && ((row_stride * (int64_t)esz) % 16 == 0);
    const int k_hint = cfg->top_k_rows ? 0 : cfg->top_k;
    const Tile t = choose_tile(B, V, dtype, (k_hint > 0 && k_hint < V) ? k_hint : 0);
    P.S = t.S;
    hipStream_t st = (hipStream_t)stream;
    hipError_t e;
    if (dtype == LLIMA_F32) {
        switch (t.E) {
            case 8: e = launch<float, 8>(P, st); break;
            case 16: e = launch<float, 16>(P, st); break;
            default: e = launch<float, 32>(P, st); break;
        }
    } else {
        switch (t.E) {
            case 8: e = launch<uint16_t, 8>(P, st); break;
            case 16: e = launch<uint16_t, 16>(P, st); break;
            case 32: e = launch<uint16_t, 32>(P, st); break;
            default: e = launch<uint16_t, 64>(P, st); break;
        }
    }
    return e == hipSuccess ? LLIMA_OK : LLIMA_E_HIP;
}
