// llima_oracle.cpp -- CPU oracle for the logits -> token-selection path.
//
// TEST INFRASTRUCTURE ONLY.  Nothing in the product (llima_amd/) links, loads
// or calls this file; only tests/, __graft_entry__.smoke() and bench.py's
// cpu_baseline leg do, and only as the checker.  It is a plain, sequential
// restatement of (1) the reference runtime's greedy selection functions and
// (2) the written sampler specification the MI355X kernels implement, chosen to
// be obviously correct rather than fast (full sorts, one row at a time, a dense
// count array per row).  OpenMP is used across rows only.
//
// Reference behaviour restated (sima-neat/llima, paths relative to the repo):
//   argmax_bf16                     sima_lmm/devkit/cpp/utils.hpp:80-152
//   _calc_next_token_id (4 parts)   sima_lmm/devkit/cpp/language_model.cpp:3689-3714
//   _argmax_lm_head_row(s)          sima_lmm/devkit/cpp/language_model.cpp:3616-3687
//   EAGLE3 verify argmax (-inf)     sima_lmm/devkit/cpp/language_model_eagle3.cpp:486-522
//   tree_decoding gather            sima_lmm/devkit/cpp/language_model_eagle3.cpp:551-567
//   evaluate_posterior              sima_lmm/devkit/cpp/eagle_helpers.hpp:153-195
//   resolve_draft_tokens            sima_lmm/devkit/cpp/gemma4_mtp_helpers.cpp:81-111
//   select_candidate_tokens         sima_lmm/devkit/cpp/gemma4_mtp_helpers.cpp:113-167
//   _argmax_gemma4_mtp_masked_row   sima_lmm/devkit/cpp/language_model_gemma4_mtp.cpp:31-97
//   score_logits                    sima_lmm/devkit/cpp/language_model.cpp:29-62
//
// The reference has no stochastic sampler.  The sampler stages below follow the
// specification adopted for this path (HF-transformers order and definitions:
// transformers/generation/logits_process.py RepetitionPenalty, Temperature,
// TopK, TopP, MinP; OpenAI presence/frequency penalties; xgrammar-style LSB-first
// uint32 token bitmask), made bit-reproducible by integer (fixed-point) weights:
//
//   W(d)  = round(exp(d) * 2^36) for d = x - x_max <= 0, computed by the shared
//           exp below (IEEE fma / rint / ldexp only); 0 for d < -26.
//   Z     = sum of W (uint64, exact, order independent).
//   top-p : keep i iff  S_i * 2^32 < P32 * Z  or x_i == x_max,
//           S_i = sum of W_j over x_j > x_i, P32 = rint(p * 2^32).
//   min-p : keep i iff  W_i >= M32 * 16   (W_max == 2^36), M32 = rint(m * 2^32).
//   draw  : U32 = floor(u * 2^32); target = (U32 * Z') >> 32; token = smallest id
//           whose ascending-id prefix sum of W exceeds target.
//
// Build: oracle/Makefile (g++ -O2 -fopenmp -ffp-contract=off).  Floating-point
// contraction is disabled so that every product and sum is the IEEE operation
// written in the source, exactly as in the HIP kernels.

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <limits>
#include <numeric>
#include <vector>

#include <omp.h>

typedef unsigned __int128 u128;

extern "C" {

// ---------------------------------------------------------------- status codes
enum { ORC_OK = 0, ORC_E_INVAL = -1, ORC_E_RANGE = -2 };

// ---------------------------------------------------------------- primitives
static inline float bf16_to_f32(uint16_t h) {
    uint32_t u = (uint32_t)h << 16;
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

static inline float load_logit(const void* base, int dtype, int64_t i) {
    if (dtype == 0) return ((const float*)base)[i];
    return bf16_to_f32(((const uint16_t*)base)[i]);
}

// exp(d) for d <= 0 by Cody-Waite reduction and a degree-7 Taylor polynomial,
// written from the mathematics (e^d = 2^n * e^r, r = d - n ln2, |r| <= ln2/2).
// Every step is a single IEEE operation (mul, rint, fma, ldexp), so the result
// is identical on any IEEE-754 machine that honours fma.
static const float ORC_LOG2E = 1.44269502162933349609375f;   // fl(log2(e))
static const float ORC_LN2_HI = 0.693145751953125f;          // 0x3F317200
static const float ORC_LN2_LO = 1.428606765330187045e-06f;   // ln2 - LN2_HI

float orc_exp_neg(float d) {
    if (!(d >= -26.0f)) return 0.0f;
    float n = rintf(d * ORC_LOG2E);
    float r = fmaf(n, -ORC_LN2_HI, d);
    r = fmaf(n, -ORC_LN2_LO, r);
    float p = 1.98412698412698412698e-04f;            // 1/5040
    p = fmaf(p, r, 1.38888888888888888889e-03f);      // 1/720
    p = fmaf(p, r, 8.33333333333333333333e-03f);      // 1/120
    p = fmaf(p, r, 4.16666666666666666667e-02f);      // 1/24
    p = fmaf(p, r, 1.66666666666666666667e-01f);      // 1/6
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    return ldexpf(p, (int)n);
}

// Fixed-point weight of a value x given the row maximum xmax (both after all
// transforms).  x == xmax (including xmax == +inf) has weight exactly 2^36.
uint64_t orc_weight(float x, float xmax) {
    if (x == xmax) return (uint64_t)1 << 36;
    float d = x - xmax;
    if (!(d >= -26.0f)) return 0;
    float e = orc_exp_neg(d);
    return (uint64_t)rintf(ldexpf(e, 36));
}

static inline uint64_t frac32(float v) {
    // rint(v * 2^32) clamped to [0, 2^32]; v is a probability-like parameter.
    double s = (double)v * 4294967296.0;
    if (!(s > 0.0)) return 0;
    if (s >= 4294967296.0) return (uint64_t)1 << 32;
    return (uint64_t)nearbyint(s);
}

static inline uint64_t uniform32(float u) {
    if (!(u > 0.0f)) return 0;                       // also NaN
    if (u >= 1.0f) return 0xFFFFFFFFull;
    return (uint64_t)floor((double)u * 4294967296.0);
}

static inline int bitlen128(u128 v) {
    int n = 0;
    while (v) { ++n; v >>= 1; }
    return n;
}

// ---------------------------------------------------------------- argmax
// mode 0: per split, argmax_bf16 semantics (best starts at the split's first
//         element, strict '>'); splits merged from (-inf, 0) keeping the greater
//         value or, on equal value, the lower index  (utils.hpp:80-152 and
//         language_model.cpp:3616-3633; one split == argmax_bf16 itself).
// mode 1: best starts at -inf, strict '>' over the whole row in order; NaN never
//         wins and an all -inf/NaN row yields id 0 (language_model_eagle3.cpp:486-522).
// mode 2: four parts [V*p/4, V*(p+1)/4), each argmax_bf16, merged from
//         (values[0], 0) with the same rule (language_model.cpp:3689-3714).
// mode 3: best starts at bf16 lowest() with index 0, strict '>' over every
//         split in order (the speculative path's multi-split scan,
//         language_model.cpp:1556-1575).
static const float ORC_BF16_LOWEST = -3.38953139e38f;   // bf16 0xFF7F

static void argmax_split(const void* row, int dtype, int64_t begin, int64_t size,
                         float* best_v, int64_t* best_i) {
    float best = load_logit(row, dtype, begin);
    int64_t idx = 0;
    for (int64_t i = 1; i < size; ++i) {
        float v = load_logit(row, dtype, begin + i);
        if (v > best) { best = v; idx = i; }
    }
    *best_v = best;
    *best_i = begin + idx;
}

// One row; mode 0 splits start at bounds[0..nb-1] (bounds[0] == 0, increasing).
static void argmax_row(const void* row, int dtype, int V, const int64_t* bounds, int nb,
                       int mode, float* out_v, int64_t* out_i) {
    float bv;
    int64_t bi = 0;
    if (mode == 1 || mode == 3) {
        bv = mode == 1 ? -std::numeric_limits<float>::infinity() : ORC_BF16_LOWEST;
        for (int64_t i = 0; i < V; ++i) {
            float v = load_logit(row, dtype, i);
            if (v > bv) { bv = v; bi = i; }
        }
    } else if (mode == 0) {
        bv = -std::numeric_limits<float>::infinity();
        for (int s = 0; s < nb; ++s) {
            int64_t begin = bounds[s], end = s + 1 < nb ? bounds[s + 1] : V;
            float v; int64_t i;
            argmax_split(row, dtype, begin, end - begin, &v, &i);
            if (v > bv || (v == bv && i < bi)) { bv = v; bi = i; }
        }
    } else {
        bv = load_logit(row, dtype, 0);
        for (int p = 0; p < 4; ++p) {
            int64_t begin = (int64_t)V * p / 4, end = (int64_t)V * (p + 1) / 4;
            if (end <= begin) continue;
            float v; int64_t i;
            argmax_split(row, dtype, begin, end - begin, &v, &i);
            if (v > bv || (v == bv && i < bi)) { bv = v; bi = i; }
        }
    }
    *out_v = bv;
    *out_i = bi;
}

static bool valid_bounds(const int64_t* bounds, int nb, int V) {
    if (nb < 1 || bounds[0] != 0) return false;
    for (int s = 1; s < nb; ++s)
        if (bounds[s] <= bounds[s - 1] || bounds[s] >= V) return false;
    return true;
}

// Split starts given explicitly (mode 0); modes 1-3 ignore them.
int orc_argmax_bounds(const void* logits, int dtype, int B, int V, int64_t row_stride,
                      const int64_t* bounds, int nb, int mode, int32_t* out_ids,
                      float* out_vals) {
    if (B < 0 || V <= 0 || (dtype != 0 && dtype != 1)) return ORC_E_INVAL;
    if (mode < 0 || mode > 3 || !valid_bounds(bounds, nb, V)) return ORC_E_INVAL;
    const size_t esz = dtype == 0 ? 4 : 2;
#pragma omp parallel for schedule(static)
    for (int b = 0; b < B; ++b) {
        const void* row = (const char*)logits + (size_t)b * row_stride * esz;
        float bv;
        int64_t bi;
        argmax_row(row, dtype, V, bounds, nb, mode, &bv, &bi);
        out_ids[b] = (int32_t)bi;
        if (out_vals) out_vals[b] = bv;
    }
    return ORC_OK;
}

static std::vector<int64_t> uniform_bounds(int V, int split_dim) {
    const int sd = (split_dim <= 0 || split_dim >= V) ? V : split_dim;
    std::vector<int64_t> b;
    for (int64_t s = 0; s < V; s += sd) b.push_back(s);
    return b;
}

int orc_argmax(const void* logits, int dtype, int B, int V, int64_t row_stride,
               int split_dim, int mode, int32_t* out_ids, float* out_vals) {
    if (V <= 0) return ORC_E_INVAL;
    const std::vector<int64_t> b = uniform_bounds(V, split_dim);
    return orc_argmax_bounds(logits, dtype, B, V, row_stride, b.data(), (int)b.size(), mode,
                             out_ids, out_vals);
}

// ---------------------------------------------------------------- sampler
typedef struct {
    float temperature;
    int32_t top_k;
    float top_p;
    float min_p;
    float repetition_penalty;
    float presence_penalty;
    float frequency_penalty;
    int32_t greedy;
} orc_sampler_config;

// Step 1-3 of the specification: mask, NaN, repetition, frequency/presence.
static void penalised_row(const void* row, int dtype, int V, const int32_t* hist, int hlen,
                          const uint32_t* mask, const orc_sampler_config* c,
                          std::vector<float>& out, std::vector<uint32_t>& counts) {
    const float NEG_INF = -std::numeric_limits<float>::infinity();
    out.resize(V);
    counts.assign(V, 0);
    for (int j = 0; j < hlen; ++j) {
        int32_t id = hist[j];
        if (id >= 0 && id < V) counts[id]++;
    }
    for (int i = 0; i < V; ++i) {
        float l = load_logit(row, dtype, i);
        if (l != l) l = NEG_INF;
        if (mask && !((mask[i >> 5] >> (i & 31)) & 1u)) l = NEG_INF;
        uint32_t cnt = counts[i];
        if (cnt) {
            // HF RepetitionPenaltyLogitsProcessor: score < 0 ? score * p : score / p
            l = (l < 0.0f) ? l * c->repetition_penalty : l / c->repetition_penalty;
            // OpenAI frequency then presence, in that order, in fp32.
            l = (l - c->frequency_penalty * (float)cnt) - c->presence_penalty;
        }
        out[i] = l;
    }
}

static bool is_greedy(const orc_sampler_config* c) {
    return c->greedy != 0 || !(c->temperature > 0.0f);
}

// Samples one row.  Returns the token (-1 when no token is admissible) and
// writes its probability under the final distribution.  keep (optional, V/32
// words) receives the final kept set restricted to finite values.
static int32_t sample_row(const void* row, int dtype, int V, const int32_t* hist, int hlen,
                          const uint32_t* mask, float u, const orc_sampler_config* c,
                          float* prob, uint32_t* keep) {
    const float NEG_INF = -std::numeric_limits<float>::infinity();
    std::vector<float> l;
    std::vector<uint32_t> counts;
    penalised_row(row, dtype, V, hist, hlen, mask, c, l, counts);
    const int nwords = (V + 31) / 32;
    if (keep) std::memset(keep, 0, sizeof(uint32_t) * nwords);

    if (is_greedy(c)) {
        float best = NEG_INF;
        int32_t id = -1;
        for (int i = 0; i < V; ++i)
            if (l[i] > best) { best = l[i]; id = i; }
        if (prob) *prob = id >= 0 ? 1.0f : 0.0f;
        if (keep && id >= 0) keep[id >> 5] |= 1u << (id & 31);
        return id;
    }

    // Temperature (IEEE division).
    std::vector<float> x(V);
    for (int i = 0; i < V; ++i) x[i] = l[i] / c->temperature;

    // Top-k: tau = k-th largest with multiplicity; keep x >= tau.
    float tau = NEG_INF;
    if (c->top_k > 0 && c->top_k < V) {
        std::vector<float> tmp(x);
        std::nth_element(tmp.begin(), tmp.begin() + (c->top_k - 1), tmp.end(),
                         [](float a, float b) { return a > b; });
        tau = tmp[c->top_k - 1];
    }
    std::vector<int32_t> kept;
    for (int i = 0; i < V; ++i)
        if (x[i] > NEG_INF && x[i] >= tau) kept.push_back(i);
    if (kept.empty()) { if (prob) *prob = 0.0f; return -1; }

    float xmax = NEG_INF;
    for (int32_t i : kept) xmax = std::max(xmax, x[i]);
    std::vector<uint64_t> w(V, 0);
    uint64_t Z = 0;
    for (int32_t i : kept) { w[i] = orc_weight(x[i], xmax); Z += w[i]; }

    // Top-p over the top-k survivors.
    std::vector<char> fin(V, 0);
    for (int32_t i : kept) fin[i] = 1;
    if (c->top_p < 1.0f) {                          // NaN compares false: disabled
        const u128 PZ = (u128)frac32(c->top_p) * Z;
        std::vector<int32_t> order(kept);
        std::sort(order.begin(), order.end(), [&](int32_t a, int32_t b) {
            return x[a] > x[b] || (x[a] == x[b] && a < b);
        });
        uint64_t above = 0;                          // mass strictly above current group
        size_t g = 0;
        while (g < order.size()) {
            size_t h = g;
            uint64_t gmass = 0;
            while (h < order.size() && x[order[h]] == x[order[g]]) { gmass += w[order[h]]; ++h; }
            bool k = ((u128)above << 32) < PZ || x[order[g]] == xmax;
            for (size_t t = g; t < h; ++t) fin[order[t]] = k ? 1 : 0;
            above += gmass;
            g = h;
        }
    }
    // Min-p relative to the maximum (whose weight is exactly 2^36).
    if (c->min_p > 0.0f) {
        const uint64_t thr = frac32(c->min_p) << 4;
        for (int32_t i : kept)
            if (fin[i] && w[i] < thr) fin[i] = 0;
    }

    uint64_t Zf = 0;
    for (int i = 0; i < V; ++i) if (fin[i]) Zf += w[i];
    if (keep)
        for (int i = 0; i < V; ++i) if (fin[i]) keep[i >> 5] |= 1u << (i & 31);
    if (Zf == 0) { if (prob) *prob = 0.0f; return -1; }
    const uint64_t target = (uint64_t)(((u128)uniform32(u) * Zf) >> 32);
    uint64_t acc = 0;
    for (int i = 0; i < V; ++i) {
        if (!fin[i]) continue;
        acc += w[i];
        if (acc > target) {
            if (prob) *prob = (float)((double)w[i] / (double)Zf);
            return i;
        }
    }
    return -1;  // unreachable: acc reaches Zf > target
}

// cfg_rows: B configs (or 1 broadcast when cfg_stride == 0).
int orc_sample(const void* logits, int dtype, int B, int V, int64_t row_stride,
               const int32_t* hist, const int32_t* hist_len, int H_max,
               const uint32_t* bitmask, const float* uniforms,
               const orc_sampler_config* cfg, int cfg_stride,
               int32_t* out_ids, float* out_probs, uint32_t* out_keep) {
    if (B < 0 || V <= 0 || (dtype != 0 && dtype != 1) || H_max < 0) return ORC_E_INVAL;
    const size_t esz = dtype == 0 ? 4 : 2;
    const int nwords = (V + 31) / 32;
#pragma omp parallel for schedule(dynamic)
    for (int b = 0; b < B; ++b) {
        const orc_sampler_config* c = cfg + (size_t)b * cfg_stride;
        const void* row = (const char*)logits + (size_t)b * row_stride * esz;
        int hl = hist ? (hist_len ? std::min(std::max(hist_len[b], 0), H_max) : H_max) : 0;
        float p = 0.0f;
        int32_t id = sample_row(row, dtype, V, hist ? hist + (size_t)b * H_max : nullptr, hl,
                                bitmask ? bitmask + (size_t)b * nwords : nullptr,
                                uniforms ? uniforms[b] : 0.0f, c, &p,
                                out_keep ? out_keep + (size_t)b * nwords : nullptr);
        out_ids[b] = id;
        if (out_probs) out_probs[b] = p;
    }
    return ORC_OK;
}

// ---------------------------------------------------------------- verification
// Greedy chain verification: argmax (mode 0, one split) of each target row, then
// resolve_draft_tokens (gemma4_mtp_helpers.cpp:81-111): accept while the draft
// equals the target argmax; emit the first mismatching target token, or the
// bonus target token after a full match.
int orc_resolve_draft_tokens(const int32_t* drafts, int D, const int32_t* targets, int T,
                             int32_t* emitted, int32_t* accepted_flags, int* n_emitted) {
    if (T <= 0 || T > D + 1) return ORC_E_RANGE;
    int n = 0;
    for (int depth = 0; depth < T; ++depth) {
        if (depth == D) {
            emitted[n] = targets[depth]; accepted_flags[n] = 0; ++n;
            *n_emitted = n; return ORC_OK;
        }
        if (drafts[depth] != targets[depth]) {
            emitted[n] = targets[depth]; accepted_flags[n] = 0; ++n;
            *n_emitted = n; return ORC_OK;
        }
        emitted[n] = drafts[depth]; accepted_flags[n] = 1; ++n;
    }
    *n_emitted = n;
    return ORC_E_RANGE;  // ended without a mismatch or bonus token
}

int orc_verify_greedy(const void* target_logits, int dtype, int B, int D, int V,
                      const int64_t* bounds, int nb, int mode, const int32_t* draft_ids,
                      int32_t* accepted_len, int32_t* emitted) {
    if (B < 0 || D < 0 || V <= 0) return ORC_E_INVAL;
    std::vector<int32_t> tgt((size_t)B * (D + 1));
    int rc = orc_argmax_bounds(target_logits, dtype, B * (D + 1), V, V, bounds, nb, mode,
                               tgt.data(), nullptr);
    if (rc) return rc;
    for (int b = 0; b < B; ++b) {
        std::vector<int32_t> em(D + 1), fl(D + 1);
        int n = 0;
        orc_resolve_draft_tokens(draft_ids + (size_t)b * D, D, tgt.data() + (size_t)b * (D + 1),
                                 D + 1, em.data(), fl.data(), &n);
        accepted_len[b] = n - 1;
        for (int j = 0; j < D + 1; ++j) emitted[(size_t)b * (D + 1) + j] = j < n ? em[j] : -1;
    }
    return ORC_OK;
}

// evaluate_posterior (eagle_helpers.hpp:153-195): per path, count leading
// positions where the target next-token equals the next candidate (a negative
// candidate ends the path); the first path with the strictly longest count wins;
// bonus = target token at the accept length on that path.
int orc_evaluate_posterior(const int32_t* next_ids, const int32_t* candidates, int n_paths,
                           int L, int32_t* best, int32_t* accept_len, int32_t* bonus) {
    if (n_paths <= 0 || L <= 0) return ORC_E_INVAL;
    int32_t win_path = 0, win_len = 0;
    for (int p = 0; p < n_paths; ++p) {
        const int32_t* tgt = next_ids + (size_t)p * L;     // target token after position i
        const int32_t* cnd = candidates + (size_t)p * L;   // the path's token at position i
        int32_t len = 0;
        while (len + 1 < L && cnd[len + 1] >= 0 && tgt[len] == cnd[len + 1]) ++len;
        if (len > win_len) { win_len = len; win_path = p; }
    }
    *best = win_path;
    *accept_len = win_len;
    *bonus = next_ids[(size_t)win_path * L + win_len];
    return ORC_OK;
}

// tree_decoding gather (language_model_eagle3.cpp:551-567): -1 -> last tree row.
int orc_tree_gather(const int32_t* row_tokens, int K, const int32_t* retrieve, int n_paths,
                    int L, int32_t* next_ids) {
    for (int p = 0; p < n_paths; ++p)
        for (int d = 0; d < L; ++d) {
            int32_t idx = retrieve[p * L + d];
            if (idx < 0) idx = K - 1;
            if (idx >= K) return ORC_E_RANGE;
            next_ids[p * L + d] = row_tokens[idx];
        }
    return ORC_OK;
}

// Rejection verification weights (the specification of this build; the
// reference verifies greedily).  A row is cut into chunks of 8192 ids; chunk c
// has its maximum m_c (NaN ignored) and the row its maximum M = max m_c:
//   w_i = rint(exp(x_i - m_c) 2^36)          (orc_weight, relative to the chunk)
//   F_c = rint(exp(m_c - M) 2^27)            (2^27 for the maximum's chunks, 0
//                                              below -26 or for an empty chunk)
//   W_i = w_i F_c,  Z = sum_c F_c S_c,  S_c = sum_{i in c} w_i   (exact)
// so a chunk's sum needs only its own maximum.  Acceptance compares
// W_t(x) Z_d >= u W_d(x) Z_t in IEEE double; the draws use W~_i = W_i >> 32
// (below 2^31), the residual max(0, W~_t z_d - W~_d z_t) >> 21 with
// z = (Z >> 27) >> s, one shift s for both rows that leaves the larger 32 bits
// wide (each product below 2^63, each residual below 2^42).
#define ORC_VR_CHUNK 8192

struct VrRow {
    std::vector<float> m;      // chunk maxima
    std::vector<uint32_t> F;   // chunk factors
    u128 Z;
};

static uint32_t vr_factor(float mc, float M) {
    if (!(mc > -std::numeric_limits<float>::infinity())) return 0;
    if (mc == M) return 1u << 27;
    const float d = mc - M;
    if (!(d >= -26.0f)) return 0;
    return (uint32_t)rintf(ldexpf(orc_exp_neg(d), 27));
}

static void vr_row(const float* row, int V, VrRow& r) {
    const int nc = (V + ORC_VR_CHUNK - 1) / ORC_VR_CHUNK;
    r.m.assign(nc, -std::numeric_limits<float>::infinity());
    r.F.assign(nc, 0);
    float M = -std::numeric_limits<float>::infinity();
    for (int i = 0; i < V; ++i) {
        float& mc = r.m[i / ORC_VR_CHUNK];
        if (row[i] > mc) mc = row[i];
    }
    for (int c = 0; c < nc; ++c) M = r.m[c] > M ? r.m[c] : M;
    r.Z = 0;
    for (int c = 0; c < nc; ++c) {
        r.F[c] = vr_factor(r.m[c], M);
        uint64_t S = 0;
        if (r.m[c] > -std::numeric_limits<float>::infinity())
            for (int i = c * ORC_VR_CHUNK; i < std::min(V, (c + 1) * ORC_VR_CHUNK); ++i)
                if (row[i] == row[i]) S += orc_weight(row[i], r.m[c]);
        r.Z += (u128)S * r.F[c];
    }
}

// W_i of the specification.
static uint64_t vr_w(const float* row, const VrRow& r, int i) {
    const float mc = r.m[i / ORC_VR_CHUNK];
    const float v = row[i];
    if (v != v || !(mc > -std::numeric_limits<float>::infinity())) return 0;
    return orc_weight(v, mc) * (uint64_t)r.F[i / ORC_VR_CHUNK];
}

// W_i of every id and Z (as two 64-bit halves) of one row (for the tests).
int orc_vr_weights(const float* row, int V, uint64_t* W, uint64_t* Z2) {
    if (V <= 0) return ORC_E_INVAL;
    VrRow r;
    vr_row(row, V, r);
    for (int i = 0; i < V; ++i) W[i] = vr_w(row, r, i);
    Z2[0] = (uint64_t)r.Z;
    Z2[1] = (uint64_t)(r.Z >> 64);
    return ORC_OK;
}

static double u128_to_double(u128 z) {
    return (double)(uint64_t)(z >> 64) * 18446744073709551616.0 + (double)(uint64_t)z;
}

static inline int bitlen64(uint64_t z) { return z ? 64 - __builtin_clzll(z) : 0; }

// The residual's normalizers: (Z >> 27) of both rows, shifted together until
// the larger is 32 bits wide.
static void vr_z32(u128 Zt, u128 Zd, uint64_t* zt, uint64_t* zd) {
    const uint64_t ht = (uint64_t)(Zt >> 27), hd = (uint64_t)(Zd >> 27);
    const int s = std::max(0, std::max(bitlen64(ht), bitlen64(hd)) - 32);
    *zt = ht >> s;
    *zd = hd >> s;
}

}  // extern "C"

// Draw by the specification's rule from integer weights given by f(i).
template <class F>
static int32_t draw_weights(int V, F f, uint64_t total, float u) {
    if (total == 0) return -1;
    const uint64_t target = (uint64_t)(((u128)uniform32(u) * total) >> 32);
    uint64_t acc = 0;
    for (int i = 0; i < V; ++i) {
        acc += f(i);
        if (acc > target) return i;
    }
    return -1;
}

extern "C" {

// Stochastic speculative verification (Leviathan et al. 2023; Chen et al. 2023)
// on the chunked fixed-point weights above.  target: [B, D+1, V] fp32, draft:
// [B, D, V] fp32.
int orc_verify_rejection(const float* tgt, const float* drf, int B, int D, int V,
                         const int32_t* draft_ids, const float* u_accept, const float* u_resample,
                         int32_t* accepted_len, int32_t* emitted) {
    if (B < 0 || D < 0 || V <= 0) return ORC_E_INVAL;
#pragma omp parallel for schedule(dynamic)
    for (int b = 0; b < B; ++b) {
        int32_t* em = emitted + (size_t)b * (D + 1);
        for (int j = 0; j <= D; ++j) em[j] = -1;
        int k = 0;
        bool rejected = false;
        VrRow rt, rd;
        auto plain = [&](const float* t) {           // a draw from W~_t
            auto wh = [&](int i) { return vr_w(t, rt, i) >> 32; };
            uint64_t tot = 0;
            for (int i = 0; i < V; ++i) tot += wh(i);
            return draw_weights(V, wh, tot, u_resample[b]);
        };
        for (; k < D; ++k) {
            const float* t = tgt + ((size_t)b * (D + 1) + k) * V;
            const float* d = drf + ((size_t)b * D + k) * V;
            vr_row(t, V, rt);
            vr_row(d, V, rd);
            const int32_t x = draft_ids[(size_t)b * D + k];
            bool acc = false;
            if (x >= 0 && x < V && rt.Z > 0) {
                const double lhs = (double)vr_w(t, rt, x) * u128_to_double(rd.Z);
                const double rhs = (double)u_accept[(size_t)b * D + k] * (double)vr_w(d, rd, x) *
                                   u128_to_double(rt.Z);
                acc = lhs >= rhs;
            }
            if (!acc) {
                uint64_t zt, zd;
                vr_z32(rt.Z, rd.Z, &zt, &zd);
                auto res = [&](int i) -> uint64_t {
                    const uint64_t a = (vr_w(t, rt, i) >> 32) * zd, c = (vr_w(d, rd, i) >> 32) * zt;
                    return a > c ? (a - c) >> 21 : 0;
                };
                uint64_t R = 0;
                for (int i = 0; i < V; ++i) R += res(i);
                em[k] = R > 0 ? draw_weights(V, res, R, u_resample[b]) : plain(t);
                rejected = true;
                break;
            }
            em[k] = x;
        }
        if (!rejected) {
            const float* t = tgt + ((size_t)b * (D + 1) + D) * V;
            vr_row(t, V, rt);
            em[D] = plain(t);
        }
        accepted_len[b] = k;
    }
    return ORC_OK;
}

// ---------------------------------------------------------------- MTP centroid selection
// select_candidate_tokens (gemma4_mtp_helpers.cpp:113-167): top-k centroids by
// (value desc, index asc), expanded through token_ordering.
int orc_select_candidate_tokens(const uint16_t* centroid_bf16, int n_centroids,
                                const uint32_t* ordering, int n_ordering, int top_k,
                                uint32_t* out_tokens, int* n_out) {
    if (n_centroids <= 0 || n_ordering <= 0 || n_ordering % n_centroids != 0) return ORC_E_INVAL;
    if (top_k <= 0 || top_k > n_centroids) return ORC_E_INVAL;
    std::vector<uint32_t> idx(n_centroids);
    std::iota(idx.begin(), idx.end(), 0u);
    std::partial_sort(idx.begin(), idx.begin() + top_k, idx.end(), [&](uint32_t a, uint32_t b) {
        float va = bf16_to_f32(centroid_bf16[a]), vb = bf16_to_f32(centroid_bf16[b]);
        return va != vb ? va > vb : a < b;
    });
    const int per = n_ordering / n_centroids;
    int n = 0;
    for (int r = 0; r < top_k; ++r)
        for (int o = 0; o < per; ++o) {
            uint32_t tok = ordering[(size_t)idx[r] * per + o];
            if (tok >= (uint32_t)n_ordering) return ORC_E_RANGE;
            out_tokens[n++] = tok;
        }
    *n_out = n;
    return ORC_OK;
}

// _argmax_gemma4_mtp_masked_row (language_model_gemma4_mtp.cpp:31-97): argmax
// over candidate ids only, from (-inf, UINT32_MAX), greater value or equal value
// with lower token id.
int orc_masked_argmax(const void* row, int dtype, int V, const uint32_t* cand, int n_cand,
                      int32_t* out_id) {
    float best = -std::numeric_limits<float>::infinity();
    uint32_t tok = 0xFFFFFFFFu;
    for (int j = 0; j < n_cand; ++j) {
        uint32_t t = cand[j];
        if (t >= (uint32_t)V) continue;
        float v = load_logit(row, dtype, t);
        if (v > best || (v == best && t < tok)) { best = v; tok = t; }
    }
    if (tok == 0xFFFFFFFFu) return ORC_E_RANGE;
    *out_id = (int32_t)tok;
    return ORC_OK;
}

// score_logits (language_model.cpp:29-62): double log-softmax at the target id
// and whether the target is the (first) argmax.
int orc_score_logits(const void* row, int dtype, int V, int32_t target, double* logprob,
                     int32_t* is_greedy_out) {
    if (target < 0 || target >= V) return ORC_E_RANGE;
    double mx = -std::numeric_limits<double>::infinity();
    int32_t am = 0;
    for (int i = 0; i < V; ++i) {
        double v = load_logit(row, dtype, i);
        if (v > mx) { mx = v; am = i; }
    }
    double s = 0.0;
    for (int i = 0; i < V; ++i) s += std::exp((double)load_logit(row, dtype, i) - mx);
    *logprob = (double)load_logit(row, dtype, target) - (mx + std::log(s));
    *is_greedy_out = am == target;
    return ORC_OK;
}

// ---------------------------------------------------------------- EAGLE3 draft tree
// topk<T> (utils.hpp:216-281) on one row: a min-heap of the first k values
// (heapified from the last parent down), a later value replaces the root only
// when it is strictly greater, and sifts down to the smaller child (the right
// one only when the left one is strictly greater; a parent equal to its
// smaller child stays).  The output is a selection sort of the heap array:
// position a takes the first strictly greatest remaining entry, whose slot
// then receives entry a.  k in [1, 32] and cols >= k.
}  // extern "C"

template <typename Get>
static void heap_topk(Get get, int64_t cols, int k, int32_t* out_idx, float* out_val) {
    float hv[32];
    int32_t hi[32];
    for (int j = 0; j < k; ++j) { hv[j] = get(j); hi[j] = j; }
    auto sift = [&](int node) {
        for (;;) {
            int c = 2 * node + 1;
            if (c >= k) return;
            if (c + 1 < k && hv[c] > hv[c + 1]) ++c;
            if (!(hv[node] > hv[c])) return;
            std::swap(hv[node], hv[c]);
            std::swap(hi[node], hi[c]);
            node = c;
        }
    };
    for (int j = k / 2 - 1; j >= 0; --j) sift(j);
    for (int64_t j = k; j < cols; ++j) {
        const float v = get(j);
        if (v > hv[0]) { hv[0] = v; hi[0] = (int32_t)j; sift(0); }
    }
    for (int a = 0; a < k; ++a) {
        int m = a;
        for (int b = a + 1; b < k; ++b)
            if (hv[b] > hv[m]) m = b;
        out_val[a] = hv[m];
        out_idx[a] = hi[m];
        hv[m] = hv[a];
        hi[m] = hi[a];
    }
}

extern "C" {

int orc_topk(const void* x, int dtype, int rows, int64_t cols, int64_t row_stride, int k,
             int32_t* out_idx, float* out_val) {
    if (rows < 0 || k < 1 || k > 32 || cols < k || (dtype != 0 && dtype != 1)) return ORC_E_INVAL;
    const size_t esz = dtype == 0 ? 4 : 2;
    for (int r = 0; r < rows; ++r) {
        const void* row = (const char*)x + (size_t)r * row_stride * esz;
        heap_topk([&](int64_t i) { return load_logit(row, dtype, i); }, cols, k,
                  out_idx + (size_t)r * k, out_val + (size_t)r * k);
    }
    return ORC_OK;
}

// logsoftmax<T> (utils.hpp:283-301) in float: the maximum, a running float sum
// of exp(v - max) in index order, then v - (log(sum) + max).  cr = 0 uses the
// C library's expf/logf as the reference does; cr = 1 uses exp and log of the
// float argument in double rounded once to float (correctly rounded but for
// double-rounding cases of probability ~2^-29), the arithmetic of the HIP path.
static inline float orc_expf(float x, int cr) { return cr ? (float)std::exp((double)x) : std::exp(x); }
static inline float orc_logf(float x, int cr) { return cr ? (float)std::log((double)x) : std::log(x); }

int orc_logsoftmax(const float* v, int n, int cr, float* out) {
    if (n <= 0) return ORC_E_INVAL;
    float mx = -std::numeric_limits<float>::infinity();
    for (int i = 0; i < n; ++i) mx = std::max(mx, v[i]);
    float sum = 0.0f;
    for (int i = 0; i < n; ++i) sum += orc_expf(v[i] - mx, cr);
    const float shift = orc_logf(sum, cr) + mx;
    for (int i = 0; i < n; ++i) out[i] = v[i] - shift;
    return ORC_OK;
}

// searchsorted (eagle_helpers.hpp:197-214), left side: the first position whose
// element is not less than q.
static int32_t lower_pos(const int32_t* sorted, int n, int32_t q) {
    return (int32_t)(std::lower_bound(sorted, sorted + n, q) - sorted);
}

// The selection side of the EAGLE3 draft tree (topk_generate,
// language_model_eagle3.cpp:808-1164), given the draft logits of every level
// (the draft model's forward passes between levels are the caller's):
//   level 0: the top K ids of the root row, their log-softmax as the node
//            scores, their d2t-mapped tokens, parent group 0;
//   level i = 1 .. depth-1: the top K ids of each of the K rows, each row's
//            log-softmax plus that row's score from the previous level (K*K
//            cumulative scores and tokens appended to the node lists); the
//            parent group of the level is (0, .., K-1) + 1 + K*K*max(0, i-2)
//            + (i > 1 ? K : 0) -- the reference's loop declares a new
//            topk_cs_index (:953) that hides the one its parent groups read
//            (:867, :906-908), so those stay 0 .. K-1; the best K cumulative
//            scores become the next scores, their rows (flat / K) the parent
//            rows, their mapped tokens the next input ids, and the draft
//            attention mask gains those rows of itself plus an identity block;
//   finish:  the best total_tokens node scores, their positions sorted; the
//            tokens there behind sample_token; each survivor's parent group
//            entry (position / K) minus 1 located among the sorted positions
//            (0 for the root group), + 1 -> mask_index; the tree mask is the
//            identity plus column 0 with each row OR-ed with its parent row in
//            order; position ids = row sums - 1; one retrieve row per node that
//            is nobody's parent, walked back to the root.
// logits are bf16 (dtype 1) or fp32 (0); level_logits holds depth-1 blocks of
// [K][Vd].  Outputs: inputs [depth][K] (input ids after the root and after
// each level), prow [depth-1][K] (parent rows), masks [depth-1][K][K*depth]
// (the attention mask after each level, K*(i+2) columns used, rest 0),
// tokens [N], mask [N][N], pos [N], retrieve [N][N] (-1 padded), dims =
// {leaf rows, retrieve columns}, with N = total_tokens + 1.
int orc_eagle3_tree(const void* root_logits, const void* level_logits, int dtype, int Vd,
                    const int32_t* d2t, int K, int depth, int total_tokens, int32_t sample_token,
                    int cr, int32_t* inputs, int32_t* prow, float* masks, int32_t* tokens,
                    float* mask, int32_t* pos, int32_t* retrieve, int32_t* dims,
                    float* node_scores) {
    if (K < 1 || K > 32 || depth < 1 || Vd < K || total_tokens < 1 || total_tokens > 32)
        return ORC_E_INVAL;
    const int n_nodes = K + (depth - 1) * K * K;
    if (total_tokens > n_nodes) return ORC_E_INVAL;
    const size_t esz = dtype == 0 ? 4 : 2;
    auto map_tok = [&](int32_t draft_id) { return (int32_t)(draft_id + d2t[draft_id]); };
    std::vector<float> node_score;
    std::vector<int32_t> node_tok, parent_flat;
    std::vector<float> cur(K);
    std::vector<int32_t> idx(K * K), tmp_i(K);
    std::vector<float> val(K * K), lp(K);
    // level 0
    heap_topk([&](int64_t i) { return load_logit(root_logits, dtype, i); }, Vd, K, idx.data(),
              val.data());
    orc_logsoftmax(val.data(), K, cr, cur.data());
    for (int j = 0; j < K; ++j) {
        node_score.push_back(cur[j]);
        node_tok.push_back(map_tok(idx[j]));
        inputs[j] = map_tok(idx[j]);
    }
    parent_flat.push_back(0);
    // draft attention mask: K rows, starts as the K x K identity
    const int mcols = K * depth;
    std::vector<float> am((size_t)K * mcols, 0.0f);
    for (int r = 0; r < K; ++r) am[(size_t)r * mcols + r] = 1.0f;
    int acols = K;
    for (int lv = 1; lv < depth; ++lv) {
        const int i = lv - 1;                               // the reference's loop counter
        const int32_t base = 1 + K * K * std::max(0, i - 1) + (i > 0 ? K : 0);
        for (int j = 0; j < K; ++j) parent_flat.push_back(j + base);
        const char* blk = (const char*)level_logits + (size_t)i * K * Vd * esz;
        std::vector<float> cu((size_t)K * K);
        for (int r = 0; r < K; ++r) {
            const void* row = blk + (size_t)r * Vd * esz;
            heap_topk([&](int64_t q) { return load_logit(row, dtype, q); }, Vd, K,
                      idx.data() + (size_t)r * K, val.data() + (size_t)r * K);
            orc_logsoftmax(val.data() + (size_t)r * K, K, cr, lp.data());
            for (int j = 0; j < K; ++j) cu[(size_t)r * K + j] = lp[j] + cur[r];
        }
        std::vector<int32_t> best(K);
        std::vector<float> bestv(K);
        heap_topk([&](int64_t q) { return cu[q]; }, (int64_t)K * K, K, best.data(), bestv.data());
        for (int j = 0; j < K; ++j) {
            cur[j] = bestv[j];
            prow[(size_t)i * K + j] = best[j] / K;
            inputs[(size_t)lv * K + j] = map_tok(idx[best[j]]);
        }
        for (int q = 0; q < K * K; ++q) {
            node_score.push_back(cu[q]);
            node_tok.push_back(map_tok(idx[q]));
        }
        std::vector<float> nm((size_t)K * mcols, 0.0f);
        for (int r = 0; r < K; ++r) {
            const int src = best[r] / K;
            for (int c = 0; c < acols; ++c) nm[(size_t)r * mcols + c] = am[(size_t)src * mcols + c];
            nm[(size_t)r * mcols + acols + r] = 1.0f;
        }
        acols += K;
        am.swap(nm);
        std::copy(am.begin(), am.end(), masks + (size_t)i * K * mcols);
    }
    // finish
    if (node_scores) std::copy(node_score.begin(), node_score.end(), node_scores);
    std::vector<int32_t> sel(total_tokens);
    std::vector<float> selv(total_tokens);
    heap_topk([&](int64_t q) { return node_score[q]; }, n_nodes, total_tokens, sel.data(),
              selv.data());
    std::sort(sel.begin(), sel.end());
    const int N = total_tokens + 1;
    tokens[0] = sample_token;
    std::vector<int32_t> up(total_tokens);                 // mask_index
    for (int q = 0; q < total_tokens; ++q) {
        tokens[q + 1] = node_tok[sel[q]];
        const int32_t par = parent_flat[sel[q] / K];
        up[q] = (par == 0 ? -1 : lower_pos(sel.data(), total_tokens, par - 1)) + 1;
    }
    std::vector<int> tm((size_t)N * N, 0);
    for (int r = 0; r < N; ++r) { tm[(size_t)r * N + r] = 1; tm[(size_t)r * N] = 1; }
    for (int q = 0; q < total_tokens; ++q)
        for (int c = 0; c < N; ++c) tm[(size_t)(q + 1) * N + c] |= tm[(size_t)up[q] * N + c];
    int maxpos = 0;
    for (int r = 0; r < N; ++r) {
        int sum = 0;
        for (int c = 0; c < N; ++c) { sum += tm[(size_t)r * N + c]; mask[(size_t)r * N + c] = (float)tm[(size_t)r * N + c]; }
        pos[r] = sum - 1;
        maxpos = std::max(maxpos, pos[r]);
    }
    const int rcols = maxpos + 1;
    std::vector<char> is_parent(N, 0);
    for (int q = 0; q < total_tokens; ++q) is_parent[up[q]] = 1;
    int n_parent = 0;
    for (int r = 0; r < N; ++r) n_parent += is_parent[r];
    const int leaves = total_tokens - (n_parent - 1);
    for (int q = 0; q < N * N; ++q) retrieve[q] = -1;
    int row = 0;
    for (int node = 0; node < N; ++node) {
        if (is_parent[node]) continue;
        if (row >= leaves) return ORC_E_RANGE;              // cannot happen: see dims
        int at = node;
        for (int j = pos[node]; j >= 0; --j) {
            retrieve[(size_t)row * N + j] = at;
            if (at > 0) at = up[at - 1];
        }
        ++row;
    }
    dims[0] = leaves;
    dims[1] = rcols;
    return ORC_OK;
}

// The decode loops' stop rule (language_model.cpp:643-671, language_model_dflash.cpp:
// 570-579, language_model_gemma4_mtp.cpp:940-956): the emitted run, cut at the
// cache room, ends after its first token in the stop set (kept).  status: 0
// none, 1 stop token, 2 cut by the room.
int orc_stop_check(const int32_t* tokens, const int32_t* count, int B, int M,
                   const int32_t* stop_ids, int n_stop, const int32_t* room, int32_t* keep,
                   int32_t* status) {
    if (B < 0 || M < 0) return ORC_E_INVAL;
    std::vector<int32_t> st(stop_ids, stop_ids + n_stop);
    std::sort(st.begin(), st.end());
    for (int b = 0; b < B; ++b) {
        int n = count ? std::min(std::max(count[b], 0), M) : M;
        int s = 0;
        // reaching the room fills the cache, also exactly (language_model_gemma4_mtp.cpp:
        // 953-955 sets cache_full after the append that reaches max_length)
        if (room && std::max(room[b], 0) <= n) { n = std::max(room[b], 0); s = 2; }
        int k = n;
        for (int i = 0; i < n; ++i) {
            if (std::binary_search(st.begin(), st.end(), tokens[(size_t)b * M + i])) {
                k = i + 1;
                s = 1;
                break;
            }
        }
        keep[b] = k;
        status[b] = s;
    }
    return ORC_OK;
}

// _calc_next_token_id (language_model.cpp:3689-3714) in the reference's own
// shape, for the CPU baseline of the greedy workloads: four OpenMP threads per
// row, each the scalar argmax_bf16 loop (utils.hpp:140-151, the path on x86)
// over a quarter, merged in a critical section from (values[0], 0).
int orc_calc_next_token_id_omp4(const void* row, int dtype, int V, int32_t* out) {
    if (V <= 0) return ORC_E_INVAL;
    float best_value = load_logit(row, dtype, 0);
    int64_t best_index = 0;
#pragma omp parallel for num_threads(4)
    for (int part = 0; part < 4; ++part) {
        const int64_t begin = (int64_t)V * part / 4, end = (int64_t)V * (part + 1) / 4;
        if (end > begin) {
            float v;
            int64_t i;
            argmax_split(row, dtype, begin, end - begin, &v, &i);
#pragma omp critical
            {
                if (v > best_value || (v == best_value && i < best_index)) {
                    best_value = v;
                    best_index = i;
                }
            }
        }
    }
    *out = (int32_t)best_index;
    return ORC_OK;
}

// Threads of the oracle's OpenMP loops over rows (the CPU baseline's 1-thread
// and many-thread figures).
void orc_set_threads(int n) { omp_set_num_threads(n > 0 ? n : 1); }

}  // extern "C"
