// verify.hip -- stochastic speculative verification (rejection sampling) for
// EAGLE3 / MTP style drafts on MI355X (gfx950).
//
// Inputs: target logits [B][D+1][V] and draft logits [B][D][V] (fp32), the D
// draft ids of each sequence, uniforms u_accept[B][D] and u_resample[B].
// Probabilities are fixed-point softmax weights W = rint(exp(x - max) * 2^36)
// with Z = sum W per row (exact uint64 sums), so every decision below is
// integer arithmetic and identical to the CPU restatement:
//   accept draft k  iff  W_t(x) * Z_d * 2^32 >= U32(u_k) * W_d(x) * Z_t
//   residual        R_i = max(0, W_t,i * Z_d - W_d,i * Z_t) >> shift,
//                   shift = max(0, bitlen(Z_t) + bitlen(Z_d) - 63)
//   draw            smallest id whose ascending prefix of weights exceeds
//                   (U32(u) * total) >> 32.
// The reference verifies drafts greedily (sima_lmm/devkit/cpp/eagle_helpers.hpp:153-195,
// sima_lmm/devkit/cpp/gemma4_mtp_helpers.cpp:81-111); with one-hot distributions
// this reduces to that rule.
//
// Four launches:
//   vr_clear    marks every chunk-maximum slot unpublished (0: every key of a
//               value, -inf included, is above 0)
//   vr_rowpass  per (row, chunk of 8192 ids), one read of the rows: the chunk's
//               maximum key, published in its slot; once every chunk of the row
//               has published, the sum of W over the chunk (from the values
//               still in registers), and W at the row's draft token
//   vr_drawsum  per (sequence, 2048 ids): the acceptance scan (recomputed from
//               the sums by every workgroup of the sequence), then, for every
//               group of 32 ids of the draw row, the sum of the residual
//               weights and the sum of the plain target weights.  Workgroup 0
//               of a sequence also writes accepted_len, the emitted drafts and
//               the draw context for vr_final
//   vr_final    per sequence: the group holding the draw target (a block scan
//               over the group sums), and the token inside it (one wave, one id
//               per lane).
// vr_rowpass workgroups wait for the other chunks of their row, which the
// dispatcher normally starts alongside them (a row's chunks are consecutive
// workgroups).  The wait never depends on that: a workgroup that has polled
// help_after times reads the lowest unpublished chunk of its row itself and
// publishes its maximum (the value the chunk's own workgroup publishes too),
// so every wait ends after at most help_after + S polls, whatever the order
// and residency of the workgroups.  Slots are written and polled with
// device-scope atomics (the chunks of a row may run on different XCDs, whose
// L2 caches are not coherent with each other).  help_after is VR_HELP_AFTER
// unless llima_verify_rejection_ex gives another count (0 makes every waiter
// read its row's late chunks itself); with ~1 us per poll, a row whose chunks
// are held back (e.g. by kernels of other streams occupying the CUs) delays
// its waiters by at most about help_after us before they read those chunks.
#include "common.hpp"
#include "../../include/llima_sampler.h"

namespace llima {

#define VR_E 32
#define VR_CHUNK (LLIMA_WG * VR_E)
#define VR_MAX_D 255
#define VR_DCHUNK (LLIMA_WG * 8)     // ids per vr_drawsum workgroup
#define VR_G 32                      // ids per draw group (4 threads of vr_drawsum)
#define VR_GB 16                     // group sums a vr_final thread loads at once
#define VR_HELP_AFTER 64             // polls (~1 us each) before a waiter reads a late chunk itself

// Draw context of a sequence: what vr_final needs of its acceptance step.
struct SeqCtx {
    uint64_t zt, zd;     // Z of the draw's target row, and of its draft row (residual draw)
    uint32_t mt, md;     // their maximum keys
    int32_t acc;         // accepted drafts: the draw uses target row acc
    int32_t shift;       // residual scaling
};

struct VerifyParams {
    const float* tgt;
    const float* drf;
    const int32_t* draft_ids;
    const float* u_accept;
    const float* u_resample;
    int32_t* accepted_len;
    int32_t* emitted;
    uint32_t* maxk;      // [NR][S]
    uint64_t* sums;      // [NR][S]
    uint64_t* wx;        // [NR]
    uint64_t* gres;      // [B][NG] residual weight per group of VR_G ids
    uint64_t* gtgt;      // [B][NG] target weight per group of VR_G ids
    SeqCtx* ctx;         // [B]
    int32_t B, D, V, S, NR, NG, SD;
    int32_t help_after;  // polls before a waiter reads a late chunk itself
    uint32_t* help_count;  // nullable: chunks read by waiters (cleared by vr_clear)
};

// Row r: target rows first ([B][D+1]), then draft rows ([B][D]).
__device__ __forceinline__ const float* row_ptr(const VerifyParams& P, int r) {
    const int NT = P.B * (P.D + 1);
    if (r < NT) return P.tgt + (size_t)r * P.V;
    return P.drf + (size_t)(r - NT) * P.V;
}
__device__ __forceinline__ int seq_of(const VerifyParams& P, int r) {
    const int NT = P.B * (P.D + 1);
    return r < NT ? r / (P.D + 1) : (r - NT) / P.D;
}
__device__ __forceinline__ int pos_of(const VerifyParams& P, int r) {
    const int NT = P.B * (P.D + 1);
    return r < NT ? r % (P.D + 1) : (r - NT) % P.D;
}
__device__ __forceinline__ int trow(const VerifyParams& P, int b, int k) { return b * (P.D + 1) + k; }
__device__ __forceinline__ int drow(const VerifyParams& P, int b, int k) {
    return P.B * (P.D + 1) + b * P.D + k;
}

// Loads the chunk of 32 values per thread: 16-byte loads from clamped,
// always-valid addresses (V is a multiple of 4), all in flight before the first
// use; in a row's last, partial chunk the values past the end become -inf.
__device__ __forceinline__ void load_chunk(const float* rowp, int c0, int c1, int V,
                                           float (&v)[VR_E]) {
    llima_u32x4 q[VR_E / 4];
#pragma unroll
    for (int j = 0; j < VR_E / 4; ++j) {
        const int i0 = c0 + j * (LLIMA_WG * 4) + (int)threadIdx.x * 4;
        const int ia = i0 < V ? i0 : V - 4;
        q[j] = __builtin_nontemporal_load((const llima_u32x4*)(rowp + ia));
    }
#pragma unroll
    for (int j = 0; j < VR_E / 4; ++j) {
        const uint32_t w4[4] = {q[j].x, q[j].y, q[j].z, q[j].w};
#pragma unroll
        for (int e = 0; e < 4; ++e) v[4 * j + e] = __uint_as_float(w4[e]);
    }
    if (c1 - c0 < VR_CHUNK) {
#pragma unroll
        for (int j = 0; j < VR_E / 4; ++j) {
            const int i0 = c0 + j * (LLIMA_WG * 4) + (int)threadIdx.x * 4;
#pragma unroll
            for (int e = 0; e < 4; ++e)
                v[4 * j + e] = i0 + e < c1 ? v[4 * j + e] : -__builtin_inff();
        }
    }
}

// Weight of a value given its row maximum key (0 when the row has no value).
__device__ __forceinline__ uint64_t row_weight(float x, uint32_t mkey) {
    if (mkey <= LLIMA_KEY_NEG_INF) return 0;
    return weight(x, key_f32(mkey));
}

// weight(x, xmax) for a finite xmax, as the integral float it converts
// (W < 2^37, exact in fp32): sums of at most 2^16 of them are exact in double,
// so the row sums skip the per-value float -> uint64 conversion.  exp_neg's
// steps with three folds that leave every result unchanged:
//   * d is clamped at -26 (NaN included) with no select after, since
//     rint(e^-26 2^36) = rint(0.35) = 0;
//   * the factor 2^36 is in the polynomial's coefficients: scaling every
//     coefficient by a power of two scales every rounded step by it (the
//     smallest, 2^36/5040, is far from the subnormals), and p 2^36 2^n with
//     n >= -38 stays normal, so ldexp(p 2^36, n) = ldexp(ldexp(p, n), 36);
//   * x == xmax needs no select: d = 0 gives n = 0, r = 0 and p = 2^36 exactly.
#define VR_TWO36 68719476736.0f
__device__ __forceinline__ float weight_f(float x, float xmax) {
    const float d = __builtin_fmaxf(x - xmax, -26.0f);   // fmaxf(NaN, -26) = -26
    const float kLog2e = 1.44269502162933349609375f;
    const float kLn2Hi = 0.693145751953125f;
    const float kLn2Lo = 1.428606765330187045e-06f;
    const float n = __builtin_rintf(d * kLog2e);
    float r = __builtin_fmaf(n, -kLn2Hi, d);
    r = __builtin_fmaf(n, -kLn2Lo, r);
    float p = 1.98412698412698412698e-04f * VR_TWO36;
    p = __builtin_fmaf(p, r, 1.38888888888888888889e-03f * VR_TWO36);
    p = __builtin_fmaf(p, r, 8.33333333333333333333e-03f * VR_TWO36);
    p = __builtin_fmaf(p, r, 4.16666666666666666667e-02f * VR_TWO36);
    p = __builtin_fmaf(p, r, 1.66666666666666666667e-01f * VR_TWO36);
    p = __builtin_fmaf(p, r, 0.5f * VR_TWO36);
    p = __builtin_fmaf(p, r, VR_TWO36);
    p = __builtin_fmaf(p, r, VR_TWO36);
    return __builtin_rintf(__builtin_ldexpf(p, (int)n));
}

__global__ __launch_bounds__(LLIMA_WG) void vr_clear(VerifyParams P) {
    const int n = P.NR * P.S;
    for (int i = (int)(blockIdx.x * LLIMA_WG + threadIdx.x); i < n; i += (int)(gridDim.x * LLIMA_WG))
        P.maxk[i] = 0;
    if (P.help_count && blockIdx.x == 0 && threadIdx.x == 0) *P.help_count = 0;
}

// Maximum key of chunk c of a row (every thread gets it), read one 16-byte
// load per thread at a time.
__device__ __forceinline__ uint32_t chunk_max_key(const float* rowp, int c, int V, BlockScratch& bs) {
    const int c0 = c * VR_CHUNK, c1 = c0 + VR_CHUNK < V ? c0 + VR_CHUNK : V;
    float m = -__builtin_inff();
#pragma unroll 1
    for (int j = 0; j < VR_E / 4; ++j) {                // few registers: the waiter's own chunk stays live
        const int i0 = c0 + j * (LLIMA_WG * 4) + (int)threadIdx.x * 4;
        const int ia = i0 < V ? i0 : V - 4;
        const llima_u32x4 q = *(const llima_u32x4*)(rowp + ia);
        const uint32_t w4[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float x = __uint_as_float(w4[e]);
            m = i0 + e < c1 && x > m ? x : m;
        }
    }
    return block_max_u32(f32_key(m), bs);
}

__global__ __launch_bounds__(LLIMA_WG) void vr_rowpass(VerifyParams P) {
    __shared__ BlockScratch bs;
    __shared__ uint32_t s_mkey;
    __shared__ int32_t s_miss;
    const int r = (int)blockIdx.x / P.S, c = (int)blockIdx.x - r * P.S;
    const int c0 = c * VR_CHUNK, c1 = c0 + VR_CHUNK < P.V ? c0 + VR_CHUNK : P.V;
    const float* rowp = row_ptr(P, r);
    float v[VR_E];
    load_chunk(rowp, c0, c1, P.V, v);
    float m = -__builtin_inff();
#pragma unroll
    for (int e = 0; e < VR_E; ++e) m = v[e] > m ? v[e] : m;   // NaN never counts
    const uint32_t k = block_max_u32(f32_key(m), bs);          // >= f32_key(-inf) > 0
    uint32_t* slot = P.maxk + (size_t)r * P.S;
    if (threadIdx.x == 0) __hip_atomic_store(&slot[c], k, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    // the row maximum: wave 0 polls the row's slots until all are published
    for (int round = 0;; ++round) {
        if (threadIdx.x < 64) {
            uint32_t best = 0, miss = 0xFFFFFFFFu;
            for (int i = (int)threadIdx.x; i < P.S; i += 64) {
                const uint32_t x = __hip_atomic_load(&slot[i], __ATOMIC_RELAXED,
                                                     __HIP_MEMORY_SCOPE_AGENT);
                if (x == 0) miss = (uint32_t)i < miss ? (uint32_t)i : miss;
                best = x > best ? x : best;
            }
            best = wave_max_u32(best);
            miss = wave_min_u32(miss);
            if (threadIdx.x == 0) { s_mkey = best; s_miss = (int32_t)miss; }
            if (miss != 0xFFFFFFFFu && round < P.help_after) __builtin_amdgcn_s_sleep(8);
        }
        __syncthreads();
        const int miss = s_miss;
        if (miss < 0) break;                                    // every chunk published
        if (round >= P.help_after) {                            // a late chunk: read it here
            const uint32_t km = chunk_max_key(rowp, miss, P.V, bs);
            if (threadIdx.x == 0) {
                __hip_atomic_store(&slot[miss], km, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                if (P.help_count)
                    __hip_atomic_fetch_add(P.help_count, 1u, __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT);
            }
        }
        __syncthreads();
    }
    const uint32_t mkey = s_mkey;
    uint64_t s = 0;
    if (mkey > LLIMA_KEY_NEG_INF) {
        const float xm = key_f32(mkey);
        double sd = 0.0;                                 // exact: 32 terms below 2^37
        if (xm == __builtin_inff()) {                    // W = 2^36 at every +inf, else 0
#pragma unroll
            for (int e = 0; e < VR_E; ++e) sd += v[e] == xm ? (double)VR_TWO36 : 0.0;
        } else {
#pragma unroll
            for (int e = 0; e < VR_E; ++e) sd += (double)weight_f(v[e], xm);
        }
        s = (uint64_t)sd;
    }
    s = block_sum_u64(s, bs);
    if (threadIdx.x == 0) {
        P.sums[(size_t)r * P.S + c] = s;
        const int b = seq_of(P, r), kk = pos_of(P, r);
        if (kk < P.D) {
            const int x = P.draft_ids[b * P.D + kk];
            if (x >= c0 && x < c1) P.wx[r] = row_weight(rowp[x], mkey);
        }
    }
}

// ------------------------------------------------------------------ acceptance
struct SeqShared {
    uint64_t z[2 * VR_MAX_D + 1];      // Z of target rows 0..D then draft rows 0..D-1
    uint32_t m[2 * VR_MAX_D + 1];      // maximum keys, same order
    uint8_t ok[VR_MAX_D];              // draft k passes its acceptance test
    int32_t acc;
    BlockScratch bs;
};

// Z and maximum of every row of sequence b, then the acceptance scan.  Every
// input is requested at once (the per-chunk sums are combined with LDS
// atomics) and the D acceptance tests run in parallel, one per thread: the
// only serial part is the first failing test, found in LDS.  Returns the
// number of accepted drafts (same in every thread).
__device__ __forceinline__ int accept_scan(const VerifyParams& P, int b, SeqShared& sh) {
    const int nr = 2 * P.D + 1, t = (int)threadIdx.x;
    for (int q = t; q < nr; q += LLIMA_WG) { sh.z[q] = 0; sh.m[q] = 0; }
    __syncthreads();
    for (int i = t; i < nr * P.S; i += LLIMA_WG) {
        const int q = i / P.S, c = i - q * P.S;
        const int r = q <= P.D ? trow(P, b, q) : drow(P, b, q - P.D - 1);
        atomicAdd((unsigned long long*)&sh.z[q], (unsigned long long)P.sums[(size_t)r * P.S + c]);
        atomicMax(&sh.m[q], P.maxk[(size_t)r * P.S + c]);
    }
    // per draft: W at the draft token in the target and the draft row
    int x = -1;
    uint64_t wt = 0, wd = 0;
    float ua = 0.0f;
    if (t < P.D) {
        x = P.draft_ids[b * P.D + t];
        wt = P.wx[trow(P, b, t)];
        wd = P.wx[drow(P, b, t)];
        ua = P.u_accept[b * P.D + t];
    }
    __syncthreads();
    for (int k = t; k < P.D; k += LLIMA_WG) {
        if (k != t) {                                   // D > LLIMA_WG: the rest one by one
            x = P.draft_ids[b * P.D + k];
            wt = P.wx[trow(P, b, k)];
            wd = P.wx[drow(P, b, k)];
            ua = P.u_accept[b * P.D + k];
        }
        const uint64_t zt = sh.z[k], zd = sh.z[P.D + 1 + k];
        bool ok = false;
        if (x >= 0 && x < P.V && zt > 0) {
            const llima_u128 lhs = ((llima_u128)wt * zd) << 32;
            const llima_u128 rhs = (llima_u128)uniform32(ua) * ((llima_u128)wd * zt);
            ok = lhs >= rhs;
        }
        sh.ok[k] = ok ? 1 : 0;
    }
    __syncthreads();
    if (t == 0) {
        int acc = 0;
        while (acc < P.D && sh.ok[acc]) ++acc;
        sh.acc = acc;
    }
    __syncthreads();
    return sh.acc;
}

__device__ __forceinline__ int bitlen64(uint64_t z) { return z ? 64 - __clzll((long long)z) : 0; }

struct DrawCtx {
    bool residual;
    const float* t;
    const float* d;
    uint32_t mt, md;
    uint64_t zt, zd;
    int shift;
};

__device__ __forceinline__ DrawCtx draw_ctx(const VerifyParams& P, int b, int acc,
                                            const SeqShared& sh) {
    DrawCtx q;
    q.residual = acc < P.D;
    const int k = acc;                                 // target row of the draw
    q.t = row_ptr(P, trow(P, b, k));
    q.mt = sh.m[k];
    q.zt = sh.z[k];
    q.d = nullptr; q.md = 0; q.zd = 0; q.shift = 0;
    if (q.residual) {
        q.d = row_ptr(P, drow(P, b, k));
        q.md = sh.m[P.D + 1 + k];
        q.zd = sh.z[P.D + 1 + k];
        const int s = bitlen64(q.zt) + bitlen64(q.zd) - 63;
        q.shift = s > 0 ? s : 0;
    }
    return q;
}


// Residual weight of one id from its target and draft values.
__device__ __forceinline__ uint64_t residual_weight(const DrawCtx& q, uint64_t wt, float xd) {
    const uint64_t wd = row_weight(xd, q.md);
    const llima_u128 a = (llima_u128)wt * q.zd, c = (llima_u128)wd * q.zt;
    return a > c ? (uint64_t)((a - c) >> q.shift) : 0ull;
}

// 8 consecutive values from id i0 (a multiple of 8): two 16-byte loads from
// clamped addresses; values past the row are -inf.
__device__ __forceinline__ void load8(const float* rowp, int i0, int V, float (&x)[8]) {
    const int ia = i0 < V ? i0 : V - 4, ib = i0 + 4 < V ? i0 + 4 : V - 4;
    const llima_u32x4 a = __builtin_nontemporal_load((const llima_u32x4*)(rowp + ia));
    const llima_u32x4 b = __builtin_nontemporal_load((const llima_u32x4*)(rowp + ib));
    const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = i0 + e < V ? __uint_as_float(w[e]) : -__builtin_inff();
}

__device__ __forceinline__ uint64_t quad_sum_u64(uint64_t v) {
    v += dpp64<DPP_QUAD_XOR1, 0xF, false>(0ull, v);
    v += dpp64<DPP_QUAD_XOR2, 0xF, false>(0ull, v);
    return v;
}

__global__ __launch_bounds__(LLIMA_WG) void vr_drawsum(VerifyParams P) {
    __shared__ SeqShared sh;
    const int b = blockIdx.x / P.SD, c = blockIdx.x % P.SD;
    const int acc = accept_scan(P, b, sh);
    const DrawCtx q = draw_ctx(P, b, acc, sh);       // residual iff a draft was rejected
    if (c == 0) {
        const int t = (int)threadIdx.x;
        if (t == 0) {
            SeqCtx x;
            x.zt = q.zt; x.zd = q.zd; x.mt = q.mt; x.md = q.md;
            x.acc = acc; x.shift = q.shift;
            P.ctx[b] = x;
            P.accepted_len[b] = acc;
        }
        if (t <= P.D)                                  // vr_final writes the drawn token at acc
            P.emitted[(size_t)b * (P.D + 1) + t] = t < acc ? P.draft_ids[b * P.D + t] : -1;
    }
    const int i0 = c * VR_DCHUNK + (int)threadIdx.x * 8;
    float xt[8], xd[8];
    load8(q.t, i0, P.V, xt);
    if (q.residual) load8(q.d, i0, P.V, xd);
    uint64_t st = 0, sr = 0;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const uint64_t wt = row_weight(xt[e], q.mt);
        st += wt;
        if (q.residual) sr += residual_weight(q, wt, xd[e]);
    }
    st = quad_sum_u64(st);                            // 4 threads = one group of 32 ids
    sr = quad_sum_u64(sr);
    const int g = i0 / VR_G;
    if ((threadIdx.x & 3u) == 0u && g < P.NG) {
        P.gtgt[(size_t)b * P.NG + g] = st;
        P.gres[(size_t)b * P.NG + g] = sr;
    }
}

__global__ __launch_bounds__(LLIMA_WG) void vr_final(VerifyParams P) {
    __shared__ uint64_t s_w2[2][LLIMA_WAVES];          // two scans at once
    __shared__ int32_t s_group, s_tok;
    __shared__ uint64_t s_before;
    const int b = blockIdx.x;
    const uint32_t t = threadIdx.x;
    // thread t owns the groups [t GPT, (t + 1) GPT): both arrays (residual and
    // plain target sums) are read once and scanned together (the residual
    // total decides which one the draw uses)
    const int NG = P.NG, GPT = (NG + LLIMA_WG - 1) / LLIMA_WG;
    const int g0 = (int)t * GPT, g1 = g0 + GPT < NG ? g0 + GPT : NG;
    const uint64_t* gr = P.gres + (size_t)b * NG;
    const uint64_t* gt = P.gtgt + (size_t)b * NG;
    uint64_t vr0[VR_GB], vt0[VR_GB];
#pragma unroll
    for (int j = 0; j < VR_GB; ++j) {
        const int gi = g0 + j < g1 ? g0 + j : 0;
        vr0[j] = gr[gi];
        vt0[j] = gt[gi];
    }
    const SeqCtx x = P.ctx[b];
    const int acc = x.acc;
    DrawCtx q;
    q.residual = acc < P.D;
    q.t = row_ptr(P, trow(P, b, acc));
    q.d = q.residual ? row_ptr(P, drow(P, b, acc)) : nullptr;
    q.mt = x.mt; q.md = x.md; q.zt = x.zt; q.zd = x.zd; q.shift = x.shift;
    if (t == 0) {
        s_group = -1;
        s_tok = -1;
    }
    uint64_t sr = 0, st = 0;
#pragma unroll
    for (int j = 0; j < VR_GB; ++j) {
        sr += g0 + j < g1 ? vr0[j] : 0ull;
        st += g0 + j < g1 ? vt0[j] : 0ull;
    }
    for (int gb = g0 + VR_GB; gb < g1; gb += VR_GB) {
        uint64_t vr[VR_GB], vt[VR_GB];
#pragma unroll
        for (int j = 0; j < VR_GB; ++j) {
            const int gi = gb + j < g1 ? gb + j : g0;
            vr[j] = gr[gi];
            vt[j] = gt[gi];
        }
#pragma unroll
        for (int j = 0; j < VR_GB; ++j) {
            sr += gb + j < g1 ? vr[j] : 0ull;
            st += gb + j < g1 ? vt[j] : 0ull;
        }
    }
    // exclusive scans of both sums over the workgroup, and their totals
    const uint64_t ir = wave_incl_scan_u64(sr), it = wave_incl_scan_u64(st);
    const uint32_t wv = t >> 6;
    if (lane_id() == 63) { s_w2[0][wv] = ir; s_w2[1][wv] = it; }
    __syncthreads();
    uint64_t br = 0, bt = 0, tr = 0, tt = 0;
#pragma unroll
    for (int i = 0; i < LLIMA_WAVES; ++i) {
        br += (uint32_t)i < wv ? s_w2[0][i] : 0ull;
        bt += (uint32_t)i < wv ? s_w2[1][i] : 0ull;
        tr += s_w2[0][i];
        tt += s_w2[1][i];
    }
    if (q.residual && tr == 0) q.residual = false;          // p_t == p_d: draw from p_t
    const uint64_t* sums = q.residual ? gr : gt;
    const uint64_t s = q.residual ? sr : st;
    const uint64_t before = q.residual ? br + ir - sr : bt + it - st;
    const uint64_t total = q.residual ? tr : tt;
    const uint64_t target = (uint64_t)(((llima_u128)uniform32(P.u_resample[b]) * total) >> 32);
    if (total > 0 && s > 0 && before <= target && target < before + s) {
        uint64_t a = before;
        bool found = false;
        for (int gb = g0; gb < g1 && !found; gb += VR_GB) {
            uint64_t v[VR_GB];
#pragma unroll
            for (int j = 0; j < VR_GB; ++j) v[j] = gb + j < g1 ? sums[gb + j] : 0ull;
#pragma unroll
            for (int j = 0; j < VR_GB; ++j) {
                if (!found && a + v[j] > target) { s_group = gb + j; s_before = a; found = true; }
                a += found ? 0ull : v[j];
            }
        }
    }
    __syncthreads();
    const int grp = s_group;
    if (grp >= 0 && t < 64) {
        // one id per lane: the group's weights, scanned in id order
        const int i = grp * VR_G + (int)t;
        uint64_t w = 0;
        if (t < VR_G && i < P.V) {
            const uint64_t wt = row_weight(q.t[i], q.mt);
            w = q.residual ? residual_weight(q, wt, q.d[i]) : wt;
        }
        const uint64_t inc = s_before + wave_incl_scan_u64(w);
        if (w > 0 && inc - w <= target && target < inc) s_tok = i;
    }
    __syncthreads();
    if (t == 0) P.emitted[(size_t)b * (P.D + 1) + acc] = s_tok;
}

static size_t al256(size_t x) { return (x + 255) & ~(size_t)255; }

}  // namespace llima

using namespace llima;

extern "C" size_t llima_verify_rejection_workspace_bytes(int32_t B, int32_t D, int32_t V) {
    if (B <= 0 || D < 0 || V <= 0) return 0;
    const size_t S = (size_t)(V + VR_CHUNK - 1) / VR_CHUNK;
    const size_t NR = (size_t)B * (2 * D + 1);
    const size_t NG = (size_t)(V + VR_G - 1) / VR_G;
    return al256(NR * S * 4) + al256(NR * S * 8) + al256(NR * 8) + 2 * al256((size_t)B * NG * 8) +
           al256((size_t)B * sizeof(SeqCtx));
}

extern "C" int llima_verify_rejection_ex(const float* target_logits, const float* draft_logits,
                                         int32_t B, int32_t D, int32_t V, const int32_t* draft_ids,
                                         const float* u_accept, const float* u_resample,
                                         int32_t* accepted_len, int32_t* emitted,
                                         int32_t help_after, uint32_t* help_count,
                                         void* workspace, size_t workspace_bytes, void* stream) {
    if (B > 0 && (!target_logits || !u_resample || !accepted_len || !emitted)) return LLIMA_E_INVAL;
    if (B > 0 && D > 0 && (!draft_logits || !draft_ids || !u_accept)) return LLIMA_E_INVAL;
    if (B < 0 || D < 0 || D > VR_MAX_D || V <= 0 || V > (1 << 22)) return LLIMA_E_INVAL;
    if ((uintptr_t)target_logits % 16 || (D > 0 && (uintptr_t)draft_logits % 16) || V % 4)
        return LLIMA_E_INVAL;                  // rows are read with 16-byte loads
    if (help_after > (1 << 20)) return LLIMA_E_INVAL;
    if (B == 0) return LLIMA_OK;
    if (!workspace || workspace_bytes < llima_verify_rejection_workspace_bytes(B, D, V))
        return LLIMA_E_WORKSPACE;
    VerifyParams P;
    P.tgt = target_logits; P.drf = draft_logits; P.draft_ids = draft_ids;
    P.u_accept = u_accept; P.u_resample = u_resample;
    P.accepted_len = accepted_len; P.emitted = emitted;
    P.B = B; P.D = D; P.V = V;
    P.S = (V + VR_CHUNK - 1) / VR_CHUNK;
    P.NR = B * (2 * D + 1);
    P.NG = (V + VR_G - 1) / VR_G;
    P.SD = (V + VR_DCHUNK - 1) / VR_DCHUNK;
    P.help_after = help_after < 0 ? VR_HELP_AFTER : help_after;
    P.help_count = help_count;
    char* w = (char*)workspace;
    P.maxk = (uint32_t*)w;  w += al256((size_t)P.NR * P.S * 4);
    P.sums = (uint64_t*)w;  w += al256((size_t)P.NR * P.S * 8);
    P.wx = (uint64_t*)w;    w += al256((size_t)P.NR * 8);
    P.gres = (uint64_t*)w;  w += al256((size_t)B * P.NG * 8);
    P.gtgt = (uint64_t*)w;  w += al256((size_t)B * P.NG * 8);
    P.ctx = (SeqCtx*)w;
    hipStream_t st = (hipStream_t)stream;
    const uint32_t g12 = (uint32_t)P.NR * (uint32_t)P.S;
    const uint32_t gc = (g12 + LLIMA_WG - 1) / LLIMA_WG;
    hipLaunchKernelGGL(vr_clear, dim3(gc < 64 ? gc : 64), dim3(LLIMA_WG), 0, st, P);
    hipLaunchKernelGGL(vr_rowpass, dim3(g12), dim3(LLIMA_WG), 0, st, P);
    hipLaunchKernelGGL(vr_drawsum, dim3((uint32_t)B * (uint32_t)P.SD), dim3(LLIMA_WG), 0, st, P);
    hipLaunchKernelGGL(vr_final, dim3((uint32_t)B), dim3(LLIMA_WG), 0, st, P);
    return hipGetLastError() == hipSuccess ? LLIMA_OK : LLIMA_E_HIP;
}

extern "C" int llima_verify_rejection(const float* target_logits, const float* draft_logits,
                                      int32_t B, int32_t D, int32_t V, const int32_t* draft_ids,
                                      const float* u_accept, const float* u_resample,
                                      int32_t* accepted_len, int32_t* emitted, void* workspace,
                                      size_t workspace_bytes, void* stream) {
    return llima_verify_rejection_ex(target_logits, draft_logits, B, D, V, draft_ids, u_accept,
                                     u_resample, accepted_len, emitted, -1, nullptr, workspace,
                                     workspace_bytes, stream);
}
