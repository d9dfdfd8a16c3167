// verify.hip -- stochastic speculative verification (rejection sampling) for
// EAGLE3 / MTP style drafts on MI355X (gfx950).
//
// Inputs: target logits [B][D+1][V] and draft logits [B][D][V] (fp32), the D
// draft ids of each sequence, uniforms u_accept[B][D] and u_resample[B].
// Probabilities are fixed-point softmax weights built per chunk of 8192 ids:
// chunk c of a row has its maximum m_c, the row its maximum M, and
//   w_i = rint(exp(x_i - m_c) 2^36),  F_c = rint(exp(m_c - M) 2^27),
//   W_i = w_i F_c,  Z = sum_c F_c sum_{i in c} w_i  (exact, 128-bit),
// so every chunk's sum needs only the chunk's own maximum: the row pass reads
// each row once and no workgroup waits for another.  Decisions:
//   accept draft k  iff  W_t(x) Z_d >= u_k W_d(x) Z_t      (IEEE double)
//   draws           on W~_i = W_i >> 32 (below 2^31); the residual at a
//                   rejection is R_i = max(0, W~_t,i z_d - W~_d,i z_t) >> 21 with
//                   z = Z >> 27 shifted (the same shift for both rows) to 32
//                   bits, so every product is one 32 x 32 -> 64-bit multiply;
//   draw            smallest id whose ascending prefix of weights exceeds
//                   (U32(u) * total) >> 32.
// The reference verifies drafts greedily (sima_lmm/devkit/cpp/eagle_helpers.hpp:153-195,
// sima_lmm/devkit/cpp/gemma4_mtp_helpers.cpp:81-111); with one-hot distributions
// this reduces to that rule.
//
// Two launches:
//   vr_rowpass  per (row, chunk of 8192 ids), one read of the rows: the chunk's
//               maximum key, the sum of w over the chunk, and w at the row's
//               draft token
//   vr_draw     per (sequence, 2048 ids): the acceptance scan (recomputed from
//               the chunk maxima and sums by every workgroup of the sequence),
//               then, for each wave's 512 ids of the draw rows, the sum of the
//               residual weights and the sum of the plain target weights.  The
//               sequence's last workgroup to finish (a per-sequence arrival
//               counter) then draws: the wave slice holding the draw target (a
//               block scan over the wave totals), then the token inside it (two
//               ids per thread, a block scan in id order), and writes
//               accepted_len and the emitted tokens.
//
// The sums that cross workgroups are stored and loaded as relaxed agent-scope
// atomics (write-through stores, loads that miss stale cache lines), and each
// workgroup waits for its stores to complete before it counts its arrival, so
// no cache writeback or invalidation is needed for the last workgroup to see
// every other workgroup's sums.
#include "common.hpp"
#include "../../include/llima_sampler.h"

namespace llima {

#define VR_E 32
#define VR_CHUNK (LLIMA_WG * VR_E)   // 8192 ids: the chunk of the weights' definition
#define VR_CSHIFT 13                 // log2(VR_CHUNK)
#define VR_MAX_D 255
#define VR_DCHUNK (LLIMA_WG * 8)     // ids per vr_drawsum workgroup (inside one chunk)
#define VR_SLICE (VR_DCHUNK / LLIMA_WAVES)   // ids per vr_draw wave: two per thread of the draw
#define VR_CNT_STRIDE 32             // arrival counters, one per 128-byte line
#define VR_WS 16                     // uint64 per vr_draw workgroup's totals: one 128-byte line
static_assert(LLIMA_WAVES == 4 && 2 * LLIMA_WAVES <= VR_WS, "a workgroup's 8 totals in its line");
#define VR_FBITS 27                  // chunk factor F_c = rint(exp(m_c - M) 2^27)
#define VR_ZBITS 32                  // width of the residual's normalizers
#define VR_RSHIFT 21                 // residual scaling (sums below 2^64 for V <= 2^22)

struct VerifyParams {
    const float* tgt;
    const float* drf;
    const int32_t* draft_ids;
    const float* u_accept;
    const float* u_resample;
    int32_t* accepted_len;
    int32_t* emitted;
    uint32_t* maxk;      // [NR][S] chunk maximum keys
    uint64_t* sums;      // [NR][S] chunk sums of w
    uint64_t* wx;        // [NR] w at the row's draft token (relative to its chunk)
    uint64_t* wsum;      // [B][SD][VR_WS]: per vr_draw workgroup, the target weight of each of
                         // its 4 waves (VR_DCHUNK / 4 ids), then their residual weight; each
                         // workgroup's line is written by it alone
    uint32_t* cnt;       // [B][VR_CNT_STRIDE] arrival counters (zeroed by vr_rowpass)
    int32_t B, D, V, S, NR, SD;
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

// Loads a chunk, E values per thread of NT: 16-byte loads from clamped,
// always-valid addresses (V is a multiple of 4), all in flight before the first
// use; in a row's last, partial chunk the values past the end become -inf.
template <int NT, int E>
__device__ __forceinline__ void load_chunk(const float* rowp, int c0, int c1, int V, float (&v)[E]) {
    llima_u32x4 q[E / 4];
#pragma unroll
    for (int j = 0; j < E / 4; ++j) {
        const int i0 = c0 + j * (NT * 4) + (int)threadIdx.x * 4;
        const int ia = i0 < V ? i0 : V - 4;
        q[j] = __builtin_nontemporal_load((const llima_u32x4*)(rowp + ia));
    }
#pragma unroll
    for (int j = 0; j < E / 4; ++j) {
        const uint32_t w4[4] = {q[j].x, q[j].y, q[j].z, q[j].w};
#pragma unroll
        for (int e = 0; e < 4; ++e) v[4 * j + e] = __uint_as_float(w4[e]);
    }
    if (c1 - c0 < VR_CHUNK) {
#pragma unroll
        for (int j = 0; j < E / 4; ++j) {
            const int i0 = c0 + j * (NT * 4) + (int)threadIdx.x * 4;
#pragma unroll
            for (int e = 0; e < 4; ++e)
                v[4 * j + e] = i0 + e < c1 ? v[4 * j + e] : -__builtin_inff();
        }
    }
}

// w of a value given its chunk's maximum key (0 when the chunk has no value).
__device__ __forceinline__ uint64_t chunk_weight(float x, uint32_t mkey) {
    if (mkey <= LLIMA_KEY_NEG_INF) return 0;
    return weight(x, key_f32(mkey));
}

// F_c = rint(exp(m_c - M) 2^27): 2^27 for the maximum's chunks, 0 for a chunk
// with no value or one more than 26 below the maximum.
__device__ __forceinline__ uint32_t chunk_factor(uint32_t mck, uint32_t Mk) {
    if (mck <= LLIMA_KEY_NEG_INF) return 0;
    if (mck == Mk) return 1u << VR_FBITS;
    const float d = key_f32(mck) - key_f32(Mk);
    if (!(d >= -26.0f)) return 0;
    return (uint32_t)__builtin_rintf(__builtin_ldexpf(exp_neg(d), VR_FBITS));
}

// ------------------------------------------------------------------ row pass
// One workgroup of VR_RT threads per (row, chunk): the chunk's maximum, its sum
// of w (relative to that maximum) and w at the row's draft token when it lies
// in the chunk.  Each reduction over the workgroup takes one barrier.
#ifndef VR_RT
#define VR_RT 256
#endif
#define VR_RE (VR_CHUNK / VR_RT)       // values per thread

__global__ __launch_bounds__(VR_RT) void vr_rowpass(VerifyParams P) {
    __shared__ uint32_t s_m[VR_RT / 64];
    __shared__ uint64_t s_s[VR_RT / 64];
    const int r = (int)blockIdx.x / P.S, c = (int)blockIdx.x - r * P.S;
    const int c0 = c * VR_CHUNK, c1 = c0 + VR_CHUNK < P.V ? c0 + VR_CHUNK : P.V;
    const float* rowp = row_ptr(P, r);
    float v[VR_RE];
    load_chunk<VR_RT, VR_RE>(rowp, c0, c1, P.V, v);
    if (blockIdx.x == 0)                                 // vr_draw's arrival counters
        for (int i = (int)threadIdx.x; i < P.B; i += VR_RT) P.cnt[(size_t)i * VR_CNT_STRIDE] = 0u;
    float m = -__builtin_inff();
#pragma unroll
    for (int e = 0; e < VR_RE; ++e) m = v[e] > m ? v[e] : m;   // NaN never counts
    const uint32_t wm = wave_max_u32(f32_key(m));
    if (lane_id() == 0) s_m[wave_id()] = wm;
    __syncthreads();
    uint32_t mkey = 0;                                  // >= f32_key(-inf) > 0
#pragma unroll
    for (int w = 0; w < VR_RT / 64; ++w) mkey = s_m[w] > mkey ? s_m[w] : mkey;
    uint64_t s = 0;
    if (mkey > LLIMA_KEY_NEG_INF) {
        const float xm = key_f32(mkey);
        double sd = 0.0;                                 // exact: VR_RE terms below 2^37
        if (xm == __builtin_inff()) {                    // w = 2^36 at every +inf, else 0
#pragma unroll
            for (int e = 0; e < VR_RE; ++e) sd += v[e] == xm ? (double)LLIMA_TWO36 : 0.0;
        } else {
#pragma unroll
            for (int e = 0; e < VR_RE; ++e) sd += (double)weight_f(v[e], xm);
        }
        s = (uint64_t)sd;
    }
    s = wave_sum_u64(s);
    if (lane_id() == 0) s_s[wave_id()] = s;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint64_t tot = 0;
#pragma unroll
        for (int w = 0; w < VR_RT / 64; ++w) tot += s_s[w];
        P.maxk[(size_t)r * P.S + c] = mkey;
        P.sums[(size_t)r * P.S + c] = tot;
        const int b = seq_of(P, r), kk = pos_of(P, r);
        if (kk < P.D) {
            const int x = P.draft_ids[b * P.D + kk];
            if (x >= c0 && x < c1) P.wx[r] = chunk_weight(rowp[x], mkey);
        }
    }
}

// ------------------------------------------------------------------ acceptance
#define VR_SEQ_ITEMS 4               // (row, chunk) items of a sequence a thread holds
#define VR_MK_LDS (VR_SEQ_ITEMS * LLIMA_WG)

struct SeqShared {
    uint32_t M[2 * VR_MAX_D + 1];          // maximum keys of target rows 0..D, then draft rows
    unsigned long long zl[2 * VR_MAX_D + 1][3];   // Z in 26-bit limbs
    uint32_t mk[VR_MK_LDS];                // chunk maxima [row q][chunk] (when they fit)
    uint8_t ok[VR_MAX_D];                  // draft k passes its acceptance test
    int32_t acc;
    int32_t last;                          // this workgroup arrived last (vr_draw)
    int32_t item, tok;                     // the draw's wave slice and token
    uint64_t before;                       // weight before that wave slice
    uint64_t w2[2][LLIMA_WAVES];           // wave totals of the draw's scans
    uint64_t w3[LLIMA_WAVES];
    BlockScratch bs;
};

__device__ __forceinline__ int row_of(const VerifyParams& P, int b, int q) {
    return q <= P.D ? trow(P, b, q) : drow(P, b, q - P.D - 1);
}

__device__ __forceinline__ llima_u128 limbs_z(const unsigned long long (&l)[3]) {
    return (llima_u128)l[0] + ((llima_u128)l[1] << 26) + ((llima_u128)l[2] << 52);
}

__device__ __forceinline__ double u128_to_double(llima_u128 z) {
    return (double)(uint64_t)(z >> 64) * 18446744073709551616.0 + (double)(uint64_t)z;
}

__device__ __forceinline__ int bitlen64(uint64_t z) { return z ? 64 - __clzll((long long)z) : 0; }

// Chunk maximum of row q (of the sequence), chunk c: from LDS when the
// sequence's maxima fit there (accept_scan staged them), else from memory.
__device__ __forceinline__ uint32_t seq_maxk(const VerifyParams& P, int b, int q, int c,
                                             const SeqShared& sh) {
    const int n = (2 * P.D + 1) * P.S;
    return n <= VR_MK_LDS ? sh.mk[q * P.S + c] : P.maxk[(size_t)row_of(P, b, q) * P.S + c];
}

// M and Z of every row of sequence b, then the acceptance scan.  Rows of at
// most 16 chunks take one DPP row each; otherwise every input is requested at
// once (up to VR_SEQ_ITEMS (row, chunk) items per thread, held in registers),
// the chunk maxima combine with LDS atomics, then each chunk's F_c S_c (below
// 2^77) is added to its row's Z in three 26-bit limbs, which sum exactly.  The D acceptance tests run in parallel, one per thread; the only
// serial part is the first failing test, found in LDS.  Returns the number of
// accepted drafts (same in every thread).
// Reduction over the 16 lanes of a DPP row (every lane gets the result).
template <class Op>
__device__ __forceinline__ uint32_t row16_reduce(uint32_t v, uint32_t identity, Op op) {
    v = op(v, dppT<DPP_QUAD_XOR1, 0xF, false>(identity, v));
    v = op(v, dppT<DPP_QUAD_XOR2, 0xF, false>(identity, v));
    v = op(v, dppT<DPP_ROW_HALF_MIRROR, 0xF, false>(identity, v));
    v = op(v, dppT<DPP_ROW_MIRROR, 0xF, false>(identity, v));
    return v;
}

__device__ __forceinline__ int accept_scan(const VerifyParams& P, int b, SeqShared& sh) {
    const int nr = 2 * P.D + 1, t = (int)threadIdx.x, n = nr * P.S;
    // per draft: w at the draft token in the target and the draft row
    int x = -1;
    uint64_t wt = 0, wd = 0;
    float ua = 0.0f;
    if (t < P.D) {
        x = P.draft_ids[b * P.D + t];
        wt = P.wx[trow(P, b, t)];
        wd = P.wx[drow(P, b, t)];
        ua = P.u_accept[b * P.D + t];
    }
    if (P.S <= 16) {
        // one DPP row of 16 lanes per sequence row, lane c holding chunk c: the
        // row maximum and the three 26-bit limbs of Z (each limb's sum of 16
        // values below 2^30) are row reductions, with no atomics
        for (int q0 = 0; q0 < nr; q0 += LLIMA_WG / 16) {          // uniform
            const int q = q0 + (t >> 4), c = t & 15;
            const bool v = q < nr && c < P.S;
            uint32_t kk = 0;
            uint64_t ss = 0;
            if (v) {
                const size_t rc = (size_t)row_of(P, b, q) * P.S + c;
                kk = P.maxk[rc];
                ss = P.sums[rc];
            }
            const uint32_t Mq = row16_reduce(kk, 0u, [](uint32_t a, uint32_t e) { return a > e ? a : e; });
            const llima_u128 fs = v ? (llima_u128)ss * chunk_factor(kk, Mq) : (llima_u128)0;
            auto add = [](uint32_t a, uint32_t e) { return a + e; };
            const uint32_t l0 = row16_reduce((uint32_t)(fs & 0x3FFFFFFu), 0u, add);
            const uint32_t l1 = row16_reduce((uint32_t)((fs >> 26) & 0x3FFFFFFu), 0u, add);
            const uint32_t l2 = row16_reduce((uint32_t)(fs >> 52), 0u, add);
            if (v && c == 0) {
                sh.M[q] = Mq;
                sh.zl[q][0] = l0; sh.zl[q][1] = l1; sh.zl[q][2] = l2;
            }
            if (v && n <= VR_MK_LDS) sh.mk[q * P.S + c] = kk;
        }
        __syncthreads();
    } else {
        for (int q = t; q < nr; q += LLIMA_WG) {
            sh.M[q] = 0;
            sh.zl[q][0] = 0; sh.zl[q][1] = 0; sh.zl[q][2] = 0;
        }
        uint32_t km[VR_SEQ_ITEMS];
        uint64_t sm[VR_SEQ_ITEMS];
#pragma unroll
        for (int j = 0; j < VR_SEQ_ITEMS; ++j) {
            const int i = t + j * LLIMA_WG;
            const int ic = i < n ? i : 0;
            const int q = ic / P.S, c = ic - q * P.S;
            const size_t rc = (size_t)row_of(P, b, q) * P.S + c;
            km[j] = P.maxk[rc];
            sm[j] = P.sums[rc];
        }
        __syncthreads();                                   // M and zl zeroed
#pragma unroll
        for (int j = 0; j < VR_SEQ_ITEMS; ++j) {
            const int i = t + j * LLIMA_WG;
            if (i < n) {
                atomicMax(&sh.M[i / P.S], km[j]);
                if (n <= VR_MK_LDS) sh.mk[i] = km[j];
            }
        }
        for (int i = t + VR_MK_LDS; i < n; i += LLIMA_WG)  // sequences with more items than that
            atomicMax(&sh.M[i / P.S], P.maxk[(size_t)row_of(P, b, i / P.S) * P.S + i % P.S]);
        __syncthreads();
        auto add_z = [&](int q, uint32_t kk, uint64_t ss) {
            const llima_u128 fs = (llima_u128)ss * chunk_factor(kk, sh.M[q]);
            atomicAdd(&sh.zl[q][0], (unsigned long long)(fs & 0x3FFFFFFull));
            atomicAdd(&sh.zl[q][1], (unsigned long long)((fs >> 26) & 0x3FFFFFFull));
            atomicAdd(&sh.zl[q][2], (unsigned long long)(fs >> 52));
        };
#pragma unroll
        for (int j = 0; j < VR_SEQ_ITEMS; ++j) {
            const int i = t + j * LLIMA_WG;
            if (i < n) add_z(i / P.S, km[j], sm[j]);
        }
        for (int i = t + VR_MK_LDS; i < n; i += LLIMA_WG) {
            const size_t rc = (size_t)row_of(P, b, i / P.S) * P.S + i % P.S;
            add_z(i / P.S, P.maxk[rc], P.sums[rc]);
        }
        __syncthreads();
    }
    // draft k passes iff W_t(x) Z_d >= u W_d(x) Z_t
    auto accept = [&](int k, int xk, uint64_t wtk, uint64_t wdk, float uk) {
        const llima_u128 zt = limbs_z(sh.zl[k]), zd = limbs_z(sh.zl[P.D + 1 + k]);
        if (!(xk >= 0 && xk < P.V && zt > 0)) return false;
        const int cx = xk >> VR_CSHIFT;
        const uint64_t Wt = wtk * chunk_factor(seq_maxk(P, b, k, cx, sh), sh.M[k]);
        const uint64_t Wd = wdk * chunk_factor(seq_maxk(P, b, P.D + 1 + k, cx, sh),
                                               sh.M[P.D + 1 + k]);
        const double lhs = (double)Wt * u128_to_double(zd);
        const double rhs = (double)uk * (double)Wd * u128_to_double(zt);
        return lhs >= rhs;
    };
    if (P.D <= 64) {
        // the tests of wave 0's lanes; the first failure is a ballot
        if (t < 64) {
            const bool ok = t < P.D && accept(t, x, wt, wd, ua);
            const uint64_t rej = ballot(t < P.D && !ok);
            if (t == 0) sh.acc = rej ? (int)__builtin_ffsll((long long)rej) - 1 : P.D;
        }
    } else {
        for (int k = t; k < P.D; k += LLIMA_WG) {
            if (k != t) {                               // D > LLIMA_WG: the rest one by one
                x = P.draft_ids[b * P.D + k];
                wt = P.wx[trow(P, b, k)];
                wd = P.wx[drow(P, b, k)];
                ua = P.u_accept[b * P.D + k];
            }
            sh.ok[k] = accept(k, x, wt, wd, ua) ? 1 : 0;
        }
        __syncthreads();
        if (t == 0) {
            int acc = 0;
            while (acc < P.D && sh.ok[acc]) ++acc;
            sh.acc = acc;
        }
    }
    __syncthreads();
    return sh.acc;
}

// The draw of a sequence: its rows and the scalars of its weights.
struct DrawCtx {
    bool residual;
    const float* t;
    const float* d;
    int rt, rd;              // row indices (for the chunk maxima)
    uint32_t Mt, Md;         // row maximum keys
    uint32_t zt, zd;         // residual normalizers
};

__device__ __forceinline__ DrawCtx draw_ctx(const VerifyParams& P, int b, int acc,
                                            const SeqShared& sh) {
    DrawCtx q;
    q.residual = acc < P.D;
    const int k = acc;                                 // target row of the draw
    q.rt = trow(P, b, k);
    q.t = row_ptr(P, q.rt);
    q.Mt = sh.M[k];
    q.d = nullptr; q.rd = 0; q.Md = 0; q.zt = 0; q.zd = 0;
    if (q.residual) {
        q.rd = drow(P, b, k);
        q.d = row_ptr(P, q.rd);
        q.Md = sh.M[P.D + 1 + k];
        const uint64_t ht = (uint64_t)(limbs_z(sh.zl[k]) >> VR_FBITS);
        const uint64_t hd = (uint64_t)(limbs_z(sh.zl[P.D + 1 + k]) >> VR_FBITS);
        const int bt = bitlen64(ht), bd = bitlen64(hd);
        const int s = (bt > bd ? bt : bd) - VR_ZBITS;
        q.zt = (uint32_t)(s > 0 ? ht >> s : ht);
        q.zd = (uint32_t)(s > 0 ? hd >> s : hd);
    }
    return q;
}

// What the draw weights of one chunk of a draw row need: the chunk's maximum
// (finite; 0 for a chunk with no value, whose factor is 0), whether it is +inf,
// and F_c 2^-32.
struct DrawChunk {
    float xm;
    bool inf;
    double fs;
};

__device__ __forceinline__ DrawChunk draw_chunk(uint32_t mck, uint32_t Mk) {
    DrawChunk c;
    const float m = key_f32(mck);
    c.inf = m == __builtin_inff();
    c.xm = mck > LLIMA_KEY_NEG_INF && !c.inf ? m : 0.0f;
    c.fs = (double)chunk_factor(mck, Mk) * 0x1p-32;
    return c;
}

// W~ = (w F) >> 32 of a value of the chunk.  w is an integral float below 2^37
// (24 significant bits at most) and F is below 2^28, so w F 2^-32 is exact in
// double and the conversion to uint32 truncates it.  In a chunk whose maximum
// is +inf, w is 2^36 at the +inf values and 0 elsewhere.
__device__ __forceinline__ uint32_t draw_weight(float x, const DrawChunk& c) {
    const float w = c.inf ? (x == __builtin_inff() ? LLIMA_TWO36 : 0.0f) : weight_f(x, c.xm);
    return (uint32_t)((double)w * c.fs);
}

// Residual weight of one id from its W~ values: each product below 2^63.
__device__ __forceinline__ uint64_t residual_weight(const DrawCtx& q, uint32_t wt, uint32_t wd) {
    const uint64_t a = (uint64_t)wt * q.zd, c = (uint64_t)wd * q.zt;
    return a > c ? (a - c) >> VR_RSHIFT : 0ull;
}

// 8 consecutive values from id i0 (a multiple of 8): two 16-byte loads from
// clamped addresses, issued by load8 and unpacked (values past the row -inf)
// by unpack8 where they are first used, so that no wait for them is placed
// before the work in between.
struct Raw8 {
    llima_u32x4 a, b;
};
__device__ __forceinline__ Raw8 load8(const float* rowp, int i0, int V) {
    const int ia = i0 < V ? i0 : V - 4, ib = i0 + 4 < V ? i0 + 4 : V - 4;
    Raw8 r;
    r.a = __builtin_nontemporal_load((const llima_u32x4*)(rowp + ia));
    r.b = __builtin_nontemporal_load((const llima_u32x4*)(rowp + ib));
    return r;
}
__device__ __forceinline__ void unpack8(const Raw8& r, int i0, int V, float (&x)[8]) {
    const uint32_t w[8] = {r.a.x, r.a.y, r.a.z, r.a.w, r.b.x, r.b.y, r.b.z, r.b.w};
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = i0 + e < V ? __uint_as_float(w[e]) : -__builtin_inff();
}

// 2 consecutive values from id j0 (even): one 8-byte load from a clamped
// address; values past the row are -inf.
__device__ __forceinline__ void load2(const float* rowp, int j0, int V, float (&x)[2]) {
    const int ja = j0 < V ? j0 : V - 2;
    const float2 a = *(const float2*)(rowp + ja);
    x[0] = j0 < V ? a.x : -__builtin_inff();
    x[1] = j0 + 1 < V ? a.y : -__builtin_inff();
}

// The draw of sequence b by its last workgroup, in two request rounds: the
// wave totals (thread t owns a contiguous range of wave slices) give the wave
// slice of VR_SLICE ids holding the target; that slice's ids, two per thread,
// scanned in id order, give the token.  The draw uses the residual unless its
// total is 0 (p_t == p_d), then the plain target weights.
__device__ __forceinline__ void draw_final(const VerifyParams& P, int b, int acc, DrawCtx q,
                                           SeqShared& sh) {
    const uint32_t t = threadIdx.x;
    const int NI = P.SD * LLIMA_WAVES, IPT = (NI + LLIMA_WG - 1) / LLIMA_WG;
    const int i0 = (int)t * IPT, i1 = i0 + IPT < NI ? i0 + IPT : NI;
    uint64_t* ws = P.wsum + (size_t)b * P.SD * VR_WS;
    auto bt = [&](int i) { return ws + (i >> 2) * VR_WS + (i & 3); };      // wave slice i
    auto br = [&](int i) { return ws + (i >> 2) * VR_WS + 4 + (i & 3); };
    const uint32_t u32 = uniform32(P.u_resample[b]);
    // the emitted drafts, requested with the totals
    const int em = (int)t < acc && (int)t < P.D ? P.draft_ids[b * P.D + t] : -1;
    if (t == 0) {
        sh.item = -1;
        sh.tok = -1;
    }
    uint64_t sr = 0, st = 0;
    for (int i = i0; i < i1; ++i) {
        sr += load_agent(br(i));
        st += load_agent(bt(i));
    }
    // exclusive scans of both sums over the workgroup, and their totals
    const uint64_t ir = wave_incl_scan_u64(sr), it = wave_incl_scan_u64(st);
    const uint32_t wv = t >> 6;
    if (lane_id() == 63) { sh.w2[0][wv] = ir; sh.w2[1][wv] = it; }
    __syncthreads();
    uint64_t brr = 0, btt = 0, tr = 0, tt = 0;
#pragma unroll
    for (int i = 0; i < LLIMA_WAVES; ++i) {
        brr += (uint32_t)i < wv ? sh.w2[0][i] : 0ull;
        btt += (uint32_t)i < wv ? sh.w2[1][i] : 0ull;
        tr += sh.w2[0][i];
        tt += sh.w2[1][i];
    }
    if (q.residual && tr == 0) q.residual = false;          // p_t == p_d: draw from p_t
    const uint64_t s = q.residual ? sr : st;
    const uint64_t before = q.residual ? brr + ir - sr : btt + it - st;
    const uint64_t total = q.residual ? tr : tt;
    const uint64_t target = (uint64_t)(((llima_u128)u32 * total) >> 32);
    if (total > 0 && s > 0 && before <= target && target < before + s) {
        if (IPT == 1) {                                    // the owner's one slice
            sh.item = i0;
            sh.before = before;
        } else {
            uint64_t a = before;
            for (int i = i0; i < i1; ++i) {                // the owner's slices, once more
                const uint64_t v = load_agent(q.residual ? br(i) : bt(i));
                if (a + v > target) { sh.item = i; sh.before = a; break; }
                a += v;
            }
        }
    }
    __syncthreads();
    const int item = sh.item;
    if (item >= 0) {
        // the slice's ids, two per thread (one chunk of both rows)
        const int j0 = item * VR_SLICE + 2 * (int)t;
        const int cc = (item * VR_SLICE) >> VR_CSHIFT;
        float xt[2], xd[2];
        load2(q.t, j0, P.V, xt);
        if (q.residual) load2(q.d, j0, P.V, xd);
        const DrawChunk ct = draw_chunk(seq_maxk(P, b, acc, cc, sh), q.Mt);
        const DrawChunk cd = draw_chunk(q.residual ? seq_maxk(P, b, P.D + 1 + acc, cc, sh) : 0u, q.Md);
        uint64_t w[2];
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const uint32_t wt = draw_weight(xt[e], ct);
            w[e] = q.residual ? residual_weight(q, wt, draw_weight(xd[e], cd)) : wt;
        }
        const uint64_t s2 = w[0] + w[1];
        const uint64_t inc = wave_incl_scan_u64(s2);
        if (lane_id() == 63) sh.w3[wv] = inc;
        __syncthreads();
        uint64_t a0 = sh.before + inc - s2;               // weight before id j0
#pragma unroll
        for (int i = 0; i < LLIMA_WAVES; ++i) a0 += (uint32_t)i < wv ? sh.w3[i] : 0ull;
        if (w[0] > 0 && a0 <= target && target < a0 + w[0]) sh.tok = j0;
        a0 += w[0];
        if (w[1] > 0 && a0 <= target && target < a0 + w[1]) sh.tok = j0 + 1;
    }
    __syncthreads();
    if ((int)t <= P.D) P.emitted[(size_t)b * (P.D + 1) + t] = (int)t == acc ? sh.tok : em;
    if (t == 0) P.accepted_len[b] = acc;
}

__global__ __launch_bounds__(LLIMA_WG) void vr_draw(VerifyParams P) {
    __shared__ SeqShared sh;
    const int b = blockIdx.x / P.SD, c = blockIdx.x % P.SD;
    const int acc = accept_scan(P, b, sh);
    // this workgroup's 2048 ids lie in one chunk of both draw rows: that
    // chunk's maxima, then the rows' values are requested before the draw
    // context is computed
    const bool residual = acc < P.D;                  // a draft was rejected
    const int cc = (c * VR_DCHUNK) >> VR_CSHIFT;
    const int rti = trow(P, b, acc), rdi = residual ? drow(P, b, acc) : rti;
    const uint32_t mkt = P.maxk[(size_t)rti * P.S + cc];
    const uint32_t mkd0 = P.maxk[(size_t)rdi * P.S + cc];
    const int i0 = c * VR_DCHUNK + (int)threadIdx.x * 8;
    const Raw8 rt = load8(row_ptr(P, rti), i0, P.V);
    Raw8 rd = {};
    if (residual) rd = load8(row_ptr(P, rdi), i0, P.V);
    const uint32_t mkd = residual ? mkd0 : 0u;
    const DrawCtx q = draw_ctx(P, b, acc, sh);
    const DrawChunk ct = draw_chunk(mkt, q.Mt);
    const DrawChunk cd = draw_chunk(mkd, q.Md);
    float xt[8], xd[8];
    unpack8(rt, i0, P.V, xt);
    unpack8(rd, i0, P.V, xd);
    uint64_t st = 0, sr = 0;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const uint32_t wt = draw_weight(xt[e], ct);
        st += wt;
        if (q.residual) sr += residual_weight(q, wt, draw_weight(xd[e], cd));
    }
    // each wave's two totals (a wave slice of VR_SLICE ids)
    const uint64_t wt_ = wave_sum_u64(st), wr_ = wave_sum_u64(sr);
    if (lane_id() == 0) {
        uint64_t* o = P.wsum + ((size_t)b * P.SD + c) * VR_WS + wave_id();
        store_agent(o, wt_);
        store_agent(o + 4, wr_);
    }
    // every store of the workgroup completes before its arrival is counted
    __builtin_amdgcn_s_waitcnt(LLIMA_WAITCNT_VM0);
    __syncthreads();
    if (threadIdx.x == 0) {
        const uint32_t n = __hip_atomic_fetch_add(P.cnt + (size_t)b * VR_CNT_STRIDE, 1u,
                                                  __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        sh.last = n + 1u == (uint32_t)P.SD;
    }
    __syncthreads();
    if (sh.last) draw_final(P, b, acc, q, sh);
}

static size_t al256(size_t x) { return (x + 255) & ~(size_t)255; }

}  // namespace llima

using namespace llima;

extern "C" size_t llima_verify_rejection_workspace_bytes(int32_t B, int32_t D, int32_t V) {
    if (B <= 0 || D < 0 || V <= 0) return 0;
    const size_t S = (size_t)(V + VR_CHUNK - 1) / VR_CHUNK;
    const size_t NR = (size_t)B * (2 * D + 1);
    const size_t SD = (size_t)(V + VR_DCHUNK - 1) / VR_DCHUNK;
    return al256(NR * S * 4) + al256(NR * S * 8) + al256(NR * 8) + al256((size_t)B * SD * VR_WS * 8) + al256((size_t)B * VR_CNT_STRIDE * 4);
}

extern "C" int llima_verify_rejection(const float* target_logits, const float* draft_logits,
                                      int32_t B, int32_t D, int32_t V, const int32_t* draft_ids,
                                      const float* u_accept, const float* u_resample,
                                      int32_t* accepted_len, int32_t* emitted, void* workspace,
                                      size_t workspace_bytes, void* stream) {
    if (B > 0 && (!target_logits || !u_resample || !accepted_len || !emitted)) return LLIMA_E_INVAL;
    if (B > 0 && D > 0 && (!draft_logits || !draft_ids || !u_accept)) return LLIMA_E_INVAL;
    if (B < 0 || D < 0 || D > VR_MAX_D || V <= 0 || V > (1 << 22)) return LLIMA_E_INVAL;
    if ((uintptr_t)target_logits % 16 || (D > 0 && (uintptr_t)draft_logits % 16) || V % 4)
        return LLIMA_E_INVAL;                  // rows are read with 16-byte loads
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
    P.SD = (V + VR_DCHUNK - 1) / VR_DCHUNK;
    char* w = (char*)workspace;
    P.maxk = (uint32_t*)w;  w += al256((size_t)P.NR * P.S * 4);
    P.sums = (uint64_t*)w;  w += al256((size_t)P.NR * P.S * 8);
    P.wx = (uint64_t*)w;    w += al256((size_t)P.NR * 8);
    P.wsum = (uint64_t*)w;  w += al256((size_t)B * P.SD * VR_WS * 8);
    P.cnt = (uint32_t*)w;
    hipStream_t st = (hipStream_t)stream;
    const uint32_t g12 = (uint32_t)P.NR * (uint32_t)P.S;
    hipLaunchKernelGGL(vr_rowpass, dim3(g12), dim3(VR_RT), 0, st, P);
    hipLaunchKernelGGL(vr_draw, dim3((uint32_t)B * (uint32_t)P.SD), dim3(LLIMA_WG), 0, st, P);
    return hipGetLastError() == hipSuccess ? LLIMA_OK : LLIMA_E_HIP;
}
