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
// Four launches, no atomics or fences between workgroups (each writes its own
// workspace slots; a later launch reads them):
//   vr_rowmax   per (row, chunk) maximum key
//   vr_rowsum   per (row, chunk) sum of W, and W at each row's draft token
//   vr_drawsum  per (sequence, chunk): the acceptance scan (recomputed from the
//               sums by every workgroup of the sequence), then the chunk's sum
//               of residual weights when a draft was rejected
//   vr_final    per sequence: acceptance, emitted drafts, the chunk holding the
//               draw target, and the scan of that chunk for the token.
// Pass 2 re-reads the rows right after pass 1; at these sizes they are still
// resident in the 256 MB Infinity Cache.
#include "common.hpp"
#include "../../include/llima_sampler.h"

namespace llima {

#define VR_E 32
#define VR_CHUNK (LLIMA_WG * VR_E)
#define VR_MAX_D 255

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
    uint64_t* res;       // [B][S]
    int32_t B, D, V, S, NR;
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
// use; values past the end of the row become -inf.
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
        const int i0 = c0 + j * (LLIMA_WG * 4) + (int)threadIdx.x * 4;
        const uint32_t w4[4] = {q[j].x, q[j].y, q[j].z, q[j].w};
#pragma unroll
        for (int e = 0; e < 4; ++e)
            v[4 * j + e] = i0 + e < c1 ? __uint_as_float(w4[e]) : -__builtin_inff();
    }
}

// Weight of a value given its row maximum key (0 when the row has no value).
__device__ __forceinline__ uint64_t row_weight(float x, uint32_t mkey) {
    if (mkey <= LLIMA_KEY_NEG_INF) return 0;
    return weight(x, key_f32(mkey));
}

__global__ __launch_bounds__(LLIMA_WG) void vr_rowmax(VerifyParams P) {
    __shared__ BlockScratch bs;
    const int r = blockIdx.x / P.S, c = blockIdx.x % P.S;
    const int c0 = c * VR_CHUNK, c1 = c0 + VR_CHUNK < P.V ? c0 + VR_CHUNK : P.V;
    float v[VR_E];
    load_chunk(row_ptr(P, r), c0, c1, P.V, v);
    uint32_t m = 0;
#pragma unroll
    for (int e = 0; e < VR_E; ++e) {
        const uint32_t k = v[e] == v[e] ? f32_key(v[e]) : 0u;   // NaN never counts
        m = k > m ? k : m;
    }
    m = block_max_u32(m, bs);
    if (threadIdx.x == 0) P.maxk[(size_t)r * P.S + c] = m;
}

__global__ __launch_bounds__(LLIMA_WG) void vr_rowsum(VerifyParams P) {
    __shared__ BlockScratch bs;
    __shared__ uint32_t s_mkey;
    const int r = blockIdx.x / P.S, c = blockIdx.x % P.S;
    const int c0 = c * VR_CHUNK, c1 = c0 + VR_CHUNK < P.V ? c0 + VR_CHUNK : P.V;
    const float* rowp = row_ptr(P, r);
    float v[VR_E];
    load_chunk(rowp, c0, c1, P.V, v);
    if (threadIdx.x < 64) {
        const uint32_t* m = P.maxk + (size_t)r * P.S;
        uint32_t best = 0;
        for (int i = (int)threadIdx.x; i < P.S; i += 64) best = m[i] > best ? m[i] : best;
        best = wave_max_u32(best);
        if (threadIdx.x == 0) s_mkey = best;
    }
    __syncthreads();
    const uint32_t mkey = s_mkey;
    uint64_t s = 0;
#pragma unroll
    for (int e = 0; e < VR_E; ++e) s += row_weight(v[e], mkey);
    s = block_sum_u64(s, bs);
    if (threadIdx.x == 0) {
        P.sums[(size_t)r * P.S + c] = s;
        const int b = seq_of(P, r), k = pos_of(P, r);
        if (k < P.D) {
            const int x = P.draft_ids[b * P.D + k];
            if (x >= c0 && x < c1) P.wx[r] = row_weight(rowp[x], mkey);
        }
    }
}

// ------------------------------------------------------------------ acceptance
struct SeqShared {
    uint64_t z[2 * VR_MAX_D + 1];      // Z of target rows 0..D then draft rows 0..D-1
    uint32_t m[2 * VR_MAX_D + 1];      // maximum keys, same order
    int32_t acc;
    BlockScratch bs;
};

// Z and maximum of every row of sequence b (one wavefront per row), then the
// acceptance scan.  Returns the number of accepted drafts (same in every thread).
__device__ __forceinline__ int accept_scan(const VerifyParams& P, int b, SeqShared& sh) {
    const int nr = 2 * P.D + 1;
    for (int q = (int)(threadIdx.x >> 6); q < nr; q += LLIMA_WAVES) {
        const int r = q <= P.D ? trow(P, b, q) : drow(P, b, q - P.D - 1);
        uint64_t z = 0;
        uint32_t m = 0;
        for (int i = (int)lane_id(); i < P.S; i += 64) {
            z += P.sums[(size_t)r * P.S + i];
            const uint32_t mk = P.maxk[(size_t)r * P.S + i];
            m = mk > m ? mk : m;
        }
        z = wave_sum_u64(z);
        m = wave_max_u32(m);
        if (lane_id() == 0) { sh.z[q] = z; sh.m[q] = m; }
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        int acc = 0;
        for (; acc < P.D; ++acc) {
            const int x = P.draft_ids[b * P.D + acc];
            const uint64_t zt = sh.z[acc], zd = sh.z[P.D + 1 + acc];
            bool ok = false;
            if (x >= 0 && x < P.V && zt > 0) {
                const uint64_t wt = P.wx[trow(P, b, acc)], wd = P.wx[drow(P, b, acc)];
                const llima_u128 lhs = ((llima_u128)wt * zd) << 32;
                const llima_u128 rhs = (llima_u128)uniform32(P.u_accept[b * P.D + acc]) *
                                       ((llima_u128)wd * zt);
                ok = lhs >= rhs;
            }
            if (!ok) break;
        }
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

__device__ __forceinline__ uint64_t draw_weight(const DrawCtx& q, int i) {
    const uint64_t wt = row_weight(q.t[i], q.mt);
    if (!q.residual) return wt;
    const uint64_t wd = row_weight(q.d[i], q.md);
    const llima_u128 a = (llima_u128)wt * q.zd, c = (llima_u128)wd * q.zt;
    return a > c ? (uint64_t)((a - c) >> q.shift) : 0ull;
}

__global__ __launch_bounds__(LLIMA_WG) void vr_drawsum(VerifyParams P) {
    __shared__ SeqShared sh;
    const int b = blockIdx.x / P.S, c = blockIdx.x % P.S;
    const int acc = accept_scan(P, b, sh);
    if (acc >= P.D) return;                          // bonus draw: no residual
    const DrawCtx q = draw_ctx(P, b, acc, sh);
    const int c0 = c * VR_CHUNK, c1 = c0 + VR_CHUNK < P.V ? c0 + VR_CHUNK : P.V;
    uint64_t s = 0;
    for (int i = c0 + (int)threadIdx.x; i < c1; i += LLIMA_WG) s += draw_weight(q, i);
    s = block_sum_u64(s, sh.bs);
    if (threadIdx.x == 0) P.res[(size_t)b * P.S + c] = s;
}

__global__ __launch_bounds__(LLIMA_WG) void vr_final(VerifyParams P) {
    __shared__ SeqShared sh;
    __shared__ int32_t s_chunk, s_tok;
    __shared__ uint64_t s_before, s_target;
    __shared__ bool s_residual;
    const int b = blockIdx.x;
    const int acc = accept_scan(P, b, sh);
    DrawCtx q = draw_ctx(P, b, acc, sh);
    const int rt = trow(P, b, acc);
    if (threadIdx.x == 0) {
        int32_t* em = P.emitted + (size_t)b * (P.D + 1);
        for (int j = 0; j < acc; ++j) em[j] = P.draft_ids[b * P.D + j];
        for (int j = acc; j <= P.D; ++j) em[j] = -1;
        P.accepted_len[b] = acc;
        // locate the chunk that holds the draw target
        const uint64_t* sums = P.res + (size_t)b * P.S;
        uint64_t total = 0;
        bool residual = q.residual;
        if (residual) {
            for (int j = 0; j < P.S; ++j) total += sums[j];
            if (total == 0) residual = false;          // p_t == p_d: draw from p_t
        }
        if (!residual) {
            sums = P.sums + (size_t)rt * P.S;
            total = q.zt;
        }
        int32_t chunk = -1;
        uint64_t before = 0, target = 0;
        if (total > 0) {
            target = (uint64_t)(((llima_u128)uniform32(P.u_resample[b]) * total) >> 32);
            for (int j = 0; j < P.S; ++j) {
                const uint64_t sj = sums[j];
                if (before + sj > target) { chunk = j; break; }
                before += sj;
            }
        }
        s_chunk = chunk; s_before = before; s_target = target; s_residual = residual;
        s_tok = -1;
    }
    __syncthreads();
    const int chunk = s_chunk;
    if (chunk >= 0) {
        q.residual = s_residual;
        const int c0 = chunk * VR_CHUNK, c1 = c0 + VR_CHUNK < P.V ? c0 + VR_CHUNK : P.V;
        // thread t owns the contiguous ids [c0 + t*VR_E, c0 + (t+1)*VR_E)
        const int lo = c0 + (int)threadIdx.x * VR_E;
        const int hi = lo + VR_E < c1 ? lo + VR_E : c1;
        uint64_t sub = 0;
        for (int i = lo; i < hi; ++i) sub += draw_weight(q, i);
        uint64_t tot;
        uint64_t a = s_before + block_excl_scan_u64(sub, &tot, sh.bs);
        const uint64_t target = s_target;
        if (sub > 0 && a <= target && target < a + sub) {
            for (int i = lo; i < hi; ++i) {
                a += draw_weight(q, i);
                if (a > target) { s_tok = i; break; }
            }
        }
    }
    __syncthreads();
    if (threadIdx.x == 0) P.emitted[(size_t)b * (P.D + 1) + acc] = s_tok;
}

static size_t al256(size_t x) { return (x + 255) & ~(size_t)255; }

}  // namespace llima

using namespace llima;

extern "C" size_t llima_verify_rejection_workspace_bytes(int32_t B, int32_t D, int32_t V) {
    if (B <= 0 || D < 0 || V <= 0) return 0;
    const size_t S = (size_t)(V + VR_CHUNK - 1) / VR_CHUNK;
    const size_t NR = (size_t)B * (2 * D + 1);
    return al256(NR * S * 4) + al256(NR * S * 8) + al256(NR * 8) + al256((size_t)B * S * 8);
}

extern "C" int llima_verify_rejection(const float* target_logits, const float* draft_logits,
                                      int32_t B, int32_t D, int32_t V, const int32_t* draft_ids,
                                      const float* u_accept, const float* u_resample,
                                      int32_t* accepted_len, int32_t* emitted, void* workspace,
                                      size_t workspace_bytes, void* stream) {
    if (!target_logits || !u_resample || !accepted_len || !emitted) return LLIMA_E_INVAL;
    if (D > 0 && (!draft_logits || !draft_ids || !u_accept)) return LLIMA_E_INVAL;
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
    char* w = (char*)workspace;
    P.maxk = (uint32_t*)w;  w += al256((size_t)P.NR * P.S * 4);
    P.sums = (uint64_t*)w;  w += al256((size_t)P.NR * P.S * 8);
    P.wx = (uint64_t*)w;    w += al256((size_t)P.NR * 8);
    P.res = (uint64_t*)w;
    hipStream_t st = (hipStream_t)stream;
    const uint32_t g12 = (uint32_t)P.NR * (uint32_t)P.S;
    hipLaunchKernelGGL(vr_rowmax, dim3(g12), dim3(LLIMA_WG), 0, st, P);
    hipLaunchKernelGGL(vr_rowsum, dim3(g12), dim3(LLIMA_WG), 0, st, P);
    hipLaunchKernelGGL(vr_drawsum, dim3((uint32_t)B * (uint32_t)P.S), dim3(LLIMA_WG), 0, st, P);
    hipLaunchKernelGGL(vr_final, dim3((uint32_t)B), dim3(LLIMA_WG), 0, st, P);
    return hipGetLastError() == hipSuccess ? LLIMA_OK : LLIMA_E_HIP;
}
