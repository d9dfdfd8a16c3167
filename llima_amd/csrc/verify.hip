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
// Three launches: (1) row maxima, (2) row sums Z, per-chunk sums and the weight
// at each draft token, with the acceptance scan run by the last workgroup of
// each sequence, (3) the residual (or bonus) draw: per-chunk residual sums, then
// the last workgroup of the sequence finds the chunk holding the target and
// scans it.  Pass (2) re-reads the rows right after pass (1); at these sizes
// they are still resident in the 256 MB Infinity Cache.
#include "common.hpp"
#include "../../include/llima_sampler.h"

namespace llima {

#define VR_E 32
#define VR_CHUNK (LLIMA_WG * VR_E)

enum { JOB_RESIDUAL = 0, JOB_BONUS = 1 };

// Workspace: one fixed-size slot per row index r (target rows first, then
// draft rows).  Slot b also carries sequence b's counters, job and residual
// chunk sums.  Positions never depend on the call's shape, so a workspace can
// be reused for any shape; the control words are left zero after every call.
#define VR_SMAX 512                       // chunks per row: V <= 2^22
struct VRowSlot {
    uint32_t row_max;     // key of the row maximum (0 = no value)
    uint32_t seq_done2;   // sequence counters (slot b)
    uint32_t seq_done3;
    int32_t job_kind;
    uint64_t row_z;
    uint64_t row_wx;      // weight of the draft token in rows k < D
    int32_t job_k;
    int32_t pad[7];
    uint64_t chunk_sum[VR_SMAX];
    uint64_t res_sum[VR_SMAX];
};

struct VerifyParams {
    const float* tgt;
    const float* drf;
    const int32_t* draft_ids;
    const float* u_accept;
    const float* u_resample;
    int32_t* accepted_len;
    int32_t* emitted;
    VRowSlot* ws;
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

// Loads the chunk of 32 values per thread (16-byte loads, -inf past the end).
__device__ __forceinline__ void load_chunk(const float* rowp, int c0, int c1, float (&v)[VR_E]) {
#pragma unroll
    for (int j = 0; j < VR_E / 4; ++j) {
        const int i0 = c0 + j * (LLIMA_WG * 4) + (int)threadIdx.x * 4;
        if (i0 + 4 <= c1) {
            float4 q = *(const float4*)(rowp + i0);
            v[4 * j] = q.x; v[4 * j + 1] = q.y; v[4 * j + 2] = q.z; v[4 * j + 3] = q.w;
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) v[4 * j + e] = i0 + e < c1 ? rowp[i0 + e] : -__builtin_inff();
        }
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
    load_chunk(row_ptr(P, r), c0, c1, v);
    uint32_t m = 0;
#pragma unroll
    for (int e = 0; e < VR_E; ++e) {
        const uint32_t k = v[e] == v[e] ? f32_key(v[e]) : 0u;   // NaN never counts
        m = k > m ? k : m;
    }
    m = block_max_u32(m, bs);
    if (threadIdx.x == 0 && m) atomicMax(&P.ws[r].row_max, m);
}

__global__ __launch_bounds__(LLIMA_WG) void vr_rowsum(VerifyParams P) {
    __shared__ BlockScratch bs;
    __shared__ uint32_t flag;
    const int r = blockIdx.x / P.S, c = blockIdx.x % P.S;
    const int c0 = c * VR_CHUNK, c1 = c0 + VR_CHUNK < P.V ? c0 + VR_CHUNK : P.V;
    const float* rowp = row_ptr(P, r);
    const uint32_t mkey = P.ws[r].row_max;
    float v[VR_E];
    load_chunk(rowp, c0, c1, v);
    uint64_t s = 0;
#pragma unroll
    for (int e = 0; e < VR_E; ++e) s += row_weight(v[e], mkey);
    s = block_sum_u64(s, bs);
    const int b = seq_of(P, r), k = pos_of(P, r);
    if (threadIdx.x == 0) {
        P.ws[r].chunk_sum[c] = s;
        if (s) atomicAdd((unsigned long long*)&P.ws[r].row_z, (unsigned long long)s);
        if (k < P.D) {
            const int x = P.draft_ids[b * P.D + k];
            if (x >= c0 && x < c1) P.ws[r].row_wx = row_weight(rowp[x], mkey);
        }
    }
    const uint32_t expected = (uint32_t)(2 * P.D + 1) * (uint32_t)P.S;
    if (!arrive_last(&P.ws[b].seq_done2, expected, &flag)) return;
    if (threadIdx.x != 0) return;

    // ---- acceptance scan of sequence b
    int32_t* em = P.emitted + (size_t)b * (P.D + 1);
    int acc = 0;
    for (; acc < P.D; ++acc) {
        const int x = P.draft_ids[b * P.D + acc];
        const int rt = trow(P, b, acc), rd = drow(P, b, acc);
        const uint64_t zt = load_coherent(&P.ws[rt].row_z), zd = load_coherent(&P.ws[rd].row_z);
        bool ok = false;
        if (x >= 0 && x < P.V && zt > 0) {
            const uint64_t wt = load_coherent(&P.ws[rt].row_wx), wd = load_coherent(&P.ws[rd].row_wx);
            const llima_u128 lhs = ((llima_u128)wt * zd) << 32;
            const llima_u128 rhs = (llima_u128)uniform32(P.u_accept[b * P.D + acc]) * ((llima_u128)wd * zt);
            ok = lhs >= rhs;
        }
        if (!ok) break;
        em[acc] = x;
    }
    for (int j = acc; j <= P.D; ++j) em[j] = -1;
    P.accepted_len[b] = acc;
    P.ws[b].job_kind = acc < P.D ? JOB_RESIDUAL : JOB_BONUS;
    P.ws[b].job_k = acc;
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

__device__ __forceinline__ uint64_t draw_weight(const DrawCtx& q, int i) {
    const uint64_t wt = row_weight(q.t[i], q.mt);
    if (!q.residual) return wt;
    const uint64_t wd = row_weight(q.d[i], q.md);
    const llima_u128 a = (llima_u128)wt * q.zd, c = (llima_u128)wd * q.zt;
    return a > c ? (uint64_t)((a - c) >> q.shift) : 0ull;
}

__global__ __launch_bounds__(LLIMA_WG) void vr_draw(VerifyParams P) {
    __shared__ BlockScratch bs;
    __shared__ uint32_t flag;
    __shared__ int32_t s_chunk, s_tok;
    __shared__ uint64_t s_before, s_target;
    __shared__ bool s_residual;
    const int b = blockIdx.x / P.S, c = blockIdx.x % P.S;
    int kind = P.ws[b].job_kind, k = P.ws[b].job_k;
    // a job is only ever {RESIDUAL, k < D} or {BONUS, D}
    if (!(kind == JOB_RESIDUAL && k >= 0 && k < P.D)) { kind = JOB_BONUS; k = P.D; }
    const int rt = trow(P, b, k);
    DrawCtx q;
    q.residual = kind == JOB_RESIDUAL;
    q.t = row_ptr(P, rt);
    q.mt = P.ws[rt].row_max;
    q.zt = P.ws[rt].row_z;
    q.d = nullptr; q.md = 0; q.zd = 0; q.shift = 0;
    if (q.residual) {
        const int rd = drow(P, b, k);
        q.d = row_ptr(P, rd);
        q.md = P.ws[rd].row_max;
        q.zd = P.ws[rd].row_z;
        const int sh = bitlen64(q.zt) + bitlen64(q.zd) - 63;
        q.shift = sh > 0 ? sh : 0;
        const int c0 = c * VR_CHUNK, c1 = c0 + VR_CHUNK < P.V ? c0 + VR_CHUNK : P.V;
        uint64_t s = 0;
        for (int i = c0 + (int)threadIdx.x; i < c1; i += LLIMA_WG) s += draw_weight(q, i);
        s = block_sum_u64(s, bs);
        if (threadIdx.x == 0) P.ws[b].res_sum[c] = s;
    }
    if (!arrive_last(&P.ws[b].seq_done3, (uint32_t)P.S, &flag)) return;

    // ---- last workgroup of the sequence: locate the chunk, then the id
    if (threadIdx.x == 0) {
        const uint64_t* sums = P.ws[b].res_sum;
        uint64_t total = 0;
        bool residual = q.residual;
        if (residual) {
            for (int j = 0; j < P.S; ++j) total += load_coherent(&sums[j]);
            if (total == 0) residual = false;          // p_t == p_d: draw from p_t
        }
        if (!residual) {
            sums = P.ws[rt].chunk_sum;
            total = q.zt;
        }
        int32_t chunk = -1;
        uint64_t before = 0, target = 0;
        if (total > 0) {
            target = (uint64_t)(((llima_u128)uniform32(P.u_resample[b]) * total) >> 32);
            for (int j = 0; j < P.S; ++j) {
                const uint64_t sj = load_coherent(&sums[j]);
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
        uint64_t acc = s_before + block_excl_scan_u64(sub, &tot, bs);
        const uint64_t target = s_target;
        if (sub > 0 && acc <= target && target < acc + sub) {
            for (int i = lo; i < hi; ++i) {
                acc += draw_weight(q, i);
                if (acc > target) { s_tok = i; break; }
            }
        }
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        P.emitted[(size_t)b * (P.D + 1) + k] = s_tok;
        // leave the workspace zeroed for the next call
        for (int j = 0; j <= P.D; ++j) {
            const int r1 = trow(P, b, j);
            P.ws[r1].row_max = 0; P.ws[r1].row_z = 0; P.ws[r1].row_wx = 0;
            if (j < P.D) {
                const int r2 = drow(P, b, j);
                P.ws[r2].row_max = 0; P.ws[r2].row_z = 0; P.ws[r2].row_wx = 0;
            }
        }
    }
}

}  // namespace llima

using namespace llima;

extern "C" size_t llima_verify_rejection_workspace_bytes(int32_t B, int32_t D, int32_t V) {
    if (B <= 0 || D < 0 || V <= 0) return 0;
    return (size_t)B * (2 * D + 1) * sizeof(VRowSlot);
}

extern "C" int llima_verify_rejection(const float* target_logits, const float* draft_logits,
                                      int32_t B, int32_t D, int32_t V, const int32_t* draft_ids,
                                      const float* u_accept, const float* u_resample,
                                      int32_t* accepted_len, int32_t* emitted, void* workspace,
                                      size_t workspace_bytes, void* stream) {
    if (!target_logits || !u_resample || !accepted_len || !emitted) return LLIMA_E_INVAL;
    if (D > 0 && (!draft_logits || !draft_ids || !u_accept)) return LLIMA_E_INVAL;
    if (B < 0 || D < 0 || V <= 0 || V > (1 << 22)) return LLIMA_E_INVAL;
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
    P.ws = (VRowSlot*)workspace;
    hipStream_t st = (hipStream_t)stream;
    const uint32_t g12 = (uint32_t)P.NR * (uint32_t)P.S;
    hipLaunchKernelGGL(vr_rowmax, dim3(g12), dim3(LLIMA_WG), 0, st, P);
    hipLaunchKernelGGL(vr_rowsum, dim3(g12), dim3(LLIMA_WG), 0, st, P);
    hipLaunchKernelGGL(vr_draw, dim3((uint32_t)B * (uint32_t)P.S), dim3(LLIMA_WG), 0, st, P);
    return hipGetLastError() == hipSuccess ? LLIMA_OK : LLIMA_E_HIP;
}
