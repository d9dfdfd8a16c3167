// lmhead.hip -- LM-head matrix-vector product with a fused softcap and argmax
// epilogue for decode-sized batches on MI355X (gfx950).
//
//   logits[b][v] = cap * tanh(s / cap) (s when cap <= 0),  s = sum_h hidden[b][h] * weight[v][h]
//
// hidden [B][H] bf16, weight [V][H] bf16 (the nn.Linear layout: one vocab row
// contiguous), fp32 products and sums; then the first index of each row's
// maximum (NaN never wins).  The reference computes the LM head on the NPU and,
// with one split, takes its argmax in-graph after Gemma's softcap
// (sima_lmm/model/language_part_base.py:171-180, sima_lmm/model/model_graph.py:601,
// 868-870); the host reads back one int32 (sima_lmm/devkit/cpp/language_model.cpp:1607-1609).
//
// At decode batch sizes the product is bound by reading the weights (V H 2
// bytes, read once per pass); an MFMA tiling pays off only for wide batches.
//
// lmh_rows: 512-thread workgroups; the pass's hidden rows (NB of them) are
// staged in LDS as fp32; each wave streams whole vocab rows (lane l holds ids
// h = 8 l + 512 j of a row, 16-byte loads, the next row's loads issued before
// the current row is summed), sums each hidden row's products in fp32 (per
// lane in h order, then across the wave), applies the softcap, optionally
// writes the logits, and keeps per hidden row the 64-bit key
// (value key << 32 | ~v) of its best vocab row.  lmh_finish: one workgroup per
// hidden row reduces the waves' keys.
#include "common.hpp"
#include "../../include/llima_sampler.h"

namespace llima {

#define LMH_WG 512
#define LMH_WAVES (LMH_WG / 64)
#define LMH_MAX_H 4096                 // 8 load rounds of 512 ids per vocab row
#define LMH_R (LMH_MAX_H / 512)
#define LMH_LDS_FLOATS 16384           // 64 KB of staged hidden values

struct LmhParams {
    const uint16_t* hidden;            // [B][H]
    const uint16_t* weight;            // [V][H]
    float* out_logits;                 // [B][V] or null
    uint64_t* keys;                    // [B][NW]
    int32_t* out_ids;
    float* out_vals;                   // or null
    int32_t B, H, V, NW;
    float cap;
};

__device__ __forceinline__ float wave_sum_f32(float v) {
    return __uint_as_float(wave_reduce<uint32_t>(
        __float_as_uint(v), 0u,
        [](uint32_t a, uint32_t b) { return __float_as_uint(__uint_as_float(a) + __uint_as_float(b)); }));
}

// One vocab row's 8 rounds of 16-byte loads (8 bf16 each) for this lane;
// rounds past H, and every round when v < 0, read the weights' first 16 bytes.
__device__ __forceinline__ void issue_row(const LmhParams& P, int v, llima_u32x4 (&w)[LMH_R]) {
    const uint16_t* row = P.weight + (size_t)(v < 0 ? 0 : v) * P.H;
#pragma unroll
    for (int j = 0; j < LMH_R; ++j) {
        const int h0 = (int)lane_id() * 8 + j * 512;
        const int ho = v >= 0 && h0 < P.H ? h0 : 0;
        w[j] = __builtin_nontemporal_load((const llima_u32x4*)(row + ho));
    }
}

template <int NB>
__global__ __launch_bounds__(LMH_WG) void lmh_rows(LmhParams P, int b0, int nb) {
    __shared__ __align__(16) float xs[LMH_LDS_FLOATS];
    const int H = P.H;
    // stage hidden rows b0 .. b0 + nb - 1 as fp32 (rows nb .. NB - 1 are zero)
    for (int i = (int)threadIdx.x * 8; i < NB * H; i += LMH_WG * 8) {
        const int b = i / H, h = i - b * H;                  // H % 8 == 0: one row per group
        llima_u32x4 q = {0u, 0u, 0u, 0u};
        if (b < nb) q = *(const llima_u32x4*)(P.hidden + (size_t)(b0 + b) * H + h);
        const uint32_t u[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            xs[i + 2 * e] = __uint_as_float(u[e] << 16);
            xs[i + 2 * e + 1] = __uint_as_float(u[e] & 0xFFFF0000u);
        }
    }
    __syncthreads();
    const uint32_t lane = lane_id();
    const int wg = (int)blockIdx.x * LMH_WAVES + (int)(threadIdx.x >> 6);
    uint64_t best[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) best[b] = 0;
    llima_u32x4 wc[LMH_R], wn[LMH_R];
    int v = wg;
    issue_row(P, v < P.V ? v : -1, wc);
    while (v < P.V) {
        const int vn = v + P.NW;
        issue_row(P, vn < P.V ? vn : -1, wn);                // in flight while this row is summed
        float acc[NB];
#pragma unroll
        for (int b = 0; b < NB; ++b) acc[b] = 0.0f;
#pragma unroll
        for (int j = 0; j < LMH_R; ++j) {
            const int h0 = (int)lane * 8 + j * 512;
            if (h0 < H) {
                const uint32_t u[4] = {wc[j].x, wc[j].y, wc[j].z, wc[j].w};
                float wf[8];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    wf[2 * e] = __uint_as_float(u[e] << 16);
                    wf[2 * e + 1] = __uint_as_float(u[e] & 0xFFFF0000u);
                }
#pragma unroll
                for (int b = 0; b < NB; ++b) {
                    const float* xr = xs + b * H + h0;
                    const float4 x0 = *(const float4*)xr, x1 = *(const float4*)(xr + 4);
                    float a = acc[b];
                    a = __builtin_fmaf(wf[0], x0.x, a); a = __builtin_fmaf(wf[1], x0.y, a);
                    a = __builtin_fmaf(wf[2], x0.z, a); a = __builtin_fmaf(wf[3], x0.w, a);
                    a = __builtin_fmaf(wf[4], x1.x, a); a = __builtin_fmaf(wf[5], x1.y, a);
                    a = __builtin_fmaf(wf[6], x1.z, a); a = __builtin_fmaf(wf[7], x1.w, a);
                    acc[b] = a;
                }
            }
        }
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            float s = wave_sum_f32(acc[b]);
            if (P.cap > 0.0f) s = P.cap * tanhf(s / P.cap);
            if (b < nb && P.out_logits && lane == 0) P.out_logits[(size_t)(b0 + b) * P.V + v] = s;
            const uint64_t key = s == s ? ((uint64_t)f32_key(s) << 32) | (uint32_t)~(uint32_t)v : 0ull;
            best[b] = key > best[b] ? key : best[b];
        }
#pragma unroll
        for (int j = 0; j < LMH_R; ++j) wc[j] = wn[j];
        v = vn;
    }
    if (lane == 0) {
#pragma unroll
        for (int b = 0; b < NB; ++b)
            if (b < nb) P.keys[(size_t)(b0 + b) * P.NW + wg] = best[b];
    }
}

// One workgroup per hidden row: the greatest key over the waves (16 loads per
// thread in flight at a time).  A row with no non-NaN logit gives id 0 and a
// NaN value.
__global__ __launch_bounds__(LLIMA_WG) void lmh_finish(LmhParams P) {
    __shared__ BlockScratch bs;
    const int b = (int)blockIdx.x;
    const uint64_t* k = P.keys + (size_t)b * P.NW;
    uint64_t best = 0;
    for (int i0 = 0; i0 < P.NW; i0 += LLIMA_WG * 16) {
        uint64_t kv[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const int i = i0 + j * LLIMA_WG + (int)threadIdx.x;
            kv[j] = k[i < P.NW ? i : 0];
        }
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const bool in = i0 + j * LLIMA_WG + (int)threadIdx.x < P.NW;
            best = in && kv[j] > best ? kv[j] : best;
        }
    }
    best = block_max_u64(best, bs);
    if (threadIdx.x == 0) {
        P.out_ids[b] = best ? (int32_t)~(uint32_t)best : 0;
        if (P.out_vals) P.out_vals[b] = best ? key_f32((uint32_t)(best >> 32)) : __builtin_nanf("");
    }
}

static size_t lmh_align256(size_t x) { return (x + 255) & ~(size_t)255; }

// Waves of the rows kernel (a whole number of workgroups): two 512-thread
// workgroups per CU (64 KB of LDS each), fewer for a short vocabulary.
static int lmh_waves(int V) {
    const int nw = 256 * 2 * LMH_WAVES;
    const int need = (V + LMH_WAVES - 1) / LMH_WAVES * LMH_WAVES;
    return need < nw ? need : nw;
}

// Hidden rows per pass: as many as fit the staging buffer, at most 8.
static int lmh_rows_per_pass(int H) {
    int nb = LMH_LDS_FLOATS / H;
    nb = nb >= 8 ? 8 : nb >= 4 ? 4 : nb >= 2 ? 2 : 1;
    return nb;
}

}  // namespace llima

using namespace llima;

extern "C" size_t llima_lm_head_argmax_workspace_bytes(int32_t B, int32_t V) {
    if (B <= 0 || V <= 0) return 0;
    return lmh_align256((size_t)B * lmh_waves(V) * sizeof(uint64_t));
}

extern "C" int llima_lm_head_argmax(const void* hidden, const void* weight, int32_t B, int32_t H,
                                    int32_t V, float softcap, int32_t* out_ids, float* out_vals,
                                    float* out_logits, void* workspace, size_t workspace_bytes,
                                    void* stream) {
    if (B < 0 || H <= 0 || V <= 0 || H > LMH_MAX_H || H % 8 != 0) return LLIMA_E_INVAL;
    if (!weight || (B > 0 && (!hidden || !out_ids))) return LLIMA_E_INVAL;
    if (!(softcap == softcap) || __builtin_isinf(softcap)) return LLIMA_E_INVAL;
    if ((uintptr_t)weight % 16 || (B > 0 && (uintptr_t)hidden % 16)) return LLIMA_E_INVAL;
    if (B == 0) return LLIMA_OK;
    if (!workspace || workspace_bytes < llima_lm_head_argmax_workspace_bytes(B, V))
        return LLIMA_E_WORKSPACE;
    LmhParams P = {};
    P.hidden = (const uint16_t*)hidden;
    P.weight = (const uint16_t*)weight;
    P.out_logits = out_logits;
    P.keys = (uint64_t*)workspace;
    P.out_ids = out_ids;
    P.out_vals = out_vals;
    P.B = B; P.H = H; P.V = V;
    P.NW = lmh_waves(V);
    P.cap = softcap;
    hipStream_t st = (hipStream_t)stream;
    const int nbp = lmh_rows_per_pass(H);
    const dim3 g((uint32_t)((P.NW + LMH_WAVES - 1) / LMH_WAVES)), blk(LMH_WG);
    for (int b0 = 0; b0 < B; b0 += nbp) {
        const int nb = B - b0 < nbp ? B - b0 : nbp;
        switch (nbp) {
            case 8: hipLaunchKernelGGL(lmh_rows<8>, g, blk, 0, st, P, b0, nb); break;
            case 4: hipLaunchKernelGGL(lmh_rows<4>, g, blk, 0, st, P, b0, nb); break;
            case 2: hipLaunchKernelGGL(lmh_rows<2>, g, blk, 0, st, P, b0, nb); break;
            default: hipLaunchKernelGGL(lmh_rows<1>, g, blk, 0, st, P, b0, nb); break;
        }
    }
    hipLaunchKernelGGL(lmh_finish, dim3((uint32_t)B), dim3(LLIMA_WG), 0, st, P);
    return hipGetLastError() == hipSuccess ? LLIMA_OK : LLIMA_E_HIP;
}
