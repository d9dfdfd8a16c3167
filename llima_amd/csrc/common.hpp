// common.hpp -- device helpers shared by the token-selection kernels (gfx950).
//
// Conventions used throughout the library:
//   * a workgroup is 256 threads = 4 wavefronts of 64 lanes;
//   * "key" is the order-preserving uint32 image of an fp32 value (larger float
//     -> larger key), with -0 folded onto +0 so that key equality is float
//     equality; key 0 is below every real key and means "no value";
//   * sampling weights are fixed-point integers W = rint(exp(x - xmax) * 2^36),
//     so every sum is an exact, order-independent uint64 (this is what makes the
//     token ids bit-identical across tilings and against the CPU restatement).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define LLIMA_WG 256
#define LLIMA_WAVES (LLIMA_WG / 64)
#define LLIMA_W_ONE (1ull << 36)

typedef unsigned __int128 llima_u128;
typedef uint32_t llima_u32x4 __attribute__((ext_vector_type(4)));   // 16-byte load unit

namespace llima {

// ------------------------------------------------------------------ floats/keys
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) {
    return __uint_as_float(h << 16);
}

__device__ __forceinline__ uint32_t f32_key(float f) {
    uint32_t u = __float_as_uint(f);
    u = (u == 0x80000000u) ? 0u : u;                    // -0 -> +0
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ float key_f32(uint32_t k) {
    uint32_t u = (k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k;
    return __uint_as_float(u);
}

#define LLIMA_KEY_NEG_INF 0x007FFFFFu   // f32_key(-inf)

// ------------------------------------------------------------------ exp / weights
// exp(d), d <= 0: Cody-Waite reduction e^d = 2^n e^r with a degree-7 Taylor
// polynomial for e^r, |r| <= ln2/2.  Only IEEE-exact operations (mul, rint,
// fma, ldexp) so the result is reproducible bit for bit on the host.
__device__ __forceinline__ float exp_neg(float d) {
    if (!(d >= -26.0f)) return 0.0f;
    const float kLog2e = 1.44269502162933349609375f;
    const float kLn2Hi = 0.693145751953125f;
    const float kLn2Lo = 1.428606765330187045e-06f;
    float n = __builtin_rintf(d * kLog2e);
    float r = __builtin_fmaf(n, -kLn2Hi, d);
    r = __builtin_fmaf(n, -kLn2Lo, r);
    float p = 1.98412698412698412698e-04f;
    p = __builtin_fmaf(p, r, 1.38888888888888888889e-03f);
    p = __builtin_fmaf(p, r, 8.33333333333333333333e-03f);
    p = __builtin_fmaf(p, r, 4.16666666666666666667e-02f);
    p = __builtin_fmaf(p, r, 1.66666666666666666667e-01f);
    p = __builtin_fmaf(p, r, 0.5f);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    return __builtin_ldexpf(p, (int)n);
}

__device__ __forceinline__ uint64_t weight(float x, float xmax) {
    if (x == xmax) return LLIMA_W_ONE;
    float d = x - xmax;
    if (!(d >= -26.0f)) return 0;
    float e = exp_neg(d);
    return (uint64_t)__builtin_rintf(__builtin_ldexpf(e, 36));
}

// rint(v * 2^32) clamped to [0, 2^32].
__device__ __forceinline__ uint64_t frac32(float v) {
    double s = (double)v * 4294967296.0;
    if (!(s > 0.0)) return 0;
    if (s >= 4294967296.0) return 1ull << 32;
    return (uint64_t)__builtin_rint(s);
}

__device__ __forceinline__ uint64_t uniform32(float u) {
    if (!(u > 0.0f)) return 0;
    if (u >= 1.0f) return 0xFFFFFFFFull;
    return (uint64_t)__builtin_floor((double)u * 4294967296.0);
}

// ------------------------------------------------------------------ wave primitives
__device__ __forceinline__ uint32_t lane_id() { return __lane_id(); }

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        uint32_t w = __shfl_xor(v, o, 64);
        v = v > w ? v : w;
    }
    return v;
}

__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int o) {
    uint32_t lo = __shfl_xor((uint32_t)v, o, 64);
    uint32_t hi = __shfl_xor((uint32_t)(v >> 32), o, 64);
    return ((uint64_t)hi << 32) | lo;
}

__device__ __forceinline__ uint64_t shfl_up_u64(uint64_t v, int o) {
    uint32_t lo = __shfl_up((uint32_t)v, o, 64);
    uint32_t hi = __shfl_up((uint32_t)(v >> 32), o, 64);
    return ((uint64_t)hi << 32) | lo;
}

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        uint64_t w = shfl_xor_u64(v, o);
        v = v > w ? v : w;
    }
    return v;
}

__device__ __forceinline__ uint64_t wave_sum_u64(uint64_t v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += shfl_xor_u64(v, o);
    return v;
}

__device__ __forceinline__ uint32_t wave_sum_u32(uint32_t v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// Inclusive prefix sum across the 64 lanes.
__device__ __forceinline__ uint64_t wave_incl_scan_u64(uint64_t v) {
    const uint32_t l = lane_id();
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        uint64_t w = shfl_up_u64(v, o);
        if (l >= (uint32_t)o) v += w;
    }
    return v;
}

__device__ __forceinline__ uint32_t wave_incl_scan_u32(uint32_t v) {
    const uint32_t l = lane_id();
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        uint32_t w = __shfl_up(v, o, 64);
        if (l >= (uint32_t)o) v += w;
    }
    return v;
}

// Descending bitonic sort of one uint32 per lane across a wavefront; returns
// this lane's element of the sorted sequence (lane 0 holds the largest).
__device__ __forceinline__ uint32_t wave_sort_desc(uint32_t v) {
    const uint32_t l = lane_id();
#pragma unroll
    for (int size = 2; size <= 64; size <<= 1) {
#pragma unroll
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            uint32_t w = __shfl_xor(v, stride, 64);
            bool desc = (l & size) == 0;          // direction of this bitonic block
            bool lower = (l & stride) == 0;       // this lane keeps the max if desc
            bool take_max = (lower == desc);
            uint32_t mx = v > w ? v : w, mn = v > w ? w : v;
            v = take_max ? mx : mn;
        }
    }
    return v;
}

// ------------------------------------------------------------------ block primitives
// All block helpers must be called by every thread of the workgroup.
struct BlockScratch {
    uint64_t w64[LLIMA_WAVES];
    uint32_t w32[LLIMA_WAVES];
    uint64_t bcast64;
    uint32_t bcast32;
};

__device__ __forceinline__ uint64_t block_sum_u64(uint64_t v, BlockScratch& s) {
    v = wave_sum_u64(v);
    const uint32_t w = threadIdx.x >> 6;
    if (lane_id() == 0) s.w64[w] = v;
    __syncthreads();
    uint64_t t = 0;
#pragma unroll
    for (int i = 0; i < LLIMA_WAVES; ++i) t += s.w64[i];
    __syncthreads();
    return t;
}

__device__ __forceinline__ uint32_t block_sum_u32(uint32_t v, BlockScratch& s) {
    v = wave_sum_u32(v);
    const uint32_t w = threadIdx.x >> 6;
    if (lane_id() == 0) s.w32[w] = v;
    __syncthreads();
    uint32_t t = 0;
#pragma unroll
    for (int i = 0; i < LLIMA_WAVES; ++i) t += s.w32[i];
    __syncthreads();
    return t;
}

__device__ __forceinline__ uint32_t block_max_u32(uint32_t v, BlockScratch& s) {
    v = wave_max_u32(v);
    const uint32_t w = threadIdx.x >> 6;
    if (lane_id() == 0) s.w32[w] = v;
    __syncthreads();
    uint32_t t = 0;
#pragma unroll
    for (int i = 0; i < LLIMA_WAVES; ++i) t = t > s.w32[i] ? t : s.w32[i];
    __syncthreads();
    return t;
}

__device__ __forceinline__ uint64_t block_max_u64(uint64_t v, BlockScratch& s) {
    v = wave_max_u64(v);
    const uint32_t w = threadIdx.x >> 6;
    if (lane_id() == 0) s.w64[w] = v;
    __syncthreads();
    uint64_t t = 0;
#pragma unroll
    for (int i = 0; i < LLIMA_WAVES; ++i) t = t > s.w64[i] ? t : s.w64[i];
    __syncthreads();
    return t;
}

// Exclusive prefix sum over the workgroup in thread order; also returns the total.
__device__ __forceinline__ uint64_t block_excl_scan_u64(uint64_t v, uint64_t* total,
                                                         BlockScratch& s) {
    uint64_t inc = wave_incl_scan_u64(v);
    const uint32_t w = threadIdx.x >> 6;
    if (lane_id() == 63) s.w64[w] = inc;
    __syncthreads();
    uint64_t before = 0, t = 0;
#pragma unroll
    for (int i = 0; i < LLIMA_WAVES; ++i) {
        if ((uint32_t)i < w) before += s.w64[i];
        t += s.w64[i];
    }
    __syncthreads();
    *total = t;
    return before + inc - v;
}

__device__ __forceinline__ uint32_t block_excl_scan_u32(uint32_t v, uint32_t* total,
                                                         BlockScratch& s) {
    uint32_t inc = wave_incl_scan_u32(v);
    const uint32_t w = threadIdx.x >> 6;
    if (lane_id() == 63) s.w32[w] = inc;
    __syncthreads();
    uint32_t before = 0, t = 0;
#pragma unroll
    for (int i = 0; i < LLIMA_WAVES; ++i) {
        if ((uint32_t)i < w) before += s.w32[i];
        t += s.w32[i];
    }
    __syncthreads();
    *total = t;
    return before + inc - v;
}

// blockIdx -> (row, chunk).  With B a multiple of 8 every chunk of a row is
// placed on the same XCD (workgroups are dispatched round-robin over the 8
// XCDs), so a row's history, candidates and completion counter stay in one L2.
__device__ __forceinline__ void map_row_chunk(uint32_t w, uint32_t B, uint32_t S,
                                              uint32_t* row, uint32_t* chunk) {
    if ((B & 7u) == 0) {
        uint32_t xcd = w & 7u, j = w >> 3;
        *row = (j / S) * 8u + xcd;
        *chunk = j % S;
    } else {
        *row = w / S;
        *chunk = w % S;
    }
}

}  // namespace llima
