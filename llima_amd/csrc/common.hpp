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
// s_waitcnt operand (gfx9 encoding) that waits for every vector memory
// operation of the wave, stores included: vmcnt 0, expcnt 7, lgkmcnt 15.
#define LLIMA_WAITCNT_VM0 0x0F70
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
// Written with selects only (no early return): the finish kernels run it on
// one wave per SIMD, where a branch costs more than the arithmetic it skips.
__device__ __forceinline__ float exp_neg(float d0) {
    const bool in = d0 >= -26.0f;                       // false for NaN
    const float d = in ? d0 : -26.0f;
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
    return in ? __builtin_ldexpf(p, (int)n) : 0.0f;
}

// An integral float in [0, 2^40) as uint64 (exact; by its bits).
__device__ __forceinline__ uint64_t f32_integral_to_u64(float f) {
    const uint32_t u = __float_as_uint(f);
    const int ex = (int)(u >> 23) - 150;                // f = m * 2^ex, m the significand
    const uint64_t m = (uint64_t)((u & 0x7FFFFFu) | 0x800000u);
    const uint64_t r = ex >= 0 ? m << ex : m >> (-ex < 63 ? -ex : 63);
    return u ? r : 0ull;
}

// weight(x, xmax) for a finite xmax, as the integral float it converts
// (W < 2^37, exact in fp32; sums of at most 2^16 of them are exact in double).
// exp_neg's steps with three folds that leave every result unchanged:
//   * d is clamped at -26 (NaN included) with no select after, since
//     rint(e^-26 2^36) = rint(0.35) = 0;
//   * the factor 2^36 is in the polynomial's coefficients: scaling every
//     coefficient by a power of two scales every rounded step by it (the
//     smallest, 2^36/5040, is far from the subnormals), and p 2^36 2^n with
//     n >= -38 stays normal, so ldexp(p 2^36, n) = ldexp(ldexp(p, n), 36);
//   * x == xmax needs no select: d = 0 gives n = 0, r = 0 and p = 2^36 exactly.
#define LLIMA_TWO36 68719476736.0f
__device__ __forceinline__ float weight_fd(float d0) {   // d0 = x - xmax
    const float d = __builtin_fmaxf(d0, -26.0f);         // fmaxf(NaN, -26) = -26
    const float kLog2e = 1.44269502162933349609375f;
    const float kLn2Hi = 0.693145751953125f;
    const float kLn2Lo = 1.428606765330187045e-06f;
    const float n = __builtin_rintf(d * kLog2e);
    float r = __builtin_fmaf(n, -kLn2Hi, d);
    r = __builtin_fmaf(n, -kLn2Lo, r);
    float p = 1.98412698412698412698e-04f * LLIMA_TWO36;
    p = __builtin_fmaf(p, r, 1.38888888888888888889e-03f * LLIMA_TWO36);
    p = __builtin_fmaf(p, r, 8.33333333333333333333e-03f * LLIMA_TWO36);
    p = __builtin_fmaf(p, r, 4.16666666666666666667e-02f * LLIMA_TWO36);
    p = __builtin_fmaf(p, r, 1.66666666666666666667e-01f * LLIMA_TWO36);
    p = __builtin_fmaf(p, r, 0.5f * LLIMA_TWO36);
    p = __builtin_fmaf(p, r, LLIMA_TWO36);
    p = __builtin_fmaf(p, r, LLIMA_TWO36);
    return __builtin_rintf(__builtin_ldexpf(p, (int)n));
}
__device__ __forceinline__ float weight_f(float x, float xmax) { return weight_fd(x - xmax); }

// An integral float below 2^52 as uint64 without branches: the part from 2^32
// up and the rest are each exact (a float's significand has 24 bits).
__device__ __forceinline__ uint64_t wf_u64(float wf) {
    const float hi = __builtin_truncf(wf * 2.3283064365386963e-10f);
    const uint32_t lo = (uint32_t)__builtin_fmaf(hi, -4294967296.0f, wf);
    return ((uint64_t)(uint32_t)hi << 32) | lo;
}

// The weight W = rint(exp(x - xmax) 2^36) of x <= xmax (LLIMA_W_ONE at x ==
// xmax, also when both are +inf; 0 below xmax - 26 and for NaN): exp_neg's
// value through weight_fd's folds, converted without branches.
__device__ __forceinline__ uint64_t weight(float x, float xmax) {
    return wf_u64(weight_fd(x == xmax ? 0.0f : x - xmax));
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
// Cross-lane steps use DPP (row shifts, mirrors and the GFX9 row broadcasts),
// which move data between lanes inside the VALU with no LDS round trip.
__device__ __forceinline__ uint32_t lane_id() { return __lane_id(); }

// Wave index as a uniform (scalar) value.
__device__ __forceinline__ uint32_t wave_id() {
    return (uint32_t)__builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
}

__device__ __forceinline__ uint64_t ballot(bool p) { return __builtin_amdgcn_ballot_w64(p); }

// Number of set bits of m below this lane.
__device__ __forceinline__ uint32_t mbcnt(uint64_t m) {
    return __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32),
                                     __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

__device__ __forceinline__ uint32_t readlane(uint32_t v, uint32_t l) {
    return (uint32_t)__builtin_amdgcn_readlane((int)v, (int)l);
}
__device__ __forceinline__ uint64_t readlane64(uint64_t v, uint32_t l) {
    return ((uint64_t)readlane((uint32_t)(v >> 32), l) << 32) | readlane((uint32_t)v, l);
}

#define DPP_QUAD_XOR1 0xB1     // quad_perm [1,0,3,2]
#define DPP_QUAD_XOR2 0x4E     // quad_perm [2,3,0,1]
#define DPP_ROW_SHR(n) (0x110 + (n))
#define DPP_ROW_MIRROR 0x140
#define DPP_ROW_HALF_MIRROR 0x141
#define DPP_ROW_BCAST15 0x142  // lane 15 of each row -> the next row
#define DPP_ROW_BCAST31 0x143  // lane 31 -> rows 2 and 3

// DPP move: lanes of rows outside ROW_MASK (and, with BC, lanes whose source
// is outside the row) receive old.
template <int CTRL, int ROW_MASK, bool BC>
__device__ __forceinline__ uint32_t dpp32(uint32_t old, uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp((int)old, (int)v, CTRL, ROW_MASK, 0xF, BC);
}
template <int CTRL, int ROW_MASK, bool BC>
__device__ __forceinline__ uint64_t dpp64(uint64_t old, uint64_t v) {
    const uint32_t lo = dpp32<CTRL, ROW_MASK, BC>((uint32_t)old, (uint32_t)v);
    const uint32_t hi = dpp32<CTRL, ROW_MASK, BC>((uint32_t)(old >> 32), (uint32_t)(v >> 32));
    return ((uint64_t)hi << 32) | lo;
}
template <int CTRL, int ROW_MASK, bool BC>
__device__ __forceinline__ uint32_t dppT(uint32_t old, uint32_t v) { return dpp32<CTRL, ROW_MASK, BC>(old, v); }
template <int CTRL, int ROW_MASK, bool BC>
__device__ __forceinline__ uint64_t dppT(uint64_t old, uint64_t v) { return dpp64<CTRL, ROW_MASK, BC>(old, v); }

__device__ __forceinline__ uint32_t readlane63(uint32_t v) { return readlane(v, 63); }
__device__ __forceinline__ uint64_t readlane63(uint64_t v) { return readlane64(v, 63); }

// Reduction over the 64 lanes (op associative and commutative, identity its
// neutral element); the result is uniform.
template <typename T, class Op>
__device__ __forceinline__ T wave_reduce(T v, T identity, Op op) {
    v = op(v, dppT<DPP_QUAD_XOR1, 0xF, false>(identity, v));
    v = op(v, dppT<DPP_QUAD_XOR2, 0xF, false>(identity, v));
    v = op(v, dppT<DPP_ROW_HALF_MIRROR, 0xF, false>(identity, v));
    v = op(v, dppT<DPP_ROW_MIRROR, 0xF, false>(identity, v));
    v = op(v, dppT<DPP_ROW_BCAST15, 0xA, false>(identity, v));
    v = op(v, dppT<DPP_ROW_BCAST31, 0xC, false>(identity, v));
    return readlane63(v);
}

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
    return wave_reduce<uint32_t>(v, 0u, [](uint32_t a, uint32_t b) { return a > b ? a : b; });
}
__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v) {
    return wave_reduce<uint32_t>(v, 0xFFFFFFFFu, [](uint32_t a, uint32_t b) { return a < b ? a : b; });
}
__device__ __forceinline__ uint32_t wave_sum_u32(uint32_t v) {
    return wave_reduce<uint32_t>(v, 0u, [](uint32_t a, uint32_t b) { return a + b; });
}
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
    return wave_reduce<uint64_t>(v, 0ull, [](uint64_t a, uint64_t b) { return a > b ? a : b; });
}
__device__ __forceinline__ uint64_t wave_sum_u64(uint64_t v) {
    return wave_reduce<uint64_t>(v, 0ull, [](uint64_t a, uint64_t b) { return a + b; });
}

// Inclusive prefix sums across the 64 lanes (Hillis-Steele inside each row of
// 16 lanes, then the two row broadcasts).
__device__ __forceinline__ uint32_t wave_incl_scan_u32(uint32_t v) {
    v += dpp32<DPP_ROW_SHR(1), 0xF, true>(0u, v);
    v += dpp32<DPP_ROW_SHR(2), 0xF, true>(0u, v);
    v += dpp32<DPP_ROW_SHR(4), 0xF, true>(0u, v);
    v += dpp32<DPP_ROW_SHR(8), 0xF, true>(0u, v);
    v += dpp32<DPP_ROW_BCAST15, 0xA, false>(0u, v);
    v += dpp32<DPP_ROW_BCAST31, 0xC, false>(0u, v);
    return v;
}
__device__ __forceinline__ uint64_t wave_incl_scan_u64(uint64_t v) {
    v += dpp64<DPP_ROW_SHR(1), 0xF, true>(0ull, v);
    v += dpp64<DPP_ROW_SHR(2), 0xF, true>(0ull, v);
    v += dpp64<DPP_ROW_SHR(4), 0xF, true>(0ull, v);
    v += dpp64<DPP_ROW_SHR(8), 0xF, true>(0ull, v);
    v += dpp64<DPP_ROW_BCAST15, 0xA, false>(0ull, v);
    v += dpp64<DPP_ROW_BCAST31, 0xC, false>(0ull, v);
    return v;
}

// The r-th largest (1-based, r <= 64) of one key per lane, with its bits below
// lowbit cleared (so a value <= the exact one); keys of 0 never count, and the
// result is 0 when fewer than r lanes hold a key.  One ballot per bit.
__device__ __forceinline__ uint32_t wave_rth_largest(uint32_t key, uint32_t r, int lowbit) {
    uint32_t t = 0;
    for (int b = 31; b >= lowbit; --b) {
        const uint32_t cand = t | (1u << b);
        if ((uint32_t)__popcll(ballot(key >= cand)) >= r) t = cand;
    }
    return t;
}

// The same value as wave_rth_largest(key, r, lowbit) for lowbit <= 23, with
// fewer serial steps in the common case: the key's top 9 bits (sign and
// exponent of the float) are taken from the wave maximum's bucket or the one
// below it (two independent ballots), leaving the mantissa bits 22..lowbit.
// Anything else takes the full search.
__device__ __forceinline__ uint32_t wave_rth_largest_exp(uint32_t key, uint32_t r, int lowbit) {
    const uint32_t e1 = wave_max_u32(key) & 0xFF800000u;
    if (e1 >= 0x00800000u) {
        const uint32_t e0 = e1 - 0x00800000u;
        const uint32_t n1 = (uint32_t)__popcll(ballot(key >= e1));
        const uint32_t n0 = (uint32_t)__popcll(ballot(key >= e0));
        if (n0 >= r) {
            uint32_t t = n1 >= r ? e1 : e0;
#pragma unroll
            for (int b = 22; b >= lowbit; --b) {
                const uint32_t cand = t | (1u << b);
                if ((uint32_t)__popcll(ballot(key >= cand)) >= r) t = cand;
            }
            return t;
        }
    }
    return wave_rth_largest(key, r, lowbit);
}

// ------------------------------------------------------------------ cross-workgroup sums
// Values that other workgroups read inside the same launch: relaxed agent-scope
// atomic stores (write-through) and loads (they miss stale cache lines).  The
// writer waits for its stores (LLIMA_WAITCNT_VM0) before it counts its arrival
// on an agent-scope counter, so the last workgroup to arrive sees every value
// with no cache writeback or invalidation.
__device__ __forceinline__ void store_agent(uint64_t* p, uint64_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t load_agent(uint64_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t arrive_agent(uint32_t* counter, uint32_t n) {
    return __hip_atomic_fetch_add(counter, n, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ------------------------------------------------------------------ block primitives
// All block helpers must be called by every thread of the workgroup.
struct BlockScratch {
    uint64_t w64[LLIMA_WAVES];
    uint32_t w32[LLIMA_WAVES];
    uint64_t bcast64;
    uint32_t bcast32;
};

__device__ __forceinline__ double wave_sum_f64(double v) {
    return __longlong_as_double((long long)wave_reduce<uint64_t>(
        (uint64_t)__double_as_longlong(v), 0ull, [](uint64_t a, uint64_t b) {
            return (uint64_t)__double_as_longlong(__longlong_as_double((long long)a) +
                                                  __longlong_as_double((long long)b));
        }));
}

// Sum over the workgroup in double (the waves' sums added in wave order).
__device__ __forceinline__ double block_sum_f64(double v, BlockScratch& s) {
    v = wave_sum_f64(v);
    const uint32_t w = threadIdx.x >> 6;
    if (lane_id() == 0) s.w64[w] = (uint64_t)__double_as_longlong(v);
    __syncthreads();
    double t = 0.0;
#pragma unroll
    for (int i = 0; i < LLIMA_WAVES; ++i) t += __longlong_as_double((long long)s.w64[i]);
    __syncthreads();
    return t;
}

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

// Finish kernels with one wavefront per row: (workgroup, wave) -> row, and the
// workgroup count.  With B a multiple of 8 the sweep put row r's chunks on XCD
// r % 8 (map_row_chunk); workgroup w runs on XCD w % 8 and takes rows of that
// XCD, so the chunk results it reads are in its own L2.  Rows past B: -1.
__device__ __forceinline__ int finish_row(uint32_t blk, uint32_t wave, uint32_t B) {
    uint32_t r;
    if ((B & 7u) == 0) r = (blk & 7u) + 8u * ((blk >> 3) * LLIMA_WAVES + wave);
    else r = blk * LLIMA_WAVES + wave;
    return r < B ? (int)r : -1;
}
inline uint32_t finish_row_blocks(uint32_t B) {
    return (B & 7u) == 0 ? 8u * ((B + 8u * LLIMA_WAVES - 1u) / (8u * LLIMA_WAVES))
                         : (B + LLIMA_WAVES - 1u) / LLIMA_WAVES;
}

}  // namespace llima
