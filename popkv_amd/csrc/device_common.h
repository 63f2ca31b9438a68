// Shared device helpers for the gfx950 PopKV kernels (wave64, CDNA4).
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#include "popkv_hip.h"

namespace popkv {

constexpr int kWave = 64;

// ---- element loads -------------------------------------------------------

struct bf16_t { uint16_t bits; };
struct f16_t { uint16_t bits; };

__device__ __forceinline__ float bits_bf16(uint32_t b) { return __uint_as_float(b << 16); }
__device__ __forceinline__ float bits_f16(uint32_t b) {
    return __half2float(__ushort_as_half(static_cast<unsigned short>(b)));
}
// fp16 round-to-nearest-even of an already-rounded float32 value
// (v_cvt_f16_f32 under the default round mode).  The empty asm pins `x` as a
// materialized float32: without it the backend fuses a producing multiply
// and this conversion into one v_fma_mixlo_f16, which rounds the exact
// product once to fp16 instead of rounding to fp32 first, and differs in the
// last fp16 bit whenever the fp32 product lands on an fp16 tie.
__device__ __forceinline__ uint16_t f16_rne(float x) {
    asm volatile("" : "+v"(x));
    return __half_as_ushort(__float2half_rn(x));
}
// bf16 round-to-nearest-even; NaN kept quiet.
__device__ __forceinline__ uint16_t bf16_rne(float x) {
    uint32_t u = __float_as_uint(x);
    if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return static_cast<uint16_t>(u >> 16);
}

template <typename T> struct Elem;
template <> struct Elem<float> {
    static constexpr int kDtype = POPKV_DTYPE_F32;
    __device__ static __forceinline__ float load(const float* p, int64_t i) { return p[i]; }
    __device__ static __forceinline__ void store(float* p, int64_t i, float v) { p[i] = v; }
};
template <> struct Elem<bf16_t> {
    static constexpr int kDtype = POPKV_DTYPE_BF16;
    __device__ static __forceinline__ float load(const bf16_t* p, int64_t i) { return bits_bf16(p[i].bits); }
    __device__ static __forceinline__ void store(bf16_t* p, int64_t i, float v) { p[i].bits = bf16_rne(v); }
};
template <> struct Elem<f16_t> {
    static constexpr int kDtype = POPKV_DTYPE_F16;
    __device__ static __forceinline__ float load(const f16_t* p, int64_t i) { return bits_f16(p[i].bits); }
    __device__ static __forceinline__ void store(f16_t* p, int64_t i, float v) { p[i].bits = f16_rne(v); }
};

// Eight consecutive elements starting at a 16-byte aligned address -> float.
template <typename T> __device__ __forceinline__ void load8(const T* p, float v[8]);
template <> __device__ __forceinline__ void load8<bf16_t>(const bf16_t* p, float v[8]) {
    uint4 u = *reinterpret_cast<const uint4*>(p);
    v[0] = __uint_as_float(u.x << 16); v[1] = __uint_as_float(u.x & 0xffff0000u);
    v[2] = __uint_as_float(u.y << 16); v[3] = __uint_as_float(u.y & 0xffff0000u);
    v[4] = __uint_as_float(u.z << 16); v[5] = __uint_as_float(u.z & 0xffff0000u);
    v[6] = __uint_as_float(u.w << 16); v[7] = __uint_as_float(u.w & 0xffff0000u);
}
template <> __device__ __forceinline__ void load8<f16_t>(const f16_t* p, float v[8]) {
    uint4 u = *reinterpret_cast<const uint4*>(p);
    v[0] = bits_f16(u.x & 0xffffu); v[1] = bits_f16(u.x >> 16);
    v[2] = bits_f16(u.y & 0xffffu); v[3] = bits_f16(u.y >> 16);
    v[4] = bits_f16(u.z & 0xffffu); v[5] = bits_f16(u.z >> 16);
    v[6] = bits_f16(u.w & 0xffffu); v[7] = bits_f16(u.w >> 16);
}
template <> __device__ __forceinline__ void load8<float>(const float* p, float v[8]) {
    float4 a = reinterpret_cast<const float4*>(p)[0];
    float4 b = reinterpret_cast<const float4*>(p)[1];
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}

// ---- representative reduction trees ---------------------------------------
// The production packers reduce one representative group's 32 (or 16) lane
// contributions with a halving tree: a_i = z_i + z_{i+16}, then +8, +4, +2, +1.
// G64 first pairs dims j and j+32.  All terms are >= +0, so adding +0 from an
// absent lane is exact and the same trees cover partial groups.

__device__ __forceinline__ float tree_halving(float* z, int n) {
#pragma unroll
    for (int h = n / 2; h >= 1; h /= 2) {
#pragma unroll
        for (int i = 0; i < 16; ++i)
            if (i < h) z[i] = z[i] + z[i + h];
    }
    return z[0];
}

// Sum of G contributions x[0..G) in the production tree order (destroys x).
template <int G>
__device__ __forceinline__ float rep_tree_sum(float* x) {
    if constexpr (G == 64) {
#pragma unroll
        for (int j = 0; j < 32; ++j) x[j] = x[j] + x[j + 32];
        return tree_halving(x, 32);
    } else {
        return tree_halving(x, G);
    }
}

// low/delta with the empty-bucket rules of the reference packers.
__device__ __forceinline__ void finish_rep(float ls, int ln, float hs, int hn, float& low, float& delta) {
    float lo, hi;
    if (ln == 0) {
        lo = hn ? hs / static_cast<float>(hn) : 0.0f;
        hi = lo;
    } else {
        lo = ls / static_cast<float>(ln);
        hi = hn ? hs / static_cast<float>(hn) : lo;
    }
    low = lo;
    delta = hi - lo;
}

// Radix order key of an fp16 bit pattern, the map PyTorch's radix top-k
// uses for half values: negatives bit-inverted, non-negatives with the sign
// bit set, every NaN mapped to the largest key.  Monotone, and -0 < +0.
__device__ __forceinline__ uint32_t order_key(uint32_t h) {
    const bool nan = ((h & 0x7c00u) == 0x7c00u) && (h & 0x3ffu);
    const uint32_t k = (h & 0x8000u) ? (~h & 0xffffu) : (h | 0x8000u);
    return nan ? 0xffffu : k;
}

// Makes the given kernel arguments live in scalar registers at this point,
// so that the compiler loads them in one batch -- one scalar-cache round
// trip -- before it; left to itself it loads a few, waits, computes with
// them and loads the rest in a second batch, all before a kernel's first
// memory loads can be issued.
template <typename A>
__device__ __forceinline__ void arg_in_sgprs(const A& a) {
    asm volatile("" : : "s"(a));
}
template <typename... A>
__device__ __forceinline__ void args_in_sgprs(const A&... a) {
    (arg_in_sgprs(a), ...);
}

// n / d for n >= 0, d > 0 (uniform values): a shift when d is a power of two
// -- the usual head, group and chunk counts -- instead of the integer
// division sequence (a float reciprocal and about twenty scalar steps).
__device__ __forceinline__ int div_nonneg(int n, int d) {
    if ((d & (d - 1)) == 0) return n >> __builtin_ctz(static_cast<unsigned>(d));
    return n / d;
}

// Raw storage of 8 consecutive elements: one 16-byte packet for 16-bit types,
// two for float32.  Rows stay packed in registers until they are consumed.
template <typename T> struct Raw8 {
    uint4 u;
    __device__ __forceinline__ void load(const T* p) { u = *reinterpret_cast<const uint4*>(p); }
    __device__ __forceinline__ void zero() { u = make_uint4(0u, 0u, 0u, 0u); }
    __device__ __forceinline__ float get(int i) const {
        const uint32_t w = i < 2 ? u.x : i < 4 ? u.y : i < 6 ? u.z : u.w;
        const uint32_t h = (i & 1) ? (w >> 16) : (w & 0xffffu);
        return Elem<T>::kDtype == POPKV_DTYPE_BF16 ? bits_bf16(h) : bits_f16(h);
    }
};
template <> struct Raw8<float> {
    float4 a, b;
    __device__ __forceinline__ void load(const float* p) {
        a = reinterpret_cast<const float4*>(p)[0];
        b = reinterpret_cast<const float4*>(p)[1];
    }
    __device__ __forceinline__ void zero() { a = make_float4(0.f, 0.f, 0.f, 0.f); b = a; }
    __device__ __forceinline__ float get(int i) const {
        const float4& x = i < 4 ? a : b;
        const int j = i & 3;
        return j == 0 ? x.x : j == 1 ? x.y : j == 2 ? x.z : x.w;
    }
};

// ---- wave / block reductions --------------------------------------------

// Wave-wide max / min / sum, the result in every lane.  max and min are
// exact in any order; the sum is a fixed tree (DPP within rows, then the four
// row totals), so it is deterministic but not a left-to-right fold.
__device__ __forceinline__ float wave_max(float v);
__device__ __forceinline__ float wave_min(float v);
__device__ __forceinline__ float wave_sum(float v);

// Sum over each row of 16 lanes (or 8-lane half rows for N = 8) with DPP
// lane permutations -- VALU-only, no LDS traffic.  Every lane of a row ends
// with the row's sum.  Control words: quad_perm [1,0,3,2] = 0xB1,
// quad_perm [2,3,0,1] = 0x4E, row_half_mirror = 0x141, row_mirror = 0x140.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
    // bound_ctrl set: every control used here reads a lane inside the same
    // row, so it changes nothing and lets the move fold into the consumer.
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xf, 0xf, true));
}
template <int N>
__device__ __forceinline__ float row_sum(float v) {
    static_assert(N == 8 || N == 16, "DPP row sums cover 8 or 16 lanes");
    v += dpp_mov<0xB1>(v);
    v += dpp_mov<0x4E>(v);
    v += dpp_mov<0x141>(v);
    if constexpr (N == 16) v += dpp_mov<0x140>(v);
    return v;
}

// Wave-wide max / min: DPP within each 16-lane row, then the four row
// results combined through readlane (the result is wave-uniform).  Exact:
// max / min do not depend on the combination order.
template <bool MAX>
__device__ __forceinline__ float wave_extreme(float v) {
    auto f = [](float a, float b) { return MAX ? fmaxf(a, b) : fminf(a, b); };
    v = f(v, dpp_mov<0xB1>(v));
    v = f(v, dpp_mov<0x4E>(v));
    v = f(v, dpp_mov<0x141>(v));
    v = f(v, dpp_mov<0x140>(v));
    const uint32_t u = __builtin_bit_cast(uint32_t, v);
    const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(u, 0));
    const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(u, 16));
    const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(u, 32));
    const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(u, 48));
    return f(f(r0, r1), f(r2, r3));
}

__device__ __forceinline__ float wave_max(float v) { return wave_extreme<true>(v); }
__device__ __forceinline__ float wave_min(float v) { return wave_extreme<false>(v); }
__device__ __forceinline__ float wave_sum(float v) {
    v += dpp_mov<0xB1>(v);
    v += dpp_mov<0x4E>(v);
    v += dpp_mov<0x141>(v);
    v += dpp_mov<0x140>(v);
    const uint32_t u = __builtin_bit_cast(uint32_t, v);
    const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(u, 0));
    const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(u, 16));
    const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(u, 32));
    const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(u, 48));
    return (r0 + r1) + (r2 + r3);
}

// Value of lane l^16 / l^32 (all 64 lanes active), with gfx950's
// v_permlane16_swap / v_permlane32_swap instead of an LDS permute.  With both
// operands equal to x, permlane32_swap returns (x[l & 31], x[(l & 31) + 32])
// and permlane16_swap returns (x[l & ~16], x[l | 16]) in every lane.
__device__ __forceinline__ float lane_xor16(float v) {
    const uint32_t u = __builtin_bit_cast(uint32_t, v);
    const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    return __builtin_bit_cast(float, (threadIdx.x & 16) ? r[0] : r[1]);
}
__device__ __forceinline__ float lane_xor32(float v) {
    const uint32_t u = __builtin_bit_cast(uint32_t, v);
    const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    return __builtin_bit_cast(float, (threadIdx.x & 32) ? r[0] : r[1]);
}
template <int M>
__device__ __forceinline__ float lane_xor(float v) {
    if constexpr (M == 16) return lane_xor16(v);
    else if constexpr (M == 32) return lane_xor32(v);
    else return __shfl_xor(v, M);
}

// Inclusive prefix sum across the wave with DPP (VALU only): row_shr 1, 2,
// 4, 8 scan each 16-lane row (lanes without a source add 0), then
// row_bcast:15 adds lane 15's total to rows 1 and 3 and row_bcast:31 adds
// lane 31's total to rows 2 and 3.  All 64 lanes must be active.
template <int CTRL, int ROW_MASK, bool BOUND_ZERO>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
    return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), CTRL, ROW_MASK, 0xf, BOUND_ZERO));
}
__device__ __forceinline__ uint32_t wave_incl_scan(uint32_t v, int /*lane*/) {
    v += dpp_u32<0x111, 0xf, true>(v);
    v += dpp_u32<0x112, 0xf, true>(v);
    v += dpp_u32<0x114, 0xf, true>(v);
    v += dpp_u32<0x118, 0xf, true>(v);
    v += dpp_u32<0x142, 0xa, false>(v);
    v += dpp_u32<0x143, 0xc, false>(v);
    return v;
}

// 16 bytes stored / loaded as two relaxed agent-scope 64-bit atomics: on
// gfx942 / gfx950 global stores / loads with the sc1 bit, which write
// through and read past the XCD's non-coherent L2, so data one workgroup
// hands to another inside a kernel needs no L2 write-back or invalidate
// (the hand-off's ordering rule is stated where it is used).
__device__ __forceinline__ void st_coh_u4(uint4* p, uint4 v) {
    uint64_t* q = reinterpret_cast<uint64_t*>(p);
    __hip_atomic_store(q, static_cast<uint64_t>(v.x) | (static_cast<uint64_t>(v.y) << 32), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(q + 1, static_cast<uint64_t>(v.z) | (static_cast<uint64_t>(v.w) << 32), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint4 ld_coh_u4(const uint4* p) {
    uint64_t* q = reinterpret_cast<uint64_t*>(const_cast<uint4*>(p));
    const uint64_t a = __hip_atomic_load(q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const uint64_t b = __hip_atomic_load(q + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return make_uint4(static_cast<uint32_t>(a), static_cast<uint32_t>(a >> 32), static_cast<uint32_t>(b),
                      static_cast<uint32_t>(b >> 32));
}
template <bool COH>
__device__ __forceinline__ uint4 ld_u4(const uint4* p) {
    if constexpr (COH) return ld_coh_u4(p);
    else return *p;
}
template <bool COH>
__device__ __forceinline__ uint2 ld_u2(const uint2* p) {
    if constexpr (COH) {
        const uint64_t a = __hip_atomic_load(reinterpret_cast<uint64_t*>(const_cast<uint2*>(p)), __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT);
        return make_uint2(static_cast<uint32_t>(a), static_cast<uint32_t>(a >> 32));
    } else {
        return *p;
    }
}

// Exclusive prefix sum across a block of `waves` wave64s with a single
// barrier: DPP scan inside each wave, wave totals through `sh` (`waves`
// words).  For one use of `sh` per kernel (nothing may still be reading it).
// Every thread of the block must call it.
__device__ __forceinline__ uint32_t block_excl_scan_once(uint32_t v, uint32_t* sh, int waves, uint32_t* total) {
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const uint32_t incl = wave_incl_scan(v, lane);
    if (lane == kWave - 1) sh[wave] = incl;
    __syncthreads();
    uint32_t base = 0, tot = 0;
    for (int w = 0; w < waves; ++w) {
        const uint32_t x = sh[w];
        base += w < wave ? x : 0u;
        tot += x;
    }
    *total = tot;
    return base + incl - v;
}

}  // namespace popkv
