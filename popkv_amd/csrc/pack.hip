// Key prepack and per-token append of PopKV retrieval metadata (gfx950).
//
// head_dim 128 (pack128_kernel, the encode itself pack128_group in
// pack128.h): one workgroup per (KV head, token group), one wave per chunk
// of max(G, 32) dimensions (2 or 4 waves).
//   Phase 1 -- lane l owns dims 2l and 2l+1; the waves stream interleaved
//              rows of the group with coalesced 4-byte loads (256 bytes per
//              wave instruction), keeping per-dimension min/max in registers;
//              the partial extrema meet in LDS and the thresholds
//              0.5*max / 0.5*min go to LDS.
//   Phase 2 -- one token per lane, each wave on its dimension chunk: the
//              lane re-reads its slice of the row (a cache hit), forms the
//              sign/magnitude words and reduces its representatives in
//              registers in the production tree order (G64 pairs dims j and
//              j+32 first), then writes its words and fp16 representatives.
// No cross-lane shuffles are needed for the bit-exact sums: the tree lives in
// one lane's registers.  Other head sizes (pack_kernel) use 256 threads per
// group: per-dimension extrema by (dimension, token stripe), then one token
// per thread.
//
// Semantics follow the reference packers: popkv_ext.cu:79-143 (G32),
// :376-500 (fused G16/G64, head_dim 128), :283-374 (generic G16/G64), with
// output rows token_offset + t (the in-place append of :1075-1092,
// :1177-1206).
#include <type_traits>

#include "device_common.h"
#include "kernels.h"
#include "pack128.h"

namespace popkv {
namespace {

constexpr int kPackThreads = 256;

// Encodes one chunk of CH = max(G, 32) dimensions of one token.
// dims [c0, c0 + CH); `valid_d` = number of real dims in the head.
template <typename T, int G, bool FAST>
__device__ __forceinline__ void encode_chunk(const T* __restrict__ row, int c0, int d,
                                             const float* s_hi, const float* s_lo,
                                             uint32_t* sw, uint32_t* mw, float* lows, float* deltas) {
    constexpr int CH = G > 32 ? G : 32;
    float v[CH];
    if constexpr (FAST) {
#pragma unroll
        for (int i = 0; i < CH; i += 8) load8<T>(row + c0 + i, v + i);
    } else {
#pragma unroll
        for (int i = 0; i < CH; ++i) v[i] = (c0 + i < d) ? Elem<T>::load(row, c0 + i) : 0.0f;
    }
    bool mag[CH];
#pragma unroll
    for (int wi = 0; wi < CH / 32; ++wi) {
        uint32_t s = 0, m = 0;
#pragma unroll
        for (int j = 0; j < 32; ++j) {
            const int i = wi * 32 + j;
            const int dim = FAST ? c0 + i : min(c0 + i, 255);
            const bool valid = FAST || (c0 + i) < d;
            const bool sg = valid && v[i] >= 0.0f;
            const bool mg = valid && (sg ? (v[i] > s_hi[dim]) : (v[i] < s_lo[dim]));
            mag[i] = mg;
            s |= static_cast<uint32_t>(sg) << j;
            m |= static_cast<uint32_t>(mg) << j;
        }
        sw[wi] = s;
        mw[wi] = m;
    }
#pragma unroll
    for (int rr = 0; rr < CH / G; ++rr) {
        float xl[G], xh[G];
        int ln = 0, hn = 0;
#pragma unroll
        for (int j = 0; j < G; ++j) {
            const int i = rr * G + j;
            const bool valid = FAST || (c0 + i) < d;
            const float a = fabsf(v[i]);
            xl[j] = (valid && !mag[i]) ? a : 0.0f;
            xh[j] = (valid && mag[i]) ? a : 0.0f;
            ln += (valid && !mag[i]) ? 1 : 0;
            hn += (valid && mag[i]) ? 1 : 0;
        }
        const float ls = rep_tree_sum<G>(xl);
        const float hs = rep_tree_sum<G>(xh);
        finish_rep(ls, ln, hs, hn, lows[rr], deltas[rr]);
    }
}

template <typename T, int G, bool FAST>
__global__ __launch_bounds__(kPackThreads) void pack_kernel(
    const T* __restrict__ keys, int64_t head_stride, int64_t tokens, int d, int tg,
    int32_t* __restrict__ k_sign, int32_t* __restrict__ k_mag,
    uint16_t* __restrict__ k_low, uint16_t* __restrict__ k_delta,
    int64_t cap, int64_t offset) {
    const int D = FAST ? 128 : d;
    const int W = (D + 31) / 32;
    const int R = (D + G - 1) / G;
    const int64_t kvh = blockIdx.y;
    const int64_t gs = static_cast<int64_t>(blockIdx.x) * tg;
    const int64_t ge = min(gs + static_cast<int64_t>(tg), tokens);
    const T* base = keys + kvh * head_stride;

    __shared__ float s_hi[256], s_lo[256];
    __shared__ float s_mx[kPackThreads], s_mn[kPackThreads];

    // Phase 1: per-dimension extrema over the token group.
    const int tid = threadIdx.x;
    const int nstripe = kPackThreads / D;
    if (tid < nstripe * D) {
        const int dim = tid % D, stripe = tid / D;
        float mn = INFINITY, mx = -INFINITY;
        for (int64_t t = gs + stripe; t < ge; t += nstripe) {
            const float x = Elem<T>::load(base, t * D + dim);
            mn = fminf(mn, x);
            mx = fmaxf(mx, x);
        }
        s_mn[tid] = mn;
        s_mx[tid] = mx;
    }
    __syncthreads();
    if (tid < D) {
        float mn = s_mn[tid], mx = s_mx[tid];
        for (int s = 1; s < nstripe; ++s) {
            mn = fminf(mn, s_mn[s * D + tid]);
            mx = fmaxf(mx, s_mx[s * D + tid]);
        }
        s_lo[tid] = mn * 0.5f;
        s_hi[tid] = mx * 0.5f;
    }
    __syncthreads();

    // Phase 2: one token per lane.
    constexpr int CH = G > 32 ? G : 32;
    for (int64_t t = gs + tid; t < ge; t += kPackThreads) {
        const T* row = base + t * D;
        const int64_t orow = kvh * cap + offset + t;
        if constexpr (FAST) {
            uint32_t sw[4], mw[4];
            float lows[128 / G], deltas[128 / G];
#pragma unroll
            for (int c = 0; c < 128 / CH; ++c)
                encode_chunk<T, G, true>(row, c * CH, 128, s_hi, s_lo, sw + c * (CH / 32), mw + c * (CH / 32),
                                         lows + c * (CH / G), deltas + c * (CH / G));
            reinterpret_cast<uint4*>(k_sign)[orow] = make_uint4(sw[0], sw[1], sw[2], sw[3]);
            reinterpret_cast<uint4*>(k_mag)[orow] = make_uint4(mw[0], mw[1], mw[2], mw[3]);
            constexpr int RR = 128 / G;
            uint32_t lo_p[RR / 2], de_p[RR / 2];
#pragma unroll
            for (int r = 0; r < RR / 2; ++r) {
                lo_p[r] = static_cast<uint32_t>(f16_rne(lows[2 * r])) |
                          (static_cast<uint32_t>(f16_rne(lows[2 * r + 1])) << 16);
                de_p[r] = static_cast<uint32_t>(f16_rne(deltas[2 * r])) |
                          (static_cast<uint32_t>(f16_rne(deltas[2 * r + 1])) << 16);
            }
            if constexpr (RR == 2) {
                reinterpret_cast<uint32_t*>(k_low)[orow] = lo_p[0];
                reinterpret_cast<uint32_t*>(k_delta)[orow] = de_p[0];
            } else if constexpr (RR == 4) {
                reinterpret_cast<uint2*>(k_low)[orow] = make_uint2(lo_p[0], lo_p[1]);
                reinterpret_cast<uint2*>(k_delta)[orow] = make_uint2(de_p[0], de_p[1]);
            } else {
                reinterpret_cast<uint4*>(k_low)[orow] = make_uint4(lo_p[0], lo_p[1], lo_p[2], lo_p[3]);
                reinterpret_cast<uint4*>(k_delta)[orow] = make_uint4(de_p[0], de_p[1], de_p[2], de_p[3]);
            }
        } else {
            for (int c0 = 0; c0 < D; c0 += CH) {
                uint32_t sw[CH / 32], mw[CH / 32];
                float lows[CH / G], deltas[CH / G];
                encode_chunk<T, G, false>(row, c0, D, s_hi, s_lo, sw, mw, lows, deltas);
#pragma unroll
                for (int wi = 0; wi < CH / 32; ++wi) {
                    const int w = c0 / 32 + wi;
                    if (w < W) {
                        k_sign[orow * W + w] = static_cast<int32_t>(sw[wi]);
                        k_mag[orow * W + w] = static_cast<int32_t>(mw[wi]);
                    }
                }
#pragma unroll
                for (int rr = 0; rr < CH / G; ++rr) {
                    const int r = c0 / G + rr;
                    if (r < R) {
                        k_low[orow * R + r] = f16_rne(lows[rr]);
                        k_delta[orow * R + r] = f16_rne(deltas[rr]);
                    }
                }
            }
        }
    }
}

// Prefix prepack (APPEND false): block (x, y) encodes token group x of KV
// head y, rows [x*tg, min(x*tg + tg, tokens)) of `keys`, into packed rows
// y*cap + offset + x*tg + t.  Fused append (APPEND true): block i appends
// the new token of (sequence, KV head) i (pack128_append).  STAGE (16-bit
// rows; tg <= 64 at G 64, tg <= 128 at G 32 / G 16): the group's rows are
// read from memory once, into LDS, and the encode pass reads them there.
template <typename T, int G, bool APPEND, bool STAGE = false>
__global__ __launch_bounds__(kWave * pack128_waves<G>()) void pack128_kernel(
    const T* __restrict__ keys, int64_t head_stride, int64_t tokens, int tg,
    int32_t* __restrict__ k_sign, int32_t* __restrict__ k_mag,
    uint16_t* __restrict__ k_low, uint16_t* __restrict__ k_delta, int64_t cap, int64_t offset,
    AppendArgs<T> ap) {
    constexpr int D = 128;
    static_assert(2 * D * static_cast<int>(sizeof(T)) / 16 <= kWave * pack128_waves<G>(),
                  "one 16-byte slice of the new K/V rows per thread");
    if constexpr (APPEND)
        args_in_sgprs(ap.counts, ap.kv_heads, ap.cache_rows, ap.new_k, ap.new_v, ap.key_cache, ap.value_cache, tg,
                      k_sign, k_mag, k_low, k_delta, cap);
    else
        args_in_sgprs(keys, head_stride, tokens, tg, k_sign, k_mag, k_low, k_delta, cap, offset);
    if constexpr (!APPEND) {
        const int64_t kvh = blockIdx.y;
        const int64_t gs = static_cast<int64_t>(blockIdx.x) * tg;
        const int n = static_cast<int>(min(gs + static_cast<int64_t>(tg), tokens) - gs);
        const T* base = keys + kvh * head_stride + gs * D;
        auto row_of = [&](int t) -> const T* { return base + static_cast<int64_t>(t) * D; };
        pack128_group<T, G, false, STAGE>(row_of, n, kvh * cap + offset + gs, k_sign, k_mag, k_low, k_delta);
    } else {
        pack128_append<T, G, false, STAGE>(blockIdx.x, ap, tg, k_sign, k_mag, k_low, k_delta, cap);
    }
}

template <typename T, int G>
hipError_t launch_pack_t(const T* keys, int64_t kvh, int64_t tokens, int d, int64_t head_stride,
                         int32_t* ks, int32_t* km, uint16_t* kl, uint16_t* kd, int64_t cap, int64_t off,
                         int tg, hipStream_t stream) {
    const int64_t groups = (tokens + tg - 1) / tg;
    dim3 grid(static_cast<unsigned>(groups), static_cast<unsigned>(kvh));
    const bool fast = d == 128 && (reinterpret_cast<uintptr_t>(keys) % 16 == 0) &&
                      ((head_stride * static_cast<int64_t>(sizeof(T))) % 16 == 0) &&
                      (reinterpret_cast<uintptr_t>(ks) % 16 == 0) && (reinterpret_cast<uintptr_t>(km) % 16 == 0) &&
                      (reinterpret_cast<uintptr_t>(kl) % 16 == 0) && (reinterpret_cast<uintptr_t>(kd) % 16 == 0);
    constexpr bool kStageable = sizeof(T) == 2;
    if (fast && kStageable && tg <= (G == 64 ? 64 : 128))
        hipLaunchKernelGGL((pack128_kernel<T, G, false, kStageable>), grid, dim3(kWave * pack128_waves<G>()), 0,
                           stream, keys, head_stride, tokens, tg, ks, km, kl, kd, cap, off, AppendArgs<T>{});
    else if (fast)
        hipLaunchKernelGGL((pack128_kernel<T, G, false>), grid, dim3(kWave * pack128_waves<G>()), 0, stream, keys,
                           head_stride, tokens, tg, ks, km, kl, kd, cap, off, AppendArgs<T>{});
    else
        hipLaunchKernelGGL((pack_kernel<T, G, false>), grid, dim3(kPackThreads), 0, stream, keys, head_stride,
                           tokens, d, tg, ks, km, kl, kd, cap, off);
    return hipGetLastError();
}

template <typename T>
hipError_t launch_pack_g(const T* keys, int64_t kvh, int64_t tokens, int d, int64_t hs, int32_t* ks,
                         int32_t* km, uint16_t* kl, uint16_t* kd, int64_t cap, int64_t off, int tg, int g,
                         hipStream_t stream) {
    switch (g) {
        case 16: return launch_pack_t<T, 16>(keys, kvh, tokens, d, hs, ks, km, kl, kd, cap, off, tg, stream);
        case 32: return launch_pack_t<T, 32>(keys, kvh, tokens, d, hs, ks, km, kl, kd, cap, off, tg, stream);
        default: return launch_pack_t<T, 64>(keys, kvh, tokens, d, hs, ks, km, kl, kd, cap, off, tg, stream);
    }
}

template <typename T>
hipError_t launch_append_t(const AppendArgs<T>& ap, int64_t rows, int tg, int g, int32_t* ks, int32_t* km,
                           uint16_t* kl, uint16_t* kd, int64_t cap, hipStream_t stream) {
    const dim3 grid(static_cast<unsigned>(rows));
    switch (g) {
        case 16:
            hipLaunchKernelGGL((pack128_kernel<T, 16, true>), grid, dim3(kWave * pack128_waves<16>()), 0, stream,
                               nullptr, 0, 0, tg, ks, km, kl, kd, cap, 0, ap);
            break;
        case 32:
            hipLaunchKernelGGL((pack128_kernel<T, 32, true>), grid, dim3(kWave * pack128_waves<32>()), 0, stream,
                               nullptr, 0, 0, tg, ks, km, kl, kd, cap, 0, ap);
            break;
        default:
            if constexpr (sizeof(T) == 2) {
                if (tg <= 64) {
                    hipLaunchKernelGGL((pack128_kernel<T, 64, true, true>), grid, dim3(kWave * pack128_waves<64>()), 0,
                                       stream, nullptr, 0, 0, tg, ks, km, kl, kd, cap, 0, ap);
                    break;
                }
            }
            hipLaunchKernelGGL((pack128_kernel<T, 64, true>), grid, dim3(kWave * pack128_waves<64>()), 0, stream,
                               nullptr, 0, 0, tg, ks, km, kl, kd, cap, 0, ap);
            break;
    }
    return hipGetLastError();
}

template <typename T>
hipError_t launch_append_dt(const void* new_k, const void* new_v, void* key_cache, void* value_cache,
                            int64_t cache_rows, const int64_t* counts, int64_t batch, int kv_heads, int32_t* k_sign,
                            int32_t* k_mag, uint16_t* k_low, uint16_t* k_delta, int64_t capacity, int tg, int g,
                            int32_t* status, hipStream_t stream) {
    AppendArgs<T> ap;
    ap.new_k = static_cast<const T*>(new_k);
    ap.new_v = static_cast<const T*>(new_v);
    ap.key_cache = static_cast<T*>(key_cache);
    ap.value_cache = static_cast<T*>(value_cache);
    ap.cache_rows = cache_rows;
    ap.counts = counts;
    ap.kv_heads = kv_heads;
    ap.status = status;
    return launch_append_t<T>(ap, batch * kv_heads, tg, g, k_sign, k_mag, k_low, k_delta, capacity, stream);
}

}  // namespace

hipError_t launch_append(const void* new_k, const void* new_v, int dtype, void* key_cache, void* value_cache,
                         int64_t cache_rows, const int64_t* counts, int64_t batch, int kv_heads, int32_t* k_sign,
                         int32_t* k_mag, uint16_t* k_low, uint16_t* k_delta, int64_t capacity,
                         int token_group_size, int dim_group_size, int32_t* status, hipStream_t stream) {
    if (batch <= 0 || kv_heads <= 0) return hipSuccess;
    switch (dtype) {
        case POPKV_DTYPE_F32:
            return launch_append_dt<float>(new_k, new_v, key_cache, value_cache, cache_rows, counts, batch, kv_heads,
                                           k_sign, k_mag, k_low, k_delta, capacity, token_group_size,
                                           dim_group_size, status, stream);
        case POPKV_DTYPE_F16:
            return launch_append_dt<f16_t>(new_k, new_v, key_cache, value_cache, cache_rows, counts, batch, kv_heads,
                                           k_sign, k_mag, k_low, k_delta, capacity, token_group_size,
                                           dim_group_size, status, stream);
        default:
            return launch_append_dt<bf16_t>(new_k, new_v, key_cache, value_cache, cache_rows, counts, batch,
                                            kv_heads, k_sign, k_mag, k_low, k_delta, capacity, token_group_size,
                                            dim_group_size, status, stream);
    }
}

hipError_t launch_pack(const void* keys, int dtype, int64_t kv_heads, int64_t tokens, int head_dim,
                       int64_t key_head_stride, int32_t* k_sign, int32_t* k_mag, uint16_t* k_low,
                       uint16_t* k_delta, int64_t capacity, int64_t token_offset, int token_group_size,
                       int dim_group_size, hipStream_t stream) {
    if (tokens <= 0) return hipSuccess;
    switch (dtype) {
        case POPKV_DTYPE_F32:
            return launch_pack_g(static_cast<const float*>(keys), kv_heads, tokens, head_dim, key_head_stride,
                                 k_sign, k_mag, k_low, k_delta, capacity, token_offset, token_group_size,
                                 dim_group_size, stream);
        case POPKV_DTYPE_F16:
            return launch_pack_g(static_cast<const f16_t*>(keys), kv_heads, tokens, head_dim, key_head_stride,
                                 k_sign, k_mag, k_low, k_delta, capacity, token_offset, token_group_size,
                                 dim_group_size, stream);
        default:
            return launch_pack_g(static_cast<const bf16_t*>(keys), kv_heads, tokens, head_dim, key_head_stride,
                                 k_sign, k_mag, k_low, k_delta, capacity, token_offset, token_group_size,
                                 dim_group_size, stream);
    }
}

}  // namespace popkv
