// The head_dim-128 token-group encode of the PopKV packers, shared by the
// prefix prepack / append kernels (pack.hip) and the batched decode step's
// select + attention launch (attention.hip), which runs the append of the
// current token in extra workgroups of its own grid.
//
// Semantics follow the reference packers: popkv_ext.cu:79-143 (G32),
// :376-500 (fused G16/G64, head_dim 128), with output rows token_offset + t
// (the in-place append of :1075-1092, :1177-1206).
#pragma once

#include "device_common.h"

namespace popkv {

// Two consecutive elements (dims 2l, 2l+1) of a row as float.
template <typename T> __device__ __forceinline__ void load2(const T* p, float& a, float& b);
template <> __device__ __forceinline__ void load2<bf16_t>(const bf16_t* p, float& a, float& b) {
    const uint32_t u = *reinterpret_cast<const uint32_t*>(p);
    a = __uint_as_float(u << 16);
    b = __uint_as_float(u & 0xffff0000u);
}
template <> __device__ __forceinline__ void load2<f16_t>(const f16_t* p, float& a, float& b) {
    const uint32_t u = *reinterpret_cast<const uint32_t*>(p);
    a = bits_f16(u & 0xffffu);
    b = bits_f16(u >> 16);
}
template <> __device__ __forceinline__ void load2<float>(const float* p, float& a, float& b) {
    const float2 f = *reinterpret_cast<const float2*>(p);
    a = f.x;
    b = f.y;
}

// Waves per workgroup of pack128_kernel: one per chunk of CH = max(G, 32)
// dimensions (whole plane words and whole representatives).
template <int G> constexpr int pack128_waves() { return 128 / (G > 32 ? G : 32); }

// Operands of the fused append (APPEND form of pack128_kernel): block i
// serves KV head i % kv_heads of sequence b = i / kv_heads, whose cache
// holds counts[b] tokens.  new_k / new_v [B*KVH, 128] are the new token's
// rows; key_cache / value_cache [B*KVH, cache_rows, 128] the static caches
// (the new rows go to row counts[b]); the packed planes have `cap` rows per
// (sequence, KV head).  A count outside [0, min(cache_rows, cap)) writes
// nothing and sets *status to 1 (when status is non-null).
template <typename T>
struct AppendArgs {
    const T* new_k = nullptr;
    const T* new_v = nullptr;
    T* key_cache = nullptr;
    T* value_cache = nullptr;
    int64_t cache_rows = 0;
    const int64_t* counts = nullptr;
    int kv_heads = 1;
    int32_t* status = nullptr;
};

// Encodes one token group (head_dim 128) into packed rows orow0 + t:
//   Phase 1 -- lane l owns dims 2l and 2l+1; the waves stream interleaved
//              rows of the group with coalesced loads, keeping
//              per-dimension min/max in registers; the partial extrema meet
//              in LDS and the thresholds 0.5*max / 0.5*min go to LDS.
//   Phase 2 -- one token per lane, each wave on its chunk of CH = max(G, 32)
//              dimensions: the sign/magnitude words and the representatives,
//              reduced in registers in the production tree order (G64 pairs
//              dims j and j+32 first).
// Rows come from row_of(t), t < n.  Every thread of the workgroup calls it;
// the workgroup has pack128_waves<G>() waves, or (WIDE) more, whose extra
// waves join the barriers only.
template <typename T, int G, bool WIDE = false, typename RowOf>
__device__ __forceinline__ void pack128_group(const RowOf& row_of, int n, int64_t orow0,
                                              int32_t* __restrict__ k_sign, int32_t* __restrict__ k_mag,
                                              uint16_t* __restrict__ k_low, uint16_t* __restrict__ k_delta) {
    constexpr int D = 128, R = D / G, CH = G > 32 ? G : 32, NW = D / CH, PH1 = 16;
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    // Phase 1: extrema of dims 2*lane, 2*lane+1; wave w takes tokens w, w+NW, ...
    float mn0 = INFINITY, mx0 = -INFINITY, mn1 = INFINITY, mx1 = -INFINITY;
    for (int t0 = wave; (!WIDE || wave < NW) && t0 < n; t0 += PH1 * NW) {
        float a[PH1], b[PH1];
#pragma unroll
        for (int i = 0; i < PH1; ++i) {
            const int t = min(t0 + i * NW, n - 1);  // repeats the last row: min/max unchanged
            load2<T>(row_of(t) + 2 * lane, a[i], b[i]);
        }
#pragma unroll
        for (int i = 0; i < PH1; ++i) {
            mn0 = fminf(mn0, a[i]); mx0 = fmaxf(mx0, a[i]);
            mn1 = fminf(mn1, b[i]); mx1 = fmaxf(mx1, b[i]);
        }
    }
    __shared__ float s_mn[NW][D], s_mx[NW][D];
    __shared__ float s_hi[D], s_nlo[D];  // 0.5*max and -(0.5*min)
    if (!WIDE || wave < NW) {
        s_mn[wave][2 * lane] = mn0; s_mn[wave][2 * lane + 1] = mn1;
        s_mx[wave][2 * lane] = mx0; s_mx[wave][2 * lane + 1] = mx1;
    }
    __syncthreads();
    if (threadIdx.x < D) {
        float mn = s_mn[0][threadIdx.x], mx = s_mx[0][threadIdx.x];
#pragma unroll
        for (int w = 1; w < NW; ++w) {
            mn = fminf(mn, s_mn[w][threadIdx.x]);
            mx = fmaxf(mx, s_mx[w][threadIdx.x]);
        }
        s_nlo[threadIdx.x] = -(mn * 0.5f);
        s_hi[threadIdx.x] = mx * 0.5f;
    }
    __syncthreads();

    // Phase 2: wave w encodes dims [w*CH, w*CH + CH) of one token per lane,
    // one 32-dimension plane word at a time.  Per dimension: sign
    // s = v >= 0, magnitude m = s ? v > hi : v < lo; the word bits are
    // shifted in from the top (w = 2w + bit); |v| goes to the low or the high
    // bucket.  G64 adds dims j and j+32 (its two plane words) before the
    // halving tree; G32 / G16 reduce within one word.
    if (WIDE && wave >= NW) return;  // (a wider workgroup's other waves: no dimensions)
    const int c0 = wave * CH;
    if constexpr (G == 64) {
        // G64: wave w owns rep w (dims c0 .. c0+63, plane words 2w, 2w+1).
        // The production tree pairs dim j with j+32 and then halves, so its
        // first level pairs (i, i+32) with (i+16, i+48); iteration i takes
        // those four dimensions and leaves z[i] = (x[i] + x[i+32]) +
        // (x[i+16] + x[i+48]) -- the same additions as the plain order, with
        // 16 partial sums live instead of 64 contributions.  Bits are placed
        // at their positions directly.  The row stays packed (8 x 16 bytes).
        for (int t = lane; t < n; t += kWave) {
            const T* row = row_of(t) + c0;
            const int64_t orow = orow0 + t;
            Raw8<T> raw[8];
#pragma unroll
            for (int c = 0; c < 8; ++c) raw[c].load(row + 8 * c);
            uint32_t sw0 = 0, mw0 = 0, sw1 = 0, mw1 = 0;
            // z(i): dims i, i+16, i+32, i+48 -> (low, high) level-16 sums;
            // i is a compile-time constant (the row registers are indexed
            // statically)
            auto z = [&](auto ic) {
                constexpr int i = decltype(ic)::value;
                float xl[4], xh[4];
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int dm = i + 16 * q;
                    // the empty asm ties the thresholds to the bit words:
                    // read one dimension at a time, not all hoisted
                    float hi = s_hi[c0 + dm], nlo = s_nlo[c0 + dm];
                    asm volatile("" : "+v"(hi), "+v"(nlo), "+v"(sw0), "+v"(sw1));
                    const float v = raw[dm / 8].get(dm % 8);
                    const float a = fabsf(v);
                    const bool sg = v >= 0.0f;
                    const bool mg = a > (sg ? hi : nlo);  // as in the plain path below
                    const int bit = dm & 31;
                    if (q < 2) {
                        sw0 |= static_cast<uint32_t>(sg) << bit;
                        mw0 |= static_cast<uint32_t>(mg) << bit;
                    } else {
                        sw1 |= static_cast<uint32_t>(sg) << bit;
                        mw1 |= static_cast<uint32_t>(mg) << bit;
                    }
                    xl[q] = mg ? 0.0f : a;
                    xh[q] = mg ? a : 0.0f;
                }
                return make_float2((xl[0] + xl[2]) + (xl[1] + xl[3]), (xh[0] + xh[2]) + (xh[1] + xh[3]));
            };
            auto add2 = [](float2 u, float2 w) { return make_float2(u.x + w.x, u.y + w.y); };
            using std::integral_constant;
            // the halving tree over z(0..15) (levels 8, 4, 2, 1), evaluated
            // depth-first so only a few partial sums are live
            auto a8 = [&](auto ic) {
                constexpr int i = decltype(ic)::value;
                const float2 u = z(integral_constant<int, i>{});
                return add2(u, z(integral_constant<int, i + 8>{}));
            };
            auto b4 = [&](auto ic) {
                constexpr int i = decltype(ic)::value;
                const float2 u = a8(integral_constant<int, i>{});
                return add2(u, a8(integral_constant<int, i + 4>{}));
            };
            auto c2 = [&](auto ic) {
                constexpr int i = decltype(ic)::value;
                const float2 u = b4(integral_constant<int, i>{});
                return add2(u, b4(integral_constant<int, i + 2>{}));
            };
            const float2 c0s = c2(integral_constant<int, 0>{});
            const float2 sums = add2(c0s, c2(integral_constant<int, 1>{}));
            const int hn = __popc(mw0) + __popc(mw1);
            float lo, de;
            finish_rep(sums.x, 64 - hn, sums.y, hn, lo, de);
            const int w0 = c0 / 32;
            *reinterpret_cast<uint2*>(k_sign + orow * 4 + w0) = make_uint2(sw0, sw1);
            *reinterpret_cast<uint2*>(k_mag + orow * 4 + w0) = make_uint2(mw0, mw1);
            k_low[orow * R + wave] = f16_rne(lo);
            k_delta[orow * R + wave] = f16_rne(de);
        }
        return;
    }
    for (int t = lane; t < n; t += kWave) {
        const T* row = row_of(t) + c0;
        const int64_t orow = orow0 + t;
        constexpr int NWD = CH / 32, NR = CH / G;
        uint32_t sw[NWD], mw[NWD];
        float lows[NR], deltas[NR];
        float pl[32], ph[32];  // G64: first-level pair sums
#pragma unroll
        for (int wi = 0; wi < NWD; ++wi) {
            float v[32];
#pragma unroll
            for (int i = 0; i < 32; i += 8) load8<T>(row + wi * 32 + i, v + i);
            uint32_t sgw = 0, mgw = 0;
            float xl[32], xh[32];
#pragma unroll
            for (int j = 31; j >= 0; --j) {
                // m = s ? v > hi : v < lo is |v| > (s ? hi : -lo): for v < 0,
                // v < lo <=> -v > -lo; for v = -0 both sides read 0 > hi; a
                // NaN has s = 0 and fails the compare.  The thresholds pass
                // through an empty asm: the same in every lane, they stay in
                // VGPRs, and the dimensions stay in order.
                float hi = s_hi[c0 + wi * 32 + j], nlo = s_nlo[c0 + wi * 32 + j];
                asm volatile("" : "+v"(hi), "+v"(nlo), "+v"(sgw), "+v"(mgw));
                const float a = fabsf(v[j]);
                const bool sg = v[j] >= 0.0f;
                const bool mg = a > (sg ? hi : nlo);
                sgw = sgw * 2u + static_cast<uint32_t>(sg);
                mgw = mgw * 2u + static_cast<uint32_t>(mg);
                xl[j] = mg ? 0.0f : a;
                xh[j] = mg ? a : 0.0f;
            }
            sw[wi] = sgw;
            mw[wi] = mgw;
            if constexpr (G == 64) {
                if (wi == 0) {
#pragma unroll
                    for (int j = 0; j < 32; ++j) { pl[j] = xl[j]; ph[j] = xh[j]; }
                } else {
#pragma unroll
                    for (int j = 0; j < 32; ++j) { pl[j] = pl[j] + xl[j]; ph[j] = ph[j] + xh[j]; }
                    const int hn = __popc(mw[0]) + __popc(mgw);
                    finish_rep(tree_halving(pl, 32), 64 - hn, tree_halving(ph, 32), hn, lows[0], deltas[0]);
                }
            } else if constexpr (G == 32) {
                const int hn = __popc(mgw);
                finish_rep(tree_halving(xl, 32), 32 - hn, tree_halving(xh, 32), hn, lows[0], deltas[0]);
            } else {
#pragma unroll
                for (int hf = 0; hf < 2; ++hf) {
                    const int hn = __popc(hf ? (mgw >> 16) : (mgw & 0xffffu));
                    finish_rep(tree_halving(xl + 16 * hf, 16), 16 - hn, tree_halving(xh + 16 * hf, 16), hn,
                               lows[hf], deltas[hf]);
                }
            }
        }
        const int w0 = c0 / 32, r0 = c0 / G;
#pragma unroll
        for (int wi = 0; wi < NWD; ++wi) {
            k_sign[orow * 4 + w0 + wi] = static_cast<int32_t>(sw[wi]);
            k_mag[orow * 4 + w0 + wi] = static_cast<int32_t>(mw[wi]);
        }
        if constexpr (NR == 1) {
            k_low[orow * R + r0] = f16_rne(lows[0]);
            k_delta[orow * R + r0] = f16_rne(deltas[0]);
        } else {
            reinterpret_cast<uint32_t*>(k_low + orow * R + r0)[0] =
                static_cast<uint32_t>(f16_rne(lows[0])) | (static_cast<uint32_t>(f16_rne(lows[1])) << 16);
            reinterpret_cast<uint32_t*>(k_delta + orow * R + r0)[0] =
                static_cast<uint32_t>(f16_rne(deltas[0])) | (static_cast<uint32_t>(f16_rne(deltas[1])) << 16);
        }
    }
}

// The fused append of one (sequence, KV head) bh (see AppendArgs): the new
// token joins its sequence's active group -- rows [sealed, count) read in
// place from the static key cache, then the new key itself, sealed = count -
// count % tg -- and the whole group is re-encoded into packed rows sealed ..
// count; the new K/V rows are written to the static caches.  Every thread
// of a workgroup of max(pack128_waves<G>(), 2 * D * sizeof(T) / 16 / 64)
// waves (or, WIDE, more) calls it.
template <typename T, int G, bool WIDE = false>
__device__ __forceinline__ void pack128_append(int64_t bh, const AppendArgs<T>& ap, int tg,
                                               int32_t* __restrict__ k_sign, int32_t* __restrict__ k_mag,
                                               uint16_t* __restrict__ k_low, uint16_t* __restrict__ k_delta,
                                               int64_t cap) {
    constexpr int D = 128;
    const int64_t count = ap.counts[bh / ap.kv_heads];
    if (count < 0 || count >= ap.cache_rows || count >= cap) {
        if (ap.status != nullptr && threadIdx.x == 0) *ap.status = 1;
        return;
    }
    // the new K and V rows into the static caches, 16 bytes per thread
    constexpr int VEC = D * static_cast<int>(sizeof(T)) / 16;
    const int64_t dst_row = (bh * ap.cache_rows + count) * D;
    if (threadIdx.x < VEC) {
        reinterpret_cast<uint4*>(ap.key_cache + dst_row)[threadIdx.x] =
            reinterpret_cast<const uint4*>(ap.new_k + bh * D)[threadIdx.x];
    } else if (threadIdx.x < 2 * VEC) {
        reinterpret_cast<uint4*>(ap.value_cache + dst_row)[threadIdx.x - VEC] =
            reinterpret_cast<const uint4*>(ap.new_v + bh * D)[threadIdx.x - VEC];
    }
    const int64_t sealed = count - count % tg;
    const int n = static_cast<int>(count - sealed) + 1;
    const T* base = ap.key_cache + (bh * ap.cache_rows + sealed) * D;
    const T* last = ap.new_k + bh * D;
    auto row_of = [&](int t) -> const T* { return t == n - 1 ? last : base + static_cast<int64_t>(t) * D; };
    pack128_group<T, G, WIDE>(row_of, n, bh * cap + sealed, k_sign, k_mag, k_low, k_delta);
}

}  // namespace popkv
