// Key prepack and per-token append of PopKV retrieval metadata (gfx950).
//
// head_dim 128 (pack128_kernel): one workgroup per (KV head, token group),
// one wave per chunk of max(G, 32) dimensions (2 or 4 waves).
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

// Prefix prepack (APPEND false): block (x, y) encodes token group x of KV
// head y, rows [x*tg, min(x*tg + tg, tokens)) of `keys`, into packed rows
// y*cap + offset + x*tg + t.
// Fused append (APPEND true, see AppendArgs): the new token joins its
// sequence's active group -- rows [sealed, count) read in place from the
// static key cache, then the new key itself, sealed = count - count % tg --
// and the whole group is re-encoded into packed rows sealed .. count; the
// new K/V rows are written to the static caches by the same block.
template <typename T, int G, bool APPEND>
__global__ __launch_bounds__(kWave * pack128_waves<G>()) void pack128_kernel(
    const T* __restrict__ keys, int64_t head_stride, int64_t tokens, int tg,
    int32_t* __restrict__ k_sign, int32_t* __restrict__ k_mag,
    uint16_t* __restrict__ k_low, uint16_t* __restrict__ k_delta, int64_t cap, int64_t offset,
    AppendArgs<T> ap) {
    constexpr int D = 128, R = D / G, CH = G > 32 ? G : 32, NW = D / CH, PH1 = 16;
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    int n;
    const T* base;             // row t < n (t < n - 1 in the append) is base + t * D
    const T* last = nullptr;   // the append's new key (row n - 1)
    int64_t orow0;             // packed row of token 0
    if constexpr (!APPEND) {
        const int64_t kvh = blockIdx.y;
        const int64_t gs = static_cast<int64_t>(blockIdx.x) * tg;
        n = static_cast<int>(min(gs + static_cast<int64_t>(tg), tokens) - gs);
        base = keys + kvh * head_stride + gs * D;
        orow0 = kvh * cap + offset + gs;
    } else {
        const int64_t bh = blockIdx.x;
        const int64_t count = ap.counts[bh / ap.kv_heads];
        if (count < 0 || count >= ap.cache_rows || count >= cap) {
            if (ap.status != nullptr && threadIdx.x == 0) *ap.status = 1;
            return;
        }
        // the new K and V rows into the static caches, 16 bytes per thread
        constexpr int VEC = D * static_cast<int>(sizeof(T)) / 16;
        static_assert(2 * VEC <= kWave * NW, "one 16-byte slice per thread");
        const int64_t dst_row = (bh * ap.cache_rows + count) * D;
        if (threadIdx.x < VEC) {
            reinterpret_cast<uint4*>(ap.key_cache + dst_row)[threadIdx.x] =
                reinterpret_cast<const uint4*>(ap.new_k + bh * D)[threadIdx.x];
        } else if (threadIdx.x < 2 * VEC) {
            reinterpret_cast<uint4*>(ap.value_cache + dst_row)[threadIdx.x - VEC] =
                reinterpret_cast<const uint4*>(ap.new_v + bh * D)[threadIdx.x - VEC];
        }
        const int64_t sealed = count - count % tg;
        n = static_cast<int>(count - sealed) + 1;
        base = ap.key_cache + (bh * ap.cache_rows + sealed) * D;
        last = ap.new_k + bh * D;
        orow0 = bh * cap + sealed;
    }
    auto row_of = [&](int t) -> const T* {
        if constexpr (APPEND) return t == n - 1 ? last : base + static_cast<int64_t>(t) * D;
        else return base + static_cast<int64_t>(t) * D;
    };

    // Phase 1: extrema of dims 2*lane, 2*lane+1; wave w takes tokens w, w+NW, ...
    float mn0 = INFINITY, mx0 = -INFINITY, mn1 = INFINITY, mx1 = -INFINITY;
    for (int t0 = wave; t0 < n; t0 += PH1 * NW) {
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
    s_mn[wave][2 * lane] = mn0; s_mn[wave][2 * lane + 1] = mn1;
    s_mx[wave][2 * lane] = mx0; s_mx[wave][2 * lane + 1] = mx1;
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
    if (fast)
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
