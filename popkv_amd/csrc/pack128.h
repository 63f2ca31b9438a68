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

// One dimension of the encode for this lane's token: the sign bit (v >= 0)
// and the magnitude bit m = (v > hi) | (v < lo) shifted into ws / wm from
// the bottom (w = 2w + bit: one add with the compare's lane mask as the
// carry-in), and |v| into the low bucket xl (m = 0) or the high bucket xh
// (m = 1), the other bucket 0.  The masks live in SGPRs written and read
// only inside this block, ordered so that each VALU read of an SGPR comes
// at least two instructions after the VALU write of it (gfx950's wait
// states for a VALU-written SGPR read by VALU, which the compiler does not
// insert into inline assembly), and the block ends with two instructions
// that write no SGPR.
__device__ __forceinline__ void encode_dim(float v, float hi, float lo, uint32_t& ws, uint32_t& wm, float& xl,
                                           float& xh) {
    uint64_t ms, m1, m2, carry;
    asm volatile(
        "v_cmp_le_f32_e64 %[ms], 0, %[v]\n\t"
        "v_cmp_gt_f32_e64 %[m1], %[v], %[hi]\n\t"
        "v_cmp_lt_f32_e64 %[m2], %[v], %[lo]\n\t"
        "v_addc_co_u32_e64 %[ws], %[carry], %[ws], %[ws], %[ms]\n\t"
        "s_or_b64 %[m1], %[m1], %[m2]\n\t"
        "v_addc_co_u32_e64 %[wm], %[carry], %[wm], %[wm], %[m1]\n\t"
        "v_cndmask_b32_e64 %[xl], |%[v]|, 0, %[m1]\n\t"
        "v_cndmask_b32_e64 %[xh], 0, |%[v]|, %[m1]"
        : [ws] "+v"(ws), [wm] "+v"(wm), [xl] "=&v"(xl), [xh] "=&v"(xh), [ms] "=&s"(ms), [m1] "=&s"(m1),
          [m2] "=&s"(m2), [carry] "=&s"(carry)
        : [v] "v"(v), [hi] "v"(hi), [lo] "v"(lo)
        : "scc");  // s_or_b64 sets SCC
}

// Encodes one token group (head_dim 128) into packed rows orow0 + t:
//   Phase 1 -- the waves stream the group's rows with coalesced loads (16
//              bytes of one of four rows per lane; in the WIDE form 4 bytes,
//              lane l owning dims 2l and 2l+1), keeping per-dimension
//              min/max in registers; the partial extrema meet in LDS and
//              the thresholds 0.5*max / 0.5*min go to LDS.
//   Phase 2 -- one token per lane, each wave on its chunk of CH = max(G, 32)
//              dimensions: the sign/magnitude words and the representatives,
//              reduced in registers in the production tree order (G64 pairs
//              dims j and j+32 first).
// Rows come from row_of(t), t < n.  Every thread of the workgroup calls it;
// the workgroup has pack128_waves<G>() waves, or (WIDE) more, whose extra
// waves join the barriers only.
template <typename T, int G, bool WIDE = false, bool STAGE = false, typename RowOf>
__device__ __forceinline__ void pack128_group(const RowOf& row_of, int n, int64_t orow0,
                                              int32_t* __restrict__ k_sign, int32_t* __restrict__ k_mag,
                                              uint16_t* __restrict__ k_low, uint16_t* __restrict__ k_delta) {
    constexpr int D = 128, R = D / G, CH = G > 32 ? G : 32, NW = D / CH, PH1 = 16;
    static_assert(!STAGE || (!WIDE && sizeof(T) == 2), "the staged form: 16-bit rows");
    // STAGE (n <= SCAP: 64 rows at G64, 128 at G32 / G16): phase 1 also
    // keeps the group's rows in LDS, at SROW bytes per row (16 more than a
    // row, so that phase 2's lanes, a row each, reading 16 bytes at one
    // offset spread over all banks), and phase 2 reads them there instead
    // of from memory.
    constexpr int SROW = D * static_cast<int>(sizeof(T)) + 16;
    constexpr int SCAP = G == 64 ? 64 : 128;
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    __shared__ __align__(16) float s_hi[D], s_lo[D];  // 0.5*max and 0.5*min, read in vectors
    __shared__ __align__(16) uint8_t s_rows[STAGE ? SCAP * SROW : 16];
    if constexpr (!WIDE) {
        // Phase 1: lane l reads dims d8 .. d8+7 (16 bytes) of row slot
        // l / 16, so one load covers four rows; in each pass of 64 rows wave
        // w reads the row quads w, w + NW, ... (rows past n repeat row n-1:
        // min/max unchanged).  The 4*NW partial extrema of a dimension meet
        // in LDS.
        constexpr int QW = 16 / NW;
        const int sub = lane >> 4, d8 = 8 * (lane & 15);
        float mn[8], mx[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) { mn[e] = INFINITY; mx[e] = -INFINITY; }
        for (int r0 = 0; r0 < n; r0 += 64) {
            Raw8<T> raw[QW];
            if (r0 + 64 <= n) {
#pragma unroll
                for (int k = 0; k < QW; ++k) raw[k].load(row_of(r0 + 4 * (wave + NW * k) + sub) + d8);
            } else {
#pragma unroll
                for (int k = 0; k < QW; ++k) raw[k].load(row_of(min(r0 + 4 * (wave + NW * k) + sub, n - 1)) + d8);
            }
            if constexpr (STAGE) {  // row slot r0 + 4*(wave + NW*k) + sub (n <= SCAP)
                if (r0 < SCAP) {
#pragma unroll
                    for (int k = 0; k < QW; ++k)
                        *reinterpret_cast<uint4*>(s_rows + (r0 + 4 * (wave + NW * k) + sub) * SROW + d8 * 2) = raw[k].u;
                }
            }
#pragma unroll
            for (int k = 0; k < QW; ++k) {
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    mn[e] = fminf(mn[e], raw[k].get(e));
                    mx[e] = fmaxf(mx[e], raw[k].get(e));
                }
            }
        }
        __shared__ __align__(16) float s_mn[4 * NW][D], s_mx[4 * NW][D];
        float4* pn = reinterpret_cast<float4*>(&s_mn[4 * wave + sub][d8]);
        float4* px = reinterpret_cast<float4*>(&s_mx[4 * wave + sub][d8]);
        pn[0] = make_float4(mn[0], mn[1], mn[2], mn[3]);
        pn[1] = make_float4(mn[4], mn[5], mn[6], mn[7]);
        px[0] = make_float4(mx[0], mx[1], mx[2], mx[3]);
        px[1] = make_float4(mx[4], mx[5], mx[6], mx[7]);
        __syncthreads();
        if (threadIdx.x < D) {
            float lo = s_mn[0][threadIdx.x], hi = s_mx[0][threadIdx.x];
#pragma unroll
            for (int w = 1; w < 4 * NW; ++w) {
                lo = fminf(lo, s_mn[w][threadIdx.x]);
                hi = fmaxf(hi, s_mx[w][threadIdx.x]);
            }
            s_lo[threadIdx.x] = lo * 0.5f;
            s_hi[threadIdx.x] = hi * 0.5f;
        }
    } else {
        // Phase 1 (a wider workgroup, one group per call): extrema of dims
        // 2*lane, 2*lane+1; wave w < NW takes tokens w, w+NW, ...
        float mn0 = INFINITY, mx0 = -INFINITY, mn1 = INFINITY, mx1 = -INFINITY;
        for (int t0 = wave; wave < NW && t0 < n; t0 += PH1 * NW) {
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
        if (wave < NW) {
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
            s_lo[threadIdx.x] = mn * 0.5f;
            s_hi[threadIdx.x] = mx * 0.5f;
        }
    }
    __syncthreads();

    // Phase 2: wave w encodes dims [w*CH, w*CH + CH) of one token per lane,
    // one 32-dimension plane word at a time.  Per dimension: sign
    // s = v >= 0, magnitude m = s ? |v| > hi : |v| > -lo; the word bits are
    // shifted in from the top (w = 2w + bit, one carry-in add); |v| goes to
    // the low or the high bucket.  m is formed as (v > hi) | (v < lo): for
    // v >= 0 (v = -0 included) v < lo cannot hold (lo is half a minimum
    // that is at most v, or negative) and for v < 0 v > hi cannot (hi is
    // half a maximum that is at least v, or at least 0), -v > -lo is
    // v < lo exactly, and a NaN fails both -- two compares instead of a
    // compare, a select and a compare.  G64 adds dims j and j+32 (its two
    // plane words) before the halving tree; G32 / G16 reduce within one
    // word.
    if (WIDE && wave >= NW) return;  // (a wider workgroup's other waves: no dimensions)
    const int c0 = wave * CH;
    if constexpr (G == 64) {
        // G64: wave w owns rep w (dims c0 .. c0+63, plane words 2w, 2w+1).
        // The production tree pairs dim j with j+32 and then halves, so its
        // first level pairs (i, i+32) with (i+16, i+48); iteration i takes
        // those four dimensions and leaves z[i] = (x[i] + x[i+32]) +
        // (x[i+16] + x[i+48]) -- the same additions as the plain order, with
        // few partial sums live instead of 64 contributions.  The iterations
        // run i = 15 .. 0, so each quarter q of the rep (dims 16q .. 16q+15)
        // gets its bits shifted in from the top, and the halving tree over
        // z[0..15] (levels 8, 4, 2, 1) forms each sum once both operands
        // exist, in its fixed order.  The row stays packed (8 x 16 bytes);
        // the thresholds of two consecutive i are read together (64-bit LDS
        // reads: at 128 bits the extra registers cost more than the reads).
        for (int t = lane; t < n; t += kWave) {
            const int64_t orow = orow0 + t;
            Raw8<T> raw[8];
            if constexpr (STAGE) {
#pragma unroll
                for (int c = 0; c < 8; ++c) raw[c].u = *reinterpret_cast<const uint4*>(s_rows + t * SROW + (c0 + 8 * c) * 2);
            } else {
                const T* row = row_of(t) + c0;
#pragma unroll
                for (int c = 0; c < 8; ++c) raw[c].load(row + 8 * c);
            }
            uint32_t sq[4] = {0u, 0u, 0u, 0u}, mq[4] = {0u, 0u, 0u, 0u};
            float2 z[16];  // z[i], then the tree's partial sums in place
            auto add2 = [](float2 u, float2 w) { return make_float2(u.x + w.x, u.y + w.y); };
            typedef float f32x2 __attribute__((ext_vector_type(2)));
#pragma unroll
            for (int ib = 7; ib >= 0; --ib) {
                // thresholds of dims 16q + 2ib, 16q + 2ib + 1; the empty asm
                // keeps the reads in this block
                f32x2 h2[4], l2[4];
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    h2[q] = *reinterpret_cast<const f32x2*>(s_hi + c0 + 16 * q + 2 * ib);
                    l2[q] = *reinterpret_cast<const f32x2*>(s_lo + c0 + 16 * q + 2 * ib);
                }
                asm volatile("" : "+v"(h2[0]), "+v"(h2[1]), "+v"(h2[2]), "+v"(h2[3]), "+v"(l2[0]), "+v"(l2[1]),
                             "+v"(l2[2]), "+v"(l2[3]));
#pragma unroll
                for (int ii = 1; ii >= 0; --ii) {
                    const int i = 2 * ib + ii;
                    float xl[4], xh[4];
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const int dm = i + 16 * q;
                        encode_dim(raw[dm / 8].get(dm % 8), h2[q][ii], l2[q][ii], sq[q], mq[q], xl[q], xh[q]);
                    }
                    z[i] = make_float2((xl[0] + xl[2]) + (xl[1] + xl[3]), (xh[0] + xh[2]) + (xh[1] + xh[3]));
                    // the tree levels whose second operand is now complete
                    if (i < 8) z[i] = add2(z[i], z[i + 8]);
                    if (i < 4) z[i] = add2(z[i], z[i + 4]);
                    if (i < 2) z[i] = add2(z[i], z[i + 2]);
                    if (i < 1) z[i] = add2(z[i], z[i + 1]);
                    // the sums are formed here, so few values stay live
                    asm volatile("" : "+v"(z[i].x), "+v"(z[i].y));
                }
            }
            const float2 sums = z[0];
            const uint32_t sw0 = sq[0] | (sq[1] << 16), sw1 = sq[2] | (sq[3] << 16);
            const uint32_t mw0 = mq[0] | (mq[1] << 16), mw1 = mq[2] | (mq[3] << 16);
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
        const T* row;
        if constexpr (STAGE) row = reinterpret_cast<const T*>(s_rows + t * SROW) + c0;
        else row = row_of(t) + c0;
        const int64_t orow = orow0 + t;
        constexpr int NWD = CH / 32, NR = CH / G;
        uint32_t sw[NWD], mw[NWD];
        float lows[NR], deltas[NR];
#pragma unroll
        for (int wi = 0; wi < NWD; ++wi) {
            float v[32];
#pragma unroll
            for (int i = 0; i < 32; i += 8) load8<T>(row + wi * 32 + i, v + i);
            uint32_t sgw = 0, mgw = 0;
            float xl[32], xh[32];
            typedef float f32x4 __attribute__((ext_vector_type(4)));
#pragma unroll
            for (int jb = 7; jb >= 0; --jb) {
                // thresholds of dims 4jb .. 4jb+3 of the word, one read each;
                // the empty asm keeps the reads in this block
                f32x4 h4 = *reinterpret_cast<const f32x4*>(s_hi + c0 + wi * 32 + 4 * jb);
                f32x4 l4 = *reinterpret_cast<const f32x4*>(s_lo + c0 + wi * 32 + 4 * jb);
                asm volatile("" : "+v"(h4), "+v"(l4));
#pragma unroll
                for (int jj = 3; jj >= 0; --jj) {
                    const int j = 4 * jb + jj;
                    encode_dim(v[j], h4[jj], l4[jj], sgw, mgw, xl[j], xh[j]);
                }
            }
            sw[wi] = sgw;
            mw[wi] = mgw;
            if constexpr (G == 32) {
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
template <typename T, int G, bool WIDE = false, bool STAGE = false>
__device__ __forceinline__ void pack128_append(int64_t bh, const AppendArgs<T>& ap, int tg,
                                               int32_t* __restrict__ k_sign, int32_t* __restrict__ k_mag,
                                               uint16_t* __restrict__ k_low, uint16_t* __restrict__ k_delta,
                                               int64_t cap) {
    constexpr int D = 128;
    const int64_t count = ap.counts[div_nonneg(static_cast<int>(bh), ap.kv_heads)];  // (bh < 2^31)
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
    pack128_group<T, G, WIDE, STAGE>(row_of, n, bh * cap + sealed, k_sign, k_mag, k_low, k_delta);
}

}  // namespace popkv
