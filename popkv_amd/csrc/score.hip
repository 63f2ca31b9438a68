// Query encode and the popcount Q.K scorer (gfx950).
//
// Query encode: one wave64 per query row.  The row is staged in LDS; the
// whole-head extrema come from a butterfly (exact for min/max); sign and
// magnitude words come from 64-bit ballots (two 32-bit words per ballot);
// lane r < R then reduces representative group r from LDS in the requested
// order -- a left fold over ascending dims (the decode-path encode,
// popkv_ext.cu:232-281, :911-957) or the production reduction tree (the
// warp encode inside score(), popkv_ext.cu:677-755).
//
// Scorer (head_dim 128): one thread per (KV head, token).  Each thread loads
// its token's 16-byte sign and magnitude words and its fp16 representatives
// once with coalesced vector loads, then scores every query head of the GQA
// group.  The query state of the group is wave-uniform: the kernel reads it
// with scalar loads, so it lives in SGPRs and the per-head popcount of the
// query magnitude word is a scalar op.  Per head and representative the
// kernel needs four signed agreement counts 2*popc(x & sel) - popc(sel)
// (v_bcnt_u32_b32) and the fp32 fma chain of popkv_ext.cu:502-515 / :867-870,
// summed from +0 over representatives, times fp32(1/sqrt(128)), rounded once
// to fp16 (popkv_ext.cu:757-876).
#include <type_traits>

#include "device_common.h"
#include "kernels.h"
#include "score128.h"
#include "select_common.h"

namespace popkv {
namespace {

// ---------------------------------------------------------------- encode

template <typename T, int G, int ORDER>
__global__ __launch_bounds__(kWave) void query_encode_kernel(
    const T* __restrict__ q, int64_t rows, int d, int32_t* __restrict__ q_sign,
    int32_t* __restrict__ q_mag, float* __restrict__ q_low, float* __restrict__ q_delta) {
    const int64_t row = blockIdx.x;
    const int lane = threadIdx.x;
    const int W = (d + 31) / 32;
    const int R = (d + G - 1) / G;
    __shared__ float s_q[256];
    // fold order: each dimension's contribution to the low and to the high
    // bucket (|q| or +0), and the magnitude words
    __shared__ __align__(16) float s_lo[256], s_hi[256];
    __shared__ uint32_t s_mag[8];
    const T* src = q + row * d;

    float mn = INFINITY, mx = -INFINITY;
    float v[4];
    // all four loads in flight at once (a dimension past d re-reads d - 1)
#pragma unroll
    for (int s = 0; s < 4; ++s) v[s] = Elem<T>::load(src, min(s * kWave + lane, d - 1));
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        const int dim = s * kWave + lane;
        if (dim < d) {
            s_q[dim] = v[s];
            mn = fminf(mn, v[s]);
            mx = fmaxf(mx, v[s]);
        } else {
            v[s] = 0.0f;
        }
    }
    mn = wave_min(mn);
    mx = wave_max(mx);
    const float neg = mn * 0.5f, pos = mx * 0.5f;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        const int dim = s * kWave + lane;
        const bool valid = dim < d;
        const bool sg = valid && v[s] >= 0.0f;
        const bool mg = valid && (sg ? v[s] > pos : v[s] < neg);
        const uint64_t bs = __ballot(sg);
        const uint64_t bm = __ballot(mg);
        if constexpr (ORDER == POPKV_ENCODE_FOLD) {
            const float a = fabsf(v[s]);
            s_lo[dim] = valid && !mg ? a : 0.0f;  // dims past d: +0 padding
            s_hi[dim] = mg ? a : 0.0f;
            if (lane == 0) {
                s_mag[2 * s] = static_cast<uint32_t>(bm);
                s_mag[2 * s + 1] = static_cast<uint32_t>(bm >> 32);
            }
        }
        if (lane == 0) {
            if (2 * s < W) {
                q_sign[row * W + 2 * s] = static_cast<int32_t>(static_cast<uint32_t>(bs));
                q_mag[row * W + 2 * s] = static_cast<int32_t>(static_cast<uint32_t>(bm));
            }
            if (2 * s + 1 < W) {
                q_sign[row * W + 2 * s + 1] = static_cast<int32_t>(static_cast<uint32_t>(bs >> 32));
                q_mag[row * W + 2 * s + 1] = static_cast<int32_t>(static_cast<uint32_t>(bm >> 32));
            }
        }
    }
    __syncthreads();
    if (lane < R) {
        const int start = lane * G;
        const int end = min(start + G, d);
        float ls = 0.0f, hs = 0.0f;
        int ln = 0, hn = 0;
        if constexpr (ORDER == POPKV_ENCODE_FOLD) {
            // the ascending fold over the contributions staged above (the
            // other bucket's +0 leaves a sum unchanged: sums start at +0 and
            // only grow), four values per LDS read
            for (int j = start; j < end; j += 4) {
                const float4 l4 = *reinterpret_cast<const float4*>(&s_lo[j]);
                const float4 h4 = *reinterpret_cast<const float4*>(&s_hi[j]);
                ls = ls + l4.x; ls = ls + l4.y; ls = ls + l4.z; ls = ls + l4.w;
                hs = hs + h4.x; hs = hs + h4.y; hs = hs + h4.z; hs = hs + h4.w;
            }
            for (int w = 0; w < 8; ++w) {  // the rep's magnitude bits
                const int lo_bit = max(start, 32 * w), hi_bit = min(end, 32 * w + 32);
                if (lo_bit >= hi_bit) continue;
                const uint32_t word = s_mag[w];
                const int nb = hi_bit - lo_bit;
                const uint32_t sel = (nb == 32 ? 0xffffffffu : ((1u << nb) - 1u)) << (lo_bit - 32 * w);
                hn += __popc(word & sel);
            }
            ln = (end - start) - hn;
        } else {
            float xl[G], xh[G];
#pragma unroll
            for (int j = 0; j < G; ++j) {
                const int i = start + j;
                const float x = i < end ? s_q[min(i, 255)] : 0.0f;
                const bool sg = x >= 0.0f;
                const bool mg = i < end && (sg ? x > pos : x < neg);
                xl[j] = (i < end && !mg) ? fabsf(x) : 0.0f;
                xh[j] = mg ? fabsf(x) : 0.0f;
                ln += (i < end && !mg) ? 1 : 0;
                hn += mg ? 1 : 0;
            }
            ls = rep_tree_sum<G>(xl);
            hs = rep_tree_sum<G>(xh);
        }
        float lo, de;
        finish_rep(ls, ln, hs, hn, lo, de);
        q_low[row * R + lane] = lo;
        q_delta[row * R + lane] = de;
    }
}

// ---------------------------------------------------------------- score, D = 128

// grid.x: token tiles of kScoreThreads * score_tokens_per_thread<G>(); grid.y: batch*kv_heads.
template <int G, int QPK, typename QT, bool WIN, int TPT>
__global__ __launch_bounds__(kScoreThreads) void score_d128_kernel(
    const int32_t* __restrict__ q_sign, const int32_t* __restrict__ q_mag,
    const float* __restrict__ q_low, const float* __restrict__ q_delta, const QT* __restrict__ q_raw,
    const uint4* __restrict__ k_sign, const uint4* __restrict__ k_mag,
    const uint16_t* __restrict__ k_low, const uint16_t* __restrict__ k_delta,
    const int64_t* __restrict__ head_to_kv, int q_heads, int kv_heads, int qpk_rt,
    int64_t cap, int64_t tokens, uint16_t* __restrict__ scores, int64_t out_stride,
    uint32_t* __restrict__ ghist, SeqTable seq, TileWindows win) {
    score_d128_body<G, QPK, QT, WIN, false, TPT>(q_sign, q_mag, q_low, q_delta, q_raw, k_sign, k_mag, k_low, k_delta,
                                            head_to_kv, q_heads, kv_heads, qpk_rt, cap, tokens, scores, out_stride,
                                            ghist, seq, win, blockIdx.x, blockIdx.y);
}

// ---------------------------------------------------------------- score, generic D

// One thread per (query row, token), float32 output (popkv_ext.cu:145-230,
// :517-675): per-head KV mapping, partial words masked, scale 1/sqrt(D).
template <int G>
__global__ __launch_bounds__(256) void score_generic_kernel(
    const int32_t* __restrict__ q_sign, const int32_t* __restrict__ q_mag,
    const float* __restrict__ q_low, const float* __restrict__ q_delta,
    const int32_t* __restrict__ k_sign, const int32_t* __restrict__ k_mag,
    const uint16_t* __restrict__ k_low, const uint16_t* __restrict__ k_delta,
    const int64_t* __restrict__ head_to_kv, int q_heads, int kv_heads, int d, int64_t cap, int64_t tokens,
    float scale, float* __restrict__ scores) {
    const int64_t row = blockIdx.y;
    const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (t >= tokens) return;
    const int W = (d + 31) / 32, R = (d + G - 1) / G;
    const int64_t kvh = min(max(head_to_kv[row % q_heads], static_cast<int64_t>(0)), static_cast<int64_t>(kv_heads - 1));
    const int64_t krow = kvh * cap + t;
    float score = 0.0f;
    for (int r = 0; r < R; ++r) {
        const float ql = q_low[row * R + r], dq = q_delta[row * R + r];
        const float kl = bits_f16(k_low[krow * R + r]), dk = bits_f16(k_delta[krow * R + r]);
        int cs = 0, cq = 0, ck = 0, cqk = 0;
        const int rs = r * G, re = min(rs + G, d);
        for (int w = rs / 32; w <= (re - 1) / 32; ++w) {
            const int ws = w * 32;
            const int begin = max(rs, ws) - ws, end = min(re, ws + 32) - ws;
            const int count = end - begin;
            const uint32_t mask = count == 32 ? 0xffffffffu : ((1u << count) - 1u) << begin;
            const uint32_t qs = static_cast<uint32_t>(q_sign[row * W + w]);
            const uint32_t qm = static_cast<uint32_t>(q_mag[row * W + w]) & mask;
            const uint32_t ks = static_cast<uint32_t>(k_sign[krow * W + w]);
            const uint32_t km = static_cast<uint32_t>(k_mag[krow * W + w]) & mask;
            const uint32_t match = ~(qs ^ ks) & mask, both = qm & km;
            cs += 2 * __popc(match) - __popc(mask);
            cq += 2 * __popc(match & qm) - __popc(qm);
            ck += 2 * __popc(match & km) - __popc(km);
            cqk += 2 * __popc(match & both) - __popc(both);
        }
        score = score + fmaf(ql * kl, static_cast<float>(cs),
                             fmaf(dq * kl, static_cast<float>(cq),
                                  fmaf(ql * dk, static_cast<float>(ck), dq * dk * static_cast<float>(cqk))));
    }
    scores[row * tokens + t] = score * scale;
}

template <typename T, int G>
hipError_t launch_encode_t(const T* q, int64_t rows, int d, int order, int32_t* qs, int32_t* qm, float* ql,
                           float* qd, hipStream_t stream) {
    if (order == POPKV_ENCODE_TREE)
        hipLaunchKernelGGL((query_encode_kernel<T, G, POPKV_ENCODE_TREE>), dim3(static_cast<unsigned>(rows)),
                           dim3(kWave), 0, stream, q, rows, d, qs, qm, ql, qd);
    else
        hipLaunchKernelGGL((query_encode_kernel<T, G, POPKV_ENCODE_FOLD>), dim3(static_cast<unsigned>(rows)),
                           dim3(kWave), 0, stream, q, rows, d, qs, qm, ql, qd);
    return hipGetLastError();
}

template <typename T>
hipError_t launch_encode_g(const T* q, int64_t rows, int d, int g, int order, int32_t* qs, int32_t* qm,
                           float* ql, float* qd, hipStream_t stream) {
    switch (g) {
        case 16: return launch_encode_t<T, 16>(q, rows, d, order, qs, qm, ql, qd, stream);
        case 32: return launch_encode_t<T, 32>(q, rows, d, order, qs, qm, ql, qd, stream);
        default: return launch_encode_t<T, 64>(q, rows, d, order, qs, qm, ql, qd, stream);
    }
}

template <int G, typename QT>
hipError_t launch_score_d128_g(const int32_t* qs, const int32_t* qm, const float* ql, const float* qd, const QT* q_raw,
                               const int32_t* ks, const int32_t* km, const uint16_t* kl, const uint16_t* kd,
                               const int64_t* h2k, int64_t batch, int qh, int kvh, int64_t cap, int64_t tokens,
                               uint16_t* out, int64_t out_stride, uint32_t* ghist, const SeqTable& seq,
                               hipStream_t stream, const TileWindows& win) {
    const int qpk = qh / kvh;
    constexpr int TPT = score_tokens_per_thread<G>();
    const int64_t per_block = static_cast<int64_t>(kScoreThreads) * TPT;
    dim3 grid(static_cast<unsigned>((tokens + per_block - 1) / per_block), static_cast<unsigned>(batch * kvh));
    const uint4* ks4 = reinterpret_cast<const uint4*>(ks);
    const uint4* km4 = reinterpret_cast<const uint4*>(km);
#define POPKV_SCORE_LAUNCH_T(Q, W, T)                                                                          \
    hipLaunchKernelGGL((score_d128_kernel<G, Q, QT, W, T>), grid, dim3(kScoreThreads), 0, stream, qs, qm, ql, qd, \
                       q_raw, ks4, km4, kl, kd, h2k, qh, kvh, qpk, cap, tokens, out, out_stride, ghist, seq, win)
#define POPKV_SCORE_LAUNCH(Q, W) POPKV_SCORE_LAUNCH_T(Q, W, TPT)
    // the tile windows: the layer step's G64 scorer with a compile-time group
    constexpr bool kWinG = G == 64 && !std::is_void_v<QT>;
    if (kWinG && win.rec != nullptr) {
        // the tiles the layout chose (step_tile_tokens): 1024 or 512 tokens
        if (win.tile_tokens == kScoreThreads) {
            grid.x = static_cast<unsigned>((tokens + kScoreThreads - 1) / kScoreThreads);
            if (static_cast<int>(grid.x) != win.tiles) return hipErrorInvalidValue;  // one record per tile
            switch (qpk) {
                case 1: POPKV_SCORE_LAUNCH_T(1, kWinG, 1); break;
                case 2: POPKV_SCORE_LAUNCH_T(2, kWinG, 1); break;
                case 4: POPKV_SCORE_LAUNCH_T(4, kWinG, 1); break;
                case 8: POPKV_SCORE_LAUNCH_T(8, kWinG, 1); break;
                default: return hipErrorInvalidValue;
            }
            return hipGetLastError();
        }
        if (win.tile_tokens != per_block || static_cast<int>(grid.x) != win.tiles) return hipErrorInvalidValue;
        switch (qpk) {
            case 1: POPKV_SCORE_LAUNCH(1, kWinG); break;
            case 2: POPKV_SCORE_LAUNCH(2, kWinG); break;
            case 4: POPKV_SCORE_LAUNCH(4, kWinG); break;
            case 8: POPKV_SCORE_LAUNCH(8, kWinG); break;
            default: return hipErrorInvalidValue;
        }
        return hipGetLastError();
    }
    if constexpr (TPT == 2) {
        // fewer two-token workgroups than the chip's 256 CUs (short rows):
        // one token per thread, twice the workgroups
        if (static_cast<int64_t>(grid.x) * grid.y < 256) {
            grid.x = static_cast<unsigned>((tokens + kScoreThreads - 1) / kScoreThreads);
            switch (qpk) {
                case 1: POPKV_SCORE_LAUNCH_T(1, false, 1); break;
                case 2: POPKV_SCORE_LAUNCH_T(2, false, 1); break;
                case 4: POPKV_SCORE_LAUNCH_T(4, false, 1); break;
                case 8: POPKV_SCORE_LAUNCH_T(8, false, 1); break;
                default: POPKV_SCORE_LAUNCH_T(0, false, 1); break;
            }
            return hipGetLastError();
        }
    }
    switch (qpk) {
        case 1: POPKV_SCORE_LAUNCH(1, false); break;
        case 2: POPKV_SCORE_LAUNCH(2, false); break;
        case 4: POPKV_SCORE_LAUNCH(4, false); break;
        case 8: POPKV_SCORE_LAUNCH(8, false); break;
        default: POPKV_SCORE_LAUNCH(0, false); break;
    }
#undef POPKV_SCORE_LAUNCH
#undef POPKV_SCORE_LAUNCH_T
    return hipGetLastError();
}

template <typename QT>
hipError_t launch_score_d128_q(const int32_t* q_sign, const int32_t* q_mag, const float* q_low, const float* q_delta,
                               const QT* q_raw, const int32_t* k_sign, const int32_t* k_mag, const uint16_t* k_low,
                               const uint16_t* k_delta, const int64_t* head_to_kv, int64_t batch, int q_heads,
                               int kv_heads, int64_t capacity, int64_t tokens, int dim_group_size, uint16_t* scores,
                               int64_t score_row_stride, uint32_t* ghist, const SeqTable& seq, hipStream_t stream,
                               const TileWindows& win = TileWindows{}) {
    switch (dim_group_size) {
        case 16:
            return launch_score_d128_g<16, QT>(q_sign, q_mag, q_low, q_delta, q_raw, k_sign, k_mag, k_low, k_delta,
                                               head_to_kv, batch, q_heads, kv_heads, capacity, tokens, scores,
                                               score_row_stride, ghist, seq, stream, win);
        case 32:
            return launch_score_d128_g<32, QT>(q_sign, q_mag, q_low, q_delta, q_raw, k_sign, k_mag, k_low, k_delta,
                                               head_to_kv, batch, q_heads, kv_heads, capacity, tokens, scores,
                                               score_row_stride, ghist, seq, stream, win);
        default:
            return launch_score_d128_g<64, QT>(q_sign, q_mag, q_low, q_delta, q_raw, k_sign, k_mag, k_low, k_delta,
                                               head_to_kv, batch, q_heads, kv_heads, capacity, tokens, scores,
                                               score_row_stride, ghist, seq, stream, win);
    }
}

}  // namespace

hipError_t launch_query_encode(const void* queries, int dtype, int64_t rows, int head_dim, int dim_group_size,
                               int order, int32_t* q_sign, int32_t* q_mag, float* q_low, float* q_delta,
                               hipStream_t stream) {
    if (rows <= 0) return hipSuccess;
    switch (dtype) {
        case POPKV_DTYPE_F32:
            return launch_encode_g(static_cast<const float*>(queries), rows, head_dim, dim_group_size, order, q_sign,
                                   q_mag, q_low, q_delta, stream);
        case POPKV_DTYPE_F16:
            return launch_encode_g(static_cast<const f16_t*>(queries), rows, head_dim, dim_group_size, order, q_sign,
                                   q_mag, q_low, q_delta, stream);
        default:
            return launch_encode_g(static_cast<const bf16_t*>(queries), rows, head_dim, dim_group_size, order,
                                   q_sign, q_mag, q_low, q_delta, stream);
    }
}

hipError_t launch_score_d128(const int32_t* q_sign, const int32_t* q_mag, const float* q_low, const float* q_delta,
                             const int32_t* k_sign, const int32_t* k_mag, const uint16_t* k_low,
                             const uint16_t* k_delta, const int64_t* head_to_kv, int64_t batch, int q_heads,
                             int kv_heads, int64_t capacity, int64_t tokens, int dim_group_size, uint16_t* scores,
                             int64_t score_row_stride, hipStream_t stream) {
    return launch_score_d128_q<void>(q_sign, q_mag, q_low, q_delta, nullptr, k_sign, k_mag, k_low, k_delta,
                                     head_to_kv, batch, q_heads, kv_heads, capacity, tokens, dim_group_size, scores,
                                     score_row_stride, nullptr, SeqTable{}, stream);
}

hipError_t launch_score_d128_raw(const void* queries, int dtype, const int32_t* k_sign, const int32_t* k_mag,
                                 const uint16_t* k_low, const uint16_t* k_delta, const int64_t* head_to_kv,
                                 int64_t batch, int q_heads, int kv_heads, int64_t capacity, int64_t tokens,
                                 int dim_group_size, uint16_t* keys, int64_t key_row_stride, uint32_t* ghist,
                                 const SeqTable& seq, hipStream_t stream, const TileWindows& win) {
    switch (dtype) {
        case POPKV_DTYPE_F32:
            return launch_score_d128_q<float>(nullptr, nullptr, nullptr, nullptr, static_cast<const float*>(queries),
                                              k_sign, k_mag, k_low, k_delta, head_to_kv, batch, q_heads, kv_heads,
                                              capacity, tokens, dim_group_size, keys, key_row_stride, ghist, seq,
                                              stream, win);
        case POPKV_DTYPE_F16:
            return launch_score_d128_q<f16_t>(nullptr, nullptr, nullptr, nullptr, static_cast<const f16_t*>(queries),
                                              k_sign, k_mag, k_low, k_delta, head_to_kv, batch, q_heads, kv_heads,
                                              capacity, tokens, dim_group_size, keys, key_row_stride, ghist, seq,
                                              stream, win);
        default:
            return launch_score_d128_q<bf16_t>(nullptr, nullptr, nullptr, nullptr,
                                               static_cast<const bf16_t*>(queries), k_sign, k_mag, k_low, k_delta,
                                               head_to_kv, batch, q_heads, kv_heads, capacity, tokens, dim_group_size,
                                               keys, key_row_stride, ghist, seq, stream, win);
    }
}

hipError_t launch_score_generic(const int32_t* q_sign, const int32_t* q_mag, const float* q_low,
                                const float* q_delta, const int32_t* k_sign, const int32_t* k_mag,
                                const uint16_t* k_low, const uint16_t* k_delta, const int64_t* head_to_kv,
                                int64_t batch, int q_heads, int kv_heads, int head_dim, int64_t capacity,
                                int64_t tokens, int dim_group_size, float* scores, hipStream_t stream) {
    const float scale = static_cast<float>(1.0 / sqrt(static_cast<double>(head_dim)));
    dim3 grid(static_cast<unsigned>((tokens + 255) / 256), static_cast<unsigned>(batch * q_heads));
    switch (dim_group_size) {
        case 16:
            hipLaunchKernelGGL((score_generic_kernel<16>), grid, dim3(256), 0, stream, q_sign, q_mag, q_low, q_delta,
                               k_sign, k_mag, k_low, k_delta, head_to_kv, q_heads, kv_heads, head_dim, capacity, tokens, scale,
                               scores);
            break;
        case 32:
            hipLaunchKernelGGL((score_generic_kernel<32>), grid, dim3(256), 0, stream, q_sign, q_mag, q_low, q_delta,
                               k_sign, k_mag, k_low, k_delta, head_to_kv, q_heads, kv_heads, head_dim, capacity, tokens, scale,
                               scores);
            break;
        default:
            hipLaunchKernelGGL((score_generic_kernel<64>), grid, dim3(256), 0, stream, q_sign, q_mag, q_low, q_delta,
                               k_sign, k_mag, k_low, k_delta, head_to_kv, q_heads, kv_heads, head_dim, capacity, tokens, scale,
                               scores);
            break;
    }
    return hipGetLastError();
}

}  // namespace popkv
