// The head_dim-128 popcount scorer's device code: the per-representative
// count chain, the in-kernel query encode, the tile windows and the scorer
// body.  score.hip wraps the body in its kernel; the layer step's fused
// kernel (attention.hip) runs it in its first workgroups.
#pragma once

#include <type_traits>

#include "device_common.h"
#include "kernels.h"
#include "select_common.h"

namespace popkv {
namespace {

// Bits of representative r inside 32-bit word w of a 128-bit plane.
template <int G>
__device__ __forceinline__ uint32_t rep_mask(int r, int w) {
    if constexpr (G == 64) return (w / 2 == r) ? 0xffffffffu : 0u;
    else if constexpr (G == 32) return w == r ? 0xffffffffu : 0u;
    else return w == r / 2 ? ((r & 1) ? 0xffff0000u : 0x0000ffffu) : 0u;
}

// popcount of the bits of representative r in a 128-bit plane.
template <int G>
__device__ __forceinline__ int rep_popc(const uint32_t* x, int r) {
    if constexpr (G == 64) return __popc(x[2 * r]) + __popc(x[2 * r + 1]);
    else if constexpr (G == 32) return __popc(x[r]);
    else return __popc(x[r / 2] & rep_mask<16>(r, r / 2));
}

// popc(x) + acc as one v_bcnt_u32_b32 (its accumulate operand).  Written
// out because the compiler re-associates 2 * (popc(x0) + popc(x1)) - p into
// an add-shift and a subtract instead of two accumulating counts and one
// shift-add.
__device__ __forceinline__ int popc_acc(uint32_t x, int acc) {
    int r;
    asm("v_bcnt_u32_b32 %0, %1, %2" : "=v"(r) : "v"(x), "v"(acc));
    return r;
}

// -p, opaque to the compiler, so that 2 * c - p stays one shift-add
// (v_lshl_add_u32) instead of a shift and a subtract.
__device__ __forceinline__ int neg_opaque(int p) {
    int r;
    asm("v_sub_u32 %0, 0, %1" : "=v"(r) : "v"(p));
    return r;
}

// Four signed agreement counts of representative r over its G dims,
// combined with the fp32 chain of the reference:
//   cs  = 2*popc(m) - G,               m = ~(qs ^ ks)
//   cq  = 2*popc(m & qm) - popc(qm)
//   ck  = 2*popc(m & km) - popc(km)
//   cqk = 2*popc(m & qm & km) - popc(qm & km)
// with popc(qm & km) - G counted as popc(~(qm & km)) down from -G, so each
// count is one accumulating popcount per word and one shift-add; cs is
// finished as a float by one fma (see below), the others are converted.
// npq = -popc(query mag bits of r), npk = -popc(key mag bits of r): they
// depend on one side only and are formed once per head / token by the caller.
template <int G>
__device__ __forceinline__ float rep_term(const uint32_t* qs, const uint32_t* qm, const uint32_t* ks,
                                          const uint32_t* km, int r, int npq, int npk, float ql, float dq,
                                          float kl, float dk) {
    constexpr int NW = G == 64 ? 2 : 1;
    const int w0 = G == 64 ? 2 * r : (G == 32 ? r : r / 2);
    // a counts up from the bit pattern of 2^23, so that as a float it reads
    // 2^23 + popc(m) exactly (the count sits in the low mantissa bits)
    int a = 0, aq = 0, ak = 0, aqk = 0, nb = -G;
#pragma unroll
    for (int i = 0; i < NW; ++i) {
        const int w = w0 + i;
        const uint32_t sel = G == 16 ? rep_mask<16>(r, w) : 0xffffffffu;
        const uint32_t m = ~(qs[w] ^ ks[w]) & sel;
        if (i == 0) {
            a = popc_acc(m, 0x4b000000);
            aq = __popc(m & qm[w]);
            ak = __popc(m & km[w]);
            aqk = __popc(m & qm[w] & km[w]);
        } else {
            a = popc_acc(m, a);
            aq = popc_acc(m & qm[w], aq);
            ak = popc_acc(m & km[w], ak);
            aqk = popc_acc(m & qm[w] & km[w], aqk);
        }
        nb = popc_acc(~(qm[w] & km[w]) & sel, nb);  // popc(~both) - G = -popc(both)
    }
    // cs = 2 popc(m) - G as a float: 2 (2^23 + popc) - (2^24 + G) in one fma,
    // exact (both operands are exact and so is the small integer result, +0
    // for 0) -- the count's add-shift and conversion in one instruction
    const float cs = fmaf(__int_as_float(a), 2.0f, -(16777216.0f + static_cast<float>(G)));
    const int cq = 2 * aq + npq, ck = 2 * ak + npk, cqk = 2 * aqk + nb;
    return fmaf(ql * kl, cs,
                fmaf(dq * kl, static_cast<float>(cq),
                     fmaf(ql * dk, static_cast<float>(ck), dq * dk * static_cast<float>(cqk))));
}

constexpr int kScoreThreads = 512;  // 8 waves: 1024 tokens x one GQA group per workgroup
// Tokens per thread: two for G64 (its per-token work is short, so the
// per-head state reads and the in-kernel encode are amortised over more
// tokens), one for G32 / G16 (longer per-token work: more waves hide it
// better).  Measured at 32K tokens: G64 7.4 vs 7.6 us, G32 8.4 vs 8.5 us,
// G16 11.6 vs 12.4 us (again with the fma-finished count: the C2 layer step
// 29.1 vs 30.2 us, two tokens taking 160 VGPRs).  Short G64 rows, whose
// two-token tiles would leave CUs without a scorer workgroup, take one token
// per thread (the launchers' choice): C3 8K step 21.4 vs 20.3 us, C3 16K
// single launch 23.3 vs 21.3 us.
template <int G> constexpr int score_tokens_per_thread() { return G == 64 ? 2 : 1; }
constexpr int kMaxGroupHeads = 64;  // query heads per KV head the LDS stage holds

// Query state of one head, contiguous in LDS (the scorer reads a head's
// whole state from one base address with 16-byte reads).
template <int G>
struct __align__(16) HeadState {
    uint32_t qs[4], qm[4];
    float ql[128 / G], qd[128 / G];
    int npq[128 / G];  // -(magnitude bits of representative r)
};

// Query state of one GQA group in LDS.
template <int G>
struct GroupState {
    HeadState<G> h[kMaxGroupHeads];
};

// Encodes the group's query rows (head_dim 128) into `st` in the
// decode-path order.  Wave w handles heads w, w+4, ...; the caller has
// already loaded dims lane and lane+64 of those rows into qv[][2] (so the
// query loads are issued ahead of the token loads).  Each wave forms the
// whole-head extrema, the sign/magnitude words and, for every dimension, its
// contribution to the low and to the high bucket (|q| or +0), staged in LDS.
// Two threads per (head, representative) then run the two
// ascending-dimension fp32 add chains over those contributions, one each --
// adding +0 for the other bucket is exact, so this is the reference's fold --
// and the bucket counts are popcounts of the magnitude words.  All threads of
// the block call it.
template <int G, int MAXW>
__device__ __forceinline__ void encode_group_fold(const float (*qv)[2], int qpk, GroupState<G>& st,
                                                  float (*lo_c)[128], float (*hi_c)[128]) {
    constexpr int R = 128 / G;
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
#pragma unroll
    for (int i = 0; i < MAXW; ++i) {
        const int h = wave + i * (kScoreThreads / kWave);
        if (h >= qpk) break;
        const float v0 = qv[i][0], v1 = qv[i][1];
        const float mn = wave_extreme<false>(fminf(v0, v1)), mx = wave_extreme<true>(fmaxf(v0, v1));
        const float neg = mn * 0.5f, pos = mx * 0.5f;
        const bool s0 = v0 >= 0.0f, s1 = v1 >= 0.0f;
        const bool m0 = s0 ? v0 > pos : v0 < neg, m1 = s1 ? v1 > pos : v1 < neg;
        const float a0 = fabsf(v0), a1 = fabsf(v1);
        lo_c[h][lane] = m0 ? 0.0f : a0;
        hi_c[h][lane] = m0 ? a0 : 0.0f;
        lo_c[h][lane + 64] = m1 ? 0.0f : a1;
        hi_c[h][lane + 64] = m1 ? a1 : 0.0f;
        const uint64_t bs0 = __ballot(s0), bs1 = __ballot(s1), bm0 = __ballot(m0), bm1 = __ballot(m1);
        if (lane == 0) {
            st.h[h].qs[0] = static_cast<uint32_t>(bs0); st.h[h].qs[1] = static_cast<uint32_t>(bs0 >> 32);
            st.h[h].qs[2] = static_cast<uint32_t>(bs1); st.h[h].qs[3] = static_cast<uint32_t>(bs1 >> 32);
            st.h[h].qm[0] = static_cast<uint32_t>(bm0); st.h[h].qm[1] = static_cast<uint32_t>(bm0 >> 32);
            st.h[h].qm[2] = static_cast<uint32_t>(bm1); st.h[h].qm[3] = static_cast<uint32_t>(bm1 >> 32);
        }
    }
    __syncthreads();
    // two threads per (head, rep): the even one runs the low-bucket chain,
    // the odd one the high-bucket chain (an even item count, so a pair is
    // always active together), then the even one finishes the rep
    for (int item = threadIdx.x; item < 2 * qpk * R; item += kScoreThreads) {
        const int hr = item >> 1, h = hr / R, r = hr % R;
        const float* src = (item & 1) ? &hi_c[h][r * G] : &lo_c[h][r * G];
        float sum = 0.0f;
        // a partial unroll: fully unrolled, the compiler loads all G
        // contributions before the (sequential) add chain, which takes G
        // registers and caps the scorer's occupancy
#pragma unroll 4
        for (int j = 0; j < G; j += 4) {
            const float4 v = *reinterpret_cast<const float4*>(src + j);
            sum = sum + v.x; sum = sum + v.y; sum = sum + v.z; sum = sum + v.w;
        }
        const float hs = __shfl_xor(sum, 1);
        if ((item & 1) == 0) {
            // high-bucket count: popcount of the G magnitude bits at r*G
            int hn = 0;
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                if ((w + 1) * 32 <= r * G || w * 32 >= (r + 1) * G) continue;
                uint32_t bits = st.h[h].qm[w];
                if constexpr (G == 16) bits = (r & 1) ? (bits >> 16) : (bits & 0xffffu);
                hn += __popc(bits);
            }
            finish_rep(sum, G - hn, hs, hn, st.h[h].ql[r], st.h[h].qd[r]);
            st.h[h].npq[r] = -hn;
        }
    }
    __syncthreads();
}

// Copies a pre-encoded group state from global memory into `st`.
template <int G>
__device__ void load_group_state(const int32_t* __restrict__ q_sign, const int32_t* __restrict__ q_mag,
                                 const float* __restrict__ q_low, const float* __restrict__ q_delta,
                                 int64_t qrow0, int qpk, GroupState<G>& st) {
    constexpr int R = 128 / G;
    for (int i = threadIdx.x; i < qpk * 4; i += kScoreThreads) {
        st.h[i / 4].qs[i % 4] = static_cast<uint32_t>(q_sign[qrow0 * 4 + i]);
        st.h[i / 4].qm[i % 4] = static_cast<uint32_t>(q_mag[qrow0 * 4 + i]);
    }
    for (int i = threadIdx.x; i < qpk * R; i += kScoreThreads) {
        st.h[i / R].ql[i % R] = q_low[qrow0 * R + i];
        st.h[i / R].qd[i % R] = q_delta[qrow0 * R + i];
        uint32_t qm[4];
#pragma unroll
        for (int w = 0; w < 4; ++w) qm[w] = static_cast<uint32_t>(q_mag[(qrow0 + i / R) * 4 + w]);
        st.h[i / R].npq[i % R] = -rep_popc<G>(qm, i % R);
    }
    __syncthreads();
}

static_assert(kScoreThreads * score_tokens_per_thread<64>() == 1024 &&
                  kScoreThreads * score_tokens_per_thread<16>() == 512 &&
                  kScoreThreads * score_tokens_per_thread<32>() == 512,
              "score_tile_tokens() states the scorer's tile");

// The tile windows of one scorer workgroup (tile `tile` of rows
// qrow0 .. qrow0 + QPK - 1, the row's sequence holding ntok tokens of which
// k are selected): wave h estimates row h's threshold bin from the tile's
// histogram s_hist[h] and writes the window record (COH: as a
// device-coherent store), then every thread adds its keys that fall in
// their row's window to the window histograms in LDS (s_win, byte counts,
// zero on entry; the caller writes them out).  A row that selects none or every token gets
// base 256 (no window; its select never reads it).  All threads of the
// block call it, after a barrier that completes s_hist and s_keys.
template <int QPK, int TILE, bool COH>
__device__ __forceinline__ void tile_windows(const uint32_t (*s_hist)[256], const uint16_t (*s_keys)[TILE],
                                             uint32_t (*s_win)[kWinBins][64], uint32_t* s_base,
                                             const TileWindows& win, int64_t qrow0, int64_t ntok, int64_t k,
                                             uint32_t tile) {
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int64_t t_lo = static_cast<int64_t>(tile) * TILE;
    const int64_t n_i = min(max(ntok - t_lo, static_cast<int64_t>(0)), static_cast<int64_t>(TILE));
    if (wave < QPK) {
        uint32_t base = 256u, above = 0u, t01 = 0u, t23 = 0u;
        if (n_i > 0 && k > 0 && k < ntok) {  // uniform
            uint32_t cnt[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) cnt[i] = s_hist[wave][255 - (4 * lane + i)];
            // the tile's share of the selection, about k * n_i / ntok, in
            // [1, n_i] (a single-precision estimate: the window only has to
            // be centred near the threshold, any centre is correct)
            const float share = static_cast<float>(k) * static_cast<float>(n_i) *
                                __builtin_amdgcn_rcpf(static_cast<float>(ntok));
            const uint32_t need = static_cast<uint32_t>(
                min(max(__builtin_ceilf(share), 1.0f), static_cast<float>(n_i)));
            uint32_t est, est_above;
            wave_find_bin(cnt, need, &est, &est_above);
            base = min(max(est, static_cast<uint32_t>(kWinBelow + 1)) - kWinBelow, static_cast<uint32_t>(256 - kWinBins));
            uint32_t part = 0u;
#pragma unroll
            for (int i = 0; i < 4; ++i) part += 255u - static_cast<uint32_t>(4 * lane + i) >= base + kWinBins ? cnt[i] : 0u;
            above = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(wave_incl_scan(part, lane)), kWave - 1));
            t01 = s_hist[wave][base] | (s_hist[wave][base + 1] << 16);
            t23 = s_hist[wave][base + 2] | (s_hist[wave][base + 3] << 16);
        }
        if (lane == 0) {
            s_base[wave] = base;
            uint4* dst = win.rec + (qrow0 + wave) * win.tiles + tile;
            if constexpr (COH) st_coh_u4(dst, make_uint4(base, above, t01, t23));
            else *dst = make_uint4(base, above, t01, t23);
        }
    }
    __syncthreads();
    // every key of this thread first (the reads would otherwise wait for
    // the atomics before them), then the atomics
    constexpr int PER = TILE / kScoreThreads;
    uint32_t kv[QPK][PER], bs[QPK];
#pragma unroll
    for (int h = 0; h < QPK; ++h) {
        bs[h] = s_base[h];
#pragma unroll
        for (int e = 0; e < PER; ++e) kv[h][e] = s_keys[h][e * kScoreThreads + threadIdx.x];
    }
#pragma unroll
    for (int h = 0; h < QPK; ++h) {
#pragma unroll
        for (int e = 0; e < PER; ++e) {
            const uint32_t key = kv[h][e];
            const uint32_t d = (key >> 8) - bs[h];  // wraps for keys below the window
            if (d < static_cast<uint32_t>(kWinBins)) atomicAdd(&s_win[h][d][(key & 0xffu) >> 2], 1u << ((key & 3u) * 8));
        }
    }
    __syncthreads();
}

// The scorer's workgroup: token tile `tile` (of kScoreThreads *
// score_tokens_per_thread<G>() tokens) of block row `grow` (sequence, KV
// group slot; batch * kv_heads rows).  QT is the raw query type when the
// kernel encodes the query itself (layer step), void when it reads a
// pre-encoded state.  HANDOFF (the layer step's single-launch form, with the
// tile windows): the select + attention workgroups of the same launch read
// what this workgroup writes, so its keys, window histograms and records go
// out with device-coherent stores, every wave waits until its stores are
// acknowledged (vmcnt(0), which on gfx942 / gfx950 covers stores), the block
// meets at a barrier, and only then are the histogram counts added into
// ghist (device-scope atomics).  A row's histogram therefore sums to its
// token count only once every tile's other outputs have reached the
// coherence point; the select polls for that sum.
template <int G, int QPK, typename QT, bool WIN, bool HANDOFF, int TPT = score_tokens_per_thread<G>()>
__device__ __forceinline__ void score_d128_body(
    const int32_t* __restrict__ q_sign, const int32_t* __restrict__ q_mag,
    const float* __restrict__ q_low, const float* __restrict__ q_delta, const QT* __restrict__ q_raw,
    const uint4* __restrict__ k_sign, const uint4* __restrict__ k_mag,
    const uint16_t* __restrict__ k_low, const uint16_t* __restrict__ k_delta,
    const int64_t* __restrict__ head_to_kv, int q_heads, int kv_heads, int qpk_rt,
    int64_t cap, int64_t tokens, uint16_t* __restrict__ scores, int64_t out_stride,
    uint32_t* __restrict__ ghist, SeqTable seq, TileWindows win, uint32_t tile, uint32_t grow_u) {
    constexpr int R = 128 / G;
    static_assert(!HANDOFF || (WIN && !std::is_void_v<QT> && QPK > 0), "the hand-off: the layer step's window form");
    // Layer-step mode (the kernel encodes the raw query): the output holds the
    // scores' radix order keys instead of fp16 bits, and the per-head 256-bin
    // histogram of the keys' high byte is accumulated into ghist[row][256]
    // for the select kernel.
    constexpr bool STEP = !std::is_void_v<QT>;
    args_in_sgprs(head_to_kv, k_sign, k_mag, k_low, k_delta, q_heads, kv_heads, qpk_rt, cap, tokens, seq.tokens,
                  seq.cache_rows);
    if constexpr (STEP) args_in_sgprs(q_raw);
    const int qpk = QPK > 0 ? QPK : qpk_rt;
    // block row (sequence b, KV group slot): 32-bit arithmetic, the row
    // count being below 2^31
    const int grow = static_cast<int>(grow_u);
    const int bi = div_nonneg(grow, kv_heads);
    const int slot = grow - bi * kv_heads;
    const int64_t b = bi;
    const int64_t qh0 = static_cast<int64_t>(slot) * qpk;
    const int64_t qrow0 = b * q_heads + qh0;

    // Loads, in issue order (they retire in that order, vmcnt): the raw
    // query values the encode needs; the group's KV mapping and (batched)
    // the sequence's token count, as vector loads at a lane-opaque zero
    // offset (as scalar loads their wait would also hold back the query
    // loads); then this thread's token rows at the KV head the mapping
    // names for the standard grouping, head_to_kv[qh0] = slot, so that
    // their latency overlaps the encode.  Once the mapping has arrived, a
    // group that maps elsewhere (clamped into [0, kv_heads), never
    // dereferenced outside) loads its rows again.
    constexpr int MAXW = QPK > 0 ? (QPK + kScoreThreads / kWave - 1) / (kScoreThreads / kWave)
                                 : kMaxGroupHeads / (kScoreThreads / kWave);
    float qv[std::is_void_v<QT> ? 1 : MAXW][2];
    if constexpr (!std::is_void_v<QT>) {
        const int lane = threadIdx.x & (kWave - 1);
        const int wave = threadIdx.x / kWave;
#pragma unroll
        for (int i = 0; i < MAXW; ++i) {
            const int h = min(wave + i * (kScoreThreads / kWave), qpk - 1);
            const QT* src = q_raw + (qrow0 + h) * 128;
            qv[i][0] = Elem<QT>::load(src, lane);
            qv[i][1] = Elem<QT>::load(src, lane + 64);
        }
    }
    int z = 0;
    asm volatile("" : "+v"(z));
    const int64_t map_v = head_to_kv[qh0 + z];
    const int64_t ntok_v = seq.tokens != nullptr ? seq.tokens[b + z] : tokens;
    static_assert(TPT == 1 || TPT == 2, "one or two tokens per thread");
    using RepWord = std::conditional_t<R == 2, uint32_t, std::conditional_t<R == 4, uint2, uint4>>;
    uint4 s4[TPT], m4[TPT];
    RepWord lw[TPT], dw[TPT];
    int64_t tok[TPT];
    // packed rows of KV head kvh (a batched step gives each sequence its own
    // cache; the reference's batch shares one); the loads stay within the
    // launch bound `tokens`, the stores below within the sequence's count
    auto load_tokens = [&](int64_t kvh) {
        const int64_t cbase = b * seq.cache_rows + kvh * cap;
#pragma unroll
        for (int it = 0; it < TPT; ++it) {
            const int64_t krow = cbase + min(tok[it], tokens - 1);
            s4[it] = k_sign[krow];
            m4[it] = k_mag[krow];
            lw[it] = reinterpret_cast<const RepWord*>(k_low)[krow];
            dw[it] = reinterpret_cast<const RepWord*>(k_delta)[krow];
        }
    };
#pragma unroll
    for (int it = 0; it < TPT; ++it) tok[it] = (static_cast<int64_t>(tile) * TPT + it) * kScoreThreads + threadIdx.x;
    load_tokens(slot);

    __shared__ GroupState<G> st;
    __shared__ uint32_t s_hist[STEP ? (QPK > 0 ? QPK : kMaxGroupHeads) : 1][256];
    // tile windows (layer step, compile-time group size; a separate
    // instantiation, so the plain scorer keeps its register count -- 79
    // VGPRs at G64, three workgroups per CU at C4 instead of two): every key
    // of the tile, and the windows' low-byte histograms (byte counts)
    constexpr bool WINK = WIN && STEP && QPK > 0;
    constexpr int TILE = kScoreThreads * TPT;
    __shared__ uint16_t s_keys[WINK ? QPK : 1][WINK ? TILE : 2];
    __shared__ uint32_t s_win[WINK ? QPK : 1][kWinBins][64];
    __shared__ uint32_t s_base[WINK ? QPK : 1];
    const bool win_on = WINK && win.rec != nullptr;
    if constexpr (STEP) {
        for (int i = threadIdx.x; i < qpk * 256; i += kScoreThreads) (&s_hist[0][0])[i] = 0u;
    }
    if constexpr (WINK) {
        if (win_on) {
            for (int i = threadIdx.x; i < QPK * TILE / 2; i += kScoreThreads)
                reinterpret_cast<uint32_t*>(&s_keys[0][0])[i] = 0u;
            for (int i = threadIdx.x; i < QPK * kWinBins * 64; i += kScoreThreads) (&s_win[0][0][0])[i] = 0u;
        }
    }
    if constexpr (std::is_void_v<QT>) {
        load_group_state<G>(q_sign, q_mag, q_low, q_delta, qrow0, qpk, st);
    } else {
        __shared__ __align__(16) float lo_c[QPK > 0 ? QPK : kMaxGroupHeads][128];
        __shared__ __align__(16) float hi_c[QPK > 0 ? QPK : kMaxGroupHeads][128];
        encode_group_fold<G, MAXW>(qv, qpk, st, lo_c, hi_c);
    }
    {
        const int m = __builtin_amdgcn_readfirstlane(static_cast<int>(min(max(map_v, static_cast<int64_t>(0)),
                                                                          static_cast<int64_t>(kv_heads - 1))));
        if (m != slot) load_tokens(m);
    }
    const int64_t ntok_b = min(max(ntok_v, static_cast<int64_t>(0)), tokens);

    // Token-side operands, decoded once and reused for every head.
    uint32_t ks[TPT][4], km[TPT][4];
    float kl[TPT][R], dk[TPT][R];
    int npk[TPT][R];
#pragma unroll
    for (int it = 0; it < TPT; ++it) {
        ks[it][0] = s4[it].x; ks[it][1] = s4[it].y; ks[it][2] = s4[it].z; ks[it][3] = s4[it].w;
        km[it][0] = m4[it].x; km[it][1] = m4[it].y; km[it][2] = m4[it].z; km[it][3] = m4[it].w;
        uint32_t lws[R / 2], dws[R / 2];
        if constexpr (R == 2) {
            lws[0] = lw[it]; dws[0] = dw[it];
        } else if constexpr (R == 4) {
            lws[0] = lw[it].x; lws[1] = lw[it].y; dws[0] = dw[it].x; dws[1] = dw[it].y;
        } else {
            lws[0] = lw[it].x; lws[1] = lw[it].y; lws[2] = lw[it].z; lws[3] = lw[it].w;
            dws[0] = dw[it].x; dws[1] = dw[it].y; dws[2] = dw[it].z; dws[3] = dw[it].w;
        }
#pragma unroll
        for (int i = 0; i < R / 2; ++i) {
            kl[it][2 * i] = bits_f16(lws[i] & 0xffffu); kl[it][2 * i + 1] = bits_f16(lws[i] >> 16);
            dk[it][2 * i] = bits_f16(dws[i] & 0xffffu); dk[it][2 * i + 1] = bits_f16(dws[i] >> 16);
        }
#pragma unroll
        for (int r = 0; r < R; ++r) npk[it][r] = neg_opaque(rep_popc<G>(km[it], r));
    }
    for (int h = 0; h < qpk; ++h) {
        // The group state is uniform but stays in vector registers (plain LDS
        // broadcast reads): a three-operand bit op on the two query planes
        // and a key plane may read only one scalar register, so scalar
        // copies would cost a move per use.
        uint32_t qs[4], qm[4];
        float ql[R], dq[R];
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            qs[w] = st.h[h].qs[w];
            qm[w] = st.h[h].qm[w];
        }
        int npq[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            ql[r] = st.h[h].ql[r];
            dq[r] = st.h[h].qd[r];
            npq[r] = st.h[h].npq[r];
        }
        uint16_t* srow = scores + (qrow0 + h) * out_stride;
        // every token's score first, without a branch (a token past the end
        // scores the clamped last row and is not stored), so the tokens'
        // independent chains interleave
        float scs[TPT];
#pragma unroll
        for (int it = 0; it < TPT; ++it) {
            float total = 0.0f;
#pragma unroll
            for (int r = 0; r < R; ++r) total = total + rep_term<G>(qs, qm, ks[it], km[it], r, npq[r], npk[it][r], ql[r], dq[r],
                                                           kl[it][r], dk[it][r]);
            scs[it] = total * 0x1.6a09e6p-4f;  // fp32(1/sqrt(128)) = 0x3DB504F3
        }
#pragma unroll
        for (int it = 0; it < TPT; ++it) {
            const int64_t t = tok[it];
            if (t >= ntok_b) break;
            const float sc = scs[it];
            const uint16_t bits = f16_rne(sc);
            // byte offset as 32 bits (tokens < 2^31): the store then takes the
            // row base from scalar registers and this offset from one VGPR
            const uint32_t off = 2u * static_cast<uint32_t>(t);
            uint16_t* dst = reinterpret_cast<uint16_t*>(reinterpret_cast<char*>(srow) + off);
            if constexpr (STEP) {
                // order_key(bits): b ^ (s | 0x8000) with s = bit 15
                // sign-extended -- every bit flips for a negative value, only
                // bit 15 for a non-negative one; the bits above 15 are left
                // as garbage (the store keeps 16 bits, the histogram takes
                // bits 8..15).  The NaN test is done on the fp32 value (an
                // fp32 NaN is exactly an fp16 NaN after the conversion).
                const uint32_t b = bits;
                const uint32_t sgn = static_cast<uint32_t>(__builtin_amdgcn_sbfe(static_cast<int32_t>(b), 15, 1));
                const uint32_t key = sc != sc ? 0xffffu : b ^ (sgn | 0x8000u);
                // written through to memory (a device-coherent store): the
                // kernel then ends with little dirty data in L2, and its
                // end-of-kernel write-back is shorter (C1 step 28.2 -> 27.7 us)
                __hip_atomic_store(dst, static_cast<uint16_t>(key), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                atomicAdd(&s_hist[h][(key >> 8) & 0xffu], 1u);
                if constexpr (WINK) {
                    if (win_on) s_keys[h][it * kScoreThreads + threadIdx.x] = static_cast<uint16_t>(key);
                }
            } else {
                *dst = bits;
            }
        }
    }
    if constexpr (STEP) {
        __syncthreads();
        // the tile windows' LDS work first, then every global write of the
        // epilogue together (the histogram atomics would otherwise hold the
        // windows' LDS work back behind their issue)
        if constexpr (WINK) {
            if (win_on) tile_windows<QPK, TILE, HANDOFF>(s_hist, s_keys, s_win, s_base, win, qrow0, ntok_b,
                                                         seq.tokens != nullptr
                                                             ? min(static_cast<int64_t>(seq.budget) - 1, ntok_b)
                                                             : static_cast<int64_t>(win.k),
                                                         tile);
        }
        auto flush_hist = [&]() {
            for (int i = threadIdx.x; i < qpk * 256; i += kScoreThreads) {
                const uint32_t c = (&s_hist[0][0])[i];
                if (c != 0u) atomicAdd(&ghist[(qrow0 + i / 256) * 256 + (i & 255)], c);
            }
        };
        auto store_windows = [&]() {
            for (int i = threadIdx.x; i < QPK * kWinBins * 16; i += kScoreThreads) {
                const int h = i / (kWinBins * 16), r = i - h * (kWinBins * 16);
                const uint4 v = reinterpret_cast<const uint4*>(&s_win[h][0][0])[r];
                uint4* dst = reinterpret_cast<uint4*>(win.bins + ((qrow0 + h) * win.tiles + tile) * (kWinBins * 64)) + r;
                if constexpr (HANDOFF) st_coh_u4(dst, v);
                else *dst = v;
            }
        };
        if constexpr (HANDOFF) {
            // the hand-off (see above): windows out, every store of the block
            // acknowledged, then the histogram counts
            if (win_on) store_windows();
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            __syncthreads();
            flush_hist();
        } else {
            flush_hist();
            if constexpr (WINK) {
                if (win_on) store_windows();
            }
        }
    }
}

}  // namespace
}  // namespace popkv
