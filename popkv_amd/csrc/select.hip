// Per-query-head top-k over PopKV scores with the current token reserving the
// last slot (gfx950).
//
// Replaces torch.topk(scores, k, dim=-1, sorted=False).indices followed by
// _append_current (reference popkv.py:1094-1098, :287-291).
//
// Keys are PyTorch's radix order of an fp16 bit pattern: negatives
// bit-inverted, non-negatives with the sign bit set, NaN largest, so
// -0 < +0.  Selection = every key > T plus the lowest-index keys == T, T the
// k-th largest key (PyTorch's gather-top-k tie rule).
//
// API path: key_hist_kernel turns fp16 scores into order keys and
// accumulates each row's 256-bin histogram of the keys' high byte;
// topk_list_kernel then finds T from that histogram plus one low-byte
// histogram and writes the selected tokens in ascending order (one
// workgroup per row).
//
// Layer step (whose scorer writes the order keys and the high-byte
// histograms itself): chunk_hist_kernel, one workgroup per (chunk, row),
// writes each chunk's low-byte histogram of the threshold's high-byte bin;
// the fused select + attention kernel (attention.hip) then derives T per
// chunk and selects and attends in the same workgroup.
#include <type_traits>

#include "device_common.h"
#include "kernels.h"
#include "select_common.h"

namespace popkv {
namespace {

constexpr int kSelThreads = 1024;
constexpr int kSelWaves = kSelThreads / kWave;
constexpr int kBins = 256;  // one byte of the key per level

// Finds the bin holding the `need`-th largest element of histogram `hist`
// (NB bins, 1 <= need <= total) with one wave: lane l sums the NB/64 bins of
// ranks [l*PER, l*PER + PER) counted from the top, one DPP wave scan, and the
// lane holding the crossing rank writes the bin and the count strictly above
// it.  Called by the whole first wave of the block (no barrier inside).
template <int NB>
__device__ __forceinline__ void find_bin(const uint32_t* hist, uint32_t need, uint32_t* s_bin, uint32_t* s_above) {
    constexpr int PER = NB / kWave;
    const int lane = threadIdx.x & (kWave - 1);
    uint32_t c[PER], local = 0;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        c[i] = hist[NB - 1 - (lane * PER + i)];
        local += c[i];
    }
    uint32_t running = wave_incl_scan(local, lane) - local;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        if (running < need && running + c[i] >= need) {
            *s_bin = static_cast<uint32_t>(NB - 1 - (lane * PER + i));
            *s_above = running;
        }
        running += c[i];
    }
}

// fp16 scores -> order keys in rows of key_stride (a multiple of 128 keys),
// plus each row's high-byte histogram added into ghist[row][256].  Block
// (row, c) covers tokens [256 TPT c, 256 TPT (c + 1)), TPT per thread;
// VEC: the rows are 16-byte aligned and read with 16-byte loads.  Peaked
// scores put many keys in a few bins, so the block's LDS histogram takes
// some same-address atomics; its non-zero bins are then added to ghist.
// WIN (TPT 8: 2048-token blocks): the block's tokens are a tile of the
// chunked select that follows, and the block also writes the tile's window
// (ApiWindows) from its histogram -- the API path's counterpart of the
// layer-step scorer's tile windows.  (Two 2048-token tiles per block of 16
// tokens per thread measured slower: 6.8 against 5.5 us at 32 x 32767.)
constexpr int kKeyHistThreads = 256;
constexpr int kKeyHistTokens = 16;                  // per thread
constexpr int kApiTileTokens = kKeyHistThreads * 8;  // the window form's tile: 2048 tokens

// Tile windows of the API select: for tile i of row r (2048 tokens) the
// tile's estimate e of the row's threshold bin b1 -- the bin where the
// tile's count from the top reaches its share ceil(k * n_i / tokens) of the
// selection -- gives a window of kWinBins bins base = e - kWinBelow .. base
// + kWinBins - 1 (clamped to [0, 256)); rec[r][i] = {base, keys above the
// window, the 4 bins' counts as 16-bit pairs} and bins[r][i][w][128] the
// low-byte histogram of window bin w (16-bit pairs).  base = 256: no window.
struct ApiWindows {
    uint4* rec = nullptr;
    uint32_t* bins = nullptr;
    int tiles = 0;
    int64_t k = 0;
};

template <bool VEC, int TPT, bool WIN>
__global__ __launch_bounds__(kKeyHistThreads) void key_hist_kernel(const uint16_t* __restrict__ scores,
                                                                   int64_t row_stride, int64_t tokens, int chunks,
                                                                   uint16_t* __restrict__ keys, int64_t key_stride,
                                                                   uint32_t* __restrict__ ghist, ApiWindows win) {
    static_assert(TPT == 8 || TPT == 16, "8 or 16 tokens per thread");
    static_assert(!WIN || TPT * kKeyHistThreads == kApiTileTokens, "the window form's tile");
    constexpr int NW = TPT / 2;  // 32-bit words of keys per thread
    const int64_t row = blockIdx.x / chunks;
    const int tile = static_cast<int>(blockIdx.x % chunks);
    const int64_t t0 = (static_cast<int64_t>(tile) * kKeyHistThreads + threadIdx.x) * TPT;
    __shared__ uint32_t s_hist[kBins];
    __shared__ uint32_t s_win[WIN ? kWinBins : 1][128];
    __shared__ uint32_t s_base;
    s_hist[threadIdx.x] = 0u;
    if constexpr (WIN) {
        for (int i = threadIdx.x; i < kWinBins * 128; i += kKeyHistThreads) (&s_win[0][0])[i] = 0u;
    }
    __syncthreads();
    uint32_t kw[NW];
#pragma unroll
    for (int i = 0; i < NW; ++i) kw[i] = 0u;
    if (t0 < tokens) {
        const uint16_t* src = scores + row * row_stride + t0;
        uint32_t w[NW];
        if (VEC && t0 + TPT <= tokens) {
#pragma unroll
            for (int b = 0; b < TPT / 8; ++b) {
                const uint4 a = reinterpret_cast<const uint4*>(src)[b];
                w[4 * b] = a.x; w[4 * b + 1] = a.y; w[4 * b + 2] = a.z; w[4 * b + 3] = a.w;
            }
        } else if (!VEC && t0 + TPT <= tokens) {
            // a row that is not 16-byte aligned (an odd row stride): the 16-byte
            // blocks holding the thread's 2 * TPT bytes (TPT / 8 when the row is
            // aligned, else one more; each holds at least one of those bytes,
            // so none reaches past the scores' own 16-byte blocks), then the
            // 16-bit shift and the word offset of the row's misalignment,
            // uniform over the block
            const uintptr_t addr = reinterpret_cast<uintptr_t>(src);
            const uint32_t mis = static_cast<uint32_t>(addr & 15u);  // even
            const uint4* blk = reinterpret_cast<const uint4*>(addr - mis);
            uint32_t x[NW + 4];
#pragma unroll
            for (int b = 0; b <= TPT / 8; ++b) {
                const uint4 a = b < TPT / 8 || mis != 0u ? blk[b] : make_uint4(0u, 0u, 0u, 0u);
                x[4 * b] = a.x; x[4 * b + 1] = a.y; x[4 * b + 2] = a.z; x[4 * b + 3] = a.w;
            }
            const uint32_t sh = mis & 3u;  // 0 or 2 bytes
            auto take = [&](auto qc) {
                constexpr int q = decltype(qc)::value;
#pragma unroll
                for (int i = 0; i < NW; ++i) w[i] = __builtin_amdgcn_alignbyte(x[q + i + 1], x[q + i], sh);
            };
            switch (mis >> 2) {
                case 0: take(std::integral_constant<int, 0>{}); break;
                case 1: take(std::integral_constant<int, 1>{}); break;
                case 2: take(std::integral_constant<int, 2>{}); break;
                default: take(std::integral_constant<int, 3>{}); break;
            }
        } else {
            // element loads, all issued before use (indices past the row's
            // end re-read its last element and are not counted below)
            const int64_t last = tokens - 1 - t0;
            uint32_t e[TPT];
#pragma unroll
            for (int i = 0; i < TPT; ++i) e[i] = src[min(static_cast<int64_t>(i), last)];
#pragma unroll
            for (int i = 0; i < NW; ++i) w[i] = e[2 * i] | (e[2 * i + 1] << 16);
        }
#pragma unroll
        for (int i = 0; i < NW; ++i) {
            const uint32_t k0 = order_key(w[i] & 0xffffu), k1 = order_key(w[i] >> 16);
            if (t0 + 2 * i < tokens) atomicAdd(&s_hist[k0 >> 8], 1u);
            if (t0 + 2 * i + 1 < tokens) atomicAdd(&s_hist[k1 >> 8], 1u);
            kw[i] = k0 | (k1 << 16);
        }
        // t0 + TPT <= key_stride: the key rows are padded to 128 keys
        uint4* dst = reinterpret_cast<uint4*>(keys + row * key_stride + t0);
#pragma unroll
        for (int b = 0; b < TPT / 8; ++b) dst[b] = make_uint4(kw[4 * b], kw[4 * b + 1], kw[4 * b + 2], kw[4 * b + 3]);
    }
    __syncthreads();
    if constexpr (WIN) {
        const int lane = threadIdx.x & (kWave - 1);
        const int64_t n_i = min(max(tokens - static_cast<int64_t>(tile) * kApiTileTokens, static_cast<int64_t>(0)),
                                static_cast<int64_t>(kApiTileTokens));
        if (threadIdx.x < kWave) {
            uint32_t base = 256u, above = 0u, t01 = 0u, t23 = 0u;
            if (n_i > 0 && win.k > 0 && win.k < tokens) {  // uniform
                uint32_t cnt[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) cnt[i] = s_hist[255 - (4 * lane + i)];
                // the tile's share of the selection, about k * n_i / tokens,
                // in [1, n_i] (a single-precision estimate: the window only
                // has to be centred near the threshold, any centre is correct)
                const float share = static_cast<float>(win.k) * static_cast<float>(n_i) *
                                    __builtin_amdgcn_rcpf(static_cast<float>(tokens));
                const uint32_t need = static_cast<uint32_t>(
                    min(max(__builtin_ceilf(share), 1.0f), static_cast<float>(n_i)));
                uint32_t est, est_above;
                wave_find_bin(cnt, need, &est, &est_above);
                base = min(max(est, static_cast<uint32_t>(kWinBelow + 1)) - kWinBelow,
                           static_cast<uint32_t>(256 - kWinBins));
                uint32_t part = 0u;
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    part += 255u - static_cast<uint32_t>(4 * lane + i) >= base + kWinBins ? cnt[i] : 0u;
                above = static_cast<uint32_t>(
                    __builtin_amdgcn_readlane(static_cast<int>(wave_incl_scan(part, lane)), kWave - 1));
                t01 = s_hist[base] | (s_hist[base + 1] << 16);
                t23 = s_hist[base + 2] | (s_hist[base + 3] << 16);
            }
            if (lane == 0) {
                s_base = base;
                win.rec[row * win.tiles + tile] = make_uint4(base, above, t01, t23);
            }
        }
        __syncthreads();
        const uint32_t bs = s_base;
#pragma unroll
        for (int i = 0; i < NW; ++i) {
#pragma unroll
            for (int hf = 0; hf < 2; ++hf) {
                const uint32_t key = (kw[i] >> (16 * hf)) & 0xffffu;
                const uint32_t d = (key >> 8) - bs;  // wraps for keys below the window
                if (t0 + 2 * i + hf < tokens && d < static_cast<uint32_t>(kWinBins))
                    atomicAdd(&s_win[d][(key & 0xffu) >> 1], 1u << ((key & 1u) * 16));
            }
        }
        __syncthreads();
        uint32_t* wb = win.bins + (row * win.tiles + tile) * (kWinBins * 128);
        for (int i = threadIdx.x; i < kWinBins * 128; i += kKeyHistThreads) wb[i] = (&s_win[0][0])[i];
    }
    const uint32_t c = s_hist[threadIdx.x];
    if (c != 0u) atomicAdd(&ghist[row * kBins + threadIdx.x], c);
}

// Layer-step select, list form.  The input rows hold radix order keys and
// the scorer has accumulated each row's high-byte histogram into ghist, so
// the first radix level costs nothing here.  One 1024-thread workgroup per
// row; thread t owns the SEG consecutive tokens [t*SEG, t*SEG + SEG), read
// with 16-byte loads and kept packed two keys per register.
//   1. bin b1 of the k-th largest key from ghist (one wave);
//   2. 256-bin histogram of the low byte of the keys with high byte b1 ->
//      the k-th largest key T and need_eq = how many keys equal to T are
//      taken (the lowest-index ties: PyTorch's gather-top-k rule);
//   3. per thread, bit masks of its keys > T and >= T, two instructions per
//      key and mask: bit = sign of (T - key) (resp. T - 1 - key), shifted
//      in with v_alignbit;
//   4. one block scan of the per-thread (greater, equal) counts: a selected
//      token's rank = greater tokens before it + min(ties before it,
//      need_eq); the thread takes the first min(its ties, need_eq - ties
//      taken before it) of its own ties;
//   5. the thread writes its selected tokens (set bits of its mask, in
//      ascending order) to list[rank...].
// The VALU work per key is a few instructions, which matters: the kernel
// runs on one CU per row.  With list non-null, its row receives the k
// selected tokens in ascending order (int32), followed by `current` in slot
// k when list_current; with idx64 non-null the same tokens are written as
// int64 followed by `current` in slot k (the reference's _append_current
// layout).  Absent tokens (past `tokens`) get key 0, below every real key
// (real keys are >= 0x03ff; NaN patterns map to 0xffff).  ghist is
// re-zeroed for the next call.
template <int SEG>
__global__ __launch_bounds__(kSelThreads) void topk_list_kernel(
    const uint16_t* __restrict__ keys, uint32_t* __restrict__ ghist, int64_t row_stride, int ntok, int k,
    int32_t* __restrict__ list, int64_t list_stride, bool list_current, int64_t* __restrict__ idx64,
    int64_t idx_stride, int64_t current) {
    static_assert(SEG % 8 == 0 && SEG <= 128, "whole 16-byte chunks, at most four 32-bit masks");
    constexpr int NM = (SEG + 31) / 32;   // 32-bit masks per thread
    constexpr int MB = SEG < 32 ? SEG : 32;  // bits per mask
    const int64_t row = blockIdx.x;
    const uint16_t* src = keys + row * row_stride;
    uint32_t* gh = ghist + row * kBins;
    int32_t* lrow = list != nullptr ? list + row * list_stride : nullptr;
    int64_t* irow = idx64 != nullptr ? idx64 + row * idx_stride : nullptr;
    const int tid = threadIdx.x;

    __shared__ uint32_t tot[kBins], hist2[kBins];
    __shared__ uint32_t s_bin, s_above;
    __shared__ uint32_t scan_a[kSelWaves + 1], scan_b[kSelWaves + 1];
    if (tid < kBins) {
        tot[tid] = gh[tid];
        gh[tid] = 0u;
        hist2[tid] = 0u;
    }
    if (tid == 0) {
        if (irow != nullptr) irow[k] = current;
        if (lrow != nullptr && list_current) lrow[k] = static_cast<int32_t>(current);
    }
    // mode 0: nothing selected (k == 0); 1: every token (k >= ntok); 2: threshold
    const int mode = k <= 0 ? 0 : (k >= ntok ? 1 : 2);
    if (mode != 2) {
        if (mode == 1) {
            for (int t = tid; t < ntok; t += kSelThreads) {
                if (lrow != nullptr) lrow[t] = t;
                if (irow != nullptr) irow[t] = t;
            }
        }
        return;
    }

    // keys of tokens [begin, begin + n); the rest of the segment reads as 0.
    // Rows are padded to a multiple of 128 keys, so a chunk that starts
    // inside the row ends inside it.  Segments of up to 64 keys stay in
    // registers; longer ones are re-read 32 keys at a time in each pass.
    constexpr bool RELOAD = SEG > 64;
    constexpr int KW = RELOAD ? 16 : SEG / 2;  // registers of packed keys
    const int begin = tid * SEG;
    const int n = max(0, min(SEG, ntok - begin));
    uint32_t kp[KW];
    // chunks [c0, c0 + KW/4) of 8 keys into kp
    // `after` orders a re-read after the work on the previous keys: an
    // opaque copy of the row pointer that depends on it keeps the compiler
    // from issuing every pass's loads at once (which would spill)
    auto load_keys = [&](int c0, uint32_t after) {
        const uint16_t* rowp = src;
        if (RELOAD) asm volatile("" : "+s"(rowp) : "v"(after) : "memory");
        const uint16_t* seg = rowp + begin;
        // every chunk's load is issued before any is used (a chunk past
        // the segment's tokens re-reads the row's first chunk and is then
        // zeroed), so the loads share one memory latency
        uint4 uc[KW / 4];
#pragma unroll
        for (int c = 0; c < KW / 4; ++c) {
            const int e0 = 8 * (c0 + c);
            uc[c] = *reinterpret_cast<const uint4*>(e0 < n ? seg + e0 : rowp);
        }
#pragma unroll
        for (int c = 0; c < KW / 4; ++c) {
            const int e0 = 8 * (c0 + c);
            uint4 u = uc[c];
            if (e0 + 8 > n) {  // the segment's tail: keys e >= n read as 0
                const int v = n - e0;  // keys of this chunk that exist (may be <= 0)
                u.x &= (v > 1 ? 0xffffffffu : 0u) | (v > 0 ? 0x0000ffffu : 0u);
                u.y &= (v > 3 ? 0xffffffffu : 0u) | (v > 2 ? 0x0000ffffu : 0u);
                u.z &= (v > 5 ? 0xffffffffu : 0u) | (v > 4 ? 0x0000ffffu : 0u);
                u.w &= (v > 7 ? 0xffffffffu : 0u) | (v > 6 ? 0x0000ffffu : 0u);
            }
            kp[4 * c] = u.x;
            kp[4 * c + 1] = u.y;
            kp[4 * c + 2] = u.z;
            kp[4 * c + 3] = u.w;
        }
    };
#define POPKV_KEY(e) ((kp[(e) >> 1] >> (((e) & 1) * 16)) & 0xffffu)
    if (!RELOAD) load_keys(0, 0u);
    __syncthreads();
    if (tid < kWave) find_bin<kBins>(tot, static_cast<uint32_t>(k), &s_bin, &s_above);
    __syncthreads();
    const uint32_t b1 = s_bin;
    const uint32_t above1 = s_above;
#pragma unroll
    for (int i = 0; i < (RELOAD ? SEG / 32 : 1); ++i) {
        if (RELOAD) load_keys(4 * i, 0u);
#pragma unroll
        for (int e = 0; e < 2 * KW; ++e) {
            const uint32_t key = POPKV_KEY(e);
            if ((key >> 8) == b1) atomicAdd(&hist2[key & 0xffu], 1u);
        }
    }
    __syncthreads();
    if (tid < kWave) find_bin<kBins>(hist2, static_cast<uint32_t>(k) - above1, &s_bin, &s_above);
    __syncthreads();
    const uint32_t thr = (b1 << 8) | s_bin;  // >= 0x03ff
    const uint32_t need_eq = static_cast<uint32_t>(k) - above1 - s_above;

    // 3. masks: bit e of m_gt[i] / m_ge[i] = key 32 i + e > T / >= T
    uint32_t m_gt[NM], m_eq[NM];
    uint32_t n_gt = 0, n_eq = 0;
#pragma unroll
    for (int i = 0; i < NM; ++i) {
        if (RELOAD) load_keys(4 * i, n_gt + n_eq);
        const int eb = RELOAD ? 0 : 32 * i;  // mask i's first key in kp
        uint32_t g = 0, ge = 0;
#pragma unroll
        for (int e = MB - 1; e >= 0; --e) {
            const uint32_t key = POPKV_KEY(eb + e);
            g = __builtin_amdgcn_alignbit(g, thr - key, 31);
            ge = __builtin_amdgcn_alignbit(ge, thr - 1u - key, 31);
        }
        m_gt[i] = g;
        m_eq[i] = ge & ~g;
        n_gt += __popc(g);
        n_eq += __popc(m_eq[i]);
    }
#undef POPKV_KEY
    // 4. ranks.  For rows of up to 65536 tokens both exclusive prefixes fit
    //    16 bits and one packed scan serves both.
    uint32_t total, gt_before, eq_before;
    if (SEG <= 64) {
        const uint32_t packed = block_excl_scan_once(n_gt | (n_eq << 16), scan_a, kSelWaves, &total);
        gt_before = packed & 0xffffu;
        eq_before = packed >> 16;
    } else {
        gt_before = block_excl_scan_once(n_gt, scan_a, kSelWaves, &total);
        eq_before = block_excl_scan_once(n_eq, scan_b, kSelWaves, &total);
    }
    // (taken_before is formed first and the subtraction below never wraps:
    // a ternary "eq_before >= need_eq ? 0 : need_eq - eq_before" here was
    // miscompiled by this toolchain's optimizer, which dropped the later
    // min as if the subtraction's no-wrap flag held everywhere)
    const uint32_t taken_before = min(eq_before, need_eq);
    uint32_t take_ties = min(n_eq, need_eq - taken_before);  // this thread's ties taken
    uint32_t pos = gt_before + taken_before;
    // 5. writes, mask by mask in token order
#pragma unroll
    for (int i = 0; i < NM; ++i) {
        uint32_t ties = m_eq[i];
        const uint32_t c = static_cast<uint32_t>(__popc(ties));
        if (take_ties < c) {  // keep only the first take_ties ties
            uint32_t rest = ties;
            for (uint32_t j = 0; j < take_ties; ++j) rest &= rest - 1u;
            ties &= ~rest;
            take_ties = 0;
        } else {
            take_ties -= c;
        }
        for (uint32_t m = m_gt[i] | ties; m != 0u; m &= m - 1u) {
            const int32_t t = begin + 32 * i + __builtin_ctz(m);
            if (pos < static_cast<uint32_t>(k)) {
                if (lrow != nullptr) lrow[pos] = t;
                if (irow != nullptr) irow[pos] = t;
            }
            ++pos;
        }
    }
}


// Layer step, first half of the chunked select (the second half is the
// fused select + attention kernel).  Block (c, h) covers chunk c of row h
// (kChunkThreads * KPT tokens): it finds the high-byte bin b1 of the k-th
// largest key from the scorer's histogram ghist[h], then writes
//   h2[h][c][256]: the chunk's histogram of the low byte of its keys with
//                  high byte b1 (uint16; a chunk holds <= 8192 tokens),
//   gt1[h][c]:     the chunk's count of keys with high byte > b1,
//   rec[h][0..1]:  b1 and the row's count of keys above bin b1 (block 0).
// Only for 0 < k < tokens.
template <int KPT>
__global__ __launch_bounds__(kChunkThreads) void chunk_hist_kernel(const uint16_t* __restrict__ keys,
                                                                   int64_t key_stride, int ntok, int k,
                                                                   const uint32_t* __restrict__ ghist,
                                                                   uint32_t* __restrict__ rec,
                                                                   uint16_t* __restrict__ h2,
                                                                   uint32_t* __restrict__ gt1, int nchunks,
                                                                   SeqTable seq) {
    constexpr int CH = kChunkThreads * KPT;
    args_in_sgprs(keys, key_stride, ntok, k, ghist, rec, h2, gt1, nchunks, seq.tokens, seq.q_heads);
    const int c = blockIdx.x;
    const int h = blockIdx.y;
    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int begin = c * CH + tid * KPT;
    ChunkKeys<KPT> kk;
    load_chunk_keys_raw<KPT>(keys + static_cast<int64_t>(h) * key_stride, begin, max(0, min(KPT, ntok - begin)), kk);
    uint32_t cnt[4];
    load_rank4(ghist + static_cast<int64_t>(h) * kBins, cnt);
    if (seq.tokens != nullptr) {  // a batched step: this row's own token count and k
        ntok = static_cast<int>(seq_tokens_of(seq, div_nonneg(h, seq.q_heads), ntok));
        k = min(seq.budget - 1, ntok);
        if (k <= 0 || k >= ntok || c * CH >= ntok) return;
    }
    mask_chunk_keys<KPT>(max(0, min(KPT, ntok - begin)), kk);
    __shared__ uint32_t s_h2[kBins];
    __shared__ uint32_t s_gt;
    s_h2[tid] = 0u;
    if (tid == 0) s_gt = 0u;
    uint32_t b1, above1;
    wave_find_bin(cnt, static_cast<uint32_t>(k), &b1, &above1);
    __syncthreads();
    uint32_t n_gt = 0;
#pragma unroll
    for (int e = 0; e < KPT; ++e) {
        const uint32_t key = kk.key(e);
        const uint32_t hb = key >> 8;
        n_gt += hb > b1 ? 1u : 0u;
        if (hb == b1) atomicAdd(&s_h2[key & 0xffu], 1u);
    }
    n_gt = wave_incl_scan(n_gt, lane);
    if (lane == kWave - 1 && n_gt != 0u) atomicAdd(&s_gt, n_gt);
    __syncthreads();
    const int64_t cell = static_cast<int64_t>(h) * nchunks + c;
    h2[cell * kBins + tid] = static_cast<uint16_t>(s_h2[tid]);
    if (tid == 0) {
        gt1[cell] = s_gt;
        if (c == 0) {
            rec[4 * h] = b1;
            rec[4 * h + 1] = above1;
        }
    }
}

// API-path top-k, second half of the chunked select (after key_hist_kernel
// and chunk_hist_kernel): block (c, h) writes the selected tokens of chunk c
// of row h at their row ranks, so the row reads in ascending token order.
// The selection rule and the ranks are those of the layer step's select: a
// selected token's rank = keys above bin b1 in earlier chunks (gt1) + keys
// of bin b1 above T in earlier chunks + ties taken by earlier chunks
// (rank0), then, inside the chunk, one block scan of each thread's (keys
// above T, ties) counts.  Block 0 of each row writes `current` to slot
// min(k, tokens) and re-zeroes ghist[h].  k <= 0: no token; k >= tokens:
// every token; otherwise the k largest keys, lowest index first among ties.
template <int KPT>
__global__ __launch_bounds__(kChunkThreads) void topk_chunk_kernel(
    const uint16_t* __restrict__ keys, int64_t key_stride, int ntok, int k, const uint32_t* __restrict__ rec,
    const uint16_t* __restrict__ h2, const uint32_t* __restrict__ gt1, int nchunks, uint32_t* __restrict__ ghist,
    int32_t* __restrict__ out32, int64_t* __restrict__ out64, int64_t out_stride, int64_t current) {
    constexpr int CH = kChunkThreads * KPT;
    constexpr int kWaves = kChunkThreads / kWave;
    const int c = blockIdx.x;
    const int h = blockIdx.y;
    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int mode = k <= 0 ? 0 : (k >= ntok ? 1 : 2);  // none / every token / threshold
    const int kk = mode == 1 ? ntok : max(k, 0);        // tokens the row selects
    const int begin = c * CH + tid * KPT;
    const int n = max(0, min(KPT, ntok - begin));
    __shared__ uint32_t s_g2[kBins], s_p2[kBins];
    __shared__ uint32_t s_scan[kWaves];
    uint32_t sel = 0u;    // bit e: token begin + e is selected
    uint32_t rank = 0u;   // row rank of this thread's first selected token
    if (mode == 1) {
        sel = n >= 32 ? 0xffffffffu : (1u << n) - 1u;
        rank = static_cast<uint32_t>(begin);
    } else if (mode == 2) {
        ChunkKeys<KPT> kv;
        load_chunk_keys<KPT>(keys + static_cast<int64_t>(h) * key_stride, begin, n, kv);
        const uint32_t b1 = rec[4 * h], above1 = rec[4 * h + 1];
        // bin tid of the chunk histograms over every chunk / over chunks before c
        uint32_t g2 = 0, p2 = 0;
        const uint16_t* hr = h2 + static_cast<int64_t>(h) * nchunks * kBins + tid;
        for (int c0 = 0; c0 < nchunks; c0 += 16) {
            uint32_t v[16];
#pragma unroll
            for (int j = 0; j < 16; ++j) v[j] = hr[static_cast<int64_t>(min(c0 + j, nchunks - 1)) * kBins];
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const uint32_t x = c0 + j < nchunks ? v[j] : 0u;
                g2 += x;
                p2 += c0 + j < c ? x : 0u;
            }
        }
        // keys above bin b1 in earlier chunks (every wave forms the same sum)
        uint32_t gt1_before = 0;
        for (int c0 = 0; c0 < c; c0 += kWave) {
            const uint32_t x = c0 + lane < c ? gt1[static_cast<int64_t>(h) * nchunks + c0 + lane] : 0u;
            gt1_before += static_cast<uint32_t>(
                __builtin_amdgcn_readlane(static_cast<int>(wave_incl_scan(x, lane)), kWave - 1));
        }
        s_g2[tid] = g2;
        s_p2[tid] = p2;
        __syncthreads();
        uint32_t cnt[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) cnt[i] = s_g2[255 - (4 * lane + i)];
        const uint32_t need1 = static_cast<uint32_t>(k) - above1;
        uint32_t t2, above2;
        wave_find_bin(cnt, need1, &t2, &above2);
        const uint32_t thr = (b1 << 8) | t2;
        const uint32_t need_eq = need1 - above2;  // ties at T the row takes
        const uint32_t eq_before = s_p2[t2];      // ties at T in earlier chunks
        // keys of bin b1 with low byte > t2 in earlier chunks
        uint32_t x = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) x += 4 * lane + i > static_cast<int>(t2) ? s_p2[4 * lane + i] : 0u;
        const uint32_t gt2_before =
            static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(wave_incl_scan(x, lane)), kWave - 1));
        uint32_t m_gt, m_eq;
        key_masks<KPT>(kv, thr, &m_gt, &m_eq);
        const uint32_t n_eq = static_cast<uint32_t>(__popc(m_eq));
        uint32_t total;
        const uint32_t packed =
            block_excl_scan_once(static_cast<uint32_t>(__popc(m_gt)) | (n_eq << 16), s_scan, kWaves, &total);
        // ties taken by earlier chunks / before this thread (each min is
        // formed before the subtraction that uses it, which then never wraps)
        const uint32_t prior = min(eq_before, need_eq);
        const uint32_t t_before = min(eq_before + (packed >> 16), need_eq);
        const uint32_t take = min(n_eq, need_eq - t_before);
        uint32_t ties = m_eq;
        if (take < n_eq) {  // keep only the first `take` ties
            uint32_t rest = ties;
            for (uint32_t j = 0; j < take; ++j) rest &= rest - 1u;
            ties &= ~rest;
        }
        sel = m_gt | ties;
        rank = gt1_before + gt2_before + prior + (packed & 0xffffu) + (t_before - prior);
    }
    const int64_t row = static_cast<int64_t>(h) * out_stride;
    for (uint32_t m = sel; m != 0u; m &= m - 1u) {
        if (rank < static_cast<uint32_t>(kk)) {
            const int t = begin + __builtin_ctz(m);
            if (out32 != nullptr) out32[row + rank] = t;
            else out64[row + rank] = t;
        }
        ++rank;
    }
    if (c == 0) {
        ghist[static_cast<int64_t>(h) * kBins + tid] = 0u;
        if (tid == 0) {
            if (out32 != nullptr) out32[row + kk] = static_cast<int32_t>(current);
            else out64[row + kk] = current;
        }
    }
}
// API-path top-k after key_hist_kernel's tile-window form (no
// chunk_hist_kernel): block (c, h) finds b1 and the count above it from
// the row's histogram ghist[h], sums the tiles' window rows at b1 (over all
// tiles, and over the tiles before chunk c) into the row's and the earlier
// chunks' low-byte histograms of bin b1, and then selects and writes chunk
// c's tokens exactly as topk_chunk_kernel does.  A tile whose window misses
// b1 (rare: the window spans the estimate -2 .. +1) is histogrammed from
// its keys by the whole block.  Keys above bin b1 in earlier chunks: the
// tiles' records (keys above the window plus the window bins above b1), or
// the scan.  For 0 < k < ntok, chunks of whole 2048-token tiles and at
// most kWinMaxTiles tiles (host-checked).  Each block takes a ticket on
// ghist[h][0] (bin 0: no real key reaches it) once it has read the
// histogram; the row's last block zeroes the row for the next call.
template <int KPT>
__global__ __launch_bounds__(kChunkThreads) void topk_chunk_win_kernel(
    const uint16_t* __restrict__ keys, int64_t key_stride, int ntok, int k, uint32_t* __restrict__ ghist,
    const uint4* __restrict__ wrec, const uint32_t* __restrict__ wbins, int tiles, int nchunks,
    int32_t* __restrict__ out32, int64_t* __restrict__ out64, int64_t out_stride, int64_t current) {
    constexpr int CH = kChunkThreads * KPT;
    constexpr int TPC = CH / kApiTileTokens;  // tiles per chunk
    static_assert(CH % kApiTileTokens == 0 && kChunkThreads == 256, "chunks of whole tiles, one bin per thread");
    constexpr int kWaves = kChunkThreads / kWave;
    const int c = blockIdx.x;
    const int h = blockIdx.y;
    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int begin = c * CH + tid * KPT;
    const int n = max(0, min(KPT, ntok - begin));
    uint32_t* const hrow = ghist + static_cast<int64_t>(h) * kBins;
    // first loads: this thread's keys, the row histogram (lane l: ranks
    // 4l .. 4l + 3), the tile records
    ChunkKeys<KPT> kv;
    load_chunk_keys<KPT>(keys + static_cast<int64_t>(h) * key_stride, begin, n, kv);
    uint32_t gcnt[4];
    load_rank4(hrow, gcnt);
    __shared__ uint4 s_rec[kWinMaxTiles];
    if (tid < tiles) s_rec[tid] = wrec[static_cast<int64_t>(h) * tiles + tid];
    uint32_t b1, above1;
    wave_find_bin(gcnt, static_cast<uint32_t>(k), &b1, &above1);
    __shared__ uint32_t s_last, s_gtb;
    __shared__ uint32_t s_mg[kBins], s_mp[kBins];
    s_mg[tid] = 0u;
    s_mp[tid] = 0u;
    if (tid == 0) s_gtb = 0u;
    __syncthreads();  // every wave has read the histogram; s_rec complete
    // the window rows at b1: thread (slot sl, quad q) adds 16-byte quad q of
    // the row of tiles sl + 8j (16-bit pairs: at most 4 tiles of 2048 tokens
    // per slot, below 2^16)
    const int c0t = c * TPC;  // this chunk's first tile
    const int sl = tid >> 5, q = tid & 31;
    const uint4* wb = reinterpret_cast<const uint4*>(wbins) + static_cast<int64_t>(h) * tiles * (kWinBins * 32) + q;
    constexpr int WJ = kWinMaxTiles / 8;
    uint4 wv[WJ];
    bool hit[WJ];
#pragma unroll
    for (int j = 0; j < WJ; ++j) {
        const int i = sl + 8 * j;
        const int r = i < tiles ? static_cast<int>(b1) - static_cast<int>(s_rec[i].x) : -1;
        hit[j] = static_cast<unsigned>(r) < static_cast<unsigned>(kWinBins);
        wv[j] = wb[hit[j] ? (i * kWinBins + r) * 32 : 0];
    }
    // the ticket, behind the window loads; its value is needed only at the end
    uint32_t ticket = 0u;
    if (tid == 0) ticket = __hip_atomic_fetch_add(&hrow[0], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    uint4 gs = make_uint4(0u, 0u, 0u, 0u), ps = gs;
#pragma unroll
    for (int j = 0; j < WJ; ++j) {
        if (hit[j]) {
            gs.x += wv[j].x; gs.y += wv[j].y; gs.z += wv[j].z; gs.w += wv[j].w;
            if (sl + 8 * j < c0t) {
                ps.x += wv[j].x; ps.y += wv[j].y; ps.z += wv[j].z; ps.w += wv[j].w;
            }
        }
    }
    __shared__ uint4 s_gp[8][32], s_pp[8][32];
    s_gp[sl][q] = gs;
    s_pp[sl][q] = ps;
    // per tile (thread i < tiles, all in wave 0): whether its window covers
    // b1 and, for a covered tile before this chunk, its keys above bin b1
    // (keys above the window plus the window bins above b1); the missed
    // tiles' keys are then scanned by the block (thread t takes keys 8t ..
    // 8t + 7 of the tile; key rows are written up to ntok and padded to 128
    // keys)
    __shared__ uint32_t s_miss, s_gt1cov;
    if (tid < kWave) {
        uint32_t cov = 0u;
        bool missed = false;
        if (tid < tiles) {
            const uint4 rc = s_rec[tid];
            const int r = static_cast<int>(b1) - static_cast<int>(rc.x);
            if (static_cast<unsigned>(r) < static_cast<unsigned>(kWinBins)) {
                if (tid < c0t) {
                    const uint32_t tot[kWinBins] = {rc.z & 0xffffu, rc.z >> 16, rc.w & 0xffffu, rc.w >> 16};
                    cov = rc.y;
#pragma unroll
                    for (int w = 0; w < kWinBins; ++w) cov += w > r ? tot[w] : 0u;
                }
            } else {
                missed = true;
            }
        }
        const uint64_t mm = __ballot(missed);
        const uint32_t cs = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(wave_incl_scan(cov, lane)), kWave - 1));
        if (tid == 0) {
            s_miss = static_cast<uint32_t>(mm);  // tiles <= 32
            s_gt1cov = cs;
        }
    }
    __syncthreads();
    const uint32_t miss_mask = s_miss;
    uint32_t gtb = 0u;
    for (uint32_t mset = miss_mask; mset != 0u; mset &= mset - 1u) {
        const int i = __builtin_ctz(mset);
        const int tb = i * kApiTileTokens + tid * 8;
        const uint4 u = tb < ntok ? *reinterpret_cast<const uint4*>(keys + static_cast<int64_t>(h) * key_stride + tb)
                                  : make_uint4(0u, 0u, 0u, 0u);
        const uint32_t wd[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            if (tb + e >= ntok) continue;
            const uint32_t key = (wd[e >> 1] >> ((e & 1) * 16)) & 0xffffu;
            const uint32_t hb = key >> 8;
            if (hb == b1) {
                atomicAdd(&s_mg[key & 0xffu], 1u);
                if (i < c0t) atomicAdd(&s_mp[key & 0xffu], 1u);
            } else if (hb > b1 && i < c0t) {
                ++gtb;
            }
        }
    }
    if (gtb != 0u) atomicAdd(&s_gtb, gtb);
    __syncthreads();
    // bin tid of the row / the earlier chunks
    __shared__ uint32_t s_g2[kBins], s_p2[kBins];
    {
        uint32_t g2 = s_mg[tid], p2 = s_mp[tid];
        const int wq = (tid >> 1) >> 2, wc = (tid >> 1) & 3, hf = tid & 1;
#pragma unroll
        for (int x = 0; x < 8; ++x) {
            const uint4 gv = s_gp[x][wq], pv = s_pp[x][wq];
            const uint32_t gw = wc == 0 ? gv.x : wc == 1 ? gv.y : wc == 2 ? gv.z : gv.w;
            const uint32_t pw = wc == 0 ? pv.x : wc == 1 ? pv.y : wc == 2 ? pv.z : pv.w;
            g2 += (gw >> (16 * hf)) & 0xffffu;
            p2 += (pw >> (16 * hf)) & 0xffffu;
        }
        s_g2[tid] = g2;
        s_p2[tid] = p2;
    }
    __shared__ uint32_t s_scan[kWaves];
    __syncthreads();
    const uint32_t gt1_before = s_gt1cov + s_gtb;
    uint32_t cnt[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) cnt[i] = s_g2[255 - (4 * lane + i)];
    const uint32_t need1 = static_cast<uint32_t>(k) - above1;
    uint32_t t2, above2;
    wave_find_bin(cnt, need1, &t2, &above2);
    const uint32_t thr = (b1 << 8) | t2;
    const uint32_t need_eq = need1 - above2;  // ties at T the row takes
    const uint32_t eq_before = s_p2[t2];      // ties at T in earlier chunks
    // keys of bin b1 with low byte > t2 in earlier chunks
    uint32_t x = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) x += 4 * lane + i > static_cast<int>(t2) ? s_p2[4 * lane + i] : 0u;
    const uint32_t gt2_before =
        static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(wave_incl_scan(x, lane)), kWave - 1));
    uint32_t m_gt, m_eq;
    key_masks<KPT>(kv, thr, &m_gt, &m_eq);
    const uint32_t n_eq = static_cast<uint32_t>(__popc(m_eq));
    if (tid == 0) s_last = ticket + 1u == static_cast<uint32_t>(nchunks) ? 1u : 0u;  // (ordered by the scan's barriers)
    uint32_t total;
    const uint32_t packed =
        block_excl_scan_once(static_cast<uint32_t>(__popc(m_gt)) | (n_eq << 16), s_scan, kWaves, &total);
    // ties taken by earlier chunks / before this thread (each min is formed
    // before the subtraction that uses it, which then never wraps)
    const uint32_t prior = min(eq_before, need_eq);
    const uint32_t t_before = min(eq_before + (packed >> 16), need_eq);
    const uint32_t take = min(n_eq, need_eq - t_before);
    uint32_t ties = m_eq;
    if (take < n_eq) {  // keep only the first `take` ties
        uint32_t rest = ties;
        for (uint32_t j = 0; j < take; ++j) rest &= rest - 1u;
        ties &= ~rest;
    }
    const uint32_t sel = m_gt | ties;
    uint32_t rank = gt1_before + gt2_before + prior + (packed & 0xffffu) + (t_before - prior);
    const int64_t orow = static_cast<int64_t>(h) * out_stride;
    for (uint32_t m = sel; m != 0u; m &= m - 1u) {
        if (rank < static_cast<uint32_t>(k)) {
            const int t = begin + __builtin_ctz(m);
            if (out32 != nullptr) out32[orow + rank] = t;
            else out64[orow + rank] = t;
        }
        ++rank;
    }
    if (c == 0 && tid == 0) {
        if (out32 != nullptr) out32[orow + k] = static_cast<int32_t>(current);
        else out64[orow + k] = current;
    }
    if (s_last != 0u) hrow[tid] = 0u;  // every block of the row has read it (before its ticket)
}

// n 32-bit words set to `value`: clears histogram regions after a failed
// launch (a kernel, not hipMemsetAsync, so it also records into HIP graphs).
__global__ __launch_bounds__(256) void fill_u32_kernel(uint32_t* __restrict__ p, int64_t n, uint32_t value) {
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * 256)
        p[i] = value;
}
}  // namespace

hipError_t launch_fill_u32(uint32_t* p, int64_t n, uint32_t value, hipStream_t stream) {
    if (n <= 0) return hipSuccess;
    const int64_t blocks = (n + 255) / 256;
    hipLaunchKernelGGL(fill_u32_kernel, dim3(static_cast<unsigned>(blocks < 1024 ? blocks : 1024)), dim3(256), 0,
                       stream, p, n, value);
    return hipGetLastError();
}

hipError_t launch_topk_list(const uint16_t* keys, uint32_t* ghist, int64_t rows, int64_t row_stride, int64_t tokens,
                            int64_t k, int32_t* list, int64_t list_stride, bool list_current, int64_t* idx64,
                            int64_t idx_stride, int64_t current, hipStream_t stream) {
    if (rows <= 0) return hipSuccess;
    const int64_t per = (tokens + kSelThreads - 1) / kSelThreads;
    const int nt = static_cast<int>(tokens), kk = static_cast<int>(k < tokens ? k : tokens);
    dim3 grid(static_cast<unsigned>(rows)), block(kSelThreads);
#define POPKV_LIST(SEG)                                                                                          \
    hipLaunchKernelGGL((topk_list_kernel<SEG>), grid, block, 0, stream, keys, ghist, row_stride, nt, kk, list, \
                       list_stride, list_current, idx64, idx_stride, current)
    if (per <= 8) POPKV_LIST(8);
    else if (per <= 16) POPKV_LIST(16);
    else if (per <= 32) POPKV_LIST(32);
    else if (per <= 64) POPKV_LIST(64);
    else POPKV_LIST(128);
#undef POPKV_LIST
    return hipGetLastError();
}

hipError_t launch_chunk_hist(const uint16_t* keys, int64_t key_stride, int64_t rows, int64_t tokens, int64_t k,
                             const uint32_t* ghist, uint32_t* rec, uint16_t* h2, uint32_t* gt1, const SeqTable& seq,
                             hipStream_t stream) {
    if (rows <= 0 || k <= 0 || k >= tokens) return hipSuccess;
    const StepChunks ch = step_chunks(tokens, k, rows);
    const int nt = static_cast<int>(tokens), kk = static_cast<int>(k), nc = static_cast<int>(ch.count);
    dim3 grid(static_cast<unsigned>(ch.count), static_cast<unsigned>(rows)), block(kChunkThreads);
#define POPKV_CH(KPT)                                                                                          \
    case KPT:                                                                                                  \
        hipLaunchKernelGGL((chunk_hist_kernel<KPT>), grid, block, 0, stream, keys, key_stride, nt, kk, ghist, \
                           rec, h2, gt1, nc, seq);                                                             \
        break
    switch (ch.kpt) {
        POPKV_CH(1); POPKV_CH(2); POPKV_CH(4); POPKV_CH(6); POPKV_CH(8); POPKV_CH(12); POPKV_CH(16); POPKV_CH(24); POPKV_CH(32);
        default: return hipErrorInvalidValue;
    }
#undef POPKV_CH
    return hipGetLastError();
}

// Workspace of the API top-k: ghist | keys | rec | gt1 | h2 | window
// records | window bins (each region 256-byte aligned; rec, gt1 and h2
// sized for the 64 chunks a row can have, the windows for the row's
// 2048-token tiles when it has at most kWinMaxTiles of them).
struct TopkWorkspace {
    size_t hist, keys, rec, gt1, h2, wrec, wbins, total;
    int tiles;
};
static TopkWorkspace topk_workspace(int64_t rows, int64_t tokens) {
    auto al = [](size_t x) { return (x + 255) / 256 * 256; };
    const int64_t key_stride = (tokens + 127) / 128 * 128;
    const size_t r = static_cast<size_t>(rows);
    const int64_t tiles = (tokens + kApiTileTokens - 1) / kApiTileTokens;
    TopkWorkspace w;
    w.tiles = tiles <= kWinMaxTiles ? static_cast<int>(tiles) : 0;
    w.hist = 0;
    w.keys = al(r * kBins * 4);
    w.rec = w.keys + al(r * static_cast<size_t>(key_stride > 0 ? key_stride : 128) * 2);
    w.gt1 = w.rec + al(r * 4 * 4);
    w.h2 = w.gt1 + al(r * 64 * 4);
    w.wrec = w.h2 + al(r * 64 * kBins * 2);
    w.wbins = w.wrec + al(r * static_cast<size_t>(w.tiles) * 16);
    w.total = w.wbins + al(r * static_cast<size_t>(w.tiles) * kWinBins * 128 * 4);
    return w;
}

size_t topk_select_workspace_bytes(int64_t rows, int64_t tokens) { return topk_workspace(rows, tokens).total; }

// Rows of at least this many tokens take the chunked select (key_hist,
// chunk_hist, topk_chunk: every CU busy); shorter rows the one-block-per-row
// list kernel (one launch fewer).  Measured with 32 rows, list vs chunked:
// 16K tokens 11.2 vs 12.8 us, 32K 13.9 vs 13.4, 64K 22.9 vs 15.7, 128K 38.3
// vs 24.5.
constexpr int64_t kTopkChunkMinTokens = 24576;
constexpr int64_t kApiWindowBlocks = 512;  // two 2048-token key_hist blocks per CU

hipError_t launch_topk_select(const uint16_t* scores, int64_t rows, int64_t row_stride, int64_t tokens, int64_t k,
                              int64_t current, void* indices, int index_dtype, int64_t index_row_stride,
                              void* workspace, hipStream_t stream) {
    if (rows <= 0) return hipSuccess;
    const TopkWorkspace w = topk_workspace(rows, tokens);
    const int64_t key_stride = (tokens + 127) / 128 * 128;
    char* base = static_cast<char*>(workspace);
    uint32_t* ghist = reinterpret_cast<uint32_t*>(base + w.hist);
    uint16_t* keys = reinterpret_cast<uint16_t*>(base + w.keys);
    const StepChunks ch = step_chunks(tokens, k > 0 && k < tokens ? k : tokens, rows);
    // the tile-window form: the chunked select of 0 < k < tokens with chunks
    // of whole 2048-token tiles, at most kWinMaxTiles tiles per row and at
    // most kApiWindowBlocks key_hist blocks (tiles) in all.  Measured with
    // the scorer's scores, kernel times summed: 32 x 32767 (512 tiles) 11.0
    // us against 13.2 for key_hist + chunk_hist + topk_chunk; 32 x 65535
    // (1024 tiles: four 2048-token key_hist blocks per CU) 13.9 against 13.5.
    const bool windows = tokens >= kTopkChunkMinTokens && k > 0 && k < tokens && w.tiles > 0 &&
                         rows * w.tiles <= kApiWindowBlocks && ch.tokens_per_chunk % kApiTileTokens == 0 &&
                         ch.kpt <= 16;  // (larger chunks need more than kApiWindowBlocks tiles: step_chunks)
    ApiWindows aw;
    if (windows) {
        aw.rec = reinterpret_cast<uint4*>(base + w.wrec);
        aw.bins = reinterpret_cast<uint32_t*>(base + w.wbins);
        aw.tiles = w.tiles;
        aw.k = k;
    }
    if (tokens > 0) {
        const int tpt = windows ? kApiTileTokens / kKeyHistThreads : kKeyHistTokens;
        const int chunks = static_cast<int>((tokens + kKeyHistThreads * tpt - 1) / (kKeyHistThreads * tpt));
        const bool vec = reinterpret_cast<uintptr_t>(scores) % 16 == 0 && row_stride % 8 == 0;
        dim3 grid(static_cast<unsigned>(rows * chunks)), block(kKeyHistThreads);
#define POPKV_KH(VEC, TPT, WIN)                                                                                   \
    hipLaunchKernelGGL((key_hist_kernel<VEC, TPT, WIN>), grid, block, 0, stream, scores, row_stride, tokens, chunks, \
                       keys, key_stride, ghist, aw)
        if (windows) {
            if (vec) POPKV_KH(true, 8, true);
            else POPKV_KH(false, 8, true);
        } else {
            if (vec) POPKV_KH(true, 16, false);
            else POPKV_KH(false, 16, false);
        }
#undef POPKV_KH
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    const bool i32 = index_dtype == POPKV_INDEX_I32;
    int32_t* out32 = i32 ? static_cast<int32_t*>(indices) : nullptr;
    int64_t* out64 = i32 ? nullptr : static_cast<int64_t*>(indices);
    if (windows) {
        const int nt = static_cast<int>(tokens), kk = static_cast<int>(k), nc = static_cast<int>(ch.count);
        dim3 grid(static_cast<unsigned>(ch.count), static_cast<unsigned>(rows)), block(kChunkThreads);
#define POPKV_TW(KPT)                                                                                            \
    case KPT:                                                                                                    \
        hipLaunchKernelGGL((topk_chunk_win_kernel<KPT>), grid, block, 0, stream, keys, key_stride, nt, kk, ghist, \
                           aw.rec, aw.bins, aw.tiles, nc, out32, out64, index_row_stride, current);              \
        break
        hipError_t e = hipSuccess;
        switch (ch.kpt) {
            POPKV_TW(8); POPKV_TW(16);
            default: e = hipErrorInvalidValue; break;
        }
#undef POPKV_TW
        if (e == hipSuccess) e = hipGetLastError();
        if (e != hipSuccess) (void)launch_fill_u32(ghist, rows * kBins, 0u, stream);
        return e;
    }
    if (tokens < kTopkChunkMinTokens) {
        const hipError_t e = launch_topk_list(keys, ghist, rows, key_stride, tokens, k, out32, index_row_stride,
                                              true, out64, index_row_stride, current, stream);
        if (e != hipSuccess) (void)launch_fill_u32(ghist, rows * kBins, 0u, stream);
        return e;
    }
    uint32_t* rec = reinterpret_cast<uint32_t*>(base + w.rec);
    uint32_t* gt1 = reinterpret_cast<uint32_t*>(base + w.gt1);
    uint16_t* h2 = reinterpret_cast<uint16_t*>(base + w.h2);
    // chunk_hist_kernel runs for 0 < k < tokens only, on step_chunks(tokens, k, rows)
    hipError_t e = launch_chunk_hist(keys, key_stride, rows, tokens, k, ghist, rec, h2, gt1, SeqTable{}, stream);
    if (e != hipSuccess) {
        (void)launch_fill_u32(ghist, rows * kBins, 0u, stream);  // the histograms stay zero between calls
        return e;
    }
    const int nt = static_cast<int>(tokens), kk = static_cast<int>(k < tokens ? k : tokens),
              nc = static_cast<int>(ch.count);
    dim3 grid(static_cast<unsigned>(ch.count), static_cast<unsigned>(rows)), block(kChunkThreads);
#define POPKV_TC(KPT)                                                                                             \
    case KPT:                                                                                                     \
        hipLaunchKernelGGL((topk_chunk_kernel<KPT>), grid, block, 0, stream, keys, key_stride, nt, kk, rec, h2,  \
                           gt1, nc, ghist, out32, out64, index_row_stride, current);                              \
        break
    switch (ch.kpt) {
        POPKV_TC(1); POPKV_TC(2); POPKV_TC(4); POPKV_TC(6); POPKV_TC(8); POPKV_TC(12); POPKV_TC(16); POPKV_TC(24); POPKV_TC(32);
        default: return hipErrorInvalidValue;
    }
#undef POPKV_TC
    return hipGetLastError();
}

}  // namespace popkv
