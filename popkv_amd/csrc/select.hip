// Per-query-head top-k over fp16 scores with the current token reserving the
// last slot (gfx950).
//
// Replaces torch.topk(scores, k, dim=-1, sorted=False).indices followed by
// _append_current (reference popkv.py:1094-1098, :287-291).
//
// One 1024-thread workgroup (16 wave64s) per row.  Thread t owns the
// contiguous segment of SEG tokens [t*SEG, t*SEG + SEG), read with 16-byte
// loads, and keeps its keys in registers (two 16-bit keys per VGPR) for the
// whole kernel.  The key is PyTorch's radix order of an fp16 bit pattern:
// negatives bit-inverted, non-negatives with the sign bit set, NaN largest,
// so -0 < +0.
//   1. 256-bin histogram of the key's high byte -> the bin b1 holding the
//      k-th largest key;
//   2. 256-bin histogram of the low byte among keys with high byte b1 ->
//      the exact k-th largest key T.
//      Both histograms are privatized per lane (bin*64 + lane): PopKV's
//      scores are peaked, so a shared histogram would serialize on
//      same-address LDS atomics; with one copy per lane no two lanes of an
//      instruction touch the same word.  The 64 copies are then summed.
//   3. keys > T are selected; keys == T fill the remaining slots in ascending
//      token order (PyTorch's gather-top-k tie rule).  One block scan of the
//      packed per-thread (greater, equal) counts gives every selected token
//      its slot in ascending token order; slots are filled in LDS and the
//      finished list is copied out with coalesced stores.
#include "device_common.h"
#include "kernels.h"

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

constexpr int kStageMax = 8192;  // selections staged in LDS (k <= 8192)

template <int SEG, bool VEC, typename IdxT>
__global__ __launch_bounds__(kSelThreads) void topk_select_kernel(
    const uint16_t* __restrict__ scores, int64_t row_stride, int64_t tokens, int64_t k, int64_t current,
    IdxT* __restrict__ out, int64_t out_stride) {
    static_assert(SEG % 8 == 0, "segments are whole 16-byte chunks");
    const int64_t row = blockIdx.x;
    const uint16_t* src = scores + row * row_stride;
    IdxT* dst = out + row * out_stride;
    const int tid = threadIdx.x;

    if (k >= tokens) {  // every cached token is selected
        for (int64_t t = tid; t < tokens; t += kSelThreads) dst[t] = static_cast<IdxT>(t);
        if (tid == 0) dst[tokens] = static_cast<IdxT>(current);
        return;
    }
    if (k == 0) {
        if (tid == 0) dst[0] = static_cast<IdxT>(current);
        return;
    }

    __shared__ uint32_t hist[kBins * kWave];  // [bin][lane]
    __shared__ uint32_t tot[kBins];
    __shared__ uint32_t scan_sh[kSelWaves + 1];
    __shared__ uint32_t s_bin, s_above;
    __shared__ int32_t stage[kStageMax];
    const int lane = tid & (kWave - 1);

    // ---- load this thread's segment; absent tokens are never counted (n below)
    const int64_t begin = static_cast<int64_t>(tid) * SEG;
    const int n = static_cast<int>(max<int64_t>(0, min<int64_t>(SEG, tokens - begin)));
    uint32_t kp[SEG / 2];
#pragma unroll
    for (int c = 0; c < SEG / 8; ++c) {
        if (VEC && 8 * c + 8 <= n) {
            const uint4 u = *reinterpret_cast<const uint4*>(src + begin + 8 * c);
            const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
            for (int j = 0; j < 4; ++j) kp[4 * c + j] = order_key(w[j] & 0xffffu) | (order_key(w[j] >> 16) << 16);
        } else {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int e = 8 * c + 2 * j;
                const uint32_t a = e < n ? order_key(src[begin + e]) : 0u;
                const uint32_t b = e + 1 < n ? order_key(src[begin + e + 1]) : 0u;
                kp[4 * c + j] = a | (b << 16);
            }
        }
    }
#define POPKV_KEY(e) ((kp[(e) >> 1] >> (((e) & 1) * 16)) & 0xffffu)

    // Sums the 64 per-lane copies into tot[]: thread (bin, quarter) adds 16
    // copies, then the four quarters of a bin (adjacent lanes) combine.  The
    // copy order is rotated by bin so a wave's 64 reads hit 64 banks.
    auto reduce_hist = [&]() {
        const int bin = tid >> 2, q = tid & 3;
        uint32_t v = 0;
#pragma unroll
        for (int c = 0; c < 16; ++c) v += hist[bin * kWave + q * 16 + ((c + bin) & 15)];
        v += __shfl_xor(v, 1);
        v += __shfl_xor(v, 2);
        if (q == 0) tot[bin] = v;
    };

    // ---- level 1: high byte
    for (int i = tid; i < kBins * kWave; i += kSelThreads) hist[i] = 0u;
    __syncthreads();
#pragma unroll
    for (int e = 0; e < SEG; ++e)
        if (e < n) atomicAdd(&hist[(POPKV_KEY(e) >> 8) * kWave + lane], 1u);
    __syncthreads();
    reduce_hist();
    __syncthreads();
    if (tid < kWave) find_bin<kBins>(tot, static_cast<uint32_t>(k), &s_bin, &s_above);
    __syncthreads();
    const uint32_t b1 = s_bin;
    const uint32_t above1 = s_above;

    // ---- level 2: low byte inside bin b1
    for (int i = tid; i < kBins * kWave; i += kSelThreads) hist[i] = 0u;
    __syncthreads();
#pragma unroll
    for (int e = 0; e < SEG; ++e) {
        const uint32_t key = POPKV_KEY(e);
        if (e < n && (key >> 8) == b1) atomicAdd(&hist[(key & 0xffu) * kWave + lane], 1u);
    }
    __syncthreads();
    reduce_hist();
    __syncthreads();
    if (tid < kWave) find_bin<kBins>(tot, static_cast<uint32_t>(k) - above1, &s_bin, &s_above);
    __syncthreads();
    const uint32_t thr = (b1 << 8) | s_bin;
    const uint32_t need_eq = static_cast<uint32_t>(k) - above1 - s_above;

    // ---- ordered selection: slot of a selected token = (#greater before it)
    //      + min(#equal before it, need_eq)
    uint32_t n_gt = 0, n_eq = 0;
#pragma unroll
    for (int e = 0; e < SEG; ++e) {
        const uint32_t key = POPKV_KEY(e);
        if (e < n) {
            n_gt += key > thr ? 1u : 0u;
            n_eq += key == thr ? 1u : 0u;
        }
    }
    uint32_t total, gt_before, eq_before;
    if (tokens <= 0xffff) {  // both prefix counts fit 16 bits: one packed scan
        const uint32_t packed = block_excl_scan(n_gt | (n_eq << 16), scan_sh, kSelWaves, &total);
        gt_before = packed & 0xffffu;
        eq_before = packed >> 16;
    } else {
        gt_before = block_excl_scan(n_gt, scan_sh, kSelWaves, &total);
        eq_before = block_excl_scan(n_eq, scan_sh, kSelWaves, &total);
    }
    const bool staged = k <= kStageMax;
#pragma unroll
    for (int e = 0; e < SEG; ++e) {
        const uint32_t key = POPKV_KEY(e);
        if (e >= n) continue;
        uint32_t slot = 0xffffffffu;
        if (key > thr) {
            slot = gt_before + min(eq_before, need_eq);
            ++gt_before;
        } else if (key == thr) {
            if (eq_before < need_eq) slot = gt_before + eq_before;
            ++eq_before;
        }
        if (slot != 0xffffffffu) {
            if (staged) stage[slot] = static_cast<int32_t>(begin + e);
            else dst[slot] = static_cast<IdxT>(begin + e);
        }
    }
#undef POPKV_KEY
    if (staged) {
        __syncthreads();
        for (int64_t i = tid; i < k; i += kSelThreads) dst[i] = static_cast<IdxT>(stage[i]);
    }
    if (tid == 0) dst[k] = static_cast<IdxT>(current);
}

// Layer-step select, bit-mask form.  The input rows hold radix order keys and
// the scorer has accumulated each row's high-byte histogram into ghist, so
// the first radix level costs nothing here.  Thread t of the block handles
// tokens t, t + 1024, t + 2048, ...: round j of a wave covers 64 consecutive
// tokens, so one ballot of a comparison is directly that 64-token word of the
// selection mask, and lane j of the wave collects round j's words for one
// store at the end.
//   1. bin b1 of the k-th largest key from ghist;
//   2. 256-bin histogram of the low byte of the keys with high byte b1 ->
//      the k-th largest key T, need_eq = how many keys equal to T are taken;
//   3. one pass builds, per 64-token word, the bits of keys > T and of keys
//      == T.  If some keys equal to T are left out, the last one taken is the
//      need_eq-th in token order (PyTorch's gather-top-k tie rule: the lowest
//      indices win): the tie words go to LDS, one wave scans their
//      popcounts, finds the word holding that tie and, one lane per bit,
//      the token tau;
//   4. mask word = (key > T bits) | (key == T bits of tokens <= tau).
// Absent tokens (past `tokens`) get key 0, below every real key (real keys
// are >= 0x03ff; NaN patterns map to 0xffff).  Rows of up to JB rounds keep
// their keys and words in registers (tokens <= 32768 for JB = 32); longer
// rows take the MULTI path, which re-reads keys per pass and keeps the words
// in LDS.  The mask row holds ceil(tokens/64) 64-bit words, bits past
// `tokens` zero.  ghist is re-zeroed for the next call.
constexpr int kMaskMaxRounds = 128;                          // tokens <= 131072
constexpr int kMaskWordSlots = kMaskMaxRounds * kSelWaves;  // 64-bit words per row

template <int JB, bool MULTI>
__global__ __launch_bounds__(kSelThreads) void topk_mask_kernel(
    const uint16_t* __restrict__ keys, uint32_t* __restrict__ ghist, int64_t row_stride, int ntok, int k,
    uint32_t* __restrict__ mask, int64_t mask_stride) {
    static_assert(JB <= kWave, "one collecting lane per round");
    constexpr int SLOTS = MULTI ? kMaskWordSlots : JB * kSelWaves;
    const int64_t row = blockIdx.x;
    const uint16_t* src = keys + row * row_stride;
    uint32_t* gh = ghist + row * kBins;
    uint32_t* mrow = mask + row * mask_stride;
    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = tid / kWave;
    const int rounds = (ntok + kSelThreads - 1) / kSelThreads;

    __shared__ uint32_t tot[kBins], hist2[kBins];
    __shared__ uint32_t s_bin, s_above, s_tau;
    __shared__ uint64_t s_eq[SLOTS];
    __shared__ uint64_t s_gt[MULTI ? SLOTS : 1];
    if (tid < kBins) {
        tot[tid] = gh[tid];
        gh[tid] = 0u;
        hist2[tid] = 0u;
    }
    // mode 0: nothing selected (k == 0); 1: every token (k >= ntok); 2: threshold
    const int mode = k <= 0 ? 0 : (k >= ntok ? 1 : 2);
    if (mode != 2) {
        for (int j0 = 0; j0 < rounds; j0 += JB) {
            uint32_t wl = 0, wh = 0;
#pragma unroll
            for (int jj = 0; jj < JB; ++jj) {
                const uint64_t word = mode == 1 ? __ballot((j0 + jj) * kSelThreads + tid < ntok) : 0ull;
                wl = lane == jj ? static_cast<uint32_t>(word) : wl;
                wh = lane == jj ? static_cast<uint32_t>(word >> 32) : wh;
            }
            const int wbase = (j0 + lane) * kSelThreads + wave * kWave;
            if (lane < JB && wbase < ntok) *reinterpret_cast<uint2*>(mrow + wbase / 32) = make_uint2(wl, wh);
        }
        return;
    }
    uint32_t kr[JB];
    auto load = [&](int j0) {
#pragma unroll
        for (int jj = 0; jj < JB; ++jj) {
            const int t = (j0 + jj) * kSelThreads + tid;
            const uint32_t v = src[min(t, ntok - 1)];
            kr[jj] = t < ntok ? v : 0u;
        }
    };
    if (!MULTI) load(0);
    __syncthreads();
    if (tid < kWave) find_bin<kBins>(tot, static_cast<uint32_t>(k), &s_bin, &s_above);
    __syncthreads();
    const uint32_t b1 = s_bin;
    const uint32_t above1 = s_above;
    for (int j0 = 0; j0 < rounds; j0 += JB) {
        if (MULTI) load(j0);
#pragma unroll
        for (int jj = 0; jj < JB; ++jj)
            if ((kr[jj] >> 8) == b1) atomicAdd(&hist2[kr[jj] & 0xffu], 1u);
        if (!MULTI) break;
    }
    __syncthreads();
    if (tid < kWave) find_bin<kBins>(hist2, static_cast<uint32_t>(k) - above1, &s_bin, &s_above);
    __syncthreads();
    const uint32_t thr = (b1 << 8) | s_bin;
    const uint32_t need_eq = static_cast<uint32_t>(k) - above1 - s_above;
    const bool partial = need_eq < hist2[s_bin];  // block-uniform

    // 3. per-word bits of key > T and key == T; lane jj of each wave holds
    //    round j0 + jj's words
    uint32_t gl = 0, gh_ = 0, el = 0, eh = 0;
    for (int j0 = 0; j0 < rounds; j0 += JB) {
        if (MULTI) load(j0);
#pragma unroll
        for (int jj = 0; jj < JB; ++jj) {
            const uint64_t gt = __ballot(kr[jj] > thr);
            const uint64_t eq = __ballot(kr[jj] == thr);
            const bool mine = lane == jj;
            gl = mine ? static_cast<uint32_t>(gt) : gl;
            gh_ = mine ? static_cast<uint32_t>(gt >> 32) : gh_;
            el = mine ? static_cast<uint32_t>(eq) : el;
            eh = mine ? static_cast<uint32_t>(eq >> 32) : eh;
        }
        if (lane < JB && j0 + lane < rounds) {
            const int e = (j0 + lane) * kSelWaves + wave;  // word index in token order
            if (MULTI || partial) s_eq[e] = (static_cast<uint64_t>(eh) << 32) | el;
            if (MULTI) s_gt[e] = (static_cast<uint64_t>(gh_) << 32) | gl;
        }
        if (!MULTI) break;
    }
    int tau = ntok;
    if (partial) {
        // the word holding the need_eq-th tie (token order = word order):
        // wave 0, lane l owns words [l*PERW, l*PERW + PERW), one DPP scan
        __syncthreads();
        if (tid < kWave) {
            constexpr int PERW = SLOTS / kWave;
            const int n_slots = rounds * kSelWaves;
            uint32_t local = 0;
            for (int i = 0; i < PERW; ++i) {
                const int e = lane * PERW + i;
                local += e < n_slots ? static_cast<uint32_t>(__popcll(s_eq[e])) : 0u;
            }
            const uint32_t excl = wave_incl_scan(local, lane) - local;
            // the crossing lane, then (uniformly) its crossing word
            const uint64_t cross = __ballot(excl < need_eq && excl + local >= need_eq);
            const int owner = static_cast<int>(__builtin_ctzll(cross));
            uint32_t run = __builtin_amdgcn_readlane(excl, owner);
            int e = owner * PERW;
            uint64_t m = s_eq[e];
            for (int i = 0; i < PERW; ++i) {
                m = s_eq[owner * PERW + i];
                const uint32_t c = static_cast<uint32_t>(__popcll(m));
                e = owner * PERW + i;
                if (run + c >= need_eq) break;
                run += c;
            }
            // the (need_eq - run)-th set bit of m: lane b holds bit b and its
            // rank among the set bits below it
            const uint32_t below = __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(m >> 32),
                                                             __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(m), 0u));
            const uint64_t hit = __ballot(((m >> lane) & 1ull) && below == need_eq - run - 1);
            if (lane == 0)
                s_tau = static_cast<uint32_t>((e / kSelWaves) * kSelThreads + (e % kSelWaves) * kWave +
                                              __builtin_ctzll(hit));
        }
        __syncthreads();
        tau = static_cast<int>(s_tau);
    }
    // 4. final words: ties only up to tau
    auto finish = [&](uint64_t gt, uint64_t eq, int wbase) {
        if (eq != 0ull && tau < wbase + kWave) {
            const int keep = tau - wbase + 1;  // tie bits [0, keep) stay
            eq = keep <= 0 ? 0ull : (eq & ((keep >= kWave) ? ~0ull : ((1ull << keep) - 1ull)));
        }
        return gt | eq;
    };
    if (!MULTI) {
        const int wbase = lane * kSelThreads + wave * kWave;
        if (lane < JB && wbase < ntok) {
            const uint64_t w = finish((static_cast<uint64_t>(gh_) << 32) | gl, (static_cast<uint64_t>(eh) << 32) | el,
                                      wbase);
            *reinterpret_cast<uint2*>(mrow + wbase / 32) = make_uint2(static_cast<uint32_t>(w),
                                                                      static_cast<uint32_t>(w >> 32));
        }
    } else {
        __syncthreads();
        for (int e = tid; e < rounds * kSelWaves; e += kSelThreads) {
            const int wbase = (e / kSelWaves) * kSelThreads + (e % kSelWaves) * kWave;
            if (wbase >= ntok) continue;
            const uint64_t w = finish(s_gt[e], s_eq[e], wbase);
            *reinterpret_cast<uint2*>(mrow + wbase / 32) = make_uint2(static_cast<uint32_t>(w),
                                                                      static_cast<uint32_t>(w >> 32));
        }
    }
}

// Ascending indices of a selection mask, the current token in slot k.
// One 1024-thread block per row; thread t owns WPT consecutive mask words.
template <int WPT, typename IdxT>
__global__ __launch_bounds__(kSelThreads) void mask_to_indices_kernel(
    const uint32_t* __restrict__ mask, int64_t mask_stride, int64_t tokens, int64_t k, int64_t current,
    IdxT* __restrict__ out, int64_t out_stride) {
    const int64_t row = blockIdx.x;
    const uint32_t* mrow = mask + row * mask_stride;
    IdxT* dst = out + row * out_stride;
    const int tid = threadIdx.x;
    const int64_t nwords = (tokens + 31) / 32;
    __shared__ uint32_t scan_sh[kSelWaves + 1];
    uint32_t w[WPT], cnt = 0;
#pragma unroll
    for (int i = 0; i < WPT; ++i) {
        const int64_t e = static_cast<int64_t>(tid) * WPT + i;
        w[i] = e < nwords ? mrow[e] : 0u;
        cnt += __popc(w[i]);
    }
    uint32_t total;
    uint32_t pos = block_excl_scan_once(cnt, scan_sh, kSelWaves, &total);
#pragma unroll
    for (int i = 0; i < WPT; ++i) {
        const int64_t tbase = (static_cast<int64_t>(tid) * WPT + i) * 32;
        for (uint32_t m = w[i]; m; m &= m - 1) {
            if (pos < static_cast<uint64_t>(k)) dst[pos] = static_cast<IdxT>(tbase + __builtin_ctz(m));
            ++pos;
        }
    }
    if (tid == 0) dst[k] = static_cast<IdxT>(current);
}

template <int SEG, typename IdxT>
void launch_seg(const uint16_t* scores, int64_t rows, int64_t row_stride, int64_t tokens, int64_t k,
                int64_t current, IdxT* out, int64_t out_stride, bool vec, hipStream_t stream) {
    dim3 grid(static_cast<unsigned>(rows)), block(kSelThreads);
    if (vec)
        hipLaunchKernelGGL((topk_select_kernel<SEG, true, IdxT>), grid, block, 0, stream, scores, row_stride, tokens,
                           k, current, out, out_stride);
    else
        hipLaunchKernelGGL((topk_select_kernel<SEG, false, IdxT>), grid, block, 0, stream, scores, row_stride,
                           tokens, k, current, out, out_stride);
}

template <typename IdxT>
hipError_t launch_select_t(const uint16_t* scores, int64_t rows, int64_t row_stride, int64_t tokens, int64_t k,
                           int64_t current, IdxT* out, int64_t out_stride, hipStream_t stream) {
    const int64_t per = (tokens + kSelThreads - 1) / kSelThreads;
    const bool vec = reinterpret_cast<uintptr_t>(scores) % 16 == 0 && row_stride % 8 == 0;
    if (per <= 8) launch_seg<8>(scores, rows, row_stride, tokens, k, current, out, out_stride, vec, stream);
    else if (per <= 16) launch_seg<16>(scores, rows, row_stride, tokens, k, current, out, out_stride, vec, stream);
    else if (per <= 32) launch_seg<32>(scores, rows, row_stride, tokens, k, current, out, out_stride, vec, stream);
    else if (per <= 64) launch_seg<64>(scores, rows, row_stride, tokens, k, current, out, out_stride, vec, stream);
    else launch_seg<128>(scores, rows, row_stride, tokens, k, current, out, out_stride, vec, stream);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_topk_mask(const uint16_t* keys, uint32_t* ghist, int64_t rows, int64_t row_stride, int64_t tokens,
                            int64_t k, uint32_t* mask, int64_t mask_stride, hipStream_t stream) {
    if (rows <= 0) return hipSuccess;
    const int64_t rounds = (tokens + kSelThreads - 1) / kSelThreads;
    const int nt = static_cast<int>(tokens), kk = static_cast<int>(k < tokens ? k : tokens);
    dim3 grid(static_cast<unsigned>(rows)), block(kSelThreads);
#define POPKV_MASK(JB, MULTI)                                                                                   \
    hipLaunchKernelGGL((topk_mask_kernel<JB, MULTI>), grid, block, 0, stream, keys, ghist, row_stride, nt, kk, \
                       mask, mask_stride)
    if (rounds <= 8) POPKV_MASK(8, false);
    else if (rounds <= 16) POPKV_MASK(16, false);
    else if (rounds <= 32) POPKV_MASK(32, false);
    else POPKV_MASK(32, true);
#undef POPKV_MASK
    return hipGetLastError();
}

hipError_t launch_mask_to_indices(const uint32_t* mask, int64_t rows, int64_t mask_stride, int64_t tokens, int64_t k,
                                  int64_t current, int64_t* indices, int64_t index_row_stride, hipStream_t stream) {
    if (rows <= 0) return hipSuccess;
    const int64_t words = (tokens + 31) / 32;
    dim3 grid(static_cast<unsigned>(rows)), block(kSelThreads);
    if (words <= kSelThreads)
        hipLaunchKernelGGL((mask_to_indices_kernel<1, int64_t>), grid, block, 0, stream, mask, mask_stride, tokens, k,
                           current, indices, index_row_stride);
    else if (words <= 2 * kSelThreads)
        hipLaunchKernelGGL((mask_to_indices_kernel<2, int64_t>), grid, block, 0, stream, mask, mask_stride, tokens, k,
                           current, indices, index_row_stride);
    else
        hipLaunchKernelGGL((mask_to_indices_kernel<4, int64_t>), grid, block, 0, stream, mask, mask_stride, tokens, k,
                           current, indices, index_row_stride);
    return hipGetLastError();
}

hipError_t launch_topk_select(const uint16_t* scores, int64_t rows, int64_t row_stride, int64_t tokens, int64_t k,
                              int64_t current, void* indices, int index_dtype, int64_t index_row_stride,
                              hipStream_t stream) {
    if (rows <= 0) return hipSuccess;
    if (index_dtype == POPKV_INDEX_I32)
        return launch_select_t(scores, rows, row_stride, tokens, k, current, static_cast<int32_t*>(indices),
                               index_row_stride, stream);
    return launch_select_t(scores, rows, row_stride, tokens, k, current, static_cast<int64_t*>(indices),
                           index_row_stride, stream);
}

}  // namespace popkv
