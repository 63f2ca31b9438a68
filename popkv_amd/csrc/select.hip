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
// runs on one CU per row.  The list row receives the k selected tokens in
// ascending order (int32); with idx64 non-null the same tokens are written
// as int64 followed by `current` in slot k (the reference's _append_current
// layout).  Absent tokens (past `tokens`) get key 0, below every real key
// (real keys are >= 0x03ff; NaN patterns map to 0xffff).  ghist is
// re-zeroed for the next call.
template <int SEG>
__global__ __launch_bounds__(kSelThreads) void topk_list_kernel(
    const uint16_t* __restrict__ keys, uint32_t* __restrict__ ghist, int64_t row_stride, int ntok, int k,
    int32_t* __restrict__ list, int64_t list_stride, int64_t* __restrict__ idx64, int64_t idx_stride,
    int64_t current) {
    static_assert(SEG % 8 == 0 && SEG <= 128, "whole 16-byte chunks, at most four 32-bit masks");
    constexpr int NM = (SEG + 31) / 32;   // 32-bit masks per thread
    constexpr int MB = SEG < 32 ? SEG : 32;  // bits per mask
    const int64_t row = blockIdx.x;
    const uint16_t* src = keys + row * row_stride;
    uint32_t* gh = ghist + row * kBins;
    int32_t* lrow = list + row * list_stride;
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
    if (irow != nullptr && tid == 0) irow[k] = current;
    // mode 0: nothing selected (k == 0); 1: every token (k >= ntok); 2: threshold
    const int mode = k <= 0 ? 0 : (k >= ntok ? 1 : 2);
    if (mode != 2) {
        if (mode == 1) {
            for (int t = tid; t < ntok; t += kSelThreads) {
                lrow[t] = t;
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
#pragma unroll
        for (int c = 0; c < KW / 4; ++c) {
            const int e0 = 8 * (c0 + c);
            uint4 u = make_uint4(0u, 0u, 0u, 0u);
            if (e0 < n) u = *reinterpret_cast<const uint4*>(seg + e0);
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
                lrow[pos] = t;
                if (irow != nullptr) irow[pos] = t;
            }
            ++pos;
        }
    }
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

hipError_t launch_topk_list(const uint16_t* keys, uint32_t* ghist, int64_t rows, int64_t row_stride, int64_t tokens,
                            int64_t k, int32_t* list, int64_t list_stride, int64_t* idx64, int64_t idx_stride,
                            int64_t current, hipStream_t stream) {
    if (rows <= 0) return hipSuccess;
    const int64_t per = (tokens + kSelThreads - 1) / kSelThreads;
    const int nt = static_cast<int>(tokens), kk = static_cast<int>(k < tokens ? k : tokens);
    dim3 grid(static_cast<unsigned>(rows)), block(kSelThreads);
#define POPKV_LIST(SEG)                                                                                          \
    hipLaunchKernelGGL((topk_list_kernel<SEG>), grid, block, 0, stream, keys, ghist, row_stride, nt, kk, list, \
                       list_stride, idx64, idx_stride, current)
    if (per <= 8) POPKV_LIST(8);
    else if (per <= 16) POPKV_LIST(16);
    else if (per <= 32) POPKV_LIST(32);
    else if (per <= 64) POPKV_LIST(64);
    else POPKV_LIST(128);
#undef POPKV_LIST
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
