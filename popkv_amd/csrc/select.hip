// Per-query-head top-k over fp16 scores with the current token reserving the
// last slot (gfx950).
//
// Replaces torch.topk(scores, k, dim=-1, sorted=False).indices followed by
// _append_current (reference popkv.py:1094-1098, :287-291).
//
// One 1024-thread workgroup (16 wave64s) per row.  Thread i owns a contiguous
// segment of the row and keeps its keys in registers (two 16-bit keys per
// VGPR).  The key is PyTorch's radix order of an fp16 bit pattern: negatives
// bit-inverted, non-negatives with the sign bit set, NaN largest, so -0 < +0.
//   1. 256-bin histogram of the key's high byte (per-wave LDS histograms),
//      suffix scan -> the high byte d1 of the k-th largest key;
//   2. 256-bin histogram of the low byte among keys with high byte d1 ->
//      the exact k-th largest key T;
//   3. every key > T is selected; keys == T fill the remaining slots in
//      ascending token order (a block scan of per-thread tie counts), which is
//      what PyTorch's gather-top-k does with ties;
//   4. a block scan of per-thread selection counts gives each thread its
//      output offset, so indices come out in ascending token order.
#include "device_common.h"
#include "kernels.h"

namespace popkv {
namespace {

constexpr int kSelThreads = 1024;
constexpr int kSelWaves = kSelThreads / kWave;

__device__ __forceinline__ uint32_t order_key(uint32_t h) {
    const bool nan = ((h & 0x7c00u) == 0x7c00u) && (h & 0x3ffu);
    const uint32_t k = (h & 0x8000u) ? (~h & 0xffffu) : (h | 0x8000u);
    return nan ? 0xffffu : k;
}

// Finds the bin holding the `need`-th largest element of a 256-bin histogram
// `tot` (1 <= need <= total).  Wave 0 scans bins from the top; the winning
// lane stores the bin and the count strictly above it.
__device__ __forceinline__ void find_bin(const uint32_t* tot, uint32_t need, uint32_t* s_bin, uint32_t* s_above) {
    const int lane = threadIdx.x & (kWave - 1);
    uint32_t c[4];
    uint32_t local = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        c[i] = tot[255 - (4 * lane + i)];
        local += c[i];
    }
    const uint32_t incl = wave_incl_scan(local, lane);
    uint32_t running = incl - local;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        if (running < need && running + c[i] >= need) {
            *s_bin = 255u - static_cast<uint32_t>(4 * lane + i);
            *s_above = running;
        }
        running += c[i];
    }
}

template <int SEG, typename IdxT>
__global__ __launch_bounds__(kSelThreads) void topk_select_kernel(
    const uint16_t* __restrict__ scores, int64_t row_stride, int64_t tokens, int64_t k, int64_t current,
    IdxT* __restrict__ out, int64_t out_stride, unsigned int* __restrict__ rearm) {
    const int64_t row = blockIdx.x;
    const uint16_t* src = scores + row * row_stride;
    IdxT* dst = out + row * out_stride;
    const int tid = threadIdx.x;
    const int wave = tid / kWave;
    // Re-arms the per-row completion counter of the fused attention merge that
    // runs after this kernel on the same stream.
    if (rearm != nullptr && tid == 0) rearm[row] = 0u;

    if (k >= tokens) {  // every cached token is selected
        for (int64_t t = tid; t < tokens; t += kSelThreads) dst[t] = static_cast<IdxT>(t);
        if (tid == 0) dst[tokens] = static_cast<IdxT>(current);
        return;
    }
    if (k == 0) {
        if (tid == 0) dst[0] = static_cast<IdxT>(current);
        return;
    }

    __shared__ uint32_t hist[kSelWaves][256];
    __shared__ uint32_t tot[256];
    __shared__ uint32_t scan_sh[kSelWaves + 1];
    __shared__ uint32_t s_bin, s_above;

    const int64_t seg = (tokens + kSelThreads - 1) / kSelThreads;
    const int64_t begin = tid * seg;
    const int n = static_cast<int>(max<int64_t>(0, min<int64_t>(seg, tokens - begin)));

    uint32_t kp[SEG / 2];
#pragma unroll
    for (int j = 0; j < SEG / 2; ++j) {
        const uint32_t a = (2 * j < n) ? order_key(src[begin + 2 * j]) : 0u;
        const uint32_t b = (2 * j + 1 < n) ? order_key(src[begin + 2 * j + 1]) : 0u;
        kp[j] = a | (b << 16);
    }
#define POPKV_KEY(j) ((kp[(j) >> 1] >> (((j) & 1) * 16)) & 0xffffu)

    // ---- level 1: high byte
    for (int i = tid; i < kSelWaves * 256; i += kSelThreads) (&hist[0][0])[i] = 0u;
    __syncthreads();
#pragma unroll
    for (int j = 0; j < SEG; ++j)
        if (j < n) atomicAdd(&hist[wave][POPKV_KEY(j) >> 8], 1u);
    __syncthreads();
    if (tid < 256) {
        uint32_t s = 0;
#pragma unroll
        for (int w = 0; w < kSelWaves; ++w) s += hist[w][tid];
        tot[tid] = s;
    }
    __syncthreads();
    if (wave == 0) find_bin(tot, static_cast<uint32_t>(k), &s_bin, &s_above);
    __syncthreads();
    const uint32_t d1 = s_bin;
    const uint32_t above1 = s_above;

    // ---- level 2: low byte within bucket d1
    for (int i = tid; i < kSelWaves * 256; i += kSelThreads) (&hist[0][0])[i] = 0u;
    __syncthreads();
#pragma unroll
    for (int j = 0; j < SEG; ++j) {
        const uint32_t key = POPKV_KEY(j);
        if (j < n && (key >> 8) == d1) atomicAdd(&hist[wave][key & 0xffu], 1u);
    }
    __syncthreads();
    if (tid < 256) {
        uint32_t s = 0;
#pragma unroll
        for (int w = 0; w < kSelWaves; ++w) s += hist[w][tid];
        tot[tid] = s;
    }
    __syncthreads();
    if (wave == 0) find_bin(tot, static_cast<uint32_t>(k) - above1, &s_bin, &s_above);
    __syncthreads();
    const uint32_t thr = (d1 << 8) | s_bin;
    const uint32_t need_eq = static_cast<uint32_t>(k) - above1 - s_above;

    // ---- level 3: ordered selection
    uint32_t n_gt = 0, n_eq = 0;
#pragma unroll
    for (int j = 0; j < SEG; ++j) {
        const uint32_t key = POPKV_KEY(j);
        if (j < n) {
            n_gt += key > thr ? 1u : 0u;
            n_eq += key == thr ? 1u : 0u;
        }
    }
    uint32_t total;
    const uint32_t eq_before = block_excl_scan(n_eq, scan_sh, kSelWaves, &total);
    const uint32_t take_eq = need_eq > eq_before ? min(need_eq - eq_before, n_eq) : 0u;
    const uint32_t pos0 = block_excl_scan(n_gt + take_eq, scan_sh, kSelWaves, &total);
    uint32_t pos = pos0, taken = 0;
#pragma unroll
    for (int j = 0; j < SEG; ++j) {
        const uint32_t key = POPKV_KEY(j);
        if (j < n) {
            const bool sel = key > thr || (key == thr && taken < take_eq);
            taken += (key == thr && taken < take_eq) ? 1u : 0u;
            if (sel) dst[pos++] = static_cast<IdxT>(begin + j);
        }
    }
#undef POPKV_KEY
    if (tid == 0) dst[k] = static_cast<IdxT>(current);
}

template <typename IdxT>
hipError_t launch_select_t(const uint16_t* scores, int64_t rows, int64_t row_stride, int64_t tokens, int64_t k,
                           int64_t current, IdxT* out, int64_t out_stride, unsigned int* rearm,
                           hipStream_t stream) {
    const int64_t seg = (tokens + kSelThreads - 1) / kSelThreads;
    dim3 grid(static_cast<unsigned>(rows)), block(kSelThreads);
#define POPKV_SEL(S)                                                                                      \
    hipLaunchKernelGGL((topk_select_kernel<S, IdxT>), grid, block, 0, stream, scores, row_stride, tokens, k, \
                       current, out, out_stride, rearm)
    if (seg <= 8) POPKV_SEL(8);
    else if (seg <= 16) POPKV_SEL(16);
    else if (seg <= 32) POPKV_SEL(32);
    else if (seg <= 64) POPKV_SEL(64);
    else POPKV_SEL(128);
#undef POPKV_SEL
    return hipGetLastError();
}

}  // namespace

hipError_t launch_topk_select(const uint16_t* scores, int64_t rows, int64_t row_stride, int64_t tokens, int64_t k,
                              int64_t current, void* indices, int index_dtype, int64_t index_row_stride,
                              unsigned int* rearm_counters, hipStream_t stream) {
    if (rows <= 0) return hipSuccess;
    if (index_dtype == POPKV_INDEX_I32)
        return launch_select_t(scores, rows, row_stride, tokens, k, current, static_cast<int32_t*>(indices),
                               index_row_stride, rearm_counters, stream);
    return launch_select_t(scores, rows, row_stride, tokens, k, current, static_cast<int64_t*>(indices),
                           index_row_stride, rearm_counters, stream);
}

}  // namespace popkv
