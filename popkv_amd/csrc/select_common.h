// Selection helpers shared by the layer step's chunked select kernels
// (select.hip: per-chunk low-byte histograms; attention.hip: the fused
// select + attention kernel).  Keys are the radix order keys of fp16 scores
// (order_key); absent tokens read as key 0, below every real key (real keys
// are >= 0x03ff), so they never reach the threshold bucket.
#pragma once
#include "device_common.h"
#include "kernels.h"

namespace popkv {

// Cached tokens of sequence b of a batched step, clamped into [0, bound].
__device__ __forceinline__ int64_t seq_tokens_of(const SeqTable& seq, int64_t b, int64_t bound) {
    const int64_t t = seq.tokens[b];
    return t < 0 ? 0 : (t > bound ? bound : t);
}

// Tokens of a chunk: one workgroup of kChunkThreads threads, KPT consecutive
// tokens per thread, so a chunk is kChunkThreads * KPT tokens.
constexpr int kChunkThreads = 256;
constexpr int kMaxChunkKeys = 32;  // KPT <= 32: one 32-bit mask per thread

// Registers holding KPT keys packed two per 32-bit word.
template <int KPT> struct ChunkKeys {
    static_assert(KPT == 1 || KPT % 2 == 0, "whole 32-bit words of keys");
    static_assert(KPT <= kMaxChunkKeys, "one mask word per thread");
    static constexpr int W = KPT >= 2 ? KPT / 2 : 1;
    uint32_t w[W];
    __device__ __forceinline__ uint32_t key(int e) const { return (w[e >> 1] >> ((e & 1) * 16)) & 0xffffu; }
};

// Keys [begin, begin + n) of a row (n in [0, KPT]); keys past n read as 0.
// `row` starts 256-byte aligned and begin is a multiple of KPT, so loads of
// the widest size that divides 2*KPT bytes are aligned.  Every load is
// issued before any is used; a load past the row's tokens re-reads the
// row's first keys and is zeroed.  load_chunk_keys_raw issues the loads for
// the first n keys (the rest re-read the row's start, unmasked);
// mask_chunk_keys then zeroes every key at or past n (which may be smaller
// than the n the loads were issued for).  COH: device-coherent loads (keys
// written by other workgroups of the same launch; KPT a multiple of 4).
template <int KPT, bool COH = false>
__device__ __forceinline__ void load_chunk_keys_raw(const uint16_t* __restrict__ row, int begin, int n,
                                                    ChunkKeys<KPT>& k) {
    static_assert(!COH || KPT % 4 == 0, "device-coherent key loads: 8-byte words");
    if constexpr (KPT % 8 == 0) {
        uint4 u[KPT / 8];
#pragma unroll
        for (int c = 0; c < KPT / 8; ++c)
            u[c] = ld_u4<COH>(reinterpret_cast<const uint4*>(8 * c < n ? row + begin + 8 * c : row));
#pragma unroll
        for (int c = 0; c < KPT / 8; ++c) {
            k.w[4 * c] = u[c].x;
            k.w[4 * c + 1] = u[c].y;
            k.w[4 * c + 2] = u[c].z;
            k.w[4 * c + 3] = u[c].w;
        }
    } else if constexpr (KPT % 4 == 0) {
        uint2 u[KPT / 4];
#pragma unroll
        for (int c = 0; c < KPT / 4; ++c) {
            const uint16_t* src = 4 * c < n ? row + begin + 4 * c : row;
            if constexpr (COH) {
                const uint64_t x = __hip_atomic_load(reinterpret_cast<uint64_t*>(const_cast<uint16_t*>(src)),
                                                     __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                u[c] = make_uint2(static_cast<uint32_t>(x), static_cast<uint32_t>(x >> 32));
            } else {
                u[c] = *reinterpret_cast<const uint2*>(src);
            }
        }
#pragma unroll
        for (int c = 0; c < KPT / 4; ++c) {
            k.w[2 * c] = u[c].x;
            k.w[2 * c + 1] = u[c].y;
        }
    } else if constexpr (KPT % 2 == 0) {
        uint32_t u[KPT / 2];
#pragma unroll
        for (int c = 0; c < KPT / 2; ++c) u[c] = *reinterpret_cast<const uint32_t*>(2 * c < n ? row + begin + 2 * c : row);
#pragma unroll
        for (int c = 0; c < KPT / 2; ++c) k.w[c] = u[c];
    } else {
        k.w[0] = row[n > 0 ? begin : 0];
    }
}

template <int KPT>
__device__ __forceinline__ void mask_chunk_keys(int n, ChunkKeys<KPT>& k) {
    if (n < KPT) {  // the row's ragged end (or a thread past it)
#pragma unroll
        for (int i = 0; i < ChunkKeys<KPT>::W; ++i)
            k.w[i] &= (2 * i + 1 < n ? 0xffff0000u : 0u) | (2 * i < n ? 0x0000ffffu : 0u);
    }
}

template <int KPT>
__device__ __forceinline__ void load_chunk_keys(const uint16_t* __restrict__ row, int begin, int n,
                                                ChunkKeys<KPT>& k) {
    load_chunk_keys_raw<KPT>(row, begin, n, k);
    mask_chunk_keys<KPT>(n, k);
}

// Bit masks of the thread's keys: bit e of *gt = key e > thr, of *eq =
// key e == thr.  Two instructions per key and mask: the sign of thr - key
// (resp. thr - 1 - key) shifted in with v_alignbit, last key first.
template <int KPT>
__device__ __forceinline__ void key_masks(const ChunkKeys<KPT>& k, uint32_t thr, uint32_t* gt, uint32_t* eq) {
    uint32_t g = 0u, ge = 0u;
#pragma unroll
    for (int e = KPT - 1; e >= 0; --e) {
        const uint32_t key = k.key(e);
        g = __builtin_amdgcn_alignbit(g, thr - key, 31);
        ge = __builtin_amdgcn_alignbit(ge, thr - 1u - key, 31);
    }
    *gt = g;
    *eq = ge & ~g;
}

// Radix-select step on a 256-bin histogram held by one wave, lane l holding
// the counts of ranks 4l .. 4l+3 counted from the top bin (rank r = bin
// 255 - r) in c[0..3].  Finds the bin where the running count from the top
// first reaches `need` (1 <= need <= total) and the count strictly above
// it.  Wave-uniform results; all 64 lanes must be active.
__device__ __forceinline__ void wave_find_bin(const uint32_t (&c)[4], uint32_t need, uint32_t* bin,
                                              uint32_t* above) {
    const int lane = threadIdx.x & (kWave - 1);
    const uint32_t local = c[0] + c[1] + c[2] + c[3];
    const uint32_t incl = wave_incl_scan(local, lane);
    uint32_t run = incl - local;
    const bool cross = run < need && need <= incl;
    uint32_t r = 0;
    bool done = false;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        if (!done && run + c[i] < need) {
            run += c[i];
            ++r;
        } else {
            done = true;
        }
    }
    const uint64_t hit = __ballot(cross);
    const int src = hit != 0 ? __builtin_ctzll(hit) : 0;
    const uint32_t rank = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(4 * lane + r), src));
    *bin = 255u - min(rank, 255u);  // (rank <= 255 whenever 1 <= need <= total)
    *above = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(run), src));
}

// Counts of the 256 bins [252 - 4l, 255 - 4l] of a histogram row in global
// memory for lane l, in rank order (one 16-byte load; the row is 16-byte
// aligned).
__device__ __forceinline__ void load_rank4(const uint32_t* __restrict__ hist, uint32_t (&c)[4]) {
    const int lane = threadIdx.x & (kWave - 1);
    const uint4 u = reinterpret_cast<const uint4*>(hist)[63 - lane];
    c[0] = u.w;
    c[1] = u.z;
    c[2] = u.y;
    c[3] = u.x;
}

// Chunking of a layer step's key rows: chunks of 256 * kpt tokens.  When
// the selection is spread evenly a chunk holds about k * chunk / tokens
// selected tokens; the chunk is the largest one expected to hold at most
// kChunkSelected of them.  At most 64 chunks; kpt from kChunkKpt (at most
// 32 keys per thread).  Measured at C1 (32K tokens, k = 4095) with 10 rows
// per slot and gather pass: 256 selected per chunk (16 chunks of 2048)
// 30.5 us per layer step, 192 (22 chunks of 1536) 33.6 us.  A step of few
// rows (query heads x sequences) also gets at least kStepMinBlocks / rows
// chunks, down to the smallest chunk (256 tokens): with the even-spread rule
// alone C0 (8 rows, k = 511 of 4095) ran 16 blocks on the GPU's 256 CUs --
// 17.3 us per step against 16.1 with 16 chunks of 256 tokens.
constexpr int kChunkSelected = 256;
constexpr int64_t kStepMinBlocks = 256;
constexpr int kChunkKpt[] = {1, 2, 4, 6, 8, 12, 16, 24, 32};

struct StepChunks {
    int kpt;
    int64_t tokens_per_chunk, count;
};

inline StepChunks step_chunks(int64_t tokens, int64_t k, int64_t rows) {
    StepChunks c{1, kChunkThreads, 0};
    if (tokens <= 0) return c;
    // tokens per chunk wanted: about kChunkSelected selected ones, few enough
    // that rows * chunks reaches kStepMinBlocks, at least tokens / 64
    int64_t want = k > 0 ? tokens * kChunkSelected / k : tokens;
    if (rows > 0 && rows < kStepMinBlocks && want > tokens * rows / kStepMinBlocks)
        want = tokens * rows / kStepMinBlocks;
    const int64_t floor64 = (tokens + 63) / 64;
    if (want < floor64) want = floor64;
    int kpt = 1;
    for (int x : kChunkKpt)
        if (static_cast<int64_t>(x) * kChunkThreads <= want) kpt = x;
    while (kpt < kMaxChunkKeys && (tokens + kpt * kChunkThreads - 1) / (kpt * kChunkThreads) > 64) {
        int next = kMaxChunkKeys;
        for (int x : kChunkKpt)
            if (x > kpt && x < next) next = x;
        kpt = next;
    }
    c.kpt = kpt;
    c.tokens_per_chunk = static_cast<int64_t>(kpt) * kChunkThreads;
    c.count = (tokens + c.tokens_per_chunk - 1) / c.tokens_per_chunk;
    return c;
}

}  // namespace popkv
