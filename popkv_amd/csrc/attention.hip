// Split sparse attention over gathered K/V rows (gfx950).
//
// Replaces indexed_attention_split_partial / _merge (reference
// sparse_kernels.py:237-387).  The step is a per-head GEMV in which every
// query head picks its own rows, so it is bound by HBM bandwidth and uses no
// MFMA.
//
// Partial kernel: one workgroup of 4 wave64s per (query head, split).  A row
// of D bf16 values is read by LPR = D/8 lanes with one 16-byte load each, so
// a wave covers 64/LPR rows per instruction.  The split's indices are staged
// in LDS with one coalesced load; each lane then issues the K and V loads of
// a whole batch of rows before using any of them (deep memory-level
// parallelism for the random 256-byte gathers).  Logits are reduced across
// the LPR lanes of a row with DPP row permutations (VALU only); every row
// slot keeps an online-softmax state (m, l, acc[8]),
// slots are merged within the wave and then across waves through LDS, and
// the split's (m, l, acc[D]) is written as float32.
//
// An index equal to prefix_tokens is the current token: its key/value come
// from current_k/current_v (sparse_kernels.py:267-286).  Rows past `selected`
// or with valid_mask == 0 are skipped.
//
// Merge: out = sum_s acc_s e^{m_s - M} / sum_s l_s e^{m_s - M}, M = max_s m_s,
// cast to the output dtype, one workgroup per query head.  (A last-block
// merge inside the partial kernel would need an agent-scope release per
// workgroup, which on gfx950 writes back the XCD's L2 each time; a separate
// launch is far cheaper.)
#include <type_traits>

#include "device_common.h"
#include "pack128.h"
#include "kernels.h"
#include "score128.h"
#include "select_common.h"

namespace popkv {
namespace {

constexpr int kAttnThreads = 256;
constexpr int kAttnWaves = kAttnThreads / kWave;
constexpr int kAttnStage = 1024;  // indices of one split staged in LDS
// Polls of the single-launch layer step's select blocks before they give up
// waiting for the scorer (each poll is a device-coherent load round trip and
// a short sleep: about 60 ms in all, against a scorer of a few microseconds).
constexpr int kHandoffPolls = 1 << 16;

template <typename T>
__device__ __forceinline__ void load_row8(const T* p, int dim0, int d, float v[8]) {
    if (dim0 + 8 <= d) {
        load8<T>(p + dim0, v);
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = 0.0f;
    }
}

struct SoftmaxState {
    float m, l, acc[8];
};

__device__ __forceinline__ void merge_state(SoftmaxState& a, float m2, float l2, const float* acc2) {
    const float mm = fmaxf(a.m, m2);
    if (mm == -INFINITY) return;
    const float wa = a.m == -INFINITY ? 0.0f : __expf(a.m - mm);
    const float wb = m2 == -INFINITY ? 0.0f : __expf(m2 - mm);
    a.l = a.l * wa + l2 * wb;
#pragma unroll
    for (int i = 0; i < 8; ++i) a.acc[i] = a.acc[i] * wa + acc2[i] * wb;
    a.m = mm;
}

// Writes a workgroup's (m, l, acc[d]) to dst: the row slots of each wave
// (lanes with equal dim slice) merge through shuffles, the waves through LDS.
// All threads of the block call it.
// Partial states handed from one workgroup to another inside a kernel (the
// layer step's fused merge) are written and read as device-scope relaxed
// atomics: plain global stores / loads with the device-coherence bit, which
// go through to memory instead of staying in one XCD's L2, so no L2
// write-back or invalidate is needed for them.
// The fused merges hand chunk states from workgroup to workgroup with no
// release/acquire pair: the states are stored with relaxed agent-scope
// atomic stores, each wave then waits with "s_waitcnt vmcnt(0)", the block
// meets at a barrier, and one relaxed agent-scope atomic add takes the
// ticket; the last block reads the states with relaxed agent-scope atomic
// loads.  That is correct on gfx942 / gfx950 because (1) an agent-scope
// atomic store or load is a global store / load with the sc1 bit, which
// writes through and reads past the XCD's non-coherent L2 to the device's
// coherence point, and (2) stores count in vmcnt on these targets, so
// vmcnt(0) returns only once every store of the wave is acknowledged by
// that point -- before the ticket is taken.  On targets that count stores
// in a separate vscnt (gfx10 and later) or that cache agent-scope stores,
// the wait would not cover the states: the build refuses them.
#if defined(__HIP_DEVICE_COMPILE__) && !defined(__gfx950__) && !defined(__gfx942__)
#error "the fused merge's hand-off relies on gfx942/gfx950 store acknowledgement (vmcnt) and sc1 write-through"
#endif

template <bool COH>
__device__ __forceinline__ void st_f32(float* p, float v) {
    if constexpr (COH) __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    else *p = v;
}
template <bool COH>
__device__ __forceinline__ float ld_f32(const float* p) {
    if constexpr (COH) return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    else return *p;
}

template <int LPR>
__device__ __forceinline__ void store_partial(SoftmaxState st, int lane, int wave, int dim0, int d, float* dst,
                                              bool coherent = false) {
    auto merge_xor = [&](auto mtag) {
        constexpr int M = decltype(mtag)::value;
        const float m2 = lane_xor<M>(st.m);
        const float l2 = lane_xor<M>(st.l);
        float a2[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) a2[i] = lane_xor<M>(st.acc[i]);
        merge_state(st, m2, l2, a2);
    };
    if constexpr (LPR <= 8) merge_xor(std::integral_constant<int, 8>{});
    if constexpr (LPR <= 16) merge_xor(std::integral_constant<int, 16>{});
    merge_xor(std::integral_constant<int, 32>{});
    __shared__ float s_m[kAttnWaves], s_l[kAttnWaves];
    __shared__ float s_acc[kAttnWaves][256];
    if (lane < LPR) {
#pragma unroll
        for (int i = 0; i < 8; ++i) s_acc[wave][dim0 + i] = st.acc[i];
        if (lane == 0) { s_m[wave] = st.m; s_l[wave] = st.l; }
    }
    __syncthreads();
    const int dim = threadIdx.x;
    float mx = -INFINITY;
#pragma unroll
    for (int w = 0; w < kAttnWaves; ++w) mx = fmaxf(mx, s_m[w]);
    float l = 0.0f, a = 0.0f;
#pragma unroll
    for (int w = 0; w < kAttnWaves; ++w) {
        if (s_m[w] == -INFINITY) continue;
        const float wt = __expf(s_m[w] - mx);
        l += s_l[w] * wt;
        if (dim < d) a += s_acc[w][dim] * wt;
    }
    if (coherent) {
        if (dim < d) st_f32<true>(dst + 2 + dim, a);
        if (dim == 0) {
            st_f32<true>(dst, mx);
            st_f32<true>(dst + 1, l);
        }
    } else {
        if (dim < d) dst[2 + dim] = a;
        if (dim == 0) {
            dst[0] = mx;
            dst[1] = l;
        }
    }
}

// Merge `nsplit` states [(m, l, acc[D])] of one head into out[0..D).  The
// states are first staged into LDS with one coalesced burst, so the whole
// merge pays a single memory latency.  With cur_q non-null one more state
// joins the merge: the current token as a single row, logit
// cur_q . cur_k * scale and value cur_v; its operands are loaded in the same
// burst as the states.
constexpr int kMergeThreads = 256;
constexpr int kMergeMaxFloats = 16384;  // 64 KB of staged state
constexpr int kMergeBatch = 16;
constexpr int kMergeMaxSplits = 1024;

template <typename T>
__device__ __forceinline__ void merge_splits(const float* __restrict__ st, int nsplit, int d, T* out,
                                             const T* cur_q = nullptr, const T* cur_k = nullptr,
                                             const T* cur_v = nullptr, float scale = 0.0f) {
    __shared__ __align__(16) float s_state[kMergeMaxFloats];
    __shared__ float s_w[kMergeMaxSplits];
    __shared__ float s_den, s_wc;
    __shared__ float s_dot[kMergeThreads / kWave];
    const int tid = threadIdx.x;
    const int n = nsplit * (d + 2);
    const bool staged = n <= kMergeMaxFloats;
    const bool has_cur = cur_q != nullptr;
    // the current token's operands for this thread's dimension
    float cq = 0.0f, ck = 0.0f, cv = 0.0f;
    if (has_cur && tid < d) {
        cq = Elem<T>::load(cur_q, tid);
        ck = Elem<T>::load(cur_k, tid);
        cv = Elem<T>::load(cur_v, tid);
    }
    if (staged && n % 4 == 0 && reinterpret_cast<uintptr_t>(st) % 16 == 0) {
        // 16-byte loads, kMergeBatch of them in flight per thread before the
        // first LDS write (a plain copy loop waits on every load)
        const float4* st4 = reinterpret_cast<const float4*>(st);
        float4* sh4 = reinterpret_cast<float4*>(s_state);
        const int n4 = n / 4;
        for (int base = 0; base < n4; base += kMergeBatch * kMergeThreads) {
            float4 v[kMergeBatch];
#pragma unroll
            for (int j = 0; j < kMergeBatch; ++j) {
                const int i = base + j * kMergeThreads + tid;
                v[j] = i < n4 ? st4[i] : make_float4(0.f, 0.f, 0.f, 0.f);
            }
#pragma unroll
            for (int j = 0; j < kMergeBatch; ++j) {
                const int i = base + j * kMergeThreads + tid;
                if (i < n4) sh4[i] = v[j];
            }
        }
    } else if (staged) {
        // Batches of kMergeBatch independent loads per thread, all in flight
        // before the first LDS write (a plain copy loop waits on every load).
        for (int base = 0; base < n; base += kMergeBatch * kMergeThreads) {
            float v[kMergeBatch];
#pragma unroll
            for (int j = 0; j < kMergeBatch; ++j) {
                const int i = base + j * kMergeThreads + tid;
                v[j] = i < n ? st[i] : 0.0f;
            }
#pragma unroll
            for (int j = 0; j < kMergeBatch; ++j) {
                const int i = base + j * kMergeThreads + tid;
                if (i < n) s_state[i] = v[j];
            }
        }
    }
    if (has_cur) {
        const float prod = wave_sum(cq * ck);
        if ((tid & (kWave - 1)) == 0) s_dot[tid / kWave] = prod;
    }
    __syncthreads();
    const float* src = staged ? s_state : st;
    // split weights e^{m_s - M} (0 for fully masked splits) and the denominator
    if (tid < kWave) {
        float cur_m = -INFINITY;
        if (has_cur) {
            float dot = 0.0f;
            for (int w = 0; w < kMergeThreads / kWave; ++w) dot += s_dot[w];
            cur_m = dot * scale;
        }
        float mx = cur_m;
        for (int s = tid; s < nsplit; s += kWave) mx = fmaxf(mx, src[s * (d + 2)]);
        mx = wave_max(mx);
        float den = 0.0f;
        for (int s = tid; s < nsplit; s += kWave) {
            const float m = src[s * (d + 2)];
            const float w = m == -INFINITY ? 0.0f : __expf(m - mx);
            s_w[s] = w;
            den += src[s * (d + 2) + 1] * w;
        }
        den = wave_sum(den);
        if (tid == 0) {
            const float wc = cur_m == -INFINITY ? 0.0f : __expf(cur_m - mx);
            s_wc = wc;
            s_den = den + wc;
        }
    }
    __syncthreads();
    for (int dim = tid; dim < d; dim += kMergeThreads) {
        float num = 0.0f;
        for (int s = 0; s < nsplit; ++s) {
            const float w = s_w[s];
            if (w != 0.0f) num += src[s * (d + 2) + 2 + dim] * w;
        }
        if (has_cur) num += s_wc * (dim == tid ? cv : Elem<T>::load(cur_v, dim));
        Elem<T>::store(out, dim, num / s_den);
    }
}

template <typename T, typename IdxT, int LPR, int NB>
__global__ __launch_bounds__(kAttnThreads) void attn_partial_kernel(
    const T* __restrict__ q, const T* __restrict__ kc, const T* __restrict__ vc,
    int64_t k_hs, int64_t k_ts, int64_t v_hs, int64_t v_ts, int64_t prefix_tokens,
    const T* __restrict__ cur_k, const T* __restrict__ cur_v,
    const IdxT* __restrict__ idx, int64_t idx_stride, const uint8_t* __restrict__ valid,
    const int64_t* __restrict__ head_to_kv, int kv_heads, int d, int64_t selected, int split, float scale,
    float* __restrict__ partials, int nsplit) {
    constexpr int SLOTS = kWave / LPR;               // row slots per wave
    constexpr int ROWS_PER_PASS = SLOTS * kAttnWaves;
    const int h = blockIdx.y;
    const int s = blockIdx.x;
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int sub = lane % LPR;                       // dim slice [8*sub, 8*sub+8)
    const int slot = wave * SLOTS + lane / LPR;
    const int dim0 = sub * 8;
    const bool dim_ok = dim0 + 8 <= d;
    // A mapping outside [0, kv_heads) is clamped, never dereferenced.
    const int64_t kvh = min(max(head_to_kv[h], static_cast<int64_t>(0)), static_cast<int64_t>(kv_heads - 1));

    float qv[8];
    load_row8<T>(q + static_cast<int64_t>(h) * d, dim0, d, qv);
    const T* kbase = kc + kvh * k_hs;
    const T* vbase = vc + kvh * v_hs;
    const T* ck = cur_k + kvh * d;
    const T* cv = cur_v + kvh * d;

    const int64_t row0 = static_cast<int64_t>(s) * split;
    const int64_t rows_here = min(static_cast<int64_t>(split), selected - row0);
    const IdxT* irow = idx + static_cast<int64_t>(h) * idx_stride + row0;
    const uint8_t* vrow = valid ? valid + static_cast<int64_t>(h) * idx_stride + row0 : nullptr;

    // Stage this split's indices (and validity) in LDS with coalesced loads;
    // -1 marks a skipped row.  Out-of-range indices are clamped into the
    // cache (as the reference's min(token, prefix_tokens - 1)), never
    // dereferenced.
    __shared__ int64_t s_tok[kAttnStage];
    const bool staged = rows_here <= kAttnStage;
    if (staged) {
        for (int r = threadIdx.x; r < rows_here; r += kAttnThreads) {
            const int64_t t = static_cast<int64_t>(irow[r]);
            const bool live = vrow == nullptr || vrow[r] != 0;
            s_tok[r] = !live ? -1 : (t == prefix_tokens ? t : min(max(t, static_cast<int64_t>(0)), prefix_tokens - 1));
        }
        __syncthreads();
    }

    SoftmaxState st;
    st.m = -INFINITY;
    st.l = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) st.acc[i] = 0.0f;

    for (int64_t base = 0; base < rows_here; base += static_cast<int64_t>(ROWS_PER_PASS) * NB) {
        int64_t tok[NB];
        bool live[NB];
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            const int64_t r = base + static_cast<int64_t>(b) * ROWS_PER_PASS + slot;
            int64_t t = -1;
            if (r < rows_here) {
                if (staged) {
                    t = s_tok[r];
                } else {
                    const int64_t raw = static_cast<int64_t>(irow[r]);
                    const bool ok = vrow == nullptr || vrow[r] != 0;
                    t = !ok ? -1 : (raw == prefix_tokens ? raw : min(max(raw, static_cast<int64_t>(0)), prefix_tokens - 1));
                }
            }
            live[b] = t >= 0;
            tok[b] = live[b] ? t : 0;
        }
        Raw8<T> kr[NB], vr[NB];
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            const bool is_cur = tok[b] == prefix_tokens;
            if (live[b] && dim_ok) {
                kr[b].load((is_cur ? ck : kbase + tok[b] * k_ts) + dim0);
                vr[b].load((is_cur ? cv : vbase + tok[b] * v_ts) + dim0);
            } else {
                kr[b].zero();
                vr[b].zero();
            }
        }
        float logit[NB];
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            float dot = 0.0f;
#pragma unroll
            for (int i = 0; i < 8; ++i) dot = fmaf(qv[i], kr[b].get(i), dot);
            if constexpr (LPR <= 16) {
                dot = row_sum<LPR>(dot);
            } else {
#pragma unroll
                for (int m = 1; m < LPR; m <<= 1) dot += __shfl_xor(dot, m);
            }
            logit[b] = live[b] ? dot * scale : -INFINITY;
        }
        float bm = -INFINITY;
#pragma unroll
        for (int b = 0; b < NB; ++b) bm = fmaxf(bm, logit[b]);
        const float mnew = fmaxf(st.m, bm);
        if (mnew != -INFINITY) {
            const float alpha = st.m == -INFINITY ? 0.0f : __expf(st.m - mnew);
            st.l *= alpha;
#pragma unroll
            for (int i = 0; i < 8; ++i) st.acc[i] *= alpha;
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                const float p = live[b] ? __expf(logit[b] - mnew) : 0.0f;
                st.l += p;
#pragma unroll
                for (int i = 0; i < 8; ++i) st.acc[i] = fmaf(p, vr[b].get(i), st.acc[i]);
            }
            st.m = mnew;
        }
    }

    store_partial<LPR>(st, lane, wave, dim0, d, partials + (static_cast<int64_t>(h) * nsplit + s) * (d + 2));
}

template <typename T>
__global__ __launch_bounds__(kMergeThreads) void attn_merge_kernel(const float* __restrict__ partials, int nsplit, int d,
                                                         T* __restrict__ out) {
    const int h = blockIdx.x;
    merge_splits<T>(partials + static_cast<int64_t>(h) * nsplit * (d + 2), nsplit, d,
                    out + static_cast<int64_t>(h) * d);
}


// Split states a merge loads in its first burst (and per batch after it).
constexpr int kMergeFirst = 16;

// Row of current_k / current_v for merge block h, and (for a batched step)
// the row's current-token index and its slot k in the indices: sequence b =
// h / q_heads has min(tokens[b], bound) cached tokens (*current holds the
// launch bound on entry).  Unbatched: KV head head_to_kv[h] (clamped), or
// h / (QH / KVH) without a mapping (the dense layers).
__device__ __forceinline__ int64_t merge_kv_row(const SeqTable& seq, const int64_t* __restrict__ head_to_kv, int h,
                                                int kv_heads, int rows, int64_t* idx_slot, int64_t* current) {
    if (seq.tokens != nullptr) {
        const int64_t b = h / seq.q_heads;
        const int64_t raw = seq.tokens[b];
        if (seq.status != nullptr && (raw < 0 || raw > *current) && (threadIdx.x & (kWave - 1)) == 0)
            atomicOr(seq.status, 2);
        *current = seq_tokens_of(seq, b, *current);
        *idx_slot = min(static_cast<int64_t>(seq.budget) - 1, *current);
        return b * seq.kv_heads +
               min(max(head_to_kv[h - b * seq.q_heads], static_cast<int64_t>(0)), static_cast<int64_t>(seq.kv_heads - 1));
    }
    return head_to_kv != nullptr ? min(max(head_to_kv[h], static_cast<int64_t>(0)), static_cast<int64_t>(kv_heads - 1))
                                 : h / (rows / kv_heads);
}

// Merge of one head by one wave (lane l owning dims l and l + 64): the
// head's nsplit states ps[s] = (m, l, acc[128]) plus the current token
// (logit qh . ck * scale, value cv), written to outh in the query dtype.
// No LDS or barrier: the split maxima and denominators are wave reductions
// (lane s holds split s of each 64-split group), and the weights reach the
// accumulation through readlane.  qh, ck, cv, the first group's maxima and
// denominators and the first NF splits' accumulators are loaded in one
// burst, so a layer step's merge pays one memory latency for all of them;
// further splits follow in batches of NF.  Accumulation
// order: the current token, then the splits in ascending order.  COH: the
// states are read with device-coherent loads (written by other workgroups
// of the same kernel).
template <typename T, bool COH, int NF = kMergeFirst>
__device__ __forceinline__ void merge_head(const float* __restrict__ ps, int nsplit, const T* __restrict__ qh,
                                           const T* __restrict__ ck, const T* __restrict__ cv, float scale,
                                           T* __restrict__ outh) {
    constexpr int S = 128 + 2;
    const int lane = threadIdx.x & (kWave - 1);
    // the burst (with nsplit == 0 the accumulator loads read split 0's slot,
    // which every workspace holds, and are not used)
    const float q0 = Elem<T>::load(qh, lane), q1 = Elem<T>::load(qh, lane + 64);
    const float k0 = Elem<T>::load(ck, lane), k1 = Elem<T>::load(ck, lane + 64);
    const float v0 = Elem<T>::load(cv, lane), v1 = Elem<T>::load(cv, lane + 64);
    float m0 = -INFINITY, l0 = 0.0f;  // split `lane`
    if (lane < nsplit) {
        m0 = ld_f32<COH>(ps + (static_cast<int64_t>(lane) * S));
        l0 = ld_f32<COH>(ps + (static_cast<int64_t>(lane) * S + 1));
    }
    const int nf = min(nsplit, NF);
    float a0[NF], a1[NF];
#pragma unroll
    for (int j = 0; j < NF; ++j) {
        const int64_t so = static_cast<int64_t>(max(min(j, nf - 1), 0)) * S + 2;
        a0[j] = ld_f32<COH>(ps + (so + lane));
        a1[j] = ld_f32<COH>(ps + (so + lane + 64));
    }
    // the maxima of every split and the current token's logit
    float mx = m0;
    for (int s0 = kWave; s0 < nsplit; s0 += kWave)
        if (s0 + lane < nsplit) mx = fmaxf(mx, ld_f32<COH>(ps + (static_cast<int64_t>(s0 + lane) * S)));
    const float cur_m = wave_sum(q0 * k0 + q1 * k1) * scale;
    mx = fmaxf(wave_max(mx), cur_m);
    const float wc = __expf(cur_m - mx);
    const float w0 = m0 == -INFINITY ? 0.0f : __expf(m0 - mx);
    float den = l0 * w0, num0 = wc * v0, num1 = wc * v1;
#pragma unroll
    for (int j = 0; j < NF; ++j) {
        if (j < nf) {
            const float ws = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, w0), j));
            num0 = fmaf(ws, a0[j], num0);
            num1 = fmaf(ws, a1[j], num1);
        }
    }
    for (int s0 = 0; s0 < nsplit; s0 += kWave) {
        float w = w0;
        if (s0 > 0) {
            float m = -INFINITY, l = 0.0f;
            if (s0 + lane < nsplit) {
                m = ld_f32<COH>(ps + (static_cast<int64_t>(s0 + lane) * S));
                l = ld_f32<COH>(ps + (static_cast<int64_t>(s0 + lane) * S + 1));
            }
            w = m == -INFINITY ? 0.0f : __expf(m - mx);
            den += l * w;
        }
        const int n = min(kWave, nsplit - s0);
        for (int b = s0 == 0 ? nf : 0; b < n; b += NF) {
            float c0[NF], c1[NF];
#pragma unroll
            for (int j = 0; j < NF; ++j) {
                const int64_t so = static_cast<int64_t>(s0 + min(b + j, n - 1)) * S + 2;
                c0[j] = ld_f32<COH>(ps + (so + lane));
                c1[j] = ld_f32<COH>(ps + (so + lane + 64));
            }
#pragma unroll
            for (int j = 0; j < NF; ++j) {
                if (b + j < n) {
                    const float ws =
                        __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, w), b + j));
                    num0 = fmaf(ws, c0[j], num0);
                    num1 = fmaf(ws, c1[j], num1);
                }
            }
        }
    }
    den = wave_sum(den) + wc;
    Elem<T>::store(outh, lane, num0 / den);
    Elem<T>::store(outh, lane + 64, num1 / den);
}

// ---------------------------------------------------------------- layer step

// Layer-step attention.  Row slot q of a workgroup (16 lanes, one 16-byte
// slice of a 256-byte row each) gathers batches of consecutive selected
// rows; the current token is not among them (the merge adds it).  Rows are
// contiguous (token stride = head_dim = 128).  For 16-bit types the Q.K
// products use v_dot2 (two products accumulated in fp32 per instruction).
constexpr int kSplitRows = 256;  // the reference's split: selected tokens per workgroup

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

// Dot product of 8 packed 16-bit elements with v_dot2 (fp32 accumulation).
template <typename T>
__device__ __forceinline__ float dot8(const uint4& a, const uint4& b) {
    auto d2 = [](uint32_t x, uint32_t y, float c) {
        if constexpr (Elem<T>::kDtype == POPKV_DTYPE_BF16)
            return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, x), __builtin_bit_cast(bf16x2_t, y), c,
                                                   false);
        else
            return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, x), __builtin_bit_cast(f16x2_t, y), c, false);
    };
    return d2(a.w, b.w, d2(a.z, b.z, d2(a.y, b.y, d2(a.x, b.x, 0.0f))));
}

__device__ __forceinline__ void init_state(SoftmaxState& st) {
    st.m = -INFINITY;
    st.l = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) st.acc[i] = 0.0f;
}

// Folds NB gathered rows (this lane's 8-element slices of K and V; the 16
// lanes of a row slot hold one row) into the lane's online-softmax state.
// Rows with live[b] false get weight exactly 0.
template <typename T, int NB>
__device__ __forceinline__ void fold_rows(SoftmaxState& st, const Raw8<T>& qr, const Raw8<T> (&kr)[NB],
                                          const Raw8<T> (&vr)[NB], const bool (&live)[NB], float scale) {
    float logit[NB];
    float bm = -INFINITY;
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        float dot;
        if constexpr (sizeof(T) == 2) {
            dot = dot8<T>(qr.u, kr[b].u);
        } else {
            dot = 0.0f;
#pragma unroll
            for (int i = 0; i < 8; ++i) dot = fmaf(qr.get(i), kr[b].get(i), dot);
        }
        dot = row_sum<16>(dot);
        logit[b] = live[b] ? dot * scale : -INFINITY;
        bm = fmaxf(bm, logit[b]);
    }
    // The compiler sinks the V loads into this branch, so a batch's V rows
    // are requested only once its K rows have arrived.  A branch-free form
    // with every K and V request in flight at once measured slower on the
    // layer step's gathers (C1 select + attention kernel 18.6 vs 17.1 us).
    const float mnew = fmaxf(st.m, bm);
    if (mnew != -INFINITY) {
        const float alpha = __expf(st.m - mnew);  // st.m = -inf gives 0
        st.l *= alpha;
#pragma unroll
        for (int i = 0; i < 8; ++i) st.acc[i] *= alpha;
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            const float p = __expf(logit[b] - mnew);  // -inf logit gives 0
            st.l += p;
#pragma unroll
            for (int i = 0; i < 8; ++i) st.acc[i] = fmaf(p, vr[b].get(i), st.acc[i]);
        }
        st.m = mnew;
    }
}

// Block -> (chunk, head) of the layer step's select + attention grid
// (nchunks * QH blocks).  With kv_groups (KV heads a multiple of 8, query
// head h in GQA group h / qpk), block i serves group
// 8 * (i / (8 * nchunks * qpk)) + i mod 8, chunk-major within the group:
// the dispatcher hands blocks to the eight XCDs round-robin, so the query
// heads of a group -- which gather overlapping K/V rows -- share one L2
// (measured at C1: 1.0 us faster than chunk-major over all heads).
// Otherwise block i is chunk i mod nchunks of head i / nchunks.  Either way
// a bijection; the mapping only affects locality, never results.
__device__ __forceinline__ void chunk_head_of_block(int id, int nchunks, int qpk, bool kv_groups, int* c, int* h) {
    if (kv_groups) {
        const int per = nchunks * qpk;
        const int j = id >> 3;
        const int g = div_nonneg(j, per), within = j - g * per;
        *c = div_nonneg(within, qpk);
        *h = ((g << 3) + (id & 7)) * qpk + (within - *c * qpk);
    } else {
        *h = div_nonneg(id, nchunks);
        *c = id - *h * nchunks;
    }
}

// The current token's append in a batched decode step's select + attention
// launch: workgroups 0 .. blocks - 1 run pack128_append for (sequence, KV
// head) blockIdx.x < batch * kv_heads (blocks is rounded up to a multiple of
// 8 so that the select + attention workgroups keep their XCD placement).
template <typename T>
struct StepAppendArgs {
    AppendArgs<T> ap;
    int32_t* k_sign = nullptr;
    int32_t* k_mag = nullptr;
    uint16_t* k_low = nullptr;
    uint16_t* k_delta = nullptr;
    int64_t cap = 0;
    int tg = 1, g = 64, blocks = 0, items = 0;
};

// Layer step: the select's second half fused with the sparse attention.
// Block (c, h) owns chunk c of head h's key row (kChunkThreads * KPT tokens,
// KPT per thread).  The selection is every key > T plus the lowest-index
// ties at T (PyTorch's gather-top-k rule), T = b1:t2 the k-th largest key;
// with k >= tokens every token.
//   1. The keys above bin b1 are selected whatever t2 is, and b1 arrives
//      with the first loads (chunk_hist_kernel's record).  Each wave lists
//      its own first SLOTS * NB of them (a wave scan) and issues its slots'
//      first gather pass over them before T is resolved.
//   2. While those rows are in flight: the chunk histograms of bin b1
//      (thread u sums bin u over every chunk and over the chunks before c)
//      give t2, need_eq = ties the row takes and eq_before = ties in
//      earlier chunks; the block lists the tokens above b1 the waves left,
//      the keys of bin b1 above T and the chunk's share of the ties (one
//      block scan).  When idx_out is non-null every selected token is also
//      written there as int64 at its row rank (selected tokens before it in
//      the row).
//   3. Attention over the block's list: 16 row slots, each taking NB
//      consecutive entries per pass, all NB K/V gathers of a pass in
//      flight before any is used.
//   4. (m, l, acc[128]) to partials[h][c] (m = -inf for an empty chunk).
// Block 0 of each head re-zeroes the scorer's histogram ghist[h] (its last
// reader, chunk_hist_kernel, has finished).  The grid is one-dimensional
// (chunk_head_of_block).
// (The batched form also carries the decode step's append code; asked for
// three waves per SIMD it keeps the residency of the plain step: 142 VGPRs
// at bf16.  Measured at C4: 160.4 us per step with the append in this
// launch, 167.9 with a separate append launch.)
//
// HANDOFF (the layer step's single-launch form, WJ > 0, not SEQ): the
// scorer's workgroups run in the same launch.  The block first polls its
// head's histogram row with device-coherent loads until the row sums to
// ntok (every tile counted: the scorer adds its counts only after its keys,
// window histograms and records were acknowledged at the coherence point),
// then reads those with device-coherent loads.  The poll is bounded
// (kHandoffPolls): the scorer's workgroups come first in the grid and the
// dispatcher places workgroups in grid order, so they are resident before
// any select block and never wait; the bound only guarantees that every
// wave ends.
template <typename T, int KPT, int NB, bool SEQ, int WJ, bool HANDOFF>
__device__ __forceinline__ void attn_select_chunk_body(
    const T* __restrict__ q, const T* __restrict__ kc, const T* __restrict__ vc, int64_t k_hs, int64_t v_hs,
    const uint16_t* __restrict__ keys, int64_t key_stride, int ntok, int k, const uint32_t* __restrict__ rec,
    const uint16_t* __restrict__ h2, const uint32_t* __restrict__ gt1, int nchunks, int qpk, bool kv_groups,
    uint32_t* __restrict__ ghist, const int64_t* __restrict__ head_to_kv, int kv_heads, float scale,
    float* __restrict__ partials, int64_t* __restrict__ idx_out, int64_t idx_stride, SeqTable seq,
    const T* __restrict__ cur_k, const T* __restrict__ cur_v, T* __restrict__ out, StepAppendArgs<T> apx,
    WindowIn win, uint32_t block_id) {
    static_assert(kAttnThreads == kChunkThreads, "one key slice per thread");
    static_assert(!HANDOFF || (WJ > 0 && !SEQ), "the hand-off: the unbatched window path");
    static_assert(WJ == 0 || kAttnWaves == 4, "the window path's tile layout: 4 waves x 2 halves");
    args_in_sgprs(q, kc, vc, k_hs, v_hs, keys, key_stride, ntok, k, rec, h2, gt1, nchunks, qpk,
                  static_cast<int>(kv_groups), head_to_kv, kv_heads);
    int block = static_cast<int>(block_id);
    if constexpr (SEQ) {
        // The decode step's append: nothing below reads what it writes (the
        // static caches' rows at the counts -- the select reads the rows
        // below them, the current K/V come from cur_k / cur_v -- and the
        // active groups' packed rows, which only the scorer read).
        if (block < apx.blocks) {
            if (block >= apx.items) return;
            if (apx.g == 16)
                pack128_append<T, 16, true>(block, apx.ap, apx.tg, apx.k_sign, apx.k_mag, apx.k_low, apx.k_delta,
                                            apx.cap);
            else if (apx.g == 32)
                pack128_append<T, 32, true>(block, apx.ap, apx.tg, apx.k_sign, apx.k_mag, apx.k_low, apx.k_delta,
                                            apx.cap);
            else
                pack128_append<T, 64, true>(block, apx.ap, apx.tg, apx.k_sign, apx.k_mag, apx.k_low, apx.k_delta,
                                            apx.cap);
            return;
        }
        block -= apx.blocks;
    }
    constexpr int D = 128, LPR = 16, SLOTS = kWave / LPR, NSLOT = SLOTS * kAttnWaves;
    constexpr int CH = kChunkThreads * KPT;
    constexpr int PASS = NSLOT * NB;  // entries per pass
    static_assert(NB % 2 == 0, "a slot's entries of one pass are whole 32-bit LDS words");
    int c, h;
    chunk_head_of_block(block, nchunks, qpk, kv_groups, &c, &h);
    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = tid / kWave;
    const int slot = wave * SLOTS + lane / LPR;
    const int dim0 = (lane % LPR) * 8;
    // SEQ (a batched step): row h is query head hl of sequence b, whose own
    // token count and k arrive with the first loads; every load below is
    // addressed within the launch's bounds (ntok tokens, nchunks chunks) and
    // masked to the row's own shape afterwards.
    int64_t b = 0;
    int hl = h;
    if constexpr (SEQ) {
        b = div_nonneg(h, seq.q_heads);
        hl = h - static_cast<int>(b) * seq.q_heads;
    }

    // 0. loads, all issued before any is used: this thread's keys, the query
    //    slice, the head's KV mapping, the threshold record and the chunk
    //    histograms.  The mapping and the record are read with vector loads
    //    at a lane-opaque zero offset: as scalar loads they would be waited
    //    for together with the kernel arguments, before the chunk histograms
    //    are even issued.
    int z = 0;
    asm volatile("" : "+v"(z));
    const int begin = c * CH + tid * KPT;
    ChunkKeys<KPT> kk;
    if constexpr (!HANDOFF)
        load_chunk_keys_raw<KPT>(keys + static_cast<int64_t>(h) * key_stride, begin, max(0, min(KPT, ntok - begin)), kk);
    Raw8<T> qr;
    qr.load(q + static_cast<int64_t>(h) * D + dim0);
    const int64_t map = head_to_kv[hl + z];
    int64_t seq_ntok = ntok, raw_ntok = ntok;
    if constexpr (SEQ) {
        raw_ntok = seq.tokens[b];
        seq_ntok = raw_ntok < 0 ? 0 : (raw_ntok > ntok ? ntok : raw_ntok);
    }
    uint32_t rank0 = 0;
    uint32_t g2 = 0, p2 = 0;  // bin tid of the chunk histograms over every chunk / over chunks before c
    // The threshold record, bin tid of the first HB chunk histograms and
    // (lane l) the keys above bin b1 in chunk l -- every chunk: a step has at
    // most 64 -- are loaded whatever the mode (the workspace always holds
    // them; unused values are ignored).  With every path issuing the same
    // loads in the same order, the waits for the keys, the record and the
    // mapping before the first gather pass count exactly and leave these in
    // flight, and the histograms are summed only once that pass is out (step
    // 2).  Measured at C1: a wait for every load before the pass -- what
    // loads on mode-dependent paths compile to -- sent it out about 3 us
    // later.
    // The window path (WJ > 0: the scorer wrote tile windows, no chunk
    // histograms) loads instead the row's high-byte histogram (every wave,
    // lane l holding ranks 4l .. 4l + 3) and one tile record per lane: lane
    // (hf, wp) of wave w holds tile w + 4 hf + 8 wp, the tiles its half
    // sums (tile w + 4 hf + 8 j for j < WJ).
    constexpr int HB = 16;
    constexpr int NHV = WJ > 0 ? 1 : HB;
    uint32_t b1 = 0u, above1 = 0u, gx = 0u;
    const uint16_t* hr = h2 + static_cast<int64_t>(h) * nchunks * 256 + tid;
    uint32_t hv[NHV];
    const int hf = lane >> 5, wp = lane & 31;
    uint32_t gcnt[4] = {0u, 0u, 0u, 0u};
    uint4 wr = make_uint4(0u, 0u, 0u, 0u);
    if constexpr (WJ == 0) {
        b1 = rec[4 * h + z];
        above1 = rec[4 * h + 1 + z];
#pragma unroll
        for (int j = 0; j < HB; ++j) hv[j] = hr[static_cast<int64_t>(min(j, nchunks - 1)) * 256];
        gx = gt1[static_cast<int64_t>(h) * nchunks + min(lane, nchunks - 1)];
    } else if constexpr (!HANDOFF) {
        load_rank4(win.hist + static_cast<int64_t>(h) * 256, gcnt);
        wr = win.rec[static_cast<int64_t>(h) * win.tiles + min(wave + 4 * hf + 8 * wp, win.tiles - 1)];
    } else {
        // the scorer's hand-off: the row's histogram counts every token once
        // all of its tiles are out (bins 0 .. 2, which no key reaches, are
        // left out: bin 0 holds the merge ticket); the counts only grow, so
        // a read that sums to ntok read every bin's final count.  Then the
        // chunk's keys and the tile records, written before those counts.
        if (k > 0 && k < ntok) {
            const uint4* hrow = reinterpret_cast<const uint4*>(win.hist + static_cast<int64_t>(h) * 256) + (63 - lane);
            for (int poll = 0;; ++poll) {
                const uint4 u = ld_coh_u4(hrow);
                gcnt[0] = u.w;
                gcnt[1] = u.z;
                gcnt[2] = u.y;
                gcnt[3] = u.x;
                const uint32_t part = lane == kWave - 1 ? u.w : u.x + u.y + u.z + u.w;
                const uint32_t sum =
                    static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(wave_incl_scan(part, lane)), kWave - 1));
                if (sum >= static_cast<uint32_t>(ntok) || poll >= kHandoffPolls) break;
                __builtin_amdgcn_s_sleep(1);
            }
        }
        load_chunk_keys_raw<KPT, true>(keys + static_cast<int64_t>(h) * key_stride, begin,
                                       max(0, min(KPT, ntok - begin)), kk);
        wr = ld_coh_u4(&win.rec[static_cast<int64_t>(h) * win.tiles + min(wave + 4 * hf + 8 * wp, win.tiles - 1)]);
    }
    int nch = nchunks;  // this row's chunks
    if constexpr (SEQ) {
        // a count outside [0, launch bound] runs clamped and is flagged (by
        // one block per sequence)
        if (seq.status != nullptr && c == 0 && hl == 0 && tid == 0 && (raw_ntok < 0 || raw_ntok > ntok))
            atomicOr(seq.status, 2);
        ntok = static_cast<int>(seq_ntok);
        k = min(seq.budget - 1, ntok);
        nch = (ntok + CH - 1) / CH;
    }
    const int n = max(0, min(KPT, ntok - begin));
    mask_chunk_keys<KPT>(n, kk);
    const int mode = k <= 0 ? 0 : (k >= ntok ? 1 : 2);  // none / every token / threshold
    __shared__ uint32_t s_g2[256], s_p2[256];
    // window path: per-half partial sums of bin b1's low-byte histogram
    // over all tiles / the tiles before this chunk (16-bit pairs: at most 8
    // tiles x the tile's tokens per bin, below 2^16), and the waves' counts
    // of keys above bin b1 in those earlier tiles.  Each half owns its slot:
    // only its own wave writes it, so no barrier orders the writes.
    __shared__ uint32_t s_gpart[WJ > 0 ? 2 * kAttnWaves : 1][128], s_ppart[WJ > 0 ? 2 * kAttnWaves : 1][128];
    __shared__ uint32_t s_gtb[kAttnWaves];
    // window path: b1 from the row's histogram, then the window rows at b1
    // of this half's tiles, issued before the gather pass.  A tile whose
    // window misses b1 (rare: the window spans the estimate -2 .. +1) is
    // histogrammed from its keys here, also before the gather pass, whose
    // loads would otherwise queue the scan's behind them.
    int ntile_row = 0, c0t = 0, rrow = 0;
    uint32_t gtb = 0u;  // keys above bin b1 in tiles before this chunk (this lane's share)
    uint2 wv[WJ > 0 ? WJ : 1];  // bins 8 wp .. 8 wp + 7 of a window row (byte counts)
    if constexpr (WJ > 0) {
        const int ts = win.tile_tokens;
        ntile_row = (ntok + ts - 1) / ts;
        c0t = c * (CH / ts);
        if (mode == 2) wave_find_bin(gcnt, static_cast<uint32_t>(k), &b1, &above1);
        rrow = static_cast<int>(b1) - static_cast<int>(wr.x);
        if (static_cast<unsigned>(rrow) < static_cast<unsigned>(kWinBins)) {
            // a bin of more than 255 of the tile's keys may have overflowed
            // its byte counts: taken from the keys, as a miss
            const uint32_t tot = (rrow < 2 ? wr.z : wr.w) >> ((rrow & 1) * 16) & 0xffffu;
            if (tot > 255u) rrow = -1;
        }
        const uint2* wb = reinterpret_cast<const uint2*>(win.bins) + static_cast<int64_t>(h) * win.tiles * (kWinBins * 32) + wp;
        bool miss = false;
#pragma unroll
        for (int j = 0; j < WJ; ++j) {
            const int i = wave + 4 * hf + 8 * j;
            const int rj = __shfl(rrow, hf * 32 + j);
            const bool in_row = i < ntile_row;
            const bool hit = in_row && static_cast<unsigned>(rj) < static_cast<unsigned>(kWinBins);
            miss = miss || (in_row && !hit);
            wv[j] = ld_u2<HANDOFF>(wb + (hit ? (i * kWinBins + rj) * 32 : 0));
        }
        const int hs = wave * 2 + hf;
        const uint4 zero4 = make_uint4(0u, 0u, 0u, 0u);
        reinterpret_cast<uint4*>(&s_gpart[hs][0])[wp] = zero4;
        reinterpret_cast<uint4*>(&s_ppart[hs][0])[wp] = zero4;
        if (mode == 2 && __ballot(miss) != 0) {
            const int per = ts / 32;
            for (int j = 0; j < WJ; ++j) {
                const int i = wave + 4 * hf + 8 * j;
                const int rj = __shfl(rrow, hf * 32 + j);
                if (i >= ntile_row || static_cast<unsigned>(rj) < static_cast<unsigned>(kWinBins)) continue;
                // the lane's per = ts / 32 keys (at most 32), every load
                // issued before any is used; keys are written up to ntok and
                // the row holds them to ntok rounded up to 128, so a load
                // past ntok re-reads the row's start and its keys are masked
                const int t_first = i * ts + wp * per;
                const uint16_t* krow = keys + static_cast<int64_t>(h) * key_stride;
                constexpr int QMAX = 4;  // 8-key loads per lane: ts <= 1024
                uint4 u[QMAX];
#pragma unroll
                for (int q = 0; q < QMAX; ++q)
                    u[q] = ld_u4<HANDOFF>(reinterpret_cast<const uint4*>(
                        krow + (8 * q < per && t_first + 8 * q < ntok ? t_first + 8 * q : 0)));
#pragma unroll
                for (int q = 0; q < QMAX; ++q) {
                    const uint32_t wd[4] = {u[q].x, u[q].y, u[q].z, u[q].w};
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        const int t = t_first + 8 * q + e;
                        if (8 * q >= per || t >= ntok) continue;
                        const uint32_t key = (wd[e >> 1] >> ((e & 1) * 16)) & 0xffffu;
                        const uint32_t hb = key >> 8, inc = 1u << ((key & 1u) * 16);
                        if (hb == b1) {
                            atomicAdd(&s_gpart[hs][(key & 0xffu) >> 1], inc);
                            if (i < c0t) atomicAdd(&s_ppart[hs][(key & 0xffu) >> 1], inc);
                        } else if (hb > b1 && i < c0t) {
                            ++gtb;
                        }
                    }
                }
            }
        }
    }
    __shared__ uint32_t s_scan1[kAttnWaves], s_scan2[kAttnWaves];
    __shared__ __align__(16) uint16_t s_list[CH];
    const bool fused = out != nullptr;  // the merge runs in the head's last block (see the end)
    if constexpr (SEQ) {
        if (c >= nch) {  // past this sequence's tokens: an empty state (the merge weighs it 0)
            if (c == 0 && (tid > 0 || !fused)) ghist[static_cast<int64_t>(h) * 256 + tid] = 0u;
            float* dst = partials + (static_cast<int64_t>(h) * nchunks + c) * (D + 2);
            if (tid < D + 2) dst[tid] = tid == 0 ? -INFINITY : 0.0f;
            if (fused && c == 0 && wave == 0) {
                // an empty sequence: no chunk takes a ticket, and the merge
                // is the current token alone
                const int64_t kvh = min(max(map, static_cast<int64_t>(0)), static_cast<int64_t>(kv_heads - 1));
                const int64_t crow = (b * seq.kv_heads + kvh) * D;
                if (idx_out != nullptr && lane == 0) idx_out[static_cast<int64_t>(h) * idx_stride + k] = ntok;
                merge_head<T, false>(dst, 0, q + static_cast<int64_t>(h) * D, cur_k + crow, cur_v + crow, scale,
                                     out + static_cast<int64_t>(h) * D);
            }
            return;
        }
    }

    // 1. the tokens selected whatever T is: keys above bin b1 (mode 2) or
    //    every token (mode 1).  Each wave lists its own first WCAP of them in
    //    ascending order (a wave scan, no block barrier) and issues its
    //    slots' first gather pass over them at once; the others join the
    //    block's list below.
    constexpr int WCAP = SLOTS * NB;  // entries of one wave's slots in one pass
    __shared__ __align__(16) uint16_t s_wlist[kAttnWaves][WCAP];
    uint32_t m_def = 0u;
    if (mode == 2) {
        uint32_t unused;
        key_masks<KPT>(kk, (b1 << 8) | 0xffu, &m_def, &unused);
    } else if (mode == 1) {
        m_def = n >= 32 ? 0xffffffffu : (1u << n) - 1u;
    }
    const uint32_t dcnt = static_cast<uint32_t>(__popc(m_def));
    const uint32_t dincl = wave_incl_scan(dcnt, lane);
    const int wfirst = min(__builtin_amdgcn_readlane(static_cast<int>(dincl), kWave - 1), WCAP);
    uint32_t m_left = 0u;  // this thread's tokens above bin b1 that the wave's first pass does not take
    {
        uint32_t pos = dincl - dcnt;
        for (uint32_t m = m_def; m != 0u; m &= m - 1u) {
            const int e = __builtin_ctz(m);
            if (pos < static_cast<uint32_t>(WCAP)) s_wlist[wave][pos] = static_cast<uint16_t>(tid * KPT + e);
            else m_left |= 1u << e;
            ++pos;
        }
    }
    // the wave reads its own list next: one wave's LDS operations complete in order
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    // 2. the first gather pass, issued now
    const int64_t kvh = min(max(map, static_cast<int64_t>(0)), static_cast<int64_t>(kv_heads - 1));
    const char* kb = reinterpret_cast<const char*>(kc + b * seq.k_bstride + kvh * k_hs) + dim0 * sizeof(T);
    const char* vb = reinterpret_cast<const char*>(vc + b * seq.v_bstride + kvh * v_hs) + dim0 * sizeof(T);
    const uint32_t t0 = static_cast<uint32_t>(c * CH);
    const uint32_t tmax = static_cast<uint32_t>(ntok - 1);  // a selected token is < ntok; clamped all the same
    Raw8<T> kr[NB], vr[NB];
    bool live[NB];
    // rows lst[e0 .. e0 + NB) of a list of `cap` entries, those below `limit`
    // live; dead rows re-read the chunk's first token and get weight 0.  e0
    // is a multiple of NB, so the widest LDS read that divides 2*NB bytes is
    // aligned.
    auto issue = [&](const uint16_t* lst, int e0, int limit, int cap) {
        uint32_t ew[NB / 2];
        if constexpr (NB % 8 == 0) {
#pragma unroll
            for (int j = 0; j < NB / 8; ++j) {
                const uint4 ev = *reinterpret_cast<const uint4*>(&lst[min(e0 + 8 * j, cap - 8)]);
                ew[4 * j] = ev.x;
                ew[4 * j + 1] = ev.y;
                ew[4 * j + 2] = ev.z;
                ew[4 * j + 3] = ev.w;
            }
        } else if constexpr (NB % 4 == 0) {
#pragma unroll
            for (int j = 0; j < NB / 4; ++j) {
                const uint2 ev = *reinterpret_cast<const uint2*>(&lst[min(e0 + 4 * j, cap - 4)]);
                ew[2 * j] = ev.x;
                ew[2 * j + 1] = ev.y;
            }
        } else {
#pragma unroll
            for (int j = 0; j < NB / 2; ++j) ew[j] = *reinterpret_cast<const uint32_t*>(&lst[min(e0 + 2 * j, cap - 2)]);
        }
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            live[b] = e0 + b < limit;
            const uint32_t t = min(t0 + (live[b] ? ((ew[b / 2] >> ((b & 1) * 16)) & 0xffffu) : 0u), tmax);
            const uint32_t off = t * (D * sizeof(T));
            kr[b].load(reinterpret_cast<const T*>(kb + off));
            vr[b].load(reinterpret_cast<const T*>(vb + off));
        }
    };
    // (issued in every block, all rows dead when the wave listed none, so
    // that the sums below wait for the histograms alone)
    issue(s_wlist[wave], (slot % SLOTS) * NB, wfirst, WCAP);
    // (and the sums stay behind the pass: the scheduler would otherwise
    // hoist some of them, with their waits, above its loads)
    __builtin_amdgcn_sched_barrier(0);
    uint32_t gt1_before = 0u;  // keys above bin b1 in earlier chunks
    if constexpr (WJ == 0) {
#pragma unroll
        for (int j = 0; j < HB; ++j) {
            const uint32_t x = j < nch ? hv[j] : 0u;
            g2 += x;
            p2 += j < c ? x : 0u;
        }
        for (int c0 = HB; c0 < nch; c0 += HB) {  // steps of more than HB chunks (large budgets)
#pragma unroll
            for (int j = 0; j < HB; ++j) hv[j] = hr[static_cast<int64_t>(min(c0 + j, nchunks - 1)) * 256];
#pragma unroll
            for (int j = 0; j < HB; ++j) {
                const uint32_t x = c0 + j < nch ? hv[j] : 0u;
                g2 += x;
                p2 += c0 + j < c ? x : 0u;
            }
        }
        gt1_before = static_cast<uint32_t>(
            __builtin_amdgcn_readlane(static_cast<int>(wave_incl_scan(lane < c ? gx : 0u, lane)), kWave - 1));
        if (mode == 2) {
            s_g2[tid] = g2;
            s_p2[tid] = p2;
        }
        // (bin 0 -- which no real key reaches -- holds the fused merge's
        // ticket; the window path re-zeroes the histogram in the merge, its
        // last reader being this kernel)
        if (c == 0 && (tid > 0 || !fused)) ghist[static_cast<int64_t>(h) * 256 + tid] = 0u;
    } else {
        // the half's window rows added to its slot (which holds the missed
        // tiles' counts), and the record lane's keys above bin b1 when its
        // tile lies before this chunk
        uint4 gs = make_uint4(0u, 0u, 0u, 0u), ps = gs;
        if (mode == 2) {
#pragma unroll
            for (int j = 0; j < WJ; ++j) {
                const int i = wave + 4 * hf + 8 * j;
                const int rj = __shfl(rrow, hf * 32 + j);
                if (i < ntile_row && static_cast<unsigned>(rj) < static_cast<unsigned>(kWinBins)) {
                    // byte counts of bins 8 wp .. 8 wp + 7 widened to the
                    // slot's 16-bit pairs (bins 2m, 2m + 1 in word m)
                    const uint32_t a = wv[j].x, b = wv[j].y;
                    const uint4 v = make_uint4((a & 0xffu) | ((a << 8) & 0xff0000u), ((a >> 16) & 0xffu) | ((a >> 8) & 0xff0000u),
                                               (b & 0xffu) | ((b << 8) & 0xff0000u), ((b >> 16) & 0xffu) | ((b >> 8) & 0xff0000u));
                    gs.x += v.x; gs.y += v.y; gs.z += v.z; gs.w += v.w;
                    if (i < c0t) {
                        ps.x += v.x; ps.y += v.y; ps.z += v.z; ps.w += v.w;
                    }
                }
            }
            const int ir = wave + 4 * hf + 8 * wp;
            if (ir < ntile_row && ir < c0t && static_cast<unsigned>(rrow) < static_cast<unsigned>(kWinBins)) {
                const uint32_t tot[kWinBins] = {wr.z & 0xffffu, wr.z >> 16, wr.w & 0xffffu, wr.w >> 16};
                uint32_t above_b1 = wr.y;  // keys above the window
#pragma unroll
                for (int w = 0; w < kWinBins; ++w) above_b1 += w > rrow ? tot[w] : 0u;
                gtb += above_b1;
            }
        }
        // (this lane's four words of the slot: written before by this wave
        // alone, whose LDS operations complete in order)
        const int hs = wave * 2 + hf;
        uint4* gw = reinterpret_cast<uint4*>(&s_gpart[hs][0]) + wp;
        uint4* pw = reinterpret_cast<uint4*>(&s_ppart[hs][0]) + wp;
        const uint4 g0 = *gw, p0 = *pw;
        *gw = make_uint4(g0.x + gs.x, g0.y + gs.y, g0.z + gs.z, g0.w + gs.w);
        *pw = make_uint4(p0.x + ps.x, p0.y + ps.y, p0.z + ps.z, p0.w + ps.w);
        gtb = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(wave_incl_scan(gtb, lane)), kWave - 1));
        if (lane == 0) s_gtb[wave] = gtb;
    }
    __syncthreads();
    if constexpr (WJ > 0) {
#pragma unroll
        for (int w = 0; w < kAttnWaves; ++w) gt1_before += s_gtb[w];
    }

    // 3. T from the chunk histograms; the block's list: the tokens above bin
    //    b1 the waves' first passes left, bin b1's keys above T and the
    //    chunk's share of the ties
    uint32_t thr = 0, need_eq = 0, eq_before = 0;
    if (mode == 2) {
        uint32_t cnt[4];
        if constexpr (WJ == 0) {
#pragma unroll
            for (int i = 0; i < 4; ++i) cnt[i] = s_g2[255 - (4 * lane + i)];
        } else {
            // bins 255 - 4l .. 252 - 4l: the high and low halves of words
            // 127 - 2l and 126 - 2l, summed over the eight half slots
            cnt[0] = cnt[1] = cnt[2] = cnt[3] = 0u;
#pragma unroll
            for (int hs = 0; hs < 2 * kAttnWaves; ++hs) {
                const uint2 v = *reinterpret_cast<const uint2*>(&s_gpart[hs][126 - 2 * lane]);
                cnt[0] += v.y >> 16;
                cnt[1] += v.y & 0xffffu;
                cnt[2] += v.x >> 16;
                cnt[3] += v.x & 0xffffu;
            }
        }
        const uint32_t need1 = static_cast<uint32_t>(k) - above1;
        uint32_t t2, above2;
        wave_find_bin(cnt, need1, &t2, &above2);
        thr = (b1 << 8) | t2;  // >= 0x03ff
        need_eq = need1 - above2;
        // bin u of the chunks (tiles) before this one
        auto p2_of = [&](int u) -> uint32_t {
            if constexpr (WJ == 0) {
                return s_p2[u];
            } else {
                uint32_t x = 0u;
#pragma unroll
                for (int hs = 0; hs < 2 * kAttnWaves; ++hs) x += (s_ppart[hs][u >> 1] >> ((u & 1) * 16)) & 0xffffu;
                return x;
            }
        };
        eq_before = p2_of(static_cast<int>(t2));
        if (idx_out != nullptr) {
            // keys of bin b1 with low byte > t2 in earlier chunks
            uint32_t x = 0;
#pragma unroll
            for (int i = 0; i < 4; ++i) x += 4 * lane + i > static_cast<int>(t2) ? p2_of(4 * lane + i) : 0u;
            const uint32_t gt2_before =
                static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(wave_incl_scan(x, lane)), kWave - 1));
            rank0 = gt1_before + gt2_before + min(eq_before, need_eq);
        }
    } else if (mode == 1) {
        rank0 = static_cast<uint32_t>(c * CH);
    }
    uint32_t m_gt = m_def, m_eq = 0u;
    if (mode == 2) key_masks<KPT>(kk, thr, &m_gt, &m_eq);
    const uint32_t m_blk = m_left | (m_gt & ~m_def);  // listed by the block (the ties follow)
    const uint32_t n_eq = static_cast<uint32_t>(__popc(m_eq));
    uint32_t total2;
    const uint32_t packed =
        block_excl_scan_once(static_cast<uint32_t>(__popc(m_blk)) | (n_eq << 16), s_scan2, kAttnWaves, &total2);
    // ties taken by earlier chunks / before this thread / by this thread
    // (each min is formed before the subtraction that uses it, which then
    // never wraps)
    const uint32_t prior = min(eq_before, need_eq);
    const uint32_t t_before = min(eq_before + (packed >> 16), need_eq);
    const uint32_t t_end = min(eq_before + (total2 >> 16), need_eq);
    const uint32_t take = min(n_eq, need_eq - t_before);
    const int n_list = static_cast<int>((total2 & 0xffffu) + (t_end - prior));
    uint32_t ties = m_eq;
    if (take < n_eq) {  // keep only the first `take` ties
        uint32_t rest = ties;
        for (uint32_t j = 0; j < take; ++j) rest &= rest - 1u;
        ties &= ~rest;
    }
    {
        uint32_t pos = (packed & 0xffffu) + (t_before - prior);
        for (uint32_t m = m_blk | ties; m != 0u; m &= m - 1u) {
            if (pos < static_cast<uint32_t>(CH)) s_list[pos] = static_cast<uint16_t>(tid * KPT + __builtin_ctz(m));
            ++pos;
        }
    }
    if (idx_out != nullptr) {
        // ascending row ranks: the selected tokens of earlier threads come first
        uint32_t gt_total;
        const uint32_t gt_pre =
            block_excl_scan_once(static_cast<uint32_t>(__popc(m_gt)), s_scan1, kAttnWaves, &gt_total);
        int64_t* irow = idx_out + static_cast<int64_t>(h) * idx_stride;
        uint32_t pos = gt_pre + (t_before - prior);
        for (uint32_t m = m_gt | ties; m != 0u; m &= m - 1u) {
            if (rank0 + pos < static_cast<uint32_t>(k)) irow[rank0 + pos] = c * CH + tid * KPT + __builtin_ctz(m);
            ++pos;
        }
    }
    __syncthreads();

    // 4. attention: the waves' first passes, then the block's list
    SoftmaxState st;
    init_state(st);
    if (wfirst > 0) fold_rows<T, NB>(st, qr, kr, vr, live, scale);
    for (int base = 0; base < n_list; base += PASS) {
        issue(s_list, base + slot * NB, n_list, CH);
        fold_rows<T, NB>(st, qr, kr, vr, live, scale);
    }
    float* const pdst = partials + (static_cast<int64_t>(h) * nchunks + c) * (D + 2);
    store_partial<LPR>(st, lane, wave, dim0, D, pdst, fused);
    if (!fused) return;
    // 5. fused merge: the state went out with device-coherent stores; once
    //    every thread's stores are acknowledged the block takes a ticket
    //    (ghist[h][0], zero between calls), and the head's last block --
    //    which sees every other chunk's stores -- merges the chunks and the
    //    current token, resets the ticket and writes the output (one wave).
    //    The ordering rests on the gfx942/gfx950 rule stated at st_f32:
    //    this vmcnt(0) covers the sc1 stores, so they have reached the
    //    coherence point before the barrier and the ticket.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    __shared__ uint32_t s_last;
    const uint32_t parts = static_cast<uint32_t>(SEQ ? max(nch, 1) : nchunks);
    if (tid == 0) {
        const uint32_t old =
            __hip_atomic_fetch_add(&ghist[static_cast<int64_t>(h) * 256], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s_last = old + 1u == parts ? 1u : 0u;
    }
    __syncthreads();
    if (s_last == 0u || wave != 0) return;
    if constexpr (WJ == 0) {
        if (lane == 0)
            __hip_atomic_store(&ghist[static_cast<int64_t>(h) * 256], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    } else {
        // every block of the head has read the histogram (before its
        // ticket): keep a copy for re-runs of this kernel alone (win.keep),
        // then zero it, ticket included, for the next step's scorer
        uint4* gh = reinterpret_cast<uint4*>(ghist + static_cast<int64_t>(h) * 256);
        if (win.keep != nullptr)
            reinterpret_cast<uint4*>(win.keep + static_cast<int64_t>(h) * 256)[63 - lane] =
                make_uint4(gcnt[3], gcnt[2], gcnt[1], gcnt[0]);
        __hip_atomic_store(&gh[lane].x, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        gh[lane].y = 0u;
        gh[lane].z = 0u;
        gh[lane].w = 0u;
    }
    if (lane == 0 && idx_out != nullptr) idx_out[static_cast<int64_t>(h) * idx_stride + k] = ntok;
    const int64_t crow = ((SEQ ? b * seq.kv_heads : 0) + kvh) * D;
    merge_head<T, true>(partials + static_cast<int64_t>(h) * nchunks * (D + 2), static_cast<int>(parts),
                        q + static_cast<int64_t>(h) * D, cur_k + crow, cur_v + crow, scale,
                        out + static_cast<int64_t>(h) * D);
}

template <typename T, int KPT, int NB, bool SEQ, int WJ>
__global__ __launch_bounds__(kAttnThreads, SEQ ? 3 : 1) void attn_select_chunk_kernel(
    const T* __restrict__ q, const T* __restrict__ kc, const T* __restrict__ vc, int64_t k_hs, int64_t v_hs,
    const uint16_t* __restrict__ keys, int64_t key_stride, int ntok, int k, const uint32_t* __restrict__ rec,
    const uint16_t* __restrict__ h2, const uint32_t* __restrict__ gt1, int nchunks, int qpk, bool kv_groups,
    uint32_t* __restrict__ ghist, const int64_t* __restrict__ head_to_kv, int kv_heads, float scale,
    float* __restrict__ partials, int64_t* __restrict__ idx_out, int64_t idx_stride, SeqTable seq,
    const T* __restrict__ cur_k, const T* __restrict__ cur_v, T* __restrict__ out, StepAppendArgs<T> apx,
    WindowIn win) {
    attn_select_chunk_body<T, KPT, NB, SEQ, WJ, false>(q, kc, vc, k_hs, v_hs, keys, key_stride, ntok, k, rec, h2, gt1,
                                                       nchunks, qpk, kv_groups, ghist, head_to_kv, kv_heads, scale,
                                                       partials, idx_out, idx_stride, seq, cur_k, cur_v, out, apx, win,
                                                       blockIdx.x);
}

// The layer step in one launch (the tile-window form): workgroups
// 0 .. nscore - 1 are the scorer's (tile id mod tiles of KV group
// id / tiles, 512 threads), the rest the select + attention blocks (block
// id - nscore, 256 threads: the upper four waves end at once).  The two
// roles hand off through the scorer's histogram counts (score_d128_body,
// attn_select_chunk_body with HANDOFF).
template <typename T, int KPT, int NB, int QPK, int TPT>
__global__ __launch_bounds__(kScoreThreads) void layer_step_fused_kernel(
    const uint4* __restrict__ k_sign, const uint4* __restrict__ k_mag, const uint16_t* __restrict__ k_low,
    const uint16_t* __restrict__ k_delta, int64_t cap, int nscore, int tiles, TileWindows tw,
    const T* __restrict__ q, const T* __restrict__ kc, const T* __restrict__ vc, int64_t k_hs, int64_t v_hs,
    uint16_t* __restrict__ keys, int64_t key_stride, int ntok, int k, int nchunks, int qpk, bool kv_groups,
    uint32_t* __restrict__ ghist, const int64_t* __restrict__ head_to_kv, int q_heads, int kv_heads, float scale,
    float* __restrict__ partials, int64_t* __restrict__ idx_out, int64_t idx_stride, const T* __restrict__ cur_k,
    const T* __restrict__ cur_v, T* __restrict__ out, WindowIn win) {
    static_assert(kScoreThreads == 2 * kAttnThreads, "a select block is the lower half of a workgroup");
    const uint32_t id = blockIdx.x;
    if (id < static_cast<uint32_t>(nscore)) {
        const uint32_t grow = id / static_cast<uint32_t>(tiles);
        score_d128_body<64, QPK, T, true, true, TPT>(nullptr, nullptr, nullptr, nullptr, q, k_sign, k_mag, k_low, k_delta,
                                                head_to_kv, q_heads, kv_heads, QPK, cap, ntok, keys, key_stride, ghist,
                                                SeqTable{}, tw, id - grow * static_cast<uint32_t>(tiles), grow);
        return;
    }
    // (a wave-uniform test, so the upper waves leave with a scalar branch;
    // the block's barriers then wait for the lower four alone)
    if (__builtin_amdgcn_readfirstlane(threadIdx.x) >= static_cast<uint32_t>(kAttnThreads)) return;
    attn_select_chunk_body<T, KPT, NB, false, kWinMaxTiles / 8, true>(
        q, kc, vc, k_hs, v_hs, keys, key_stride, ntok, k, nullptr, nullptr, nullptr, nchunks, qpk, kv_groups, ghist,
        head_to_kv, kv_heads, scale, partials, idx_out, idx_stride, SeqTable{}, cur_k, cur_v, out,
        StepAppendArgs<T>{}, win, id - static_cast<uint32_t>(nscore));
}

// Dense attention (the reference's full layers, popkv.py:1022-1038): every
// prefix token attends; the current token joins in the merge, as in the
// layer step.  Splits of kDenseSplit tokens.
constexpr int kDenseSplit = 512;
// The MFMA kernel fuses the merge for up to this many splits (64 x 512 =
// 32768 tokens: the merge loads every split's accumulators in one burst);
// longer prefixes take the separate wide merge.
constexpr int kDenseFusedMaxSplits = 64;

// Dense attention, one GQA group per workgroup: the QPK query heads of KV
// head g share every K/V row, so workgroup (s, g) reads each row of its
// 512-token split once and folds it into QPK online-softmax states (one Q.K
// dot and one V update per head per row).  Memory traffic is one pass over
// the KV head's rows instead of QPK.
template <typename T, int NB, int QPK>
__global__ __launch_bounds__(kAttnThreads) void attn_dense_gqa_kernel(
    const T* __restrict__ q, const T* __restrict__ kc, const T* __restrict__ vc, int64_t k_hs, int64_t v_hs,
    int64_t tokens, float scale, float* __restrict__ partials, int nsplit) {
    constexpr int D = 128, LPR = 16, SLOTS = kWave / LPR, ROWS_PER_PASS = SLOTS * kAttnWaves;
    const int g = blockIdx.y;
    const int s = blockIdx.x;
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int slot = wave * SLOTS + lane / LPR;
    const int dim0 = (lane % LPR) * 8;
    Raw8<T> qr[QPK];
#pragma unroll
    for (int j = 0; j < QPK; ++j) qr[j].load(q + static_cast<int64_t>(g * QPK + j) * D + dim0);
    const int t0 = s * kDenseSplit;
    const int n_rows = static_cast<int>(min<int64_t>(kDenseSplit, tokens - t0));
    const char* kb = reinterpret_cast<const char*>(kc + g * k_hs) + dim0 * sizeof(T);
    const char* vb = reinterpret_cast<const char*>(vc + g * v_hs) + dim0 * sizeof(T);
    SoftmaxState st[QPK];
#pragma unroll
    for (int j = 0; j < QPK; ++j) init_state(st[j]);
    for (int base = 0; base < n_rows; base += ROWS_PER_PASS * NB) {
        Raw8<T> kr[NB], vr[NB];
        bool live[NB];
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            const int r = base + b * ROWS_PER_PASS + slot;
            live[b] = r < n_rows;
            const uint32_t off = static_cast<uint32_t>(t0 + (live[b] ? r : 0)) * (D * sizeof(T));
            kr[b].load(reinterpret_cast<const T*>(kb + off));
            vr[b].load(reinterpret_cast<const T*>(vb + off));
        }
#pragma unroll
        for (int j = 0; j < QPK; ++j) fold_rows<T, NB>(st[j], qr[j], kr, vr, live, scale);
    }
#pragma unroll
    for (int j = 0; j < QPK; ++j) {
        store_partial<LPR>(st[j], lane, wave, dim0, D,
                           partials + (static_cast<int64_t>(g * QPK + j) * nsplit + s) * (D + 2));
        __syncthreads();  // store_partial's LDS is reused by the next head
    }
}

// Dense attention for GQA groups of four query heads in 16-bit types, with
// Q.K on the matrix cores: per 16-token tile one v_mfma_f32_16x16x32 chain
// (4 steps of 32 dims) multiplies A = the group's query rows (rows 0-3; rows
// 4-15 zero) by B = the tile's K rows (column n = token n), so lanes 0-15
// end with the four heads' logits of token `lane` (C layout: lane l holds
// rows 4*(l/16) .. +3 of column l % 16; A and B: lane l holds k-elements
// 8*(l/16) .. +7 of row / column l % 16).  The tile's softmax runs on those
// lanes (DPP row maxima, one running max per head and wave), the weights go
// through LDS to the four 16-lane row slots, and each slot folds 4 of the
// tile's V rows into its accumulators (8 dims per lane) with the VALU.
// Workgroup (split, KV head) = 4 waves of 128 tokens; tiles double-buffered
// (the next tile's K and V loads issued before the current tile is folded).
template <typename T> struct MfmaVec8;
template <> struct MfmaVec8<bf16_t> { typedef __bf16 type __attribute__((ext_vector_type(8))); };
template <> struct MfmaVec8<f16_t> { typedef _Float16 type __attribute__((ext_vector_type(8))); };
typedef float mfma_f32x4 __attribute__((ext_vector_type(4)));

template <typename T>
__device__ __forceinline__ mfma_f32x4 mfma_16x16x32(uint4 a, uint4 b, mfma_f32x4 c) {
    using V = typename MfmaVec8<T>::type;
    if constexpr (std::is_same_v<T, bf16_t>)
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(V, a), __builtin_bit_cast(V, b), c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(V, a), __builtin_bit_cast(V, b), c, 0, 0, 0);
}

template <typename T>
__global__ __launch_bounds__(kAttnThreads) void attn_dense_mfma_kernel(
    const T* __restrict__ q, const T* __restrict__ kc, const T* __restrict__ vc, int64_t k_hs, int64_t v_hs,
    int64_t tokens, float scale, float* __restrict__ partials, int nsplit, uint32_t* __restrict__ tickets,
    const T* __restrict__ cur_k, const T* __restrict__ cur_v, T* __restrict__ out) {
    constexpr int D = 128, QPK = 4, TILE = 16;
    constexpr int WTOK = kDenseSplit / kAttnWaves;  // tokens per wave
    constexpr int NT = WTOK / TILE;                  // tiles per wave
    const int g = blockIdx.y;
    const int s = blockIdx.x;
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int col = lane & 15;  // MFMA row / column; the V dim slice 8*col
    const int grp = lane >> 4;  // MFMA k-group; the V row slot
    const int t0 = s * kDenseSplit;
    const int n_rows = static_cast<int>(min<int64_t>(kDenseSplit, tokens - t0));
    const int w0 = wave * WTOK;
    uint4 qa[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
        qa[i] = col < QPK ? *reinterpret_cast<const uint4*>(q + static_cast<int64_t>(g * QPK + col) * D + 32 * i + 8 * grp)
                          : make_uint4(0u, 0u, 0u, 0u);
    const char* kb = reinterpret_cast<const char*>(kc + g * k_hs) + 8 * grp * sizeof(T);
    const char* vb = reinterpret_cast<const char*>(vc + g * v_hs) + 8 * col * sizeof(T);
    // rows past the split's end re-read the split's first row (weight 0)
    auto load_tile = [&](int it, uint4 (&kt)[4], uint4 (&vt)[4]) {
        const int rk = w0 + it * TILE + col;
        const uint32_t ko = static_cast<uint32_t>(t0 + (rk < n_rows ? rk : 0)) * (D * sizeof(T));
#pragma unroll
        for (int i = 0; i < 4; ++i) kt[i] = *reinterpret_cast<const uint4*>(kb + ko + 32 * i * sizeof(T));
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int rv = w0 + it * TILE + 4 * grp + r;
            const uint32_t vo = static_cast<uint32_t>(t0 + (rv < n_rows ? rv : 0)) * (D * sizeof(T));
            vt[r] = *reinterpret_cast<const uint4*>(vb + vo);
        }
    };
    __shared__ float4 s_p[kAttnWaves][TILE];
    float m_run[QPK], lsum[QPK], acc[QPK][8];
#pragma unroll
    for (int j = 0; j < QPK; ++j) {
        m_run[j] = -INFINITY;
        lsum[j] = 0.0f;
#pragma unroll
        for (int d = 0; d < 8; ++d) acc[j][d] = 0.0f;
    }
    auto fold_tile = [&](int it, const uint4 (&kt)[4], const uint4 (&vt)[4]) {
        mfma_f32x4 c = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int i = 0; i < 4; ++i) c = mfma_16x16x32<T>(qa[i], kt[i], c);
        const bool live = w0 + it * TILE + col < n_rows;
        float p[QPK], alpha[QPK];
        bool rescale = false;
#pragma unroll
        for (int j = 0; j < QPK; ++j) {
            const float sj = live ? c[j] * scale : -INFINITY;
            float mx = fmaxf(sj, dpp_mov<0xB1>(sj));
            mx = fmaxf(mx, dpp_mov<0x4E>(mx));
            mx = fmaxf(mx, dpp_mov<0x141>(mx));
            mx = fmaxf(mx, dpp_mov<0x140>(mx));
            const float mt = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, mx), 0));
            const float mn = fmaxf(m_run[j], mt);
            alpha[j] = mn == -INFINITY ? 1.0f : __expf(m_run[j] - mn);  // m_run = -inf gives 0
            p[j] = mn == -INFINITY ? 0.0f : __expf(sj - mn);           // dead rows give 0
            rescale = rescale || mn != m_run[j];
            m_run[j] = mn;
        }
        if (lane < TILE) s_p[wave][col] = make_float4(p[0], p[1], p[2], p[3]);
        // the wave reads its own weights next: one wave's LDS operations complete in order
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        if (rescale) {  // wave-uniform: some head's running max moved
#pragma unroll
            for (int j = 0; j < QPK; ++j) {
                lsum[j] *= alpha[j];
#pragma unroll
                for (int d = 0; d < 8; ++d) acc[j][d] *= alpha[j];
            }
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float4 pr = s_p[wave][4 * grp + r];
            Raw8<T> v;
            v.u = vt[r];
            float vf[8];
#pragma unroll
            for (int d = 0; d < 8; ++d) vf[d] = v.get(d);
            const float pj[QPK] = {pr.x, pr.y, pr.z, pr.w};
#pragma unroll
            for (int j = 0; j < QPK; ++j) {
                lsum[j] += pj[j];
#pragma unroll
                for (int d = 0; d < 8; ++d) acc[j][d] = fmaf(pj[j], vf[d], acc[j][d]);
            }
        }
        // the next tile's weights overwrite s_p[wave] only after every lane has read
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    };
    // a ring of AHEAD + 1 tiles: tile it + AHEAD is issued before tile it is
    // folded (fully unrolled, so every ring index is a constant)
    constexpr int AHEAD = 1;
    uint4 kt[AHEAD + 1][4], vt[AHEAD + 1][4];
#pragma unroll
    for (int it = 0; it < AHEAD; ++it) load_tile(it, kt[it], vt[it]);
#pragma unroll
    for (int it = 0; it < NT; ++it) {
        if (it + AHEAD < NT) load_tile(it + AHEAD, kt[(it + AHEAD) % (AHEAD + 1)], vt[(it + AHEAD) % (AHEAD + 1)]);
        fold_tile(it, kt[it % (AHEAD + 1)], vt[it % (AHEAD + 1)]);
    }
    const bool fused = tickets != nullptr;  // the merge runs in the group's last block (below)
#pragma unroll
    for (int j = 0; j < QPK; ++j) {
        SoftmaxState st;
        st.m = m_run[j];
        st.l = lsum[j];
#pragma unroll
        for (int d = 0; d < 8; ++d) st.acc[d] = acc[j][d];
        store_partial<16>(st, lane, wave, 8 * col, D,
                          partials + (static_cast<int64_t>(g * QPK + j) * nsplit + s) * (D + 2), fused);
        __syncthreads();  // store_partial's LDS is reused by the next head
    }
    if (!fused) return;
    // Fused merge, as in the layer step's select + attention kernel: the
    // states went out with device-coherent stores; once this block's are
    // acknowledged (the gfx942 / gfx950 rule stated at st_f32) it takes a
    // ticket on tickets[g] (zero between calls), and the group's last block
    // merges each of its heads' splits with the current token (wave j: head
    // g * QPK + j, every split's accumulators loaded in one burst of up to
    // 64) and resets the ticket.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    __shared__ uint32_t s_last;
    if (threadIdx.x == 0) {
        const uint32_t old = __hip_atomic_fetch_add(&tickets[g], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s_last = old + 1u == static_cast<uint32_t>(nsplit) ? 1u : 0u;
    }
    __syncthreads();
    if (s_last == 0u) return;
    if (threadIdx.x == 0) __hip_atomic_store(&tickets[g], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int h = g * QPK + wave;
    merge_head<T, true, 64>(partials + static_cast<int64_t>(h) * nsplit * (D + 2), nsplit,
                            q + static_cast<int64_t>(h) * D, cur_k + static_cast<int64_t>(g) * D,
                            cur_v + static_cast<int64_t>(g) * D, scale, out + static_cast<int64_t>(h) * D);
}


// Layer-step merge kernel (the unfused form: popkv_layer_step_attention's
// timing runs, and the dense layers): one wave per head, see merge_head.
template <typename T>
__global__ __launch_bounds__(kWave) void attn_merge_current_kernel(
    const float* __restrict__ partials, int nsplit, const T* __restrict__ q, const T* __restrict__ cur_k,
    const T* __restrict__ cur_v, const int64_t* __restrict__ head_to_kv, int kv_heads, float scale,
    T* __restrict__ out, int64_t* __restrict__ idx_out, int64_t idx_stride, int64_t idx_slot, int64_t current,
    SeqTable seq) {
    constexpr int D = 128, S = D + 2;
    const int h = blockIdx.x;
    const int lane = threadIdx.x;
    // the current token's index slot of the layer step's int64 indices, and
    // the KV row of its current k/v (no mapping: the plain GQA grouping of
    // the dense layers)
    const int64_t kvh = merge_kv_row(seq, head_to_kv, h, kv_heads, gridDim.x, &idx_slot, &current);
    if (idx_out != nullptr && lane == 0) idx_out[static_cast<int64_t>(h) * idx_stride + idx_slot] = current;
    merge_head<T, false>(partials + static_cast<int64_t>(h) * nsplit * S, nsplit, q + static_cast<int64_t>(h) * D,
                         cur_k + kvh * D, cur_v + kvh * D, scale, out + static_cast<int64_t>(h) * D);
}

// Merge for many splits (dense layers: one split per 512 tokens): four
// waves per head, wave w folding splits [16w, 16w + 16), [64 + 16w, ...) --
// each batch of 16 in one load burst -- into a running (m, l, acc) state;
// wave 0 then combines the four states with the current token.  The layer
// step's merge (at most 16 splits at C1) keeps the one-wave kernel above.
constexpr int kMergeWaves = 4;

template <typename T>
__global__ __launch_bounds__(kWave * kMergeWaves) void attn_merge_wide_kernel(
    const float* __restrict__ partials, int nsplit, const T* __restrict__ q, const T* __restrict__ cur_k,
    const T* __restrict__ cur_v, const int64_t* __restrict__ head_to_kv, int kv_heads, float scale,
    T* __restrict__ out, int64_t* __restrict__ idx_out, int64_t idx_stride, int64_t idx_slot, int64_t current,
    SeqTable seq) {
    constexpr int D = 128, S = D + 2;
    const int h = blockIdx.x;
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int64_t kvh = merge_kv_row(seq, head_to_kv, h, kv_heads, gridDim.x, &idx_slot, &current);
    if (idx_out != nullptr && threadIdx.x == 0) idx_out[static_cast<int64_t>(h) * idx_stride + idx_slot] = current;
    const float* ps = partials + static_cast<int64_t>(h) * nsplit * S;
    float q0 = 0.0f, q1 = 0.0f, k0 = 0.0f, k1 = 0.0f, v0 = 0.0f, v1 = 0.0f;
    if (wave == 0) {  // the current token's operands, in flight during the splits
        const T* qh = q + static_cast<int64_t>(h) * D;
        q0 = Elem<T>::load(qh, lane);
        q1 = Elem<T>::load(qh, lane + 64);
        k0 = Elem<T>::load(cur_k + kvh * D, lane);
        k1 = Elem<T>::load(cur_k + kvh * D, lane + 64);
        v0 = Elem<T>::load(cur_v + kvh * D, lane);
        v1 = Elem<T>::load(cur_v + kvh * D, lane + 64);
    }
    float wm = -INFINITY, wl = 0.0f, a0 = 0.0f, a1 = 0.0f;
    for (int s0 = wave * kMergeFirst; s0 < nsplit; s0 += kMergeWaves * kMergeFirst) {
        const int nb = min(kMergeFirst, nsplit - s0);
        float m = -INFINITY, l = 0.0f;
        if (lane < nb) {
            m = ps[static_cast<int64_t>(s0 + lane) * S];
            l = ps[static_cast<int64_t>(s0 + lane) * S + 1];
        }
        float c0[kMergeFirst], c1[kMergeFirst];
#pragma unroll
        for (int j = 0; j < kMergeFirst; ++j) {
            const int64_t so = static_cast<int64_t>(s0 + min(j, nb - 1)) * S + 2;
            c0[j] = ps[so + lane];
            c1[j] = ps[so + lane + 64];
        }
        const float nm = fmaxf(wm, wave_max(m));
        const float alpha = wm == -INFINITY ? 0.0f : __expf(wm - nm);
        const float w = m == -INFINITY ? 0.0f : __expf(m - nm);
        wl = wl * alpha + wave_sum(l * w);
        a0 *= alpha;
        a1 *= alpha;
#pragma unroll
        for (int j = 0; j < kMergeFirst; ++j) {
            if (j < nb) {
                const float ws = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, w), j));
                a0 = fmaf(ws, c0[j], a0);
                a1 = fmaf(ws, c1[j], a1);
            }
        }
        wm = nm;
    }
    __shared__ float s_m[kMergeWaves], s_l[kMergeWaves], s_a[kMergeWaves][D];
    if (lane == 0) {
        s_m[wave] = wm;
        s_l[wave] = wl;
    }
    s_a[wave][lane] = a0;
    s_a[wave][lane + 64] = a1;
    __syncthreads();
    if (wave == 0) {
        const float cur_m = wave_sum(q0 * k0 + q1 * k1) * scale;
        float mx = cur_m;
#pragma unroll
        for (int w = 0; w < kMergeWaves; ++w) mx = fmaxf(mx, s_m[w]);
        const float wc = __expf(cur_m - mx);
        float den = wc, num0 = wc * v0, num1 = wc * v1;
#pragma unroll
        for (int w = 0; w < kMergeWaves; ++w) {
            if (s_m[w] != -INFINITY) {
                const float f = __expf(s_m[w] - mx);
                den += s_l[w] * f;
                num0 = fmaf(f, s_a[w][lane], num0);
                num1 = fmaf(f, s_a[w][lane + 64], num1);
            }
        }
        Elem<T>::store(out + static_cast<int64_t>(h) * D, lane, num0 / den);
        Elem<T>::store(out + static_cast<int64_t>(h) * D, lane + 64, num1 / den);
    }
}

// API-path partial attention, fast form (head_dim 128, contiguous K/V rows,
// the reference's 256-row splits, 16-byte aligned index rows): row slot q
// owns the split's entries [16q, 16q + 16) and reads them with 16-byte
// loads; the rows come from the caller's index
// tensor (int32 or int64) with its validity mask and the current-token
// convention of sparse_kernels.py:267-286 (an index equal to prefix_tokens
// reads current_k / current_v; any other index is clamped into the cache).
// Entries past `selected` are never read from the index tensor; dead or
// masked rows re-read a clamped, in-bounds row with weight 0.
template <typename T, typename IdxT, int NB>
__global__ __launch_bounds__(kAttnThreads) void attn_partial128_kernel(
    const T* __restrict__ q, const T* __restrict__ kc, const T* __restrict__ vc, int64_t k_hs, int64_t v_hs,
    int64_t prefix_tokens, const T* __restrict__ cur_k, const T* __restrict__ cur_v, const IdxT* __restrict__ idx,
    int64_t idx_stride, const uint8_t* __restrict__ valid, const int64_t* __restrict__ head_to_kv, int kv_heads,
    int64_t selected, float scale, float* __restrict__ partials, int nsplit) {
    constexpr int D = 128, LPR = 16, SLOTS = kWave / LPR, NSLOT = SLOTS * kAttnWaves, SPLIT = kSplitRows;
    constexpr int RPS = SPLIT / NSLOT;                                 // entries per row slot
    constexpr int PER = 16 / static_cast<int>(sizeof(IdxT));          // indices per 16-byte load
    static_assert(RPS == 16 && RPS % NB == 0, "16 entries per slot, NB per pass");
    const int h = blockIdx.y;
    const int s = blockIdx.x;
    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = tid / kWave;
    const int slot = wave * SLOTS + lane / LPR;
    const int dim0 = (lane % LPR) * 8;
    const int64_t kvh = min(max(head_to_kv[h], static_cast<int64_t>(0)), static_cast<int64_t>(kv_heads - 1));

    const int n_rows = static_cast<int>(min<int64_t>(SPLIT, selected - static_cast<int64_t>(s) * SPLIT));
    const int r0 = slot * RPS;  // this slot's first row in the split
    const int64_t e0 = static_cast<int64_t>(h) * idx_stride + static_cast<int64_t>(s) * SPLIT + r0;
    // whole 16-byte packets first, all in flight before any is used; the
    // split's ragged tail (rare) is read element by element afterwards
    // (a packet past the split's rows re-reads the head's first packet: an
    // index row holds a positive multiple of 16 bytes)
    uint4 uc[RPS / PER];
#pragma unroll
    for (int c = 0; c < RPS; c += PER) {
        const bool in = r0 + c + PER <= n_rows;
        uc[c / PER] = *reinterpret_cast<const uint4*>(idx + (in ? e0 + c : static_cast<int64_t>(h) * idx_stride));
    }
    int64_t tk[RPS];
#pragma unroll
    for (int c = 0; c < RPS; c += PER) {
        const IdxT* v = reinterpret_cast<const IdxT*>(&uc[c / PER]);
#pragma unroll
        for (int i = 0; i < PER; ++i) tk[c + i] = static_cast<int64_t>(v[i]);
        if (r0 + c + PER > n_rows) {  // rows past n_rows are dead below
#pragma unroll
            for (int i = 0; i < PER; ++i) tk[c + i] = r0 + c + i < n_rows ? static_cast<int64_t>(idx[e0 + c + i]) : 0;
        }
    }
    uint32_t live = 0;  // bit j: row r0 + j exists and is not masked out
#pragma unroll
    for (int j = 0; j < RPS; ++j) live |= (r0 + j < n_rows ? 1u : 0u) << j;
    if (valid != nullptr && live != 0u) {
        if (r0 + RPS <= n_rows) {
            const uint4 u = *reinterpret_cast<const uint4*>(valid + e0);
            const uint8_t* b = reinterpret_cast<const uint8_t*>(&u);
#pragma unroll
            for (int j = 0; j < RPS; ++j) live &= ~((b[j] == 0 ? 1u : 0u) << j);
        } else {
#pragma unroll
            for (int j = 0; j < RPS; ++j)
                if (r0 + j < n_rows && valid[e0 + j] == 0) live &= ~(1u << j);
        }
    }
    Raw8<T> qr;
    qr.load(q + static_cast<int64_t>(h) * D + dim0);
    const T* kb = kc + kvh * k_hs + dim0;
    const T* vb = vc + kvh * v_hs + dim0;
    const T* ckp = cur_k + kvh * D + dim0;
    const T* cvp = cur_v + kvh * D + dim0;

    SoftmaxState st;
    init_state(st);
#pragma unroll
    for (int p = 0; p < RPS / NB; ++p) {
        Raw8<T> kr[NB], vr[NB];
        bool lv[NB];
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            const int j = p * NB + b;
            lv[b] = (live >> j) & 1u;
            const int64_t t = tk[j];
            const bool is_cur = lv[b] && t == prefix_tokens;
            const int64_t tc = min(max(t, static_cast<int64_t>(0)), prefix_tokens - 1);
            kr[b].load(is_cur ? ckp : kb + tc * D);
            vr[b].load(is_cur ? cvp : vb + tc * D);
        }
        fold_rows<T, NB>(st, qr, kr, vr, lv, scale);
    }
    store_partial<LPR>(st, lane, wave, dim0, D, partials + (static_cast<int64_t>(h) * nsplit + s) * (D + 2));
}

// Typed arguments of one partial-attention launch.
template <typename T, typename IdxT>
struct PartialArgs {
    const T *q, *kc, *vc, *ck, *cv;
    int64_t k_hs, k_ts, v_hs, v_ts, prefix_tokens;
    const IdxT* idx;
    int64_t idx_stride;
    const uint8_t* valid;
    const int64_t* h2k;
    int qh, kvh, d;
    int64_t selected;
    int split;
    float* partials;
};

template <int LPR, typename T, typename IdxT>
hipError_t launch_partial_lpr(const PartialArgs<T, IdxT>& a, hipStream_t stream) {
    constexpr int NB = (sizeof(T) == 4 || LPR == 32) ? 8 : 16;
    const int nsplit = static_cast<int>((a.selected + a.split - 1) / a.split);
    const float scale = static_cast<float>(1.0 / sqrt(static_cast<double>(a.d)));
    dim3 grid(static_cast<unsigned>(nsplit), static_cast<unsigned>(a.qh));
    hipLaunchKernelGGL((attn_partial_kernel<T, IdxT, LPR, NB>), grid, dim3(kAttnThreads), 0, stream, a.q, a.kc, a.vc,
                       a.k_hs, a.k_ts, a.v_hs, a.v_ts, a.prefix_tokens, a.ck, a.cv, a.idx, a.idx_stride, a.valid,
                       a.h2k, a.kvh, a.d, a.selected, a.split, scale, a.partials, nsplit);
    return hipGetLastError();
}

// The fast form's preconditions: head_dim 128, contiguous rows, 256-row
// splits, 16-byte aligned q / K / V / current rows, index and mask rows.
template <typename T, typename IdxT>
bool partial128_ok(const PartialArgs<T, IdxT>& a) {
    auto al = [](const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
    return a.d == 128 && a.k_ts == 128 && a.v_ts == 128 && a.split == kSplitRows && al(a.q) && al(a.kc) &&
           al(a.vc) && al(a.ck) && al(a.cv) && (a.k_hs * static_cast<int64_t>(sizeof(T))) % 16 == 0 &&
           (a.v_hs * static_cast<int64_t>(sizeof(T))) % 16 == 0 && al(a.idx) &&
           (a.idx_stride * static_cast<int64_t>(sizeof(IdxT))) % 16 == 0 &&
           (a.valid == nullptr || (al(a.valid) && a.idx_stride % 16 == 0));
}

template <typename T, typename IdxT>
hipError_t launch_partial_t(const PartialArgs<T, IdxT>& a, hipStream_t stream) {
    if (partial128_ok(a)) {
        const int nsplit = static_cast<int>((a.selected + a.split - 1) / a.split);
        const float scale = static_cast<float>(1.0 / sqrt(128.0));
        dim3 grid(static_cast<unsigned>(nsplit), static_cast<unsigned>(a.qh));
        hipLaunchKernelGGL((attn_partial128_kernel<T, IdxT, 8>), grid, dim3(kAttnThreads), 0, stream, a.q, a.kc, a.vc,
                           a.k_hs, a.v_hs, a.prefix_tokens, a.ck, a.cv, a.idx, a.idx_stride, a.valid, a.h2k, a.kvh,
                           a.selected, scale, a.partials, nsplit);
        return hipGetLastError();
    }
    if (a.d <= 64) return launch_partial_lpr<8>(a, stream);
    if (a.d <= 128) return launch_partial_lpr<16>(a, stream);
    return launch_partial_lpr<32>(a, stream);
}

template <typename T>
hipError_t launch_partial_dt(const void* q, const void* kc, const void* vc, int64_t k_hs, int64_t k_ts, int64_t v_hs,
                             int64_t v_ts, int64_t prefix_tokens, const void* ck, const void* cv, const void* idx,
                             int index_dtype, int64_t idx_stride, const uint8_t* valid, const int64_t* h2k, int qh,
                             int kvh, int d, int64_t selected, int split, float* partials, hipStream_t stream) {
    const T* q_ = static_cast<const T*>(q);
    const T* k_ = static_cast<const T*>(kc);
    const T* v_ = static_cast<const T*>(vc);
    const T* ck_ = static_cast<const T*>(ck);
    const T* cv_ = static_cast<const T*>(cv);
    if (index_dtype == POPKV_INDEX_I32) {
        PartialArgs<T, int32_t> a{q_, k_, v_, ck_, cv_, k_hs, k_ts, v_hs, v_ts, prefix_tokens,
                                  static_cast<const int32_t*>(idx), idx_stride, valid, h2k, qh, kvh, d, selected,
                                  split, partials};
        return launch_partial_t(a, stream);
    }
    PartialArgs<T, int64_t> a{q_, k_, v_, ck_, cv_, k_hs, k_ts, v_hs, v_ts, prefix_tokens,
                              static_cast<const int64_t*>(idx), idx_stride, valid, h2k, qh, kvh, d, selected, split,
                              partials};
    return launch_partial_t(a, stream);
}

}  // namespace

hipError_t launch_attention_partial(const void* queries, int dtype, const void* prefix_k, const void* prefix_v,
                                    int64_t k_head_stride, int64_t k_token_stride, int64_t v_head_stride,
                                    int64_t v_token_stride, int64_t prefix_tokens, const void* current_k,
                                    const void* current_v, const void* indices, int index_dtype,
                                    int64_t index_row_stride, const uint8_t* valid_mask, const int64_t* head_to_kv,
                                    int q_heads, int kv_heads, int head_dim, int64_t selected, int split_tokens,
                                    float* partials, hipStream_t stream) {
    switch (dtype) {
        case POPKV_DTYPE_F32:
            return launch_partial_dt<float>(queries, prefix_k, prefix_v, k_head_stride, k_token_stride, v_head_stride,
                                            v_token_stride, prefix_tokens, current_k, current_v, indices, index_dtype,
                                            index_row_stride, valid_mask, head_to_kv, q_heads, kv_heads, head_dim,
                                            selected, split_tokens, partials, stream);
        case POPKV_DTYPE_F16:
            return launch_partial_dt<f16_t>(queries, prefix_k, prefix_v, k_head_stride, k_token_stride, v_head_stride,
                                            v_token_stride, prefix_tokens, current_k, current_v, indices, index_dtype,
                                            index_row_stride, valid_mask, head_to_kv, q_heads, kv_heads, head_dim,
                                            selected, split_tokens, partials, stream);
        default:
            return launch_partial_dt<bf16_t>(queries, prefix_k, prefix_v, k_head_stride, k_token_stride,
                                             v_head_stride, v_token_stride, prefix_tokens, current_k, current_v,
                                             indices, index_dtype, index_row_stride, valid_mask, head_to_kv, q_heads,
                                             kv_heads, head_dim, selected, split_tokens, partials, stream);
    }
}

hipError_t launch_attention_merge(const float* partials, int q_heads, int64_t splits, int head_dim, void* output,
                                  int out_dtype, hipStream_t stream) {
    dim3 grid(static_cast<unsigned>(q_heads)), block(kMergeThreads);
    const int ns = static_cast<int>(splits);
    switch (out_dtype) {
        case POPKV_DTYPE_F32:
            hipLaunchKernelGGL((attn_merge_kernel<float>), grid, block, 0, stream, partials, ns, head_dim,
                               static_cast<float*>(output));
            break;
        case POPKV_DTYPE_F16:
            hipLaunchKernelGGL((attn_merge_kernel<f16_t>), grid, block, 0, stream, partials, ns, head_dim,
                               static_cast<f16_t*>(output));
            break;
        default:
            hipLaunchKernelGGL((attn_merge_kernel<bf16_t>), grid, block, 0, stream, partials, ns, head_dim,
                               static_cast<bf16_t*>(output));
            break;
    }
    return hipGetLastError();
}


namespace {
template <typename T>
hipError_t launch_select_chunks_t(const void* q, const void* kc, const void* vc, int64_t k_hs, int64_t v_hs,
                                  const uint16_t* keys, int64_t key_stride, int64_t tokens, int64_t k,
                                  const uint32_t* rec, const uint16_t* h2, const uint32_t* gt1, uint32_t* ghist,
                                  const int64_t* h2k, int q_heads, int kv_heads, float* partials, int64_t* idx_out,
                                  int64_t idx_stride, const SeqTable& seq, const void* cur_k, const void* cur_v,
                                  void* out, hipStream_t stream, const DecodeAppend* app, const WindowIn* win) {
    // 10 rows per slot and pass: 160 per pass, so a chunk holding up to 320
    // selected tokens (C1: 204-294 in chunks of 2048) is gathered in two
    // passes.  Measured at C1, select + attention: 8 rows 16.5 us (three
    // passes above 256), 10 rows 15.5 us, 12 rows 16.4 us.
    constexpr int NB = 10;
    const StepChunks ch = step_chunks(tokens, k, q_heads);
    const float scale = static_cast<float>(1.0 / sqrt(128.0));
    const int nt = static_cast<int>(tokens), kk = static_cast<int>(k), nc = static_cast<int>(ch.count);
    // q_heads: rows of the step (a batched step: B * QH); the placement
    // groups rows by GQA group (a batched step's groups are b * KVH + j)
    const bool batched = seq.tokens != nullptr;
    const int qpk_all = batched ? seq.q_heads / seq.kv_heads : (kv_heads > 0 ? q_heads / kv_heads : 1);
    const int kv_all = batched ? q_heads / qpk_all : kv_heads;
    const bool groups = kv_all % 8 == 0 && (batched || q_heads % kv_heads == 0);
    const int qpk = groups ? qpk_all : 1;
    const int kv_clamp = batched ? seq.kv_heads : kv_heads;
    StepAppendArgs<T> apx;
    if (app != nullptr && batched) {
        apx.ap.new_k = static_cast<const T*>(app->new_k);
        apx.ap.new_v = static_cast<const T*>(app->new_v);
        apx.ap.key_cache = static_cast<T*>(app->key_cache);
        apx.ap.value_cache = static_cast<T*>(app->value_cache);
        apx.ap.cache_rows = app->cache_rows;
        apx.ap.counts = seq.tokens;
        apx.ap.kv_heads = seq.kv_heads;
        apx.ap.status = app->status;
        apx.k_sign = app->k_sign;
        apx.k_mag = app->k_mag;
        apx.k_low = app->k_low;
        apx.k_delta = app->k_delta;
        apx.cap = app->capacity;
        apx.tg = app->token_group_size;
        apx.g = app->dim_group_size;
        apx.items = (q_heads / seq.q_heads) * seq.kv_heads;
        apx.blocks = (apx.items + 7) / 8 * 8;
    }
    const dim3 grid(static_cast<unsigned>(ch.count * q_heads + apx.blocks));
    const T *q_ = static_cast<const T*>(q), *k_ = static_cast<const T*>(kc), *v_ = static_cast<const T*>(vc);
    const T *ck_ = static_cast<const T*>(cur_k), *cv_ = static_cast<const T*>(cur_v);
    T* o_ = static_cast<T*>(out);
    const WindowIn wi = win != nullptr ? *win : WindowIn{};
#define POPKV_SC_W(KPT, WJ)                                                                                       \
    if (batched)                                                                                                 \
        hipLaunchKernelGGL((attn_select_chunk_kernel<T, KPT, NB, true, WJ>), grid, dim3(kAttnThreads), 0, stream,   \
                           q_, k_, v_, k_hs, v_hs, keys, key_stride, nt, kk, rec, h2, gt1, nc, qpk, groups, ghist, h2k, \
                           kv_clamp, scale, partials, idx_out, idx_stride, seq, ck_, cv_, o_, apx, wi);            \
    else                                                                                                         \
        hipLaunchKernelGGL((attn_select_chunk_kernel<T, KPT, NB, false, WJ>), grid, dim3(kAttnThreads), 0, stream,  \
                           q_, k_, v_, k_hs, v_hs, keys, key_stride, nt, kk, rec, h2, gt1, nc, qpk, groups, ghist, h2k, \
                           kv_clamp, scale, partials, idx_out, idx_stride, seq, ck_, cv_, o_, apx, wi)
#define POPKV_SC(KPT)             \
    case KPT:                     \
        POPKV_SC_W(KPT, 0);       \
        break
#define POPKV_SC_WIN(KPT)                                 \
    case KPT:                                             \
        POPKV_SC_W(KPT, kWinMaxTiles / 8);                \
        break
    if (win != nullptr) {
        // the tile windows (host-checked: window_kpt_ok, at most
        // kWinMaxTiles tiles of whole chunks)
        if (wi.tiles <= 0 || wi.tiles > kWinMaxTiles || wi.tile_tokens <= 0 || ch.tokens_per_chunk % wi.tile_tokens)
            return hipErrorInvalidValue;
        switch (ch.kpt) {
            POPKV_SC_WIN(4); POPKV_SC_WIN(8); POPKV_SC_WIN(16);
            default: return hipErrorInvalidValue;
        }
    } else {
        switch (ch.kpt) {
            POPKV_SC(1); POPKV_SC(2); POPKV_SC(4); POPKV_SC(6); POPKV_SC(8); POPKV_SC(12); POPKV_SC(16); POPKV_SC(24); POPKV_SC(32);
            default: return hipErrorInvalidValue;
        }
    }
#undef POPKV_SC_WIN
#undef POPKV_SC
#undef POPKV_SC_W
    return hipGetLastError();
}

template <typename T>
hipError_t launch_merge_current_t(const float* partials, int nsplit, const void* q, const void* cur_k,
                                  const void* cur_v, const int64_t* h2k, int q_heads, int kv_heads, void* out,
                                  int64_t* idx_out, int64_t idx_stride, int64_t idx_slot, int64_t current,
                                  const SeqTable& seq, hipStream_t stream) {
    const float scale = static_cast<float>(1.0 / sqrt(128.0));
    if (nsplit > kMergeFirst)
        hipLaunchKernelGGL((attn_merge_wide_kernel<T>), dim3(static_cast<unsigned>(q_heads)),
                           dim3(kWave * kMergeWaves), 0, stream, partials, nsplit, static_cast<const T*>(q),
                           static_cast<const T*>(cur_k), static_cast<const T*>(cur_v), h2k, kv_heads, scale,
                           static_cast<T*>(out), idx_out, idx_stride, idx_slot, current, seq);
    else
        hipLaunchKernelGGL((attn_merge_current_kernel<T>), dim3(static_cast<unsigned>(q_heads)), dim3(kWave), 0,
                           stream, partials, nsplit, static_cast<const T*>(q), static_cast<const T*>(cur_k),
                           static_cast<const T*>(cur_v), h2k, kv_heads, scale, static_cast<T*>(out), idx_out,
                           idx_stride, idx_slot, current, seq);
    return hipGetLastError();
}
template <typename T>
hipError_t launch_layer_step_fused_t(const void* queries, const int32_t* k_sign, const int32_t* k_mag,
                                     const uint16_t* k_low, const uint16_t* k_delta, int64_t capacity,
                                     const void* prefix_k, const void* prefix_v, int64_t k_hs, int64_t v_hs,
                                     uint16_t* keys, int64_t key_stride, int64_t tokens, int64_t k,
                                     const TileWindows& tw, const WindowIn& win, uint32_t* ghist,
                                     const int64_t* h2k, int q_heads, int kv_heads, float* partials, int64_t* idx_out,
                                     int64_t idx_stride, const void* cur_k, const void* cur_v, void* out,
                                     hipStream_t stream) {
    constexpr int NB = 10;  // as the two-launch form
    const StepChunks ch = step_chunks(tokens, k, q_heads);
    const float scale = static_cast<float>(1.0 / sqrt(128.0));
    const int qpk_all = q_heads / kv_heads;
    const bool groups = kv_heads % 8 == 0;
    const int qpk = groups ? qpk_all : 1;
    const int nscore = tw.tiles * kv_heads;
    const dim3 grid(static_cast<unsigned>(nscore + ch.count * q_heads));
    const uint4* ks4 = reinterpret_cast<const uint4*>(k_sign);
    const uint4* km4 = reinterpret_cast<const uint4*>(k_mag);
    const T *q_ = static_cast<const T*>(queries), *k_ = static_cast<const T*>(prefix_k),
            *v_ = static_cast<const T*>(prefix_v);
    const T *ck_ = static_cast<const T*>(cur_k), *cv_ = static_cast<const T*>(cur_v);
    T* o_ = static_cast<T*>(out);
    const int nt = static_cast<int>(tokens), kk = static_cast<int>(k), nc = static_cast<int>(ch.count);
#define POPKV_FUSED_T(KPT, QPK, TPT)                                                                                \
    hipLaunchKernelGGL((layer_step_fused_kernel<T, KPT, NB, QPK, TPT>), grid, dim3(kScoreThreads), 0, stream, ks4, \
                       km4, k_low, k_delta, capacity, nscore, tw.tiles, tw, q_, k_, v_, k_hs, v_hs, keys, key_stride, \
                       nt, kk, nc, qpk, groups, ghist, h2k, q_heads, kv_heads, scale, partials, idx_out, idx_stride,  \
                       ck_, cv_, o_, win)
    // 1024-token tiles (two tokens per scorer thread) or 512 (one)
    const bool one = win.tile_tokens == kScoreThreads;
#define POPKV_FUSED(KPT, QPK)             \
    if (one)                              \
        POPKV_FUSED_T(KPT, QPK, 1);       \
    else                                  \
        POPKV_FUSED_T(KPT, QPK, 2)
#define POPKV_FUSED_Q(KPT)                              \
    switch (qpk_all) {                                  \
        case 1: POPKV_FUSED(KPT, 1); break;             \
        case 2: POPKV_FUSED(KPT, 2); break;             \
        case 4: POPKV_FUSED(KPT, 4); break;             \
        case 8: POPKV_FUSED(KPT, 8); break;             \
        default: return hipErrorInvalidValue;           \
    }
    switch (ch.kpt) {
        case 4: POPKV_FUSED_Q(4); break;
        case 8: POPKV_FUSED_Q(8); break;
        case 16: POPKV_FUSED_Q(16); break;
        default: return hipErrorInvalidValue;
    }
#undef POPKV_FUSED_Q
#undef POPKV_FUSED
#undef POPKV_FUSED_T
    return hipGetLastError();
}

}  // namespace

hipError_t launch_layer_step_fused(const void* queries, int dtype, const int32_t* k_sign, const int32_t* k_mag,
                                   const uint16_t* k_low, const uint16_t* k_delta, int64_t capacity,
                                   const void* prefix_k, const void* prefix_v, int64_t k_head_stride,
                                   int64_t v_head_stride, uint16_t* keys, int64_t key_stride, int64_t tokens,
                                   int64_t k, const TileWindows& tw, const WindowIn& win, uint32_t* ghist,
                                   const int64_t* head_to_kv, int q_heads, int kv_heads, float* partials,
                                   int64_t* idx_out, int64_t idx_stride, const void* current_k,
                                   const void* current_v, void* output, hipStream_t stream) {
    // the shapes the window form takes (the caller checks them too)
    if (tokens <= 0 || k <= 0 || k >= tokens || q_heads <= 0 || kv_heads <= 0 || q_heads % kv_heads ||
        tw.tiles <= 0 || tw.tiles > kWinMaxTiles || win.tiles != tw.tiles ||
        (win.tile_tokens != 1024 && win.tile_tokens != 512) || tw.tile_tokens != win.tile_tokens ||
        (tokens + win.tile_tokens - 1) / win.tile_tokens != tw.tiles || output == nullptr)
        return hipErrorInvalidValue;
    const StepChunks ch = step_chunks(tokens, k, q_heads);
    if (!window_kpt_ok(ch.kpt) || ch.tokens_per_chunk % win.tile_tokens) return hipErrorInvalidValue;
    switch (dtype) {
        case POPKV_DTYPE_F32:
            return launch_layer_step_fused_t<float>(queries, k_sign, k_mag, k_low, k_delta, capacity, prefix_k,
                                                    prefix_v, k_head_stride, v_head_stride, keys, key_stride, tokens,
                                                    k, tw, win, ghist, head_to_kv, q_heads, kv_heads, partials,
                                                    idx_out, idx_stride, current_k, current_v, output, stream);
        case POPKV_DTYPE_F16:
            return launch_layer_step_fused_t<f16_t>(queries, k_sign, k_mag, k_low, k_delta, capacity, prefix_k,
                                                    prefix_v, k_head_stride, v_head_stride, keys, key_stride, tokens,
                                                    k, tw, win, ghist, head_to_kv, q_heads, kv_heads, partials,
                                                    idx_out, idx_stride, current_k, current_v, output, stream);
        default:
            return launch_layer_step_fused_t<bf16_t>(queries, k_sign, k_mag, k_low, k_delta, capacity, prefix_k,
                                                     prefix_v, k_head_stride, v_head_stride, keys, key_stride,
                                                     tokens, k, tw, win, ghist, head_to_kv, q_heads, kv_heads,
                                                     partials, idx_out, idx_stride, current_k, current_v, output,
                                                     stream);
    }
}

hipError_t launch_attention_select_chunks(const void* queries, int dtype, const void* prefix_k, const void* prefix_v,
                                          int64_t k_head_stride, int64_t v_head_stride, const uint16_t* keys,
                                          int64_t key_stride, int64_t tokens, int64_t k, const uint32_t* rec,
                                          const uint16_t* h2, const uint32_t* gt1, uint32_t* ghist,
                                          const int64_t* head_to_kv, int q_heads, int kv_heads, float* partials,
                                          int64_t* idx_out, int64_t idx_stride, const SeqTable& seq,
                                          const void* current_k, const void* current_v, void* output,
                                          hipStream_t stream, const DecodeAppend* append, const WindowIn* win) {
    if (tokens <= 0 || q_heads <= 0) return hipSuccess;
    switch (dtype) {
        case POPKV_DTYPE_F32:
            return launch_select_chunks_t<float>(queries, prefix_k, prefix_v, k_head_stride, v_head_stride, keys,
                                                 key_stride, tokens, k, rec, h2, gt1, ghist, head_to_kv, q_heads,
                                                 kv_heads, partials, idx_out, idx_stride, seq, current_k,
                                                 current_v, output, stream, append, win);
        case POPKV_DTYPE_F16:
            return launch_select_chunks_t<f16_t>(queries, prefix_k, prefix_v, k_head_stride, v_head_stride, keys,
                                                 key_stride, tokens, k, rec, h2, gt1, ghist, head_to_kv, q_heads,
                                                 kv_heads, partials, idx_out, idx_stride, seq, current_k,
                                                 current_v, output, stream, append, win);
        default:
            return launch_select_chunks_t<bf16_t>(queries, prefix_k, prefix_v, k_head_stride, v_head_stride, keys,
                                                  key_stride, tokens, k, rec, h2, gt1, ghist, head_to_kv, q_heads,
                                                  kv_heads, partials, idx_out, idx_stride, seq, current_k,
                                                 current_v, output, stream, append, win);
    }
}

hipError_t launch_merge_current(const float* partials, int nsplit, const void* queries, int dtype,
                                const void* current_k, const void* current_v, const int64_t* head_to_kv, int q_heads,
                                int kv_heads, void* output, int64_t* idx_out, int64_t idx_stride, int64_t idx_slot,
                                int64_t current, const SeqTable& seq, hipStream_t stream) {
    switch (dtype) {
        case POPKV_DTYPE_F32:
            return launch_merge_current_t<float>(partials, nsplit, queries, current_k, current_v, head_to_kv, q_heads,
                                                 kv_heads, output, idx_out, idx_stride, idx_slot, current, seq,
                                                 stream);
        case POPKV_DTYPE_F16:
            return launch_merge_current_t<f16_t>(partials, nsplit, queries, current_k, current_v, head_to_kv, q_heads,
                                                 kv_heads, output, idx_out, idx_stride, idx_slot, current, seq,
                                                 stream);
        default:
            return launch_merge_current_t<bf16_t>(partials, nsplit, queries, current_k, current_v, head_to_kv,
                                                  q_heads, kv_heads, output, idx_out, idx_stride, idx_slot, current,
                                                  seq, stream);
    }
}


namespace {
template <typename T>
hipError_t launch_dense_t(const void* q, const void* kc, const void* vc, int64_t k_hs, int64_t v_hs, int64_t tokens,
                          int nsplit, int q_heads, int kv_heads, float* partials, const DenseMerge* merge,
                          hipStream_t stream) {
    const float scale = static_cast<float>(1.0 / sqrt(128.0));
    const dim3 grid(static_cast<unsigned>(nsplit), static_cast<unsigned>(kv_heads));
    const T *q_ = static_cast<const T*>(q), *k_ = static_cast<const T*>(kc), *v_ = static_cast<const T*>(vc);
#define POPKV_DENSE(NB, QPK)                                                                                   \
    hipLaunchKernelGGL((attn_dense_gqa_kernel<T, NB, QPK>), grid, dim3(kAttnThreads), 0, stream, q_, k_, v_, k_hs, \
                       v_hs, tokens, scale, partials, nsplit)
    if constexpr (sizeof(T) == 2) {
        if (q_heads == 4 * kv_heads) {
            const bool fuse = merge != nullptr && nsplit <= kDenseFusedMaxSplits;
            hipLaunchKernelGGL((attn_dense_mfma_kernel<T>), grid, dim3(kAttnThreads), 0, stream, q_, k_, v_, k_hs, v_hs,
                               tokens, scale, partials, nsplit, fuse ? merge->tickets : nullptr,
                               fuse ? static_cast<const T*>(merge->current_k) : nullptr,
                               fuse ? static_cast<const T*>(merge->current_v) : nullptr,
                               fuse ? static_cast<T*>(merge->output) : nullptr);
            return hipGetLastError();
        }
    }
    switch (q_heads / kv_heads) {
        case 1: POPKV_DENSE((sizeof(T) == 4 ? 8 : 16), 1); break;
        case 2: POPKV_DENSE(8, 2); break;
        case 4: POPKV_DENSE(4, 4); break;  // 127 VGPRs; 8 rows: 180 (measured 0.3 us slower)
        default: POPKV_DENSE(4, 8); break;
    }
#undef POPKV_DENSE
    return hipGetLastError();
}
}  // namespace

int dense_splits(int64_t tokens) { return static_cast<int>((tokens + kDenseSplit - 1) / kDenseSplit); }

bool dense_merge_fuses(int dtype, int64_t tokens, int q_heads, int kv_heads) {
    const int ns = dense_splits(tokens);
    return dtype != POPKV_DTYPE_F32 && q_heads == 4 * kv_heads && ns > 0 && ns <= kDenseFusedMaxSplits;
}

hipError_t launch_attention_dense(const void* queries, int dtype, const void* prefix_k, const void* prefix_v,
                                  int64_t k_head_stride, int64_t v_head_stride, int64_t tokens, int q_heads,
                                  int kv_heads, float* partials, hipStream_t stream, const DenseMerge* merge) {
    const int ns = dense_splits(tokens);
    switch (dtype) {
        case POPKV_DTYPE_F32:
            return launch_dense_t<float>(queries, prefix_k, prefix_v, k_head_stride, v_head_stride, tokens, ns,
                                         q_heads, kv_heads, partials, merge, stream);
        case POPKV_DTYPE_F16:
            return launch_dense_t<f16_t>(queries, prefix_k, prefix_v, k_head_stride, v_head_stride, tokens, ns,
                                         q_heads, kv_heads, partials, merge, stream);
        default:
            return launch_dense_t<bf16_t>(queries, prefix_k, prefix_v, k_head_stride, v_head_stride, tokens, ns,
                                          q_heads, kv_heads, partials, merge, stream);
    }
}
}  // namespace popkv
