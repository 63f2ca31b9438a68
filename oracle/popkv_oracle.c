/*
 * CPU oracle for the PopKV decode-time retrieval path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file restates, in plain IEEE-754 single
 * precision C, the arithmetic of the reference's production CUDA path so that
 * the HIP kernels can be checked bit for bit.  Only tests/, the smoke() entry
 * and bench.py's CPU-baseline leg may load it; no product code path calls it.
 *
 * Build (oracle/Makefile): gcc -O2 -fPIC -shared -ffp-contract=off
 * -fno-fast-math.  x86-64 SSE arithmetic is IEEE binary32 with
 * round-to-nearest-even, no flush-to-zero, correctly rounded division, and
 * glibc's fmaf is a correctly rounded fused multiply-add.
 *
 * Reference (kw78999/PopKV) citations are file:line into the upstream tree.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ */
/* Scalar conversions                                                  */
/* ------------------------------------------------------------------ */

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* binary32 -> binary16, round to nearest even, subnormals kept, overflow to
 * inf, NaN kept quiet.  Plays the role of __float2half_rn
 * (popkv_ext.cu:139-140, :430-431, :496-497, :873). */
uint16_t po_f32_to_f16(float f) {
    uint32_t x = f2u(f);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ex = (x >> 23) & 0xffu;
    uint32_t man = x & 0x7fffffu;
    if (ex == 0xffu) return (uint16_t)(sign | 0x7c00u | (man ? 0x200u | (man >> 13) : 0u));
    int e = (int)ex - 127 + 15;
    if (e >= 0x1f) return (uint16_t)(sign | 0x7c00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;                /* below half the smallest subnormal */
        uint32_t m = man | 0x800000u;                       /* implicit bit */
        int shift = 14 - e;                                 /* 14..24 */
        uint32_t half = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t mid = 1u << (shift - 1);
        if (rem > mid || (rem == mid && (half & 1u))) half++;
        return (uint16_t)(sign | half);
    }
    uint32_t half = ((uint32_t)e << 10) | (man >> 13);
    uint32_t rem = man & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (half & 1u))) half++;   /* may carry into inf */
    return (uint16_t)(sign | half);
}

float po_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t ex = (h >> 10) & 0x1fu;
    uint32_t man = h & 0x3ffu;
    if (ex == 0) {
        if (man == 0) return u2f(sign);
        float v = (float)man * 5.9604644775390625e-08f;       /* man * 2^-24, exact */
        return sign ? -v : v;
    }
    if (ex == 0x1f) return u2f(sign | 0x7f800000u | (man << 13));
    return u2f(sign | ((ex - 15 + 127) << 23) | (man << 13));
}

float po_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

void po_f32_to_f16_array(const float* x, uint16_t* y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = po_f32_to_f16(x[i]);
}

/* 1/sqrt(D) rounded once to binary32.  The reference evaluates rsqrtf(D)
 * (popkv_ext.cu:203, :572, :776) under --use_fast_math; the contract here is
 * the correctly rounded value (0x3DB504F3 for D = 128). */
float po_inv_sqrt_dim(int64_t d) { return (float)(1.0 / sqrt((double)d)); }

/* ------------------------------------------------------------------ */
/* Representative sums: the reduction trees of the production kernels   */
/* ------------------------------------------------------------------ */

/* tree5 over 32 lanes, the shfl_down tree of popkv_ext.cu:122-127:
 * a_i = z_i + z_{i+16}, b_i = a_i + a_{i+8}, c_i = b_i + b_{i+4},
 * e_i = c_i + c_{i+2}, s = e_0 + e_1. */
static float tree5(const float* z) {
    float a[16], b[8], c[4], e[2];
    for (int i = 0; i < 16; ++i) a[i] = z[i] + z[i + 16];
    for (int i = 0; i < 8; ++i) b[i] = a[i] + a[i + 8];
    for (int i = 0; i < 4; ++i) c[i] = b[i] + b[i + 4];
    for (int i = 0; i < 2; ++i) e[i] = c[i] + c[i + 2];
    return e[0] + e[1];
}

/* tree4 over 16 lanes, the width-16 shfl_down tree of popkv_ext.cu:408-414. */
static float tree4(const float* z) {
    float a[8], b[4], c[2];
    for (int i = 0; i < 8; ++i) a[i] = z[i] + z[i + 8];
    for (int i = 0; i < 4; ++i) b[i] = a[i] + a[i + 4];
    for (int i = 0; i < 2; ++i) c[i] = b[i] + b[i + 2];
    return c[0] + c[1];
}

/* Sum of one representative group's contributions x[] (already zero where a
 * dimension is outside the head or in the other bucket), in the order of the
 * production packers:
 *   G32: tree5 over the word's 32 lanes       (popkv_ext.cu:117-127)
 *   G16: tree4 over the 16 lanes of the group (popkv_ext.cu:406-414; the
 *        generic kernel :338-360 runs tree5 with lanes 16..31 at +0, which
 *        is the same sum because every term is >= +0)
 *   G64: p_j = x_j + x_{j+32}, then tree5      (popkv_ext.cu:470-480; the
 *        generic kernel :338-360 gives (0 + x_j) + x_{j+32}, the same value)
 * x points at the group's first dimension and holds G entries. */
static float rep_tree_sum(const float* x, int g) {
    if (g == 32) return tree5(x);
    if (g == 16) return tree4(x);
    float p[32];
    for (int j = 0; j < 32; ++j) p[j] = x[j] + x[j + 32];
    return tree5(p);
}

/* low/delta with the empty-bucket rules of popkv_ext.cu:128-135. */
static void finish_rep(float ls, int ln, float hs, int hn, float* low, float* delta) {
    float lo, hi;
    if (ln == 0) {
        lo = hn ? hs / (float)hn : 0.0f;
        hi = lo;
    } else {
        lo = ls / (float)ln;
        hi = hn ? hs / (float)hn : lo;
    }
    *low = lo;
    *delta = hi - lo;
}

/* ------------------------------------------------------------------ */
/* Query encode                                                        */
/* ------------------------------------------------------------------ */

/* order 0: decode-path encode, representative sums as a left fold over
 *          ascending dimensions (popkv_ext.cu:232-281 for G32, :911-957
 *          for G16/G64; also the prelude of the generic scorers :169-201,
 *          :533-570).
 * order 1: score()-path warp encode for head_dim 128 (popkv_ext.cu:677-755),
 *          representative sums in the reduction-tree order above.
 * Thresholds use the whole head: neg = min*0.5, pos = max*0.5.
 * Outputs: sign/mag int32 [rows, W]; low/delta float [rows, R]. */
void po_query_encode(const float* q, int64_t rows, int64_t d, int g, int order,
                     int32_t* sign, int32_t* mag, float* low, float* delta) {
    int64_t words = (d + 31) / 32, reps = (d + g - 1) / g;
    for (int64_t row = 0; row < rows; ++row) {
        const float* v = q + row * d;
        float mn = v[0], mx = v[0];
        for (int64_t i = 1; i < d; ++i) { mn = fminf(mn, v[i]); mx = fmaxf(mx, v[i]); }
        float neg = mn * 0.5f, pos = mx * 0.5f;
        for (int64_t w = 0; w < words; ++w) {
            uint32_t sw = 0, mw = 0;
            for (int64_t i = w * 32; i < d && i < w * 32 + 32; ++i) {
                int s = v[i] >= 0.0f;
                int m = s ? (v[i] > pos) : (v[i] < neg);
                if (s) sw |= 1u << (i - w * 32);
                if (m) mw |= 1u << (i - w * 32);
            }
            sign[row * words + w] = (int32_t)sw;
            mag[row * words + w] = (int32_t)mw;
        }
        for (int64_t r = 0; r < reps; ++r) {
            float ls = 0.0f, hs = 0.0f;
            int ln = 0, hn = 0;
            int64_t start = r * g, end = start + g < d ? start + g : d;
            if (order == 0) {
                for (int64_t i = start; i < end; ++i) {
                    int s = v[i] >= 0.0f;
                    int m = s ? (v[i] > pos) : (v[i] < neg);
                    if (m) { hs += fabsf(v[i]); ++hn; } else { ls += fabsf(v[i]); ++ln; }
                }
            } else {
                float xl[64], xh[64];
                for (int j = 0; j < g; ++j) {
                    int64_t i = start + j;
                    xl[j] = 0.0f; xh[j] = 0.0f;
                    if (i < end) {
                        int s = v[i] >= 0.0f;
                        int m = s ? (v[i] > pos) : (v[i] < neg);
                        if (m) { xh[j] = fabsf(v[i]); ++hn; } else { xl[j] = fabsf(v[i]); ++ln; }
                    }
                }
                ls = rep_tree_sum(xl, g);
                hs = rep_tree_sum(xh, g);
            }
            finish_rep(ls, ln, hs, hn, &low[row * reps + r], &delta[row * reps + r]);
        }
    }
}

/* ------------------------------------------------------------------ */
/* Key pack / append                                                   */
/* ------------------------------------------------------------------ */

/* Encodes tokens [0, n) of keys [kvh, n, d] (contiguous) and writes rows
 * [off, off + n) of the packed cache: sign/mag int32 [kvh, cap, W],
 * low/delta fp16 bits [kvh, cap, R].  Token groups are [g*tg, (g+1)*tg)
 * clipped to n; per-dimension min/max use only the group's present tokens;
 * mag = sign ? v > 0.5*max : v < 0.5*min (popkv_ext.cu:79-143, :376-500,
 * :283-374; the in-place append popkv_ext.cu:1075-1092, :1177-1206). */
void po_pack_keys(const float* keys, int64_t kvh, int64_t n, int64_t d, int tg, int g,
                  int32_t* sign, int32_t* mag, uint16_t* low, uint16_t* delta,
                  int64_t cap, int64_t off) {
    int64_t words = (d + 31) / 32, reps = (d + g - 1) / g;
    float* mn = (float*)malloc(sizeof(float) * (size_t)d);
    float* mx = (float*)malloc(sizeof(float) * (size_t)d);
    for (int64_t h = 0; h < kvh; ++h) {
        for (int64_t gs = 0; gs < n; gs += tg) {
            int64_t ge = gs + tg < n ? gs + tg : n;
            for (int64_t i = 0; i < d; ++i) {
                float a = keys[(h * n + gs) * d + i];
                mn[i] = a; mx[i] = a;
                for (int64_t t = gs + 1; t < ge; ++t) {
                    float b = keys[(h * n + t) * d + i];
                    mn[i] = fminf(mn[i], b); mx[i] = fmaxf(mx[i], b);
                }
            }
            for (int64_t t = gs; t < ge; ++t) {
                const float* v = keys + (h * n + t) * d;
                int64_t orow = h * cap + off + t;
                for (int64_t w = 0; w < words; ++w) {
                    uint32_t sw = 0, mw = 0;
                    for (int64_t i = w * 32; i < d && i < w * 32 + 32; ++i) {
                        int s = v[i] >= 0.0f;
                        int m = s ? (v[i] > mx[i] * 0.5f) : (v[i] < mn[i] * 0.5f);
                        if (s) sw |= 1u << (i - w * 32);
                        if (m) mw |= 1u << (i - w * 32);
                    }
                    sign[orow * words + w] = (int32_t)sw;
                    mag[orow * words + w] = (int32_t)mw;
                }
                for (int64_t r = 0; r < reps; ++r) {
                    float xl[64], xh[64];
                    int ln = 0, hn = 0;
                    for (int j = 0; j < g; ++j) {
                        int64_t i = r * g + j;
                        xl[j] = 0.0f; xh[j] = 0.0f;
                        if (i < d) {
                            int s = v[i] >= 0.0f;
                            int m = s ? (v[i] > mx[i] * 0.5f) : (v[i] < mn[i] * 0.5f);
                            if (m) { xh[j] = fabsf(v[i]); ++hn; } else { xl[j] = fabsf(v[i]); ++ln; }
                        }
                    }
                    float lo, de;
                    finish_rep(rep_tree_sum(xl, g), ln, rep_tree_sum(xh, g), hn, &lo, &de);
                    low[orow * reps + r] = po_f32_to_f16(lo);
                    delta[orow * reps + r] = po_f32_to_f16(de);
                }
            }
        }
    }
    free(mn);
    free(mx);
}

/* ------------------------------------------------------------------ */
/* Popcount score                                                      */
/* ------------------------------------------------------------------ */

static inline int popc(uint32_t x) { return __builtin_popcount(x); }

/* popkv_reconstruct_u32 (popkv_ext.cu:502-515). */
static float recon_u32(uint32_t qs, uint32_t qm, uint32_t ks, uint32_t km, uint32_t mask,
                       float ql, float dq, float kl, float dk) {
    qm &= mask; km &= mask;
    uint32_t match = ~(qs ^ ks) & mask, both = qm & km;
    int cs = 2 * popc(match) - popc(mask);
    int cq = 2 * popc(match & qm) - popc(qm);
    int ck = 2 * popc(match & km) - popc(km);
    int cqk = 2 * popc(match & both) - popc(both);
    return fmaf(ql * kl, (float)cs, fmaf(dq * kl, (float)cq, fmaf(ql * dk, (float)ck, dq * dk * (float)cqk)));
}

/* head_dim 128 GQA scorer (popkv_ext.cu:757-876): every query head of KV
 * group j uses kvh = head_to_kv[j * QH/KVH]; total starts at +0 and adds one
 * term per representative; score = fp16_rne(total * 1/sqrt(128)).
 * q state [B, QH, 4] / [B, QH, R]; packed [KVH, cap, 4] / [KVH, cap, R];
 * out fp16 bits [B, QH, tokens]. */
void po_score_d128(const int32_t* q_sign, const int32_t* q_mag, const float* q_low, const float* q_delta,
                   const int32_t* k_sign, const int32_t* k_mag, const uint16_t* k_low, const uint16_t* k_delta,
                   const int64_t* head_to_kv, int64_t batch, int64_t qh_count, int64_t kvh_count,
                   int64_t cap, int64_t tokens, int g, uint16_t* out) {
    const int words = 4, reps = 128 / g;
    const float norm = po_inv_sqrt_dim(128);
    int64_t qpk = qh_count / kvh_count;
    for (int64_t b = 0; b < batch; ++b)
    for (int64_t slot = 0; slot < kvh_count; ++slot) {
        int64_t kvh = head_to_kv[slot * qpk];
        for (int64_t t = 0; t < tokens; ++t) {
            const int64_t krow = kvh * cap + t;
            const uint32_t* ks = (const uint32_t*)(k_sign + krow * words);
            const uint32_t* km = (const uint32_t*)(k_mag + krow * words);
            for (int64_t ql_i = 0; ql_i < qpk; ++ql_i) {
                int64_t row = b * qh_count + slot * qpk + ql_i;
                const uint32_t* qs = (const uint32_t*)(q_sign + row * words);
                const uint32_t* qm = (const uint32_t*)(q_mag + row * words);
                float total = 0.0f;
                for (int r = 0; r < reps; ++r) {
                    float ql = q_low[row * reps + r], dq = q_delta[row * reps + r];
                    float kl = po_f16_to_f32(k_low[krow * reps + r]);
                    float dk = po_f16_to_f32(k_delta[krow * reps + r]);
                    if (g == 16) {
                        int w = r / 2;
                        uint32_t mask = (r & 1) ? 0xffff0000u : 0x0000ffffu;
                        total += recon_u32(qs[w], qm[w], ks[w], km[w], mask, ql, dq, kl, dk);
                    } else if (g == 32) {
                        total += recon_u32(qs[r], qm[r], ks[r], km[r], 0xffffffffu, ql, dq, kl, dk);
                    } else {
                        int cs = 0, cq = 0, ck = 0, cqk = 0;
                        for (int half = 0; half < 2; ++half) {
                            int w = 2 * r + half;
                            uint32_t match = ~(qs[w] ^ ks[w]), both = qm[w] & km[w];
                            cs += 2 * popc(match) - 32;
                            cq += 2 * popc(match & qm[w]) - popc(qm[w]);
                            ck += 2 * popc(match & km[w]) - popc(km[w]);
                            cqk += 2 * popc(match & both) - popc(both);
                        }
                        total += fmaf(ql * kl, (float)cs, fmaf(dq * kl, (float)cq,
                                 fmaf(ql * dk, (float)ck, dq * dk * (float)cqk)));
                    }
                }
                out[row * tokens + t] = po_f32_to_f16(total * norm);
            }
        }
    }
}

/* Generic-head-dim scorers, float32 output (popkv_ext.cu:145-230 for G32,
 * :517-675 for G16/G64).  Each query head uses head_to_kv[qh]; partial words
 * are masked; score = total * (1/sqrt(D)). */
void po_score_generic(const int32_t* q_sign, const int32_t* q_mag, const float* q_low, const float* q_delta,
                      const int32_t* k_sign, const int32_t* k_mag, const uint16_t* k_low, const uint16_t* k_delta,
                      const int64_t* head_to_kv, int64_t batch, int64_t qh_count, int64_t d,
                      int64_t cap, int64_t tokens, int g, float* out) {
    int64_t words = (d + 31) / 32, reps = (d + g - 1) / g;
    const float scale = po_inv_sqrt_dim(d);
    for (int64_t row = 0; row < batch * qh_count; ++row) {
        int64_t kvh = head_to_kv[row % qh_count];
        const uint32_t* qs = (const uint32_t*)(q_sign + row * words);
        const uint32_t* qm = (const uint32_t*)(q_mag + row * words);
        for (int64_t t = 0; t < tokens; ++t) {
            int64_t krow = kvh * cap + t;
            const uint32_t* ks = (const uint32_t*)(k_sign + krow * words);
            const uint32_t* km = (const uint32_t*)(k_mag + krow * words);
            float score = 0.0f;
            for (int64_t r = 0; r < reps; ++r) {
                float ql = q_low[row * reps + r], dq = q_delta[row * reps + r];
                float kl = po_f16_to_f32(k_low[krow * reps + r]);
                float dk = po_f16_to_f32(k_delta[krow * reps + r]);
                if (g == 32) {
                    uint32_t mask = 0xffffffffu;
                    if (r == words - 1 && (d & 31)) mask = (1u << (uint32_t)(d & 31)) - 1u;
                    score += recon_u32(qs[r], qm[r], ks[r], km[r], mask, ql, dq, kl, dk);
                    continue;
                }
                int cs = 0, cq = 0, ck = 0, cqk = 0;
                int64_t rs = r * g, re = rs + g < d ? rs + g : d;
                for (int64_t w = rs / 32; w <= (re - 1) / 32; ++w) {
                    int64_t ws = w * 32;
                    int begin = (int)((rs > ws ? rs : ws) - ws);
                    int end = (int)((re < ws + 32 ? re : ws + 32) - ws);
                    int count = end - begin;
                    uint32_t mask = count == 32 ? 0xffffffffu : ((1u << (uint32_t)count) - 1u) << begin;
                    uint32_t qmm = qm[w] & mask, kmm = km[w] & mask;
                    uint32_t match = ~(qs[w] ^ ks[w]) & mask, both = qmm & kmm;
                    cs += 2 * popc(match) - popc(mask);
                    cq += 2 * popc(match & qmm) - popc(qmm);
                    ck += 2 * popc(match & kmm) - popc(kmm);
                    cqk += 2 * popc(match & both) - popc(both);
                }
                score += fmaf(ql * kl, (float)cs, fmaf(dq * kl, (float)cq,
                         fmaf(ql * dk, (float)ck, dq * dk * (float)cqk)));
            }
            out[row * tokens + t] = score * scale;
        }
    }
}

/* ------------------------------------------------------------------ */
/* Top-k select                                                        */
/* ------------------------------------------------------------------ */

/* Radix order key of an fp16 bit pattern, as PyTorch's radix select maps
 * half values: negatives are bit-inverted, non-negatives get the sign bit
 * set, NaN sorts above everything; -0 < +0. */
uint16_t po_order_key_f16(uint16_t h) {
    if ((h & 0x7c00u) == 0x7c00u && (h & 0x3ffu)) return 0xffffu;
    return (h & 0x8000u) ? (uint16_t)(~h & 0xffffu) : (uint16_t)(h | 0x8000u);
}

typedef struct { uint16_t key; int64_t idx; } po_item;

static int cmp_desc_key_asc_idx(const void* a, const void* b) {
    const po_item* x = (const po_item*)a;
    const po_item* y = (const po_item*)b;
    if (x->key != y->key) return x->key > y->key ? -1 : 1;
    return x->idx < y->idx ? -1 : (x->idx > y->idx);
}

static int cmp_i64(const void* a, const void* b) {
    int64_t x = *(const int64_t*)a, y = *(const int64_t*)b;
    return x < y ? -1 : (x > y);
}

/* Per row: the k tokens with the largest fp16 scores, ties at the k-th
 * key resolved toward lower token indices, written in ascending index order,
 * then `current` in slot k (torch.topk(..., sorted=False) followed by
 * _append_current, popkv.py:1094-1098, :287-291).  scores fp16 bits
 * [rows, row_stride]; out [rows, k + 1]. */
void po_select(const uint16_t* scores, int64_t rows, int64_t row_stride, int64_t tokens,
               int64_t k, int64_t current, int64_t* out) {
    po_item* items = (po_item*)malloc(sizeof(po_item) * (size_t)(tokens > 0 ? tokens : 1));
    for (int64_t r = 0; r < rows; ++r) {
        for (int64_t t = 0; t < tokens; ++t) {
            items[t].key = po_order_key_f16(scores[r * row_stride + t]);
            items[t].idx = t;
        }
        qsort(items, (size_t)tokens, sizeof(po_item), cmp_desc_key_asc_idx);
        int64_t* o = out + r * (k + 1);
        for (int64_t i = 0; i < k; ++i) o[i] = items[i].idx;
        qsort(o, (size_t)k, sizeof(int64_t), cmp_i64);
        o[k] = current;
    }
    free(items);
}

/* ------------------------------------------------------------------ */
/* Sparse attention                                                    */
/* ------------------------------------------------------------------ */

/* Materialized softmax attention over gathered rows (float64 accumulation;
 * the tolerance reference of tests/test_sparse_kernels.py:30-48).  Rows whose
 * index equals prefix_tokens use the current key/value (sparse_kernels.py:
 * 267-286).  valid (may be NULL) masks rows out.  q [QH, D]; K/V rows at
 * k + kvh*hs + idx*ts; cur [KVH, D]; idx [QH, S]; out [QH, D]. */
void po_attention(const float* q, const float* k, const float* v, int64_t k_hs, int64_t k_ts,
                  int64_t v_hs, int64_t v_ts, int64_t prefix_tokens, const float* cur_k,
                  const float* cur_v, const int64_t* idx, const uint8_t* valid,
                  const int64_t* head_to_kv, int64_t qh_count, int64_t d, int64_t s, float* out) {
    double scale = (double)po_inv_sqrt_dim(d);
    double* logit = (double*)malloc(sizeof(double) * (size_t)s);
    for (int64_t h = 0; h < qh_count; ++h) {
        int64_t kvh = head_to_kv[h];
        double m = -INFINITY;
        for (int64_t j = 0; j < s; ++j) {
            logit[j] = -INFINITY;
            if (valid && !valid[h * s + j]) continue;
            int64_t t = idx[h * s + j];
            const float* kr = t == prefix_tokens ? cur_k + kvh * d : k + kvh * k_hs + t * k_ts;
            double acc = 0.0;
            for (int64_t i = 0; i < d; ++i) acc += (double)q[h * d + i] * (double)kr[i];
            logit[j] = acc * scale;
            if (logit[j] > m) m = logit[j];
        }
        double l = 0.0;
        for (int64_t i = 0; i < d; ++i) out[h * d + i] = 0.0f;
        double* acc = (double*)calloc((size_t)d, sizeof(double));
        for (int64_t j = 0; j < s; ++j) {
            if (logit[j] == -INFINITY) continue;
            int64_t t = idx[h * s + j];
            const float* vr = t == prefix_tokens ? cur_v + kvh * d : v + kvh * v_hs + t * v_ts;
            double p = exp(logit[j] - m);
            l += p;
            for (int64_t i = 0; i < d; ++i) acc[i] += p * (double)vr[i];
        }
        for (int64_t i = 0; i < d; ++i) out[h * d + i] = (float)(acc[i] / l);
        free(acc);
    }
    free(logit);
}

/* Log-sum-exp merge of split states [QH, S, D+2] = (m, l, acc[D])
 * (sparse_kernels.py:297-318), float64 accumulation. */
void po_attention_merge(const float* partials, int64_t qh_count, int64_t splits, int64_t d, float* out) {
    for (int64_t h = 0; h < qh_count; ++h) {
        const float* p = partials + h * splits * (d + 2);
        double mx = -INFINITY;
        for (int64_t s = 0; s < splits; ++s) if (p[s * (d + 2)] > mx) mx = p[s * (d + 2)];
        double den = 0.0;
        for (int64_t s = 0; s < splits; ++s) {
            double m = p[s * (d + 2)];
            if (m == -INFINITY) continue;
            den += (double)p[s * (d + 2) + 1] * exp(m - mx);
        }
        for (int64_t i = 0; i < d; ++i) {
            double num = 0.0;
            for (int64_t s = 0; s < splits; ++s) {
                double m = p[s * (d + 2)];
                if (m == -INFINITY) continue;
                num += (double)p[s * (d + 2) + 2 + i] * exp(m - mx);
            }
            out[h * d + i] = (float)(num / den);
        }
    }
}
