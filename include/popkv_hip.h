/*
 * popkv_hip.h -- C ABI of the MI355X (gfx950) PopKV decode-time retrieval path.
 *
 * Plain C: device pointers, sizes and a stream handle (a hipStream_t passed as
 * void*, NULL = the default stream).  No entry point allocates device memory
 * or synchronizes with the host; every launch is asynchronous on `stream`.
 * Callers that need scratch memory pass a workspace sized by the matching
 * *_workspace_bytes() query.
 *
 * Every entry point returns POPKV_OK (0) or a negative status; the detail of
 * the last failure on the calling thread is available from popkv_last_error().
 *
 * Layouts (row-major, element counts):
 *   keys       [KVH, tokens, D]; rows of one head are contiguous (token stride
 *              D), heads are key_head_stride elements apart.
 *   k_sign/mag int32 [KVH, capacity, W], W = ceil(D/32); dim 32w+j is bit j.
 *   k_low/delta fp16 bit patterns [KVH, capacity, R], R = ceil(D/G).
 *   q_sign/mag int32 [B*QH, W];  q_low/delta float32 [B*QH, R].
 *   scores     fp16 [B, QH, tokens] (D == 128) or float32 (other D).
 *   indices    [QH, S] int64 or int32; an index equal to prefix_tokens names
 *              the current (not yet cached) token.
 *   partials   float32 [QH, ceil(S/split), D+2] = (m, l, acc[D]).
 */
#ifndef POPKV_HIP_H
#define POPKV_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ------------------------------------------------------ */
#define POPKV_OK                0
#define POPKV_ERR_INVALID      -1  /* bad argument: shape, dtype, group size, null pointer */
#define POPKV_ERR_CAPACITY     -2  /* "Pop-KV cache capacity exceeded" */
#define POPKV_ERR_TOKENS       -3  /* "invalid score token count" */
#define POPKV_ERR_UNSUPPORTED  -4  /* valid, but outside what the kernels implement */
#define POPKV_ERR_LAUNCH       -5  /* the HIP runtime rejected a launch */
#define POPKV_ERR_WORKSPACE    -6  /* workspace pointer null or too small */

/* ---- element types ----------------------------------------------------- */
#define POPKV_DTYPE_F32   0
#define POPKV_DTYPE_F16   1
#define POPKV_DTYPE_BF16  2
#define POPKV_INDEX_I64   0
#define POPKV_INDEX_I32   1

/* ---- query-encode summation order -------------------------------------- */
#define POPKV_ENCODE_FOLD 0  /* left fold over ascending dims: decode path */
#define POPKV_ENCODE_TREE 1  /* reduction-tree order: score() path, D == 128 */

const char* popkv_status_string(int status);
const char* popkv_last_error(void);
const char* popkv_version(void);

/* Key prepack and in-place append.  Encodes tokens [0, tokens) of `keys`
 * into rows [token_offset, token_offset + tokens) of the packed cache, token
 * groups of token_group_size (1..4096) counted from the first key, dimension
 * groups of dim_group_size (16, 32, 64).  D <= 256.
 * Replaces popkv_pack_cuda / popkv_pack_into_cuda / popkv_pack_dim_cuda /
 * popkv_pack_into_dim_cuda (reference csrc/popkv_ext.cu:1058-1206, bound at
 * csrc/popkv_ext.cpp:44-45, :48-49) and their kernels (popkv_ext.cu:79-143,
 * :283-500). */
int popkv_pack(const void* keys, int32_t dtype, int64_t kv_heads, int64_t tokens,
               int64_t head_dim, int64_t key_head_stride,
               int32_t* k_sign, int32_t* k_mag, void* k_low, void* k_delta,
               int64_t capacity, int64_t token_offset,
               int32_t token_group_size, int32_t dim_group_size, void* stream);

/* Query encode: rows = B*QH rows of D values.  order POPKV_ENCODE_FOLD
 * replaces popkv_query_encode_out_cuda (popkv_ext.cu:1315-1358, kernels
 * :232-281, :911-957, bound at popkv_ext.cpp:47); POPKV_ENCODE_TREE is the
 * warp encode the reference runs inside score() (popkv_ext.cu:677-755). */
int popkv_query_encode(const void* queries, int32_t dtype, int64_t rows, int64_t head_dim,
                       int32_t dim_group_size, int32_t order,
                       int32_t* q_sign, int32_t* q_mag, float* q_low, float* q_delta,
                       void* stream);

/* Popcount scorer on a pre-encoded query, head_dim 128 only (W = 4).
 * Query head qh of KV group j reads KV head head_to_kv[j * QH/KVH]; output is
 * fp16 [B, QH, tokens], 0 < tokens <= capacity.
 * Replaces popkv_score_encoded_cuda (popkv_ext.cu:1533-1593, kernel :757-876,
 * bound at popkv_ext.cpp:51). */
int popkv_score_encoded(const int32_t* q_sign, const int32_t* q_mag,
                        const float* q_low, const float* q_delta,
                        const int32_t* k_sign, const int32_t* k_mag,
                        const void* k_low, const void* k_delta,
                        const int64_t* head_to_kv, int64_t batch, int64_t q_heads,
                        int64_t kv_heads, int64_t capacity, int64_t tokens,
                        int32_t dim_group_size, void* scores, void* stream);

/* Score from raw queries [B, QH, D]: D == 128 encodes in tree order and runs
 * the GQA scorer (fp16 out); other D encode in fold order and run the generic
 * per-head scorer (float32 out).  Needs popkv_score_workspace_bytes() bytes.
 * Replaces popkv_score_cuda / popkv_score_dim_cuda (popkv_ext.cu:1208-1313,
 * bound at popkv_ext.cpp:46, :50). */
size_t popkv_score_workspace_bytes(int64_t batch, int64_t q_heads, int64_t head_dim,
                                   int32_t dim_group_size);
int popkv_score(const void* queries, int32_t dtype, int64_t batch, int64_t q_heads,
                int64_t head_dim, const int32_t* k_sign, const int32_t* k_mag,
                const void* k_low, const void* k_delta, const int64_t* head_to_kv,
                int64_t kv_heads, int64_t capacity, int64_t tokens, int32_t dim_group_size,
                void* scores, void* workspace, size_t workspace_bytes, void* stream);

/* Per-row top-k over fp16 scores: the k largest (PyTorch's fp16 radix order,
 * -0 < +0, NaN largest), ties at the k-th value taken in ascending token
 * order, written in ascending token order to indices[r, 0..k), and `current`
 * written to indices[r, k].  0 <= k <= tokens.  tokens <= 524288 per row.
 * Needs popkv_topk_select_workspace_bytes(rows, tokens) bytes of 256-byte
 * aligned workspace whose first rows * 1024 bytes (the per-row histograms)
 * are zero when the call begins; every call leaves them zero again, so the
 * workspace can be reused by later calls with the same row count (after a
 * call with fewer rows, clear the larger histogram region first).  Calls
 * sharing one workspace must be stream-ordered.
 * Replaces torch.topk(scores, k, dim=-1, sorted=False).indices followed by
 * _append_current (reference popkv.py:1094-1098, :287-291). */
size_t popkv_topk_select_workspace_bytes(int64_t rows, int64_t tokens);
int popkv_topk_select(const void* scores, int64_t rows, int64_t row_stride, int64_t tokens,
                      int64_t k, int64_t current, void* indices, int32_t index_dtype,
                      int64_t index_row_stride, void* workspace, size_t workspace_bytes,
                      void* stream);

/* Split sparse attention, partial pass: for query head h and split s, the
 * online-softmax state of rows indices[h, s*split .. s*split+split) of
 * prefix K/V head head_to_kv[h] (the current k/v where the index equals
 * prefix_tokens; rows with valid_mask == 0 skipped).  D % 8 == 0, D <= 256,
 * split_tokens a positive multiple of 16.  A head_to_kv entry outside
 * [0, kv_heads) is clamped into range, and a row index outside
 * [0, prefix_tokens] is clamped to the nearest cached row (the reference
 * clamps with min(token, prefix_tokens - 1)), so no input can read out of
 * bounds.
 * Replaces indexed_attention_split_partial (reference sparse_kernels.py:
 * 321-364, Triton kernel :237-294). */
int popkv_sparse_attention_partial(const void* queries, int32_t dtype,
                                   const void* prefix_k, const void* prefix_v,
                                   int64_t k_head_stride, int64_t k_token_stride,
                                   int64_t v_head_stride, int64_t v_token_stride,
                                   int64_t prefix_tokens,
                                   const void* current_k, const void* current_v,
                                   const void* indices, int32_t index_dtype,
                                   const uint8_t* valid_mask, const int64_t* head_to_kv,
                                   int64_t q_heads, int64_t kv_heads, int64_t head_dim, int64_t selected,
                                   int32_t split_tokens, float* partials, void* stream);

/* Log-sum-exp merge of split states into output [QH, D] of out_dtype
 * (at most 1024 splits per head).
 * Replaces indexed_attention_split_merge (sparse_kernels.py:367-387,
 * Triton kernel :297-318). */
int popkv_sparse_attention_merge(const float* partials, int64_t q_heads, int64_t splits,
                                 int64_t head_dim, void* output, int32_t out_dtype,
                                 void* stream);

/* One decode step of one sparse layer (batch 1, head_dim 128): query encode,
 * popcount score over `tokens` cached tokens, per-head top-k with
 * k = min(budget-1, tokens) plus the current token (index `tokens`), and
 * split sparse attention with the log-sum-exp merge (the splits are token
 * chunks of the cache, each attending over its selected tokens).
 * queries/prefix/current K/V share `dtype`; output [QH, 128] has `dtype`.
 * indices_out (int64 [QH, k+1]) may be NULL; when given, the selection is
 * also written there.  Needs popkv_layer_step_workspace_bytes() bytes of
 * 16-byte aligned workspace whose first q_heads * 1024 bytes (the per-head
 * key histograms) are zero when the call begins; every call leaves them zero
 * again, so the workspace can be reused by later calls with the same head
 * count (after a call with fewer heads, clear the larger histogram region
 * first).  Calls sharing one workspace must be stream-ordered.
 * Replaces the PopKV branch of LlamaSparseDecoder.decode (reference
 * popkv.py:1076-1115): query_encode, score_encoded, torch.topk +
 * _append_current, indexed_attention_split_partial and _merge. */
size_t popkv_layer_step_workspace_bytes(int64_t q_heads, int64_t tokens, int64_t budget,
                                        int32_t dim_group_size);
/* The kernel launches popkv_layer_step makes for a shape: 1 when the layer
 * fits the tile-window form (64-dimension groups, at most 32 scorer tiles of
 * 1024 tokens, GQA groups of 1, 2, 4 or 8: scorer, select, attention and
 * merge in one launch) or the budget covers every cached token (select +
 * attention only), 3 otherwise (scorer, chunk histograms, select +
 * attention); 0 for an invalid shape.  No counterpart in the reference: a
 * query for profilers and benchmarks. */
int popkv_layer_step_launches(int64_t q_heads, int64_t kv_heads, int64_t tokens, int64_t budget,
                              int32_t dim_group_size);
int popkv_layer_step(const void* queries, int32_t dtype,
                     const int32_t* k_sign, const int32_t* k_mag,
                     const void* k_low, const void* k_delta, int64_t capacity,
                     const void* prefix_k, const void* prefix_v,
                     int64_t k_head_stride, int64_t v_head_stride,
                     const void* current_k, const void* current_v,
                     const int64_t* head_to_kv, int64_t q_heads, int64_t kv_heads,
                     int64_t tokens, int64_t budget, int32_t dim_group_size,
                     void* output, int64_t* indices_out,
                     void* workspace, size_t workspace_bytes, void* stream);

/* Batched decode step of one sparse layer over B independent sequences of
 * different lengths, head_dim 128, in one call (popkv_layer_step's scorer
 * and select + attention as launches of their own -- with the chunk
 * histograms between them where popkv_layer_step takes three launches --
 * every row at its own sequence's shape; with budget - 1 >= max_tokens
 * every sequence selects all its cached tokens and only the select +
 * attention kernel runs).  Layouts, all
 * contiguous:
 *   queries, output        [B, QH, 128]       (dtype)
 *   k_sign/k_mag           [B, KVH, capacity, 4]    int32
 *   k_low/k_delta          [B, KVH, capacity, 128/G] fp16
 *   key_cache/value_cache  [B, KVH, cache_rows, 128] (dtype; the static
 *                          K/V caches, read in place)
 *   current_k/current_v    [B, KVH, 128]      (dtype)
 *   head_to_kv             [QH] int64: one sequence's GQA mapping
 *   token_counts           [B] int64 IN DEVICE MEMORY: sequence b has
 *                          token_counts[b] cached tokens (rows 0 .. count-1
 *                          of its caches); the current token is index count.
 * max_tokens (host) bounds every count (1 <= max_tokens <= capacity,
 * cache_rows, 524288) and sizes the launch; a count above it is treated as
 * max_tokens.  Sequence b selects k_b = min(budget - 1, count_b) tokens;
 * indices_out (optional) [B, QH, index_row_stride] int64 receives them in
 * ascending order with the current token at slot k_b (entries past k_b are
 * left untouched).  Workspace: popkv_layer_step_batched_workspace_bytes()
 * bytes, 16-byte aligned, first B*QH*1024 bytes zero on entry (left zero),
 * as for popkv_layer_step.  Because the counts are read on the device, one
 * HIP graph of a decode step stays valid while the sequences grow.
 * Replaces the PopKV branch of LlamaSparseDecoder.decode (reference
 * popkv.py:1076-1115) for a batch: the reference's packed caches have no
 * batch dimension (popkv_ext.cu:769-806; popkv.py:763-1129 decodes one
 * sequence). */
size_t popkv_layer_step_batched_workspace_bytes(int64_t batch, int64_t q_heads, int64_t max_tokens,
                                                int64_t budget, int32_t dim_group_size);
int popkv_layer_step_batched(const void* queries, int32_t dtype,
                             const int32_t* k_sign, const int32_t* k_mag,
                             const void* k_low, const void* k_delta, int64_t capacity,
                             const void* key_cache, const void* value_cache, int64_t cache_rows,
                             const void* current_k, const void* current_v,
                             const int64_t* head_to_kv, int64_t batch, int64_t q_heads, int64_t kv_heads,
                             const int64_t* token_counts, int64_t max_tokens, int64_t budget,
                             int32_t dim_group_size, void* output, int64_t* indices_out,
                             int64_t index_row_stride, void* workspace, size_t workspace_bytes,
                             void* stream);

/* Fused per-token append, head_dim 128, one call per layer for a batch of
 * B sequences (B = 1 for a single one): writes the new token's K/V rows
 * new_k/new_v [B, KVH, 128] to row token_counts[b] of the static caches
 * key_cache/value_cache [B, KVH, cache_rows, 128], and re-encodes each
 * sequence's active token group -- rows s .. token_counts[b], s =
 * token_counts[b] rounded down to a multiple of token_group_size, the older
 * ones read in place from key_cache -- into the packed planes
 * [B, KVH, capacity, .] (a group seals when it reaches token_group_size
 * tokens: the next append starts a new one).  token_counts (device int64
 * [B]) is read, not advanced: the caller adds 1 after every layer of the
 * step has appended.  A count outside [0, min(cache_rows, capacity))
 * writes nothing for that sequence and sets *status = 1 (device int32,
 * may be NULL) -- the reference's "Pop-KV cache reserve exhausted".
 * Replaces append_popkv / append_retrieval_caches (reference popkv.py:
 * 438-459, :883-942: torch.cat staging of the active keys, then
 * pack_keys_into, popkv_cuda.py:72-87, popkv_ext.cu:1075-1092) together
 * with the static cache row write of popkv.py:964-972. */
int popkv_append(const void* new_k, const void* new_v, int32_t dtype,
                 void* key_cache, void* value_cache, int64_t cache_rows,
                 int32_t* k_sign, int32_t* k_mag, void* k_low, void* k_delta, int64_t capacity,
                 const int64_t* token_counts, int64_t batch, int64_t kv_heads,
                 int32_t token_group_size, int32_t dim_group_size, int32_t* status, void* stream);

/* One layer of a batched decode step: popkv_layer_step_batched followed by
 * popkv_append of the current token (new_k/new_v = current_k/current_v,
 * token_group_size, status as for popkv_append), with the same results as
 * the two calls in that order, with one launch fewer than the two: the
 * append runs in extra workgroups of the select + attention launch, beside
 * the selection and the attention (neither reads what the append writes:
 * the static caches' rows at the counts, the active groups' packed rows).
 * A sequence whose device count lies outside [0, max_tokens] is stepped
 * at the clamped count and sets *status |= 2 (status may be NULL): a
 * captured step replayed past the bound it was captured with reports it
 * there, so poll status after replays.
 * No counterpart in the reference: it replaces, for one layer, the
 * reference decode loop's retrieval step and append (popkv.py:1076-1115
 * with :438-459 / :883-942 and the static cache write of :964-972) for a
 * batch. */
int popkv_decode_layer_batched(const void* queries, int32_t dtype,
                               int32_t* k_sign, int32_t* k_mag, void* k_low, void* k_delta,
                               int64_t capacity, void* key_cache, void* value_cache, int64_t cache_rows,
                               const void* current_k, const void* current_v,
                               const int64_t* head_to_kv, int64_t batch, int64_t q_heads, int64_t kv_heads,
                               const int64_t* token_counts, int64_t max_tokens, int64_t budget,
                               int32_t dim_group_size, int32_t token_group_size, void* output,
                               int64_t* indices_out, int64_t index_row_stride, int32_t* status,
                               void* workspace, size_t workspace_bytes, void* stream);

/* Allocation-free form of popkv_layer_step: the same kernels and results,
 * with the workspace taken from a library-owned device array of
 * POPKV_LAYER_STEP_SCRATCH_BYTES per GPU (a file-scope __device__ array,
 * held until the process ends) instead of a caller argument.  It calls no
 * hipMalloc/hipFree and no allocating library routine; the caller passes
 * inputs and outputs only.  Each call first clears the array's histogram
 * region with a fill kernel (no hipMemsetAsync, so it records into HIP
 * graphs).  A step whose workspace (popkv_layer_step_workspace_bytes) would
 * exceed the array fails with POPKV_ERR_WORKSPACE.  Every call on one GPU
 * shares that GPU's array: calls that overlap on one GPU (different streams
 * without ordering, or several host threads) race and must be serialized
 * by the caller.  No counterpart in the reference: for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid allocation). */
#define POPKV_LAYER_STEP_SCRATCH_BYTES (16u << 20)
size_t popkv_layer_step_scratch_bytes(void);
int popkv_layer_step_noalloc(const void* queries, int32_t dtype,
                             const int32_t* k_sign, const int32_t* k_mag,
                             const void* k_low, const void* k_delta, int64_t capacity,
                             const void* prefix_k, const void* prefix_v,
                             int64_t k_head_stride, int64_t v_head_stride,
                             const void* current_k, const void* current_v,
                             const int64_t* head_to_kv, int64_t q_heads, int64_t kv_heads,
                             int64_t tokens, int64_t budget, int32_t dim_group_size,
                             void* output, int64_t* indices_out, void* stream);

/* Re-runs only the fused select + sparse-attention kernel of the last
 * popkv_layer_step that used `workspace` (same shapes, budget and
 * dim_group_size): it reads the order keys and threshold data the step left
 * there (the kept key histograms and tile windows, or the chunk
 * histograms) and rewrites the chunk partials, leaving the scorer's
 * histogram region zero, so it can be repeated.  For timing the step's
 * select + attention half as a launch of its own (where the step is one
 * launch, the same code without the hand-off); no counterpart in the
 * reference. */
int popkv_layer_step_attention(const void* queries, int32_t dtype,
                               const void* prefix_k, const void* prefix_v,
                               int64_t k_head_stride, int64_t v_head_stride,
                               const int64_t* head_to_kv, int64_t q_heads, int64_t kv_heads,
                               int64_t tokens, int64_t budget, int32_t dim_group_size,
                               void* workspace, size_t workspace_bytes, void* stream);

/* Dense attention of one decode step over every prefix token plus the
 * current one: out[h] = softmax(q_h . [K_prefix; k_cur] / sqrt(128)) .
 * [V_prefix; v_cur] with the plain GQA grouping (query head h reads KV head
 * h / (QH / KVH); 1, 2, 4 or 8 query heads per KV head), written in `dtype`
 * to output [QH, 128].  prefix K/V [KVH, tokens, 128], rows contiguous, any
 * head stride; tokens may be 0.  Needs
 * popkv_dense_attention_workspace_bytes() bytes of 16-byte aligned
 * workspace whose first q_heads * 4 bytes, rounded up to 256 (the merge
 * tickets), are zero when the call begins; every call leaves them zero
 * (after a call with fewer query heads, clear the larger region first).
 * fp16/bf16 groups of 4 query heads over at most 32768 tokens run in one
 * launch (each KV group's last workgroup merges), others in two.
 * Replaces the full-layer branch of
 * LlamaSparseDecoder.decode (reference popkv.py:1022-1038: torch.cat of the
 * prefix and current K/V, then scaled_dot_product_attention on the grouped
 * view q.view(KVH, QH/KVH, 1, D)). */
size_t popkv_dense_attention_workspace_bytes(int64_t q_heads, int64_t tokens);
int popkv_dense_attention(const void* queries, int32_t dtype,
                          const void* prefix_k, const void* prefix_v,
                          int64_t k_head_stride, int64_t v_head_stride,
                          const void* current_k, const void* current_v,
                          int64_t q_heads, int64_t kv_heads, int64_t tokens, void* output,
                          void* workspace, size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* POPKV_HIP_H */
