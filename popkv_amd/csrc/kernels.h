// Host-side launchers shared between the kernel translation units and the
// C ABI (capi.hip).  Every launcher validates nothing: the C ABI checks the
// arguments before calling.  All take a hipStream_t and return the launch
// status from hipGetLastError().
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace popkv {

// Per-sequence shape of a batched layer step (B independent sequences of
// different lengths, one launch).  Row h of the step (query head h % q_heads
// of sequence b = h / q_heads) covers min(max(tokens[b], 0), ntok) cached
// tokens, ntok being the launch's token bound, and selects
// min(budget - 1, that) of them.  Packed caches are [B, KVH, capacity, .]
// (cache_rows = KVH * capacity rows per sequence), K/V storage
// [B, KVH, rows, 128] (k_bstride / v_bstride elements per sequence), current
// k/v [B, KVH, 128], queries and outputs [B, QH, 128]; head_to_kv maps a
// sequence's query heads to its KV heads.  tokens == nullptr: a single
// sequence (the unbatched entries), every row at the launch's token count.
struct SeqTable {
    const int64_t* tokens = nullptr;
    int64_t cache_rows = 0;
    int64_t k_bstride = 0, v_bstride = 0;
    int q_heads = 0, kv_heads = 0, budget = 0;
    // When non-null: the merge sets bit 1 (value 2) when a sequence's count
    // lies outside [0, bound] (the step then ran on the clamped count).
    int32_t* status = nullptr;
};

// n 32-bit words of device memory set to `value` (a fill kernel).
hipError_t launch_fill_u32(uint32_t* p, int64_t n, uint32_t value, hipStream_t stream);

hipError_t launch_pack(const void* keys, int dtype, int64_t kv_heads, int64_t tokens, int head_dim,
                       int64_t key_head_stride, int32_t* k_sign, int32_t* k_mag, uint16_t* k_low,
                       uint16_t* k_delta, int64_t capacity, int64_t token_offset, int token_group_size,
                       int dim_group_size, hipStream_t stream);

// Fused per-token append (head_dim 128): for every (sequence b, KV head j)
// of a batch, write new_k / new_v [B*KVH, 128] to row counts[b] of the
// static caches [B*KVH, cache_rows, 128] and re-encode the sequence's active
// token group (rows counts[b] - counts[b] % tg .. counts[b], read in place)
// into the packed planes [B*KVH, capacity, .].  counts: device int64 [B],
// not modified; a count outside [0, min(cache_rows, capacity)) writes
// nothing and sets *status = 1 (status may be null).
hipError_t launch_append(const void* new_k, const void* new_v, int dtype, void* key_cache, void* value_cache,
                         int64_t cache_rows, const int64_t* counts, int64_t batch, int kv_heads, int32_t* k_sign,
                         int32_t* k_mag, uint16_t* k_low, uint16_t* k_delta, int64_t capacity,
                         int token_group_size, int dim_group_size, int32_t* status, hipStream_t stream);

hipError_t launch_query_encode(const void* queries, int dtype, int64_t rows, int head_dim,
                               int dim_group_size, int order, int32_t* q_sign, int32_t* q_mag,
                               float* q_low, float* q_delta, hipStream_t stream);

hipError_t launch_score_d128(const int32_t* q_sign, const int32_t* q_mag, const float* q_low,
                             const float* q_delta, const int32_t* k_sign, const int32_t* k_mag,
                             const uint16_t* k_low, const uint16_t* k_delta, const int64_t* head_to_kv,
                             int64_t batch, int q_heads, int kv_heads, int64_t capacity, int64_t tokens,
                             int dim_group_size, uint16_t* scores, int64_t score_row_stride,
                             hipStream_t stream);

// Tile windows of the layer step (the select's threshold without a
// chunk-histogram pass).  The scorer's workgroup scores one tile of
// step_tile_tokens() tokens of a GQA group's rows; for each (row, tile)
// it estimates the high-byte bin of the row's k-th largest key from the
// tile's own histogram (the bin where the tile's count from the top first
// reaches its share ceil(k * tile tokens / row tokens)), takes the window
// of kWinBins bins starting kWinBelow below that estimate and writes
//   rec:  uint4 {window base bin, keys of the tile above the window,
//                counts of window bins 0|1 and 2|3 as 16-bit pairs}
//   bins: [kWinBins][64] uint32: the low-byte histograms of the window's
//         bins as byte counts, bin 4m + e in byte e of word m (a bin whose
//         tile count exceeds 255 may overflow its bytes: the select takes
//         that bin from the keys instead).
// The select kernel then sums one window row per tile (the row's threshold
// bin) instead of a histogram pass over the keys; a tile whose window misses
// that bin is histogrammed from its keys there.
constexpr int kWinBins = 4;
constexpr int kWinBelow = 2;
// per row: longer rows take launch_chunk_hist (measured: with 64-tile rows
// -- C2's 512-token tiles, C4's 64K sequences -- the select blocks' window
// reads, then one 512-byte row per tile, cost more than the kernel they
// replace)
constexpr int kWinMaxTiles = 32;
inline int score_tile_tokens(int dim_group_size) { return dim_group_size == 64 ? 1024 : 512; }
// The layer step's scorer tile: score_tile_tokens(G), except that rows of
// 64-dimension groups short enough that their 1024-token tiles would give
// at most 512 (tile, query row) pairs -- at GQA 4 fewer than half the
// chip's 256 CUs in scorer workgroups -- take 512-token tiles (one token
// per thread) and twice the workgroups.
inline int step_tile_tokens(int dim_group_size, int64_t rows, int64_t tokens) {
    if (dim_group_size == 64 && (tokens + 1023) / 1024 * rows <= 512) return 512;
    return score_tile_tokens(dim_group_size);
}
struct TileWindows {
    uint4* rec = nullptr;    // [rows][tiles]
    uint32_t* bins = nullptr;  // [rows][tiles][kWinBins][64]
    int tiles = 0;           // tiles per row (the scorer's grid.x)
    int k = 0;               // selected tokens of an unbatched step
    int tile_tokens = 0;     // tokens per tile: 1024 (two per thread) or 512 (one)
};

// Layer-step scorer: encodes the raw query rows [batch*QH, 128] in-kernel
// (fold order), writes the scores' radix order keys (uint16) instead of fp16
// bits, and adds each row's 256-bin high-byte key histogram into
// ghist[row][256] (which must hold zeros on entry).  With win.rec non-null
// (dim_group_size 64, GQA groups of 1, 2, 4 or 8 query heads) it also writes
// the tile windows.
hipError_t launch_score_d128_raw(const void* queries, int dtype, const int32_t* k_sign, const int32_t* k_mag,
                                 const uint16_t* k_low, const uint16_t* k_delta, const int64_t* head_to_kv,
                                 int64_t batch, int q_heads, int kv_heads, int64_t capacity, int64_t tokens,
                                 int dim_group_size, uint16_t* keys, int64_t key_row_stride, uint32_t* ghist,
                                 const SeqTable& seq, hipStream_t stream, const TileWindows& win = TileWindows{});

hipError_t launch_score_generic(const int32_t* q_sign, const int32_t* q_mag, const float* q_low,
                                const float* q_delta, const int32_t* k_sign, const int32_t* k_mag,
                                const uint16_t* k_low, const uint16_t* k_delta, const int64_t* head_to_kv,
                                int64_t batch, int q_heads, int kv_heads, int head_dim, int64_t capacity,
                                int64_t tokens, int dim_group_size, float* scores, hipStream_t stream);

// API-path top-k: fp16 scores [rows, row_stride] -> indices [rows,
// index_row_stride] (int32 or int64), k selected tokens ascending and
// `current` in slot k.  workspace: topk_select_workspace_bytes(rows, tokens)
// bytes, 256-byte aligned, its first rows*1 KiB zero on entry (left zero).
size_t topk_select_workspace_bytes(int64_t rows, int64_t tokens);
hipError_t launch_topk_select(const uint16_t* scores, int64_t rows, int64_t row_stride, int64_t tokens,
                              int64_t k, int64_t current, void* indices, int index_dtype,
                              int64_t index_row_stride, void* workspace, hipStream_t stream);

// Select over radix order keys with the high-byte histograms ghist[row][256]
// already accumulated: writes each row's k selected tokens in ascending
// order to list[row][0..k) (int32; `current` in slot k when list_current)
// and/or idx64[row][0..k) (int64, `current` in slot k); either may be null.
// Re-zeroes ghist.  Key rows are padded to a multiple of 128 keys;
// tokens <= 131072.
hipError_t launch_topk_list(const uint16_t* keys, uint32_t* ghist, int64_t rows, int64_t row_stride, int64_t tokens,
                            int64_t k, int32_t* list, int64_t list_stride, bool list_current, int64_t* idx64,
                            int64_t idx_stride, int64_t current, hipStream_t stream);

hipError_t launch_attention_partial(const void* queries, int dtype, const void* prefix_k, const void* prefix_v,
                                    int64_t k_head_stride, int64_t k_token_stride, int64_t v_head_stride,
                                    int64_t v_token_stride, int64_t prefix_tokens, const void* current_k,
                                    const void* current_v, const void* indices, int index_dtype,
                                    int64_t index_row_stride, const uint8_t* valid_mask,
                                    const int64_t* head_to_kv, int q_heads, int kv_heads, int head_dim,
                                    int64_t selected, int split_tokens, float* partials, hipStream_t stream);

hipError_t launch_attention_merge(const float* partials, int q_heads, int64_t splits, int head_dim,
                                  void* output, int out_dtype, hipStream_t stream);

// Layer-step chunked select + attention (head_dim 128, contiguous rows).
// Key rows hold radix order keys (rows padded to 128 keys, tokens <=
// 131072) and ghist[row][256] their high-byte histograms; the rows are cut
// into step_chunks(tokens, k, rows) chunks.  launch_chunk_hist (for 0 < k <
// tokens only) writes rec[row][4] (threshold bin, count above it),
// h2[row][chunk][256] (uint16 low-byte histograms of the threshold bin) and
// gt1[row][chunk] (counts above the bin).  launch_attention_select_chunks
// then selects, per (chunk, head), the chunk's tokens among the row's k
// largest keys (lowest index first among ties), attends over them into
// partials[head][chunk][130], writes them as int64 to idx_out[head][rank]
// when idx_out is non-null, and re-zeroes ghist.  With output non-null the
// merge is fused: the last workgroup of each head merges its chunks with
// the current token (current_k / current_v) into output (and writes the
// current token's index), so no merge launch follows.
hipError_t launch_chunk_hist(const uint16_t* keys, int64_t key_stride, int64_t rows, int64_t tokens, int64_t k,
                             const uint32_t* ghist, uint32_t* rec, uint16_t* h2, uint32_t* gt1, const SeqTable& seq,
                             hipStream_t stream);
// The current token's append run inside a batched step's select + attention
// launch (popkv_decode_layer_batched): the operands of popkv_append.
struct DecodeAppend {
    const void* new_k;
    const void* new_v;
    void* key_cache;
    void* value_cache;
    int64_t cache_rows;
    int32_t* status;
    int32_t* k_sign;
    int32_t* k_mag;
    uint16_t* k_low;
    uint16_t* k_delta;
    int64_t capacity;
    int token_group_size;
    int dim_group_size;
};
// The select's inputs on the window path (no chunk histograms): the rows'
// high-byte histograms (`hist`: the scorer's ghist in a layer step, the
// kept copy when the kernel is re-run alone), the tile windows, and `keep`
// (non-null: the fused merge copies each row's histogram there before
// zeroing ghist).  Taken for chunks of a whole number of tiles
// (window_kpt_ok), at most kWinMaxTiles tiles per row.
struct WindowIn {
    const uint32_t* hist = nullptr;
    uint32_t* keep = nullptr;
    const uint4* rec = nullptr;
    const uint32_t* bins = nullptr;
    int tiles = 0;
    int tile_tokens = 0;
};
inline bool window_kpt_ok(int kpt) { return kpt == 4 || kpt == 8 || kpt == 16; }

hipError_t launch_attention_select_chunks(const void* queries, int dtype, const void* prefix_k, const void* prefix_v,
                                          int64_t k_head_stride, int64_t v_head_stride, const uint16_t* keys,
                                          int64_t key_stride, int64_t tokens, int64_t k, const uint32_t* rec,
                                          const uint16_t* h2, const uint32_t* gt1, uint32_t* ghist,
                                          const int64_t* head_to_kv, int q_heads, int kv_heads, float* partials,
                                          int64_t* idx_out, int64_t idx_stride, const SeqTable& seq,
                                          const void* current_k, const void* current_v, void* output,
                                          hipStream_t stream, const DecodeAppend* append = nullptr,
                                          const WindowIn* win = nullptr);
// The layer step's tile-window form in one launch (G64 scorer with the tile
// windows, then the select + attention blocks with the fused merge; 0 < k <
// tokens, at most kWinMaxTiles tiles of 1024 or 512 tokens (step_tile_tokens), window_kpt_ok chunks of
// whole tiles, GQA groups of 1, 2, 4 or 8): the operands of
// launch_score_d128_raw and launch_attention_select_chunks together.  ghist
// must hold zeros on entry and does again on exit.
hipError_t launch_layer_step_fused(const void* queries, int dtype, const int32_t* k_sign, const int32_t* k_mag,
                                   const uint16_t* k_low, const uint16_t* k_delta, int64_t capacity,
                                   const void* prefix_k, const void* prefix_v, int64_t k_head_stride,
                                   int64_t v_head_stride, uint16_t* keys, int64_t key_stride, int64_t tokens,
                                   int64_t k, const TileWindows& tw, const WindowIn& win, uint32_t* ghist,
                                   const int64_t* head_to_kv, int q_heads, int kv_heads, float* partials,
                                   int64_t* idx_out, int64_t idx_stride, const void* current_k,
                                   const void* current_v, void* output, hipStream_t stream);
// Dense attention over every prefix token (head_dim 128, contiguous rows):
// partials[h][s][130] for dense_splits(tokens) splits of 512 tokens.
// Query head h reads KV head h / (QH / KVH) (group sizes 1, 2, 4, 8); one
// workgroup serves a whole group.
int dense_splits(int64_t tokens);
// The dense layer's merge fused into its attention launch: tickets[KVH]
// (zero on entry, left zero), the current token and the output.  Taken when
// dense_merge_fuses(): fp16 / bf16, GQA groups of 4 (the MFMA kernel), at
// most 64 splits; otherwise launch_merge_current follows the launch.
struct DenseMerge {
    uint32_t* tickets;
    const void* current_k;
    const void* current_v;
    void* output;
};
bool dense_merge_fuses(int dtype, int64_t tokens, int q_heads, int kv_heads);
hipError_t launch_attention_dense(const void* queries, int dtype, const void* prefix_k, const void* prefix_v,
                                  int64_t k_head_stride, int64_t v_head_stride, int64_t tokens, int q_heads,
                                  int kv_heads, float* partials, hipStream_t stream,
                                  const DenseMerge* merge = nullptr);

// Layer-step merge of the split partials plus the current token (head_dim
// 128); with idx_out non-null, also writes `current` to idx_out[h][idx_slot].
hipError_t launch_merge_current(const float* partials, int nsplit, const void* queries, int dtype,
                                const void* current_k, const void* current_v, const int64_t* head_to_kv, int q_heads,
                                int kv_heads, void* output, int64_t* idx_out, int64_t idx_stride, int64_t idx_slot,
                                int64_t current, const SeqTable& seq, hipStream_t stream);

}  // namespace popkv
