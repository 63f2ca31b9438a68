// extern "C" entry points of libpopkv_hip.so (declared in include/popkv_hip.h).
//
// Each entry point validates its arguments on the host, records a readable
// message for popkv_last_error() on failure, and launches asynchronously on
// the caller's stream.  Nothing here allocates device memory or synchronizes.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <mutex>

#include "kernels.h"
#include "popkv_hip.h"
#include "select_common.h"

namespace {

thread_local char g_last_error[512] = "";

int fail(int status, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
    va_end(ap);
    return status;
}

int launched(hipError_t err, const char* what) {
    if (err != hipSuccess) return fail(POPKV_ERR_LAUNCH, "%s: %s", what, hipGetErrorString(err));
    return POPKV_OK;
}

bool valid_dtype(int32_t dt) {
    return dt == POPKV_DTYPE_F32 || dt == POPKV_DTYPE_F16 || dt == POPKV_DTYPE_BF16;
}
bool valid_group(int32_t g) { return g == 16 || g == 32 || g == 64; }
size_t elem_size(int32_t dt) { return dt == POPKV_DTYPE_F32 ? 4 : 2; }
bool aligned16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }
int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }
hipStream_t as_stream(void* s) { return static_cast<hipStream_t>(s); }

// Longest row the selects take: 64 chunks of 32 keys per thread x 256
// threads (a chunk's in-chunk offsets and low-byte histogram counts are
// 16-bit, its chunk counts one per lane of a wave); step_chunks raises the
// keys per thread until a row fits in 64 chunks.
constexpr int64_t kMaxSelectTokens = int64_t{64} * popkv::kMaxChunkKeys * popkv::kChunkThreads;
static_assert(kMaxSelectTokens == 524288, "64 chunks of 8192 tokens");
constexpr int64_t kMaxGroupHeads = 64;
constexpr size_t kAlign = 256;

size_t align_up(size_t x) { return (x + kAlign - 1) / kAlign * kAlign; }

// Workspace layout of popkv_layer_step (batch 1, head_dim 128).
struct StepLayout {
    size_t hist, rec, h2, gt1, scores, partials, keep, wrec, wbins, total;
    int64_t score_stride, k, nchunks, tiles, tile_tokens;
    bool windows;  // the tile-window select applies to this shape (for GQA groups of 1, 2, 4 or 8)
};

// Layer-step workspace: [QH][256] u32 high-byte key histograms (zero between
// calls) | [QH][4] u32 threshold records | [QH][chunks][256] u16 chunk
// low-byte histograms | [QH][chunks] u32 chunk counts | [QH][score_stride]
// u16 order keys | [QH][chunks][130] f32 chunk partials, and for the
// tile-window select: [QH][256] u32 kept histograms | [QH][tiles] uint4
// window records | [QH][tiles][kWinBins][64] u32 window byte histograms.  The
// window path applies to 64-dimension groups when 0 < k < tokens, the row
// has at most kWinMaxTiles scorer tiles and a chunk is a whole number of
// them.
StepLayout step_layout(int64_t qh, int64_t tokens, int64_t budget, int32_t g) {
    StepLayout L{};
    L.k = budget - 1 < tokens ? budget - 1 : tokens;
    L.score_stride = ceil_div(tokens > 0 ? tokens : 1, 128) * 128;
    const popkv::StepChunks ch = popkv::step_chunks(tokens, L.k, qh);
    L.nchunks = ch.count;
    L.tile_tokens = popkv::step_tile_tokens(g, qh, tokens);
    L.tiles = ceil_div(tokens > 0 ? tokens : 1, L.tile_tokens);
    L.windows = g == 64 && L.k > 0 && L.k < tokens && L.tiles <= popkv::kWinMaxTiles &&
                popkv::window_kpt_ok(ch.kpt) && ch.tokens_per_chunk % L.tile_tokens == 0;
    const size_t nc = static_cast<size_t>(L.nchunks > 0 ? L.nchunks : 1);
    const size_t nt = L.windows ? static_cast<size_t>(L.tiles) : 0;
    size_t off = 0;
    L.hist = off; off = align_up(off + static_cast<size_t>(qh) * 256 * 4);
    L.rec = off; off = align_up(off + static_cast<size_t>(qh) * 4 * 4);
    L.h2 = off; off = align_up(off + static_cast<size_t>(qh) * nc * 256 * 2);
    L.gt1 = off; off = align_up(off + static_cast<size_t>(qh) * nc * 4);
    L.scores = off; off = align_up(off + static_cast<size_t>(qh * L.score_stride) * 2);
    L.partials = off; off = align_up(off + static_cast<size_t>(qh) * nc * (128 + 2) * 4);
    L.keep = off; off = align_up(off + (L.windows ? static_cast<size_t>(qh) * 256 * 4 : 0));
    L.wrec = off; off = align_up(off + static_cast<size_t>(qh) * nt * 16);
    L.wbins = off; off = align_up(off + static_cast<size_t>(qh) * nt * popkv::kWinBins * 64 * 4);
    L.total = off;
    return L;
}

bool group_fits_windows(int64_t q_heads, int64_t kv_heads) {
    const int64_t qpk = kv_heads > 0 ? q_heads / kv_heads : 0;
    return qpk == 1 || qpk == 2 || qpk == 4 || qpk == 8;
}

// The allocation-free layer step's workspace: one array per GPU, held until
// the process ends.  In host code `scratch` names a host-side stand-in, not
// the device address, so it is never passed to a kernel or a copy; its
// address on each device comes from hipGetSymbolAddress (device_scratch).
static __device__ __align__(256) unsigned char scratch[POPKV_LAYER_STEP_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices] = {};

// The current device's address of `scratch`, looked up once per device
// (with that device current) and kept.
int device_scratch(void** out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return fail(POPKV_ERR_LAUNCH, "hipGetDevice: %s", hipGetErrorString(e));
    if (dev < 0 || dev >= kMaxDevices) return fail(POPKV_ERR_UNSUPPORTED, "device index %d out of range", dev);
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (g_scratch_ptr[dev] == nullptr) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || p == nullptr)
            return fail(POPKV_ERR_LAUNCH, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return POPKV_OK;
}

}  // namespace

extern "C" {

const char* popkv_status_string(int status) {
    switch (status) {
        case POPKV_OK: return "ok";
        case POPKV_ERR_INVALID: return "invalid argument";
        case POPKV_ERR_CAPACITY: return "Pop-KV cache capacity exceeded";
        case POPKV_ERR_TOKENS: return "invalid score token count";
        case POPKV_ERR_UNSUPPORTED: return "unsupported shape";
        case POPKV_ERR_LAUNCH: return "kernel launch failed";
        case POPKV_ERR_WORKSPACE: return "workspace too small";
        default: return "unknown status";
    }
}

const char* popkv_last_error(void) { return g_last_error; }

const char* popkv_version(void) { return "popkv-hip 0.1 gfx950"; }

int popkv_pack(const void* keys, int32_t dtype, int64_t kv_heads, int64_t tokens, int64_t head_dim,
               int64_t key_head_stride, int32_t* k_sign, int32_t* k_mag, void* k_low, void* k_delta,
               int64_t capacity, int64_t token_offset, int32_t token_group_size, int32_t dim_group_size,
               void* stream) {
    if (!keys || !k_sign || !k_mag || !k_low || !k_delta) return fail(POPKV_ERR_INVALID, "null pointer");
    if (!valid_dtype(dtype)) return fail(POPKV_ERR_INVALID, "keys must be fp32/fp16/bf16");
    if (kv_heads <= 0 || kv_heads > 65535 || tokens < 0 || head_dim <= 0)
        return fail(POPKV_ERR_INVALID, "keys must be [KVH, tokens, head dim]");
    if (head_dim > 256) return fail(POPKV_ERR_UNSUPPORTED, "head_dim must be <= 256");
    if (key_head_stride < tokens * head_dim) return fail(POPKV_ERR_INVALID, "key head stride too small");
    if (token_group_size < 1 || token_group_size > 4096)
        return fail(POPKV_ERR_INVALID, "token_group_size must be between 1 and 4096");
    if (!valid_group(dim_group_size)) return fail(POPKV_ERR_INVALID, "dim_group_size must be 16, 32, or 64");
    if (token_offset < 0 || token_offset + tokens > capacity)
        return fail(POPKV_ERR_CAPACITY, "Pop-KV cache capacity exceeded");
    return launched(popkv::launch_pack(keys, dtype, kv_heads, tokens, static_cast<int>(head_dim), key_head_stride,
                                       k_sign, k_mag, static_cast<uint16_t*>(k_low), static_cast<uint16_t*>(k_delta),
                                       capacity, token_offset, token_group_size, dim_group_size, as_stream(stream)),
                    "popkv_pack");
}

int popkv_query_encode(const void* queries, int32_t dtype, int64_t rows, int64_t head_dim, int32_t dim_group_size,
                       int32_t order, int32_t* q_sign, int32_t* q_mag, float* q_low, float* q_delta, void* stream) {
    if (!queries || !q_sign || !q_mag || !q_low || !q_delta) return fail(POPKV_ERR_INVALID, "null pointer");
    if (!valid_dtype(dtype)) return fail(POPKV_ERR_INVALID, "queries must be fp32/fp16/bf16");
    if (rows < 0 || head_dim <= 0) return fail(POPKV_ERR_INVALID, "queries must be [rows, non-empty head dim]");
    if (head_dim > 256) return fail(POPKV_ERR_UNSUPPORTED, "head_dim must be <= 256");
    if (rows > 0x7fffffff) return fail(POPKV_ERR_UNSUPPORTED, "too many query rows");
    if (!valid_group(dim_group_size)) return fail(POPKV_ERR_INVALID, "dim_group_size must be 16, 32, or 64");
    if (order != POPKV_ENCODE_FOLD && order != POPKV_ENCODE_TREE)
        return fail(POPKV_ERR_INVALID, "order must be POPKV_ENCODE_FOLD or POPKV_ENCODE_TREE");
    return launched(popkv::launch_query_encode(queries, dtype, rows, static_cast<int>(head_dim), dim_group_size,
                                               order, q_sign, q_mag, q_low, q_delta, as_stream(stream)),
                    "popkv_query_encode");
}

static int check_score_common(const int64_t* head_to_kv, int64_t batch, int64_t q_heads, int64_t kv_heads,
                              int64_t capacity, int64_t tokens, int32_t g) {
    if (!head_to_kv) return fail(POPKV_ERR_INVALID, "null head mapping");
    if (!valid_group(g)) return fail(POPKV_ERR_INVALID, "dim_group_size must be 16, 32, or 64");
    if (batch <= 0 || q_heads <= 0 || kv_heads <= 0) return fail(POPKV_ERR_INVALID, "empty batch or heads");
    if (tokens <= 0 || tokens > capacity) return fail(POPKV_ERR_TOKENS, "invalid score token count");
    if (q_heads % kv_heads != 0) return fail(POPKV_ERR_INVALID, "GQA query heads must be divisible by KV heads");
    if (q_heads / kv_heads > kMaxGroupHeads) return fail(POPKV_ERR_UNSUPPORTED, "at most 64 query heads per KV head");
    if (batch * q_heads > 65535 || batch * kv_heads > 65535) return fail(POPKV_ERR_UNSUPPORTED, "too many rows");
    return POPKV_OK;
}

int popkv_score_encoded(const int32_t* q_sign, const int32_t* q_mag, const float* q_low, const float* q_delta,
                        const int32_t* k_sign, const int32_t* k_mag, const void* k_low, const void* k_delta,
                        const int64_t* head_to_kv, int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t capacity,
                        int64_t tokens, int32_t dim_group_size, void* scores, void* stream) {
    if (!q_sign || !q_mag || !q_low || !q_delta || !k_sign || !k_mag || !k_low || !k_delta || !scores)
        return fail(POPKV_ERR_INVALID, "null pointer");
    int st = check_score_common(head_to_kv, batch, q_heads, kv_heads, capacity, tokens, dim_group_size);
    if (st) return st;
    if (!aligned16(k_sign) || !aligned16(k_mag) || !aligned16(k_low) || !aligned16(k_delta))
        return fail(POPKV_ERR_INVALID, "packed cache tensors must be 16-byte aligned");
    return launched(popkv::launch_score_d128(q_sign, q_mag, q_low, q_delta, k_sign, k_mag,
                                             static_cast<const uint16_t*>(k_low),
                                             static_cast<const uint16_t*>(k_delta), head_to_kv, batch,
                                             static_cast<int>(q_heads), static_cast<int>(kv_heads), capacity, tokens,
                                             dim_group_size, static_cast<uint16_t*>(scores), tokens, as_stream(stream)),
                    "popkv_score_encoded");
}

size_t popkv_score_workspace_bytes(int64_t batch, int64_t q_heads, int64_t head_dim, int32_t dim_group_size) {
    if (batch <= 0 || q_heads <= 0 || head_dim <= 0 || !valid_group(dim_group_size)) return 0;
    const int64_t rows = batch * q_heads;
    const int64_t w = ceil_div(head_dim, 32), r = ceil_div(head_dim, dim_group_size);
    return align_up(rows * w * 4) * 2 + align_up(rows * r * 4) * 2;
}

int popkv_score(const void* queries, int32_t dtype, int64_t batch, int64_t q_heads, int64_t head_dim,
                const int32_t* k_sign, const int32_t* k_mag, const void* k_low, const void* k_delta,
                const int64_t* head_to_kv, int64_t kv_heads, int64_t capacity, int64_t tokens, int32_t dim_group_size,
                void* scores, void* workspace, size_t workspace_bytes, void* stream) {
    if (!queries || !k_sign || !k_mag || !k_low || !k_delta || !scores) return fail(POPKV_ERR_INVALID, "null pointer");
    if (!valid_dtype(dtype)) return fail(POPKV_ERR_INVALID, "queries must be fp32/fp16/bf16");
    if (head_dim <= 0) return fail(POPKV_ERR_INVALID, "empty head dim");
    if (head_dim > 256) return fail(POPKV_ERR_UNSUPPORTED, "head_dim must be <= 256");
    int st = check_score_common(head_to_kv, batch, q_heads, kv_heads, capacity, tokens, dim_group_size);
    if (st) return st;
    const size_t need = popkv_score_workspace_bytes(batch, q_heads, head_dim, dim_group_size);
    if (!workspace || workspace_bytes < need) return fail(POPKV_ERR_WORKSPACE, "score needs %zu workspace bytes", need);
    const int64_t rows = batch * q_heads;
    const int64_t w = ceil_div(head_dim, 32), r = ceil_div(head_dim, dim_group_size);
    char* ws = static_cast<char*>(workspace);
    int32_t* qs = reinterpret_cast<int32_t*>(ws);
    int32_t* qm = reinterpret_cast<int32_t*>(ws + align_up(rows * w * 4));
    float* ql = reinterpret_cast<float*>(ws + 2 * align_up(rows * w * 4));
    float* qd = reinterpret_cast<float*>(ws + 2 * align_up(rows * w * 4) + align_up(rows * r * 4));
    const bool d128 = head_dim == 128;
    st = launched(popkv::launch_query_encode(queries, dtype, rows, static_cast<int>(head_dim), dim_group_size,
                                             d128 ? POPKV_ENCODE_TREE : POPKV_ENCODE_FOLD, qs, qm, ql, qd,
                                             as_stream(stream)),
                  "popkv_score(encode)");
    if (st) return st;
    if (d128) {
        if (!aligned16(k_sign) || !aligned16(k_mag) || !aligned16(k_low) || !aligned16(k_delta))
            return fail(POPKV_ERR_INVALID, "packed cache tensors must be 16-byte aligned");
        return launched(popkv::launch_score_d128(qs, qm, ql, qd, k_sign, k_mag, static_cast<const uint16_t*>(k_low),
                                                 static_cast<const uint16_t*>(k_delta), head_to_kv, batch,
                                                 static_cast<int>(q_heads), static_cast<int>(kv_heads), capacity,
                                                 tokens, dim_group_size, static_cast<uint16_t*>(scores), tokens,
                                                 as_stream(stream)),
                        "popkv_score");
    }
    return launched(popkv::launch_score_generic(qs, qm, ql, qd, k_sign, k_mag, static_cast<const uint16_t*>(k_low),
                                                static_cast<const uint16_t*>(k_delta), head_to_kv, batch,
                                                static_cast<int>(q_heads), static_cast<int>(kv_heads),
                                                static_cast<int>(head_dim), capacity,
                                                tokens, dim_group_size, static_cast<float*>(scores), as_stream(stream)),
                    "popkv_score");
}

size_t popkv_topk_select_workspace_bytes(int64_t rows, int64_t tokens) {
    if (rows < 0 || tokens < 0) return 0;
    return popkv::topk_select_workspace_bytes(rows, tokens);
}

int popkv_topk_select(const void* scores, int64_t rows, int64_t row_stride, int64_t tokens, int64_t k,
                      int64_t current, void* indices, int32_t index_dtype, int64_t index_row_stride,
                      void* workspace, size_t workspace_bytes, void* stream) {
    if (!scores || !indices || !workspace) return fail(POPKV_ERR_INVALID, "null pointer");
    if (rows < 0 || tokens < 0 || row_stride < tokens) return fail(POPKV_ERR_INVALID, "bad score shape");
    if (k < 0 || k > tokens) return fail(POPKV_ERR_INVALID, "k must satisfy 0 <= k <= tokens");
    if (index_row_stride < k + 1) return fail(POPKV_ERR_INVALID, "index row stride too small");
    if (index_dtype != POPKV_INDEX_I64 && index_dtype != POPKV_INDEX_I32)
        return fail(POPKV_ERR_INVALID, "index dtype must be int64 or int32");
    if (tokens > kMaxSelectTokens) return fail(POPKV_ERR_UNSUPPORTED, "select supports at most 524288 tokens per row");
    if (rows > 0x7fffffff / 32) return fail(POPKV_ERR_UNSUPPORTED, "too many rows");
    if (workspace_bytes < popkv::topk_select_workspace_bytes(rows, tokens))
        return fail(POPKV_ERR_WORKSPACE, "top-k select needs %zu workspace bytes",
                    popkv::topk_select_workspace_bytes(rows, tokens));
    if (reinterpret_cast<uintptr_t>(workspace) % 256) return fail(POPKV_ERR_INVALID, "workspace must be 256-byte aligned");
    return launched(popkv::launch_topk_select(static_cast<const uint16_t*>(scores), rows, row_stride, tokens, k,
                                              current, indices, index_dtype, index_row_stride, workspace,
                                              as_stream(stream)),
                    "popkv_topk_select");
}

static int check_attention_common(int32_t dtype, int64_t q_heads, int64_t head_dim) {
    if (!valid_dtype(dtype)) return fail(POPKV_ERR_INVALID, "attention tensors must be fp32/fp16/bf16");
    if (q_heads <= 0 || q_heads > 65535) return fail(POPKV_ERR_INVALID, "bad query head count");
    if (head_dim <= 0 || head_dim % 8 != 0 || head_dim > 256)
        return fail(POPKV_ERR_UNSUPPORTED, "head_dim must be a multiple of 8 and <= 256");
    return POPKV_OK;
}

int popkv_sparse_attention_partial(const void* queries, int32_t dtype, const void* prefix_k, const void* prefix_v,
                                   int64_t k_head_stride, int64_t k_token_stride, int64_t v_head_stride,
                                   int64_t v_token_stride, int64_t prefix_tokens, const void* current_k,
                                   const void* current_v, const void* indices, int32_t index_dtype,
                                   const uint8_t* valid_mask, const int64_t* head_to_kv, int64_t q_heads,
                                   int64_t kv_heads, int64_t head_dim, int64_t selected, int32_t split_tokens,
                                   float* partials, void* stream) {
    if (!queries || !prefix_k || !prefix_v || !current_k || !current_v || !indices || !head_to_kv || !partials)
        return fail(POPKV_ERR_INVALID, "null pointer");
    int st = check_attention_common(dtype, q_heads, head_dim);
    if (st) return st;
    if (kv_heads <= 0) return fail(POPKV_ERR_INVALID, "bad KV head count");
    if (prefix_tokens <= 0 || selected <= 0)
        return fail(POPKV_ERR_INVALID, "indexed attention requires non-empty prefix and selection");
    if (split_tokens <= 0 || split_tokens % 16) return fail(POPKV_ERR_INVALID, "split_tokens must be a positive multiple of 16");
    if (index_dtype != POPKV_INDEX_I64 && index_dtype != POPKV_INDEX_I32)
        return fail(POPKV_ERR_INVALID, "index dtype must be int64 or int32");
    if (ceil_div(selected, split_tokens) > 65535) return fail(POPKV_ERR_UNSUPPORTED, "too many splits");
    const size_t es = elem_size(dtype);
    if (!aligned16(queries) || !aligned16(prefix_k) || !aligned16(prefix_v) || !aligned16(current_k) ||
        !aligned16(current_v) || (k_head_stride * es) % 16 || (k_token_stride * es) % 16 ||
        (v_head_stride * es) % 16 || (v_token_stride * es) % 16)
        return fail(POPKV_ERR_UNSUPPORTED, "attention tensors need 16-byte aligned rows");
    if (k_token_stride < head_dim || v_token_stride < head_dim) return fail(POPKV_ERR_INVALID, "token stride < head_dim");
    return launched(popkv::launch_attention_partial(queries, dtype, prefix_k, prefix_v, k_head_stride, k_token_stride,
                                                    v_head_stride, v_token_stride, prefix_tokens, current_k, current_v,
                                                    indices, index_dtype, selected, valid_mask, head_to_kv,
                                                    static_cast<int>(q_heads), static_cast<int>(kv_heads),
                                                    static_cast<int>(head_dim), selected,
                                                    split_tokens, partials, as_stream(stream)),
                    "popkv_sparse_attention_partial");
}

int popkv_sparse_attention_merge(const float* partials, int64_t q_heads, int64_t splits, int64_t head_dim,
                                 void* output, int32_t out_dtype, void* stream) {
    if (!partials || !output) return fail(POPKV_ERR_INVALID, "null pointer");
    if (!valid_dtype(out_dtype)) return fail(POPKV_ERR_INVALID, "output must be fp32/fp16/bf16");
    if (q_heads <= 0 || q_heads > 65535 || splits <= 0 || head_dim <= 0)
        return fail(POPKV_ERR_INVALID, "partials must be [QH, splits, D+2]");
    if (splits > 1024) return fail(POPKV_ERR_UNSUPPORTED, "merge supports at most 1024 splits per head");
    if (head_dim > 256) return fail(POPKV_ERR_UNSUPPORTED, "head_dim must be <= 256");
    return launched(popkv::launch_attention_merge(partials, static_cast<int>(q_heads), splits,
                                                  static_cast<int>(head_dim), output, out_dtype, as_stream(stream)),
                    "popkv_sparse_attention_merge");
}

size_t popkv_layer_step_workspace_bytes(int64_t q_heads, int64_t tokens, int64_t budget, int32_t dim_group_size) {
    if (q_heads <= 0 || tokens < 0 || budget <= 1 || !valid_group(dim_group_size)) return 0;
    return step_layout(q_heads, tokens, budget, dim_group_size).total;
}

int popkv_layer_step_launches(int64_t q_heads, int64_t kv_heads, int64_t tokens, int64_t budget,
                              int32_t dim_group_size) {
    if (q_heads <= 0 || kv_heads <= 0 || q_heads % kv_heads || tokens < 0 || tokens > kMaxSelectTokens ||
        budget <= 1 || !valid_group(dim_group_size))
        return 0;
    const StepLayout L = step_layout(q_heads, tokens, budget, dim_group_size);
    if (L.k <= 0 || L.k >= tokens) return 1;
    return L.windows && group_fits_windows(q_heads, kv_heads) ? 1 : 3;
}

}  // extern "C"

// The layer step on a given workspace.  clear_first: the histogram region is
// set to zero by a fill kernel before the scorer adds into it (for a
// workspace whose contents are not known to be zero).
static int layer_step_run(const void* queries, int32_t dtype, const int32_t* k_sign, const int32_t* k_mag,
                          const void* k_low, const void* k_delta, int64_t capacity, const void* prefix_k,
                          const void* prefix_v, int64_t k_head_stride, int64_t v_head_stride, const void* current_k,
                          const void* current_v, const int64_t* head_to_kv, int64_t q_heads, int64_t kv_heads,
                          int64_t tokens, int64_t budget, int32_t dim_group_size, void* output, int64_t* indices_out,
                          void* workspace, size_t workspace_bytes, bool clear_first, void* stream) {
    if (!queries || !k_sign || !k_mag || !k_low || !k_delta || !prefix_k || !prefix_v || !current_k || !current_v ||
        !head_to_kv || !output)
        return fail(POPKV_ERR_INVALID, "null pointer");
    if (!valid_dtype(dtype)) return fail(POPKV_ERR_INVALID, "tensors must be fp32/fp16/bf16");
    if (budget <= 1) return fail(POPKV_ERR_INVALID, "budget must reserve at least one retrieved and one current token");
    int st = check_score_common(head_to_kv, 1, q_heads, kv_heads, capacity, tokens, dim_group_size);
    if (st) return st;
    if (tokens > kMaxSelectTokens) return fail(POPKV_ERR_UNSUPPORTED, "select supports at most 524288 tokens");
    const StepLayout L = step_layout(q_heads, tokens, budget, dim_group_size);
    if (!workspace || workspace_bytes < L.total)
        return fail(POPKV_ERR_WORKSPACE, "layer step needs %zu workspace bytes", L.total);
    if (!aligned16(workspace)) return fail(POPKV_ERR_INVALID, "workspace must be 16-byte aligned");
    const size_t es = elem_size(dtype);
    if (!aligned16(k_sign) || !aligned16(k_mag) || !aligned16(k_low) || !aligned16(k_delta) || !aligned16(queries) ||
        !aligned16(prefix_k) || !aligned16(prefix_v) || !aligned16(current_k) || !aligned16(current_v) ||
        (k_head_stride * es) % 16 || (v_head_stride * es) % 16)
        return fail(POPKV_ERR_UNSUPPORTED, "layer step tensors need 16-byte alignment");
    char* ws = static_cast<char*>(workspace);
    uint32_t* hist = reinterpret_cast<uint32_t*>(ws + L.hist);
    uint32_t* rec = reinterpret_cast<uint32_t*>(ws + L.rec);
    uint16_t* h2 = reinterpret_cast<uint16_t*>(ws + L.h2);
    uint32_t* gt1 = reinterpret_cast<uint32_t*>(ws + L.gt1);
    uint16_t* keys = reinterpret_cast<uint16_t*>(ws + L.scores);
    float* partials = reinterpret_cast<float*>(ws + L.partials);
    const bool windows = L.windows && group_fits_windows(q_heads, kv_heads);
    popkv::TileWindows tw;
    popkv::WindowIn wi;
    if (windows) {
        tw.rec = reinterpret_cast<uint4*>(ws + L.wrec);
        tw.bins = reinterpret_cast<uint32_t*>(ws + L.wbins);
        tw.tiles = static_cast<int>(L.tiles);
        tw.k = static_cast<int>(L.k);
        tw.tile_tokens = static_cast<int>(L.tile_tokens);
        wi.hist = hist;
        wi.keep = reinterpret_cast<uint32_t*>(ws + L.keep);
        wi.rec = tw.rec;
        wi.bins = tw.bins;
        wi.tiles = tw.tiles;
        wi.tile_tokens = static_cast<int>(L.tile_tokens);
    }
    hipStream_t s = as_stream(stream);
    if (clear_first) {
        st = launched(popkv::launch_fill_u32(hist, q_heads * 256, 0u, s), "popkv_layer_step(clear histograms)");
        if (st) return st;
    }
    // The tile-window form runs in one launch: the scorer's workgroups hand
    // their keys, windows and histogram counts to the select + attention
    // blocks of the same grid (launch_layer_step_fused), no kernel boundary
    // between them.
    if (windows) {
        st = launched(popkv::launch_layer_step_fused(
                          queries, dtype, k_sign, k_mag, static_cast<const uint16_t*>(k_low),
                          static_cast<const uint16_t*>(k_delta), capacity, prefix_k, prefix_v, k_head_stride,
                          v_head_stride, keys, L.score_stride, tokens, L.k, tw, wi, hist, head_to_kv,
                          static_cast<int>(q_heads), static_cast<int>(kv_heads), partials, indices_out, L.k + 1,
                          current_k, current_v, output, s),
                      "popkv_layer_step(score + select + attention + merge)");
        return st;  // (a launch that failed ran nothing: the histograms are still zero)
    }

    // 1. query encode + popcount score -> radix order keys of the fp16 scores
    //    (rows padded to a multiple of 128 tokens, so every row starts
    //    256-byte aligned) + per-head high-byte key histograms.  With
    //    k >= tokens every cached token is selected (k <= 0: none), so no
    //    score can change the result: the scorer and the chunk histograms
    //    are skipped and the select + attention kernel takes its
    //    every-token (no-token) path, which reads none of their outputs.
    if (L.k > 0 && L.k < tokens) {
        st = launched(popkv::launch_score_d128_raw(queries, dtype, k_sign, k_mag,
                                                   static_cast<const uint16_t*>(k_low),
                                                   static_cast<const uint16_t*>(k_delta), head_to_kv, 1,
                                                   static_cast<int>(q_heads), static_cast<int>(kv_heads), capacity,
                                                   tokens, dim_group_size, keys, L.score_stride, hist,
                                                   popkv::SeqTable{}, s, tw),
                      "popkv_layer_step(score)");
        if (st) return st;
    }
    // From here on the scorer has added into the histogram region, which
    // must be zero when the next call begins: a failed launch clears it.
    auto clear_hist = [&](int status) {
        (void)popkv::launch_fill_u32(hist, q_heads * 256, 0u, s);
        return status;
    };
    // 2. per-chunk low-byte histograms of the threshold's high-byte bin (the
    //    tile-window path has them from the scorer's windows instead)
    if (!windows) {
        st = launched(popkv::launch_chunk_hist(keys, L.score_stride, q_heads, tokens, L.k, hist, rec, h2, gt1,
                                               popkv::SeqTable{}, s),
                      "popkv_layer_step(chunk histograms)");
        if (st) return clear_hist(st);
    }
    // 3. per (chunk, head): the chunk's selected tokens (also written as
    //    int64 at their rank when indices_out is given) and the sparse
    //    attention over them (re-zeroes the histograms); the head's last
    //    chunk to finish does
    // 4. the log-sum-exp merge of the chunks and the current token (whose
    //    index goes to slot k)
    st = launched(popkv::launch_attention_select_chunks(queries, dtype, prefix_k, prefix_v, k_head_stride,
                                                        v_head_stride, keys, L.score_stride, tokens, L.k, rec, h2,
                                                        gt1, hist, head_to_kv, static_cast<int>(q_heads),
                                                        static_cast<int>(kv_heads), partials, indices_out, L.k + 1,
                                                        popkv::SeqTable{}, current_k, current_v, output, s, nullptr,
                                                        windows ? &wi : nullptr),
                  "popkv_layer_step(select + attention + merge)");
    if (st) return clear_hist(st);
    return POPKV_OK;
}

extern "C" {

int popkv_layer_step(const void* queries, int32_t dtype, const int32_t* k_sign, const int32_t* k_mag,
                     const void* k_low, const void* k_delta, int64_t capacity, const void* prefix_k,
                     const void* prefix_v, int64_t k_head_stride, int64_t v_head_stride, const void* current_k,
                     const void* current_v, const int64_t* head_to_kv, int64_t q_heads, int64_t kv_heads,
                     int64_t tokens, int64_t budget, int32_t dim_group_size, void* output, int64_t* indices_out,
                     void* workspace, size_t workspace_bytes, void* stream) {
    return layer_step_run(queries, dtype, k_sign, k_mag, k_low, k_delta, capacity, prefix_k, prefix_v, k_head_stride,
                          v_head_stride, current_k, current_v, head_to_kv, q_heads, kv_heads, tokens, budget,
                          dim_group_size, output, indices_out, workspace, workspace_bytes, false, stream);
}

size_t popkv_layer_step_scratch_bytes(void) { return POPKV_LAYER_STEP_SCRATCH_BYTES; }

int popkv_layer_step_noalloc(const void* queries, int32_t dtype, const int32_t* k_sign, const int32_t* k_mag,
                             const void* k_low, const void* k_delta, int64_t capacity, const void* prefix_k,
                             const void* prefix_v, int64_t k_head_stride, int64_t v_head_stride,
                             const void* current_k, const void* current_v, const int64_t* head_to_kv,
                             int64_t q_heads, int64_t kv_heads, int64_t tokens, int64_t budget,
                             int32_t dim_group_size, void* output, int64_t* indices_out, void* stream) {
    if (q_heads > 0 && tokens >= 0 && budget > 1 && valid_group(dim_group_size)) {
        const size_t need = step_layout(q_heads, tokens, budget, dim_group_size).total;
        if (need > POPKV_LAYER_STEP_SCRATCH_BYTES)
            return fail(POPKV_ERR_WORKSPACE,
                        "popkv_layer_step_noalloc: this step needs %zu bytes of scratch, more than the "
                        "library's %zu-byte array; call popkv_layer_step with a workspace instead",
                        need, static_cast<size_t>(POPKV_LAYER_STEP_SCRATCH_BYTES));
    }
    void* scratch_ptr = nullptr;
    const int st = device_scratch(&scratch_ptr);
    if (st) return st;
    return layer_step_run(queries, dtype, k_sign, k_mag, k_low, k_delta, capacity, prefix_k, prefix_v, k_head_stride,
                          v_head_stride, current_k, current_v, head_to_kv, q_heads, kv_heads, tokens, budget,
                          dim_group_size, output, indices_out, scratch_ptr, POPKV_LAYER_STEP_SCRATCH_BYTES, true,
                          stream);
}

size_t popkv_layer_step_batched_workspace_bytes(int64_t batch, int64_t q_heads, int64_t max_tokens, int64_t budget,
                                                int32_t dim_group_size) {
    if (batch <= 0 || q_heads <= 0 || max_tokens < 0 || budget <= 1 || !valid_group(dim_group_size)) return 0;
    return step_layout(batch * q_heads, max_tokens, budget, dim_group_size).total;
}

// The current token's append in a decode step (popkv_decode_layer_batched).
struct StepAppend {
    int32_t token_group_size;
    int32_t* status;
};

// popkv_layer_step_batched, and with `app` the decode step: the append runs
// in extra workgroups of the select + attention launch.  Neither that
// kernel nor the chunk-histogram kernel before it reads what the append
// writes: the static caches' rows at the sequences' counts (the select
// reads rows below them; the current K/V come from current_k / current_v)
// and the active groups' packed rows (read by the scorer, which has
// finished).
static int batched_step_run(const void* queries, int32_t dtype, const int32_t* k_sign, const int32_t* k_mag,
                            const void* k_low, const void* k_delta, int64_t capacity, const void* key_cache,
                            const void* value_cache, int64_t cache_rows, const void* current_k,
                            const void* current_v, const int64_t* head_to_kv, int64_t batch, int64_t q_heads,
                            int64_t kv_heads, const int64_t* token_counts, int64_t max_tokens, int64_t budget,
                            int32_t dim_group_size, void* output, int64_t* indices_out, int64_t index_row_stride,
                            void* workspace, size_t workspace_bytes, const StepAppend* app, void* stream) {
    if (!queries || !k_sign || !k_mag || !k_low || !k_delta || !key_cache || !value_cache || !current_k ||
        !current_v || !head_to_kv || !token_counts || !output)
        return fail(POPKV_ERR_INVALID, "null pointer");
    if (!valid_dtype(dtype)) return fail(POPKV_ERR_INVALID, "tensors must be fp32/fp16/bf16");
    if (budget <= 1) return fail(POPKV_ERR_INVALID, "budget must reserve at least one retrieved and one current token");
    if (batch <= 0) return fail(POPKV_ERR_INVALID, "empty batch");
    int st = check_score_common(head_to_kv, batch, q_heads, kv_heads, capacity, max_tokens, dim_group_size);
    if (st) return st;
    if (max_tokens > kMaxSelectTokens) return fail(POPKV_ERR_UNSUPPORTED, "select supports at most 524288 tokens");
    if (max_tokens > cache_rows) return fail(POPKV_ERR_CAPACITY, "max_tokens exceeds the static cache rows");
    const int64_t kmax = budget - 1 < max_tokens ? budget - 1 : max_tokens;
    if (indices_out && index_row_stride < kmax + 1) return fail(POPKV_ERR_INVALID, "index row stride too small");
    const int64_t rows = batch * q_heads;
    const StepLayout L = step_layout(rows, max_tokens, budget, dim_group_size);
    if (!workspace || workspace_bytes < L.total)
        return fail(POPKV_ERR_WORKSPACE, "batched layer step needs %zu workspace bytes", L.total);
    if (!aligned16(workspace)) return fail(POPKV_ERR_INVALID, "workspace must be 16-byte aligned");
    const size_t es = elem_size(dtype);
    if (!aligned16(k_sign) || !aligned16(k_mag) || !aligned16(k_low) || !aligned16(k_delta) || !aligned16(queries) ||
        !aligned16(key_cache) || !aligned16(value_cache) || !aligned16(current_k) || !aligned16(current_v) ||
        (cache_rows * 128 * static_cast<int64_t>(es)) % 16)
        return fail(POPKV_ERR_UNSUPPORTED, "batched layer step tensors need 16-byte alignment");
    if (app && (app->token_group_size < 1 || app->token_group_size > 4096))
        return fail(POPKV_ERR_INVALID, "token_group_size must be between 1 and 4096");
    if (app && batch * kv_heads > 0x7fffffff) return fail(POPKV_ERR_INVALID, "bad batch or KV head count");
    popkv::DecodeAppend dapp{};
    if (app) {
        dapp.new_k = current_k;
        dapp.new_v = current_v;
        dapp.key_cache = const_cast<void*>(key_cache);
        dapp.value_cache = const_cast<void*>(value_cache);
        dapp.cache_rows = cache_rows;
        dapp.status = app->status;
        dapp.k_sign = const_cast<int32_t*>(k_sign);
        dapp.k_mag = const_cast<int32_t*>(k_mag);
        dapp.k_low = static_cast<uint16_t*>(const_cast<void*>(k_low));
        dapp.k_delta = static_cast<uint16_t*>(const_cast<void*>(k_delta));
        dapp.capacity = capacity;
        dapp.token_group_size = app->token_group_size;
        dapp.dim_group_size = dim_group_size;
    }
    popkv::SeqTable seq;
    seq.tokens = token_counts;
    seq.cache_rows = kv_heads * capacity;
    seq.k_bstride = seq.v_bstride = kv_heads * cache_rows * 128;
    seq.q_heads = static_cast<int>(q_heads);
    seq.kv_heads = static_cast<int>(kv_heads);
    seq.budget = static_cast<int>(budget < 0x7fffffff ? budget : 0x7fffffff);
    seq.status = app ? app->status : nullptr;
    char* ws = static_cast<char*>(workspace);
    uint32_t* hist = reinterpret_cast<uint32_t*>(ws + L.hist);
    uint32_t* rec = reinterpret_cast<uint32_t*>(ws + L.rec);
    uint16_t* h2 = reinterpret_cast<uint16_t*>(ws + L.h2);
    uint32_t* gt1 = reinterpret_cast<uint32_t*>(ws + L.gt1);
    uint16_t* keys = reinterpret_cast<uint16_t*>(ws + L.scores);
    float* partials = reinterpret_cast<float*>(ws + L.partials);
    const bool windows = L.windows && group_fits_windows(q_heads, kv_heads);
    popkv::TileWindows tw;
    popkv::WindowIn wi;
    if (windows) {
        tw.rec = reinterpret_cast<uint4*>(ws + L.wrec);
        tw.bins = reinterpret_cast<uint32_t*>(ws + L.wbins);
        tw.tiles = static_cast<int>(L.tiles);
        tw.k = static_cast<int>(L.k);
        tw.tile_tokens = static_cast<int>(L.tile_tokens);
        wi.hist = hist;
        wi.keep = reinterpret_cast<uint32_t*>(ws + L.keep);
        wi.rec = tw.rec;
        wi.bins = tw.bins;
        wi.tiles = tw.tiles;
        wi.tile_tokens = static_cast<int>(L.tile_tokens);
    }
    hipStream_t s = as_stream(stream);
    // popkv_layer_step's kernels as launches of their own (scorer, chunk
    // histograms unless the tile windows apply, select + attention), every
    // row at its own sequence's token count (see popkv::SeqTable).  With budget - 1 >=
    // max_tokens every sequence selects all its cached tokens (its count is
    // at most the bound), so, as in popkv_layer_step, the scorer and the
    // chunk histograms are skipped and every select + attention workgroup
    // takes its every-token (or, for an empty sequence, no-token) path.
    if (L.k < max_tokens) {
        st = launched(popkv::launch_score_d128_raw(queries, dtype, k_sign, k_mag,
                                                   static_cast<const uint16_t*>(k_low),
                                                   static_cast<const uint16_t*>(k_delta), head_to_kv, batch,
                                                   static_cast<int>(q_heads), static_cast<int>(kv_heads), capacity,
                                                   max_tokens, dim_group_size, keys, L.score_stride, hist, seq, s,
                                                   tw),
                      "popkv_layer_step_batched(score)");
        if (st) return st;
    }
    auto clear_hist = [&](int status) {
        (void)popkv::launch_fill_u32(hist, rows * 256, 0u, s);
        return status;
    };
    if (!windows) {
        st = launched(popkv::launch_chunk_hist(keys, L.score_stride, rows, max_tokens, L.k, hist, rec, h2, gt1, seq, s),
                      "popkv_layer_step_batched(chunk histograms)");
        if (st) return clear_hist(st);
    }
    st = launched(popkv::launch_attention_select_chunks(queries, dtype, key_cache, value_cache, cache_rows * 128,
                                                        cache_rows * 128, keys, L.score_stride, max_tokens, L.k, rec,
                                                        h2, gt1, hist, head_to_kv, static_cast<int>(rows),
                                                        static_cast<int>(kv_heads), partials, indices_out,
                                                        index_row_stride, seq, current_k, current_v, output, s,
                                                        app ? &dapp : nullptr, windows ? &wi : nullptr),
                  app ? "popkv_decode_layer_batched(select + attention + merge + append)"
                      : "popkv_layer_step_batched(select + attention + merge)");
    if (st) return clear_hist(st);
    return POPKV_OK;
}

int popkv_layer_step_batched(const void* queries, int32_t dtype, const int32_t* k_sign, const int32_t* k_mag,
                             const void* k_low, const void* k_delta, int64_t capacity, const void* key_cache,
                             const void* value_cache, int64_t cache_rows, const void* current_k,
                             const void* current_v, const int64_t* head_to_kv, int64_t batch, int64_t q_heads,
                             int64_t kv_heads, const int64_t* token_counts, int64_t max_tokens, int64_t budget,
                             int32_t dim_group_size, void* output, int64_t* indices_out, int64_t index_row_stride,
                             void* workspace, size_t workspace_bytes, void* stream) {
    return batched_step_run(queries, dtype, k_sign, k_mag, k_low, k_delta, capacity, key_cache, value_cache,
                            cache_rows, current_k, current_v, head_to_kv, batch, q_heads, kv_heads, token_counts,
                            max_tokens, budget, dim_group_size, output, indices_out, index_row_stride, workspace,
                            workspace_bytes, nullptr, stream);
}

int popkv_decode_layer_batched(const void* queries, int32_t dtype, int32_t* k_sign, int32_t* k_mag, void* k_low,
                               void* k_delta, int64_t capacity, void* key_cache, void* value_cache,
                               int64_t cache_rows, const void* current_k, const void* current_v,
                               const int64_t* head_to_kv, int64_t batch, int64_t q_heads, int64_t kv_heads,
                               const int64_t* token_counts, int64_t max_tokens, int64_t budget,
                               int32_t dim_group_size, int32_t token_group_size, void* output, int64_t* indices_out,
                               int64_t index_row_stride, int32_t* status, void* workspace, size_t workspace_bytes,
                               void* stream) {
    const StepAppend app{token_group_size, status};
    return batched_step_run(queries, dtype, k_sign, k_mag, k_low, k_delta, capacity, key_cache, value_cache,
                            cache_rows, current_k, current_v, head_to_kv, batch, q_heads, kv_heads, token_counts,
                            max_tokens, budget, dim_group_size, output, indices_out, index_row_stride, workspace,
                            workspace_bytes, &app, stream);
}

int popkv_append(const void* new_k, const void* new_v, int32_t dtype, void* key_cache, void* value_cache,
                 int64_t cache_rows, int32_t* k_sign, int32_t* k_mag, void* k_low, void* k_delta, int64_t capacity,
                 const int64_t* token_counts, int64_t batch, int64_t kv_heads, int32_t token_group_size,
                 int32_t dim_group_size, int32_t* status, void* stream) {
    if (!new_k || !new_v || !key_cache || !value_cache || !k_sign || !k_mag || !k_low || !k_delta || !token_counts)
        return fail(POPKV_ERR_INVALID, "null pointer");
    if (!valid_dtype(dtype)) return fail(POPKV_ERR_INVALID, "keys must be fp32/fp16/bf16");
    if (batch <= 0 || kv_heads <= 0 || batch * kv_heads > 0x7fffffff)
        return fail(POPKV_ERR_INVALID, "bad batch or KV head count");
    if (cache_rows <= 0 || capacity <= 0) return fail(POPKV_ERR_CAPACITY, "Pop-KV cache capacity exceeded");
    if (token_group_size < 1 || token_group_size > 4096)
        return fail(POPKV_ERR_INVALID, "token_group_size must be between 1 and 4096");
    if (!valid_group(dim_group_size)) return fail(POPKV_ERR_INVALID, "dim_group_size must be 16, 32, or 64");
    const size_t es = elem_size(dtype);
    if (!aligned16(new_k) || !aligned16(new_v) || !aligned16(key_cache) || !aligned16(value_cache) ||
        !aligned16(k_sign) || !aligned16(k_mag) || !aligned16(k_low) || !aligned16(k_delta) ||
        (cache_rows * 128 * static_cast<int64_t>(es)) % 16)
        return fail(POPKV_ERR_UNSUPPORTED, "append tensors need 16-byte alignment");
    return launched(popkv::launch_append(new_k, new_v, dtype, key_cache, value_cache, cache_rows, token_counts, batch,
                                         static_cast<int>(kv_heads), k_sign, k_mag, static_cast<uint16_t*>(k_low),
                                         static_cast<uint16_t*>(k_delta), capacity, token_group_size, dim_group_size,
                                         status, as_stream(stream)),
                    "popkv_append");
}

int popkv_layer_step_attention(const void* queries, int32_t dtype, const void* prefix_k, const void* prefix_v,
                               int64_t k_head_stride, int64_t v_head_stride, const int64_t* head_to_kv,
                               int64_t q_heads, int64_t kv_heads, int64_t tokens, int64_t budget,
                               int32_t dim_group_size, void* workspace, size_t workspace_bytes, void* stream) {
    if (!queries || !prefix_k || !prefix_v || !head_to_kv || !workspace) return fail(POPKV_ERR_INVALID, "null pointer");
    if (!valid_dtype(dtype)) return fail(POPKV_ERR_INVALID, "tensors must be fp32/fp16/bf16");
    if (budget <= 1) return fail(POPKV_ERR_INVALID, "budget must reserve at least one retrieved and one current token");
    if (q_heads <= 0 || kv_heads <= 0 || q_heads > 65535) return fail(POPKV_ERR_INVALID, "empty or too many heads");
    if (tokens <= 0 || tokens > kMaxSelectTokens) return fail(POPKV_ERR_TOKENS, "invalid score token count");
    if (!valid_group(dim_group_size)) return fail(POPKV_ERR_INVALID, "dim_group_size must be 16, 32, or 64");
    const StepLayout L = step_layout(q_heads, tokens, budget, dim_group_size);
    if (workspace_bytes < L.total) return fail(POPKV_ERR_WORKSPACE, "layer step needs %zu workspace bytes", L.total);
    const size_t es = elem_size(dtype);
    if (!aligned16(workspace) || !aligned16(queries) || !aligned16(prefix_k) || !aligned16(prefix_v) ||
        (k_head_stride * es) % 16 || (v_head_stride * es) % 16)
        return fail(POPKV_ERR_UNSUPPORTED, "layer step tensors need 16-byte alignment");
    char* ws = static_cast<char*>(workspace);
    // the window path reads the histograms the last step kept (its merge
    // zeroed the scorer's); this re-run keeps and zeroes nothing
    const bool windows = L.windows && group_fits_windows(q_heads, kv_heads);
    popkv::WindowIn wi;
    if (windows) {
        wi.hist = reinterpret_cast<const uint32_t*>(ws + L.keep);
        wi.rec = reinterpret_cast<const uint4*>(ws + L.wrec);
        wi.bins = reinterpret_cast<const uint32_t*>(ws + L.wbins);
        wi.tiles = static_cast<int>(L.tiles);
        wi.tile_tokens = static_cast<int>(L.tile_tokens);
    }
    return launched(popkv::launch_attention_select_chunks(
                        queries, dtype, prefix_k, prefix_v, k_head_stride, v_head_stride,
                        reinterpret_cast<const uint16_t*>(ws + L.scores), L.score_stride, tokens, L.k,
                        reinterpret_cast<const uint32_t*>(ws + L.rec), reinterpret_cast<const uint16_t*>(ws + L.h2),
                        reinterpret_cast<const uint32_t*>(ws + L.gt1), reinterpret_cast<uint32_t*>(ws + L.hist),
                        head_to_kv, static_cast<int>(q_heads), static_cast<int>(kv_heads),
                        reinterpret_cast<float*>(ws + L.partials), nullptr, 0, popkv::SeqTable{}, nullptr, nullptr,
                        nullptr, as_stream(stream), nullptr, windows ? &wi : nullptr),
                    "popkv_layer_step_attention");
}

// Dense-attention workspace: [align_up(QH * 4)] u32 merge tickets (zero
// between calls; KVH <= QH of them used) | [QH][splits][130] f32 partials.
size_t dense_tickets_bytes(int64_t q_heads) { return align_up(static_cast<size_t>(q_heads) * 4); }

size_t popkv_dense_attention_workspace_bytes(int64_t q_heads, int64_t tokens) {
    if (q_heads <= 0 || tokens < 0) return 0;
    const int64_t ns = popkv::dense_splits(tokens);
    return dense_tickets_bytes(q_heads) + align_up(static_cast<size_t>(q_heads * (ns > 0 ? ns : 1) * (128 + 2)) * 4);
}

int popkv_dense_attention(const void* queries, int32_t dtype, const void* prefix_k, const void* prefix_v,
                          int64_t k_head_stride, int64_t v_head_stride, const void* current_k, const void* current_v,
                          int64_t q_heads, int64_t kv_heads, int64_t tokens, void* output, void* workspace,
                          size_t workspace_bytes, void* stream) {
    if (!queries || !current_k || !current_v || !output || !workspace || (tokens > 0 && (!prefix_k || !prefix_v)))
        return fail(POPKV_ERR_INVALID, "null pointer");
    if (!valid_dtype(dtype)) return fail(POPKV_ERR_INVALID, "tensors must be fp32/fp16/bf16");
    if (q_heads <= 0 || kv_heads <= 0 || q_heads > 65535 || kv_heads > 65535)
        return fail(POPKV_ERR_INVALID, "empty or too many heads");
    const int64_t group = q_heads / kv_heads;
    if (q_heads % kv_heads != 0 || (group != 1 && group != 2 && group != 4 && group != 8))
        return fail(POPKV_ERR_UNSUPPORTED, "dense attention supports 1, 2, 4 or 8 query heads per KV head");
    if (tokens < 0 || tokens > (int64_t{1} << 31) / 256) return fail(POPKV_ERR_TOKENS, "invalid token count");
    if (workspace_bytes < popkv_dense_attention_workspace_bytes(q_heads, tokens))
        return fail(POPKV_ERR_WORKSPACE, "dense attention needs %zu workspace bytes",
                    popkv_dense_attention_workspace_bytes(q_heads, tokens));
    const size_t es = elem_size(dtype);
    if (!aligned16(workspace) || !aligned16(queries) || (tokens > 0 && (!aligned16(prefix_k) || !aligned16(prefix_v))) ||
        (k_head_stride * es) % 16 || (v_head_stride * es) % 16)
        return fail(POPKV_ERR_UNSUPPORTED, "dense attention tensors need 16-byte alignment");
    hipStream_t s = as_stream(stream);
    uint32_t* tickets = static_cast<uint32_t*>(workspace);
    float* partials = reinterpret_cast<float*>(static_cast<char*>(workspace) + dense_tickets_bytes(q_heads));
    const int ns = popkv::dense_splits(tokens);
    if (ns > 0) {
        // the merge inside the attention launch where it fuses (the group's
        // last block merges), else the merge kernel below
        const bool fused = popkv::dense_merge_fuses(dtype, tokens, static_cast<int>(q_heads), static_cast<int>(kv_heads));
        const popkv::DenseMerge dm{tickets, current_k, current_v, output};
        const int st = launched(popkv::launch_attention_dense(queries, dtype, prefix_k, prefix_v, k_head_stride,
                                                              v_head_stride, tokens, static_cast<int>(q_heads),
                                                              static_cast<int>(kv_heads), partials, s,
                                                              fused ? &dm : nullptr),
                                "popkv_dense_attention(attention)");
        if (st || fused) return st;
    }
    return launched(popkv::launch_merge_current(partials, ns, queries, dtype, current_k, current_v, nullptr,
                                                static_cast<int>(q_heads), static_cast<int>(kv_heads), output,
                                                nullptr, 0, 0, 0, popkv::SeqTable{}, s),
                    "popkv_dense_attention(merge)");
}

}  // extern "C"
