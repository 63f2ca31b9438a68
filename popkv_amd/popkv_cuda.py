"""PopKV kernel API on MI355X: the drop-in for the reference's ``popkv_cuda``.

Same names, keyword-only arguments, dtypes, shapes and exception types as the
reference's PopKV entry points (popkv_cuda.py:27-87, :141-204): Python-side
argument validation raises ValueError; the checks the reference makes in its
native extension (TORCH_CHECK) raise RuntimeError with the same messages.
Every function launches hand-written gfx950 HIP kernels through the C ABI of
``libpopkv_hip.so`` on the tensors' current stream, asynchronously.
"""
from __future__ import annotations

import math

import torch

from . import _native as nat

MAX_TOKEN_GROUP_SIZE = 4096
SPECIALIZED_TOKEN_GROUP_SIZES = (8, 16, 32, 64, 128)
SUPPORTED_DIM_KERNELS = ("g16", "g32", "g64-u32", "g64-u64")


def _validate_token_group_size(token_group_size: int) -> int:
    """popkv_cuda.py:28-32."""
    value = int(token_group_size)
    if not 1 <= value <= MAX_TOKEN_GROUP_SIZE:
        raise ValueError(f"token_group_size must be between 1 and {MAX_TOKEN_GROUP_SIZE}")
    return value


def _validate_dim_group_size(dim_group_size: int) -> int:
    """popkv_cuda.py:35-39."""
    value = int(dim_group_size)
    if value not in (16, 32, 64):
        raise ValueError("dim_group_size must be one of 16, 32, 64")
    return value


def _validate_dim_kernel(dim_group_size: int, dim_kernel: str | None) -> str:
    """popkv_cuda.py:42-50.  The g64-u32 / g64-u64 choice only names the
    reference's popcount width; both compute the same integers, so one HIP
    scorer serves both."""
    default = {16: "g16", 32: "g32", 64: "g64-u32"}[dim_group_size]
    value = default if dim_kernel is None or dim_kernel == "auto" else str(dim_kernel)
    if value not in SUPPORTED_DIM_KERNELS:
        raise ValueError(f"dim_kernel must be one of {SUPPORTED_DIM_KERNELS}")
    expected = 64 if value.startswith("g64-") else int(value[1:])
    if expected != dim_group_size:
        raise ValueError(f"dim_kernel={value} requires dim_group_size={expected}")
    return value


def _check(cond: bool, message: str) -> None:
    if not cond:
        raise RuntimeError(message)


def _check_floatish(t: torch.Tensor, name: str) -> None:
    _check(t.dtype in (torch.float32, torch.float16, torch.bfloat16), f"{name} must be fp32/fp16/bf16")


def _rep_groups(head_dim: int, dim_group_size: int) -> int:
    return math.ceil(head_dim / dim_group_size)


def _check_packed(packed, device: torch.device, kv_heads: int, words: int, reps: int) -> None:
    """The packed-cache checks of popkv_ext.cu:1080-1087, :1182-1202."""
    k_sign, k_mag, k_low, k_delta = packed
    for t in packed:
        _check(t.is_cuda, "packed tensors must be CUDA tensors")
        _check(t.is_contiguous(), "packed tensors must be contiguous")
    _check(k_sign.dtype == torch.int32 and k_mag.dtype == torch.int32, "k_sign/k_mag must be int32")
    _check(k_low.dtype == torch.float16 and k_delta.dtype == torch.float16,
           "Pop-KV representative metadata must be float16")
    _check(k_sign.ndim == 3 and k_sign.shape[0] == kv_heads and k_sign.shape[2] == words
           and k_mag.shape == k_sign.shape, "packed bitplane shape mismatch")
    _check(k_low.ndim == 3 and k_low.shape[0] == kv_heads and k_low.shape[1] == k_sign.shape[1]
           and k_low.shape[2] == reps and k_delta.shape == k_low.shape,
           "representative metadata shape mismatch")
    _check(all(t.device == device for t in packed), "Pop-KV packing tensors must share a CUDA device")


def _launch_pack(keys: torch.Tensor, packed, token_offset: int, token_group_size: int,
                 dim_group_size: int) -> None:
    k_sign, k_mag, k_low, k_delta = packed
    kv_heads, tokens, head_dim = (int(x) for x in keys.shape)
    with torch.cuda.device(keys.device):
        nat.call("popkv_pack", keys.data_ptr(), nat.dtype_code(keys), kv_heads, tokens, head_dim,
                 tokens * head_dim, k_sign.data_ptr(), k_mag.data_ptr(), k_low.data_ptr(), k_delta.data_ptr(),
                 int(k_sign.shape[1]), int(token_offset), token_group_size, dim_group_size,
                 nat.stream_of(keys.device))


def pack_keys(
    keys: torch.Tensor, *, token_capacity: int | None = None,
    token_group_size: int = 32, dim_group_size: int = 32,
):
    """Pack fixed uint32 K bitplanes plus G_dim low/delta representatives.

    keys [KV heads, tokens, head dim] contiguous fp32/fp16/bf16 ->
    (k_sign int32 [KVH, cap, W], k_mag int32, k_low fp16 [KVH, cap, R],
    k_delta fp16); rows >= tokens are left uninitialised (popkv_cuda.py:53-69,
    popkv_ext.cu:1058-1073, :1153-1175).
    """
    if keys.ndim != 3 or not keys.is_cuda or not keys.is_contiguous():
        raise ValueError("keys must be contiguous CUDA [KV heads, tokens, head dim]")
    capacity = int(keys.shape[1]) if token_capacity is None else int(token_capacity)
    token_group_size = _validate_token_group_size(token_group_size)
    dim_group_size = _validate_dim_group_size(dim_group_size)
    if dim_group_size != 32 and token_group_size not in SPECIALIZED_TOKEN_GROUP_SIZES:
        raise ValueError("non-specialized token group sizes require dim_group_size=32")
    _check_floatish(keys, "keys")
    kv_heads, tokens, head_dim = (int(x) for x in keys.shape)
    if dim_group_size != 32:
        _check(tokens > 0 and head_dim > 0, "keys must be [KVH, non-empty tokens, non-empty head dim]")
    _check(capacity >= tokens, "token capacity is too small")
    words = math.ceil(head_dim / 32)
    reps = words if dim_group_size == 32 else _rep_groups(head_dim, dim_group_size)
    dev = keys.device
    k_sign = torch.empty((kv_heads, capacity, words), device=dev, dtype=torch.int32)
    k_mag = torch.empty_like(k_sign)
    k_low = torch.empty((kv_heads, capacity, reps), device=dev, dtype=torch.float16)
    k_delta = torch.empty_like(k_low)
    packed = (k_sign, k_mag, k_low, k_delta)
    if tokens > 0:
        _launch_pack(keys, packed, 0, token_group_size, dim_group_size)
    return packed


def pack_keys_into(
    keys: torch.Tensor, packed, *, token_offset: int,
    token_group_size: int = 32, dim_group_size: int = 32,
) -> None:
    """Re-encode `keys` into rows [token_offset, token_offset + tokens) of an
    existing packed cache, in place (popkv_cuda.py:72-87, popkv_ext.cu:1075-1092,
    :1177-1206)."""
    if keys.ndim != 3 or not keys.is_cuda or not keys.is_contiguous():
        raise ValueError("keys must be contiguous CUDA [KV heads, tokens, head dim]")
    token_group_size = _validate_token_group_size(token_group_size)
    dim_group_size = _validate_dim_group_size(dim_group_size)
    if dim_group_size != 32 and token_group_size not in SPECIALIZED_TOKEN_GROUP_SIZES:
        raise ValueError("non-specialized token group sizes require dim_group_size=32")
    packed = tuple(packed)
    _check_floatish(keys, "keys")
    kv_heads, tokens, head_dim = (int(x) for x in keys.shape)
    words = math.ceil(head_dim / 32)
    reps = words if dim_group_size == 32 else _rep_groups(head_dim, dim_group_size)
    _check(len(packed) == 4, "packed must contain k_sign, k_mag, k_low, k_delta")
    _check_packed(packed, keys.device, kv_heads, words, reps)
    token_offset = int(token_offset)
    _check(token_offset >= 0 and token_offset + tokens <= int(packed[0].shape[1]), "Pop-KV cache capacity exceeded")
    if tokens > 0:
        _launch_pack(keys, packed, token_offset, token_group_size, dim_group_size)


def allocate_query_encode_outputs(queries: torch.Tensor, *, dim_group_size: int = 32):
    """Allocate the query-state tuple of the fused scorer (popkv_cuda.py:141-154)."""
    if queries.ndim != 3 or not queries.is_cuda or not queries.is_contiguous():
        raise ValueError("queries must be contiguous CUDA [batch, query heads, head dim]")
    words = (int(queries.shape[2]) + 31) // 32
    dim_group_size = _validate_dim_group_size(dim_group_size)
    groups = (int(queries.shape[2]) + dim_group_size - 1) // dim_group_size
    bit_shape = (int(queries.shape[0]), int(queries.shape[1]), words)
    rep_shape = (int(queries.shape[0]), int(queries.shape[1]), groups)
    sign = torch.empty(bit_shape, device=queries.device, dtype=torch.int32)
    magnitude = torch.empty_like(sign)
    low = torch.empty(rep_shape, device=queries.device, dtype=torch.float32)
    delta = torch.empty_like(low)
    return sign, magnitude, low, delta


def query_encode(queries: torch.Tensor, *, out=None, dim_group_size: int = 32):
    """Encode a PopKV query into bitplanes and dimension-group representatives
    (decode-path order; popkv_cuda.py:157-167, popkv_ext.cu:1315-1358)."""
    if queries.ndim != 3 or not queries.is_cuda or not queries.is_contiguous():
        raise ValueError("queries must be contiguous CUDA [batch, query heads, head dim]")
    dim_group_size = _validate_dim_group_size(dim_group_size)
    outputs = (allocate_query_encode_outputs(queries, dim_group_size=dim_group_size)
               if out is None else tuple(out))
    if len(outputs) != 4:
        raise ValueError("out must contain q_sign, q_mag, q_low, q_delta")
    _check_floatish(queries, "queries")
    q_sign, q_mag, q_low, q_delta = outputs
    for t in outputs:
        _check(t.is_cuda, "query encoding outputs must be CUDA tensors")
        _check(t.is_contiguous(), "query encoding outputs must be contiguous")
    _check(q_sign.dtype == torch.int32 and q_mag.dtype == torch.int32, "q_sign/q_mag must be int32")
    _check(q_low.dtype == torch.float32 and q_delta.dtype == torch.float32, "query low/delta outputs must be float32")
    _check(int(queries.shape[2]) > 0, "queries must be [batch, query heads, non-empty head dim]")
    batch, q_heads, head_dim = (int(x) for x in queries.shape)
    bit_expected = (batch, q_heads, (head_dim + 31) // 32)
    rep_expected = (batch, q_heads, _rep_groups(head_dim, dim_group_size))
    _check(tuple(q_sign.shape) == bit_expected and tuple(q_mag.shape) == bit_expected
           and tuple(q_low.shape) == rep_expected and tuple(q_delta.shape) == rep_expected,
           "query encoding outputs have incorrect shape")
    _check(all(t.device == queries.device for t in outputs), "query encoding tensors must share a CUDA device")
    with torch.cuda.device(queries.device):
        nat.call("popkv_query_encode", queries.data_ptr(), nat.dtype_code(queries), batch * q_heads, head_dim,
                 dim_group_size, nat.ENCODE_FOLD, q_sign.data_ptr(), q_mag.data_ptr(), q_low.data_ptr(),
                 q_delta.data_ptr(), nat.stream_of(queries.device))
    return outputs


def score_encoded(
    encoded_query, packed, *, head_to_kv: torch.Tensor, tokens: int,
    dim_group_size: int = 32, dim_kernel: str | None = None,
) -> torch.Tensor:
    """Score compressed keys from a pre-encoded head-dim-128 PopKV query ->
    fp16 [B, QH, tokens] (popkv_cuda.py:170-187, popkv_ext.cu:1533-1593)."""
    dim_group_size = _validate_dim_group_size(dim_group_size)
    _validate_dim_kernel(dim_group_size, dim_kernel)
    encoded_query = tuple(encoded_query)
    packed = tuple(packed)
    if len(encoded_query) != 4:
        raise ValueError("encoded_query must contain q_sign, q_mag, q_low, q_delta")
    if len(packed) != 4:
        raise ValueError("packed must contain k_sign, k_mag, k_low, k_delta")
    if any(not tensor.is_cuda or not tensor.is_contiguous() for tensor in encoded_query):
        raise ValueError("encoded query tensors must be contiguous CUDA tensors")
    head_to_kv = head_to_kv.contiguous()
    q_sign, q_mag, q_low, q_delta = encoded_query
    k_sign, k_mag, k_low, k_delta = packed
    for t in (*packed, head_to_kv):
        _check(t.is_cuda, "score tensors must be CUDA tensors")
        _check(t.is_contiguous(), "score tensors must be contiguous")
    _check(all(t.dtype == torch.int32 for t in (q_sign, q_mag, k_sign, k_mag)), "bitplanes must be int32")
    _check(q_low.dtype == torch.float32 and q_delta.dtype == torch.float32,
           "encoded Pop-KV query representatives must be float32")
    _check(k_low.dtype == torch.float16 and k_delta.dtype == torch.float16,
           "Pop-KV key representatives must be float16")
    _check(head_to_kv.dtype == torch.int64, "head mapping must be int64")
    _check(q_sign.ndim == 3 and q_sign.shape[2] == 4 and q_mag.shape == q_sign.shape,
           "encoded Pop-KV query bitplanes must be [batch, query heads, 4]")
    batch, q_heads = int(q_sign.shape[0]), int(q_sign.shape[1])
    reps, kv_heads = 128 // dim_group_size, int(k_sign.shape[0])
    _check(q_low.shape == q_delta.shape and q_low.ndim == 3 and tuple(q_low.shape) == (batch, q_heads, reps),
           "encoded Pop-KV query representative shape mismatch")
    _check(k_sign.ndim == 3 and k_sign.shape[2] == 4 and k_mag.shape == k_sign.shape,
           "Pop-KV key bitplanes must be [KV heads, capacity, 4]")
    _check(k_low.shape == k_delta.shape and k_low.ndim == 3 and k_low.shape[0] == kv_heads
           and k_low.shape[1] == k_sign.shape[1] and k_low.shape[2] == reps,
           "Pop-KV key representative shape mismatch")
    tokens = int(tokens)
    _check(0 < tokens <= int(k_sign.shape[1]), "invalid score token count")
    _check(head_to_kv.numel() == q_heads and q_heads % kv_heads == 0, "invalid GQA head mapping")
    dev = k_sign.device
    _check(all(t.device == dev for t in (*encoded_query, *packed, head_to_kv)),
           "encoded score tensors must share a CUDA device")
    scores = torch.empty((batch, q_heads, tokens), device=dev, dtype=torch.float16)
    with torch.cuda.device(dev):
        nat.call("popkv_score_encoded", q_sign.data_ptr(), q_mag.data_ptr(), q_low.data_ptr(), q_delta.data_ptr(),
                 k_sign.data_ptr(), k_mag.data_ptr(), k_low.data_ptr(), k_delta.data_ptr(), head_to_kv.data_ptr(),
                 batch, q_heads, kv_heads, int(k_sign.shape[1]), tokens, dim_group_size, scores.data_ptr(),
                 nat.stream_of(dev))
    return scores


def score(
    queries: torch.Tensor, packed, *, head_to_kv: torch.Tensor, tokens: int,
    dim_group_size: int = 32, dim_kernel: str | None = None,
) -> torch.Tensor:
    """Approximate QK scores; the head-dim-128 path emits fp16, others fp32
    (popkv_cuda.py:190-204, popkv_ext.cu:1208-1313)."""
    if queries.ndim != 3 or not queries.is_cuda or not queries.is_contiguous():
        raise ValueError("queries must be contiguous CUDA [batch, query heads, head dim]")
    dim_group_size = _validate_dim_group_size(dim_group_size)
    _validate_dim_kernel(dim_group_size, dim_kernel)
    packed = tuple(packed)
    head_to_kv = head_to_kv.contiguous()
    _check_floatish(queries, "queries")
    k_sign, k_mag, k_low, k_delta = packed
    for t in (*packed, head_to_kv):
        _check(t.is_cuda, "score tensors must be CUDA tensors")
    _check(k_sign.dtype == torch.int32 and k_mag.dtype == torch.int32, "k_sign/k_mag must be int32")
    _check(k_low.dtype == torch.float16 and k_delta.dtype == torch.float16,
           "Pop-KV representative metadata must be float16")
    _check(head_to_kv.dtype == torch.int64, "head mapping must be int64")
    batch, q_heads, head_dim = (int(x) for x in queries.shape)
    capacity, kv_heads = int(k_sign.shape[1]), int(k_sign.shape[0])
    words = (head_dim + 31) // 32
    reps = words if dim_group_size == 32 else _rep_groups(head_dim, dim_group_size)
    tokens = int(tokens)
    _check(0 < tokens <= capacity, "invalid score token count")
    _check_packed(packed, queries.device, kv_heads, words, reps)
    _check(head_to_kv.numel() == q_heads, "head mapping size mismatch")
    _check(q_heads % kv_heads == 0, "GQA query heads must be divisible by KV heads")
    dev = queries.device
    out_dtype = torch.float16 if (head_dim == 128 and words == 4) else torch.float32
    scores = torch.empty((batch, q_heads, tokens), device=dev, dtype=out_dtype)
    ws_bytes = int(nat.lib().popkv_score_workspace_bytes(batch, q_heads, head_dim, dim_group_size))
    workspace = torch.empty(ws_bytes, device=dev, dtype=torch.uint8)
    with torch.cuda.device(dev):
        nat.call("popkv_score", queries.data_ptr(), nat.dtype_code(queries), batch, q_heads, head_dim,
                 k_sign.data_ptr(), k_mag.data_ptr(), k_low.data_ptr(), k_delta.data_ptr(), head_to_kv.data_ptr(),
                 kv_heads, capacity, tokens, dim_group_size, scores.data_ptr(), workspace.data_ptr(), ws_bytes,
                 nat.stream_of(dev))
    return scores
