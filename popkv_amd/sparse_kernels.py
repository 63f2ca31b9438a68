"""Split sparse attention on MI355X: the drop-in for the reference's
``sparse_kernels`` split-attention entry points (sparse_kernels.py:321-401).

Same signatures, shapes and exceptions.  The partial pass writes the
reference's state layout, float32 [QH, ceil(S/split), D+2] = (m, l, acc[D]),
so either half can be swapped independently.  Kernels: hand-written gfx950
HIP (``attention.hip``) through the C ABI; no Triton.

Implementation limits (raise RuntimeError): head_dim a multiple of 8 and at
most 256; queries, current K/V and the prefix K/V share one dtype; rows of
the prefix K/V 16-byte aligned (true for any contiguous cache of such D).
"""
from __future__ import annotations

import math

import torch

from . import _native as nat

_INDEX_CODES = {torch.int64: nat.INDEX_I64, torch.int32: nat.INDEX_I32}


def _unit_last_stride(t: torch.Tensor) -> torch.Tensor:
    return t if t.stride(-1) == 1 else t.contiguous()


def indexed_attention_split_partial(
    queries: torch.Tensor, prefix_keys: torch.Tensor, prefix_values: torch.Tensor,
    current_keys: torch.Tensor, current_values: torch.Tensor, indices: torch.Tensor,
    head_to_kv: torch.Tensor, valid_mask: torch.Tensor | None = None, *,
    split_tokens: int = 256,
) -> torch.Tensor:
    """Online-softmax partial states per (query head, split of selected tokens).

    prefix_keys/values: [KVH, T, D], any head stride, row stride >= D (the
    strided views of a static cache work as they are).  An index equal to T
    is the current token.  Returns float32 [QH, ceil(S/split_tokens), D+2].
    """
    if queries.ndim != 2 or prefix_keys.ndim != 3 or prefix_values.shape != prefix_keys.shape:
        raise ValueError("invalid indexed-attention tensor ranks or K/V shapes")
    if indices.ndim != 2 or int(indices.shape[0]) != int(queries.shape[0]):
        raise ValueError("indices must be [query heads, selected tokens]")
    if valid_mask is not None and valid_mask.shape != indices.shape:
        raise ValueError("valid mask must match indices")
    if split_tokens <= 0 or split_tokens % 16:
        raise ValueError("split_tokens must be a positive multiple of 16")
    if not queries.is_cuda or any(x.device != queries.device for x in (
        prefix_keys, prefix_values, current_keys, current_values, indices, head_to_kv
    )):
        raise RuntimeError("indexed-attention tensors must share a CUDA device")
    q_heads, head_dim = (int(x) for x in queries.shape)
    prefix_tokens = int(prefix_keys.shape[1])
    selected_tokens = int(indices.shape[1])
    if prefix_tokens <= 0 or selected_tokens <= 0:
        raise ValueError("indexed attention requires non-empty prefix and selection")
    dtype = prefix_keys.dtype
    if any(t.dtype != dtype for t in (prefix_values, queries, current_keys, current_values)):
        raise RuntimeError("queries, current K/V and prefix K/V must share a dtype")
    kv_heads = int(prefix_keys.shape[0])
    num_splits = math.ceil(selected_tokens / split_tokens)
    partials = torch.empty((q_heads, num_splits, head_dim + 2), device=queries.device, dtype=torch.float32)
    pk, pv = _unit_last_stride(prefix_keys), _unit_last_stride(prefix_values)
    q = queries.contiguous()
    ck, cv = current_keys.contiguous(), current_values.contiguous()
    idx = indices if indices.dtype in _INDEX_CODES else indices.long()
    idx = idx.contiguous()
    vm = None if valid_mask is None else valid_mask.contiguous().to(torch.bool).view(torch.uint8)
    mapping = head_to_kv.to(device=queries.device, dtype=torch.int64).contiguous()
    with torch.cuda.device(queries.device):
        nat.call("popkv_sparse_attention_partial", q.data_ptr(), nat.dtype_code(q), pk.data_ptr(), pv.data_ptr(),
                 pk.stride(0), pk.stride(1), pv.stride(0), pv.stride(1), prefix_tokens, ck.data_ptr(), cv.data_ptr(),
                 idx.data_ptr(), _INDEX_CODES[idx.dtype], nat.ptr(vm), mapping.data_ptr(), q_heads, kv_heads,
                 head_dim, selected_tokens, int(split_tokens), partials.data_ptr(), nat.stream_of(queries.device))
    return partials


def indexed_attention_split_merge(
    partials: torch.Tensor, output_like: torch.Tensor,
) -> torch.Tensor:
    """Merge split online-softmax states into one output per query head
    (sparse_kernels.py:367-387); the output has output_like's dtype."""
    if partials.ndim != 3 or partials.dtype != torch.float32 or not partials.is_cuda:
        raise ValueError("partials must be CUDA float32 [query heads, splits, D+2]")
    if output_like.ndim != 2 or output_like.device != partials.device:
        raise ValueError("output_like must be [query heads, head dim] on the partial device")
    q_heads, num_splits, state_d = (int(x) for x in partials.shape)
    head_dim = int(output_like.shape[1])
    if int(output_like.shape[0]) != q_heads or state_d != head_dim + 2:
        raise ValueError("partial/output shape mismatch")
    output = torch.empty(output_like.shape, device=output_like.device, dtype=output_like.dtype)
    p = partials.contiguous()
    with torch.cuda.device(output.device):
        nat.call("popkv_sparse_attention_merge", p.data_ptr(), q_heads, num_splits, head_dim, output.data_ptr(),
                 nat.dtype_code(output), nat.stream_of(output.device))
    return output


def indexed_attention_split(
    queries: torch.Tensor, prefix_keys: torch.Tensor, prefix_values: torch.Tensor,
    current_keys: torch.Tensor, current_values: torch.Tensor, indices: torch.Tensor,
    head_to_kv: torch.Tensor, valid_mask: torch.Tensor | None = None, *,
    split_tokens: int = 256,
) -> torch.Tensor:
    """Split-token indexed attention with online-softmax merging (sparse_kernels.py:390-401)."""
    partials = indexed_attention_split_partial(
        queries, prefix_keys, prefix_values, current_keys, current_values,
        indices, head_to_kv, valid_mask, split_tokens=split_tokens,
    )
    return indexed_attention_split_merge(partials, queries)
