"""PopKV retrieval-cache management and the per-layer decode retrieval step.

The PopKV part of the reference's ``popkv.py``, with the same names and
semantics: presets and ``RetrievalConfig`` (popkv.py:18-64), ``PopKVCache``
with prefix prepack and per-token append (popkv.py:89-96, :414-459), the
batched append phases of ``append_retrieval_caches`` (popkv.py:883-942), the
static K/V cache append (popkv.py:105-111, :964-972), ``_append_current`` /
``_sparse_layer_indices`` (popkv.py:283-291), and the PopKV branch of
``LlamaSparseDecoder.decode`` (popkv.py:1076-1115) as ``popkv_retrieval_step``.

``popkv_layer_step`` is the same step as one C-ABI call: encode + score
with per-head key histograms and tile windows, the per-chunk select +
sparse attention, and the log-sum-exp merge with the current token in each
head's last workgroup.  Where the tile-window form applies (64-dimension
groups, at most 32 scorer tiles, GQA groups of 1, 2, 4 or 8) that is one
kernel launch; otherwise three (the scorer, per-chunk histograms of the
threshold bin, the select + attention); with k >= tokens only the select +
attention.
"""
from __future__ import annotations


import math
from dataclasses import dataclass
from typing import Callable, Sequence

import torch

from . import _native as nat
from .popkv_cuda import pack_keys, pack_keys_into, query_encode, score_encoded
from .sparse_kernels import indexed_attention_split_merge, indexed_attention_split_partial
from .topk import select_with_current, topk_indices

METHODS = ("full", "quest", "fier", "popkv-normal", "popkv-q", "popkv-s")
POPKV_METHODS = ("popkv-normal", "popkv-q", "popkv-s")

POPKV_PRESETS = {
    "popkv-normal": (32, 32),
    "popkv-q": (128, 16),
    "popkv-s": (64, 64),
}
TOKEN_GROUP_SIZE = 32
SPECIALIZED_TOKEN_GROUP_SIZES = (8, 16, 32, 64, 128)
MAX_TOKEN_GROUP_SIZE = 4096
SUPPORTED_TOKEN_GROUP_SIZES = SPECIALIZED_TOKEN_GROUP_SIZES
PACKING_WORD_BITS = 32
SUPPORTED_DIM_GROUP_SIZES = (16, 32, 64)
SUPPORTED_DIM_KERNELS = ("auto", "g16", "g32", "g64-u32", "g64-u64")
SPLIT_TOKENS = 256


@dataclass(frozen=True)
class RetrievalConfig:
    """popkv.py:34-64 (the QUEST/FIER fields are kept so configs round-trip)."""
    budget: int = 4096
    group_size: int = 32  # token-axis magnitude-threshold group (B_token)
    dim_group_size: int = 32  # dimensions sharing low/delta representatives (G_dim)
    dim_kernel: str = "auto"
    quest_page_size: int = 16
    fier_kernel: str = "fier"
    full_layers: tuple[int, ...] = (0, 1)

    def validate(self) -> None:
        if self.budget <= 1:
            raise ValueError("budget must reserve at least one retrieved and one current token")
        if not 1 <= self.group_size <= MAX_TOKEN_GROUP_SIZE:
            raise ValueError(f"group_size must be between 1 and {MAX_TOKEN_GROUP_SIZE}")
        if self.dim_group_size != 32 and self.group_size not in SPECIALIZED_TOKEN_GROUP_SIZES:
            raise ValueError("non-specialized token group sizes require dim_group_size=32")
        if self.dim_group_size not in SUPPORTED_DIM_GROUP_SIZES:
            raise ValueError("dim_group_size must be one of 16, 32, 64")
        if self.dim_kernel not in SUPPORTED_DIM_KERNELS:
            raise ValueError(f"dim_kernel must be one of {SUPPORTED_DIM_KERNELS}")
        if self.dim_kernel != "auto":
            expected = 64 if self.dim_kernel.startswith("g64-") else int(self.dim_kernel[1:])
            if expected != self.dim_group_size:
                raise ValueError(f"dim_kernel={self.dim_kernel} requires dim_group_size={expected}")
        if self.quest_page_size <= 0:
            raise ValueError("quest_page_size must be positive")
        if self.fier_kernel != "fier":
            raise ValueError("the public FIER method is fixed to the FIER implementation")

    @classmethod
    def preset(cls, method: str, **overrides) -> "RetrievalConfig":
        try:
            group_size, dim_group_size = POPKV_PRESETS[method]
        except KeyError as exc:
            raise ValueError(f"unknown PopKV preset: {method}") from exc
        return cls(group_size=group_size, dim_group_size=dim_group_size, **overrides)


@dataclass
class PopKVCache:
    """popkv.py:89-96."""
    group_size: int
    dim_group_size: int
    token_count: int
    sealed_tokens: int
    packed: tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]
    active_keys: torch.Tensor


@dataclass
class RetrievalCaches:
    method: str
    layers: dict[int, PopKVCache]


@dataclass
class StaticKVCache:
    """popkv.py:105-111: per-layer K/V storage [B, KVH, capacity, D]."""
    key_storage: list[torch.Tensor]
    value_storage: list[torch.Tensor]
    length: int
    capacity: int


def _sparse_layer_indices(num_layers: int, full_layers: Sequence[int]) -> tuple[int, ...]:
    return tuple(layer for layer in range(num_layers) if layer not in full_layers)


def _append_current(indices: torch.Tensor, num_tokens: int) -> torch.Tensor:
    """popkv.py:287-291: append the current token (index num_tokens - 1)."""
    current = torch.full((*indices.shape[:-1], 1), num_tokens - 1, device=indices.device, dtype=torch.long)
    return torch.cat([indices.long(), current], dim=-1)


def build_popkv_cache(
    keys: torch.Tensor, *, group_size: int, dim_group_size: int = 32, reserve_tokens: int,
) -> PopKVCache:
    """Prefix prepack (popkv.py:416-435): capacity ceil((L+reserve)/TG)*TG,
    the partial last token group kept as active keys."""
    if not 1 <= group_size <= MAX_TOKEN_GROUP_SIZE:
        raise ValueError(f"Pop-KV group_size must be between 1 and {MAX_TOKEN_GROUP_SIZE}")
    if dim_group_size != 32 and group_size not in SPECIALIZED_TOKEN_GROUP_SIZES:
        raise ValueError("non-specialized token group sizes require dim_group_size=32")
    if dim_group_size not in (16, 32, 64):
        raise ValueError("dim_group_size must be one of 16, 32, 64")
    tokens = int(keys.shape[1])
    capacity = math.ceil((tokens + reserve_tokens) / group_size) * group_size
    packed = pack_keys(keys.contiguous(), token_capacity=capacity,
                       token_group_size=group_size, dim_group_size=dim_group_size)
    sealed = (tokens // group_size) * group_size
    return PopKVCache(group_size, dim_group_size, tokens, sealed, packed,
                      keys[:, sealed:].detach().clone().contiguous())


def append_popkv(cache: PopKVCache, keys: torch.Tensor, timer=None) -> None:
    """Per-token append (popkv.py:438-459): stage the key into the active
    group, re-encode the whole active group in place, seal at TG tokens."""
    cache.active_keys = torch.cat([cache.active_keys, keys.detach()], dim=1).contiguous()
    if timer: timer.mark("active_key_staging")
    if cache.sealed_tokens + int(cache.active_keys.shape[1]) > int(cache.packed[0].shape[1]):
        raise RuntimeError("Pop-KV cache reserve exhausted")
    pack_keys_into(
        cache.active_keys, cache.packed, token_offset=cache.sealed_tokens,
        token_group_size=cache.group_size, dim_group_size=cache.dim_group_size,
    )
    if timer:
        timer.mark("k_metadata_encoding")
        timer.mark("metadata_write")
    cache.token_count += 1
    if int(cache.active_keys.shape[1]) == cache.group_size:
        cache.sealed_tokens += cache.group_size
        cache.active_keys = cache.active_keys[:, :0].contiguous()
        if timer: timer.mark("group_sealing")


def build_retrieval_caches(layer_keys: dict[int, torch.Tensor], *, method: str,
                           reserve_tokens: int = 2048) -> RetrievalCaches:
    """Prepack every sparse layer's prefix keys [KVH, L, D] with a PopKV preset
    (the PopKV part of popkv.py:853-881)."""
    if method not in POPKV_PRESETS:
        raise ValueError(f"unknown PopKV preset: {method}")
    group_size, dim_group_size = POPKV_PRESETS[method]
    return RetrievalCaches(method, {
        layer: build_popkv_cache(keys, group_size=group_size, dim_group_size=dim_group_size,
                                 reserve_tokens=reserve_tokens)
        for layer, keys in layer_keys.items()})


def append_retrieval_caches(caches: RetrievalCaches, new_keys: Sequence[torch.Tensor], *,
                            timer=None) -> None:
    """Batched per-token append across layers in three phases -- stage all,
    re-encode all, seal all (popkv.py:897-942).  new_keys[layer] is
    [1, KVH, 1, D] (the decoder's k) or [KVH, 1, D]."""
    items = []
    for layer, cache in caches.layers.items():
        k = new_keys[layer]
        items.append((cache, k[0] if k.ndim == 4 else k))
    for cache, keys in items:
        cache.active_keys = torch.cat([cache.active_keys, keys.detach()], dim=1).contiguous()
        if cache.sealed_tokens + int(cache.active_keys.shape[1]) > int(cache.packed[0].shape[1]):
            raise RuntimeError("Pop-KV cache reserve exhausted")
        cache.token_count += 1
    if timer: timer.mark("active_key_staging")
    for cache, _ in items:
        pack_keys_into(cache.active_keys, cache.packed, token_offset=cache.sealed_tokens,
                       token_group_size=cache.group_size, dim_group_size=cache.dim_group_size)
    if timer:
        timer.mark("k_metadata_encoding")
        timer.mark("metadata_write")
    for cache, _ in items:
        if int(cache.active_keys.shape[1]) == cache.group_size:
            cache.sealed_tokens += cache.group_size
            cache.active_keys = cache.active_keys[:, :0].contiguous()
    if timer: timer.mark("group_sealing")


def append_kv(cache: StaticKVCache, new_keys: Sequence[torch.Tensor], new_values: Sequence[torch.Tensor]) -> None:
    """Static K/V append at position `length` (popkv.py:964-972)."""
    if cache.length >= cache.capacity:
        raise RuntimeError("static KV cache capacity exhausted")
    position = cache.length
    for layer, (keys, values) in enumerate(zip(new_keys, new_values)):
        cache.key_storage[layer][..., position:position + 1, :].copy_(keys)
        cache.value_storage[layer][..., position:position + 1, :].copy_(values)
    cache.length += 1


def topk_popkv(scores: torch.Tensor, k: int):
    """HIP stand-in for ``torch.topk(scores, k, dim=-1, sorted=False)`` with the
    ``.indices`` attribute, as used by popkv.py:1094-1097."""
    class _TopK:
        __slots__ = ("indices",)
    result = _TopK()
    result.indices = topk_indices(scores, k)
    return result


def popkv_retrieval_step(
    q: torch.Tensor, prefix_k: torch.Tensor, prefix_v: torch.Tensor,
    k: torch.Tensor, v: torch.Tensor, cache: PopKVCache, head_to_kv: torch.Tensor, *,
    budget: int, scorer: Callable | None = None, topk: Callable | None = None, timer=None,
) -> torch.Tensor:
    """The PopKV branch of one sparse layer's decode (popkv.py:1076-1115).

    q: [QH, D] (the decoder's q[0, :, 0]); prefix_k/prefix_v: [KVH, L, D]
    (views of the static cache); k, v: [KVH, D] (the current token);
    returns attention output [QH, D] in q's dtype.  ``scorer`` / ``topk`` are
    the reference's experimental_scorer / experimental_topk hooks."""
    prefix_length = int(prefix_k.shape[1])
    num_tokens = prefix_length + 1
    encoded_query = query_encode(q.unsqueeze(0).contiguous(), dim_group_size=cache.dim_group_size)
    if timer: timer.mark("retrieval_query_encode")
    score_fn = scorer or score_encoded
    scores = score_fn(
        encoded_query, cache.packed, head_to_kv=head_to_kv, tokens=cache.token_count,
        dim_group_size=cache.dim_group_size,
        dim_kernel={16: "g16", 32: "g32", 64: "g64-u32"}[cache.dim_group_size],
    )
    if timer: timer.mark("retrieval_score")
    kk = min(budget - 1, prefix_length)
    if topk is not None:
        indices = _append_current(topk(scores, kk)[0], num_tokens)
    else:
        indices = select_with_current(scores, kk, num_tokens)
    if timer: timer.mark("topk")
    partials = indexed_attention_split_partial(q, prefix_k, prefix_v, k, v, indices, head_to_kv, None,
                                               split_tokens=SPLIT_TOKENS)
    if timer: timer.mark("sparse_attention_partial")
    output = indexed_attention_split_merge(partials, q)
    if timer: timer.mark("sparse_attention_merge")
    return output


class LayerStepWorkspace:
    """Reusable device workspace for ``popkv_layer_step`` (grown on demand).

    The C ABI keeps per-head key histograms at the start of the workspace
    (1 KiB per query head) and needs them zero when a call begins; every call
    leaves them zero.  New buffers are allocated zeroed, and when the head
    count changes the new histogram region is cleared, because it may cover
    data a call with fewer heads left behind."""

    def __init__(self) -> None:
        self.buffer: torch.Tensor | None = None
        self.rows = 0

    def get(self, nbytes: int, device: torch.device, rows: int = 0) -> torch.Tensor:
        if self.buffer is None or self.buffer.numel() < nbytes or self.buffer.device != device:
            self.buffer = torch.zeros(max(nbytes, 1), device=device, dtype=torch.uint8)
        elif rows != self.rows:
            self.buffer[: min(self.buffer.numel(), rows * 1024)].zero_()
        self.rows = rows
        return self.buffer


def layer_step_workspace_bytes(q_heads: int, tokens: int, budget: int, dim_group_size: int) -> int:
    return int(nat.lib().popkv_layer_step_workspace_bytes(q_heads, tokens, budget, dim_group_size))


def _check_step_operands(name: str, q: torch.Tensor, prefix_k: torch.Tensor, prefix_v: torch.Tensor,
                         k: torch.Tensor, v: torch.Tensor, out: torch.Tensor | None) -> tuple[int, int]:
    """Shape checks shared by the fused decode entries.

    The C ABI receives raw pointers and head counts only, so every size it
    derives addresses from is checked before any device call: q [QH, 128];
    prefix K/V [KVH, L, 128] with contiguous rows; current k/v [KVH, 128];
    QH a positive multiple of KVH; `out` (when given) a contiguous
    [QH, 128] tensor.  Raises ValueError (the reference's Python-side
    checks); dtypes and devices are checked by _check_same_device.
    Returns (QH, KVH)."""
    if q.ndim != 2 or int(q.shape[1]) != 128:
        raise ValueError(f"{name} requires q [query heads, 128]")
    if prefix_k.ndim != 3 or prefix_v.shape != prefix_k.shape or int(prefix_k.shape[2]) != 128:
        raise ValueError("prefix K/V must be [KV heads, tokens, 128]")
    if prefix_k.stride(1) != 128 or prefix_k.stride(2) != 1 or prefix_v.stride(1) != 128 or prefix_v.stride(2) != 1:
        raise ValueError("prefix K/V rows must be contiguous (token stride 128)")
    q_heads, kv_heads = int(q.shape[0]), int(prefix_k.shape[0])
    if q_heads <= 0 or kv_heads <= 0 or q_heads % kv_heads != 0:
        raise ValueError("query heads must be a positive multiple of the KV heads")
    for t, what in ((k, "current k"), (v, "current v")):
        if tuple(t.shape) != (kv_heads, 128):
            raise ValueError(f"{what} must be [KV heads, 128] = [{kv_heads}, 128], got {tuple(t.shape)}")
    if out is not None:
        if tuple(out.shape) != (q_heads, 128):
            raise ValueError(f"out must be [{q_heads}, 128], got {tuple(out.shape)}")
        if not out.is_contiguous():
            raise ValueError("out must be contiguous")
    return q_heads, kv_heads


def _check_same_device(name: str, q: torch.Tensor, *tensors: torch.Tensor | None) -> None:
    """Every operand of q's dtype and on q's CUDA device (RuntimeError, as
    the reference's TORCH_CHECKs)."""
    ts = (q,) + tuple(t for t in tensors if t is not None)
    if any(t.dtype != q.dtype for t in ts):
        raise RuntimeError("queries, current K/V, prefix K/V and out must share a dtype")
    if any(not t.is_cuda or t.device != q.device for t in ts):
        raise RuntimeError(f"{name}: every tensor must be on the same CUDA device")


def _check_packed_cache(cache: PopKVCache, kv_heads: int) -> None:
    """The packed planes the scorer reads: int32 [KVH, cap, 4] sign/mag and
    fp16 [KVH, cap, 128/G] low/delta with the prefix's KV head count, and
    token_count within the capacity (ValueError before any device call)."""
    if len(cache.packed) != 4:
        raise ValueError("packed must contain (k_sign, k_mag, k_low, k_delta)")
    if cache.dim_group_size not in (16, 32, 64):
        raise ValueError("dim_group_size must be one of 16, 32, 64")
    k_sign = cache.packed[0]
    cap = int(k_sign.shape[1]) if k_sign.ndim == 3 else -1
    reps = 128 // cache.dim_group_size
    for t, dt, width, what in zip(cache.packed, (torch.int32, torch.int32, torch.float16, torch.float16),
                                  (4, 4, reps, reps), ("k_sign", "k_mag", "k_low", "k_delta")):
        if tuple(t.shape) != (kv_heads, cap, width):
            raise ValueError(f"packed {what} must be [{kv_heads}, capacity, {width}], got {tuple(t.shape)}")
        if t.dtype != dt or not t.is_contiguous():
            raise ValueError(f"packed {what} must be a contiguous {dt} tensor")
    if not 0 < cache.token_count <= cap:
        raise ValueError("invalid score token count")


def _check_packed_device(cache: PopKVCache, device: torch.device) -> None:
    if any(not t.is_cuda or t.device != device for t in cache.packed):
        raise RuntimeError("the packed cache must be on the queries' CUDA device")


def _check_head_mapping(head_to_kv: torch.Tensor, q_heads: int) -> None:
    if head_to_kv.ndim != 1 or int(head_to_kv.numel()) != q_heads:
        raise ValueError(f"head_to_kv must be a vector of {q_heads} KV head indices")
    if head_to_kv.dtype not in (torch.int64, torch.int32):
        raise ValueError("head_to_kv must be int64 or int32")


def popkv_layer_step(
    q: torch.Tensor, cache: PopKVCache, prefix_k: torch.Tensor, prefix_v: torch.Tensor,
    k: torch.Tensor, v: torch.Tensor, head_to_kv: torch.Tensor, *, budget: int,
    workspace: LayerStepWorkspace | torch.Tensor | None = None, out: torch.Tensor | None = None,
    return_indices: bool = False,
):
    """One sparse layer's retrieval step (head_dim 128, batch 1) in a single
    C-ABI call: encode + popcount score, top-k + current, split attention,
    merge.  Same result as ``popkv_retrieval_step``.

    prefix_k/prefix_v: [KVH, L, 128] with unit row stride 128 (any head
    stride); q: [QH, 128]; k, v: [KVH, 128].  Returns out [QH, 128] (and the
    int64 [QH, k+1] selection when return_indices)."""
    q_heads, kv_heads = _check_step_operands("popkv_layer_step", q, prefix_k, prefix_v, k, v, out)
    tokens = int(prefix_k.shape[1])
    if tokens != cache.token_count:
        raise ValueError("prefix length must equal the retrieval cache's token_count")
    if budget <= 1:
        raise ValueError("budget must reserve at least one retrieved and one current token")
    _check_head_mapping(head_to_kv, q_heads)
    _check_packed_cache(cache, kv_heads)
    _check_same_device("popkv_layer_step", q, prefix_k, prefix_v, k, v, out)
    dev = q.device
    _check_packed_device(cache, dev)
    qc, kc, vc = q.contiguous(), k.contiguous(), v.contiguous()
    mapping = head_to_kv.to(device=dev, dtype=torch.int64).contiguous()
    nbytes = layer_step_workspace_bytes(q_heads, tokens, budget, cache.dim_group_size)
    if isinstance(workspace, torch.Tensor):
        ws = workspace  # caller-owned: zero-filled before its first use
    else:
        ws = (workspace or LayerStepWorkspace()).get(nbytes, dev, q_heads)
    output = torch.empty_like(qc) if out is None else out
    kk = min(budget - 1, tokens)
    idx = torch.empty((q_heads, kk + 1), device=dev, dtype=torch.int64) if return_indices else None
    k_sign, k_mag, k_low, k_delta = cache.packed
    with torch.cuda.device(dev):
        nat.call("popkv_layer_step", qc.data_ptr(), nat.dtype_code(qc), k_sign.data_ptr(), k_mag.data_ptr(),
                 k_low.data_ptr(), k_delta.data_ptr(), int(k_sign.shape[1]), prefix_k.data_ptr(), prefix_v.data_ptr(),
                 prefix_k.stride(0), prefix_v.stride(0), kc.data_ptr(), vc.data_ptr(), mapping.data_ptr(), q_heads,
                 kv_heads, tokens, int(budget), cache.dim_group_size, output.data_ptr(), nat.ptr(idx),
                 ws.data_ptr(), ws.numel(), nat.stream_of(dev))
    return (output, idx) if return_indices else output


def popkv_layer_step_attention(q: torch.Tensor, prefix_k: torch.Tensor, prefix_v: torch.Tensor,
                               head_to_kv: torch.Tensor, *, budget: int, dim_group_size: int,
                               workspace: LayerStepWorkspace | torch.Tensor) -> None:
    """Re-run only the fused select + sparse-attention kernel of the last
    ``popkv_layer_step`` that used ``workspace`` (same shapes, budget and
    dim_group_size); it reads the keys and threshold data the step left
    there and rewrites the chunk partials inside the workspace.  A timing
    aid for the step's select + attention half as a launch of its own."""
    if q.ndim != 2 or int(q.shape[1]) != 128 or not q.is_contiguous():
        raise ValueError("popkv_layer_step_attention requires a contiguous q [query heads, 128]")
    if prefix_k.ndim != 3 or prefix_v.shape != prefix_k.shape or int(prefix_k.shape[2]) != 128:
        raise ValueError("prefix K/V must be [KV heads, tokens, 128]")
    if prefix_k.stride(1) != 128 or prefix_k.stride(2) != 1 or prefix_v.stride(1) != 128 or prefix_v.stride(2) != 1:
        raise ValueError("prefix K/V rows must be contiguous (token stride 128)")
    q_heads, kv_heads, tokens = int(q.shape[0]), int(prefix_k.shape[0]), int(prefix_k.shape[1])
    if q_heads <= 0 or kv_heads <= 0 or q_heads % kv_heads != 0:
        raise ValueError("query heads must be a positive multiple of the KV heads")
    if tokens <= 0:
        raise ValueError("invalid score token count")
    if budget <= 1:
        raise ValueError("budget must reserve at least one retrieved and one current token")
    if dim_group_size not in (16, 32, 64):
        raise ValueError("dim_group_size must be one of 16, 32, 64")
    _check_head_mapping(head_to_kv, q_heads)
    ws = workspace if isinstance(workspace, torch.Tensor) else workspace.buffer
    if ws is None:
        raise ValueError("the workspace has not been used by popkv_layer_step")
    _check_same_device("popkv_layer_step_attention", q, prefix_k, prefix_v)
    if ws.device != q.device:
        raise RuntimeError("popkv_layer_step_attention: every tensor must be on the same CUDA device")
    dev = q.device
    mapping = head_to_kv.to(device=dev, dtype=torch.int64).contiguous()
    with torch.cuda.device(dev):
        nat.call("popkv_layer_step_attention", q.data_ptr(), nat.dtype_code(q), prefix_k.data_ptr(),
                 prefix_v.data_ptr(), prefix_k.stride(0), prefix_v.stride(0), mapping.data_ptr(), q_heads, kv_heads,
                 tokens, int(budget), int(dim_group_size), ws.data_ptr(), ws.numel(), nat.stream_of(dev))


def dense_attention_step(q: torch.Tensor, prefix_k: torch.Tensor, prefix_v: torch.Tensor, k: torch.Tensor,
                         v: torch.Tensor, *, workspace: LayerStepWorkspace | None = None,
                         out: torch.Tensor | None = None) -> torch.Tensor:
    """Full attention of one decode step over every prefix token plus the
    current one (the reference's full layers, popkv.py:1022-1038), one C-ABI
    call: q [QH, 128], prefix K/V [KVH, L, 128] with contiguous rows, current
    k/v [KVH, 128] -> [QH, 128], query head h reading KV head h // (QH/KVH).
    The workspace holds merge tickets and split partials; do not share it
    with popkv_layer_step, whose histogram region must stay zero."""
    q_heads, kv_heads = _check_step_operands("dense_attention_step", q, prefix_k, prefix_v, k, v, out)
    if q_heads // kv_heads not in (1, 2, 4, 8):
        raise ValueError("dense attention supports 1, 2, 4 or 8 query heads per KV head")
    _check_same_device("dense_attention_step", q, prefix_k, prefix_v, k, v, out)
    dev = q.device
    qc, kc, vc = q.contiguous(), k.contiguous(), v.contiguous()
    tokens = int(prefix_k.shape[1])
    nbytes = int(nat.lib().popkv_dense_attention_workspace_bytes(q_heads, tokens))
    # (its first bytes hold the merge tickets: zero on entry, left zero; a
    # change of head count clears them, as for the layer step's histograms)
    ws = (workspace or LayerStepWorkspace()).get(nbytes, dev, q_heads)
    output = torch.empty_like(qc) if out is None else out
    with torch.cuda.device(dev):
        nat.call("popkv_dense_attention", qc.data_ptr(), nat.dtype_code(qc), prefix_k.data_ptr(), prefix_v.data_ptr(),
                 prefix_k.stride(0), prefix_v.stride(0), kc.data_ptr(), vc.data_ptr(), q_heads, kv_heads, tokens,
                 output.data_ptr(), ws.data_ptr(), ws.numel(), nat.stream_of(dev))
    return output


class SparseDecodeStack:
    """The attention half of one ``LlamaSparseDecoder.decode`` step across a
    layer stack (popkv.py:1022-1115): a layer listed in ``full_layers`` takes
    dense attention over every cached token plus the current one
    (``dense_attention_step``), every other layer the PopKV retrieval step
    over its ``PopKVCache`` (``popkv_layer_step``).  One workspace serves the
    sparse layers and one the dense layers, so a whole step records into one
    HIP graph without allocating.

    caches: layer -> PopKVCache for the sparse layers; head_to_kv: the GQA
    mapping of the sparse layers (dense layers use h // (QH / KVH))."""

    def __init__(self, caches: dict[int, PopKVCache], head_to_kv: torch.Tensor, *, budget: int,
                 full_layers: Sequence[int] = (0, 1)) -> None:
        if budget <= 1:
            raise ValueError("budget must reserve at least one retrieved and one current token")
        overlap = set(caches) & set(full_layers)
        if overlap:
            raise ValueError(f"layers {sorted(overlap)} are full layers and cannot have a retrieval cache")
        self.caches = caches
        self.head_to_kv = head_to_kv
        self.budget = int(budget)
        self.full_layers = tuple(full_layers)
        self.sparse_workspace = LayerStepWorkspace()
        self.dense_workspace = LayerStepWorkspace()

    def layer(self, layer: int, q: torch.Tensor, prefix_k: torch.Tensor, prefix_v: torch.Tensor, k: torch.Tensor,
              v: torch.Tensor, *, out: torch.Tensor | None = None) -> torch.Tensor:
        """Attention output [QH, 128] of one layer for the current token."""
        if layer in self.full_layers:
            return dense_attention_step(q, prefix_k, prefix_v, k, v, workspace=self.dense_workspace, out=out)
        try:
            cache = self.caches[layer]
        except KeyError:
            raise ValueError(f"layer {layer} is sparse but has no retrieval cache") from None
        return popkv_layer_step(q, cache, prefix_k, prefix_v, k, v, self.head_to_kv, budget=self.budget,
                                workspace=self.sparse_workspace, out=out)

    def step(self, operands: Sequence[tuple], outs: Sequence[torch.Tensor] | None = None) -> list[torch.Tensor]:
        """Every layer in order; operands[layer] = (q, prefix_k, prefix_v, k, v)."""
        return [self.layer(i, *ops, out=None if outs is None else outs[i]) for i, ops in enumerate(operands)]
