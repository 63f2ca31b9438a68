"""Batched decode over sequences of different lengths, with the static K/V
cache and the PopKV retrieval metadata maintained in place.

The reference decodes one sequence at a time: its packed caches have no
batch dimension (popkv_ext.cu:769-806), and every decode step stages the new
key with ``torch.cat`` into ``active_keys`` before re-encoding the active
token group (``append_popkv``, popkv.py:438-459; ``append_retrieval_caches``,
:883-942) and copies the new K/V rows into the static cache separately
(popkv.py:964-972).  Here a layer's caches carry a leading batch dimension:

  * ``SequenceLengths``: every sequence's cached-token count, on the device
    (int64 [B], read by the kernels, so one HIP graph of a decode step stays
    valid while the sequences grow) with a host mirror for the capacity
    checks; shared by every layer of the model;
  * ``BatchedPopKVCache``: one sparse layer's packed planes
    [B, KVH, capacity, .] next to its static K/V caches [B, KVH, rows, 128]
    (the reference's StaticKVCache layout, popkv.py:105-111);
  * ``append_batched``: one C-ABI call per layer writes every sequence's new
    K/V row into the static caches and re-encodes its active token group,
    reading the group's older keys in place (no staging copy);
  * ``popkv_layer_step_batched``: one C-ABI call per layer runs the
    retrieval step of every sequence (each at its own length);
  * ``SequenceLengths.advance``: after every layer of the step has appended.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from . import _native as nat
from .popkv import LayerStepWorkspace, MAX_TOKEN_GROUP_SIZE, SPECIALIZED_TOKEN_GROUP_SIZES


@dataclass
class SequenceLengths:
    """Cached tokens per sequence: ``device`` int64 [B] (what the kernels
    read) and ``host`` (the same counts, for checks made before a launch)."""
    device: torch.Tensor
    host: list[int]

    @classmethod
    def create(cls, lengths, device) -> "SequenceLengths":
        host = [int(x) for x in lengths]
        if not host or min(host) < 0:
            raise ValueError("lengths must be a non-empty list of non-negative token counts")
        return cls(torch.tensor(host, dtype=torch.int64, device=device), host)

    @property
    def batch(self) -> int:
        return len(self.host)

    def advance(self) -> None:
        """Every sequence gained the token its decode step appended."""
        self.device.add_(1)
        self.host = [x + 1 for x in self.host]


@dataclass
class BatchedPopKVCache:
    """One sparse layer's retrieval metadata for a batch, beside the
    layer's static K/V caches (written in place by ``append_batched``)."""
    group_size: int
    dim_group_size: int
    packed: tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]
    key_cache: torch.Tensor
    value_cache: torch.Tensor

    @property
    def capacity(self) -> int:
        """Tokens a sequence can hold: the static cache rows."""
        return int(self.key_cache.shape[2])


def _check_static(key_cache: torch.Tensor, value_cache: torch.Tensor) -> None:
    if key_cache.ndim != 4 or int(key_cache.shape[3]) != 128 or value_cache.shape != key_cache.shape:
        raise ValueError("static K/V caches must be [batch, KV heads, rows, 128]")
    if not key_cache.is_contiguous() or not value_cache.is_contiguous():
        raise ValueError("static K/V caches must be contiguous")
    if key_cache.dtype != value_cache.dtype or key_cache.dtype not in (torch.float32, torch.float16, torch.bfloat16):
        raise ValueError("static K/V caches must share an fp32/fp16/bf16 dtype")


def _check_planes(cache: BatchedPopKVCache) -> int:
    """The packed planes every batched kernel addresses: contiguous int32
    sign/mag [B, KVH, cap, 4] and fp16 low/delta [B, KVH, cap, 128/G], with
    the static caches' batch and KV head counts and one capacity
    (ValueError; devices are checked by _check_on_device after the
    host-side checks).  Returns the planes' capacity."""
    _check_static(cache.key_cache, cache.value_cache)
    if cache.dim_group_size not in (16, 32, 64):
        raise ValueError("dim_group_size must be one of 16, 32, 64")
    if not 1 <= cache.group_size <= MAX_TOKEN_GROUP_SIZE:
        raise ValueError(f"Pop-KV group_size must be between 1 and {MAX_TOKEN_GROUP_SIZE}")
    if len(cache.packed) != 4:
        raise ValueError("packed must contain (k_sign, k_mag, k_low, k_delta)")
    batch, kv_heads = (int(x) for x in cache.key_cache.shape[:2])
    sign = cache.packed[0]
    cap = int(sign.shape[2]) if sign.ndim == 4 else -1
    reps = 128 // cache.dim_group_size
    for t, dt, width, what in zip(cache.packed, (torch.int32, torch.int32, torch.float16, torch.float16),
                                  (4, 4, reps, reps), ("k_sign", "k_mag", "k_low", "k_delta")):
        if tuple(t.shape) != (batch, kv_heads, cap, width) or cap <= 0:
            raise ValueError(f"packed {what} must be [{batch}, {kv_heads}, capacity, {width}], got {tuple(t.shape)}")
        if t.dtype != dt or not t.is_contiguous():
            raise ValueError(f"packed {what} must be a contiguous {dt} tensor")
    return cap


def _check_on_device(cache: BatchedPopKVCache, lengths: SequenceLengths, *tensors: torch.Tensor | None) -> None:
    """The device token counts (a contiguous int64 [B]), the static caches,
    the packed planes and every operand on one CUDA device: the kernels
    dereference them all (RuntimeError, as the reference's TORCH_CHECKs)."""
    if lengths.device.dtype != torch.int64 or lengths.device.ndim != 1 or not lengths.device.is_contiguous() \
            or int(lengths.device.numel()) != lengths.batch:
        raise ValueError("sequence lengths must be a contiguous int64 [batch] tensor")
    dev = cache.key_cache.device
    if dev.type != "cuda":
        raise RuntimeError("the static caches must be on a CUDA device")
    for t in (cache.value_cache, lengths.device) + tuple(cache.packed) + tuple(t for t in tensors if t is not None):
        if t.device != dev:
            raise RuntimeError(f"every operand must be on the caches' device {dev}, got {t.device}")


def build_batched_popkv_cache(key_cache: torch.Tensor, value_cache: torch.Tensor, lengths: SequenceLengths, *,
                              group_size: int, dim_group_size: int) -> BatchedPopKVCache:
    """Prepack each sequence's cached prefix (rows [0, lengths[b]) of its
    static keys, read in place) with the reference's prefix prepack
    (popkv.py:416-435): token groups of ``group_size`` counted from the first
    token, the partial last group left active for the appends."""
    _check_static(key_cache, value_cache)
    if not 1 <= group_size <= MAX_TOKEN_GROUP_SIZE:
        raise ValueError(f"Pop-KV group_size must be between 1 and {MAX_TOKEN_GROUP_SIZE}")
    if dim_group_size != 32 and group_size not in SPECIALIZED_TOKEN_GROUP_SIZES:
        raise ValueError("non-specialized token group sizes require dim_group_size=32")
    if dim_group_size not in (16, 32, 64):
        raise ValueError("dim_group_size must be one of 16, 32, 64")
    batch, kv_heads, rows = (int(x) for x in key_cache.shape[:3])
    if lengths.batch != batch:
        raise ValueError(f"{lengths.batch} lengths for a batch of {batch}")
    if max(lengths.host) > rows:
        raise RuntimeError("Pop-KV cache capacity exceeded")
    cap = math.ceil(rows / group_size) * group_size
    dev = key_cache.device
    if dev.type != "cuda" or value_cache.device != dev:
        raise RuntimeError("the static caches must be on one CUDA device")
    reps = 128 // dim_group_size
    packed = (torch.zeros(batch, kv_heads, cap, 4, dtype=torch.int32, device=dev),
              torch.zeros(batch, kv_heads, cap, 4, dtype=torch.int32, device=dev),
              torch.zeros(batch, kv_heads, cap, reps, dtype=torch.float16, device=dev),
              torch.zeros(batch, kv_heads, cap, reps, dtype=torch.float16, device=dev))
    cache = BatchedPopKVCache(group_size, dim_group_size, packed, key_cache, value_cache)
    prepack_batched(cache, lengths)
    return cache


def prepack_batched(cache: BatchedPopKVCache, lengths: SequenceLengths) -> None:
    """(Re-)encode every sequence's cached prefix into the cache's packed
    planes: one popkv_pack launch per non-empty sequence, reading rows
    [0, lengths[b]) of its static keys in place."""
    cap = _check_planes(cache)
    batch, kv_heads = (int(x) for x in cache.key_cache.shape[:2])
    if lengths.batch != batch:
        raise ValueError(f"{lengths.batch} lengths for a batch of {batch}")
    if max(lengths.host) > min(cache.capacity, cap):
        raise RuntimeError("Pop-KV cache capacity exceeded")
    dev = cache.key_cache.device
    _check_on_device(cache, lengths)
    with torch.cuda.device(dev):
        stream = nat.stream_of(dev)
        if len(set(lengths.host)) == 1 and lengths.host[0] > 0:
            # equal lengths: one launch, the batch's B*KVH heads side by side
            # (head stride = the static cache rows in both layouts)
            kc = cache.key_cache
            nat.call("popkv_pack", kc.data_ptr(), nat.dtype_code(kc), batch * kv_heads, lengths.host[0], 128,
                     kc.stride(1), cache.packed[0].data_ptr(), cache.packed[1].data_ptr(),
                     cache.packed[2].data_ptr(), cache.packed[3].data_ptr(), cap, 0, cache.group_size,
                     cache.dim_group_size, stream)
            return
        for b, n in enumerate(lengths.host):
            if n == 0:
                continue
            kb = cache.key_cache[b]
            nat.call("popkv_pack", kb.data_ptr(), nat.dtype_code(kb), kv_heads, n, 128, kb.stride(0),
                     cache.packed[0][b].data_ptr(), cache.packed[1][b].data_ptr(), cache.packed[2][b].data_ptr(),
                     cache.packed[3][b].data_ptr(), cap, 0, cache.group_size, cache.dim_group_size, stream)


def append_batched(cache: BatchedPopKVCache, lengths: SequenceLengths, new_k: torch.Tensor, new_v: torch.Tensor,
                   *, status: torch.Tensor | None = None) -> None:
    """Append every sequence's new token (new_k / new_v [B, KVH, 128]) to
    one layer: its K/V rows go to row lengths[b] of the static caches and
    the sequence's active token group is re-encoded in place (sealing at
    ``group_size`` tokens).  One C-ABI call for the batch; call
    ``lengths.advance()`` once every layer has appended.  Raises
    RuntimeError("Pop-KV cache reserve exhausted") when a sequence is full
    (popkv.py:445-446); ``status`` (device int32 [1]) additionally records a
    full sequence met on the device (for replays of a captured step)."""
    batch, kv_heads = (int(x) for x in cache.key_cache.shape[:2])
    if tuple(new_k.shape) != (batch, kv_heads, 128) or new_v.shape != new_k.shape:
        raise ValueError(f"new K/V must be [{batch}, {kv_heads}, 128]")
    if lengths.batch != batch:
        raise ValueError(f"{lengths.batch} lengths for a batch of {batch}")
    cap = _check_planes(cache)
    if max(lengths.host) >= min(cache.capacity, cap):
        raise RuntimeError("Pop-KV cache reserve exhausted")
    if status is not None and (status.dtype != torch.int32 or status.numel() < 1):
        raise ValueError("status must be an int32 tensor of at least one element")
    nk, nv = new_k.contiguous(), new_v.contiguous()
    if nk.dtype != cache.key_cache.dtype or nv.dtype != cache.key_cache.dtype:
        raise RuntimeError("new K/V must have the static caches' dtype")
    dev = cache.key_cache.device
    _check_on_device(cache, lengths, nk, nv, status)
    ks, km, kl, kd = cache.packed
    with torch.cuda.device(dev):
        nat.call("popkv_append", nk.data_ptr(), nv.data_ptr(), nat.dtype_code(nk), cache.key_cache.data_ptr(),
                 cache.value_cache.data_ptr(), cache.capacity, ks.data_ptr(), km.data_ptr(), kl.data_ptr(),
                 kd.data_ptr(), int(ks.shape[2]), lengths.device.data_ptr(), batch, kv_heads, cache.group_size,
                 cache.dim_group_size, nat.ptr(status), nat.stream_of(dev))


def popkv_layer_step_batched(q: torch.Tensor, cache: BatchedPopKVCache, lengths: SequenceLengths,
                             k: torch.Tensor, v: torch.Tensor, head_to_kv: torch.Tensor, *, budget: int,
                             max_tokens: int | None = None, workspace: LayerStepWorkspace | None = None,
                             out: torch.Tensor | None = None, return_indices: bool = False,
                             append: bool = False, status: torch.Tensor | None = None):
    """The retrieval step of one sparse layer for every sequence of the
    batch (q [B, QH, 128], current k/v [B, KVH, 128], head_to_kv [QH]):
    sequence b scores its lengths[b] cached tokens, selects
    min(budget - 1, lengths[b]) of them plus the current token and attends
    over them.  ``max_tokens`` (default: the longest host length) bounds the
    device lengths for the launch -- give the largest length a captured
    graph will see.  Returns out [B, QH, 128] (and int64 indices
    [B, QH, min(budget - 1, max_tokens) + 1] whose row (b, h) holds
    k_b + 1 valid entries, the current token last).

    ``append=True`` also appends the current token (k, v) to the layer's
    caches, with the results of ``append_batched(cache, lengths, k, v,
    status=status)`` after the step, in one C-ABI call
    (popkv_decode_layer_batched) whose append runs in extra workgroups of
    the step's select + attention launch.  With ``append=True``, ``status``
    (int32, on the cache's device) also gets bit 1 (value 2) when a
    sequence's device count exceeds ``max_tokens`` (the step then ran on
    the clamped count): poll it after replaying a captured step.  It is
    only read with ``append=True``."""
    cap = _check_planes(cache)
    batch, kv_heads = (int(x) for x in cache.key_cache.shape[:2])
    if q.ndim != 3 or int(q.shape[0]) != batch or int(q.shape[2]) != 128:
        raise ValueError(f"q must be [{batch}, query heads, 128]")
    q_heads = int(q.shape[1])
    if q_heads % kv_heads != 0:
        raise ValueError("query heads must be a multiple of the KV heads")
    for t, what in ((k, "current k"), (v, "current v")):
        if tuple(t.shape) != (batch, kv_heads, 128):
            raise ValueError(f"{what} must be [{batch}, {kv_heads}, 128]")
    if head_to_kv.ndim != 1 or int(head_to_kv.numel()) != q_heads:
        raise ValueError(f"head_to_kv must be a vector of {q_heads} KV head indices")
    if budget <= 1:
        raise ValueError("budget must reserve at least one retrieved and one current token")
    if lengths.batch != batch:
        raise ValueError(f"{lengths.batch} lengths for a batch of {batch}")
    bound = max(lengths.host) if max_tokens is None else int(max_tokens)
    if bound < max(lengths.host) or bound < 1:
        raise ValueError("max_tokens must be at least 1 and cover every sequence's length")
    if bound > min(cache.capacity, cap):
        raise RuntimeError("invalid score token count")
    if out is not None and (tuple(out.shape) != tuple(q.shape) or not out.is_contiguous() or out.dtype != q.dtype):
        raise ValueError("out must be a contiguous tensor shaped and typed like q")
    if append:
        if max(lengths.host) >= min(cache.capacity, cap):
            raise RuntimeError("Pop-KV cache reserve exhausted")
    if status is not None and (not append or status.dtype != torch.int32 or status.numel() < 1):
        raise ValueError("status must be an int32 tensor of at least one element, given with append=True")
    if any(t.dtype != q.dtype for t in (k, v, cache.key_cache)):
        raise RuntimeError("queries, current K/V and the static caches must share a dtype")
    dev = cache.key_cache.device
    _check_on_device(cache, lengths, q, k, v, out, status)
    qc, kc, vc = q.contiguous(), k.contiguous(), v.contiguous()
    mapping = head_to_kv.to(device=dev, dtype=torch.int64).contiguous()
    g = cache.dim_group_size
    nbytes = int(nat.lib().popkv_layer_step_batched_workspace_bytes(batch, q_heads, bound, budget, g))
    ws = (workspace or LayerStepWorkspace()).get(nbytes, dev, batch * q_heads)
    output = torch.empty_like(qc) if out is None else out
    kk = min(budget - 1, bound)
    idx = torch.full((batch, q_heads, kk + 1), -1, device=dev, dtype=torch.int64) if return_indices else None
    ks, km, kl, kd = cache.packed
    with torch.cuda.device(dev):
        if append:
            nat.call("popkv_decode_layer_batched", qc.data_ptr(), nat.dtype_code(qc), ks.data_ptr(), km.data_ptr(),
                     kl.data_ptr(), kd.data_ptr(), int(ks.shape[2]), cache.key_cache.data_ptr(),
                     cache.value_cache.data_ptr(), cache.capacity, kc.data_ptr(), vc.data_ptr(), mapping.data_ptr(),
                     batch, q_heads, kv_heads, lengths.device.data_ptr(), bound, int(budget), g, cache.group_size,
                     output.data_ptr(), nat.ptr(idx), kk + 1, nat.ptr(status), ws.data_ptr(), ws.numel(),
                     nat.stream_of(dev))
        else:
            nat.call("popkv_layer_step_batched", qc.data_ptr(), nat.dtype_code(qc), ks.data_ptr(), km.data_ptr(),
                     kl.data_ptr(), kd.data_ptr(), int(ks.shape[2]), cache.key_cache.data_ptr(),
                     cache.value_cache.data_ptr(), cache.capacity, kc.data_ptr(), vc.data_ptr(), mapping.data_ptr(),
                     batch, q_heads, kv_heads, lengths.device.data_ptr(), bound, int(budget), g, output.data_ptr(),
                     nat.ptr(idx), kk + 1, ws.data_ptr(), ws.numel(), nat.stream_of(dev))
    return (output, idx) if return_indices else output
