"""Seeded synthetic workloads at the benchmark configurations.

Inputs are drawn on the CPU with ``torch.Generator().manual_seed(seed)`` in a
fixed order, cast, and only then moved to the device, so every run (GPU,
tests, CPU baseline) sees identical bits.

Configurations (by index):
  C0  CPU plumbing: 1 layer, QH 8 / KVH 2, D 128, context 4096, budget 512,
      popkv-normal (TG 32, G 32); K, V, Q fp32 i.i.d. N(0,1), seed 0.
  C1  PopKV-S single layer at Llama-3.1-8B shapes: QH 32 / KVH 8, D 128,
      context 32768, budget 4096, bf16, TG 64 / G 64.  K ~ N(0,1) with 4
      outlier channels per KV head scaled x10; V ~ N(0,1); each query head is
      0.5 * mean of 64 random rows of its KV head's keys + N(0,1).  Seed 42.
  C2  PopKV-Q (TG 128 / G 16) at the same shapes, per layer seed 42 + layer.
  C3  PopKV-S context sweep 4K..128K, budget 4096, seed 7.
  C4  PopKV-S, 8 sequences x 64K context, budget 4096, seed 123 + b for
      sequence b; the tokens a decode step appends are N(0,1)
      (``new_tokens``).
The current token is the last row of K/V (C4: a ``new_tokens`` row); the
prefix holds L = context - 1 tokens.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch


@dataclass(frozen=True)
class Workload:
    name: str
    method: str
    q_heads: int
    kv_heads: int
    head_dim: int
    context: int
    budget: int
    token_group: int
    dim_group: int
    dtype: torch.dtype
    seed: int
    peaked: bool
    batch: int = 1

    @property
    def prefix_tokens(self) -> int:
        return self.context - 1

    @property
    def k(self) -> int:
        return min(self.budget - 1, self.prefix_tokens)


C0 = Workload("C0-popkv-normal-4k", "popkv-normal", 8, 2, 128, 4096, 512, 32, 32, torch.float32, 0, False)
C1 = Workload("C1-popkv-s-32k-b4096", "popkv-s", 32, 8, 128, 32768, 4096, 64, 64, torch.bfloat16, 42, True)
C2_LAYER = Workload("C2-popkv-q-32k-b4096", "popkv-q", 32, 8, 128, 32768, 4096, 128, 16, torch.bfloat16, 42, True)
C3_CONTEXTS = (4096, 8192, 16384, 32768, 65536, 131072)
C4 = Workload("C4-popkv-s-b8-64k", "popkv-s", 32, 8, 128, 65536, 4096, 64, 64, torch.bfloat16, 123, True, batch=8)


def c3(context: int) -> Workload:
    return Workload(f"C3-popkv-s-{context // 1024}k-b4096", "popkv-s", 32, 8, 128, context, 4096, 64, 64,
                    torch.bfloat16, 7, True)


def c2_layer(layer: int) -> Workload:
    return Workload(f"C2-popkv-q-layer{layer}", "popkv-q", 32, 8, 128, 32768, 4096, 128, 16, torch.bfloat16,
                    42 + layer, True)


def scaled(w: Workload, *, context: int | None = None, budget: int | None = None) -> Workload:
    """Same distribution at a smaller context/budget (for fast parity cases)."""
    return Workload(w.name + "-scaled", w.method, w.q_heads, w.kv_heads, w.head_dim,
                    context if context is not None else w.context, budget if budget is not None else w.budget,
                    w.token_group, w.dim_group, w.dtype, w.seed, w.peaked, w.batch)


@dataclass
class LayerInputs:
    """One layer's synthetic K/V/Q on the CPU, already cast to the workload dtype.

    keys/values: [KVH, context, D] (the static cache rows; the last row is the
    current token); queries: [QH, D]."""
    keys: torch.Tensor
    values: torch.Tensor
    queries: torch.Tensor

    @property
    def prefix_tokens(self) -> int:
        return int(self.keys.shape[1]) - 1

    def prefix_k(self) -> torch.Tensor:
        return self.keys[:, :-1]

    def prefix_v(self) -> torch.Tensor:
        return self.values[:, :-1]

    def current_k(self) -> torch.Tensor:
        return self.keys[:, -1].contiguous()

    def current_v(self) -> torch.Tensor:
        return self.values[:, -1].contiguous()

    def to(self, device) -> "LayerInputs":
        return LayerInputs(self.keys.to(device), self.values.to(device), self.queries.to(device))


def make_layer(w: Workload, *, seed: int | None = None) -> LayerInputs:
    """Draw one layer's inputs for workload `w` (see the module docstring)."""
    g = torch.Generator().manual_seed(w.seed if seed is None else seed)
    kvh, qh, d, ctx = w.kv_heads, w.q_heads, w.head_dim, w.context
    if not w.peaked:
        keys = torch.randn(kvh, ctx, d, generator=g)
        values = torch.randn(kvh, ctx, d, generator=g)
        queries = torch.randn(qh, d, generator=g)
    else:
        keys = torch.randn(kvh, ctx, d, generator=g)
        for h in range(kvh):
            channels = torch.randperm(d, generator=g)[:4]
            keys[h, :, channels] *= 10.0
        values = torch.randn(kvh, ctx, d, generator=g)
        prefix = ctx - 1
        qpk = qh // kvh
        queries = torch.empty(qh, d)
        for h in range(qh):
            rows = torch.randint(0, prefix, (64,), generator=g)
            queries[h] = 0.5 * keys[h // qpk, rows].mean(0) + torch.randn(d, generator=g)
    return LayerInputs(keys.to(w.dtype), values.to(w.dtype), queries.to(w.dtype))


def new_tokens(w: Workload, step: int = 0) -> tuple[torch.Tensor, torch.Tensor]:
    """The N(0,1) key and value rows of the token a batched decode step
    appends (C4: "the new tokens are N(0,1)"): [batch, KVH, D] each, drawn
    on the CPU from seed ``w.seed + 10000 + step`` and cast to the workload
    dtype."""
    g = torch.Generator().manual_seed(w.seed + 10000 + step)
    shape = (w.batch, w.kv_heads, w.head_dim)
    k = torch.randn(shape, generator=g)
    v = torch.randn(shape, generator=g)
    return k.to(w.dtype), v.to(w.dtype)


def head_to_kv(w: Workload, device=None) -> torch.Tensor:
    return torch.arange(w.q_heads, device=device, dtype=torch.long) // (w.q_heads // w.kv_heads)


def algorithmic_bytes(w: Workload, *, tokens: int | None = None) -> dict[str, int]:
    """Logical HBM bytes per layer step under the reference's cost-model
    convention (estimate_resource_costs.py:113-133, :166-218): each unit
    counted once; gathered K/V rows counted per query head; indices as int32.
      score   KVH*L*(32 + 4R) + QH*L*2  (+ query encode QH*(2D + 8W + 8R))
      select  QH*L*2 + QH*(k+1)*4
      attn    QH*(k+1)*D*2*2 + QH*(k+1)*4 + QH*D*2*2
    """
    L = w.prefix_tokens if tokens is None else tokens
    kk = min(w.budget - 1, L)
    R = w.head_dim // w.dim_group
    W = (w.head_dim + 31) // 32
    esz = 2 if w.dtype != torch.float32 else 4
    score = w.kv_heads * L * (32 + 4 * R) + w.q_heads * L * 2
    encode = w.q_heads * (2 * w.head_dim + 8 * W + 8 * R)
    select = w.q_heads * L * 2 + w.q_heads * (kk + 1) * 4
    attn = (w.q_heads * (kk + 1) * w.head_dim * esz * 2 + w.q_heads * (kk + 1) * 4
            + w.q_heads * w.head_dim * esz * 2)
    prepack = w.kv_heads * L * w.head_dim * esz + w.kv_heads * L * (32 + 4 * R)
    return {"score": score, "encode": encode, "select": select, "attention": attn,
            "step": score + encode + select + attn, "prepack": prepack}
