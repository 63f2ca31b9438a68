"""torch-CPU counterpart of the reference's readable retrieval path.

TEST INFRASTRUCTURE ONLY: the CPU baseline that ``bench.py`` times beside
the HIP path (and that tests compare against within tolerances); never the
product.  It restates, with plain torch CPU ops on every host thread, the
semantics of the reference's readable functions (popkv.py:462-735):

  * ``key_encode`` / ``query_encode``: ``reference_key_encode`` /
    ``reference_query_encode`` (popkv.py:514-536, :573-596): sign bits,
    magnitude bits against half the token-group (keys) or whole-head
    (queries) extremum, per dimension-group low / high means with the
    empty-bucket rules of ``_reference_representatives`` (popkv.py:474-511);
  * ``scores``: ``popkv_reference_scores`` (popkv.py:655-689), the dense
    reconstruction qhat . khat / sqrt(D), with khat built once per prefix
    (the packed cache is static between appends) and one batched product
    per step;
  * ``select``: ``torch.topk(scores, k, sorted=False)`` followed by
    ``_append_current`` (popkv.py:1094-1098, :287-291);
  * ``attention``: fp32 softmax attention over the gathered rows, as the
    reference's ``materialized_attention`` test helper
    (tests/test_sparse_kernels.py:30-48).

Scores here are fp32 dense reconstructions (the reference's readable
definition), not the production kernel's fp16 popcount bits, so a selected
set can differ from the HIP path's at near-equal scores; it is a timing
baseline of the same work, not a parity oracle.
"""
from __future__ import annotations

import math

import torch


def _representatives(a: torch.Tensor, mag: torch.Tensor, g: int) -> tuple[torch.Tensor, torch.Tensor]:
    """Per dim-group (low, high - low) means of |x| over the non-magnitude /
    magnitude dims; an empty low bucket takes the high mean (0 when both are
    empty), an empty high bucket the low mean (popkv.py:474-511)."""
    d = a.shape[-1]
    reps = math.ceil(d / g)
    pad = reps * g - d
    if pad:
        a = torch.nn.functional.pad(a, (0, pad))
        mag = torch.nn.functional.pad(mag, (0, pad))
        valid = torch.nn.functional.pad(torch.ones(d, dtype=torch.bool), (0, pad))
    else:
        valid = torch.ones(d, dtype=torch.bool)
    a = a.reshape(*a.shape[:-1], reps, g)
    mag = mag.reshape(*mag.shape[:-1], reps, g)
    valid = valid.reshape(reps, g)
    lo_m = ~mag & valid
    hc = mag.sum(-1)
    lc = lo_m.sum(-1)
    hs = (a * mag).sum(-1)
    ls = (a * lo_m).sum(-1)
    high_mean = hs / hc.clamp(min=1)
    low = torch.where(lc > 0, ls / lc.clamp(min=1), torch.where(hc > 0, high_mean, torch.zeros_like(hs)))
    high = torch.where(hc > 0, high_mean, low)
    return low, high - low


def query_encode(q: torch.Tensor, g: int):
    """q [QH, D] fp32 -> (sign, mag) bool [QH, D], (low, delta) [QH, R]."""
    q = q.float()
    mn = q.amin(-1, keepdim=True)
    mx = q.amax(-1, keepdim=True)
    sign = q >= 0
    mag = torch.where(sign, q > mx * 0.5, q < mn * 0.5)
    low, delta = _representatives(q.abs(), mag, g)
    return sign, mag, low, delta


def key_encode(k: torch.Tensor, tg: int, g: int):
    """k [KVH, L, D] -> (sign, mag) bool [KVH, L, D], (low, delta) [KVH, L, R];
    magnitude thresholds per token group of tg tokens (the last one partial)."""
    k = k.float()
    kvh, n, d = k.shape
    full = n // tg * tg
    mn = torch.empty_like(k)
    mx = torch.empty_like(k)
    if full:
        grp = k[:, :full].reshape(kvh, full // tg, tg, d)
        mn[:, :full] = grp.amin(2, keepdim=True).expand_as(grp).reshape(kvh, full, d)
        mx[:, :full] = grp.amax(2, keepdim=True).expand_as(grp).reshape(kvh, full, d)
    if full < n:
        mn[:, full:] = k[:, full:].amin(1, keepdim=True)
        mx[:, full:] = k[:, full:].amax(1, keepdim=True)
    sign = k >= 0
    mag = torch.where(sign, k > mx * 0.5, k < mn * 0.5)
    low, delta = _representatives(k.abs(), mag, g)
    return sign, mag, low, delta


def reconstruct(sign: torch.Tensor, mag: torch.Tensor, low: torch.Tensor, delta: torch.Tensor,
                g: int) -> torch.Tensor:
    """The dense reconstruction xhat = +-(low + mag * delta) per dimension
    (popkv.py:655-689)."""
    d = sign.shape[-1]
    lo = low.repeat_interleave(g, -1)[..., :d]
    hi = (low + delta).repeat_interleave(g, -1)[..., :d]
    return torch.where(sign, 1.0, -1.0) * torch.where(mag, hi, lo)


class CpuRetrievalLayer:
    """One sparse layer's retrieval step on the host: the prefix keys are
    encoded (and their reconstruction khat kept) once; ``step`` runs query
    encode, scores, top-k + current token and the attention."""

    def __init__(self, prefix_k: torch.Tensor, prefix_v: torch.Tensor, head_to_kv: torch.Tensor, *,
                 token_group: int, dim_group: int) -> None:
        self.k = prefix_k.float().contiguous()
        self.v = prefix_v.float().contiguous()
        self.g = dim_group
        self.h2k = head_to_kv.long()
        self.khat = reconstruct(*key_encode(self.k, token_group, dim_group), dim_group)  # [KVH, L, D]
        kvh = self.k.shape[0]
        self.qpk = int(self.h2k.numel()) // kvh

    def step(self, q: torch.Tensor, cur_k: torch.Tensor, cur_v: torch.Tensor, budget: int) -> torch.Tensor:
        """q [QH, D], current k/v [KVH, D] -> attention output [QH, D] (fp32)."""
        qf = q.float()
        kvh, n, d = self.k.shape
        qhat = reconstruct(*query_encode(qf, self.g), self.g)  # [QH, D]
        # GQA groups are contiguous (the scorer's rule): [KVH, QPK, D] x [KVH, D, L]
        scores = torch.bmm(qhat.view(kvh, self.qpk, d), self.khat.transpose(1, 2)) / math.sqrt(d)
        scores = scores.reshape(-1, n).to(torch.float16)
        kk = min(budget - 1, n)
        idx = torch.topk(scores, kk, dim=-1, sorted=False).indices  # [QH, k]
        kvi = self.h2k.view(-1, 1)
        kr = self.k[kvi, idx]  # [QH, k, D]
        vr = self.v[kvi, idx]
        kr = torch.cat([kr, cur_k.float()[self.h2k].unsqueeze(1)], 1)  # the current token, last slot
        vr = torch.cat([vr, cur_v.float()[self.h2k].unsqueeze(1)], 1)
        logits = torch.einsum("hd,htd->ht", qf, kr) / math.sqrt(d)
        p = torch.softmax(logits, -1)
        return torch.einsum("ht,htd->hd", p, vr)
