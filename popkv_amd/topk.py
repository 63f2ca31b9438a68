"""Per-query-head top-k over fp16 PopKV scores, with the current token
reserving the last slot -- the HIP replacement of the reference's
``torch.topk(scores, k, dim=-1, sorted=False).indices`` + ``_append_current``
(popkv.py:1090-1099, :287-291).

Selection rule (the one the reference inherits from PyTorch's radix select):
the k largest scores in fp16 radix order (-0 < +0, NaN largest); among scores
equal to the k-th largest, the lowest token indices.  Indices are returned in
ascending token order (``sorted=False`` leaves the order unspecified, so any
order is a valid drop-in; ascending order also makes the attention gather
walk K/V memory forward).
"""
from __future__ import annotations

import torch

from . import _native as nat

MAX_SELECT_TOKENS = 524288  # 64 chunks of 8192 tokens (the C ABI checks the same bound)


# Reusable workspaces, one per (device, stream): the native select keeps
# per-row histograms at the start of the workspace (1 KiB per row), needs
# them zero when a call begins and leaves them zero, so a buffer is allocated
# zeroed and only its histogram region is cleared when the row count changes
# (the new region may cover keys a call with fewer rows left there).
_WORKSPACES: dict[tuple[int, int], tuple[torch.Tensor, int]] = {}


def _workspace(device: torch.device, stream: int, nbytes: int, rows: int) -> torch.Tensor:
    key = (device.index if device.index is not None else torch.cuda.current_device(), stream)
    buf, last_rows = _WORKSPACES.get(key, (None, 0))
    if buf is None or buf.numel() < nbytes:
        buf = torch.zeros(max(nbytes, 256), device=device, dtype=torch.uint8)
    elif rows != last_rows:
        buf[: min(buf.numel(), rows * 1024)].zero_()
    _WORKSPACES[key] = (buf, rows)
    return buf


def _launch(scores2d: torch.Tensor, k: int, current: int, out: torch.Tensor) -> None:
    rows, tokens = (int(x) for x in scores2d.shape)
    with torch.cuda.device(scores2d.device):
        stream = nat.stream_of(scores2d.device)
        nbytes = int(nat.lib().popkv_topk_select_workspace_bytes(rows, tokens))
        ws = _workspace(scores2d.device, int(stream or 0), nbytes, rows)
        nat.call("popkv_topk_select", scores2d.data_ptr(), rows, scores2d.stride(0), tokens, int(k), int(current),
                 out.data_ptr(), nat.INDEX_I64 if out.dtype == torch.int64 else nat.INDEX_I32, out.stride(0),
                 ws.data_ptr(), ws.numel(), stream)


def _rows(scores: torch.Tensor) -> torch.Tensor:
    if not scores.is_cuda:
        raise ValueError("scores must be a CUDA tensor")
    if scores.dtype != torch.float16:
        raise ValueError("scores must be float16 (the PopKV scorer's output)")
    if scores.ndim < 1:
        raise ValueError("scores must have a token dimension")
    s = scores.reshape(-1, scores.shape[-1]) if scores.ndim != 2 else scores
    if s.stride(-1) != 1:
        s = s.contiguous()
    return s


def topk_indices(scores: torch.Tensor, k: int) -> torch.Tensor:
    """int64 [..., k] indices of the k largest fp16 scores along the last dim.
    Usable as ``LlamaSparseDecoder.experimental_topk`` (popkv.py:1091-1093)."""
    s = _rows(scores)
    tokens = int(s.shape[-1])
    k = int(k)
    if not 0 <= k <= tokens:
        raise RuntimeError("selected index k out of range")
    out = torch.empty((int(s.shape[0]), k + 1), device=s.device, dtype=torch.int64)
    if s.shape[0] > 0:
        _launch(s, k, tokens, out)
    return out[:, :k].reshape(*scores.shape[:-1], k)


def select_with_current(scores: torch.Tensor, k: int, num_tokens: int) -> torch.Tensor:
    """Fused ``_append_current(topk(scores[0] or scores, k), num_tokens)``.

    scores: fp16 [1, QH, T] or [QH, T]; returns int64 [QH, k+1] whose last
    column is num_tokens - 1 (the current token's index)."""
    s = _rows(scores[0] if scores.ndim == 3 else scores)
    tokens = int(s.shape[-1])
    k = int(k)
    if not 0 <= k <= tokens:
        raise RuntimeError("selected index k out of range")
    out = torch.empty((int(s.shape[0]), k + 1), device=s.device, dtype=torch.int64)
    _launch(s, k, int(num_tokens) - 1, out)
    return out
