"""Decode timing support: the reference's ``DecodeEventPool``
(decode_runtime.py:7-35) and a stage timer over it.

HIP events (``torch.cuda.Event`` on ROCm) are created and recorded once up
front so that timing a decode step never creates events or triggers lazy
runtime initialization inside the measured region.
"""
from __future__ import annotations

import torch


class DecodeEventPool:
    """Create and initialize timing events before measuring any decode token.

    One decoder owns one pool and executes tokens sequentially; the caller
    waits for the final event before a subsequent token reuses the handles.
    """

    def __init__(self, device: torch.device, capacity: int) -> None:
        self.device = device
        self.events = []
        with torch.cuda.device(device):
            stream = torch.cuda.current_stream(device)
            for _ in range(capacity):
                event = torch.cuda.Event(enable_timing=True)
                event.record(stream)  # force the runtime's lazy initialization
                self.events.append(event)
            stream.synchronize()
        self.cursor = 0

    def reset(self) -> None:
        self.cursor = 0

    def record(self):
        if self.cursor >= len(self.events):
            raise RuntimeError("decode event pool exhausted; increase reserved capacity")
        event = self.events[self.cursor]
        self.cursor += 1
        event.record(torch.cuda.current_stream(self.device))
        return event


RETRIEVAL_STAGES = (
    "retrieval_query_encode", "retrieval_score", "topk",
    "sparse_attention_partial", "sparse_attention_merge",
)


class StageTimer:
    """Mutually exclusive stage intervals from pooled events, read once at
    finish() -- the retrieval-stage subset of the reference's
    _DecodeStageTimer (popkv.py:145-206)."""

    def __init__(self, pool: DecodeEventPool, stages=RETRIEVAL_STAGES) -> None:
        self.pool = pool
        self.stages = tuple(stages)
        self.pool.reset()
        self.segments: list[tuple[str, object, object]] = []
        self.start = self.last = self.pool.record()

    def mark(self, name: str) -> None:
        if name not in self.stages:
            raise ValueError(f"unknown decode stage: {name}")
        end = self.pool.record()
        self.segments.append((name, self.last, end))
        self.last = end

    def finish(self) -> dict[str, float]:
        self.last.synchronize()
        totals = {name: 0.0 for name in self.stages}
        for name, a, b in self.segments:
            totals[name] += float(a.elapsed_time(b))
        totals["total"] = float(self.start.elapsed_time(self.last))
        return totals
