#!/usr/bin/env python3
"""Benchmark of the PopKV decode-time retrieval step on one MI355X.

    python bench.py [--steps K] [--warmup W] [--gpus 1]
    python bench.py --copy-calibration     # plain 256 MiB copies (PMC scale)

A "step" is one sparse layer's retrieval step at configuration C1 (PopKV-S,
Llama-3.1-8B shapes: 32 query heads / 8 KV heads, head_dim 128, 32K context,
budget 4096, bf16 K/V): query encode + popcount score over 32767 cached
tokens + per-head top-4095 + current token + 256-token split sparse
attention with the log-sum-exp merge -- one ``popkv_layer_step`` C-ABI call
(four kernels), replayed from a HIP graph.  Inputs are resident in HBM; eight
independent K/V + metadata sets (about 1.1 GB) rotate so the 256 MB MALL
cannot hold the working set.

Prints ONE JSON line: µs per layer step (lower is better), the achieved
algorithmic HBM GB/s of the step, per-stage kernel times of the layer step
(HIP events recorded between its kernels), the roofline of the dominant
kernel (the layer step's sparse attention) and a CPU baseline (the C oracle,
one thread, on a bounded sample of the same workload).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "µs/layer score+top-k+sparse-attn @32K ctx, B=4096; achieved HBM GB/s"
HBM_PEAK_GBPS = 8000.0
N_BUFFERS = 8
# HBM bytes per launch of the layer step's attention kernel at C1, from
# rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE runs of this script (KiB per
# dispatch), each scaled by the same counter on a plain 256 MiB copy
# (bench.py --copy-calibration): FETCH_SIZE reads 131084.5 KiB for the copy's
# 262144 KiB (x 1.99981), WRITE_SIZE reads 262144.0 KiB (x 1.0).  Attention:
# FETCH_SIZE 28020.6 KiB, WRITE_SIZE 272.0 KiB per dispatch.
ATTN_TRAFFIC_BYTES = round(28020.6 * 1024 * (262144 / 131084.5) + 272.0 * 1024)


def parse_args():
    p = argparse.ArgumentParser(description=__doc__.splitlines()[1])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=400)
    p.add_argument("--warmup", type=int, default=40)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--cpu-seconds", type=float, default=10.0, help="CPU-baseline time budget")
    p.add_argument("--no-graph", action="store_true", help="time eager launches only")
    p.add_argument("--copy-calibration", action="store_true",
                   help="run plain 256 MiB device copies (scale for rocprofv3 FETCH_SIZE / WRITE_SIZE)")
    return p.parse_args()


def copy_calibration(steps: int) -> int:
    """torch's device-to-device copy of a 256 MiB buffer, `steps` times: a
    kernel of known HBM traffic (256 MiB read + 256 MiB written per dispatch)
    that rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE runs scale against."""
    import torch

    n = 256 << 20
    src = torch.empty(n, dtype=torch.uint8, device="cuda").random_(0, 255)
    dst = torch.empty_like(src)
    for _ in range(steps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes": n, "dispatches": steps}), flush=True)
    return 0


def main() -> int:
    args = parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: the PopKV retrieval path is built and timed on a single "
              "MI355X (multi-GPU sharding is a design note only); run with --gpus 1", file=sys.stderr)
        return 2

    if args.copy_calibration:
        return copy_calibration(args.steps)

    import torch

    from popkv_amd import popkv, popkv_cuda, sparse_kernels, topk, workloads

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    w = workloads.C1
    L, kk = w.prefix_tokens, w.k
    alg = workloads.algorithmic_bytes(w)

    # ---- inputs: one seeded layer, copied into N_BUFFERS independent sets
    layer = workloads.make_layer(w)
    mapping = workloads.head_to_kv(w, dev)
    q = layer.queries.to(dev)
    cur_k, cur_v = layer.current_k().to(dev), layer.current_v().to(dev)
    sets = []
    for _ in range(N_BUFFERS):
        keys = layer.keys.to(dev)      # static-cache rows [KVH, C, D]; prefix = first L rows
        values = layer.values.to(dev)
        cache = popkv.build_popkv_cache(keys[:, :L], group_size=w.token_group, dim_group_size=w.dim_group,
                                        reserve_tokens=64)
        sets.append((keys[:, :L], values[:, :L], cache))
    ws = popkv.LayerStepWorkspace()
    ws.get(popkv.layer_step_workspace_bytes(w.q_heads, L, w.budget, w.dim_group), dev)
    outs = [torch.empty_like(q) for _ in range(N_BUFFERS)]

    def step(i: int) -> None:
        pk, pv, cache = sets[i % N_BUFFERS]
        popkv.popkv_layer_step(q, cache, pk, pv, cur_k, cur_v, mapping, budget=w.budget, workspace=ws,
                               out=outs[i % N_BUFFERS])

    stream = torch.cuda.current_stream(dev)

    def timed(fn, n: int) -> float:
        """Average ms per call of fn(i) over n calls, HIP events on `stream`."""
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        for i in range(n):
            fn(i)
        b.record(stream)
        torch.cuda.synchronize()
        return a.elapsed_time(b) / n

    # ---- eager layer steps
    for i in range(args.warmup):
        step(i)
    eager_ms = timed(step, args.steps)

    def graph_timed(fn, reps: int):
        """Average ms per call of fn(i), captured N_BUFFERS calls to a HIP
        graph (after a warm-up on a side stream) and replayed `reps` times."""
        g = torch.cuda.CUDAGraph()
        side = torch.cuda.Stream(dev)
        side.wait_stream(stream)
        with torch.cuda.stream(side):
            for i in range(N_BUFFERS):
                fn(i)
        stream.wait_stream(side)
        torch.cuda.synchronize()
        with torch.cuda.graph(g):
            for i in range(N_BUFFERS):
                fn(i)
        for _ in range(2):
            g.replay()
        return timed(lambda i: g.replay(), reps) / N_BUFFERS

    # ---- HIP-graph replay of N_BUFFERS consecutive layer steps
    graph_ms = None
    reps = max(1, args.steps // N_BUFFERS)
    if not args.no_graph:
        eager_out = [o.clone() for o in outs]
        graph_ms = graph_timed(step, reps)
        torch.cuda.synchronize()
        if not all(torch.equal(a, b) for a, b in zip(outs, eager_out)):
            print("graph replay changed the layer outputs", file=sys.stderr)
            return 1
    ms_per_step = graph_ms if graph_ms is not None else eager_ms

    # ---- the dominant kernel alone: the layer step's sparse attention,
    #      re-run on the selection the last step left in the workspace
    #      (popkv_layer_step_attention), timed with HIP events around
    #      back-to-back launches on the step's stream
    def attention_only(i: int) -> None:
        pk, pv, _ = sets[i % N_BUFFERS]
        popkv.popkv_layer_step_attention(q, pk, pv, mapping, budget=w.budget, workspace=ws)

    for i in range(args.warmup):
        attention_only(i)
    attn_step_ms = timed(attention_only, args.steps)

    # ---- prepack of the 32K prefix and the per-token append (re-encode of
    #      the active token group incl. the new token), pack_keys_into into a
    #      scratch copy of the packed cache, replayed from a HIP graph
    prefix0 = sets[0][0].contiguous()
    scratch = tuple(t.clone() for t in sets[0][2].packed)
    sealed = (L // w.token_group) * w.token_group
    active = layer.keys[:, sealed:L + 1].to(dev).contiguous()
    prepack_ms = graph_timed(lambda i: popkv_cuda.pack_keys_into(
        prefix0, scratch, token_offset=0, token_group_size=w.token_group, dim_group_size=w.dim_group), 4)
    append_ms = graph_timed(lambda i: popkv_cuda.pack_keys_into(
        active, scratch, token_offset=sealed, token_group_size=w.token_group, dim_group_size=w.dim_group), reps)
    meta_row = 32 + 4 * (w.head_dim // w.dim_group)
    prepack_bytes = w.kv_heads * L * (w.head_dim * 2 + meta_row)
    append_bytes = w.kv_heads * int(active.shape[1]) * (w.head_dim * 2 + meta_row)

    # ---- reference-API stages (the entry points popkv_cuda / topk /
    #      sparse_kernels expose, same inputs), for comparison with the
    #      reference's per-stage numbers
    stage_timer = timed if args.no_graph else graph_timed
    enc = popkv_cuda.query_encode(q.unsqueeze(0).contiguous(), dim_group_size=w.dim_group)
    score_ms = stage_timer(lambda i: popkv_cuda.score_encoded(enc, sets[i % N_BUFFERS][2].packed, head_to_kv=mapping,
                                                              tokens=L, dim_group_size=w.dim_group), reps)
    scores = popkv_cuda.score_encoded(enc, sets[0][2].packed, head_to_kv=mapping, tokens=L,
                                      dim_group_size=w.dim_group)
    score_bufs = [scores.clone() for _ in range(N_BUFFERS)]
    select_ms = stage_timer(lambda i: topk.select_with_current(score_bufs[i % N_BUFFERS], kk, L + 1), reps)
    indices = topk.select_with_current(scores, kk, L + 1)
    attn_ms = stage_timer(lambda i: sparse_kernels.indexed_attention_split_partial(
        q, sets[i % N_BUFFERS][0], sets[i % N_BUFFERS][1], cur_k, cur_v, indices, mapping, split_tokens=256), reps)
    encode_ms = stage_timer(lambda i: popkv_cuda.query_encode(q.unsqueeze(0).contiguous(),
                                                              dim_group_size=w.dim_group), reps)
    unique_rows = int(sum(torch.unique(indices[h * 4:(h + 1) * 4].flatten()).numel() for h in range(w.kv_heads)))

    step_gbps = alg["step"] / (ms_per_step * 1e-3) / 1e9
    attn_gbps = alg["attention"] / (attn_step_ms * 1e-3) / 1e9
    result = {
        "metric": METRIC,
        "value": round(ms_per_step * 1e3, 3),
        "unit": "us/layer",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 6),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded C1 distribution: outlier-channel K, peaked Q; generated on host, resident in HBM)",
        "config": {"workload": w.name, "method": w.method, "q_heads": w.q_heads, "kv_heads": w.kv_heads,
                   "head_dim": w.head_dim, "context": w.context, "budget": w.budget, "token_group": w.token_group,
                   "dim_group": w.dim_group, "batch": 1, "rotating_buffers": N_BUFFERS,
                   "timing": "hip-graph replay" if graph_ms is not None else "eager"},
        "achieved_GBps": round(step_gbps, 1),
        "step_algorithmic_bytes": alg["step"],
        "eager_us_per_layer": round(eager_ms * 1e3, 3),
        "graph_us_per_layer": None if graph_ms is None else round(graph_ms * 1e3, 3),
        "api_stages_us": {"query_encode": round(encode_ms * 1e3, 3), "score_encoded": round(score_ms * 1e3, 3),
                          "select_with_current": round(select_ms * 1e3, 3),
                          "indexed_attention_split_partial": round(attn_ms * 1e3, 3)},
        "prepack": {"tokens": L, "us": round(prepack_ms * 1e3, 3), "algorithmic_bytes": prepack_bytes,
                    "GBps": round(prepack_bytes / (prepack_ms * 1e-3) / 1e9, 1)},
        "append": {"active_tokens": int(active.shape[1]), "us": round(append_ms * 1e3, 3),
                   "algorithmic_bytes": append_bytes, "GBps": round(append_bytes / (append_ms * 1e-3) / 1e9, 1)},
        "unique_kv_rows_per_step": unique_rows,
        "roofline": {"bound": "hbm", "kernel": "attn_rank_kernel (layer step attention)",
                     "achieved": round(attn_gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(attn_gbps / HBM_PEAK_GBPS, 4), "traffic": ATTN_TRAFFIC_BYTES,
                     "algorithmic_bytes_per_launch": alg["attention"], "avg_launch_us": round(attn_step_ms * 1e3, 3)},
        "cpu_baseline": None,
    }
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(layer, w, args.cpu_seconds)
    print(json.dumps(result), flush=True)
    return 0


def cpu_baseline(layer, w, budget_s: float) -> dict:
    """The C oracle (oracle/popkv_oracle.c, one thread) running the same layer
    step -- fold query encode, GQA popcount scores, top-k select, float64
    attention over the gathered rows -- on the host, repeated until about
    `budget_s` seconds have been spent; the median step time is reported."""
    import numpy as np

    from oracle import core
    from popkv_amd import workloads

    L = w.prefix_tokens
    keys = layer.keys.float().numpy()
    values = layer.values.float().numpy()
    q = layer.queries.float().numpy()
    h2k = workloads.head_to_kv(w).numpy()
    packed = core.pack_keys(np.ascontiguousarray(keys[:, :L]), token_group_size=w.token_group,
                            dim_group_size=w.dim_group)
    pk, pv = np.ascontiguousarray(keys[:, :L]), np.ascontiguousarray(values[:, :L])
    ck, cv = keys[:, L].copy(), values[:, L].copy()
    times = []
    t_end = time.perf_counter() + budget_s
    while not times or (time.perf_counter() < t_end and len(times) < 200):
        t0 = time.perf_counter()
        enc = core.query_encode(q[None], w.dim_group, order="fold")
        sc = core.score_encoded(enc, packed, head_to_kv=h2k, tokens=L, dim_group_size=w.dim_group)[0]
        idx = core.select(sc, w.k, L)
        core.attention(q, pk, pv, ck, cv, idx, h2k)
        times.append(time.perf_counter() - t0)
    med = float(np.median(times))
    return {"value": round(med * 1e6, 1), "unit": "us/layer", "cores": 1, "kind": "port",
            "sample": f"{len(times)} full C1 layer steps (encode+score+select+attention) of the C oracle, "
                      f"one thread, median; host has {os.cpu_count()} logical CPUs"}


if __name__ == "__main__":
    sys.exit(main())
