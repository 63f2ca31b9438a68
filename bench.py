#!/usr/bin/env python3
"""Benchmark of the PopKV decode-time retrieval step on one MI355X.

    python bench.py [--steps K] [--warmup W] [--gpus 1]
    python bench.py --copy-calibration     # plain 256 MiB copies (PMC scale)

A "step" is one sparse layer's retrieval step at configuration C1 (PopKV-S,
Llama-3.1-8B shapes: 32 query heads / 8 KV heads, head_dim 128, 32K context,
budget 4096, bf16 K/V): query encode + popcount score over 32767 cached
tokens + per-head top-4095 + current token + sparse attention over 2048-token
chunks with the log-sum-exp merge -- one ``popkv_layer_step`` C-ABI call
(one kernel launch at C1: the scorer's workgroups hand their keys and
histograms to the select + attention workgroups of the same grid),
replayed from a HIP graph.  Inputs are resident in HBM; eight
independent K/V + metadata sets (about 1.1 GB) rotate so the 256 MB MALL
cannot hold the working set.

Prints ONE JSON line: µs per layer step (lower is better), the achieved
algorithmic HBM GB/s of the step, the roofline of the dominant kernel (the
layer step's single launch where the shape takes it, else its select +
sparse attention kernel), the select + attention kernel timed alone, the
achievable
stream-copy bandwidth, and a CPU baseline (the torch-CPU counterpart of the
reference's readable path on every host thread, a bounded sample of the same
workload).  Beside them: the prepack of the prefix, the standalone append,
one whole decode layer (the step plus the append of the current token, one
``popkv_decode_layer_batched`` call at B = 1) and the reference-API stages.
``value`` is the median of --trials trials, each exactly --steps
consecutive layer steps replayed from one HIP graph.
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "µs/layer score+top-k+sparse-attn @32K ctx, B=4096; achieved HBM GB/s"
HBM_PEAK_GBPS = 8000.0
N_BUFFERS = 8
# HBM bytes per launch at C1, from rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE
# runs of this script (KiB per dispatch, median), each scaled by the same
# counter on a plain 256 MiB copy (bench.py --copy-calibration): FETCH_SIZE
# reads 131083.5 KiB for the copy's 262144 KiB (x 1.99982), WRITE_SIZE
# reads 262144.0 KiB (x 1.0) (profiles/layer_step_c1_hbm_traffic.md).
_FETCH_SCALE = 262144 / 131083.5
# layer_step_fused_kernel (the whole C1 step in one launch): FETCH_SIZE
# 34179.1 KiB, WRITE_SIZE 5007.0 KiB
STEP_TRAFFIC_BYTES = round(34179.1 * 1024 * _FETCH_SCALE + 5007.0 * 1024)
# attn_select_chunk_kernel (the tile-window select + attention, run alone
# by popkv_layer_step_attention): FETCH_SIZE 28707.7 KiB, WRITE_SIZE 260.0 KiB
ATTN_TRAFFIC_BYTES = round(28707.7 * 1024 * _FETCH_SCALE + 260.0 * 1024)


def parse_args():
    p = argparse.ArgumentParser(description=__doc__.splitlines()[1])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=400)
    p.add_argument("--warmup", type=int, default=40)
    p.add_argument("--trials", type=int, default=10, help="timed trials of --steps steps (the median is reported)")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--cpu-seconds", type=float, default=10.0, help="CPU-baseline time budget")
    p.add_argument("--no-graph", action="store_true", help="time eager launches only")
    p.add_argument("--workload", default="c1",
                   help="c1 (default), c3-<context> (PopKV-S context sweep), c2-layer<l> (PopKV-Q layer l), c0, "
                        "c4 (8 sequences x 64K, step = layer step + append), "
                        "c2 (32-layer PopKV-Q stack, layers 0-1 dense)")
    p.add_argument("--copy-calibration", action="store_true",
                   help="run plain 256 MiB device copies (scale for rocprofv3 FETCH_SIZE / WRITE_SIZE)")
    return p.parse_args()


def pick_workload(name: str):
    """The named configuration of workloads.py (C1 is the headline one)."""
    from popkv_amd import workloads

    if name == "c1":
        return workloads.C1
    if name == "c0":
        return workloads.C0
    if name.startswith("c3-"):
        return workloads.c3(int(name[3:]))
    if name.startswith("c2-layer"):
        return workloads.c2_layer(int(name[len("c2-layer"):]))
    raise SystemExit(f"unknown workload {name!r}")


def bench_c2(args) -> int:
    """C2: one decode step through a 32-layer stack at Llama-3.1-8B shapes,
    32K context, budget 4096, bf16.  Layers 0-1 run dense attention over
    all tokens (popkv_dense_attention); layers 2-31 run the PopKV-Q layer
    step (TG 128, G 16).  Each layer has its own K/V, packed cache and query
    (seed 42 + layer); the 32 layers (4.6 GB) rotate through HBM naturally.
    The whole stack is one HIP graph; value = µs per stack step."""
    import torch

    from popkv_amd import popkv, workloads

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    n_layers, dense_layers = 32, (0, 1)
    operands, caches, outs = [], {}, []
    for li in range(n_layers):
        w = workloads.c2_layer(li)
        lay = workloads.make_layer(w).to(dev)
        if li not in dense_layers:
            caches[li] = popkv.build_popkv_cache(lay.prefix_k(), group_size=w.token_group,
                                                 dim_group_size=w.dim_group, reserve_tokens=128)
        operands.append((lay.queries, lay.prefix_k(), lay.prefix_v(), lay.current_k(), lay.current_v()))
        outs.append(torch.empty_like(lay.queries))
    w0 = workloads.c2_layer(0)
    stack = popkv.SparseDecodeStack(caches, workloads.head_to_kv(w0, dev), budget=w0.budget,
                                    full_layers=dense_layers)
    stream = torch.cuda.current_stream(dev)

    def stack_step() -> None:
        stack.step(operands, outs)

    for _ in range(max(1, args.warmup // 8)):
        stack_step()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream(dev)
    side.wait_stream(stream)
    with torch.cuda.stream(side):
        stack_step()
    stream.wait_stream(side)
    torch.cuda.synchronize()
    with torch.cuda.graph(g):
        stack_step()
    g.replay()
    torch.cuda.synchronize()
    # value = the median over trials of `reps` replays each
    reps = max(1, args.steps // 16)
    trial_ms = []
    for _ in range(max(5, args.trials)):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        for _ in range(reps):
            g.replay()
        b.record(stream)
        torch.cuda.synchronize()
        trial_ms.append(a.elapsed_time(b) / reps)
    ms = statistics.median(trial_ms)
    L = w0.prefix_tokens
    sparse_bytes = workloads.algorithmic_bytes(workloads.c2_layer(2))["step"]
    # dense layer: every K/V row of a KV head read once (shared by its GQA
    # group), plus q in / out per query head
    dense_bytes = w0.kv_heads * (L + 1) * w0.head_dim * 2 * 2 + w0.q_heads * w0.head_dim * 2 * 2
    total = (n_layers - len(dense_layers)) * sparse_bytes + len(dense_layers) * dense_bytes
    print(json.dumps({
        "metric": "us per decode step through the 32-layer stack (C2: PopKV-Q, layers 0-1 dense); achieved HBM GB/s",
        "value": round(ms * 1e3, 3), "unit": "us/step", "n_gpus": 1, "steps": reps, "warmup": args.warmup,
        "ms_per_step": round(ms, 6), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16", "data": "synthetic (seeded per layer; outlier-channel K, peaked Q; resident in HBM)",
        "config": {"workload": "C2-popkv-q-32-layers", "layers": n_layers, "dense_layers": list(dense_layers),
                   "q_heads": w0.q_heads, "kv_heads": w0.kv_heads, "head_dim": w0.head_dim, "context": w0.context,
                   "budget": w0.budget, "timing": "hip-graph replay of the stack, median of trials"},
        "step_algorithmic_bytes": total, "achieved_GBps": round(total / (ms * 1e-3) / 1e9, 1),
        "per_layer_us": round(ms * 1e3 / n_layers, 3),
        "trials": {"count": len(trial_ms), "replays_each": reps, "us_min": round(min(trial_ms) * 1e3, 3),
                   "us_max": round(max(trial_ms) * 1e3, 3)},
    }), flush=True)
    return 0


def bench_c4(args) -> int:
    """C4: a batch of 8 independent sequences x 64K context (PopKV-S, budget
    4096, bf16), each with its own static K/V cache [8, 8, rows, 128] and
    packed metadata [8, 8, capacity, .] (popkv_amd.batch).  A step is one
    layer's decode step for the whole batch in one C-ABI call
    (popkv_decode_layer_batched): the batched layer step (encode, score,
    top-k + current, split attention, merge; every sequence at its own
    device-side length) and the fused append (the new token's K/V rows into
    the static caches and the re-encode of each sequence's active token
    group, read in place), the append running in extra workgroups of the
    step's select + attention launch.  The appended (current) token is
    N(0,1) (workloads.new_tokens), the prefixes follow the C1 distribution
    with seed 123 + b.  The replays repeat
    the same token position (the lengths are not advanced inside the timed
    graph; advancing them is one 8-element add per decode step, not per
    layer).  The one-time prepack of the eight 64K prefixes is timed on its
    own.  Two input sets rotate (4.4 GB)."""
    import torch

    from popkv_amd import batch as pb
    from popkv_amd import popkv, workloads

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    w = workloads.C4
    B, L = w.batch, w.prefix_tokens
    rows = L + 1 + 63  # prefix + current token + reserve
    n_sets = 2
    sets = []
    kc0 = torch.empty(B, w.kv_heads, rows, 128, dtype=w.dtype, device=dev)
    vc0 = torch.empty_like(kc0)
    qs = []
    for b in range(B):
        lay = workloads.make_layer(w, seed=w.seed + b)
        kc0[b, :, :L] = lay.keys[:, :L].to(dev)
        vc0[b, :, :L] = lay.values[:, :L].to(dev)
        qs.append(lay.queries)
        del lay
    q = torch.stack(qs).to(dev)
    # the token the timed step appends (and attends as the current one): N(0,1)
    cur_k, cur_v = (t.to(dev) for t in workloads.new_tokens(w, 0))
    for i in range(n_sets):
        kc, vc = (kc0, vc0) if i == 0 else (kc0.clone(), vc0.clone())
        lengths = pb.SequenceLengths.create([L] * B, dev)
        cache = pb.build_batched_popkv_cache(kc, vc, lengths, group_size=w.token_group, dim_group_size=w.dim_group)
        sets.append((cache, lengths, torch.empty_like(q)))
    mapping = workloads.head_to_kv(w, dev)
    ws = popkv.LayerStepWorkspace()
    stream = torch.cuda.current_stream(dev)

    def step(i: int) -> None:
        cache, lengths, out = sets[i % n_sets]
        pb.popkv_layer_step_batched(q, cache, lengths, cur_k, cur_v, mapping, budget=w.budget, workspace=ws,
                                    out=out, append=True)

    def prepack(i: int) -> None:
        cache, lengths, _ = sets[i % n_sets]
        pb.prepack_batched(cache, lengths)

    def graph_ms(fn, reps: int, trials: int = 1) -> float:
        for i in range(n_sets):
            fn(i)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        side = torch.cuda.Stream(dev)
        side.wait_stream(stream)
        with torch.cuda.stream(side):
            for i in range(n_sets):
                fn(i)
        stream.wait_stream(side)
        torch.cuda.synchronize()
        with torch.cuda.graph(g):
            for i in range(n_sets):
                fn(i)
        g.replay()
        torch.cuda.synchronize()
        times = []
        for _ in range(trials):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record(stream)
            for _ in range(reps):
                g.replay()
            b.record(stream)
            torch.cuda.synchronize()
            times.append(a.elapsed_time(b) / (reps * n_sets))
        return statistics.median(times)

    for i in range(args.warmup):
        step(i)
    step_ms = graph_ms(step, max(1, args.steps // n_sets), trials=max(10, args.trials))
    # the one-time prepack of the eight 64K prefixes, into the existing planes: median of 5 trials
    prepack_ms = graph_ms(prepack, 2, trials=5)
    per_seq = workloads.algorithmic_bytes(w)
    meta_row = 32 + 4 * (w.head_dim // w.dim_group)
    active = L % w.token_group + 1  # tokens re-encoded by the append (the new one included)
    append_bytes = B * w.kv_heads * (active * (w.head_dim * 2 + meta_row) + 2 * w.head_dim * 2)
    step_bytes = B * per_seq["step"] + append_bytes
    prepack_bytes = B * per_seq["prepack"]
    print(json.dumps({
        "metric": "us per batched decode step per layer (C4: 8 x 64K, layer step + fused append); achieved HBM GB/s",
        "value": round(step_ms * 1e3, 3), "unit": "us/step-layer", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(step_ms, 6), "higher_is_better": False, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded per sequence; outlier-channel K, peaked Q, N(0,1) decode token; resident in HBM)",
        "config": {"workload": w.name, "method": w.method, "batch": B, "q_heads": w.q_heads, "kv_heads": w.kv_heads,
                   "head_dim": w.head_dim, "context": w.context, "budget": w.budget, "rotating_buffers": n_sets,
                   "timing": "hip-graph replay, median of trials"},
        "step_algorithmic_bytes": step_bytes, "achieved_GBps": round(step_bytes / (step_ms * 1e-3) / 1e9, 1),
        "append": {"active_tokens_per_sequence": active, "algorithmic_bytes": append_bytes},
        "prepack": {"tokens_per_sequence": L, "us": round(prepack_ms * 1e3, 3), "algorithmic_bytes": prepack_bytes,
                    "GBps": round(prepack_bytes / (prepack_ms * 1e-3) / 1e9, 1)},
    }), flush=True)
    return 0


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
    if args.workload == "c4":
        return bench_c4(args)
    if args.workload == "c2":
        return bench_c2(args)

    import torch

    from popkv_amd import _native as nat
    from popkv_amd import popkv, popkv_cuda, sparse_kernels, topk, workloads

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    w = pick_workload(args.workload)
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

    # ---- eager layer steps (reported beside the graph figure)
    for i in range(args.warmup):
        step(i)
    eager_ms = timed(step, args.steps)

    def capture(fn, n: int):
        """fn(0) .. fn(n - 1) recorded into one HIP graph (after a warm-up
        pass on a side stream, as torch's graph capture asks)."""
        g = torch.cuda.CUDAGraph()
        side = torch.cuda.Stream(dev)
        side.wait_stream(stream)
        with torch.cuda.stream(side):
            for i in range(min(n, N_BUFFERS)):
                fn(i)
        stream.wait_stream(side)
        torch.cuda.synchronize()
        with torch.cuda.graph(g):
            for i in range(n):
                fn(i)
        for _ in range(2):
            g.replay()
        torch.cuda.synchronize()
        return g

    def graph_timed(fn, reps: int):
        """Average ms per call of fn(i): N_BUFFERS calls in one HIP graph,
        replayed `reps` times, HIP events on `stream`."""
        g = capture(fn, N_BUFFERS)
        return timed(lambda i: g.replay(), reps) / N_BUFFERS

    # ---- the timed steps: exactly K consecutive layer steps (rotating the
    #      N_BUFFERS input sets) in one HIP graph; each trial replays it once,
    #      bracketed by synchronizations and HIP events on the step's stream;
    #      value = the median trial / K
    graph_ms = None
    trial_ms: list[float] = []
    reps = max(1, args.steps // N_BUFFERS)
    if not args.no_graph:
        eager_out = [o.clone() for o in outs]
        g_steps = capture(step, args.steps)
        for _ in range(max(10, args.trials)):
            trial_ms.append(timed(lambda i: g_steps.replay(), 1) / args.steps)
        graph_ms = statistics.median(trial_ms)
        torch.cuda.synchronize()
        if not all(torch.equal(a, b) for a, b in zip(outs, eager_out)):
            print("graph replay changed the layer outputs", file=sys.stderr)
            return 1
        del g_steps
    ms_per_step = graph_ms if graph_ms is not None else eager_ms

    # ---- the dominant kernel alone: the layer step's fused select +
    #      sparse attention, re-run on the keys and threshold histograms the
    #      last step left in the workspace (popkv_layer_step_attention):
    #      N_BUFFERS launches captured in a HIP graph, replayed, timed with
    #      HIP events on the step's stream (host-side launch cost excluded)
    def attention_only(i: int) -> None:
        pk, pv, _ = sets[i % N_BUFFERS]
        popkv.popkv_layer_step_attention(q, pk, pv, mapping, budget=w.budget, dim_group_size=w.dim_group,
                                         workspace=ws)

    aux_reps = max(reps, 25)  # replays of N_BUFFERS launches for the per-kernel / per-stage figures
    for i in range(args.warmup):
        attention_only(i)
    attn_step_ms = (timed(attention_only, aux_reps * N_BUFFERS) if args.no_graph
                    else graph_timed(attention_only, aux_reps))

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
        active, scratch, token_offset=sealed, token_group_size=w.token_group, dim_group_size=w.dim_group), aux_reps)
    meta_row = 32 + 4 * (w.head_dim // w.dim_group)
    prepack_bytes = w.kv_heads * L * (w.head_dim * 2 + meta_row)
    append_bytes = w.kv_heads * int(active.shape[1]) * (w.head_dim * 2 + meta_row)

    # ---- one whole decode layer: the step plus the append of the current
    #      token (its K/V rows into static caches, its active token group
    #      re-encoded in place), one popkv_decode_layer_batched call at B = 1
    #      whose append runs in extra workgroups of the select + attention
    #      launch; the same N_BUFFERS rotation (the lengths are not advanced,
    #      so every call appends the same token at row L)
    from popkv_amd import batch as pb
    dsets = []
    for pk, pv, _ in sets:
        kc = torch.zeros(1, w.kv_heads, L + 64, w.head_dim, dtype=pk.dtype, device=dev)
        vc = torch.zeros_like(kc)
        kc[0, :, :L] = pk
        vc[0, :, :L] = pv
        lengths1 = pb.SequenceLengths.create([L], dev)
        dsets.append((pb.build_batched_popkv_cache(kc, vc, lengths1, group_size=w.token_group,
                                                   dim_group_size=w.dim_group), lengths1, torch.empty_like(q)[None]))
    dws = popkv.LayerStepWorkspace()
    q1, k1, v1 = q[None].contiguous(), cur_k[None].contiguous(), cur_v[None].contiguous()

    def decode_layer(i: int) -> None:
        cache1, lengths1, out1 = dsets[i % N_BUFFERS]
        pb.popkv_layer_step_batched(q1, cache1, lengths1, k1, v1, mapping, budget=w.budget, workspace=dws,
                                    out=out1, append=True)

    for i in range(N_BUFFERS):
        decode_layer(i)
    decode_ms = timed(decode_layer, aux_reps * N_BUFFERS) if args.no_graph else graph_timed(decode_layer, aux_reps)
    del dsets

    # ---- reference-API stages (the entry points popkv_cuda / topk /
    #      sparse_kernels expose, same inputs), for comparison with the
    #      reference's per-stage numbers
    def stage_timer(fn, n):
        return timed(fn, n * N_BUFFERS) if args.no_graph else graph_timed(fn, n)

    enc = popkv_cuda.query_encode(q.unsqueeze(0).contiguous(), dim_group_size=w.dim_group)
    score_ms = stage_timer(lambda i: popkv_cuda.score_encoded(enc, sets[i % N_BUFFERS][2].packed, head_to_kv=mapping,
                                                              tokens=L, dim_group_size=w.dim_group), aux_reps)
    scores = popkv_cuda.score_encoded(enc, sets[0][2].packed, head_to_kv=mapping, tokens=L,
                                      dim_group_size=w.dim_group)
    score_bufs = [scores.clone() for _ in range(N_BUFFERS)]
    select_ms = stage_timer(lambda i: topk.select_with_current(score_bufs[i % N_BUFFERS], kk, L + 1), aux_reps)
    indices = topk.select_with_current(scores, kk, L + 1)
    attn_ms = stage_timer(lambda i: sparse_kernels.indexed_attention_split_partial(
        q, sets[i % N_BUFFERS][0], sets[i % N_BUFFERS][1], cur_k, cur_v, indices, mapping, split_tokens=256),
        aux_reps)
    encode_ms = stage_timer(lambda i: popkv_cuda.query_encode(q.unsqueeze(0).contiguous(),
                                                              dim_group_size=w.dim_group), aux_reps)
    qpk = w.q_heads // w.kv_heads
    unique_rows = int(sum(torch.unique(indices[h * qpk:(h + 1) * qpk].flatten()).numel() for h in range(w.kv_heads)))

    copy_gbps = stream_copy_gbps(torch, dev, stream)
    step_gbps = alg["step"] / (ms_per_step * 1e-3) / 1e9
    # the select + attention kernel: the attention's bytes plus the select's
    # pass over the key rows
    sel_bytes = alg["attention"] + w.q_heads * L * 2
    sel_gbps = sel_bytes / (attn_step_ms * 1e-3) / 1e9
    es = q.element_size()
    sel_distinct = unique_rows * w.head_dim * es * 2 + w.q_heads * L * 2 + w.q_heads * w.head_dim * es * 2
    # the layer step's launches at this shape: one kernel (scorer and select
    # + attention workgroups in one grid) where 0 < k < L and the tile-window
    # form applies; otherwise the select + attention kernel dominates
    launches = int(nat.lib().popkv_layer_step_launches(w.q_heads, w.kv_heads, L, w.budget, w.dim_group))
    single = launches == 1 and 0 < kk < L
    c1 = w.name == workloads.C1.name  # the PMC traffic figures belong to C1's shape
    if single:
        # one launch per step: its duration is the graph-replayed step time
        roof = {"kernel": "layer_step_fused_kernel (the whole layer step: score, select, sparse attention, merge)",
                "bytes": alg["step"], "us": ms_per_step * 1e3, "traffic": STEP_TRAFFIC_BYTES if c1 else None,
                "distinct": sel_distinct + alg["score"] + alg["encode"]}
    else:
        roof = {"kernel": "attn_select_chunk_kernel (the layer step's select + attention, timed alone)",
                "bytes": sel_bytes, "us": attn_step_ms * 1e3, "traffic": ATTN_TRAFFIC_BYTES if c1 else None,
                "distinct": sel_distinct}
    roof_gbps = roof["bytes"] / (roof["us"] * 1e-6) / 1e9
    traffic = roof["traffic"]
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
        "dtype": {torch.bfloat16: "bf16", torch.float16: "f16", torch.float32: "f32"}[w.dtype],
        "data": ("synthetic (seeded; outlier-channel K, peaked Q; generated on host, resident in HBM)" if w.peaked
                 else "synthetic (seeded i.i.d. N(0,1) K/V/Q; generated on host, resident in HBM)"),
        "config": {"workload": w.name, "method": w.method, "q_heads": w.q_heads, "kv_heads": w.kv_heads,
                   "head_dim": w.head_dim, "context": w.context, "budget": w.budget, "token_group": w.token_group,
                   "dim_group": w.dim_group, "batch": 1, "rotating_buffers": N_BUFFERS,
                   "timing": "hip-graph replay" if graph_ms is not None else "eager"},
        "achieved_GBps": round(step_gbps, 1),
        "step_algorithmic_bytes": alg["step"],
        "step_frac_of_peak": round(step_gbps / HBM_PEAK_GBPS, 4),
        "stream_copy_GBps": round(copy_gbps, 1),
        "step_frac_of_stream_copy": round(step_gbps / copy_gbps, 4),
        "trials": {"count": len(trial_ms), "steps_each": args.steps,
                   "us_min": round(min(trial_ms) * 1e3, 3) if trial_ms else None,
                   "us_median": round(statistics.median(trial_ms) * 1e3, 3) if trial_ms else None,
                   "us_max": round(max(trial_ms) * 1e3, 3) if trial_ms else None},
        "eager_us_per_layer": round(eager_ms * 1e3, 3),
        "graph_us_per_layer": None if graph_ms is None else round(graph_ms * 1e3, 3),
        "api_stages_us": {"query_encode": round(encode_ms * 1e3, 3), "score_encoded": round(score_ms * 1e3, 3),
                          "select_with_current": round(select_ms * 1e3, 3),
                          "indexed_attention_split_partial": round(attn_ms * 1e3, 3)},
        "prepack": {"tokens": L, "us": round(prepack_ms * 1e3, 3), "algorithmic_bytes": prepack_bytes,
                    "GBps": round(prepack_bytes / (prepack_ms * 1e-3) / 1e9, 1)},
        "append": {"active_tokens": int(active.shape[1]), "us": round(append_ms * 1e3, 3),
                   "algorithmic_bytes": append_bytes, "GBps": round(append_bytes / (append_ms * 1e-3) / 1e9, 1)},
        "decode_layer_with_append_us": round(decode_ms * 1e3, 3),
        "unique_kv_rows_per_step": unique_rows,
        "layer_step_launches": launches,
        "roofline": {"bound": "hbm", "kernel": roof["kernel"],
                     "achieved": round(roof_gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(roof_gbps / HBM_PEAK_GBPS, 4), "traffic": traffic,
                     "algorithmic_bytes_per_launch": roof["bytes"], "avg_launch_us": round(roof["us"], 3),
                     # the reference's convention counts every selected (query head, row) once; the heads
                     # of a GQA group share rows, so the kernel's DRAM traffic is lower
                     "algorithmic_convention": "per query head",
                     # the distinct K/V rows the launch gathers (each once) plus its other operands, over
                     # the same time: a bandwidth figure free of the per-head convention
                     "distinct_bytes_per_launch": roof["distinct"],
                     "distinct_GBps": round(roof["distinct"] / (roof["us"] * 1e-6) / 1e9, 1),
                     # DRAM bytes per launch (PMC, measured at C1 only) over the same time
                     "traffic_GBps": None if traffic is None else round(traffic / (roof["us"] * 1e-6) / 1e9, 1),
                     "traffic_frac": None if traffic is None else
                     round(traffic / (roof["us"] * 1e-6) / 1e9 / HBM_PEAK_GBPS, 4)},
        # the select + attention kernel alone (popkv_layer_step_attention: re-run on the keys and
        # thresholds the last step left), the dominant kernel of the multi-launch form
        "select_attention_alone": {"us": round(attn_step_ms * 1e3, 3), "algorithmic_bytes": sel_bytes,
                                   "GBps": round(sel_gbps, 1), "frac": round(sel_gbps / HBM_PEAK_GBPS, 4),
                                   "distinct_GBps": round(sel_distinct / (attn_step_ms * 1e-3) / 1e9, 1),
                                   "traffic": ATTN_TRAFFIC_BYTES if c1 else None},
        "cpu_baseline": None,
    }
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(layer, w, args.cpu_seconds)
    print(json.dumps(result), flush=True)
    return 0


def stream_copy_gbps(torch, dev, stream) -> float:
    """Achievable HBM bandwidth: a plain device-to-device copy of 1 GiB
    (1 GiB read + 1 GiB written per copy), median of 10 event-timed copies."""
    n = 1 << 30
    src = torch.empty(n, dtype=torch.uint8, device=dev).random_(0, 255)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    times = []
    for _ in range(10):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        a.record(stream)
        dst.copy_(src)
        b.record(stream)
        torch.cuda.synchronize()
        times.append(a.elapsed_time(b) * 1e-3)
    del src, dst
    return 2 * n / statistics.median(times) / 1e9


def _cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def cpu_baseline(layer, w, budget_s: float) -> dict:
    """The torch-CPU counterpart of the reference's readable retrieval path
    (oracle/torch_cpu.py: dense-reconstruction scores of the prepacked
    keys, torch.topk + the current token, fp32 attention over the gathered
    rows) on every host thread this process may use: the same C1 layer step,
    2 warm-up steps, then steps until about `budget_s` seconds (at least 5);
    the median step time is reported.  The one-time prefix encode is timed
    separately."""
    import torch

    from oracle import torch_cpu
    from popkv_amd import workloads

    cores = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    prev = torch.get_num_threads()
    torch.set_num_threads(cores)
    try:
        t0 = time.perf_counter()
        cl = torch_cpu.CpuRetrievalLayer(layer.prefix_k(), layer.prefix_v(), workloads.head_to_kv(w),
                                         token_group=w.token_group, dim_group=w.dim_group)
        prepack_s = time.perf_counter() - t0
        q, ck, cv = layer.queries, layer.current_k(), layer.current_v()
        for _ in range(2):
            cl.step(q, ck, cv, w.budget)
        times = []
        t_end = time.perf_counter() + budget_s
        while len(times) < 5 or (time.perf_counter() < t_end and len(times) < 500):
            t0 = time.perf_counter()
            cl.step(q, ck, cv, w.budget)
            times.append(time.perf_counter() - t0)
    finally:
        torch.set_num_threads(prev)
    med = statistics.median(times)
    return {"value": round(med * 1e6, 1), "unit": "us/layer", "cores": cores, "kind": "port",
            "sample": f"{len(times)} full {w.name} layer steps (query encode + dense-reconstruction scores of "
                      f"the prepacked prefix + torch.topk + current token + fp32 attention over the gathered "
                      f"rows), torch-CPU on {cores} threads, median after 2 warm-ups",
            "cpu_model": _cpu_model(), "torch": torch.__version__,
            "host_logical_cpus": os.cpu_count(), "prefix_encode_us": round(prepack_s * 1e6, 1)}


if __name__ == "__main__":
    sys.exit(main())
