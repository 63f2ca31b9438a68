"""GPU parity at the benchmark configurations of the north star (C0, C2, C3)
and at every chunk plan of the layer step's select, against the CPU oracle:
prepack bits, fp16 score bits and selected indices bit-exact, attention
within 2e-2 max-abs / 1e-2 relative of the float64 materialized reference
(the reference's own check: tests/test_popkv.py:275-372,
tests/test_sparse_kernels.py:118-140).  Also pins the tie rule against
``torch.topk`` on ROCm at the row shapes where PyTorch takes its multi-block
radix select (the path the reference's decode loop inherits,
popkv.py:1094-1098).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import core
from popkv_amd import _native, popkv, popkv_cuda, topk, workloads

pytestmark = pytest.mark.gpu

DEV = "cuda"
ATTN_ATOL, ATTN_RTOL = 2e-2, 1e-2


def f32(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy()


def bits(t: torch.Tensor) -> np.ndarray:
    t = t.detach().cpu().contiguous()
    if t.dtype in (torch.float16, torch.bfloat16):
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def _packed_np(cache):
    return tuple(bits(t) if t.dtype != torch.int32 else t.cpu().numpy() for t in cache.packed)


def _setup(w, seed=None):
    layer = workloads.make_layer(w, seed=seed).to(DEV)
    mapping = workloads.head_to_kv(w, DEV)
    cache = popkv.build_popkv_cache(layer.prefix_k(), group_size=w.token_group, dim_group_size=w.dim_group,
                                    reserve_tokens=64)
    return layer, mapping, cache


def _oracle(w, layer, mapping, cache):
    """fold encode -> GQA popcount scores -> select -> float64 attention."""
    L = layer.prefix_tokens
    enc = core.query_encode(f32(layer.queries)[None], w.dim_group, order="fold")
    h2k = mapping.cpu().numpy()
    sc = core.score_encoded(enc, _packed_np(cache), head_to_kv=h2k, tokens=L, dim_group_size=w.dim_group)[0]
    idx = core.select(sc, w.k, L)
    out = core.attention(f32(layer.queries), f32(layer.prefix_k()), f32(layer.prefix_v()), f32(layer.current_k()),
                         f32(layer.current_v()), idx, h2k)
    return sc, idx, out


def _assert_attention(got: torch.Tensor, want: np.ndarray) -> None:
    err = np.abs(f32(got) - want)
    assert (err <= ATTN_ATOL + ATTN_RTOL * np.abs(want)).all(), float(err.max())


def _check_full_layer(w, *, seed=None, check_prepack=True, api_path=True):
    """Prepack (bit-exact), the reference-API path (score bits, indices) and
    the fused layer step (indices exact, attention within tolerance)."""
    layer, mapping, cache = _setup(w, seed)
    L = layer.prefix_tokens
    if check_prepack:
        want_pack = core.pack_keys(f32(layer.prefix_k()), token_group_size=w.token_group, dim_group_size=w.dim_group)
        for a, b in zip(_packed_np(cache), want_pack):
            assert np.array_equal(a[:, :L], b)
    sc, idx, out = _oracle(w, layer, mapping, cache)
    if api_path:
        enc = popkv_cuda.query_encode(layer.queries.unsqueeze(0).contiguous(), dim_group_size=w.dim_group)
        scores = popkv_cuda.score_encoded(enc, cache.packed, head_to_kv=mapping, tokens=L, dim_group_size=w.dim_group)
        assert np.array_equal(bits(scores[0]), sc)
        assert np.array_equal(topk.select_with_current(scores, w.k, L + 1).cpu().numpy(), idx)
        o1 = popkv.popkv_retrieval_step(layer.queries, layer.prefix_k(), layer.prefix_v(), layer.current_k(),
                                        layer.current_v(), cache, mapping, budget=w.budget)
        _assert_attention(o1, out)
    o, got = popkv.popkv_layer_step(layer.queries, cache, layer.prefix_k(), layer.prefix_v(), layer.current_k(),
                                    layer.current_v(), mapping, budget=w.budget, return_indices=True)
    assert np.array_equal(got.cpu().numpy(), idx)
    _assert_attention(o, out)
    return layer, mapping, cache, out


# ------------------------------------------------------------------ C0

def test_c0_exact_workload():
    """C0 as specified: one layer, QH 8 / KVH 2, 4096 context, budget 512,
    popkv-normal (TG 32 / G 32), fp32 K/V/Q i.i.d. N(0,1), seed 0."""
    w = workloads.C0
    assert (w.q_heads, w.kv_heads, w.context, w.budget, w.token_group, w.dim_group, w.dtype, w.seed) == \
        (8, 2, 4096, 512, 32, 32, torch.float32, 0)
    _check_full_layer(w)


# ------------------------------------------------------------------ C2

def test_c2_popkv_q_sparse_layer_full_size():
    """A C2 sparse layer at full size: PopKV-Q (TG 128 / G 16), 32K context,
    budget 4096, bf16, seed 42 + 2 (layer 2, the first sparse layer)."""
    w = workloads.c2_layer(2)
    assert (w.token_group, w.dim_group, w.context, w.budget, w.seed) == (128, 16, 32768, 4096, 44)
    _check_full_layer(w)


def test_c2_stack_dense_and_sparse_layers_eager_and_graph():
    """The C2 stack path bench.py captures (SparseDecodeStack): layers 0-1
    dense over every token, layer 2 the PopKV-Q layer step, each against its
    own oracle; then the same step recorded into a HIP graph and replayed
    three times, with eager work and synchronizations between the replays,
    every replay equal to the eager result."""
    n_layers, dense = 3, (0, 1)
    ops, caches, wants = [], {}, []
    for li in range(n_layers):
        w = workloads.c2_layer(li)
        lay = workloads.make_layer(w).to(DEV)
        mapping = workloads.head_to_kv(w, DEV)
        ops.append((lay.queries, lay.prefix_k(), lay.prefix_v(), lay.current_k(), lay.current_v()))
        if li in dense:
            L = lay.prefix_tokens
            idx = np.tile(np.arange(L + 1, dtype=np.int64), (w.q_heads, 1))
            wants.append(core.attention(f32(lay.queries), f32(lay.prefix_k()), f32(lay.prefix_v()),
                                        f32(lay.current_k()), f32(lay.current_v()), idx, mapping.cpu().numpy()))
        else:
            caches[li] = popkv.build_popkv_cache(lay.prefix_k(), group_size=w.token_group,
                                                 dim_group_size=w.dim_group, reserve_tokens=128)
            wants.append(_oracle(w, lay, mapping, caches[li])[2])
    w0 = workloads.c2_layer(0)
    stack = popkv.SparseDecodeStack(caches, workloads.head_to_kv(w0, DEV), budget=w0.budget, full_layers=dense)
    outs = [torch.empty_like(o[0]) for o in ops]
    stack.step(ops, outs)
    torch.cuda.synchronize()
    for got, want in zip(outs, wants):
        _assert_attention(got, want)
    eager = [o.clone() for o in outs]
    stream = torch.cuda.current_stream()
    side = torch.cuda.Stream()
    side.wait_stream(stream)
    with torch.cuda.stream(side):
        stack.step(ops, outs)
    stream.wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        stack.step(ops, outs)
    for rep in range(3):
        for o in outs:
            o.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        for i, (a, b) in enumerate(zip(outs, eager)):
            assert torch.equal(a, b), (rep, i)
        stack.step(ops)  # eager work between replays
        torch.cuda.synchronize()


def _c2_layer_case(li: int, dense: tuple[int, ...]):
    """One C2 layer on the CPU: its bf16 inputs and its oracle -- for a
    dense layer the attention over every token, for a sparse layer the
    oracle's own prepack (bit patterns), selection and attention."""
    w = workloads.c2_layer(li)
    lay = workloads.make_layer(w)
    h2k = workloads.head_to_kv(w).numpy()
    q, pk, pv = f32(lay.queries), f32(lay.prefix_k()), f32(lay.prefix_v())
    ck, cv = f32(lay.current_k()), f32(lay.current_v())
    L = lay.prefix_tokens
    if li in dense:
        idx = np.tile(np.arange(L + 1, dtype=np.int64), (w.q_heads, 1))
        return lay, None, None, core.attention(q, pk, pv, ck, cv, idx, h2k)
    pack = core.pack_keys(pk, token_group_size=w.token_group, dim_group_size=w.dim_group)
    enc = core.query_encode(q[None], w.dim_group, order="fold")
    sc = core.score_encoded(enc, pack, head_to_kv=h2k, tokens=L, dim_group_size=w.dim_group)[0]
    idx = core.select(sc, w.k, L)
    return lay, pack, idx, core.attention(q, pk, pv, ck, cv, idx, h2k)


def test_c2_full_32_layer_stack():
    """C2 as specified: the whole 32-layer decode step (layers 0-1 dense,
    2-31 PopKV-Q: TG 128 / G 16, 32K context, budget 4096, bf16, seed
    42 + layer) through SparseDecodeStack.  Every sparse layer's prepack is
    bit-exact with the oracle's and its indices equal the oracle's; every
    layer's output is within 2e-2 / 1e-2 of its own oracle, eagerly and in a
    captured HIP graph replayed twice."""
    from concurrent.futures import ThreadPoolExecutor

    n_layers, dense = 32, (0, 1)
    with ThreadPoolExecutor(max_workers=8) as pool:  # the C oracle releases the GIL
        cases = list(pool.map(lambda li: _c2_layer_case(li, dense), range(n_layers)))
    w0 = workloads.c2_layer(0)
    mapping = workloads.head_to_kv(w0, DEV)
    ops, caches = [], {}
    for li, (lay, pack, _, _) in enumerate(cases):
        lay = lay.to(DEV)
        ops.append((lay.queries, lay.prefix_k(), lay.prefix_v(), lay.current_k(), lay.current_v()))
        if li not in dense:
            w = workloads.c2_layer(li)
            caches[li] = popkv.build_popkv_cache(lay.prefix_k(), group_size=w.token_group,
                                                 dim_group_size=w.dim_group, reserve_tokens=128)
    stack = popkv.SparseDecodeStack(caches, mapping, budget=w0.budget, full_layers=dense)
    outs = [torch.empty_like(o[0]) for o in ops]
    stack.step(ops, outs)
    torch.cuda.synchronize()
    L = w0.prefix_tokens
    for li, ((_, pack, idx, want), got) in enumerate(zip(cases, outs)):
        _assert_attention(got, want)
        if li in dense:
            continue
        for a, b in zip(_packed_np(caches[li]), pack):
            assert np.array_equal(a[:, :L], b), li
        o, sel = popkv.popkv_layer_step(*ops[li][:1], caches[li], *ops[li][1:], mapping, budget=w0.budget,
                                        return_indices=True)
        assert np.array_equal(sel.cpu().numpy(), idx), li
        assert torch.equal(o, got), li
    eager = [o.clone() for o in outs]
    stream = torch.cuda.current_stream()
    side = torch.cuda.Stream()
    side.wait_stream(stream)
    with torch.cuda.stream(side):
        stack.step(ops, outs)
    stream.wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        stack.step(ops, outs)
    for rep in range(2):
        for o in outs:
            o.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        for i, (a, b) in enumerate(zip(outs, eager)):
            assert torch.equal(a, b), (rep, i)


# ------------------------------------------------------------------ C3

@pytest.mark.parametrize("context", [4096, 8192, 16384, 32768])
def test_c3_context_points(context):
    """C3's contexts up to 32K at full size (PopKV-S, budget 4096, seed 7):
    at 4096 the budget covers every cached token (k = L, select-all); 32768
    is C1's shape at C3's seed."""
    w = workloads.c3(context)
    assert w.seed == 7 and w.budget == 4096
    if context == 4096:
        assert w.k == w.prefix_tokens
    _check_full_layer(w, check_prepack=context != 16384)


# ------------------------------------------------------------------ chunk plans

def _step_kpt(tokens: int, k: int, rows: int = 32) -> int:
    """Keys per thread of the layer step's chunked select: the plan of
    step_chunks() in csrc/select_common.h (chunks of 256 * kpt tokens holding
    about 256 selected tokens each, small enough that rows * chunks reaches
    256 blocks, at most 64 chunks)."""
    kpts = (1, 2, 4, 6, 8, 12, 16, 24, 32)
    want = tokens * 256 // k if k > 0 else tokens
    if rows < 256:
        want = min(want, tokens * rows // 256)
    want = max(want, (tokens + 63) // 64)
    kpt = 1
    for x in kpts:
        if x * 256 <= want:
            kpt = x
    while kpt < 32 and -(-tokens // (kpt * 256)) > 64:
        kpt = min(x for x in kpts if x > kpt)
    return kpt


@pytest.mark.parametrize("context,budget,kpt", [(3001, 2001, 1), (8192, 4096, 2), (16384, 4096, 4),
                                                (28001, 4096, 6), (32768, 2501, 12), (65536, 2501, 24)])
def test_layer_step_every_chunk_plan(context, budget, kpt):
    """Each keys-per-thread instantiation of the chunk-histogram and the
    fused select + attention kernels that the other tests leave out (8, 16
    and 32 run at C1, 64K and 128K)."""
    w = workloads.scaled(workloads.C1, context=context, budget=budget)
    assert _step_kpt(w.prefix_tokens, w.k) == kpt
    _check_full_layer(w, seed=300 + kpt, check_prepack=False, api_path=False)


@pytest.mark.parametrize("context,ramp", [(32768, 4.0), (16384, 0.35), (16384, 8.0)])
def test_layer_step_tile_windows_that_miss_the_threshold(context, ramp):
    """Keys scaled by a ramp along the tokens (1 + ramp * t / L), so the
    scorer's per-tile estimates of a row's threshold bin drift away from
    the row's own: many tiles' windows miss it (ramp 4) or a few do (ramp
    0.35), and the select histograms those tiles from their keys.
    Indices exact and attention within tolerance against the oracle."""
    w = workloads.scaled(workloads.C1, context=context, budget=min(4096, context // 2))
    layer = workloads.make_layer(w, seed=900 + context)
    scale = (1.0 + ramp * torch.arange(context, dtype=torch.float32) / context)[None, :, None]
    layer = workloads.LayerInputs((layer.keys.float() * scale).to(w.dtype), layer.values, layer.queries)
    layer = layer.to(DEV)
    mapping = workloads.head_to_kv(w, DEV)
    cache = popkv.build_popkv_cache(layer.prefix_k(), group_size=w.token_group, dim_group_size=w.dim_group,
                                    reserve_tokens=64)
    sc, idx, out = _oracle(w, layer, mapping, cache)
    o, got = popkv.popkv_layer_step(layer.queries, cache, layer.prefix_k(), layer.prefix_v(), layer.current_k(),
                                    layer.current_v(), mapping, budget=w.budget, return_indices=True)
    assert np.array_equal(got.cpu().numpy(), idx)
    _assert_attention(o, out)


# ------------------------------------------------------------------ tie rule vs torch.topk

def _tie_rows(kind: str, rows: int, tokens: int, seed: int) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    if kind == "ties":
        x = torch.randint(-3, 4, (rows, tokens), generator=g).float()
    elif kind == "two_values":
        x = torch.where(torch.rand(rows, tokens, generator=g) < 0.5, 1.0, 2.0)
    elif kind == "signed_zero":
        x = torch.where(torch.rand(rows, tokens, generator=g) < 0.5, -0.0, 0.0)
    else:  # peaked scores with a NaN row and a row of few distinct values
        x = torch.randn(rows, tokens, generator=g) * 0.5
        x[:, ::97] += 4.0
        x[3, ::37] = float("nan")
        x[5] = torch.randint(0, 2, (tokens,), generator=g).float()
    return x.to(torch.float16).to(DEV)


@pytest.mark.parametrize("tokens", [32767, 131071])
@pytest.mark.parametrize("kind", ["ties", "two_values", "signed_zero", "nan"])
def test_tie_rule_matches_torch_topk_multi_block(kind, tokens):
    """32 rows of 32767 and 131071 tokens: the shapes of the reference's
    decode loop, where torch.topk takes its multi-block radix select.  The
    selected sets equal PyTorch's for k = 1, 100, 4095 and 16383 (fewer NaNs
    than k and more; ties cut inside one token chunk and across chunks)."""
    s = _tie_rows(kind, 32, tokens, seed=tokens % 1000 + len(kind))
    for k in (1, 100, 4095, 16383):
        ours = topk.topk_indices(s, k).cpu().numpy()
        ref = torch.topk(s, k, dim=-1, sorted=False).indices.cpu().numpy()
        for r in range(s.shape[0]):
            assert set(ours[r].tolist()) == set(ref[r].tolist()), (kind, tokens, k, r)
        want = core.select(bits(s), k, tokens)
        assert np.array_equal(topk.select_with_current(s, k, tokens + 1).cpu().numpy(), want)


# ------------------------------------------------------------------ wire format

def test_packed_metadata_hand_off_through_the_wire_format():
    """Prefill -> decode hand-off: a cache prepacked on the GPU is
    serialized (popkv_amd.wire), loaded back onto the device, and the layer
    step over it gives the same output and selection; appends then resume
    from the transported active keys, bit-exact with the oracle."""
    from popkv_amd import wire

    w = workloads.scaled(workloads.C1, context=5000, budget=1024)
    layer, mapping, cache = _setup(w)
    blob = wire.to_bytes(cache)
    back = wire.from_bytes(blob, device=DEV)
    args = (layer.prefix_k(), layer.prefix_v(), layer.current_k(), layer.current_v(), mapping)
    o1, i1 = popkv.popkv_layer_step(layer.queries, cache, *args, budget=w.budget, return_indices=True)
    o2, i2 = popkv.popkv_layer_step(layer.queries, back, *args, budget=w.budget, return_indices=True)
    assert torch.equal(i1, i2) and torch.equal(o1, o2)
    keys = layer.prefix_k()
    for step in range(3):
        new = torch.randn(w.kv_heads, 1, 128, generator=torch.Generator().manual_seed(step)).to(w.dtype).to(DEV)
        popkv.append_popkv(back, new)
        keys = torch.cat([keys, new], 1)
        n = keys.shape[1]
        want = core.pack_keys(f32(keys), token_group_size=w.token_group, dim_group_size=w.dim_group)
        for a, b in zip(_packed_np(back), want):
            assert np.array_equal(a[:, :n], b)


@pytest.mark.parametrize("g", [16, 32, 64])
def test_permuted_head_mapping(g):
    """A head_to_kv that is not the plain grouping (group j reads KV head
    7 - j): the scorer reads the mapped rows, and the scores, indices and
    attention follow the mapping exactly as the oracle does."""
    base = workloads.scaled(workloads.C1, context=5000, budget=700)
    w = workloads.Workload(base.name, base.method, 32, 8, 128, 5000, 700, 64 if g == 64 else 128, g,
                           torch.bfloat16, 31 + g, True)
    layer, _, cache = _setup(w)
    mapping = (7 - torch.arange(32, device=DEV) // 4).to(torch.int64)
    sc, idx, out = _oracle(w, layer, mapping, cache)
    enc = popkv_cuda.query_encode(layer.queries.unsqueeze(0).contiguous(), dim_group_size=g)
    scores = popkv_cuda.score_encoded(enc, cache.packed, head_to_kv=mapping, tokens=layer.prefix_tokens,
                                      dim_group_size=g)
    assert np.array_equal(bits(scores[0]), sc)
    o, got = popkv.popkv_layer_step(layer.queries, cache, layer.prefix_k(), layer.prefix_v(), layer.current_k(),
                                    layer.current_v(), mapping, budget=w.budget, return_indices=True)
    assert np.array_equal(got.cpu().numpy(), idx)
    _assert_attention(o, out)



def test_single_launch_with_more_scorer_workgroups_than_cus():
    """The single-launch layer step with 128 query heads over 32 KV heads at
    16K: 512 scorer workgroups (two per CU of the MI355X's 256) ahead of
    1024 select + attention workgroups in one grid.  The select workgroups
    are dispatched only after every scorer workgroup, so the later ones
    still run to their hand-off; indices exact and attention within
    tolerance against the oracle."""
    w = workloads.Workload("wide", "popkv-s", 128, 32, 128, 16384, 2048, 64, 64, torch.bfloat16, 4242, True)
    assert int(_native.lib().popkv_layer_step_launches(w.q_heads, w.kv_heads, w.prefix_tokens, w.budget,
                                                      w.dim_group)) == 1
    layer, mapping, cache = _setup(w)
    sc, idx, out = _oracle(w, layer, mapping, cache)
    o, got = popkv.popkv_layer_step(layer.queries, cache, layer.prefix_k(), layer.prefix_v(), layer.current_k(),
                                    layer.current_v(), mapping, budget=w.budget, return_indices=True)
    assert np.array_equal(got.cpu().numpy(), idx)
    _assert_attention(o, out)


@pytest.mark.parametrize("q_heads,kv_heads,context,budget", [(12, 4, 6000, 700), (24, 8, 7000, 1100),
                                                             (40, 8, 3000, 500)])
def test_layer_step_head_ratios_and_chunk_counts_not_powers_of_two(q_heads, kv_heads, context, budget):
    """GQA groups of 3 and 5 query heads and chunk counts that are not powers
    of two: the block -> (chunk, head) and (sequence, group) divisions take
    their general path (the power-of-two ones are shifts); scores, indices
    and attention against the oracle."""
    w = workloads.Workload("ratio", "popkv-s", q_heads, kv_heads, 128, context, budget, 64, 64, torch.bfloat16,
                           q_heads + context, True)
    layer, mapping, cache = _setup(w)
    sc, idx, out = _oracle(w, layer, mapping, cache)
    o, got = popkv.popkv_layer_step(layer.queries, cache, layer.prefix_k(), layer.prefix_v(), layer.current_k(),
                                    layer.current_v(), mapping, budget=w.budget, return_indices=True)
    assert np.array_equal(got.cpu().numpy(), idx)
    err = np.abs(f32(o) - out)
    assert (err <= ATTN_ATOL + ATTN_RTOL * np.abs(out)).all(), float(err.max())
