"""Batched decode with in-place cache maintenance on the GPU, against the
CPU oracle.

  * The fused append (popkv_append) re-encodes each sequence's active token
    group from the static K cache in place; the packed planes stay
    bit-exact with the oracle's prefix encode of the whole sequence across
    every token-group boundary (the reference's incremental == prefix test,
    tests/test_popkv.py:354-372, at TG 8..128 and G 16/32/64), and the new
    K/V rows land in the static caches.
  * The batched layer step (popkv_layer_step_batched) serves sequences of
    different lengths in one call; each sequence's indices equal its own
    oracle's and its attention is within 2e-2 / 1e-2 -- before and after an
    append, and for a decode step captured once in a HIP graph and replayed
    while the device lengths grow.
  * C4 as specified: eight 64K sequences with N(0,1) decode tokens, each
    checked against its own oracle after an append and a decode layer.
  * A captured decode layer replayed past its launch bound reports it in
    its status word.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import core
from popkv_amd import batch as pb
from popkv_amd import workloads

pytestmark = pytest.mark.gpu

DEV = "cuda"
ATTN_ATOL, ATTN_RTOL = 2e-2, 1e-2


def f32(t):
    return t.detach().float().cpu().numpy()


def bits(t):
    t = t.detach().cpu().contiguous()
    if t.dtype in (torch.float16, torch.bfloat16):
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def _packed_np(cache, b):
    return tuple(bits(t[b]) if t.dtype != torch.int32 else t[b].cpu().numpy() for t in cache.packed)


def _seq_data(batch, kv_heads, rows, seed, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    k = torch.randn(batch, kv_heads, rows, 128, generator=g).to(dtype)
    v = torch.randn(batch, kv_heads, rows, 128, generator=g).to(dtype)
    return k, v


@pytest.mark.parametrize("tg", [8, 16, 32, 64, 128])
def test_fused_append_crosses_every_token_group_boundary(tg):
    """Three sequences starting at TG-2, 3TG-1 and 2TG tokens; three
    appends seal a group, fill one and start new ones.  After every append
    each sequence's packed rows equal the oracle's prefix encode of its
    whole key sequence, bit for bit, and the static caches hold the new
    rows."""
    starts = [tg - 2, 3 * tg - 1, 2 * tg]
    rows = 3 * tg + 8
    for g in (16, 32, 64):
        keys, values = _seq_data(3, 2, rows, seed=70 + tg + g)
        kc = torch.zeros(3, 2, rows, 128, dtype=torch.bfloat16, device=DEV)
        vc = torch.zeros_like(kc)
        for b, n in enumerate(starts):
            kc[b, :, :n] = keys[b, :, :n].to(DEV)
            vc[b, :, :n] = values[b, :, :n].to(DEV)
        lengths = pb.SequenceLengths.create(starts, DEV)
        cache = pb.build_batched_popkv_cache(kc, vc, lengths, group_size=tg, dim_group_size=g)
        status = torch.zeros(1, dtype=torch.int32, device=DEV)
        for step in range(3):
            cur = lengths.host
            nk = torch.stack([keys[b, :, cur[b]] for b in range(3)]).to(DEV)
            nv = torch.stack([values[b, :, cur[b]] for b in range(3)]).to(DEV)
            pb.append_batched(cache, lengths, nk, nv, status=status)
            lengths.advance()
            torch.cuda.synchronize()
            for b in range(3):
                n = lengths.host[b]
                want = core.pack_keys(f32(keys[b, :, :n]), token_group_size=tg, dim_group_size=g)
                for a, w in zip(_packed_np(cache, b), want):
                    assert np.array_equal(a[:, :n], w), (tg, g, step, b)
                assert torch.equal(kc[b, :, n - 1].cpu(), keys[b, :, n - 1])
                assert torch.equal(vc[b, :, n - 1].cpu(), values[b, :, n - 1])
        assert int(status.item()) == 0


def test_fused_append_full_sequence_is_refused():
    kc = torch.zeros(2, 2, 16, 128, dtype=torch.bfloat16, device=DEV)
    lengths = pb.SequenceLengths.create([16, 3], DEV)
    cache = pb.build_batched_popkv_cache(kc, kc.clone(), lengths, group_size=8, dim_group_size=32)
    nk = torch.zeros(2, 2, 128, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(RuntimeError, match="reserve exhausted"):
        pb.append_batched(cache, lengths, nk, nk)
    # the device check: a count the host mirror does not know about
    status = torch.zeros(1, dtype=torch.int32, device=DEV)
    lengths.host = [3, 3]
    before = cache.key_cache.clone()
    pb.append_batched(cache, lengths, nk + 1, nk + 1, status=status)
    torch.cuda.synchronize()
    assert int(status.item()) == 1
    assert torch.equal(cache.key_cache[0], before[0])  # the full sequence is untouched
    assert torch.equal(cache.key_cache[1, :, 3].float().cpu(), torch.ones(2, 128))


def _oracle_seq(q, kc, vc, ck, cv, cache, b, n, mapping, budget, g):
    """Oracle of one sequence of the batch at n cached tokens, from the
    static rows alone (its own prefix encode, not the GPU's planes: an
    append re-encodes the active group's earlier rows too)."""
    h2k = mapping.cpu().numpy()
    enc = core.query_encode(f32(q[b])[None], g, order="fold")
    pk = core.pack_keys(f32(kc[b, :, :n]), token_group_size=cache.group_size, dim_group_size=g)
    sc = core.score_encoded(enc, pk, head_to_kv=h2k, tokens=n, dim_group_size=g)[0]
    kk = min(budget - 1, n)
    idx = core.select(sc, kk, n)
    out = core.attention(f32(q[b]), f32(kc[b, :, :n]), f32(vc[b, :, :n]), f32(ck[b]), f32(cv[b]), idx, h2k)
    return idx, out


def _assert_attention(got, want):
    err = np.abs(f32(got) - want)
    assert (err <= ATTN_ATOL + ATTN_RTOL * np.abs(want)).all(), float(err.max())


def _check_batch(q, cache, lengths, ck, cv, mapping, budget, out, idx, check=None):
    for b in (range(lengths.batch) if check is None else check):
        n = lengths.host[b]
        want_idx, want_out = _oracle_seq(q, cache.key_cache, cache.value_cache, ck, cv, cache, b, n, mapping,
                                         budget, cache.dim_group_size)
        kk = min(budget - 1, n)
        assert np.array_equal(idx[b, :, :kk + 1].cpu().numpy(), want_idx), (b, n)
        _assert_attention(out[b], want_out)


@pytest.mark.parametrize("g,tg", [(64, 64), (16, 128), (32, 32)])
def test_batched_layer_step_ragged_lengths(g, tg):
    """Sequences of 5000, 3001, 700 (budget covers it: select-all), 7777 and
    0 cached tokens in one call; then each appends a token and the step runs
    again at the new lengths."""
    starts = [5000, 3001, 700, 7777, 0]
    batch, qh, kvh, rows, budget = len(starts), 32, 8, 7800, 1024
    keys, values = _seq_data(batch, kvh, rows, seed=g + tg)
    kc, vc = keys.to(DEV), values.to(DEV)
    gq = torch.Generator().manual_seed(5)
    lengths = pb.SequenceLengths.create(starts, DEV)
    cache = pb.build_batched_popkv_cache(kc, vc, lengths, group_size=tg, dim_group_size=g)
    mapping = torch.arange(qh, device=DEV) // (qh // kvh)
    ws = pb.LayerStepWorkspace()
    for step in range(2):
        q = torch.randn(batch, qh, 128, generator=gq).to(torch.bfloat16).to(DEV)
        ck = torch.randn(batch, kvh, 128, generator=gq).to(torch.bfloat16).to(DEV)
        cv = torch.randn(batch, kvh, 128, generator=gq).to(torch.bfloat16).to(DEV)
        out, idx = pb.popkv_layer_step_batched(q, cache, lengths, ck, cv, mapping, budget=budget, workspace=ws,
                                               return_indices=True)
        _check_batch(q, cache, lengths, ck, cv, mapping, budget, out, idx)
        out2 = pb.popkv_layer_step_batched(q, cache, lengths, ck, cv, mapping, budget=budget, workspace=ws)
        assert torch.equal(out2, out)
        pb.append_batched(cache, lengths, ck, cv)
        lengths.advance()


@pytest.mark.parametrize("append", [False, True])
def test_batched_step_within_budget_and_past_it(append):
    """A batch whose every sequence is within the budget (lengths 700, 1, 0,
    1022 at budget 1024: the launch bound 1022 <= k, so the scorer and the
    chunk histograms are skipped and every sequence selects all its tokens),
    then a batch past it on the same workspace (the scorer runs), then the
    first again: each call against the oracle; with the fused append, the
    new rows and the re-encoded planes too."""
    qh, kvh, rows, budget, g, tg = 32, 8, 3000, 1024, 64, 64
    mapping = torch.arange(qh, device=DEV) // (qh // kvh)
    ws = pb.LayerStepWorkspace()
    runs = []
    for starts, seed in (([700, 1, 0, 1022], 91), ([2900, 1, 0, 1500], 92)):
        keys, values = _seq_data(len(starts), kvh, rows, seed=seed)
        kc, vc = keys.to(DEV), values.to(DEV)
        lengths = pb.SequenceLengths.create(starts, DEV)
        cache = pb.build_batched_popkv_cache(kc, vc, lengths, group_size=tg, dim_group_size=g)
        gq = torch.Generator().manual_seed(seed)
        q = torch.randn(len(starts), qh, 128, generator=gq).to(torch.bfloat16).to(DEV)
        ck = torch.randn(len(starts), kvh, 128, generator=gq).to(torch.bfloat16).to(DEV)
        cv = torch.randn(len(starts), kvh, 128, generator=gq).to(torch.bfloat16).to(DEV)
        runs.append((cache, lengths, q, ck, cv))
    for cache, lengths, q, ck, cv in (runs[0], runs[1], runs[0]):
        out, idx = pb.popkv_layer_step_batched(q, cache, lengths, ck, cv, mapping, budget=budget, workspace=ws,
                                               return_indices=True, append=append)
        _check_batch(q, cache, lengths, ck, cv, mapping, budget, out, idx)
        if append:
            for b, n in enumerate(lengths.host):
                assert torch.equal(cache.key_cache[b, :, n], ck[b]) and torch.equal(cache.value_cache[b, :, n], cv[b])
                want = core.pack_keys(f32(cache.key_cache[b, :, :n + 1]), token_group_size=tg, dim_group_size=g)
                for a, w in zip(_packed_np(cache, b), want):
                    assert np.array_equal(a[:, :n + 1], w), (b, n)


@pytest.mark.parametrize("starts", [[3000, 1500, 2200], [300, 150, 220]])
def test_batched_step_graph_replays_follow_growing_lengths(starts):
    """One decode step -- layer step, fused append, lengths += 1 -- captured
    once in a HIP graph, then replayed three times with new tokens copied in
    between: every replay's output and indices match the oracle at that
    replay's lengths (the counts are read on the device).  The second batch
    stays within the budget, so the captured step has no scorer launch."""
    batch, qh, kvh, budget, g, tg = 3, 32, 8, 512, 64, 64
    rows = max(starts) + 100
    keys, values = _seq_data(batch, kvh, rows, seed=17)
    kc = torch.zeros(batch, kvh, rows, 128, dtype=torch.bfloat16, device=DEV)
    vc = torch.zeros_like(kc)
    for b, n in enumerate(starts):
        kc[b, :, :n] = keys[b, :, :n].to(DEV)
        vc[b, :, :n] = values[b, :, :n].to(DEV)
    lengths = pb.SequenceLengths.create(starts, DEV)
    cache = pb.build_batched_popkv_cache(kc, vc, lengths, group_size=tg, dim_group_size=g)
    mapping = torch.arange(qh, device=DEV) // (qh // kvh)
    ws = pb.LayerStepWorkspace()
    gq = torch.Generator().manual_seed(8)
    q = torch.empty(batch, qh, 128, dtype=torch.bfloat16, device=DEV)
    ck = torch.empty(batch, kvh, 128, dtype=torch.bfloat16, device=DEV)
    cv = torch.empty_like(ck)
    out = torch.empty_like(q)
    bound = max(starts) + 8
    idx = torch.empty(batch, qh, min(budget - 1, bound) + 1, dtype=torch.int64, device=DEV)

    def step():
        o, i = pb.popkv_layer_step_batched(q, cache, lengths, ck, cv, mapping, budget=budget, max_tokens=bound,
                                           workspace=ws, out=out, return_indices=True)
        idx.copy_(i)
        pb.append_batched(cache, lengths, ck, cv)
        lengths.device.add_(1)

    def next_token(r):
        q.copy_(torch.randn(batch, qh, 128, generator=gq).to(torch.bfloat16))
        ck.copy_(torch.stack([keys[b, :, lengths.host[b]] for b in range(batch)]))
        cv.copy_(torch.stack([values[b, :, lengths.host[b]] for b in range(batch)]))

    # warm-up on a side stream (it advances the lengths once), then capture
    next_token(0)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    lengths.host = [x + 1 for x in lengths.host]
    graph = torch.cuda.CUDAGraph()
    next_token(0)
    with torch.cuda.graph(graph):
        step()
    torch.cuda.synchronize()
    # capture ran nothing: the device lengths are still the host's
    assert lengths.device.cpu().tolist() == lengths.host
    for r in range(3):
        next_token(r)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        _check_batch(q, cache, lengths, ck, cv, mapping, budget, out, idx)
        lengths.host = [x + 1 for x in lengths.host]
        assert lengths.device.cpu().tolist() == lengths.host


def _c4_sequence_oracle(w, keys, values, q, ck, cv, L):
    """One C4 sequence's oracle at L cached tokens: selection and attention
    over its prefix encode, and the encode of the sequence grown by the
    current token (what the decode layer's append leaves in the planes)."""
    h2k = workloads.head_to_kv(w).numpy()
    pk, pv = f32(keys[:, :L]), f32(values[:, :L])
    pack = core.pack_keys(pk, token_group_size=w.token_group, dim_group_size=w.dim_group)
    enc = core.query_encode(f32(q)[None], w.dim_group, order="fold")
    sc = core.score_encoded(enc, pack, head_to_kv=h2k, tokens=L, dim_group_size=w.dim_group)[0]
    idx = core.select(sc, w.k, L)
    grown = core.pack_keys(np.concatenate([pk, f32(ck)[:, None]], 1), token_group_size=w.token_group,
                           dim_group_size=w.dim_group)
    return grown, idx, core.attention(f32(q), pk, pv, f32(ck), f32(cv), idx, h2k)


def test_c4_batch_after_an_append():
    """C4 as specified: eight sequences of 64K (PopKV-S, budget 4096, bf16;
    sequence b's prefix from the C1 distribution with seed 123 + b) whose
    decode tokens are N(0,1) (workloads.new_tokens).  The prefixes hold
    65534 tokens; the append adds N(0,1) token 0 (static K/V rows and
    metadata), then one batched decode layer with N(0,1) token 1 as the
    current one also appends it.  All eight sequences are checked against
    their own oracles: indices exact, attention within 2e-2 / 1e-2, and the
    packed planes of all 65536 tokens after the decode layer's append (which
    seals the last token group) bit-exact."""
    from concurrent.futures import ThreadPoolExecutor

    w = workloads.C4
    batch, rows = w.batch, w.context + 64
    L = w.prefix_tokens  # 65535 cached tokens once token 0 is appended
    new_k, new_v = workloads.new_tokens(w, 0)
    cur_k, cur_v = workloads.new_tokens(w, 1)
    kc = torch.zeros(batch, w.kv_heads, rows, 128, dtype=torch.bfloat16, device=DEV)
    vc = torch.zeros_like(kc)
    layers = []
    for b in range(batch):
        lay = workloads.make_layer(w, seed=w.seed + b)
        keys = torch.cat([lay.keys[:, :L - 1], new_k[b, :, None]], 1)
        values = torch.cat([lay.values[:, :L - 1], new_v[b, :, None]], 1)
        kc[b, :, :L - 1] = keys[:, :L - 1].to(DEV)
        vc[b, :, :L - 1] = values[:, :L - 1].to(DEV)
        layers.append((keys, values, lay.queries))
        del lay
    with ThreadPoolExecutor(max_workers=8) as pool:  # the C oracle releases the GIL
        wants = list(pool.map(lambda b: _c4_sequence_oracle(w, *layers[b], cur_k[b], cur_v[b], L), range(batch)))
    lengths = pb.SequenceLengths.create([L - 1] * batch, DEV)
    cache = pb.build_batched_popkv_cache(kc, vc, lengths, group_size=w.token_group, dim_group_size=w.dim_group)
    pb.append_batched(cache, lengths, new_k.to(DEV), new_v.to(DEV))
    lengths.advance()
    q = torch.stack([t[2] for t in layers]).to(DEV)
    mapping = workloads.head_to_kv(w, DEV)
    out, idx = pb.popkv_layer_step_batched(q, cache, lengths, cur_k.to(DEV), cur_v.to(DEV), mapping,
                                           budget=w.budget, return_indices=True, append=True)
    torch.cuda.synchronize()
    for b, (grown, want_idx, want_out) in enumerate(wants):
        assert np.array_equal(idx[b].cpu().numpy(), want_idx), b
        _assert_attention(out[b], want_out)
        # the decode layer's own append: token 1 at row L, and the planes of
        # all L + 1 tokens (its token group now sealed) equal to the oracle's
        assert torch.equal(kc[b, :, L].cpu(), cur_k[b]) and torch.equal(vc[b, :, L].cpu(), cur_v[b])
        for a, wp in zip(_packed_np(cache, b), grown):
            assert np.array_equal(a[:, :L + 1], wp), b


def test_decode_layer_flags_counts_past_the_bound():
    """A captured decode layer replayed past the launch bound it was
    captured with: the step runs at the clamped count and sets status bit 1
    (value 2); within the bound the flag stays clear."""
    starts = [900, 400]
    batch, qh, kvh, rows, budget, g, tg = 2, 32, 8, 1100, 256, 64, 64
    keys, values = _seq_data(batch, kvh, rows, seed=41)
    kc, vc = keys.to(DEV), values.to(DEV)
    lengths = pb.SequenceLengths.create(starts, DEV)
    cache = pb.build_batched_popkv_cache(kc, vc, lengths, group_size=tg, dim_group_size=g)
    mapping = torch.arange(qh, device=DEV) // (qh // kvh)
    gq = torch.Generator().manual_seed(3)
    q = torch.randn(batch, qh, 128, generator=gq).to(torch.bfloat16).to(DEV)
    ck = torch.randn(batch, kvh, 128, generator=gq).to(torch.bfloat16).to(DEV)
    status = torch.zeros(1, dtype=torch.int32, device=DEV)
    ws = pb.LayerStepWorkspace()
    bound = max(starts) + 1
    out = torch.empty_like(q)

    def step():
        pb.popkv_layer_step_batched(q, cache, lengths, ck, ck, mapping, budget=budget, max_tokens=bound,
                                    workspace=ws, out=out, append=True, status=status)
        lengths.device.add_(1)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    assert int(status.item()) == 0  # count 900 <= bound 901
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    graph.replay()  # count 901 == bound: still clear
    torch.cuda.synchronize()
    assert int(status.item()) == 0
    graph.replay()  # count 902 > bound 901
    torch.cuda.synchronize()
    assert int(status.item()) == 2
    assert lengths.device.cpu().tolist() == [903, 403]


def test_decode_layer_equals_step_then_append():
    """popkv_decode_layer_batched (the step with append=True: the append in
    extra workgroups of the select + attention launch) gives the same
    output, indices, static caches and packed planes as the layer step
    followed by append_batched -- eagerly, and in a HIP graph captured once
    and replayed while the sequences grow (each replay checked against the
    oracle at its own lengths)."""
    starts = [3000, 1499, 2200]
    batch, qh, kvh, rows, budget, g, tg = 3, 32, 8, 3100, 512, 64, 64
    keys, values = _seq_data(batch, kvh, rows, seed=29)
    mapping = torch.arange(qh, device=DEV) // (qh // kvh)

    def fresh():
        kc = torch.zeros(batch, kvh, rows, 128, dtype=torch.bfloat16, device=DEV)
        vc = torch.zeros_like(kc)
        for b, n in enumerate(starts):
            kc[b, :, :n] = keys[b, :, :n].to(DEV)
            vc[b, :, :n] = values[b, :, :n].to(DEV)
        lengths = pb.SequenceLengths.create(starts, DEV)
        return pb.build_batched_popkv_cache(kc, vc, lengths, group_size=tg, dim_group_size=g), lengths

    gq = torch.Generator().manual_seed(5)
    q = torch.randn(batch, qh, 128, generator=gq).to(torch.bfloat16).to(DEV)
    ck = torch.stack([keys[b, :, starts[b]] for b in range(batch)]).to(DEV)
    cv = torch.stack([values[b, :, starts[b]] for b in range(batch)]).to(DEV)
    ca, la = fresh()
    o1, i1 = pb.popkv_layer_step_batched(q, ca, la, ck, cv, mapping, budget=budget, return_indices=True)
    pb.append_batched(ca, la, ck, cv)
    cb, lb = fresh()
    o2, i2 = pb.popkv_layer_step_batched(q, cb, lb, ck, cv, mapping, budget=budget, return_indices=True,
                                         append=True)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2) and torch.equal(i1, i2)
    assert torch.equal(ca.key_cache, cb.key_cache) and torch.equal(ca.value_cache, cb.value_cache)
    for x, y in zip(ca.packed, cb.packed):
        assert torch.equal(x, y)

    # captured once, replayed with new tokens while the lengths grow
    cache, lengths = fresh()
    ws = pb.LayerStepWorkspace()
    out = torch.empty_like(q)
    bound = max(starts) + 8
    idx = torch.empty(batch, qh, min(budget - 1, bound) + 1, dtype=torch.int64, device=DEV)

    def step():
        _, i = pb.popkv_layer_step_batched(q, cache, lengths, ck, cv, mapping, budget=budget, max_tokens=bound,
                                           workspace=ws, out=out, return_indices=True, append=True)
        idx.copy_(i)
        lengths.device.add_(1)

    def next_token():
        q.copy_(torch.randn(batch, qh, 128, generator=gq).to(torch.bfloat16))
        ck.copy_(torch.stack([keys[b, :, lengths.host[b]] for b in range(batch)]))
        cv.copy_(torch.stack([values[b, :, lengths.host[b]] for b in range(batch)]))

    next_token()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    lengths.host = [x + 1 for x in lengths.host]
    graph = torch.cuda.CUDAGraph()
    next_token()
    with torch.cuda.graph(graph):
        step()
    torch.cuda.synchronize()
    assert lengths.device.cpu().tolist() == lengths.host
    for _ in range(3):
        next_token()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        _check_batch(q, cache, lengths, ck, cv, mapping, budget, out, idx)
        lengths.host = [x + 1 for x in lengths.host]
        assert lengths.device.cpu().tolist() == lengths.host


@pytest.mark.parametrize("g, tg, dtype", [(16, 128, torch.bfloat16), (32, 32, torch.bfloat16), (64, 8, torch.bfloat16),
                                         (64, 64, torch.float16), (32, 32, torch.float32)])
def test_decode_layer_append_other_group_shapes(g, tg, dtype):
    """The append inside the select + attention launch for the 16- and
    32-dimension encodes (four waves of the launch's workgroup), a short
    token group and the fp16 / fp32 caches: the same output, indices, static caches and packed planes
    as the layer step followed by append_batched, and the planes equal to
    the oracle's pack of the grown sequences.  The lengths put the new token
    at a group's first row, inside a group and at its last row."""
    batch, qh, kvh, rows, budget = 3, 32, 8, 1200, 256
    starts = [tg * 7, tg * 5 + 3, tg * 6 - 1]
    keys, values = _seq_data(batch, kvh, rows, seed=31 + g, dtype=dtype)
    mapping = torch.arange(qh, device=DEV) // (qh // kvh)

    def fresh():
        kc = torch.zeros(batch, kvh, rows, 128, dtype=dtype, device=DEV)
        vc = torch.zeros_like(kc)
        for b, n in enumerate(starts):
            kc[b, :, :n] = keys[b, :, :n].to(DEV)
            vc[b, :, :n] = values[b, :, :n].to(DEV)
        lengths = pb.SequenceLengths.create(starts, DEV)
        return pb.build_batched_popkv_cache(kc, vc, lengths, group_size=tg, dim_group_size=g), lengths

    gq = torch.Generator().manual_seed(7 + g)
    q = torch.randn(batch, qh, 128, generator=gq).to(dtype).to(DEV)
    ck = torch.stack([keys[b, :, starts[b]] for b in range(batch)]).to(DEV)
    cv = torch.stack([values[b, :, starts[b]] for b in range(batch)]).to(DEV)
    ca, la = fresh()
    o1, i1 = pb.popkv_layer_step_batched(q, ca, la, ck, cv, mapping, budget=budget, return_indices=True)
    pb.append_batched(ca, la, ck, cv)
    cb, lb = fresh()
    o2, i2 = pb.popkv_layer_step_batched(q, cb, lb, ck, cv, mapping, budget=budget, return_indices=True,
                                         append=True)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2) and torch.equal(i1, i2)
    assert torch.equal(ca.key_cache, cb.key_cache) and torch.equal(ca.value_cache, cb.value_cache)
    for x, y in zip(ca.packed, cb.packed):
        assert torch.equal(x, y)
    for b, n in enumerate(starts):
        want = core.pack_keys(f32(cb.key_cache[b, :, :n + 1]), token_group_size=tg, dim_group_size=g)
        for a, wp in zip(_packed_np(cb, b), want):
            assert np.array_equal(a[:, :n + 1], wp), (g, tg, dtype, b)
