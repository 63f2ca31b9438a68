"""GPU parity of the HIP path against the CPU oracle (bit-exact for planes,
representatives, popcount scores and selected indices; attention within
2e-2 max-abs / 1e-2 relative of a float64 materialized reference).

Mirrors the reference's GPU tests (tests/test_popkv.py:199-372,
tests/test_sparse_kernels.py:118-140) and extends them to the benchmark
configuration C1 at full size.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import core
from popkv_amd import _native, popkv, popkv_cuda, sparse_kernels, topk, workloads

pytestmark = pytest.mark.gpu

DEV = "cuda"
DIMS = (32, 64, 96, 127, 128)
GROUPS = (16, 32, 64)
DTYPES = (torch.bfloat16, torch.float16, torch.float32)
ATTN_ATOL, ATTN_RTOL = 2e-2, 1e-2


def f32(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy()


def bits(t: torch.Tensor) -> np.ndarray:
    t = t.detach().cpu().contiguous()
    if t.dtype in (torch.float16, torch.bfloat16):
        return t.view(torch.int16).numpy().view(np.uint16)
    if t.dtype == torch.float32:
        return t.view(torch.int32).numpy().view(np.uint32)
    return t.numpy()


def randn(*shape, dtype=torch.bfloat16, seed=0, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(dtype).to(DEV)


# ------------------------------------------------------------------ query encode

@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("g", GROUPS)
@pytest.mark.parametrize("d", DIMS)
def test_query_encode_bit_exact(d, g, dtype):
    q = randn(2, 8, d, dtype=dtype, seed=17 + d + g)
    got = popkv_cuda.query_encode(q.contiguous(), dim_group_size=g)
    want = core.query_encode(f32(q), g, order="fold")
    assert np.array_equal(bits(got[0]), want[0]) and np.array_equal(bits(got[1]), want[1])
    assert np.array_equal(bits(got[2]), want[2].view(np.uint32))
    assert np.array_equal(bits(got[3]), want[3].view(np.uint32))


@pytest.mark.parametrize("g", GROUPS)
def test_query_encode_tree_order_bit_exact(g):
    q = randn(4, 8, 128, seed=3 + g, scale=7.0)
    outs = popkv_cuda.allocate_query_encode_outputs(q, dim_group_size=g)
    with torch.cuda.device(q.device):
        _native.call("popkv_query_encode", q.data_ptr(), _native.DTYPE_BF16, 32, 128, g, _native.ENCODE_TREE,
                     *(t.data_ptr() for t in outs), _native.stream_of(q.device))
    want = core.query_encode(f32(q), g, order="tree")
    for a, b in zip(outs, want):
        assert np.array_equal(bits(a), b.view(np.uint32) if b.dtype == np.float32 else b)


# ------------------------------------------------------------------ pack

@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("g", GROUPS)
@pytest.mark.parametrize("d", DIMS)
def test_pack_bit_exact(d, g, dtype):
    keys = randn(2, 37, d, dtype=dtype, seed=31 + d + g)
    packed = popkv_cuda.pack_keys(keys.contiguous(), dim_group_size=g)
    want = core.pack_keys(f32(keys), token_group_size=32, dim_group_size=g)
    for a, b in zip(packed, want):
        assert a.shape == b.shape
        assert np.array_equal(bits(a), b)


@pytest.mark.parametrize("tg", (1, 5, 8, 10, 16, 32, 64, 125, 128, 500, 4096))
def test_pack_token_groups_bit_exact(tg):
    tokens = tg + 3
    keys = randn(2, tokens, 128, seed=37 + tg)
    for g in (GROUPS if tg in popkv_cuda.SPECIALIZED_TOKEN_GROUP_SIZES else (32,)):
        packed = popkv_cuda.pack_keys(keys.contiguous(), token_group_size=tg, dim_group_size=g)
        want = core.pack_keys(f32(keys), token_group_size=tg, dim_group_size=g)
        for a, b in zip(packed, want):
            assert np.array_equal(bits(a), b)


def test_pack_outlier_keys_and_capacity_tail():
    w = workloads.scaled(workloads.C1, context=1000)
    layer = workloads.make_layer(w).to(DEV)
    keys = layer.prefix_k().contiguous()
    packed = popkv_cuda.pack_keys(keys, token_capacity=1100, token_group_size=64, dim_group_size=64)
    want = core.pack_keys(f32(keys), token_group_size=64, dim_group_size=64)
    for a, b in zip(packed, want):
        assert a.shape[1] == 1100
        assert np.array_equal(bits(a)[:, :999], b)


def _special_keys(dtype, heads: int, tokens: int, seed: int) -> torch.Tensor:
    """Keys whose encode sits on every edge of the magnitude test
    mag = v >= 0 ? v > 0.5*max : v < 0.5*min: values equal to half a
    group extremum, dimensions with a positive minimum or a negative
    maximum, signed zeros only, the dtype's subnormals, NaNs and
    infinities, beside random dimensions."""
    g = torch.Generator().manual_seed(seed)
    shape = (heads, tokens, 128)
    vals = torch.tensor([-4.0, -2.0, -1.0, -0.5, -0.0, 0.0, 0.5, 1.0, 2.0, 4.0])
    x = vals[torch.randint(0, len(vals), shape, generator=g)]
    x[..., 0:8] = x[..., 0:8].abs() + 0.5
    x[..., 8:16] = -(x[..., 8:16].abs() + 0.5)
    x[..., 16:24] = torch.where(torch.rand(heads, tokens, 8, generator=g) < 0.5, -0.0, 0.0)
    tiny = {torch.bfloat16: 2.0 ** -133, torch.float16: 2.0 ** -24, torch.float32: 2.0 ** -149}[dtype]
    x[..., 24:32] = torch.randint(-3, 4, (heads, tokens, 8), generator=g).float() * tiny
    x[:, ::7, 40] = float("nan")
    x[:, 3::11, 70] = float("nan")
    x[0, 5::13, 90] = float("inf")
    x[-1, 9::17, 100] = float("-inf")
    x[..., 110:] = torch.randn(heads, tokens, 18, generator=g) * 3.0
    return x.to(dtype).to(DEV)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("g", GROUPS)
@pytest.mark.parametrize("tg", (64, 128))
def test_pack_edge_values_bit_exact(tg, g, dtype):
    """Sign and magnitude planes bit-exact on the edge values above; the
    representatives bit-exact wherever the oracle's is a number, NaN where
    it is NaN (a NaN's payload is not compared)."""
    keys = _special_keys(dtype, 2, 2 * tg + 37, seed=tg + g)
    packed = popkv_cuda.pack_keys(keys.contiguous(), token_group_size=tg, dim_group_size=g)
    want = core.pack_keys(f32(keys), token_group_size=tg, dim_group_size=g)
    assert np.array_equal(bits(packed[0]), want[0]) and np.array_equal(bits(packed[1]), want[1])
    for a, b in zip(packed[2:], want[2:]):
        got = bits(a)
        nan = (b & 0x7C00 == 0x7C00) & (b & 0x03FF != 0)
        assert np.array_equal(got[~nan], b[~nan])
        assert np.all((got[nan] & 0x7C00 == 0x7C00) & (got[nan] & 0x03FF != 0))
        assert nan.any() and (~nan).any()


@pytest.mark.parametrize("dtype", (torch.bfloat16, torch.float16))
@pytest.mark.parametrize("g", GROUPS)
@pytest.mark.parametrize("tg", (8, 16, 32, 64, 128))
def test_pack_staged_groups_bit_exact(tg, g, dtype):
    """The encode that keeps each group's rows in LDS (16-bit keys, token
    groups of at most 64 at G64 and 128 at G32 / G16; G64 at TG 128 takes
    the unstaged form), through the C-ABI: every fill level of the last
    group, keys at a head stride wider than their rows, packed rows written
    at an offset; rows outside the written range keep their fill."""
    r = 128 // g
    for n_last in (1, tg // 2 + 1, tg):
        tokens, offset = 2 * tg + n_last, 3
        buf = _special_keys(dtype, 3, tokens + 5, seed=tg + n_last + g)
        keys = buf[:, :tokens]  # head stride (tokens + 5) rows
        cap = tokens + offset + 2
        planes = (torch.full((3, cap, 4), -7, dtype=torch.int32, device=DEV),
                  torch.full((3, cap, 4), -7, dtype=torch.int32, device=DEV),
                  torch.full((3, cap, r), 1.5, dtype=torch.float16, device=DEV),
                  torch.full((3, cap, r), 1.5, dtype=torch.float16, device=DEV))
        with torch.cuda.device(DEV):
            _native.call("popkv_pack", keys.data_ptr(), _native.dtype_code(keys), 3, tokens, 128, buf.stride(0),
                         *(t.data_ptr() for t in planes), cap, offset, tg, g, _native.stream_of(DEV))
        want = core.pack_keys(f32(keys.contiguous()), token_group_size=tg, dim_group_size=g)
        for a, b, fill in zip(planes, want, (-7, -7, 1.5, 1.5)):
            got = bits(a)
            assert np.array_equal(got[:, :offset], bits(torch.full_like(a[:, :offset], fill)))
            assert np.array_equal(got[:, offset + tokens:], bits(torch.full_like(a[:, offset + tokens:], fill)))
            mid = got[:, offset:offset + tokens]
            if a.dtype == torch.int32:
                assert np.array_equal(mid, b)
            else:
                nan = (b & 0x7C00 == 0x7C00) & (b & 0x03FF != 0)
                assert np.array_equal(mid[~nan], b[~nan])
                assert np.all((mid[nan] & 0x7C00 == 0x7C00) & (mid[nan] & 0x03FF != 0))


@pytest.mark.parametrize("tg", (8, 16, 32, 64, 128))
def test_incremental_cache_crosses_every_token_group_boundary(tg):
    """tests/test_popkv.py:354-372 on the HIP path, bit-exact."""
    for g in GROUPS:
        keys = randn(2, tg - 1, 128, seed=41 + tg + g)
        cache = popkv.build_popkv_cache(keys, group_size=tg, dim_group_size=g, reserve_tokens=3)
        for step in range(2):
            current = randn(2, 1, 128, seed=1000 + step + tg + g)
            popkv.append_popkv(cache, current)
            keys = torch.cat((keys, current), dim=1)
            want = core.pack_keys(f32(keys), token_group_size=tg, dim_group_size=g)
            n = keys.shape[1]
            for a, b in zip(cache.packed, want):
                assert np.array_equal(bits(a)[:, :n], b)
            assert cache.token_count == n


def test_pack_into_capacity_exceeded():
    keys = randn(2, 10, 128)
    packed = popkv_cuda.pack_keys(keys.contiguous(), token_capacity=12)
    with pytest.raises(RuntimeError, match="capacity exceeded"):
        popkv_cuda.pack_keys_into(keys.contiguous(), packed, token_offset=3)


# ------------------------------------------------------------------ score

@pytest.mark.parametrize("g", GROUPS)
@pytest.mark.parametrize("d", DIMS)
def test_score_bit_exact(d, g):
    keys = randn(2, 37, d, seed=31 + d)
    q = randn(1, 8, d, seed=131 + d)
    mapping = torch.arange(8, device=DEV) // 4
    packed = popkv_cuda.pack_keys(keys.contiguous(), dim_group_size=g)
    got = popkv_cuda.score(q.contiguous(), packed, head_to_kv=mapping, tokens=37, dim_group_size=g)
    assert got.dtype == (torch.float16 if d == 128 else torch.float32)
    want = core.score(f32(q), tuple(bits(t) if t.dtype != torch.int32 else t.cpu().numpy() for t in packed),
                      head_to_kv=mapping.cpu().numpy(), tokens=37, dim_group_size=g)
    assert np.array_equal(bits(got), want.view(np.uint32) if want.dtype == np.float32 else want)
    if d == 128:
        enc = popkv_cuda.query_encode(q.contiguous(), dim_group_size=g)
        sep = popkv_cuda.score_encoded(enc, packed, head_to_kv=mapping, tokens=37, dim_group_size=g)
        want_sep = core.score_encoded(tuple(t.cpu().numpy() for t in enc),
                                      tuple(bits(t) if t.dtype != torch.int32 else t.cpu().numpy() for t in packed),
                                      head_to_kv=mapping.cpu().numpy(), tokens=37, dim_group_size=g)
        assert np.array_equal(bits(sep), want_sep)


@pytest.mark.parametrize("g", GROUPS)
def test_score_multiple_batches_and_tokens(g):
    """tests/test_popkv.py:302-317 shape (batch 2, 257 tokens) plus a long row."""
    for tokens in (257, 5000):
        keys = randn(2, tokens, 128, seed=32 + tokens)
        q = randn(2, 8, 128, seed=33 + tokens)
        mapping = torch.arange(8, device=DEV) // 4
        packed = popkv_cuda.pack_keys(keys.contiguous(), dim_group_size=g)
        got = popkv_cuda.score(q.contiguous(), packed, head_to_kv=mapping, tokens=tokens, dim_group_size=g)
        pk = tuple(bits(t) if t.dtype != torch.int32 else t.cpu().numpy() for t in packed)
        want = core.score(f32(q), pk, head_to_kv=mapping.cpu().numpy(), tokens=tokens, dim_group_size=g)
        assert np.array_equal(bits(got), want)


def test_score_rejects_bad_token_count():
    keys = randn(2, 8, 128)
    packed = popkv_cuda.pack_keys(keys.contiguous())
    mapping = torch.arange(8, device=DEV) // 4
    with pytest.raises(RuntimeError, match="invalid score token count"):
        popkv_cuda.score(randn(1, 8, 128).contiguous(), packed, head_to_kv=mapping, tokens=9)


# ------------------------------------------------------------------ select

def _scores(kind: str, rows: int, tokens: int, seed: int) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    if kind == "random":
        x = torch.randn(rows, tokens, generator=g)
    elif kind == "ties":
        x = torch.randint(-3, 4, (rows, tokens), generator=g).float()
    elif kind == "two_values":
        x = torch.where(torch.rand(rows, tokens, generator=g) < 0.5, 1.0, 2.0)
    elif kind == "signed_zero":
        x = torch.where(torch.rand(rows, tokens, generator=g) < 0.5, -0.0, 0.0)
    elif kind == "nan":
        x = torch.randn(rows, tokens, generator=g)
        x[:, ::37] = float("nan")
    elif kind == "drift":  # scores rising along the row: tile-local threshold estimates miss
        x = torch.randn(rows, tokens, generator=g) * 0.5 + torch.linspace(-6.0, 6.0, tokens)
    else:  # peaked fp16 scores, as the scorer produces
        x = torch.randn(rows, tokens, generator=g) * 0.5
        x[:, ::97] += 4.0
    return x.to(torch.float16).to(DEV)


@pytest.mark.parametrize("kind", ["random", "ties", "two_values", "signed_zero", "nan", "peaked"])
@pytest.mark.parametrize("tokens", [1, 7, 1000, 4095, 32767])
def test_select_matches_oracle(kind, tokens):
    s = _scores(kind, 4, tokens, seed=tokens + len(kind))
    for k in sorted({0, 1, min(511, tokens), min(4095, tokens), max(tokens - 1, 0), tokens}):
        got = topk.select_with_current(s, k, tokens + 1)
        want = core.select(bits(s), k, tokens)
        assert np.array_equal(got.cpu().numpy(), want), (kind, tokens, k)


@pytest.mark.parametrize("kind", ["random", "ties", "nan", "peaked", "drift"])
@pytest.mark.parametrize("rows,tokens,k", [(32, 32767, 4095), (32, 32767, 2731), (32, 24576, 3000),
                                           (24, 40000, 4500), (16, 65536, 8000), (16, 65536, 4000)])
def test_select_tile_window_path(kind, rows, tokens, k):
    """Shapes whose API-select chunks are whole 2048-token tiles (and at
    most 512 tiles in all), so key_hist_kernel writes tile windows and the
    select takes its threshold from them (no chunk-histogram launch):
    chunks of 2048 and 4096 tokens, up to 32 tiles per row, a partial last
    tile, tiles whose window misses the row's threshold bin (drift), ties,
    NaN -- index-exact against the oracle."""
    s = _scores(kind, rows, tokens, seed=tokens + k + len(kind))
    got = topk.select_with_current(s, k, tokens + 1)
    assert np.array_equal(got.cpu().numpy(), core.select(bits(s), k, tokens)), (kind, tokens, k)


def test_select_tile_window_path_int32_unaligned_rows():
    """The window path through the C-ABI with int32 indices and score rows
    at an odd stride (not 16-byte aligned: key_hist's shifted loads), twice
    on one workspace (its histograms left zero by the first call)."""
    rows, tokens, k = 32, 32767, 4095
    buf = _scores("peaked", rows, tokens + 1, seed=77)
    s = buf[:, :tokens]  # row stride tokens + 1
    nbytes = int(_native.lib().popkv_topk_select_workspace_bytes(rows, tokens))
    ws = torch.zeros(nbytes, device=DEV, dtype=torch.uint8)
    want = core.select(bits(s.contiguous()), k, tokens)
    for rep in range(2):
        out = torch.full((rows, k + 2), -7, device=DEV, dtype=torch.int32)
        with torch.cuda.device(DEV):
            _native.call("popkv_topk_select", s.data_ptr(), rows, s.stride(0), tokens, k, 999, out.data_ptr(),
                         _native.INDEX_I32, out.stride(0), ws.data_ptr(), nbytes, _native.stream_of(s.device))
        got = out.cpu().numpy()
        assert np.array_equal(got[:, :k], want[:, :k]), rep
        assert (got[:, k] == 999).all() and (got[:, k + 1] == -7).all()
    assert int(ws[: rows * 1024].count_nonzero()) == 0


@pytest.mark.parametrize("tokens", [65535, 131071, 200000, 524288])
def test_select_long_rows(tokens):
    s = _scores("peaked", 3, tokens, seed=5)
    got = topk.select_with_current(s, 4095, tokens + 1)
    assert np.array_equal(got.cpu().numpy(), core.select(bits(s), 4095, tokens))


def test_select_rows_past_131072_tokens_ties_and_torch_topk():
    """32 rows of 200000 tie-heavy fp16 scores (values -3 .. 3): the select
    equals the oracle's stable order and torch.topk's index sets at k = 4095
    and 100000; a row of 524289 tokens is refused."""
    s = _scores("ties", 32, 200000, seed=21)
    for k in (4095, 100000):
        got = topk.select_with_current(s, k, 200001).cpu().numpy()
        assert np.array_equal(got, core.select(bits(s), k, 200000)), k
        ref = torch.topk(s, k, dim=-1, sorted=False).indices.cpu().numpy()
        for r in range(0, 32, 7):
            assert set(got[r, :k].tolist()) == set(ref[r].tolist()), (k, r)
    with pytest.raises(RuntimeError, match="524288"):
        topk.select_with_current(torch.zeros(1, 524289, dtype=torch.float16, device=DEV), 10, 524290)


@pytest.mark.parametrize("kind", ["ties", "two_values", "signed_zero", "random"])
def test_select_agrees_with_torch_topk_on_rocm(kind):
    """The tie rule (lowest indices among scores equal to the k-th) is the one
    PyTorch's radix top-k applies; checked against torch.topk on this GPU."""
    s = _scores(kind, 8, 4096, seed=11)
    for k in (1, 100, 511, 2048, 4095):
        ours = topk.topk_indices(s, k).cpu().numpy()
        ref = torch.topk(s, k, dim=-1, sorted=False).indices.cpu().numpy()
        for r in range(s.shape[0]):
            assert set(ours[r].tolist()) == set(ref[r].tolist()), (kind, k, r)


def test_topk_indices_shape_matches_torch():
    s = _scores("random", 8, 1000, seed=3).view(1, 8, 1000)
    idx = topk.topk_indices(s, 31)
    assert idx.shape == (1, 8, 31) and idx.dtype == torch.int64
    ref = torch.topk(s, 31, dim=-1, sorted=False).indices
    assert torch.equal(idx.sort(-1).values, ref.sort(-1).values)


# ------------------------------------------------------------------ attention

def _attn_case(q_heads=8, kv_heads=2, tokens=32768, dim=128, selected=4096, dtype=torch.bfloat16, seed=104,
               capacity=None):
    g = torch.Generator().manual_seed(seed)
    cap = tokens if capacity is None else capacity
    queries = torch.randn(q_heads, dim, generator=g).to(dtype).to(DEV)
    kstore = torch.randn(kv_heads, cap, dim, generator=g).to(dtype).to(DEV)
    vstore = torch.randn(kv_heads, cap, dim, generator=g).to(dtype).to(DEV)
    ck = torch.randn(kv_heads, dim, generator=g).to(dtype).to(DEV)
    cv = torch.randn(kv_heads, dim, generator=g).to(dtype).to(DEV)
    mapping = (torch.arange(q_heads) // (q_heads // kv_heads)).to(DEV)
    indices = torch.randint(tokens, (q_heads, selected), generator=g).to(DEV)
    indices[:, -1] = tokens
    return queries, kstore[:, :tokens], vstore[:, :tokens], ck, cv, indices, mapping


def _oracle_attention(q, k, v, ck, cv, idx, mapping, valid=None):
    return core.attention(f32(q), f32(k), f32(v), f32(ck), f32(cv), idx.cpu().numpy(), mapping.cpu().numpy(),
                          None if valid is None else valid.cpu().numpy())


def test_split_attention_matches_reference_shape():
    """tests/test_sparse_kernels.py:118-140: 32K tokens, 4096 selected, split 256, valid mask."""
    q, k, v, ck, cv, idx, mapping = _attn_case()
    valid = torch.ones_like(idx, dtype=torch.bool)
    valid[:, -7:-1] = False
    for vm in (None, valid):
        got = sparse_kernels.indexed_attention_split(q, k, v, ck, cv, idx, mapping, vm, split_tokens=256)
        assert got.dtype == q.dtype and got.shape == q.shape
        want = _oracle_attention(q, k, v, ck, cv, idx, mapping, vm)
        np.testing.assert_allclose(f32(got), want, atol=ATTN_ATOL, rtol=ATTN_RTOL)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("dim", (64, 128, 256))
def test_split_attention_dtypes_dims_and_strided_cache(dtype, dim):
    q, k, v, ck, cv, idx, mapping = _attn_case(q_heads=8, kv_heads=4, tokens=3000, dim=dim, selected=700,
                                               dtype=dtype, seed=dim, capacity=3500)
    assert not k.is_contiguous()  # static-cache view: head stride = capacity * D
    for split in (16, 256, 512):
        got = sparse_kernels.indexed_attention_split(q, k, v, ck, cv, idx, mapping, split_tokens=split)
        want = _oracle_attention(q, k, v, ck, cv, idx, mapping)
        np.testing.assert_allclose(f32(got), want, atol=ATTN_ATOL, rtol=ATTN_RTOL)


def test_split_attention_partials_merge_like_oracle():
    q, k, v, ck, cv, idx, mapping = _attn_case(tokens=5000, selected=1000, seed=9)
    parts = sparse_kernels.indexed_attention_split_partial(q, k, v, ck, cv, idx, mapping, split_tokens=256)
    assert parts.shape == (8, 4, 130) and parts.dtype == torch.float32
    merged = sparse_kernels.indexed_attention_split_merge(parts, q.float())
    np.testing.assert_allclose(f32(merged), core.attention_merge(f32(parts)), atol=1e-5, rtol=1e-5)
    np.testing.assert_allclose(f32(merged), _oracle_attention(q, k, v, ck, cv, idx, mapping), atol=ATTN_ATOL,
                               rtol=ATTN_RTOL)


def test_split_attention_int32_indices_and_all_masked_split():
    q, k, v, ck, cv, idx, mapping = _attn_case(tokens=4000, selected=600, seed=12)
    valid = torch.ones_like(idx, dtype=torch.bool)
    valid[:, 256:512] = False  # an entire split masked out
    got = sparse_kernels.indexed_attention_split(q, k, v, ck, cv, idx.int(), mapping, valid)
    want = _oracle_attention(q, k, v, ck, cv, idx, mapping, valid)
    np.testing.assert_allclose(f32(got), want, atol=ATTN_ATOL, rtol=ATTN_RTOL)


# ------------------------------------------------------------------ decode step

def _layer_setup(w: workloads.Workload, seed=None):
    layer = workloads.make_layer(w, seed=seed).to(DEV)
    mapping = workloads.head_to_kv(w, DEV)
    cache = popkv.build_popkv_cache(layer.prefix_k(), group_size=w.token_group, dim_group_size=w.dim_group,
                                    reserve_tokens=64)
    return layer, mapping, cache


def _oracle_step(w, layer, mapping, cache):
    """Oracle for one layer: fold encode -> GQA popcount scores -> select ->
    float64 attention.  Returns (fp16 score bits, indices, output)."""
    L = layer.prefix_tokens
    enc = core.query_encode(f32(layer.queries)[None], w.dim_group, order="fold")
    pk = tuple(bits(t) if t.dtype != torch.int32 else t.cpu().numpy() for t in cache.packed)
    h2k = mapping.cpu().numpy()
    sc = core.score_encoded(enc, pk, head_to_kv=h2k, tokens=L, dim_group_size=w.dim_group)[0]
    idx = core.select(sc, w.k, L)
    out = core.attention(f32(layer.queries), f32(layer.prefix_k()), f32(layer.prefix_v()), f32(layer.current_k()),
                         f32(layer.current_v()), idx, h2k)
    return sc, idx, out


@pytest.mark.parametrize("method", ["popkv-s", "popkv-q", "popkv-normal"])
def test_retrieval_step_and_layer_step_match_oracle(method):
    tg, g = popkv.POPKV_PRESETS[method]
    base = workloads.scaled(workloads.C1, context=6000, budget=1024)
    w = workloads.Workload(base.name, method, base.q_heads, base.kv_heads, 128, 6000, 1024, tg, g,
                           torch.bfloat16, 42, True)
    layer, mapping, cache = _layer_setup(w)
    sc, idx, out = _oracle_step(w, layer, mapping, cache)
    enc = popkv_cuda.query_encode(layer.queries.unsqueeze(0).contiguous(), dim_group_size=g)
    scores = popkv_cuda.score_encoded(enc, cache.packed, head_to_kv=mapping, tokens=cache.token_count,
                                      dim_group_size=g)
    assert np.array_equal(bits(scores[0]), sc)
    sel = topk.select_with_current(scores, w.k, layer.prefix_tokens + 1)
    assert np.array_equal(sel.cpu().numpy(), idx)
    o1 = popkv.popkv_retrieval_step(layer.queries, layer.prefix_k(), layer.prefix_v(), layer.current_k(),
                                    layer.current_v(), cache, mapping, budget=w.budget)
    np.testing.assert_allclose(f32(o1), out, atol=ATTN_ATOL, rtol=ATTN_RTOL)
    o2, idx2 = popkv.popkv_layer_step(layer.queries, cache, layer.prefix_k(), layer.prefix_v(), layer.current_k(),
                                      layer.current_v(), mapping, budget=w.budget, return_indices=True)
    assert np.array_equal(idx2.cpu().numpy(), idx)
    np.testing.assert_allclose(f32(o2), out, atol=ATTN_ATOL, rtol=ATTN_RTOL)
    o3 = popkv.popkv_layer_step(layer.queries, cache, layer.prefix_k(), layer.prefix_v(), layer.current_k(),
                                layer.current_v(), mapping, budget=w.budget)
    assert torch.equal(o3, o2)


def _check_layer_step(w, layer, mapping, cache):
    sc, idx, out = _oracle_step(w, layer, mapping, cache)
    o, got = popkv.popkv_layer_step(layer.queries, cache, layer.prefix_k(), layer.prefix_v(), layer.current_k(),
                                    layer.current_v(), mapping, budget=w.budget, return_indices=True)
    assert np.array_equal(got.cpu().numpy(), idx)
    np.testing.assert_allclose(f32(o), out, atol=ATTN_ATOL, rtol=ATTN_RTOL)
    o2 = popkv.popkv_layer_step(layer.queries, cache, layer.prefix_k(), layer.prefix_v(), layer.current_k(),
                                layer.current_v(), mapping, budget=w.budget)
    assert torch.equal(o2, o)


@pytest.mark.parametrize("distinct", [1, 3, 16])
def test_layer_step_heavy_ties(distinct):
    """Every prefix key is a copy of one of `distinct` rows, so each head's
    scores take at most `distinct` values and the k-th key is shared by many
    tokens: only the lowest-index ties may be taken."""
    w = workloads.scaled(workloads.C1, context=5000, budget=700)
    layer = workloads.make_layer(w, seed=5)
    g = torch.Generator().manual_seed(9)
    pick = torch.randint(0, distinct, (w.context,), generator=g)
    layer.keys[:, :] = layer.keys[:, :distinct][:, pick]
    layer = layer.to(DEV)
    mapping = workloads.head_to_kv(w, DEV)
    cache = popkv.build_popkv_cache(layer.prefix_k(), group_size=w.token_group, dim_group_size=w.dim_group,
                                    reserve_tokens=64)
    _check_layer_step(w, layer, mapping, cache)


@pytest.mark.parametrize("distinct", [1, 3, 16])
def test_layer_step_heavy_ties_single_launch(distinct):
    """The same ties in the single-launch tile-window form (10000 tokens:
    ten 1024-token tiles, the last one ragged, in chunks of whole tiles):
    with 1 or 3 distinct rows a tile holds more than 255 keys of the
    threshold bin, more than its window's byte counts can hold (the tile is
    histogrammed from its keys), with 16 the byte counts hold them; windows
    estimated from one tile's keys may miss the row's bin."""
    w = workloads.scaled(workloads.C1, context=10000, budget=1200)
    assert _native.lib().popkv_layer_step_launches(w.q_heads, w.kv_heads, w.context, w.budget, w.dim_group) == 1
    layer = workloads.make_layer(w, seed=6)
    g = torch.Generator().manual_seed(10 + distinct)
    pick = torch.randint(0, distinct, (w.context,), generator=g)
    layer.keys[:, :] = layer.keys[:, :distinct][:, pick]
    layer = layer.to(DEV)
    mapping = workloads.head_to_kv(w, DEV)
    cache = popkv.build_popkv_cache(layer.prefix_k(), group_size=w.token_group, dim_group_size=w.dim_group,
                                    reserve_tokens=64)
    _check_layer_step(w, layer, mapping, cache)


@pytest.mark.parametrize("context,budget", [(300, 512), (1025, 1025), (64, 2), (2, 2)])
def test_layer_step_budget_covers_or_exceeds_context(context, budget):
    w = workloads.scaled(workloads.C1, context=context, budget=budget)
    layer, mapping, cache = _layer_setup(w)
    _check_layer_step(w, layer, mapping, cache)


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_layer_step_dtypes(dtype):
    base = workloads.scaled(workloads.C1, context=4500, budget=600)
    w = workloads.Workload(base.name, base.method, base.q_heads, base.kv_heads, 128, base.context, base.budget,
                           base.token_group, base.dim_group, dtype, 3, True)
    layer, mapping, cache = _layer_setup(w)
    _check_layer_step(w, layer, mapping, cache)


@pytest.mark.parametrize("q_heads,kv_heads,context,budget", [(32, 8, 16384, 4096), (32, 8, 32768, 4096),
                                                             (64, 16, 32768, 2048)])
@pytest.mark.parametrize("dtype", DTYPES)
def test_layer_step_single_launch_dtypes_and_chunk_plans(dtype, q_heads, kv_heads, context, budget):
    """The single launch in bf16, fp16 and fp32, with chunks of 1024, 2048
    and 4096 tokens (4, 8 and 16 keys per select thread), each shape taking
    the one-launch form."""
    w = workloads.Workload("single", "popkv-s", q_heads, kv_heads, 128, context, budget, 64, 64, dtype,
                           11 + q_heads + budget, True)
    assert int(_native.lib().popkv_layer_step_launches(w.q_heads, w.kv_heads, w.prefix_tokens, w.budget,
                                                  w.dim_group)) == 1
    layer, mapping, cache = _layer_setup(w)
    _check_layer_step(w, layer, mapping, cache)


@pytest.mark.parametrize("q_heads,kv_heads", [(32, 32), (64, 32), (64, 8)])
def test_layer_step_single_launch_gqa_group_sizes(q_heads, kv_heads):
    """The single launch with GQA groups of 1, 2 and 8 query heads (the
    scorer's and the select's group-size instantiations besides C1's 4) at
    16K, budget 4096."""
    w = workloads.Workload("gqa", "popkv-s", q_heads, kv_heads, 128, 16384, 4096, 64, 64, torch.bfloat16,
                           q_heads + kv_heads, True)
    assert int(_native.lib().popkv_layer_step_launches(w.q_heads, w.kv_heads, w.prefix_tokens, w.budget,
                                                      w.dim_group)) == 1
    layer, mapping, cache = _layer_setup(w)
    _check_layer_step(w, layer, mapping, cache)


@pytest.mark.parametrize("q_heads,kv_heads,context,budget", [(32, 8, 10001, 2048), (32, 4, 12001, 2048),
                                                             (32, 8, 9001, 1024)])
def test_layer_step_single_launch_512_token_tiles(q_heads, kv_heads, context, budget):
    """Short rows in the single launch: at most 512 (1024-token tile, query
    row) pairs, so the scorer takes 512-token tiles of one token per thread
    (twice the workgroups) and the select reads their windows; ragged last
    tiles, GQA groups of 4 and 8."""
    w = workloads.Workload("short", "popkv-s", q_heads, kv_heads, 128, context, budget, 64, 64, torch.bfloat16,
                           context % 97, True)
    assert int(_native.lib().popkv_layer_step_launches(w.q_heads, w.kv_heads, w.prefix_tokens, w.budget,
                                                      w.dim_group)) == 1
    assert -(-w.prefix_tokens // 1024) * w.q_heads <= 512
    layer, mapping, cache = _layer_setup(w)
    _check_layer_step(w, layer, mapping, cache)


@pytest.mark.parametrize("context", [65536, 131072])
def test_layer_step_long_context(context):
    """C3's long contexts: more than 32 key rounds per select thread (keys
    re-read per pass) and 4096-token attention chunks."""
    w = workloads.scaled(workloads.c3(context), context=context)
    layer, mapping, cache = _layer_setup(w)
    _check_layer_step(w, layer, mapping, cache)


@pytest.mark.parametrize("context,budget", [(200001, 4096), (262145, 65536)])
def test_layer_step_rows_past_131072_tokens(context, budget):
    """Rows beyond 131072 tokens (the selects take up to 64 chunks of 8192):
    200000 cached tokens at budget 4096 (25 chunks) and 262144 at budget
    65536 (32 chunks holding about 2048 selected tokens each).  Indices
    exact, attention within tolerance, against the oracle."""
    w = workloads.scaled(workloads.c3(131072), context=context, budget=budget)
    layer, mapping, cache = _layer_setup(w)
    _check_layer_step(w, layer, mapping, cache)


def test_layer_step_batch_laid_along_heads_equals_per_sequence_steps():
    """C4's batching: sequences side by side along the head axis (K/V and
    packed caches [B*KVH, ...], queries [B*QH, D], head i -> KV head i // 4)
    give exactly the per-sequence selection, and attention outputs within two
    bf16 rounding steps of theirs (the chunk plan -- hence the order in which
    the chunks' partial states are merged -- depends on the step's row count,
    96 here against 32)."""
    w = workloads.scaled(workloads.C1, context=3000, budget=700)
    seqs = [workloads.make_layer(w, seed=11 + b).to(DEV) for b in range(3)]
    mapping = workloads.head_to_kv(w, DEV)
    singles = []
    for lay in seqs:
        cache = popkv.build_popkv_cache(lay.prefix_k(), group_size=w.token_group, dim_group_size=w.dim_group,
                                        reserve_tokens=64)
        singles.append(popkv.popkv_layer_step(lay.queries, cache, lay.prefix_k(), lay.prefix_v(), lay.current_k(),
                                              lay.current_v(), mapping, budget=w.budget, return_indices=True))
    keys = torch.cat([x.keys for x in seqs], 0)
    values = torch.cat([x.values for x in seqs], 0)
    L = w.prefix_tokens
    cache = popkv.build_popkv_cache(keys[:, :L], group_size=w.token_group, dim_group_size=w.dim_group,
                                    reserve_tokens=64)
    qh = len(seqs) * w.q_heads
    bmap = torch.arange(qh, device=DEV) // (w.q_heads // w.kv_heads)
    out, idx = popkv.popkv_layer_step(torch.cat([x.queries for x in seqs], 0), cache, keys[:, :L], values[:, :L],
                                      keys[:, L].contiguous(), values[:, L].contiguous(), bmap, budget=w.budget,
                                      return_indices=True)
    assert torch.equal(idx, torch.cat([i for _, i in singles], 0))
    ref = torch.cat([o for o, _ in singles], 0).float()
    assert ((out.float() - ref).abs() <= 2.0 ** -7 * ref.abs() + 1e-4).all()


@pytest.mark.parametrize("context,dtype", [(3000, torch.bfloat16), (700, torch.float32), (1, torch.bfloat16),
                                           (1537, torch.float16), (12000, torch.bfloat16), (40000, torch.bfloat16)])
def test_dense_attention_matches_oracle(context, dtype):
    """The full layers: every prefix token plus the current one.  12000 and
    40000 tokens give 24 and 79 splits of 512: the four-wave merge, with a
    second batch round for 79."""
    base = workloads.scaled(workloads.C1, context=context, budget=2)
    w = workloads.Workload(base.name, base.method, base.q_heads, base.kv_heads, 128, context, 2, base.token_group,
                           base.dim_group, dtype, 5, context > 1)
    lay = workloads.make_layer(w).to(DEV)
    mapping = workloads.head_to_kv(w, DEV)
    L = lay.prefix_tokens
    out = popkv.dense_attention_step(lay.queries, lay.prefix_k(), lay.prefix_v(), lay.current_k(), lay.current_v())
    idx = np.tile(np.arange(L + 1, dtype=np.int64), (w.q_heads, 1))
    want = core.attention(f32(lay.queries), f32(lay.prefix_k()), f32(lay.prefix_v()), f32(lay.current_k()),
                          f32(lay.current_v()), idx, mapping.cpu().numpy())
    np.testing.assert_allclose(f32(out), want, atol=ATTN_ATOL, rtol=ATTN_RTOL)


def test_dense_attention_fused_merge_tickets_and_split_limit():
    """The MFMA dense kernel's fused merge (each KV group's last workgroup
    merges; tickets zero between calls): one reused workspace, calls at 64
    splits (32768 tokens: fused), 65 splits (the separate merge), 8 query
    heads and again 32 (the ticket region cleared on the head-count change),
    each against the oracle; and the same call twice gives equal bits."""
    ws = popkv.LayerStepWorkspace()
    for q_heads, kv_heads, context, seed in ((32, 8, 32769, 1), (32, 8, 33281, 2), (8, 2, 5000, 3),
                                             (32, 8, 32769, 4)):
        base = workloads.scaled(workloads.C1, context=context, budget=2)
        w = workloads.Workload(base.name, base.method, q_heads, kv_heads, 128, context, 2, base.token_group,
                               base.dim_group, torch.bfloat16, seed, True)
        lay = workloads.make_layer(w).to(DEV)
        mapping = workloads.head_to_kv(w, DEV)
        L = lay.prefix_tokens
        args = (lay.queries, lay.prefix_k(), lay.prefix_v(), lay.current_k(), lay.current_v())
        out = popkv.dense_attention_step(*args, workspace=ws)
        again = popkv.dense_attention_step(*args, workspace=ws)
        assert torch.equal(out, again), (q_heads, context)
        idx = np.tile(np.arange(L + 1, dtype=np.int64), (w.q_heads, 1))
        want = core.attention(f32(lay.queries), f32(lay.prefix_k()), f32(lay.prefix_v()), f32(lay.current_k()),
                              f32(lay.current_v()), idx, mapping.cpu().numpy())
        np.testing.assert_allclose(f32(out), want, atol=ATTN_ATOL, rtol=ATTN_RTOL)
        assert not ws.buffer[: 256].any(), "merge tickets left non-zero"


@pytest.mark.parametrize("q_heads,kv_heads,dtype", [(8, 8, torch.bfloat16), (8, 4, torch.float16),
                                                     (16, 2, torch.bfloat16), (8, 2, torch.float16),
                                                     (16, 4, torch.float32)])
def test_dense_attention_group_sizes(q_heads, kv_heads, dtype):
    """Dense layers at every GQA group size the launcher distinguishes: 1, 2
    and 8 query heads per KV head (VALU kernel), 4 in fp16 (matrix-core
    kernel) and 4 in fp32 (VALU kernel); 2100 tokens end in a ragged split."""
    base = workloads.scaled(workloads.C1, context=2101, budget=2)
    w = workloads.Workload(base.name, base.method, q_heads, kv_heads, 128, 2101, 2, base.token_group,
                           base.dim_group, dtype, 9, True)
    lay = workloads.make_layer(w).to(DEV)
    mapping = workloads.head_to_kv(w, DEV)
    L = lay.prefix_tokens
    out = popkv.dense_attention_step(lay.queries, lay.prefix_k(), lay.prefix_v(), lay.current_k(), lay.current_v())
    idx = np.tile(np.arange(L + 1, dtype=np.int64), (w.q_heads, 1))
    want = core.attention(f32(lay.queries), f32(lay.prefix_k()), f32(lay.prefix_v()), f32(lay.current_k()),
                          f32(lay.current_v()), idx, mapping.cpu().numpy())
    np.testing.assert_allclose(f32(out), want, atol=ATTN_ATOL, rtol=ATTN_RTOL)


def test_retrieval_step_with_torch_topk_hook():
    w = workloads.scaled(workloads.C1, context=3000, budget=512)
    layer, mapping, cache = _layer_setup(w)
    ours = popkv.popkv_retrieval_step(layer.queries, layer.prefix_k(), layer.prefix_v(), layer.current_k(),
                                      layer.current_v(), cache, mapping, budget=w.budget)
    hooked = popkv.popkv_retrieval_step(
        layer.queries, layer.prefix_k(), layer.prefix_v(), layer.current_k(), layer.current_v(), cache, mapping,
        budget=w.budget, topk=lambda s, k: torch.topk(s, k=k, dim=-1, sorted=False).indices)
    np.testing.assert_allclose(f32(hooked), f32(ours), atol=ATTN_ATOL, rtol=ATTN_RTOL)
    # the reference's experimental_topk hook set to this build's select: the
    # loop reads hook(scores, k)[0] (popkv.py:1091-1093)
    ours_hook = popkv.popkv_retrieval_step(
        layer.queries, layer.prefix_k(), layer.prefix_v(), layer.current_k(), layer.current_v(), cache, mapping,
        budget=w.budget, topk=topk.topk_indices)
    assert torch.equal(ours_hook, ours)


def test_c1_full_size_parity():
    """The headline configuration: PopKV-S, QH 32 / KVH 8, 32K context,
    budget 4096, bf16.  Prepack bit-exact, scores bit-exact, indices exact,
    attention within tolerance; then a decode append keeps all of it."""
    w = workloads.C1
    layer, mapping, cache = _layer_setup(w)
    L = layer.prefix_tokens
    want_pack = core.pack_keys(f32(layer.prefix_k()), token_group_size=64, dim_group_size=64)
    for a, b in zip(cache.packed, want_pack):
        assert np.array_equal(bits(a)[:, :L], b)
    sc, idx, out = _oracle_step(w, layer, mapping, cache)
    o, got_idx = popkv.popkv_layer_step(layer.queries, cache, layer.prefix_k(), layer.prefix_v(),
                                        layer.current_k(), layer.current_v(), mapping, budget=w.budget,
                                        return_indices=True)
    assert np.array_equal(got_idx.cpu().numpy(), idx)
    err = np.abs(f32(o) - out)
    assert (err <= ATTN_ATOL + ATTN_RTOL * np.abs(out)).all(), err.max()
    # size-independent properties of the selection
    assert (got_idx[:, -1] == L).all()
    assert (got_idx[:, :-1].diff(dim=-1) > 0).all()
    # append the current token to the retrieval cache, as the decode loop does
    popkv.append_popkv(cache, layer.current_k()[:, None])
    keys_all = layer.keys
    want_tail = core.pack_keys(f32(keys_all[:, L - (L % 64):]), token_group_size=64, dim_group_size=64)
    start = L - (L % 64)
    for a, b in zip(cache.packed, want_tail):
        assert np.array_equal(bits(a)[:, start:L + 1], b)


def test_topk_workspace_reused_across_row_counts():
    """The select keeps per-row histograms at the start of its workspace; a
    call with more rows than the last one must not see the keys a smaller
    call left there (the Python wrapper clears the larger region)."""
    for rows, tokens, seed in ((32, 5000, 1), (8, 3000, 2), (32, 5000, 3), (40, 700, 4), (24, 30000, 5),
                               (40, 9000, 6)):
        s = _scores("random", rows, tokens, seed=seed)
        for k in (1, 257, tokens - 1):
            ours = topk.topk_indices(s, k).cpu().numpy()
            ref = torch.topk(s, k, dim=-1, sorted=False).indices.cpu().numpy()
            for r in range(rows):
                assert set(ours[r].tolist()) == set(ref[r].tolist()), (rows, tokens, k, r)


def test_layer_step_workspace_reused_across_head_counts():
    """One LayerStepWorkspace serving steps with 8 and then 32 query heads
    (and back) gives each step the oracle's indices and output."""
    ws = popkv.LayerStepWorkspace()
    for q_heads, kv_heads, context, seed in ((8, 2, 3000, 21), (32, 8, 3000, 22), (8, 2, 5000, 23)):
        base = workloads.scaled(workloads.C1, context=context, budget=700)
        w = workloads.Workload(base.name, base.method, q_heads, kv_heads, 128, context, 700, base.token_group,
                               base.dim_group, torch.bfloat16, seed, True)
        layer, mapping, cache = _layer_setup(w)
        sc, idx, out = _oracle_step(w, layer, mapping, cache)
        o, got = popkv.popkv_layer_step(layer.queries, cache, layer.prefix_k(), layer.prefix_v(), layer.current_k(),
                                        layer.current_v(), mapping, budget=w.budget, workspace=ws,
                                        return_indices=True)
        assert np.array_equal(got.cpu().numpy(), idx), (q_heads, context)
        np.testing.assert_allclose(f32(o), out, atol=ATTN_ATOL, rtol=ATTN_RTOL)


def test_layer_step_back_to_back_on_one_workspace():
    """Steps of different layers queued back to back on one workspace, with
    no host synchronization between them (the single-launch window form:
    each step's select blocks read what its own scorer blocks wrote in the
    same launch, never the previous step's keys, windows or histogram), the
    last at another shape: each gives the oracle's indices and output."""
    ws = popkv.LayerStepWorkspace()
    cases = []
    for context, budget, seed in ((32767, 4096, 31), (32767, 4096, 32), (8192, 1024, 33), (32767, 4096, 34)):
        w = workloads.scaled(workloads.C1, context=context, budget=budget)
        layer, mapping, cache = _layer_setup(w, seed=seed)
        o, got = popkv.popkv_layer_step(layer.queries, cache, layer.prefix_k(), layer.prefix_v(), layer.current_k(),
                                        layer.current_v(), mapping, budget=w.budget, workspace=ws,
                                        return_indices=True)
        cases.append((w, layer, mapping, cache, o, got))
    for w, layer, mapping, cache, o, got in cases:
        sc, idx, out = _oracle_step(w, layer, mapping, cache)
        assert np.array_equal(got.cpu().numpy(), idx), w.context
        np.testing.assert_allclose(f32(o), out, atol=ATTN_ATOL, rtol=ATTN_RTOL)


@pytest.mark.parametrize("tokens", [1000, 4095, 32767])
def test_select_int32_output_through_the_c_abi(tokens):
    """popkv_topk_select with int32 indices (row stride k + 3): the same
    selection as the oracle, current token in slot k, padding untouched."""
    s = _scores("peaked", 5, tokens, seed=31)
    k = min(511, tokens)
    out = torch.full((5, k + 3), -7, device=DEV, dtype=torch.int32)
    nbytes = int(_native.lib().popkv_topk_select_workspace_bytes(5, tokens))
    ws = torch.zeros(nbytes, device=DEV, dtype=torch.uint8)
    with torch.cuda.device(DEV):
        _native.call("popkv_topk_select", s.data_ptr(), 5, s.stride(0), tokens, k, 12345, out.data_ptr(),
                     _native.INDEX_I32, out.stride(0), ws.data_ptr(), nbytes, _native.stream_of(s.device))
    got = out.cpu().numpy()
    want = core.select(bits(s), k, tokens)
    assert np.array_equal(got[:, :k], want[:, :k])
    assert (got[:, k] == 12345).all() and (got[:, k + 1:] == -7).all()


def test_split_attention_unaligned_index_rows_take_the_general_kernel():
    """701 int64 indices per head (rows not 16-byte aligned) use the general
    kernel; 704 use the fast one; both match the oracle."""
    for selected in (701, 704):
        q, k, v, ck, cv, idx, mapping = _attn_case(q_heads=8, kv_heads=2, tokens=3000, selected=selected, seed=selected)
        valid = torch.ones_like(idx, dtype=torch.bool)
        valid[:, 5:9] = False
        got = sparse_kernels.indexed_attention_split(q, k, v, ck, cv, idx, mapping, valid, split_tokens=256)
        want = _oracle_attention(q, k, v, ck, cv, idx, mapping, valid)
        np.testing.assert_allclose(f32(got), want, atol=ATTN_ATOL, rtol=ATTN_RTOL)
