"""The allocation-free layer step (popkv_layer_step_noalloc) through the C
ABI: on two calls in a row -- the second with fewer query/KV heads, a
shorter context and a smaller budget -- its output and selection equal
those of popkv_layer_step with a caller workspace, bit for bit (the same
kernels), and the oracle's.  The process's first call is made inside HIP
graph capture and the graph replayed on new inputs.  Also: a step too large
for the library's scratch array is rejected before any launch."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import core
from popkv_amd import _native, popkv, workloads

pytestmark = pytest.mark.gpu

DEV = "cuda"


def f32(t):
    return t.detach().float().cpu().numpy()


def bits(t):
    t = t.detach().cpu().contiguous()
    return t.view(torch.int16).numpy().view(np.uint16) if t.dtype in (torch.float16, torch.bfloat16) else t.numpy()


def _case(q_heads, kv_heads, context, budget, seed):
    base = workloads.scaled(workloads.C1, context=context, budget=budget)
    w = workloads.Workload(base.name, base.method, q_heads, kv_heads, 128, context, budget, base.token_group,
                           base.dim_group, torch.bfloat16, seed, True)
    layer = workloads.make_layer(w).to(DEV)
    mapping = workloads.head_to_kv(w, DEV)
    cache = popkv.build_popkv_cache(layer.prefix_k(), group_size=w.token_group, dim_group_size=w.dim_group,
                                    reserve_tokens=64)
    return w, layer, mapping, cache


def _noalloc(w, layer, mapping, cache):
    L = layer.prefix_tokens
    out = torch.full_like(layer.queries, float("nan"))
    idx = torch.full((w.q_heads, w.k + 1), -1, device=DEV, dtype=torch.int64)
    q, ck, cv = layer.queries.contiguous(), layer.current_k(), layer.current_v()
    pk, pv = layer.prefix_k(), layer.prefix_v()
    ks, km, kl, kd = cache.packed
    with torch.cuda.device(q.device):
        _native.call("popkv_layer_step_noalloc", q.data_ptr(), _native.dtype_code(q), ks.data_ptr(), km.data_ptr(),
                     kl.data_ptr(), kd.data_ptr(), int(ks.shape[1]), pk.data_ptr(), pv.data_ptr(), pk.stride(0),
                     pv.stride(0), ck.data_ptr(), cv.data_ptr(), mapping.data_ptr(), w.q_heads, w.kv_heads, L,
                     w.budget, w.dim_group, out.data_ptr(), idx.data_ptr(), _native.stream_of(q.device))
    return out, idx


def test_noalloc_first_call_inside_graph_capture():
    """The process's first popkv_layer_step_noalloc call (which looks up the
    scratch array's device address) made inside HIP graph capture; the
    graph is then replayed with new queries and current K/V copied into its
    input tensors in place, and each replay's output and selection equal
    eager popkv_layer_step on the same inputs, bit for bit."""
    w, layer, mapping, cache = _case(32, 8, 6000, 1024, 63)
    L = layer.prefix_tokens
    q = layer.queries.clone()
    ck, cv = layer.current_k().clone(), layer.current_v().clone()
    pk, pv = layer.prefix_k(), layer.prefix_v()
    out = torch.full_like(q, float("nan"))
    idx = torch.full((w.q_heads, w.k + 1), -1, device=DEV, dtype=torch.int64)
    ks, km, kl, kd = cache.packed
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        _native.call("popkv_layer_step_noalloc", q.data_ptr(), _native.dtype_code(q), ks.data_ptr(), km.data_ptr(),
                     kl.data_ptr(), kd.data_ptr(), int(ks.shape[1]), pk.data_ptr(), pv.data_ptr(), pk.stride(0),
                     pv.stride(0), ck.data_ptr(), cv.data_ptr(), mapping.data_ptr(), w.q_heads, w.kv_heads, L,
                     w.budget, w.dim_group, out.data_ptr(), idx.data_ptr(), _native.stream_of(q.device))
    torch.cuda.synchronize()
    gen = torch.Generator().manual_seed(64)
    for rep in range(3):
        q.copy_((layer.queries.float().cpu() + 0.5 * torch.randn(q.shape, generator=gen)).to(q.dtype))
        ck.copy_(torch.randn(ck.shape, generator=gen).to(ck.dtype))
        cv.copy_(torch.randn(cv.shape, generator=gen).to(cv.dtype))
        out.fill_(float("nan"))
        idx.fill_(-1)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        want_out, want_idx = popkv.popkv_layer_step(q, cache, pk, pv, ck, cv, mapping, budget=w.budget,
                                                    return_indices=True)
        torch.cuda.synchronize()
        assert torch.equal(idx, want_idx), rep
        assert torch.equal(out, want_out), rep


def test_noalloc_layer_step_equals_workspace_entry_on_two_calls():
    assert int(_native.lib().popkv_layer_step_scratch_bytes()) == 16 << 20
    for q_heads, kv_heads, context, budget, seed in ((32, 8, 12000, 2048, 61), (8, 2, 3000, 512, 62)):
        w, layer, mapping, cache = _case(q_heads, kv_heads, context, budget, seed)
        want_out, want_idx = popkv.popkv_layer_step(layer.queries, cache, layer.prefix_k(), layer.prefix_v(),
                                                    layer.current_k(), layer.current_v(), mapping, budget=w.budget,
                                                    return_indices=True)
        got_out, got_idx = _noalloc(w, layer, mapping, cache)
        torch.cuda.synchronize()
        assert torch.equal(got_idx, want_idx), (q_heads, context)
        assert torch.equal(got_out, want_out), (q_heads, context)
        # and the oracle's selection / attention (the parity bar)
        L = layer.prefix_tokens
        enc = core.query_encode(f32(layer.queries)[None], w.dim_group, order="fold")
        pk = tuple(bits(t) if t.dtype != torch.int32 else t.cpu().numpy() for t in cache.packed)
        sc = core.score_encoded(enc, pk, head_to_kv=mapping.cpu().numpy(), tokens=L, dim_group_size=w.dim_group)[0]
        idx = core.select(sc, w.k, L)
        assert np.array_equal(got_idx.cpu().numpy(), idx)
        out = core.attention(f32(layer.queries), f32(layer.prefix_k()), f32(layer.prefix_v()),
                             f32(layer.current_k()), f32(layer.current_v()), idx, mapping.cpu().numpy())
        err = np.abs(f32(got_out) - out)
        assert (err <= 2e-2 + 1e-2 * np.abs(out)).all(), float(err.max())


def test_noalloc_rejects_a_step_larger_than_the_scratch_array():
    # 256 query heads x 131071 tokens: 64 MiB of order keys alone
    lib = _native.lib()
    need = int(lib.popkv_layer_step_workspace_bytes(256, 131071, 4096, 64))
    assert need > int(lib.popkv_layer_step_scratch_bytes())
    status = lib.popkv_layer_step_noalloc(None, 2, None, None, None, None, 131072, None, None, 0, 0, None, None,
                                          None, 256, 64, 131071, 4096, 64, None, None, None)
    assert status == -6 and b"scratch" in lib.popkv_last_error()
