"""Host-side logic of the drop-in API, runnable without a GPU: argument
validation and exception types (the reference raises ValueError from Python
and RuntimeError from its native checks), cache bookkeeping that fails
before any device call, the reference's CPU tests for the PopKV subset
(tests/test_popkv.py:38-64), the event pool with a fake clock
(tests/test_mlp_fairness.py:31-58 style), the workload generator and the
C ABI's exports."""
from __future__ import annotations

import json
import re
from pathlib import Path

import pytest
import torch

from popkv_amd import _native, decode_runtime, popkv, popkv_cuda, sparse_kernels, topk, workloads

ROOT = Path(__file__).resolve().parent.parent
GOLDEN = json.loads((ROOT / "tests" / "golden" / "reference_kats.json").read_text())


# ---------------------------------------------------------------- reference CPU tests

def test_public_methods_include_normal_ablation():
    assert popkv.METHODS == tuple(GOLDEN["methods"]["value"])


def test_sparse_methods_skip_configured_full_layers():
    c = GOLDEN["sparse_layer_indices"]
    assert popkv._sparse_layer_indices(c["num_layers"], tuple(c["full_layers"])) == tuple(c["expected"])


def test_current_token_is_always_reserved():
    c = GOLDEN["append_current"]
    actual = popkv._append_current(torch.tensor(c["selected"]), c["num_tokens"])
    assert torch.equal(actual[:, -1], torch.tensor(c["expected_last_column"]))
    assert actual.dtype == torch.long and actual.shape == (2, 3)


def test_release_configuration_is_explicit():
    c = GOLDEN["retrieval_config"]
    popkv.RetrievalConfig().validate()
    popkv.RetrievalConfig(fier_kernel="fier").validate()
    for size in c["valid_group_sizes"]:
        popkv.RetrievalConfig(group_size=size).validate()
    for size in c["invalid_group_sizes"]:
        with pytest.raises(ValueError):
            popkv.RetrievalConfig(group_size=size).validate()
    for size in c["valid_dim_group_sizes"]:
        popkv.RetrievalConfig(dim_group_size=size).validate()
    for size in c["invalid_dim_group_sizes"]:
        with pytest.raises(ValueError):
            popkv.RetrievalConfig(dim_group_size=size).validate()


def test_config_rules():
    with pytest.raises(ValueError, match="budget"):
        popkv.RetrievalConfig(budget=1).validate()
    with pytest.raises(ValueError, match="non-specialized"):
        popkv.RetrievalConfig(group_size=5, dim_group_size=64).validate()
    with pytest.raises(ValueError, match="requires dim_group_size"):
        popkv.RetrievalConfig(dim_kernel="g64-u32", dim_group_size=32).validate()
    for method, (tg, g) in popkv.POPKV_PRESETS.items():
        cfg = popkv.RetrievalConfig.preset(method)
        cfg.validate()
        assert (cfg.group_size, cfg.dim_group_size) == (tg, g)
    with pytest.raises(ValueError):
        popkv.RetrievalConfig.preset("popkv")


# ---------------------------------------------------------------- validation before the device

def test_pack_keys_rejects_non_cuda_and_bad_groups():
    keys = torch.zeros(2, 8, 128)
    with pytest.raises(ValueError, match="contiguous CUDA"):
        popkv_cuda.pack_keys(keys)
    with pytest.raises(ValueError, match="contiguous CUDA"):
        popkv_cuda.pack_keys_into(keys, (None,) * 4, token_offset=0)
    with pytest.raises(ValueError, match="token_group_size"):
        popkv_cuda._validate_token_group_size(0)
    with pytest.raises(ValueError, match="token_group_size"):
        popkv_cuda._validate_token_group_size(4097)
    with pytest.raises(ValueError, match="dim_group_size"):
        popkv_cuda._validate_dim_group_size(8)
    assert popkv_cuda._validate_dim_kernel(64, None) == "g64-u32"
    assert popkv_cuda._validate_dim_kernel(64, "g64-u64") == "g64-u64"
    with pytest.raises(ValueError, match="dim_kernel"):
        popkv_cuda._validate_dim_kernel(16, "g99")
    with pytest.raises(ValueError, match="requires dim_group_size"):
        popkv_cuda._validate_dim_kernel(16, "g32")


def test_query_and_score_reject_non_cuda():
    q = torch.zeros(1, 8, 128)
    with pytest.raises(ValueError, match="contiguous CUDA"):
        popkv_cuda.query_encode(q)
    with pytest.raises(ValueError, match="contiguous CUDA"):
        popkv_cuda.allocate_query_encode_outputs(q)
    with pytest.raises(ValueError, match="contiguous CUDA"):
        popkv_cuda.score(q, (None,) * 4, head_to_kv=torch.zeros(8, dtype=torch.long), tokens=1)
    with pytest.raises(ValueError, match="encoded_query"):
        popkv_cuda.score_encoded((q,), (None,) * 4, head_to_kv=torch.zeros(8, dtype=torch.long), tokens=1)
    with pytest.raises(ValueError, match="packed must contain"):
        popkv_cuda.score_encoded((q,) * 4, (None,) * 3, head_to_kv=torch.zeros(8, dtype=torch.long), tokens=1)
    with pytest.raises(ValueError, match="contiguous CUDA tensors"):
        popkv_cuda.score_encoded((q,) * 4, (None,) * 4, head_to_kv=torch.zeros(8, dtype=torch.long), tokens=1)


def test_attention_validation():
    q = torch.zeros(8, 128)
    k = torch.zeros(2, 16, 128)
    idx = torch.zeros(8, 4, dtype=torch.long)
    h2k = torch.zeros(8, dtype=torch.long)
    with pytest.raises(ValueError, match="ranks"):
        sparse_kernels.indexed_attention_split_partial(q[0], k, k, k[:, 0], k[:, 0], idx, h2k)
    with pytest.raises(ValueError, match="indices"):
        sparse_kernels.indexed_attention_split_partial(q, k, k, k[:, 0], k[:, 0], idx[:4], h2k)
    with pytest.raises(ValueError, match="valid mask"):
        sparse_kernels.indexed_attention_split_partial(q, k, k, k[:, 0], k[:, 0], idx, h2k,
                                                       torch.ones(8, 3, dtype=torch.bool))
    with pytest.raises(ValueError, match="multiple of 16"):
        sparse_kernels.indexed_attention_split_partial(q, k, k, k[:, 0], k[:, 0], idx, h2k, split_tokens=20)
    with pytest.raises(RuntimeError, match="CUDA device"):
        sparse_kernels.indexed_attention_split_partial(q, k, k, k[:, 0], k[:, 0], idx, h2k)
    with pytest.raises(ValueError, match="CUDA float32"):
        sparse_kernels.indexed_attention_split_merge(torch.zeros(8, 1, 130), q)


def test_topk_validation():
    with pytest.raises(ValueError, match="CUDA"):
        topk.topk_indices(torch.zeros(2, 10, dtype=torch.float16), 3)


def test_append_reserve_exhausted_before_device_call():
    """popkv.py:445-446: raises before any kernel runs."""
    packed = tuple(torch.zeros(2, 8, 4, dtype=torch.int32) for _ in range(2)) + \
        tuple(torch.zeros(2, 8, 2, dtype=torch.float16) for _ in range(2))
    cache = popkv.PopKVCache(group_size=8, dim_group_size=64, token_count=8, sealed_tokens=8,
                             packed=packed, active_keys=torch.zeros(2, 0, 128))
    with pytest.raises(RuntimeError, match="reserve exhausted"):
        popkv.append_popkv(cache, torch.zeros(2, 1, 128))
    caches = popkv.RetrievalCaches("popkv-s", {0: popkv.PopKVCache(8, 64, 8, 8, packed, torch.zeros(2, 0, 128))})
    with pytest.raises(RuntimeError, match="reserve exhausted"):
        popkv.append_retrieval_caches(caches, [torch.zeros(1, 2, 1, 128)])


def test_build_cache_validation():
    keys = torch.zeros(2, 8, 128)
    with pytest.raises(ValueError, match="group_size"):
        popkv.build_popkv_cache(keys, group_size=0, reserve_tokens=1)
    with pytest.raises(ValueError, match="non-specialized"):
        popkv.build_popkv_cache(keys, group_size=5, dim_group_size=64, reserve_tokens=1)
    with pytest.raises(ValueError, match="dim_group_size"):
        popkv.build_popkv_cache(keys, group_size=8, dim_group_size=8, reserve_tokens=1)


def _step_operands(q_heads=8, kv_heads=2, tokens=40, cap=64, g=64):
    q = torch.zeros(q_heads, 128, dtype=torch.bfloat16)
    pk = torch.zeros(kv_heads, tokens, 128, dtype=torch.bfloat16)
    k = torch.zeros(kv_heads, 128, dtype=torch.bfloat16)
    packed = (torch.zeros(kv_heads, cap, 4, dtype=torch.int32), torch.zeros(kv_heads, cap, 4, dtype=torch.int32),
              torch.zeros(kv_heads, cap, 128 // g, dtype=torch.float16),
              torch.zeros(kv_heads, cap, 128 // g, dtype=torch.float16))
    cache = popkv.PopKVCache(64, g, tokens, 0, packed, pk[:, :0])
    mapping = torch.arange(q_heads) // (q_heads // kv_heads)
    return q, pk, k, cache, mapping


def test_layer_step_rejects_every_mismatched_operand_before_the_device():
    """The C ABI gets raw pointers and head counts only, so each size it
    derives addresses from is checked in Python first (ValueError), then
    dtypes and devices (RuntimeError); CPU tensors reach the device check
    only when every shape is right."""
    q, pk, k, cache, h2k = _step_operands()
    step = lambda **kw: popkv.popkv_layer_step(  # noqa: E731
        kw.get("q", q), kw.get("cache", cache), kw.get("pk", pk), kw.get("pv", pk), kw.get("k", k), kw.get("v", k),
        kw.get("h2k", h2k), budget=kw.get("budget", 16), out=kw.get("out"))
    cases = [
        (dict(q=q[:, :64]), "requires q"),
        (dict(pv=pk[:, :10]), "prefix K/V must be"),
        (dict(q=q[:7]), "positive multiple"),
        (dict(k=k[:1]), "current k must be"),
        (dict(v=torch.zeros(2, 64, dtype=torch.bfloat16)), "current v must be"),
        (dict(out=torch.zeros(8, 64, dtype=torch.bfloat16)), "out must be"),
        (dict(out=torch.zeros(128, 8, dtype=torch.bfloat16).t()), "out must be contiguous"),
        (dict(h2k=h2k[:4]), "head_to_kv must be a vector of 8"),
        (dict(h2k=h2k.float()), "int64 or int32"),
        (dict(budget=1), "budget"),
        (dict(pk=pk[:, :39], pv=pk[:, :39]), "token_count"),
    ]
    for kw, msg in cases:
        with pytest.raises(ValueError, match=msg):
            step(**kw)
    q4, pk4, k4, cache4, h2k4 = _step_operands(q_heads=8, kv_heads=4)
    with pytest.raises(ValueError, match="packed k_sign must be"):  # packed for 4 KV heads, prefix for 2
        popkv.popkv_layer_step(q, cache4, pk, pk, k, k, h2k, budget=16)
    bad = popkv.PopKVCache(64, 64, 40, 0, (cache.packed[0], cache.packed[1], cache.packed[2][:, :, :1],
                                           cache.packed[3]), pk[:, :0])
    with pytest.raises(ValueError, match="packed k_low must be"):
        popkv.popkv_layer_step(q, bad, pk, pk, k, k, h2k, budget=16)
    bad = popkv.PopKVCache(64, 64, 40, 0, (cache.packed[0].float(),) + cache.packed[1:], pk[:, :0])
    with pytest.raises(ValueError, match="contiguous torch.int32"):
        popkv.popkv_layer_step(q, bad, pk, pk, k, k, h2k, budget=16)
    big = popkv.PopKVCache(64, 64, 65, 0, cache.packed, pk[:, :0])
    pk65 = torch.zeros(2, 65, 128, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="invalid score token count"):
        popkv.popkv_layer_step(q, big, pk65, pk65, k, k, h2k, budget=16)
    with pytest.raises(RuntimeError, match="share a dtype"):
        step(k=k.float())
    with pytest.raises(RuntimeError, match="same CUDA device"):
        step()


def test_layer_step_attention_rejects_mismatched_operands_before_the_device():
    q, pk, k, _, h2k = _step_operands()
    ws = torch.zeros(1 << 16, dtype=torch.uint8)
    att = lambda **kw: popkv.popkv_layer_step_attention(  # noqa: E731
        kw.get("q", q), kw.get("pk", pk), kw.get("pv", pk), kw.get("h2k", h2k), budget=kw.get("budget", 16),
        dim_group_size=kw.get("g", 64), workspace=kw.get("ws", ws))
    for kw, msg in [(dict(q=q[:, :64]), "requires a contiguous q"), (dict(pv=pk[:1]), "prefix K/V must be"),
                    (dict(q=q[:7]), "positive multiple"), (dict(h2k=h2k[:3]), "head_to_kv"),
                    (dict(budget=1), "budget"), (dict(pk=pk[:, :0], pv=pk[:, :0]), "token count"),
                    (dict(g=8), "dim_group_size"),
                    (dict(ws=popkv.LayerStepWorkspace()), "has not been used")]:
        with pytest.raises(ValueError, match=msg):
            att(**kw)
    with pytest.raises(RuntimeError, match="same CUDA device"):
        att()


def test_dense_step_rejects_mismatched_operands_before_the_device():
    q, pk, k, _, _ = _step_operands()
    dense = lambda **kw: popkv.dense_attention_step(  # noqa: E731
        kw.get("q", q), kw.get("pk", pk), kw.get("pv", pk), kw.get("k", k), kw.get("v", k), out=kw.get("out"))
    for kw, msg in [(dict(k=k[:1]), "current k must be"), (dict(out=q[:4]), "out must be"),
                    (dict(q=torch.zeros(6, 128, dtype=torch.bfloat16)), "1, 2, 4 or 8"),
                    (dict(pv=pk[:1]), "prefix K/V must be")]:
        with pytest.raises(ValueError, match=msg):
            dense(**kw)
    with pytest.raises(RuntimeError, match="share a dtype"):
        dense(out=torch.zeros(8, 128))
    with pytest.raises(RuntimeError, match="same CUDA device"):
        dense()


def test_static_cache_append_and_exhaustion():
    cache = popkv.StaticKVCache([torch.zeros(1, 2, 4, 8)], [torch.zeros(1, 2, 4, 8)], length=3, capacity=4)
    popkv.append_kv(cache, [torch.ones(1, 2, 1, 8)], [torch.full((1, 2, 1, 8), 2.0)])
    assert cache.length == 4
    assert torch.equal(cache.key_storage[0][:, :, 3], torch.ones(1, 2, 8))
    with pytest.raises(RuntimeError, match="capacity exhausted"):
        popkv.append_kv(cache, [torch.ones(1, 2, 1, 8)], [torch.ones(1, 2, 1, 8)])


# ---------------------------------------------------------------- event pool (fake clock)

class _FakeEvent:
    clock = 0.0

    def __init__(self, enable_timing=True):
        self.t = None

    def record(self, stream=None):
        _FakeEvent.clock += 1.5
        self.t = _FakeEvent.clock

    def synchronize(self):
        pass

    def elapsed_time(self, other):
        return other.t - self.t


class _FakeStream:
    def synchronize(self):
        pass


class _FakeDevice:
    def __init__(self, device):
        pass

    def __enter__(self):
        return self

    def __exit__(self, *a):
        return False


def test_event_pool_and_stage_timer(monkeypatch):
    monkeypatch.setattr(torch.cuda, "Event", _FakeEvent)
    monkeypatch.setattr(torch.cuda, "device", _FakeDevice)
    monkeypatch.setattr(torch.cuda, "current_stream", lambda device=None: _FakeStream())
    pool = decode_runtime.DecodeEventPool(torch.device("cpu"), 1 + len(decode_runtime.RETRIEVAL_STAGES))
    timer = decode_runtime.StageTimer(pool)
    for name in decode_runtime.RETRIEVAL_STAGES:
        timer.mark(name)
    totals = timer.finish()
    assert totals["total"] == pytest.approx(sum(totals[n] for n in decode_runtime.RETRIEVAL_STAGES))
    with pytest.raises(ValueError, match="unknown decode stage"):
        timer.mark("mlp")
    with pytest.raises(RuntimeError, match="exhausted"):
        pool.record()


# ---------------------------------------------------------------- workloads

def test_algorithmic_bytes_match_baseline_table():
    b = workloads.algorithmic_bytes(workloads.C1)
    assert (b["score"], b["select"], b["attention"], b["encode"]) == (12582528, 2621376, 67649536, 9728)
    assert b["step"] == 82863168
    sweep = [round(workloads.algorithmic_bytes(workloads.c3(c))["step"] / 1e6, 2) for c in workloads.C3_CONTEXTS]
    assert sweep == [70.02, 71.85, 75.52, 82.86, 97.54, 126.90]


def test_workload_generator_is_deterministic():
    w = workloads.scaled(workloads.C1, context=512, budget=64)
    a, b = workloads.make_layer(w), workloads.make_layer(w)
    assert torch.equal(a.keys.view(torch.int16), b.keys.view(torch.int16))
    assert torch.equal(a.queries.view(torch.int16), b.queries.view(torch.int16))
    assert a.keys.dtype == torch.bfloat16 and a.keys.shape == (8, 512, 128) and a.queries.shape == (32, 128)
    # outlier channels: 4 per KV head with ~10x the spread of the rest
    std = a.keys.float().std(dim=1)
    assert ((std > 5).sum(dim=1) == 4).all()
    c0 = workloads.make_layer(workloads.C0)
    assert c0.keys.dtype == torch.float32 and c0.keys.shape == (2, 4096, 128)


# ---------------------------------------------------------------- C ABI

def _header_functions() -> set[str]:
    text = _native.HEADER_PATH.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b(popkv_[a-z0-9_]+)\s*\(", text))


def test_library_exports_every_header_symbol():
    lib = _native.lib()
    declared = _header_functions()
    assert declared == set(_native.exported_symbols())
    for name in declared:
        assert hasattr(lib, name), name


def test_library_host_only_entry_points():
    lib = _native.lib()
    assert lib.popkv_version().decode().startswith("popkv-hip")
    assert lib.popkv_status_string(-2).decode() == "Pop-KV cache capacity exceeded"
    assert lib.popkv_layer_step_workspace_bytes(32, 32767, 4096, 64) > 32 * 32767 * 2
    assert lib.popkv_layer_step_workspace_bytes(32, 32767, 1, 64) == 0
    # the layer step's launches: one at C1 and C3 up to 32K (the tile-window
    # form), one when the budget covers the context (select + attention
    # only), three past 32 tiles, for 16-dimension groups and GQA groups of 3
    launches = lib.popkv_layer_step_launches
    assert launches(32, 8, 32767, 4096, 64) == 1 and launches(32, 8, 16383, 4096, 64) == 1
    assert launches(32, 8, 4095, 4096, 64) == 1 and launches(32, 8, 300, 512, 16) == 1
    assert launches(32, 8, 65535, 4096, 64) == 3 and launches(32, 8, 32767, 4096, 16) == 3
    assert launches(24, 8, 32767, 4096, 64) == 3
    assert launches(32, 8, 32767, 1, 64) == 0 and launches(30, 8, 32767, 4096, 64) == 0
    assert launches(32, 8, 524289, 4096, 64) == 0
    assert lib.popkv_score_workspace_bytes(1, 32, 128, 64) > 0
    # argument errors are reported before anything touches a device
    st = lib.popkv_pack(None, 2, 8, 10, 128, 1280, None, None, None, None, 10, 0, 64, 64, None)
    assert st == -1 and "null" in lib.popkv_last_error().decode()
    fake = 0x1000
    st = lib.popkv_pack(fake, 2, 8, 10, 128, 1280, fake, fake, fake, fake, 12, 3, 64, 64, None)
    assert st == -2 and "capacity exceeded" in lib.popkv_last_error().decode()
    ws_bytes = lib.popkv_topk_select_workspace_bytes(4, 100)
    assert ws_bytes >= 4 * 256 * 4 + 4 * 128 * 2
    st = lib.popkv_topk_select(fake, 4, 10, 10, 11, 10, fake, 0, 12, fake, ws_bytes, None)
    assert st == -1
    st = lib.popkv_topk_select(fake, 4, 524289, 524289, 11, 10, fake, 0, 12, fake, 1 << 30, None)
    assert st == -4
    st = lib.popkv_topk_select(fake, 4, 100, 100, 11, 10, fake, 0, 12, None, ws_bytes, None)
    assert st == -1 and "null" in lib.popkv_last_error().decode()
    st = lib.popkv_topk_select(fake, 4, 100, 100, 11, 10, fake, 0, 12, fake, ws_bytes - 1, None)
    assert st == -6 and "workspace" in lib.popkv_last_error().decode()
    with pytest.raises(RuntimeError, match="capacity exceeded"):
        _native.check(lib.popkv_pack(fake, 2, 8, 10, 128, 1280, fake, fake, fake, fake, 12, 3, 64, 64, None))


def test_batched_api_validation_before_the_device():
    """popkv_amd.batch checks shapes, lengths and capacity on the host
    before any launch (CPU tensors never reach the C ABI)."""
    from popkv_amd import batch as pb

    with pytest.raises(ValueError, match="non-negative"):
        pb.SequenceLengths.create([3, -1], "cpu")
    lengths = pb.SequenceLengths.create([3, 5], "cpu")
    lengths.advance()
    assert lengths.host == [4, 6] and lengths.device.tolist() == [4, 6]
    kc = torch.zeros(2, 2, 8, 128, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="static K/V caches must be"):
        pb.build_batched_popkv_cache(kc[..., :64], kc[..., :64], lengths, group_size=8, dim_group_size=32)
    with pytest.raises(ValueError, match="3 lengths"):
        pb.build_batched_popkv_cache(kc, kc, pb.SequenceLengths.create([1, 1, 1], "cpu"), group_size=8,
                                     dim_group_size=32)
    with pytest.raises(RuntimeError, match="capacity exceeded"):
        pb.build_batched_popkv_cache(kc, kc, pb.SequenceLengths.create([9, 1], "cpu"), group_size=8,
                                     dim_group_size=32)
    with pytest.raises(ValueError, match="non-specialized"):
        pb.build_batched_popkv_cache(kc, kc, lengths, group_size=5, dim_group_size=64)
    planes = (torch.zeros(2, 2, 8, 4, dtype=torch.int32), torch.zeros(2, 2, 8, 4, dtype=torch.int32),
              torch.zeros(2, 2, 8, 4, dtype=torch.float16), torch.zeros(2, 2, 8, 4, dtype=torch.float16))
    cache = pb.BatchedPopKVCache(8, 32, planes, kc, kc.clone())
    nk = torch.zeros(2, 2, 128, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="new K/V must be"):
        pb.append_batched(cache, lengths, nk[:1], nk[:1])
    with pytest.raises(RuntimeError, match="reserve exhausted"):
        pb.append_batched(cache, pb.SequenceLengths.create([8, 2], "cpu"), nk, nk)
    q = torch.zeros(2, 8, 128, dtype=torch.bfloat16)
    h2k = torch.arange(8) // 4
    step = pb.popkv_layer_step_batched
    with pytest.raises(ValueError, match="q must be"):
        step(q[:1], cache, lengths, nk, nk, h2k, budget=4)
    with pytest.raises(ValueError, match="current k must be"):
        step(q, cache, lengths, nk[:, :1], nk, h2k, budget=4)
    with pytest.raises(ValueError, match="head_to_kv"):
        step(q, cache, lengths, nk, nk, h2k[:4], budget=4)
    with pytest.raises(ValueError, match="budget"):
        step(q, cache, lengths, nk, nk, h2k, budget=1)
    with pytest.raises(ValueError, match="max_tokens"):
        step(q, cache, lengths, nk, nk, h2k, budget=4, max_tokens=5)
    with pytest.raises(RuntimeError, match="invalid score token count"):
        step(q, cache, lengths, nk, nk, h2k, budget=4, max_tokens=9)
    # every plane's shape and dtype against (B, KVH, capacity, 4 or 128/G),
    # before any device check
    def with_plane(i, t):
        p = list(planes)
        p[i] = t
        return pb.BatchedPopKVCache(8, 32, tuple(p), kc, kc.clone())

    bad_planes = [
        (with_plane(0, planes[0][:1]), "packed k_sign must be \\[2, 2, capacity, 4\\]"),
        (with_plane(1, planes[1][:, :, :4]), "packed k_mag must be"),
        (with_plane(2, planes[2][..., :2]), "packed k_low must be"),
        (with_plane(3, torch.zeros(2, 2, 8, 4, dtype=torch.float32)), "packed k_delta must be a contiguous"),
        (with_plane(2, torch.zeros(2, 2, 4, 8, dtype=torch.float16).transpose(2, 3)), "contiguous"),
        (pb.BatchedPopKVCache(8, 32, planes[:3], kc, kc.clone()), "packed must contain"),
        (pb.BatchedPopKVCache(8, 16, planes, kc, kc.clone()), "packed k_low must be"),
        (pb.BatchedPopKVCache(8, 32, planes, kc, kc[..., :64]), "static K/V caches must be"),
    ]
    for bad, msg in bad_planes:
        with pytest.raises(ValueError, match=msg):
            step(q, bad, lengths, nk, nk, h2k, budget=4)
        with pytest.raises(ValueError, match=msg):
            pb.append_batched(bad, lengths, nk, nk)
        with pytest.raises(ValueError, match=msg):
            pb.prepack_batched(bad, lengths)
    with pytest.raises(ValueError, match="status"):
        step(q, cache, lengths, nk, nk, h2k, budget=4, status=torch.zeros(1, dtype=torch.int32))
    with pytest.raises(ValueError, match="status must be an int32"):
        pb.append_batched(cache, lengths, nk, nk, status=torch.zeros(1, dtype=torch.int64))
    odd = pb.SequenceLengths(torch.tensor([4, 6], dtype=torch.int32), [4, 6])
    with pytest.raises(ValueError, match="contiguous int64"):
        step(q, cache, odd, nk, nk, h2k, budget=4)
    # shapes right, host tensors: refused before any pointer reaches the C ABI
    with pytest.raises(RuntimeError, match="CUDA device"):
        step(q, cache, lengths, nk, nk, h2k, budget=4)
    with pytest.raises(RuntimeError, match="CUDA device"):
        pb.append_batched(cache, lengths, nk, nk)
    with pytest.raises(RuntimeError, match="CUDA device"):
        pb.prepack_batched(cache, lengths)
    with pytest.raises(RuntimeError, match="CUDA device"):
        pb.build_batched_popkv_cache(kc, kc, lengths, group_size=8, dim_group_size=32)


def _oracle_cache(tokens=150, tg=64, g=64, cap=256, seed=3, dtype=torch.bfloat16):
    import numpy as np

    from oracle import core

    gen = torch.Generator().manual_seed(seed)
    keys = torch.randn(2, tokens, 128, generator=gen).to(dtype)
    ks, km, kl, kd = core.pack_keys(keys.float().numpy(), token_group_size=tg, dim_group_size=g)
    planes = []
    for a, dt in ((ks, torch.int32), (km, torch.int32), (kl, torch.float16), (kd, torch.float16)):
        full = torch.zeros(2, cap, a.shape[2], dtype=dt)
        src = torch.from_numpy(np.ascontiguousarray(a).view(np.int16 if dt == torch.float16 else np.int32))
        full[:, :tokens] = src.view(dt)
        planes.append(full)
    sealed = tokens // tg * tg
    return popkv.PopKVCache(tg, g, tokens, sealed, tuple(planes), keys[:, sealed:].clone())


def test_packed_metadata_wire_round_trip_and_validation(tmp_path):
    """The packed-metadata format (popkv_amd.wire): a cache encoded by the
    oracle survives to_bytes / from_bytes and save / load bit for bit (rows
    past token_count come back zero); corrupted, truncated, foreign and
    inconsistent blobs are refused."""
    from popkv_amd import wire

    for tokens, tg, g, dtype in ((150, 64, 64, torch.bfloat16), (128, 128, 16, torch.float16),
                                 (37, 32, 32, torch.float32), (0, 8, 32, torch.bfloat16)):
        cache = _oracle_cache(tokens, tg, g, cap=256, dtype=dtype)
        blob = wire.to_bytes(cache)
        back = wire.from_bytes(blob)
        assert (back.group_size, back.dim_group_size, back.token_count, back.sealed_tokens) == \
            (tg, g, tokens, tokens // tg * tg)
        for a, b in zip(back.packed, cache.packed):
            assert a.dtype == b.dtype and a.shape == b.shape
            assert torch.equal(a[:, :tokens].view(torch.int16 if a.dtype != torch.int32 else torch.int32),
                               b[:, :tokens].view(torch.int16 if b.dtype != torch.int32 else torch.int32))
            assert not a[:, tokens:].view(torch.int16 if a.dtype != torch.int32 else torch.int32).any()
        assert back.active_keys.dtype == dtype and torch.equal(back.active_keys, cache.active_keys)
        path = str(tmp_path / f"c{tokens}.pkv")
        wire.save(cache, path)
        assert wire.to_bytes(wire.load(path)) == blob
    blob = bytearray(wire.to_bytes(_oracle_cache()))
    bad = bytearray(blob)
    bad[100] ^= 1
    with pytest.raises(ValueError, match="checksum"):
        wire.from_bytes(bytes(bad))
    with pytest.raises(ValueError, match="magic"):
        wire.from_bytes(b"NOTPOPKV" + bytes(blob[8:]))
    with pytest.raises(ValueError):
        wire.from_bytes(bytes(blob[:-40]))
    cache = _oracle_cache()
    with pytest.raises(ValueError, match="sealed_tokens"):
        wire.validate(popkv.PopKVCache(64, 64, 150, 64, cache.packed, cache.active_keys))
    with pytest.raises(ValueError, match="active_keys"):
        wire.validate(popkv.PopKVCache(64, 64, 150, 128, cache.packed, cache.active_keys[:, :3]))
    with pytest.raises(ValueError, match="k_low must be"):
        wire.validate(popkv.PopKVCache(64, 64, 150, 128, (cache.packed[0], cache.packed[1],
                                                           cache.packed[2][:, :, :1], cache.packed[3]),
                                       cache.active_keys))
    neg = cache.packed[3].clone()
    neg[0, 5, 0] = -1.0
    with pytest.raises(ValueError, match="delta must be non-negative"):
        wire.validate(popkv.PopKVCache(64, 64, 150, 128, cache.packed[:3] + (neg,), cache.active_keys),
                      check_values=True)
    # keys past fp16's range (bf16 / fp32 caches) and NaN keys: the reference
    # packer stores fp16(low), fp16(high - low) unchecked (popkv_ext.cu:139-140),
    # so such caches are valid and serialize bit for bit; the value checks are opt-in
    hot = _oracle_cache(tokens=100, tg=64, g=64, cap=128, dtype=torch.float32)
    keys = torch.randn(2, 100, 128, generator=torch.Generator().manual_seed(9))
    keys[0, 3, 7] = 1e6
    keys[1, 70, 0] = float("nan")
    from oracle import core
    import numpy as np
    planes = []
    for a, dt in zip(core.pack_keys(keys.numpy(), token_group_size=64, dim_group_size=64),
                     (torch.int32, torch.int32, torch.float16, torch.float16)):
        full = torch.zeros(2, 128, a.shape[2], dtype=dt)
        full[:, :100] = torch.from_numpy(np.ascontiguousarray(a).view(np.int32 if dt == torch.int32 else np.int16)).view(dt)
        planes.append(full)
    hot = popkv.PopKVCache(64, 64, 100, 64, tuple(planes), keys[:, 64:].clone())
    assert not bool(torch.isfinite(hot.packed[2][:, :100].float()).all() and
                    torch.isfinite(hot.packed[3][:, :100].float()).all())
    back = wire.from_bytes(wire.to_bytes(hot))
    for a, b in zip(back.packed, hot.packed):
        assert torch.equal(a.view(torch.int32 if a.dtype == torch.int32 else torch.int16),
                           b.view(torch.int32 if b.dtype == torch.int32 else torch.int16))
    with pytest.raises(ValueError, match="finite"):
        wire.to_bytes(hot, check_values=True)
    with pytest.raises(ValueError, match="token_count"):
        wire.validate(popkv.PopKVCache(64, 64, 300, 256, cache.packed, torch.zeros(2, 44, 128)))
