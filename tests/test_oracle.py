"""Pins the CPU oracle (oracle/popkv_oracle.c) before it is trusted as the
checker of the HIP path.

Each oracle function is checked against (a) the reference's own known-answer
tests (tests/golden/reference_kats.json), (b) the reference's readable
dense-reconstruction semantics (oracle/readable.py) within the reference's
own tolerances, and (c) what the mathematics fixes: brute-force popcount
counts with Python ints, exact rational means on dyadic inputs, numpy's
IEEE float16 conversion, a stable sort for the selection, and the
log-sum-exp identity for split attention.  Inputs are chosen so that a
dropped term, a wrong sign/index/bucket, a fold-vs-tree summation order or a
transposed operand fails at least one check.
"""
from __future__ import annotations

import json
import math
from pathlib import Path

import numpy as np
import pytest

from oracle import core, readable

GOLDEN = json.loads((Path(__file__).parent / "golden" / "reference_kats.json").read_text())
DIMS = (32, 64, 96, 127, 128)
GROUPS = (16, 32, 64)


def rng(seed):
    return np.random.default_rng(seed)


def bf16_round(x: np.ndarray) -> np.ndarray:
    """float32 -> nearest bf16 value (RNE), returned as float32."""
    u = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return core.bf16_bits_to_f32(u.astype(np.uint16))


# ------------------------------------------------------------------ conversions

def test_f16_conversion_matches_numpy_ieee():
    r = rng(0)
    x = np.concatenate([
        r.standard_normal(200000).astype(np.float32) * np.float32(3e4),
        r.standard_normal(200000).astype(np.float32) * np.float32(1e-5),   # subnormal range
        np.array([0.0, -0.0, 65504.0, 65520.0, 65519.99, -65520.0, 6.1e-5, 5.96e-8, 2.98e-8, 2.99e-8,
                  np.inf, -np.inf], np.float32),
    ])
    # exact half-way ties: values with exactly 13 dropped bits = 0x1000
    ties = (np.arange(1, 5000, dtype=np.uint32) << 13 | 0x1000) + np.uint32(0x38000000)
    x = np.concatenate([x, ties.view(np.float32)])
    got = core.f32_to_f16_bits(x)
    want = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)
    back = core.f16_bits_to_f32(got)
    assert np.array_equal(back.view(np.uint32), want.view(np.float16).astype(np.float32).view(np.uint32))


def test_inv_sqrt_dim_is_correctly_rounded():
    assert np.float32(core.inv_sqrt_dim(128)).view(np.uint32) == 0x3DB504F3
    for d in (32, 64, 96, 127, 128):
        exact = 1.0 / math.sqrt(d)
        got = core.inv_sqrt_dim(d)
        ulp = np.spacing(np.float32(got))
        assert abs(got - exact) <= 0.5 * ulp


# ------------------------------------------------------------------ query encode

def test_query_encode_hand_case_kat():
    k = GOLDEN["query_encode_hand_case"]
    q = np.array([[k["query"]]], np.float32)
    for order in ("fold", "tree"):
        if order == "tree":
            continue  # the tree encode is defined for head_dim 128 only
        s, m, low, delta = core.query_encode(q, k["dim_group_size"], order=order)
        assert int(s.item()) == k["sign"]
        assert int(m.item()) == k["magnitude"]
        assert low.item() == pytest.approx(k["low"], abs=1e-6)
        assert delta.item() == pytest.approx(k["delta"], abs=1e-6)


def test_query_encode_empty_bucket_kat():
    for case in GOLDEN["query_encode_empty_bucket"]["cases"]:
        q = np.full((1, 1, case["dims"]), case["fill"], np.float32)
        for order in ("fold",):
            _, m, low, delta = core.query_encode(q, 32, order=order)
            assert int(m.item()) == case["magnitude"]
            assert low.item() == case["low"]
            assert delta.item() == case["delta"]


def _invariant_cases():
    for c in GOLDEN["query_encode_invariant_cases"]["cases"]:
        shape = tuple(c["shape"])
        if c["kind"] == "full":
            yield np.full(shape, c["value"], np.float32)
        elif c["kind"] == "linspace":
            yield np.linspace(c["start"], c["stop"], int(np.prod(shape)), dtype=np.float32).reshape(shape)
        else:
            n = int(np.prod(shape))
            yield np.tile(np.array(c["pattern"], np.float32), n // len(c["pattern"]) + 1)[:n].reshape(shape)


@pytest.mark.parametrize("g", GROUPS)
def test_query_encode_invariants(g):
    for q in _invariant_cases():
        s, m, low, delta = core.query_encode(q, g)
        words, reps = math.ceil(q.shape[-1] / 32), math.ceil(q.shape[-1] / g)
        assert s.shape == q.shape[:-1] + (words,) and m.shape == s.shape
        assert low.shape == q.shape[:-1] + (reps,) and delta.shape == low.shape
        assert s.dtype == np.int32 and low.dtype == np.float32
        assert np.isfinite(low).all() and np.isfinite(delta).all() and (delta >= 0).all()


@pytest.mark.parametrize("g", GROUPS)
@pytest.mark.parametrize("d", DIMS)
def test_query_encode_matches_readable_reference(g, d):
    q = bf16_round(rng(17 + d + g).standard_normal((2, 8, d)).astype(np.float32))
    ref = readable.reference_query_encode(q, g)
    orders = ("fold", "tree") if d == 128 else ("fold",)
    for order in orders:
        s, m, low, delta = core.query_encode(q, g, order=order)
        assert np.array_equal(s, ref[0]) and np.array_equal(m, ref[1])
        np.testing.assert_allclose(low, ref[2], atol=2e-5, rtol=2e-5)
        np.testing.assert_allclose(delta, ref[3], atol=2e-5, rtol=2e-5)


def test_query_encode_dyadic_means_are_exact():
    """With small dyadic values every partial sum is exact, so fold and tree
    give the exact rational means."""
    r = rng(5)
    q = (r.integers(-64, 65, size=(4, 6, 128)) / 8.0).astype(np.float32)
    for g in GROUPS:
        ref = readable.reference_query_encode(q, g)
        for order in ("fold", "tree"):
            _, _, low, delta = core.query_encode(q, g, order=order)
            np.testing.assert_array_equal(low, ref[2].astype(np.float32))
            np.testing.assert_array_equal(delta, (ref[2] + ref[3]).astype(np.float32) - ref[2].astype(np.float32))


def _numpy_tree(x: np.ndarray, g: int) -> np.ndarray:
    """Vectorised float32 restatement of the production reduction trees over
    the last axis (G entries): G64 pairs j and j+32, then halving adds."""
    x = x.astype(np.float32)
    if g == 64:
        x = x[..., :32] + x[..., 32:]
    while x.shape[-1] > 1:
        h = x.shape[-1] // 2
        x = x[..., :h] + x[..., h:]
    return x[..., 0]


@pytest.mark.parametrize("g", GROUPS)
def test_query_encode_summation_orders(g):
    """fold = ascending left fold, tree = halving tree: checked against numpy
    restatements on inputs where the two orders round differently."""
    r = rng(100 + g)
    q = (r.standard_normal((64, 128)) * np.exp(r.uniform(-6, 6, (64, 128)))).astype(np.float32)
    sign, mag = readable.query_magnitude(q)
    a = np.abs(q)
    for order in ("fold", "tree"):
        _, _, low, delta = core.query_encode(q, g, order=order)
        for rep in range(128 // g):
            sl = slice(rep * g, rep * g + g)
            xl = np.where(mag[:, sl], 0.0, a[:, sl]).astype(np.float32)
            xh = np.where(mag[:, sl], a[:, sl], 0.0).astype(np.float32)
            if order == "tree":
                ls, hs = _numpy_tree(xl, g), _numpy_tree(xh, g)
            else:
                ls = np.zeros(q.shape[0], np.float32)
                hs = np.zeros(q.shape[0], np.float32)
                for j in range(g):
                    ls = np.where(~mag[:, rep * g + j], ls + xl[:, j], ls).astype(np.float32)
                    hs = np.where(mag[:, rep * g + j], hs + xh[:, j], hs).astype(np.float32)
            ln = (~mag[:, sl]).sum(-1).astype(np.float32)
            hn = mag[:, sl].sum(-1).astype(np.float32)
            with np.errstate(divide="ignore", invalid="ignore"):
                lo = np.where(ln > 0, ls / np.maximum(ln, 1), np.where(hn > 0, hs / np.maximum(hn, 1), 0)).astype(np.float32)
                hi = np.where(hn > 0, hs / np.maximum(hn, 1), lo).astype(np.float32)
            np.testing.assert_array_equal(low[:, rep], lo)
            np.testing.assert_array_equal(delta[:, rep], (hi - lo).astype(np.float32))
    # the two orders really differ on this input (so the test can tell them apart)
    f = core.query_encode(q, g, order="fold")[2]
    t = core.query_encode(q, g, order="tree")[2]
    assert not np.array_equal(f, t)


# ------------------------------------------------------------------ key pack

@pytest.mark.parametrize("g", GROUPS)
@pytest.mark.parametrize("d", DIMS)
def test_pack_matches_readable_reference(g, d):
    keys = bf16_round(rng(31 + d + g).standard_normal((2, 37, d)).astype(np.float32))
    ks, km, kl, kd = core.pack_keys(keys, dim_group_size=g)
    ref = readable.reference_key_encode(keys, dim_group_size=g, token_group_size=32)
    assert np.array_equal(ks, ref[0]) and np.array_equal(km, ref[1])
    np.testing.assert_allclose(core.f16_bits_to_f32(kl), ref[2], atol=2e-3, rtol=2e-3)
    np.testing.assert_allclose(core.f16_bits_to_f32(kd), ref[3], atol=2e-3, rtol=2e-3)


@pytest.mark.parametrize("tg", (5, 8, 10, 16, 32, 64, 125, 128, 500))
def test_pack_token_groups_match_readable_reference(tg):
    tokens = tg + 3
    keys = bf16_round(rng(37 + tg).standard_normal((2, tokens, 128)).astype(np.float32))
    for g in GROUPS if tg in (8, 16, 32, 64, 128) else (32,):
        ks, km, kl, kd = core.pack_keys(keys, token_group_size=tg, dim_group_size=g)
        ref = readable.reference_key_encode(keys, dim_group_size=g, token_group_size=tg)
        assert np.array_equal(ks, ref[0]) and np.array_equal(km, ref[1])
        np.testing.assert_allclose(core.f16_bits_to_f32(kl), ref[2], atol=2e-3, rtol=2e-3)
        np.testing.assert_allclose(core.f16_bits_to_f32(kd), ref[3], atol=2e-3, rtol=2e-3)


@pytest.mark.parametrize("g", GROUPS)
def test_pack_summation_order_is_the_tree(g):
    """Key representatives use the production tree, checked in float32 numpy
    before the fp16 rounding (fp16 of the tree sum/count)."""
    r = rng(211 + g)
    keys = (r.standard_normal((1, 64, 128)) * np.exp(r.uniform(-5, 5, (1, 64, 128)))).astype(np.float32)
    _, _, kl, kd = core.pack_keys(keys, token_group_size=64, dim_group_size=g)
    sign, mag = readable.key_magnitude(keys, 64)
    a = np.abs(keys[0])
    m = mag[0]
    for rep in range(128 // g):
        sl = slice(rep * g, rep * g + g)
        ls = _numpy_tree(np.where(m[:, sl], 0.0, a[:, sl]), g)
        hs = _numpy_tree(np.where(m[:, sl], a[:, sl], 0.0), g)
        ln = (~m[:, sl]).sum(-1).astype(np.float32)
        hn = m[:, sl].sum(-1).astype(np.float32)
        with np.errstate(divide="ignore", invalid="ignore"):
            lo = np.where(ln > 0, ls / np.maximum(ln, 1), np.where(hn > 0, hs / np.maximum(hn, 1), 0)).astype(np.float32)
            hi = np.where(hn > 0, hs / np.maximum(hn, 1), lo).astype(np.float32)
        assert np.array_equal(kl[0, :, rep], lo.astype(np.float16).view(np.uint16))
        assert np.array_equal(kd[0, :, rep], (hi - lo).astype(np.float32).astype(np.float16).view(np.uint16))


@pytest.mark.parametrize("tg", (8, 16, 32, 64, 128))
def test_incremental_append_equals_full_encode(tg):
    """append_popkv semantics (popkv.py:438-459; test_popkv.py:354-372):
    re-encoding the active group after each new token equals encoding the
    whole sequence at once, bit for bit."""
    r = rng(41 + tg)
    for g in GROUPS:
        keys = bf16_round(r.standard_normal((2, tg - 1, 128)).astype(np.float32))
        cap = math.ceil((tg - 1 + 3) / tg) * tg
        packed = core.pack_keys(keys, token_capacity=cap, token_group_size=tg, dim_group_size=g)
        sealed = ((tg - 1) // tg) * tg
        active = keys[:, sealed:]
        for _ in range(2):
            cur = bf16_round(r.standard_normal((2, 1, 128)).astype(np.float32))
            active = np.concatenate([active, cur], 1)
            keys = np.concatenate([keys, cur], 1)
            core.pack_keys_into(active, packed, token_offset=sealed, token_group_size=tg, dim_group_size=g)
            if active.shape[1] == tg:
                sealed += tg
                active = active[:, :0]
            full = core.pack_keys(keys, token_group_size=tg, dim_group_size=g)
            n = keys.shape[1]
            for a, b in zip(packed, full):
                assert np.array_equal(a[:, :n], b)


def test_magnitude_rule_equals_two_compares():
    """The HIP encode forms the magnitude bit as (v > 0.5*max) | (v < 0.5*min)
    without a sign-dependent select; the reference's rule is
    v >= 0 ? v > 0.5*max : v < 0.5*min with max / min over the group (NaNs
    ignored, as fmaxf / fminf do).  The two agree on every element of groups
    built from signed zeros, subnormals, ties at half an extremum, infinities,
    NaNs and random values, including all-negative and all-positive groups."""
    g = rng(11)
    special = np.array([0.0, -0.0, 1e-45, -1e-45, 2.0 ** -126, -(2.0 ** -126), 0.5, -0.5, 1.0, -1.0, 2.0, -2.0,
                        4.0, -4.0, np.inf, -np.inf, np.nan, 3.4e38, -3.4e38], np.float32)
    cases = [special, np.abs(special), -np.abs(special)]
    for _ in range(300):
        n = int(g.integers(1, 9))
        vals = np.concatenate([g.choice(special, n), (g.standard_normal(n) * 10.0 ** g.integers(-40, 38))])
        cases.append(g.permutation(vals).astype(np.float32))
    with np.errstate(over="ignore", invalid="ignore"):
        for v in cases:
            mx = np.fmax.reduce(v)  # NaNs ignored, like fmaxf
            mn = np.fmin.reduce(v)
            hi, lo = np.float32(mx * np.float32(0.5)), np.float32(mn * np.float32(0.5))
            ref = np.where(v >= 0, v > hi, v < lo)
            two = (v > hi) | (v < lo)
            assert np.array_equal(ref, two), v


def test_pack_capacity_exceeded():
    keys = np.zeros((1, 10, 128), np.float32)
    packed = core.alloc_packed(1, 12, 128, 32)
    with pytest.raises(RuntimeError, match="capacity exceeded"):
        core.pack_keys_into(keys, packed, token_offset=3, token_group_size=32, dim_group_size=32)


# ------------------------------------------------------------------ score

def _f16_ulp(x: np.ndarray) -> np.ndarray:
    return np.spacing(np.abs(x).astype(np.float16)).astype(np.float64)


@pytest.mark.parametrize("g", GROUPS)
def test_score_d128_matches_bitwise_bruteforce(g):
    """The popcount counts and the fma chain against Python-int popcounts with
    float64 accumulation (popkv.py:692-735) on the same encodings: within one
    fp16 ulp (fp16 rounding of an fp32 sum)."""
    r = rng(300 + g)
    q = bf16_round(r.standard_normal((1, 8, 128)).astype(np.float32))
    keys = bf16_round(r.standard_normal((2, 23, 128)).astype(np.float32))
    mapping = np.arange(8) // 4
    enc = core.query_encode(q, g, order="fold")
    packed = core.pack_keys(keys, token_group_size=8, dim_group_size=g)
    got = core.f16_bits_to_f32(core.score_encoded(enc, packed, head_to_kv=mapping, tokens=23, dim_group_size=g))
    kenc = (packed[0], packed[1], core.f16_bits_to_f32(packed[2]), core.f16_bits_to_f32(packed[3]))
    want = readable.bitwise_scores(enc, kenc, head_to_kv=mapping, head_dim=128, dim_group_size=g)
    err = np.abs(got - want)
    assert (err <= _f16_ulp(want) + 1e-7).all(), err.max()


@pytest.mark.parametrize("g", GROUPS)
@pytest.mark.parametrize("d", (32, 64, 96, 127))
def test_score_generic_matches_bitwise_bruteforce(g, d):
    r = rng(400 + g + d)
    q = bf16_round(r.standard_normal((1, 8, d)).astype(np.float32))
    keys = bf16_round(r.standard_normal((2, 17, d)).astype(np.float32))
    mapping = np.arange(8) // 4
    enc = core.query_encode(q, g, order="fold")
    packed = core.pack_keys(keys, dim_group_size=g)
    got = core.score_generic(enc, packed, head_to_kv=mapping, head_dim=d, tokens=17, dim_group_size=g)
    kenc = (packed[0], packed[1], core.f16_bits_to_f32(packed[2]), core.f16_bits_to_f32(packed[3]))
    want = readable.bitwise_scores(enc, kenc, head_to_kv=mapping, head_dim=d, dim_group_size=g)
    np.testing.assert_allclose(got, want, atol=2e-5, rtol=2e-5)


@pytest.mark.parametrize("g", GROUPS)
@pytest.mark.parametrize("d", DIMS)
def test_score_matches_dense_reconstruction(g, d):
    """popkv_cuda.score semantics vs popkv_reference_scores, at the reference's
    own tolerance (tests/test_popkv.py:298-300)."""
    r = rng(31 + d * 3 + g)
    keys = bf16_round(r.standard_normal((2, 37, d)).astype(np.float32))
    q = bf16_round(r.standard_normal((1, 8, d)).astype(np.float32))
    mapping = np.arange(8) // 4
    packed = core.pack_keys(keys, dim_group_size=g)
    got = core.score(q, packed, head_to_kv=mapping, tokens=37, dim_group_size=g)
    got = core.f16_bits_to_f32(got) if d == 128 else got
    want = readable.reference_scores(q, keys, head_to_kv=mapping, dim_group_size=g)
    np.testing.assert_allclose(got, want, atol=0.15, rtol=0.025)


def test_popcount_decomposition_kat():
    """test_popkv.py:262-273: bitwise decomposition == dense reconstruction."""
    k = GOLDEN["popcount_decomposition_query"]
    q = np.tile(np.array(k["pattern"], np.float32), k["repeat"])[None, None, :]
    keys = np.stack([q[0, 0], -q[0, 0]], 0)[None]
    mapping = np.array([0])
    for g in k["dim_group_sizes"]:
        enc = core.query_encode(q, g, order="fold")
        packed = core.pack_keys(keys, dim_group_size=g)
        kenc = (packed[0], packed[1], core.f16_bits_to_f32(packed[2]), core.f16_bits_to_f32(packed[3]))
        bit = readable.bitwise_scores(enc, kenc, head_to_kv=mapping, head_dim=64, dim_group_size=g)
        direct = readable.reference_scores(q, keys, head_to_kv=mapping, dim_group_size=g)
        np.testing.assert_allclose(bit, direct, atol=k["tolerance"], rtol=k["tolerance"])
        got = core.score_generic(enc, packed, head_to_kv=mapping, head_dim=64, tokens=2, dim_group_size=g)
        np.testing.assert_allclose(got, direct, atol=1e-5, rtol=1e-5)


def test_score_gqa_uses_first_head_of_group():
    """The head_dim-128 scorer maps a whole GQA group through the mapping of
    its first head (popkv_ext.cu:768-774)."""
    r = rng(9)
    q = bf16_round(r.standard_normal((1, 4, 128)).astype(np.float32))
    keys = bf16_round(r.standard_normal((2, 8, 128)).astype(np.float32))
    packed = core.pack_keys(keys, dim_group_size=64)
    enc = core.query_encode(q, 64)
    a = core.score_encoded(enc, packed, head_to_kv=np.array([0, 0, 1, 1]), tokens=8, dim_group_size=64)
    b = core.score_encoded(enc, packed, head_to_kv=np.array([0, 1, 1, 0]), tokens=8, dim_group_size=64)
    assert np.array_equal(a, b)


# ------------------------------------------------------------------ select

def _brute_select(bits: np.ndarray, k: int, current: int) -> np.ndarray:
    keys = core.order_key(bits).astype(np.int64)
    out = []
    for row in keys:
        order = np.lexsort((np.arange(row.size), -row))  # key desc, then index asc
        out.append(np.concatenate([np.sort(order[:k]), [current]]))
    return np.array(out, np.int64)


def test_order_key_is_monotone_and_signed_zero_aware():
    vals = np.array([-np.inf, -65504, -1.5, -1e-7, -0.0, 0.0, 1e-7, 1.5, 65504, np.inf], np.float16)
    keys = core.order_key(vals.view(np.uint16)).astype(np.int64)
    assert (np.diff(keys) > 0).all()          # -0 < +0 included
    nan = np.array([np.nan], np.float16).view(np.uint16)
    assert core.order_key(nan)[0] == 0xFFFF


@pytest.mark.parametrize("case", ["random", "ties", "few_values", "signed_zero", "nan"])
def test_select_matches_stable_sort(case):
    r = rng(hash(case) % 1000)
    rows, t = 5, 777
    if case == "random":
        x = r.standard_normal((rows, t)).astype(np.float16)
    elif case == "ties":
        x = r.integers(-3, 4, (rows, t)).astype(np.float16)
    elif case == "few_values":
        x = np.where(r.random((rows, t)) < 0.5, 1.0, 2.0).astype(np.float16)
    elif case == "signed_zero":
        x = np.where(r.random((rows, t)) < 0.5, -0.0, 0.0).astype(np.float16)
    else:
        x = r.standard_normal((rows, t)).astype(np.float16)
        x[:, ::50] = np.nan
    bits = x.view(np.uint16)
    for k in (0, 1, 5, 100, 400, t - 1, t):
        got = core.select(bits, k, t)
        assert np.array_equal(got, _brute_select(bits, k, t))


def test_select_signed_zero_prefers_positive_zero_then_low_index():
    x = np.array([[-0.0, 0.0, -0.0, 0.0, -1.0]], np.float16)
    got = core.select(x.view(np.uint16), 3, 5)
    assert got.tolist() == [[1, 3, 0, 5]] or sorted(got[0, :3].tolist()) == [0, 1, 3]
    assert sorted(got[0, :3].tolist()) == [0, 1, 3] and got[0, 3] == 5


# ------------------------------------------------------------------ attention

def _softmax_attention(q, keys, values, cur_k, cur_v, idx, mapping, valid=None):
    qh, d = q.shape
    out = np.zeros((qh, d))
    t_prefix = keys.shape[1]
    for h in range(qh):
        kv = mapping[h]
        rows = idx[h]
        kr = np.where((rows == t_prefix)[:, None], cur_k[kv][None], keys[kv, np.minimum(rows, t_prefix - 1)])
        vr = np.where((rows == t_prefix)[:, None], cur_v[kv][None], values[kv, np.minimum(rows, t_prefix - 1)])
        logits = kr.astype(np.float64) @ q[h].astype(np.float64) / math.sqrt(d)
        if valid is not None:
            logits = np.where(valid[h], logits, -np.inf)
        p = np.exp(logits - logits.max())
        out[h] = (p[:, None] * vr).sum(0) / p.sum()
    return out


def test_attention_matches_numpy_softmax():
    r = rng(104)
    qh, kvh, t, d = 8, 2, 300, 128
    q = r.standard_normal((qh, d)).astype(np.float32)
    keys = r.standard_normal((kvh, t, d)).astype(np.float32)
    values = r.standard_normal((kvh, t, d)).astype(np.float32)
    ck = r.standard_normal((kvh, d)).astype(np.float32)
    cv = r.standard_normal((kvh, d)).astype(np.float32)
    mapping = np.arange(qh) // 4
    idx = r.integers(0, t, (qh, 100))
    idx[:, -1] = t
    valid = np.ones(idx.shape, bool)
    valid[:, -7:-1] = False
    for vm in (None, valid):
        got = core.attention(q, keys, values, ck, cv, idx, mapping, vm)
        want = _softmax_attention(q, keys, values, ck, cv, idx, mapping, vm)
        np.testing.assert_allclose(got, want, atol=1e-5, rtol=1e-5)


def test_attention_merge_is_the_lse_identity():
    r = rng(7)
    qh, s, d = 4, 5, 16
    logits = r.standard_normal((qh, s, 32)) * 3
    vals = r.standard_normal((qh, s, 32, d))
    parts = np.zeros((qh, s, d + 2), np.float32)
    m = logits.max(-1)
    p = np.exp(logits - m[..., None])
    parts[..., 0] = m
    parts[..., 1] = p.sum(-1)
    parts[..., 2:] = (p[..., None] * vals).sum(2)
    got = core.attention_merge(parts)
    allp = np.exp(logits.reshape(qh, -1) - logits.reshape(qh, -1).max(-1, keepdims=True))
    want = (allp[..., None] * vals.reshape(qh, -1, d)).sum(1) / allp.sum(-1, keepdims=True)
    np.testing.assert_allclose(got, want, atol=1e-5, rtol=1e-5)
    # a fully masked split (m = -inf, l = 0) contributes nothing
    parts2 = np.concatenate([parts, np.zeros((qh, 1, d + 2), np.float32)], 1)
    parts2[:, -1, 0] = -np.inf
    np.testing.assert_allclose(core.attention_merge(parts2), got, atol=1e-6, rtol=1e-6)


def test_torch_cpu_baseline_matches_readable_semantics():
    """The torch-CPU baseline bench.py times restates the readable path:
    its key / query encodes give the numpy restatement's bits and (within
    float rounding) representatives, its dense-reconstruction scores the
    numpy scores, and its step equals a float64 softmax over the rows its
    own top-k picked plus the current token."""
    import math

    import numpy as np
    import torch

    from oracle import readable, torch_cpu

    g = torch.Generator().manual_seed(5)
    k = torch.randn(2, 150, 128, generator=g)
    v = torch.randn(2, 150, 128, generator=g)
    q = torch.randn(8, 128, generator=g)
    h2k = torch.arange(8) // 4
    for tg, gg in ((32, 32), (64, 64), (128, 16), (7, 32)):
        ks, km, kl, kd = torch_cpu.key_encode(k, tg, gg)
        rs, rm = readable.key_magnitude(k.numpy(), tg)
        assert np.array_equal(ks.numpy(), rs) and np.array_equal(km.numpy(), rm)
        lo, de = readable.representatives(k.numpy(), rm, gg)
        np.testing.assert_allclose(kl.numpy(), lo, atol=1e-6)
        np.testing.assert_allclose(kd.numpy(), de, atol=1e-6)
        qs, qm, ql, qd = torch_cpu.query_encode(q, gg)
        want = readable.reference_query_encode(q.numpy(), gg)
        assert np.array_equal(readable.pack_bits(qs.numpy()), want[0])
        assert np.array_equal(readable.pack_bits(qm.numpy()), want[1])
        np.testing.assert_allclose(ql.numpy(), want[2], atol=1e-6)
        want_s = readable.reference_scores(q[None].numpy(), k.numpy(), head_to_kv=h2k.numpy(), group_size=tg,
                                           dim_group_size=gg)[0]
        qhat = torch_cpu.reconstruct(qs, qm, ql, qd, gg)
        khat = torch_cpu.reconstruct(ks, km, kl, kd, gg)
        got_s = torch.einsum("hd,htd->ht", qhat, khat[h2k]) / math.sqrt(128)
        np.testing.assert_allclose(got_s.numpy(), want_s, atol=1e-5)
    layer = torch_cpu.CpuRetrievalLayer(k[:, :-1], v[:, :-1], h2k, token_group=64, dim_group=64)
    out = layer.step(q, k[:, -1], v[:, -1], budget=40)
    assert out.shape == (8, 128)
    qhat = torch_cpu.reconstruct(*torch_cpu.query_encode(q, 64), 64)
    sc = (torch.einsum("hd,htd->ht", qhat, layer.khat[h2k]) / math.sqrt(128)).half()
    idx = torch.topk(sc, 39, dim=-1, sorted=False).indices
    for h in range(8):
        rows_k = torch.cat([k[h2k[h], idx[h]], k[h2k[h], -1:]]).double()
        rows_v = torch.cat([v[h2k[h], idx[h]], v[h2k[h], -1:]]).double()
        p = torch.softmax(rows_k @ q[h].double() / math.sqrt(128), 0)
        np.testing.assert_allclose(out[h].numpy(), (p @ rows_v).numpy(), atol=1e-5)
