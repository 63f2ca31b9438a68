"""numpy restatement of the reference's readable PopKV references.

TEST INFRASTRUCTURE ONLY.  These are the dense-reconstruction semantics of
``popkv.py:462-735`` (``_reference_pack_bits``, ``_reference_representatives``,
``reference_query_encode``, ``reference_key_encode``, ``popkv_reference_scores``,
``popkv_reference_bitwise_scores``).  The reference compares its production
kernels against them only within tolerances (tests/test_popkv.py:208-211,
:286-289, :300); the tests here do the same for the bit-exact C oracle, so
that a dropped term, a wrong sign, index or bucket in the oracle shows up.
Sums here use float64 so the comparison is against the exact value.
"""
from __future__ import annotations

import math

import numpy as np


def pack_bits(bits: np.ndarray) -> np.ndarray:
    """Boolean [..., D] -> int32 words [..., ceil(D/32)], dim 32w+j at bit j (popkv.py:462-471)."""
    d = bits.shape[-1]
    words = math.ceil(d / 32)
    out = np.zeros((*bits.shape[:-1], words), dtype=np.int64)
    for w in range(words):
        seg = bits[..., w * 32:min((w + 1) * 32, d)].astype(np.int64)
        weights = np.left_shift(np.int64(1), np.arange(seg.shape[-1], dtype=np.int64))
        out[..., w] = (seg * weights).sum(-1)
    return out.astype(np.uint32).view(np.int32)


def representatives(values: np.ndarray, magnitude: np.ndarray, g: int):
    """Per dim-group low/high means with the empty-bucket rules (popkv.py:474-511)."""
    d = values.shape[-1]
    groups = math.ceil(d / g)
    lows, deltas = [], []
    a = np.abs(values.astype(np.float64))
    for r in range(groups):
        s, e = r * g, min((r + 1) * g, d)
        m = magnitude[..., s:e]
        lc, hc = (~m).sum(-1), m.sum(-1)
        ls = (a[..., s:e] * ~m).sum(-1)
        hs = (a[..., s:e] * m).sum(-1)
        low = np.where(lc > 0, ls / np.maximum(lc, 1), np.where(hc > 0, hs / np.maximum(hc, 1), 0.0))
        high = np.where(hc > 0, hs / np.maximum(hc, 1), low)
        lows.append(low)
        deltas.append(high - low)
    return np.stack(lows, -1), np.stack(deltas, -1)


def query_magnitude(q: np.ndarray):
    q = q.astype(np.float32)
    mn, mx = q.min(-1, keepdims=True), q.max(-1, keepdims=True)
    sign = q >= 0
    mag = np.where(sign, q > mx * np.float32(0.5), q < mn * np.float32(0.5))
    return sign, mag


def key_magnitude(k: np.ndarray, token_group_size: int):
    k = k.astype(np.float32)
    kvh, t, d = k.shape
    mn = np.empty_like(k)
    mx = np.empty_like(k)
    for s in range(0, t, token_group_size):
        e = min(s + token_group_size, t)
        mn[:, s:e] = k[:, s:e].min(1, keepdims=True)
        mx[:, s:e] = k[:, s:e].max(1, keepdims=True)
    sign = k >= 0
    mag = np.where(sign, k > mx * np.float32(0.5), k < mn * np.float32(0.5))
    return sign, mag


def reference_query_encode(q: np.ndarray, g: int = 32):
    """popkv.py:514-536."""
    sign, mag = query_magnitude(q)
    low, delta = representatives(q, mag, g)
    return pack_bits(sign), pack_bits(mag), low, delta


def reference_key_encode(k: np.ndarray, *, dim_group_size: int = 32, token_group_size: int = 32):
    """popkv.py:573-596."""
    sign, mag = key_magnitude(k, token_group_size)
    low, delta = representatives(k, mag, dim_group_size)
    return pack_bits(sign), pack_bits(mag), low, delta


def reference_scores(q, k, *, head_to_kv, group_size: int = 32, dim_group_size: int = 32) -> np.ndarray:
    """Dense reconstruction qhat . khat / sqrt(D) (popkv.py:655-689)."""
    q = q.astype(np.float32)
    k = k.astype(np.float32)
    d = q.shape[-1]
    g = dim_group_size
    qsign, qmag = query_magnitude(q)
    ql, qd = representatives(q, qmag, g)
    ksign, kmag = key_magnitude(k, group_size)
    kl, kd = representatives(k, kmag, g)
    h2k = np.asarray(head_to_kv, dtype=np.int64)
    rep = lambda x: np.repeat(x, g, -1)[..., :d]  # noqa: E731
    qhat = np.where(qsign, 1.0, -1.0) * np.where(qmag, rep(ql + qd), rep(ql))
    kl_m, kh_m = rep(kl[h2k]), rep((kl + kd)[h2k])
    khat = np.where(ksign[h2k], 1.0, -1.0) * np.where(kmag[h2k], kh_m, kl_m)
    return np.einsum("bhd,htd->bht", qhat, khat) / math.sqrt(d)


def bitwise_scores(q_enc, k_enc, *, head_to_kv, head_dim: int, dim_group_size: int) -> np.ndarray:
    """Slow popcount decomposition over already-encoded inputs (popkv.py:692-735),
    with Python int.bit_count and float64 accumulation.  Tiny inputs only."""
    qs, qm, ql, qd = q_enc
    ks, km, kl, kd = k_enc
    b_n, qh_n = qs.shape[:2]
    t_n = ks.shape[1]
    g = dim_group_size
    reps = math.ceil(head_dim / g)
    full = (1 << 32) - 1
    out = np.empty((b_n, qh_n, t_n), np.float64)
    for b in range(b_n):
        for h in range(qh_n):
            kvh = int(head_to_kv[h])
            for t in range(t_n):
                total = 0.0
                for r in range(reps):
                    s, e = r * g, min(r * g + g, head_dim)
                    c = [0, 0, 0, 0]
                    for w in range(s // 32, (e - 1) // 32 + 1):
                        ws = w * 32
                        begin, finish = max(s, ws) - ws, min(e, ws + 32) - ws
                        width = finish - begin
                        mask = (full if width == 32 else (1 << width) - 1) << begin
                        a_qs = int(qs[b, h, w]) & full
                        a_qm = int(qm[b, h, w]) & mask
                        a_ks = int(ks[kvh, t, w]) & full
                        a_km = int(km[kvh, t, w]) & mask
                        agree = (~(a_qs ^ a_ks)) & mask
                        both = a_qm & a_km
                        for i, sel in enumerate((mask, a_qm, a_km, both)):
                            c[i] += 2 * (agree & sel).bit_count() - sel.bit_count()
                    q_l, q_d = float(ql[b, h, r]), float(qd[b, h, r])
                    k_l, k_d = float(kl[kvh, t, r]), float(kd[kvh, t, r])
                    total += q_l * k_l * c[0] + q_d * k_l * c[1] + q_l * k_d * c[2] + q_d * k_d * c[3]
                out[b, h, t] = total / math.sqrt(head_dim)
    return out
