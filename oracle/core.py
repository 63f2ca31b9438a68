"""ctypes front end of the C oracle (``oracle/popkv_oracle.c``).

TEST INFRASTRUCTURE ONLY: the checker for the HIP path, never the product.

Every function takes and returns numpy arrays.  Float inputs are float32
(bf16/fp16 tensors are widened exactly before they get here); fp16 outputs
are returned as their uint16 bit patterns so comparisons are bit-exact.
"""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

_DIR = Path(__file__).resolve().parent
_LIB_PATH = _DIR / "libpopkv_oracle.so"
_lib = None

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
_i64p = np.ctypeslib.ndpointer(np.int64, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
_i64 = ctypes.c_int64
_int = ctypes.c_int


def build(force: bool = False) -> Path:
    """Compile the oracle with its Makefile (gcc, IEEE binary32); with
    ``force`` even when the library is newer than its source."""
    subprocess.run(["make", "-s"] + (["-B"] if force else []) + ["-C", str(_DIR), "libpopkv_oracle.so"], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        src = _DIR / "popkv_oracle.c"
        if not _LIB_PATH.exists() or _LIB_PATH.stat().st_mtime < src.stat().st_mtime:
            build()
        L = ctypes.CDLL(str(_LIB_PATH))
        L.po_f32_to_f16.argtypes = [ctypes.c_float]
        L.po_f32_to_f16.restype = ctypes.c_uint16
        L.po_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.po_f16_to_f32.restype = ctypes.c_float
        L.po_f32_to_f16_array.argtypes = [_f32p, _u16p, _i64]
        L.po_inv_sqrt_dim.argtypes = [_i64]
        L.po_inv_sqrt_dim.restype = ctypes.c_float
        L.po_order_key_f16.argtypes = [ctypes.c_uint16]
        L.po_order_key_f16.restype = ctypes.c_uint16
        L.po_query_encode.argtypes = [_f32p, _i64, _i64, _int, _int, _i32p, _i32p, _f32p, _f32p]
        L.po_pack_keys.argtypes = [_f32p, _i64, _i64, _i64, _int, _int, _i32p, _i32p, _u16p, _u16p, _i64, _i64]
        L.po_score_d128.argtypes = [_i32p, _i32p, _f32p, _f32p, _i32p, _i32p, _u16p, _u16p, _i64p,
                                    _i64, _i64, _i64, _i64, _i64, _int, _u16p]
        L.po_score_generic.argtypes = [_i32p, _i32p, _f32p, _f32p, _i32p, _i32p, _u16p, _u16p, _i64p,
                                       _i64, _i64, _i64, _i64, _i64, _int, _f32p]
        L.po_select.argtypes = [_u16p, _i64, _i64, _i64, _i64, _i64, _i64p]
        L.po_attention.argtypes = [_f32p, _f32p, _f32p, _i64, _i64, _i64, _i64, _i64, _f32p, _f32p,
                                   _i64p, ctypes.c_void_p, _i64p, _i64, _i64, _i64, _f32p]
        L.po_attention_merge.argtypes = [_f32p, _i64, _i64, _i64, _f32p]
        _lib = L
    return _lib


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


# ---------------------------------------------------------------- conversions

def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return np.asarray(bits, dtype=np.uint16).view(np.float16).astype(np.float32)


def f32_to_f16_bits(x: np.ndarray) -> np.ndarray:
    x = _c(x, np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().po_f32_to_f16_array(x.reshape(-1), out.reshape(-1), x.size)
    return out


def inv_sqrt_dim(d: int) -> float:
    return float(lib().po_inv_sqrt_dim(int(d)))


def order_key(bits: np.ndarray) -> np.ndarray:
    """Vectorised po_order_key_f16."""
    h = np.asarray(bits, dtype=np.uint16).astype(np.uint32)
    key = np.where(h & 0x8000, (~h) & 0xFFFF, h | 0x8000)
    nan = ((h & 0x7C00) == 0x7C00) & ((h & 0x3FF) != 0)
    return np.where(nan, 0xFFFF, key).astype(np.uint16)


# ---------------------------------------------------------------- encode / pack

def query_encode(q: np.ndarray, dim_group_size: int = 32, *, order: str = "fold"):
    """q [..., D] float32 -> (sign i32 [..., W], mag i32, low f32 [..., R], delta f32).

    order="fold": decode-path encode (popkv_ext.cu:232-281, :911-957).
    order="tree": score()-path warp encode, D == 128 (popkv_ext.cu:677-755).
    """
    q = _c(q, np.float32)
    lead, d = q.shape[:-1], int(q.shape[-1])
    rows = int(np.prod(lead)) if lead else 1
    g = int(dim_group_size)
    w, r = (d + 31) // 32, (d + g - 1) // g
    sign = np.empty((rows, w), np.int32)
    mag = np.empty((rows, w), np.int32)
    low = np.empty((rows, r), np.float32)
    delta = np.empty((rows, r), np.float32)
    lib().po_query_encode(q.reshape(rows, d), rows, d, g, 0 if order == "fold" else 1, sign, mag, low, delta)
    return (sign.reshape(*lead, w), mag.reshape(*lead, w), low.reshape(*lead, r), delta.reshape(*lead, r))


def alloc_packed(kv_heads: int, capacity: int, head_dim: int, dim_group_size: int):
    w = (head_dim + 31) // 32
    r = (head_dim + dim_group_size - 1) // dim_group_size
    return (np.zeros((kv_heads, capacity, w), np.int32), np.zeros((kv_heads, capacity, w), np.int32),
            np.zeros((kv_heads, capacity, r), np.uint16), np.zeros((kv_heads, capacity, r), np.uint16))


def pack_keys_into(keys: np.ndarray, packed, *, token_offset: int, token_group_size: int,
                   dim_group_size: int) -> None:
    """Encode keys [KVH, n, D] into rows [token_offset, token_offset+n) of packed."""
    keys = _c(keys, np.float32)
    kvh, n, d = (int(x) for x in keys.shape)
    sign, mag, low, delta = packed
    cap = int(sign.shape[1])
    if token_offset < 0 or token_offset + n > cap:
        raise RuntimeError("Pop-KV cache capacity exceeded")
    lib().po_pack_keys(keys, kvh, n, d, int(token_group_size), int(dim_group_size),
                       sign, mag, low, delta, cap, int(token_offset))


def pack_keys(keys: np.ndarray, *, token_capacity: int | None = None, token_group_size: int = 32,
              dim_group_size: int = 32):
    keys = _c(keys, np.float32)
    kvh, n, d = (int(x) for x in keys.shape)
    packed = alloc_packed(kvh, n if token_capacity is None else int(token_capacity), d, dim_group_size)
    pack_keys_into(keys, packed, token_offset=0, token_group_size=token_group_size,
                   dim_group_size=dim_group_size)
    return packed


# ---------------------------------------------------------------- score

def score_encoded(encoded, packed, *, head_to_kv, tokens: int, dim_group_size: int) -> np.ndarray:
    """head_dim 128 GQA scorer (popkv_ext.cu:757-876) -> fp16 bits [B, QH, tokens]."""
    qs, qm, ql, qd = (_c(x, t) for x, t in zip(encoded, (np.int32, np.int32, np.float32, np.float32)))
    ks, km, kl, kd = (_c(x, t) for x, t in zip(packed, (np.int32, np.int32, np.uint16, np.uint16)))
    b, qh = int(qs.shape[0]), int(qs.shape[1])
    kvh, cap = int(ks.shape[0]), int(ks.shape[1])
    out = np.empty((b, qh, int(tokens)), np.uint16)
    lib().po_score_d128(qs, qm, ql, qd, ks, km, kl, kd, _c(head_to_kv, np.int64), b, qh, kvh, cap,
                        int(tokens), int(dim_group_size), out)
    return out


def score_generic(encoded, packed, *, head_to_kv, head_dim: int, tokens: int, dim_group_size: int) -> np.ndarray:
    """Generic-D scorers (popkv_ext.cu:145-230, :517-675) -> float32 [B, QH, tokens]."""
    qs, qm, ql, qd = (_c(x, t) for x, t in zip(encoded, (np.int32, np.int32, np.float32, np.float32)))
    ks, km, kl, kd = (_c(x, t) for x, t in zip(packed, (np.int32, np.int32, np.uint16, np.uint16)))
    b, qh = int(qs.shape[0]), int(qs.shape[1])
    out = np.empty((b, qh, int(tokens)), np.float32)
    lib().po_score_generic(qs, qm, ql, qd, ks, km, kl, kd, _c(head_to_kv, np.int64), b, qh,
                           int(head_dim), int(ks.shape[1]), int(tokens), int(dim_group_size), out)
    return out


def score(q: np.ndarray, packed, *, head_to_kv, tokens: int, dim_group_size: int = 32) -> np.ndarray:
    """popkv_cuda.score semantics (popkv_cuda.py:190-204): D == 128 -> tree-order
    warp encode + GQA scorer, fp16 bits; otherwise fold encode + generic scorer, f32."""
    q = _c(q, np.float32)
    d = int(q.shape[-1])
    if d == 128 and int(packed[0].shape[2]) == 4:
        enc = query_encode(q, dim_group_size, order="tree")
        return score_encoded(enc, packed, head_to_kv=head_to_kv, tokens=tokens, dim_group_size=dim_group_size)
    enc = query_encode(q, dim_group_size, order="fold")
    return score_generic(enc, packed, head_to_kv=head_to_kv, head_dim=d, tokens=tokens,
                         dim_group_size=dim_group_size)


# ---------------------------------------------------------------- select

def select(scores_f16_bits: np.ndarray, k: int, current: int) -> np.ndarray:
    """[rows, T] fp16 bits -> int64 [rows, k+1]: top-k ascending + current."""
    s = _c(scores_f16_bits, np.uint16)
    rows, t = int(s.shape[0]), int(s.shape[1])
    out = np.empty((rows, int(k) + 1), np.int64)
    lib().po_select(s, rows, t, t, int(k), int(current), out)
    return out


# ---------------------------------------------------------------- attention

def attention(q, prefix_k, prefix_v, cur_k, cur_v, indices, head_to_kv, valid=None) -> np.ndarray:
    """float64-accumulated materialized attention over gathered rows -> f32 [QH, D].
    prefix_k/prefix_v: [KVH, T, D] float32 (contiguous)."""
    q = _c(q, np.float32)
    pk, pv = _c(prefix_k, np.float32), _c(prefix_v, np.float32)
    kvh, t, d = (int(x) for x in pk.shape)
    idx = _c(indices, np.int64)
    qh, s = int(idx.shape[0]), int(idx.shape[1])
    out = np.empty((qh, d), np.float32)
    vm = None if valid is None else _c(valid, np.uint8)
    lib().po_attention(q, pk, pv, t * d, d, t * d, d, t, _c(cur_k, np.float32), _c(cur_v, np.float32),
                       idx, None if vm is None else vm.ctypes.data_as(ctypes.c_void_p),
                       _c(head_to_kv, np.int64), qh, d, s, out)
    return out


def attention_merge(partials: np.ndarray) -> np.ndarray:
    p = _c(partials, np.float32)
    qh, s, sd = (int(x) for x in p.shape)
    out = np.empty((qh, sd - 2), np.float32)
    lib().po_attention_merge(p, qh, s, sd - 2, out)
    return out
