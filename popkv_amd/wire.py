"""On-disk / wire format of a PopKV retrieval cache (prefill -> decode hand-off).

The packed metadata is the reference's layout (popkv_ext.cu:1066-1070,
:1166-1171): token-major planes ``k_sign``, ``k_mag`` int32 [KVH, cap, W]
(W = 4 words of 32 dimensions, dimension 32w + j at bit j) and ``k_low``,
``k_delta`` fp16 [KVH, cap, R] (R = 128 / dim_group_size).  The reference
keeps it only in device memory and never serializes it; this module fixes a
byte format for it so a prefill process can hand a cache to a decode
process (or store it) and the receiver can check what it got:

    offset  size  field
    0       8     magic b"POPKVMD1"
    8       4     header length H (uint32, little-endian)
    12      H     header: UTF-8 JSON object (fields below)
    12+H    ...   sections, in header["sections"] order, each the raw
                  little-endian bytes of a C-contiguous array
    end-4   4     CRC-32 (zlib) of every byte before it (uint32, LE)

Header fields: ``version`` (1), ``kv_heads``, ``capacity``, ``token_count``,
``sealed_tokens``, ``group_size``, ``dim_group_size``, ``head_dim`` (128),
``words``, ``reps`` and ``sections``: a list of {"name", "dtype", "shape"}.
Only the first ``token_count`` rows of each plane are stored (rows past it
are unspecified in the reference, whose planes come from ``torch::empty``,
popkv.py:416-435); ``load`` restores the full capacity with zeros there.
The active (unsealed) keys of the last token group travel as the
``active_keys`` section so appends can resume exactly where they stopped
(popkv.py:438-459).

``validate`` checks the structural contract (dtypes, shapes, capacity and
seal rules of popkv.py:416-459); with ``check_values=True`` also the value
invariants the reference's tests assert on encoded keys of ordinary range
(tests/test_popkv.py:161-182: finite representatives, delta >= 0; low >= 0
as a mean of magnitudes).  The value checks are opt-in: the reference's
packer stores fp16(low) and fp16(high - low) with no range check
(popkv_ext.cu:139-140), so keys beyond fp16's range (|x| > 65504, possible
in fp32 or bf16) or NaN keys give valid caches with inf / NaN
representatives, and those serialize like any other.
"""
from __future__ import annotations

import json
import struct
import zlib
from typing import BinaryIO

import numpy as np
import torch

from .popkv import MAX_TOKEN_GROUP_SIZE, SPECIALIZED_TOKEN_GROUP_SIZES, PopKVCache

MAGIC = b"POPKVMD1"
VERSION = 1
_PLANES = (("k_sign", torch.int32), ("k_mag", torch.int32), ("k_low", torch.float16), ("k_delta", torch.float16))
_NP = {torch.int32: "<i4", torch.float16: "<f2", torch.bfloat16: "<i2", torch.float32: "<f4"}
_TORCH = {"int32": torch.int32, "float16": torch.float16, "bfloat16": torch.bfloat16, "float32": torch.float32}


def validate(cache: PopKVCache, *, check_values: bool = False) -> None:
    """Raise ValueError unless ``cache`` obeys the packed-metadata contract."""
    g, tg = cache.dim_group_size, cache.group_size
    if g not in (16, 32, 64):
        raise ValueError("dim_group_size must be one of 16, 32, 64")
    if not 1 <= tg <= MAX_TOKEN_GROUP_SIZE:
        raise ValueError(f"group_size must be between 1 and {MAX_TOKEN_GROUP_SIZE}")
    if g != 32 and tg not in SPECIALIZED_TOKEN_GROUP_SIZES:
        raise ValueError("non-specialized token group sizes require dim_group_size=32")
    if len(cache.packed) != 4:
        raise ValueError("packed must contain (k_sign, k_mag, k_low, k_delta)")
    k_sign = cache.packed[0]
    if k_sign.ndim != 3:
        raise ValueError("k_sign must be [KV heads, capacity, 4]")
    kvh, cap = int(k_sign.shape[0]), int(k_sign.shape[1])
    reps = 128 // g
    for t, (name, dt), width in zip(cache.packed, _PLANES, (4, 4, reps, reps)):
        if t.dtype != dt or tuple(t.shape) != (kvh, cap, width):
            raise ValueError(f"{name} must be {dt} [{kvh}, {cap}, {width}], got {t.dtype} {tuple(t.shape)}")
    n = cache.token_count
    if not 0 <= n <= cap:
        raise ValueError(f"token_count {n} outside [0, capacity {cap}]")
    if cap % tg != 0:
        raise ValueError("capacity must be a whole number of token groups")
    if cache.sealed_tokens != n // tg * tg:
        raise ValueError(f"sealed_tokens must be token_count rounded down to the group size ({n // tg * tg})")
    ak = cache.active_keys
    if ak.ndim != 3 or int(ak.shape[0]) != kvh or int(ak.shape[2]) != 128 or int(ak.shape[1]) != n - cache.sealed_tokens:
        raise ValueError(f"active_keys must be [{kvh}, {n - cache.sealed_tokens}, 128]")
    if check_values and n > 0:
        low = cache.packed[2][:, :n].float()
        delta = cache.packed[3][:, :n].float()
        if not bool(torch.isfinite(low).all()) or not bool(torch.isfinite(delta).all()):
            raise ValueError("representatives must be finite")
        if bool((delta < 0).any()):
            raise ValueError("delta must be non-negative (high >= low)")
        if bool((low < 0).any()):
            raise ValueError("low must be non-negative (a mean of magnitudes)")


def to_bytes(cache: PopKVCache, *, check_values: bool = False) -> bytes:
    """Serialize ``cache`` (validated first) in the format above."""
    validate(cache, check_values=check_values)
    n = cache.token_count
    arrays = [(name, t[:, :n]) for (name, _), t in zip(_PLANES, cache.packed)]
    arrays.append(("active_keys", cache.active_keys))
    sections, blobs = [], []
    for name, t in arrays:
        c = t.detach().cpu().contiguous()
        raw = c.view(torch.int16) if c.dtype == torch.bfloat16 else c
        blobs.append(raw.numpy().astype(_NP[c.dtype], copy=False).tobytes())
        sections.append({"name": name, "dtype": str(c.dtype).removeprefix("torch."), "shape": list(c.shape)})
    kvh, cap = int(cache.packed[0].shape[0]), int(cache.packed[0].shape[1])
    header = {"version": VERSION, "kv_heads": kvh, "capacity": cap, "token_count": n,
              "sealed_tokens": cache.sealed_tokens, "group_size": cache.group_size,
              "dim_group_size": cache.dim_group_size, "head_dim": 128, "words": 4,
              "reps": 128 // cache.dim_group_size, "sections": sections}
    hb = json.dumps(header, sort_keys=True).encode()
    body = MAGIC + struct.pack("<I", len(hb)) + hb + b"".join(blobs)
    return body + struct.pack("<I", zlib.crc32(body) & 0xFFFFFFFF)


def from_bytes(buf: bytes, *, device=None, check_values: bool = False) -> PopKVCache:
    """Parse and validate a serialized cache; the planes are restored at
    full capacity (zeros past token_count) on ``device``."""
    if len(buf) < 16 or buf[:8] != MAGIC:
        raise ValueError("not a PopKV metadata blob (bad magic)")
    (crc,) = struct.unpack("<I", buf[-4:])
    if zlib.crc32(buf[:-4]) & 0xFFFFFFFF != crc:
        raise ValueError("PopKV metadata checksum mismatch")
    (hlen,) = struct.unpack("<I", buf[8:12])
    try:
        header = json.loads(buf[12:12 + hlen].decode())
    except (UnicodeDecodeError, json.JSONDecodeError) as exc:
        raise ValueError("PopKV metadata header is not valid JSON") from exc
    if header.get("version") != VERSION:
        raise ValueError(f"unsupported PopKV metadata version {header.get('version')}")
    if header.get("head_dim") != 128 or header.get("words") != 4:
        raise ValueError("PopKV metadata must describe head_dim 128 (4 plane words)")
    kvh, cap, n = int(header["kv_heads"]), int(header["capacity"]), int(header["token_count"])
    g = int(header["dim_group_size"])
    if g not in (16, 32, 64) or header.get("reps") != 128 // g:
        raise ValueError("inconsistent dim_group_size / reps")
    names = [s["name"] for s in header["sections"]]
    if names != [p for p, _ in _PLANES] + ["active_keys"]:
        raise ValueError(f"unexpected sections {names}")
    off = 12 + hlen
    tensors = {}
    for sec in header["sections"]:
        dt = _TORCH.get(sec["dtype"])
        if dt is None:
            raise ValueError(f"unsupported section dtype {sec['dtype']}")
        shape = tuple(int(x) for x in sec["shape"])
        size = int(np.prod(shape, dtype=np.int64)) * torch.empty((), dtype=dt).element_size()
        if off + size > len(buf) - 4:
            raise ValueError("PopKV metadata blob is truncated")
        arr = np.frombuffer(buf, dtype=_NP[dt], count=size // np.dtype(_NP[dt]).itemsize, offset=off).reshape(shape)
        t = torch.from_numpy(arr.copy())
        tensors[sec["name"]] = t.view(torch.bfloat16) if dt == torch.bfloat16 else t
        off += size
    if off != len(buf) - 4:
        raise ValueError("PopKV metadata blob has trailing bytes")
    planes = []
    for (name, dt), width in zip(_PLANES, (4, 4, 128 // g, 128 // g)):
        part = tensors[name]
        if tuple(part.shape) != (kvh, n, width) or part.dtype != dt:
            raise ValueError(f"section {name} must be {dt} [{kvh}, {n}, {width}]")
        full = torch.zeros(kvh, cap, width, dtype=dt)
        full[:, :n] = part
        planes.append(full.to(device) if device is not None else full)
    ak = tensors["active_keys"]
    cache = PopKVCache(int(header["group_size"]), g, n, int(header["sealed_tokens"]), tuple(planes),
                       ak.to(device) if device is not None else ak)
    validate(cache, check_values=check_values)
    return cache


def save(cache: PopKVCache, f: str | BinaryIO, *, check_values: bool = False) -> None:
    data = to_bytes(cache, check_values=check_values)
    if isinstance(f, str):
        with open(f, "wb") as fh:
            fh.write(data)
    else:
        f.write(data)


def load(f: str | BinaryIO, *, device=None, check_values: bool = False) -> PopKVCache:
    if isinstance(f, str):
        with open(f, "rb") as fh:
            data = fh.read()
    else:
        data = f.read()
    return from_bytes(data, device=device, check_values=check_values)
