"""ctypes binding of libpopkv_hip.so, the C ABI declared in include/popkv_hip.h.

The binding is deliberately thin: torch supplies device memory and the
current stream; every call passes raw device pointers, sizes and the
hipStream_t of ``torch.cuda.current_stream(device)``.  A nonzero status from
the library becomes a RuntimeError carrying ``popkv_last_error()`` (the
reference's TORCH_CHECK failures are RuntimeErrors as well).

There is no fallback: if the library is missing or cannot be loaded, every
call raises.
"""
from __future__ import annotations

import ctypes
import functools
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "_lib" / "libpopkv_hip.so"
HEADER_PATH = Path(__file__).resolve().parent.parent / "include" / "popkv_hip.h"

POPKV_OK = 0
DTYPE_F32, DTYPE_F16, DTYPE_BF16 = 0, 1, 2
INDEX_I64, INDEX_I32 = 0, 1
ENCODE_FOLD, ENCODE_TREE = 0, 1

_DTYPES = {torch.float32: DTYPE_F32, torch.float16: DTYPE_F16, torch.bfloat16: DTYPE_BF16}

_c_i32, _c_i64, _c_size, _vp = ctypes.c_int32, ctypes.c_int64, ctypes.c_size_t, ctypes.c_void_p

# name -> (restype, argtypes), in header order.
_SIGNATURES = {
    "popkv_status_string": (ctypes.c_char_p, [ctypes.c_int]),
    "popkv_last_error": (ctypes.c_char_p, []),
    "popkv_version": (ctypes.c_char_p, []),
    "popkv_pack": (ctypes.c_int, [_vp, _c_i32, _c_i64, _c_i64, _c_i64, _c_i64, _vp, _vp, _vp, _vp,
                                  _c_i64, _c_i64, _c_i32, _c_i32, _vp]),
    "popkv_query_encode": (ctypes.c_int, [_vp, _c_i32, _c_i64, _c_i64, _c_i32, _c_i32, _vp, _vp, _vp, _vp, _vp]),
    "popkv_score_encoded": (ctypes.c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_i64, _c_i64, _c_i64,
                                           _c_i64, _c_i64, _c_i32, _vp, _vp]),
    "popkv_score_workspace_bytes": (_c_size, [_c_i64, _c_i64, _c_i64, _c_i32]),
    "popkv_score": (ctypes.c_int, [_vp, _c_i32, _c_i64, _c_i64, _c_i64, _vp, _vp, _vp, _vp, _vp, _c_i64, _c_i64,
                                   _c_i64, _c_i32, _vp, _vp, _c_size, _vp]),
    "popkv_topk_select_workspace_bytes": (_c_size, [_c_i64, _c_i64]),
    "popkv_topk_select": (ctypes.c_int, [_vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _vp, _c_i32, _c_i64, _vp,
                                         _c_size, _vp]),
    "popkv_sparse_attention_partial": (ctypes.c_int, [_vp, _c_i32, _vp, _vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
                                                      _vp, _vp, _vp, _c_i32, _vp, _vp, _c_i64, _c_i64, _c_i64,
                                                      _c_i64, _c_i32, _vp, _vp]),
    "popkv_sparse_attention_merge": (ctypes.c_int, [_vp, _c_i64, _c_i64, _c_i64, _vp, _c_i32, _vp]),
    "popkv_layer_step_workspace_bytes": (_c_size, [_c_i64, _c_i64, _c_i64, _c_i32]),
    "popkv_layer_step_launches": (_c_i32, [_c_i64, _c_i64, _c_i64, _c_i64, _c_i32]),
    "popkv_layer_step": (ctypes.c_int, [_vp, _c_i32, _vp, _vp, _vp, _vp, _c_i64, _vp, _vp, _c_i64, _c_i64, _vp, _vp,
                                        _vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_i32, _vp, _vp, _vp, _c_size, _vp]),
    "popkv_layer_step_batched_workspace_bytes": (_c_size, [_c_i64, _c_i64, _c_i64, _c_i64, _c_i32]),
    "popkv_layer_step_batched": (ctypes.c_int, [_vp, _c_i32, _vp, _vp, _vp, _vp, _c_i64, _vp, _vp, _c_i64, _vp, _vp,
                                                _vp, _c_i64, _c_i64, _c_i64, _vp, _c_i64, _c_i64, _c_i32, _vp, _vp,
                                                _c_i64, _vp, _c_size, _vp]),
    "popkv_decode_layer_batched": (ctypes.c_int, [_vp, _c_i32, _vp, _vp, _vp, _vp, _c_i64, _vp, _vp, _c_i64, _vp, _vp,
                                                  _vp, _c_i64, _c_i64, _c_i64, _vp, _c_i64, _c_i64, _c_i32, _c_i32,
                                                  _vp, _vp, _c_i64, _vp, _vp, _c_size, _vp]),
    "popkv_append": (ctypes.c_int, [_vp, _vp, _c_i32, _vp, _vp, _c_i64, _vp, _vp, _vp, _vp, _c_i64, _vp, _c_i64,
                                    _c_i64, _c_i32, _c_i32, _vp, _vp]),
    "popkv_layer_step_scratch_bytes": (_c_size, []),
    "popkv_layer_step_noalloc": (ctypes.c_int, [_vp, _c_i32, _vp, _vp, _vp, _vp, _c_i64, _vp, _vp, _c_i64, _c_i64,
                                                _vp, _vp, _vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_i32, _vp, _vp, _vp]),
    "popkv_layer_step_attention": (ctypes.c_int, [_vp, _c_i32, _vp, _vp, _c_i64, _c_i64, _vp, _c_i64, _c_i64, _c_i64,
                                                  _c_i64, _c_i32, _vp, _c_size, _vp]),
    "popkv_dense_attention_workspace_bytes": (_c_size, [_c_i64, _c_i64]),
    "popkv_dense_attention": (ctypes.c_int, [_vp, _c_i32, _vp, _vp, _c_i64, _c_i64, _vp, _vp, _c_i64, _c_i64,
                                             _c_i64, _vp, _vp, _c_size, _vp]),
}


@functools.lru_cache(maxsize=1)
def lib() -> ctypes.CDLL:
    """Load the HIP library once; raise if it has not been built."""
    if not LIB_PATH.exists():
        raise RuntimeError(
            f"PopKV HIP library not found at {LIB_PATH}; build it with "
            "`python -m popkv_amd.build` (hipcc, gfx950)")
    handle = ctypes.CDLL(str(LIB_PATH))
    for name, (restype, argtypes) in _SIGNATURES.items():
        fn = getattr(handle, name)
        fn.restype = restype
        fn.argtypes = argtypes
    return handle


def exported_symbols() -> tuple[str, ...]:
    return tuple(_SIGNATURES)


def check(status: int) -> None:
    if status != POPKV_OK:
        L = lib()
        detail = L.popkv_last_error().decode()
        raise RuntimeError(detail or L.popkv_status_string(status).decode())


def dtype_code(t: torch.Tensor) -> int:
    try:
        return _DTYPES[t.dtype]
    except KeyError:
        raise RuntimeError(f"{t.dtype} is not supported; expected fp32/fp16/bf16") from None


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream_of(device: torch.device) -> int:
    """hipStream_t of torch's current stream on `device`, as an integer."""
    return torch.cuda.current_stream(device).cuda_stream


def call(name: str, *args) -> None:
    check(getattr(lib(), name)(*args))
