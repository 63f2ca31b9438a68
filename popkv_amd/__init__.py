"""MI355X-native PopKV decode-time KV retrieval.

Hand-written gfx950 HIP kernels behind a C ABI (``include/popkv_hip.h``,
``popkv_amd/_lib/libpopkv_hip.so``), with the reference's Python surface:

* ``popkv_amd.popkv_cuda``      pack_keys, pack_keys_into, query_encode,
                                score_encoded, score (reference popkv_cuda.py)
* ``popkv_amd.sparse_kernels``  indexed_attention_split_partial / _merge
                                (reference sparse_kernels.py)
* ``popkv_amd.topk``            the top-k + current-token select
* ``popkv_amd.popkv``           RetrievalConfig, PopKVCache, build/append,
                                the per-layer retrieval step (reference popkv.py)
* ``popkv_amd.decode_runtime``  DecodeEventPool (reference decode_runtime.py)
"""
from __future__ import annotations

__all__ = ["popkv_cuda", "sparse_kernels", "topk", "popkv", "decode_runtime", "workloads"]
__version__ = "0.1.0"
