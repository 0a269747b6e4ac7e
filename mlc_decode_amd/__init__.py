"""MI355X (gfx950) split-KV MLA decode behind the reference's Python entry points.

The hot path is hand-written HIP (``csrc/mla_decode.hip``) reached through the C ABI of
``include/mla_decode_amd.h``; this package is the torch-side host code around it.
"""
from .api import (Fp8KVCache, flash_mla_with_kvcache, fp8_kv_cache, get_mla_metadata,
                  get_mla_metadata_host, kv_append, merge_partials, mla_decode_absorbed,
                  mla_decode_with_kvcache, num_parts_for, prepare_w_uv, quantize_kv_cache)
from .legacy import MlaKernel

__all__ = [
    "Fp8KVCache",
    "flash_mla_with_kvcache",
    "fp8_kv_cache",
    "get_mla_metadata",
    "get_mla_metadata_host",
    "kv_append",
    "merge_partials",
    "mla_decode_absorbed",
    "mla_decode_with_kvcache",
    "num_parts_for",
    "prepare_w_uv",
    "quantize_kv_cache",
    "MlaKernel",
]
