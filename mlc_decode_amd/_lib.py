"""ctypes binding of the C ABI in ``include/mla_decode_amd.h``.

Mirrors the reference's ctypes host wrapper (handmade/mla_handmade.py:97-107: CDLL +
explicit argtypes) with explicit restypes, a nonzero-status check and the library's
error message.  There is no fallback: if the built library is missing, loading raises.
"""
from __future__ import annotations

import ctypes
import os
import threading

from .build import LIB_PATH

MLA_DTYPE_BF16 = 0
MLA_DTYPE_F16 = 1
MLA_SCHED_WORDS = 8
MLA_DEFAULT_SPLIT_OVERHEAD = 3  # pages; the default schedule's per-split overhead
MLA_KV_NATIVE = 0
MLA_KV_FP8_E4M3 = 1
MLA_SPARSE_MAX_TOPK = 2048
MLA_NOALLOC_SCRATCH_BYTES = 160 << 20  # the allocation-free decode's static scratch per GPU
MLA_DIM_QK = 576
MLA_DIM_V = 512
MLA_PAGE_TOKENS = 64

# Every symbol include/mla_decode_amd.h declares.
EXPORTED = (
    "mla_version",
    "mla_last_error",
    "mla_num_parts",
    "mla_variant",
    "mla_get_metadata",
    "mla_get_metadata_host",
    "mla_workspace_bytes",
    "mla_decode_fwd",
    "mla_decode_fwd_noalloc",
    "mla_splitkv_fwd",
    "mla_combine_fwd",
    "mla_merge_partials",
    "mla_split_plan",
    "mla_launch",
    "mla_kv_append",
    "mla_combine_absorb",
)

_i32, _i64, _f32, _vp = ctypes.c_int32, ctypes.c_int64, ctypes.c_float, ctypes.c_void_p
_pi32 = ctypes.POINTER(ctypes.c_int32)


class MlaDecodeArgs(ctypes.Structure):
    """Layout of ``mla_decode_args`` (include/mla_decode_amd.h)."""

    _fields_ = [
        ("batch", _i32),
        ("s_q", _i32),
        ("heads_q", _i32),
        ("heads_k", _i32),
        ("dtype", _i32),
        ("causal", _i32),
        ("sm_scale", _f32),
        ("num_blocks", _i32),
        ("q_nope", _vp),
        ("q_rope", _vp),
        ("q_stride_b", _i64),
        ("q_stride_s", _i64),
        ("q_stride_h", _i64),
        ("q_rope_stride_b", _i64),
        ("q_rope_stride_s", _i64),
        ("q_rope_stride_h", _i64),
        ("kv_nope", _vp),
        ("kv_rope", _vp),
        ("kv_stride_page", _i64),
        ("kv_stride_tok", _i64),
        ("kv_stride_batch", _i64),
        ("kv_rope_stride_page", _i64),
        ("kv_rope_stride_tok", _i64),
        ("kv_rope_stride_batch", _i64),
        ("block_table", _vp),
        ("block_table_stride", _i32),
        ("num_parts", _i32),
        ("cache_seqlens", _vp),
        ("tile_sched", _vp),
        ("num_splits", _vp),
        ("out", _vp),
        ("o_stride_b", _i64),
        ("o_stride_s", _i64),
        ("o_stride_h", _i64),
        ("lse", _vp),
        ("workspace", _vp),
        ("workspace_bytes", _i64),
        ("kv_format", _i32),
        ("kv_reserved", _i32),
        ("kv_scale", _vp),
        ("kv_scale_stride_page", _i64),
        ("kv_scale_stride_blk", _i64),
        ("indices", _vp),
        ("indices_stride", _i32),
        ("topk", _i32),
        ("block_table_width", _i32),
        ("table_reserved", _i32),
        ("status", _vp),
    ]


class MlaKvAppendArgs(ctypes.Structure):
    """Layout of ``mla_kv_append_args`` (include/mla_decode_amd.h)."""

    _fields_ = [
        ("batch", _i32),
        ("n_new", _i32),
        ("dtype", _i32),
        ("num_blocks", _i32),
        ("kv_new", _vp),
        ("new_stride_b", _i64),
        ("new_stride_t", _i64),
        ("kv_nope", _vp),
        ("kv_rope", _vp),
        ("kv_stride_page", _i64),
        ("kv_stride_tok", _i64),
        ("kv_rope_stride_page", _i64),
        ("kv_rope_stride_tok", _i64),
        ("block_table", _vp),
        ("block_table_stride", _i32),
        ("max_pages", _i32),
        ("cache_seqlens", _vp),
        ("status", _vp),
        ("kv_format", _i32),
        ("kv_reserved", _i32),
        ("kv_scale", _vp),
        ("kv_scale_stride_page", _i64),
        ("kv_scale_stride_blk", _i64),
    ]


class MlaError(RuntimeError):
    """A nonzero status from the C ABI, carrying the library's message."""

    def __init__(self, fn: str, code: int, msg: str):
        super().__init__(f"{fn} failed with status {code}: {msg}")
        self.code = code


_lock = threading.Lock()
_lib = None


def library_path() -> str:
    return LIB_PATH


def load() -> ctypes.CDLL:
    """Load the built library (once).  Raises if it has not been built."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -m mlc_decode_amd.build` "
                "(the HIP library is required; there is no CPU fallback)"
            )
        lib = ctypes.CDLL(LIB_PATH)
        lib.mla_version.argtypes = []
        lib.mla_version.restype = ctypes.c_int
        lib.mla_last_error.argtypes = []
        lib.mla_last_error.restype = ctypes.c_char_p
        lib.mla_num_parts.argtypes = [_i32, _i32, _i32, _i32, _i32]
        lib.mla_num_parts.restype = ctypes.c_int
        lib.mla_variant.argtypes = [_i32, _pi32, _pi32, _pi32, _pi32]
        lib.mla_variant.restype = ctypes.c_int
        lib.mla_get_metadata.argtypes = [_vp, _i32, _i32, _i32, _i32, _vp, _vp, _vp]
        lib.mla_get_metadata.restype = ctypes.c_int
        lib.mla_get_metadata_host.argtypes = [_pi32, _i32, _i32, _i32, _i32, _pi32, _pi32]
        lib.mla_get_metadata_host.restype = ctypes.c_int
        lib.mla_workspace_bytes.argtypes = [_i32, _i32, _i32, _i32]
        lib.mla_workspace_bytes.restype = ctypes.c_int64
        lib.mla_decode_fwd.argtypes = [ctypes.POINTER(MlaDecodeArgs), _vp]
        lib.mla_decode_fwd.restype = ctypes.c_int
        lib.mla_decode_fwd_noalloc.argtypes = [ctypes.POINTER(MlaDecodeArgs), _vp]
        lib.mla_decode_fwd_noalloc.restype = ctypes.c_int
        lib.mla_splitkv_fwd.argtypes = [ctypes.POINTER(MlaDecodeArgs), _vp]
        lib.mla_splitkv_fwd.restype = ctypes.c_int
        lib.mla_combine_fwd.argtypes = [ctypes.POINTER(MlaDecodeArgs), _vp]
        lib.mla_combine_fwd.restype = ctypes.c_int
        lib.mla_merge_partials.argtypes = [_vp, _vp, _vp, _i32, _i32, _i32, _vp, _vp, _vp]
        lib.mla_merge_partials.restype = ctypes.c_int
        lib.mla_split_plan.argtypes = [_i32, _i32, _i32, _i32, _pi32, _pi32, _pi32]
        lib.mla_split_plan.restype = ctypes.c_int
        # the reference's binding of its handmade entry point (handmade/mla_handmade.py:97-107)
        lib.mla_launch.argtypes = [_vp] * 7 + [ctypes.c_int]
        lib.mla_launch.restype = None
        lib.mla_kv_append.argtypes = [ctypes.POINTER(MlaKvAppendArgs), _vp]
        lib.mla_kv_append.restype = ctypes.c_int
        lib.mla_combine_absorb.argtypes = [ctypes.POINTER(MlaDecodeArgs), _vp, _vp, _vp]
        lib.mla_combine_absorb.restype = ctypes.c_int
        _lib = lib
        return lib


def check(fn: str, status: int) -> None:
    """Raise MlaError for a nonzero status returned by ``fn``."""
    if status != 0:
        msg = load().mla_last_error().decode(errors="replace")
        raise MlaError(fn, status, msg)
