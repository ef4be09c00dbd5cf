"""ctypes binding of libflagattention_amd.so (the C ABI in include/flagattention_amd.h).

The library is loaded on first use.  If it is missing or was built for another ABI
version, every call raises ``RuntimeError``: there is no fallback path.
"""
from __future__ import annotations

import ctypes
import os
import threading

ABI_VERSION = 3
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libflagattention_amd.so")

FA_OK = 0

_c_i32p = ctypes.POINTER(ctypes.c_int32)
_c_f32p = ctypes.POINTER(ctypes.c_float)


class DecodeArgs(ctypes.Structure):
    """Mirror of ``fa_mla_decode_args`` (field order and types must match the header)."""

    _fields_ = [
        ("q", ctypes.c_void_p),
        ("q_stride_b", ctypes.c_int64),
        ("q_stride_s", ctypes.c_int64),
        ("q_stride_h", ctypes.c_int64),
        ("kv", ctypes.c_void_p),
        ("kv_block_stride", ctypes.c_int64),
        ("kv_row_stride", ctypes.c_int64),
        ("num_kv_blocks", ctypes.c_int64),
        ("block_table", ctypes.c_void_p),
        ("bt_stride_b", ctypes.c_int64),
        ("max_blocks_per_seq", ctypes.c_int32),
        ("cache_seqlens", ctypes.c_void_p),
        ("indices", ctypes.c_void_p),
        ("idx_stride_b", ctypes.c_int64),
        ("idx_stride_s", ctypes.c_int64),
        ("topk", ctypes.c_int32),
        ("sparse_rows", ctypes.c_void_p),
        ("tile_md", ctypes.c_void_p),
        ("num_splits", ctypes.c_void_p),
        ("num_parts", ctypes.c_int32),
        ("out", ctypes.c_void_p),
        ("lse", ctypes.c_void_p),
        ("o_accum", ctypes.c_void_p),
        ("lse_accum", ctypes.c_void_p),
        ("batch", ctypes.c_int32),
        ("s_q", ctypes.c_int32),
        ("h_q", ctypes.c_int32),
        ("softmax_scale", ctypes.c_float),
        ("causal", ctypes.c_int32),
    ]


class GqaArgs(ctypes.Structure):
    """Mirror of ``fa_gqa_decode_args`` (field order and types must match the header)."""

    _fields_ = [
        ("q", ctypes.c_void_p),
        ("q_stride_b", ctypes.c_int64),
        ("q_stride_h", ctypes.c_int64),
        ("q_stride_m", ctypes.c_int64),
        ("k", ctypes.c_void_p),
        ("v", ctypes.c_void_p),
        ("k_stride_0", ctypes.c_int64),
        ("k_stride_h", ctypes.c_int64),
        ("k_stride_t", ctypes.c_int64),
        ("v_stride_0", ctypes.c_int64),
        ("v_stride_h", ctypes.c_int64),
        ("v_stride_t", ctypes.c_int64),
        ("block_table", ctypes.c_void_p),
        ("bt_stride_b", ctypes.c_int64),
        ("max_blocks_per_seq", ctypes.c_int32),
        ("block_size", ctypes.c_int32),
        ("num_blocks", ctypes.c_int64),
        ("seqlens", ctypes.c_void_p),
        ("n", ctypes.c_int32),
        ("out", ctypes.c_void_p),
        ("o_stride_b", ctypes.c_int64),
        ("o_stride_h", ctypes.c_int64),
        ("o_stride_m", ctypes.c_int64),
        ("lse", ctypes.c_void_p),
        ("o_part", ctypes.c_void_p),
        ("lse_part", ctypes.c_void_p),
        ("batch", ctypes.c_int32),
        ("h_q", ctypes.c_int32),
        ("h_kv", ctypes.c_int32),
        ("m", ctypes.c_int32),
        ("d", ctypes.c_int32),
        ("num_splits", ctypes.c_int32),
        ("split_tokens", ctypes.c_int32),
        ("scale", ctypes.c_float),
        ("causal", ctypes.c_int32),
        ("dtype", ctypes.c_int32),
    ]


# name -> (restype, argtypes) for every symbol declared in the header
SIGNATURES = {
    "fa_abi_version": (ctypes.c_int, []),
    "fa_last_error": (ctypes.c_char_p, []),
    "fa_device_cu_count": (ctypes.c_int, [ctypes.c_int, _c_i32p]),
    "fa_mla_decode_args_size": (ctypes.c_int64, []),
    "fa_mla_get_metadata": (
        ctypes.c_int,
        [ctypes.c_void_p, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,
         ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p],
    ),
    "fa_mla_decode_dense": (ctypes.c_int, [ctypes.POINTER(DecodeArgs), ctypes.c_void_p]),
    "fa_mla_sparse_rows": (ctypes.c_int, [ctypes.POINTER(DecodeArgs), ctypes.c_void_p]),
    "fa_mla_decode_sparse": (
        ctypes.c_int, [ctypes.POINTER(DecodeArgs), ctypes.c_int32, ctypes.c_void_p]),
    "fa_mla_combine": (ctypes.c_int, [ctypes.POINTER(DecodeArgs), ctypes.c_void_p]),
    "fa_mla_kvcache_write": (
        ctypes.c_int,
        [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p,
         ctypes.c_int32, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64,
         ctypes.c_int32, ctypes.c_void_p]),
    "fa_mla_topk_indices": (
        ctypes.c_int,
        [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int32,
         ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_void_p,
         ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p]),
    "fa_mla_topk_workspace_bytes": (
        ctypes.c_int64, [ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32]),
    "fa_gqa_decode_args_size": (ctypes.c_int64, []),
    "fa_gqa_decode": (ctypes.c_int, [ctypes.POINTER(GqaArgs), ctypes.c_void_p]),
    "fa_gqa_combine": (ctypes.c_int, [ctypes.POINTER(GqaArgs), ctypes.c_void_p]),
    "fa_mla_noalloc_scratch_bytes": (ctypes.c_int64, [ctypes.POINTER(DecodeArgs), ctypes.c_int32]),
    "fa_mla_decode_noalloc": (
        ctypes.c_int, [ctypes.POINTER(DecodeArgs), ctypes.c_int32, ctypes.c_void_p]),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def load() -> ctypes.CDLL:
    """Load (once) and type the shared library; raise RuntimeError if unusable."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"flagattention_amd: native library not found at {LIB_PATH}; "
                "build it with `python -m flagattention_amd.build`")
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        ver = lib.fa_abi_version()
        if ver != ABI_VERSION:
            raise RuntimeError(f"flagattention_amd: library ABI {ver} != binding ABI {ABI_VERSION}")
        size = lib.fa_mla_decode_args_size()
        if size != ctypes.sizeof(DecodeArgs):
            raise RuntimeError(
                f"flagattention_amd: fa_mla_decode_args is {size} bytes in the library, "
                f"{ctypes.sizeof(DecodeArgs)} in the binding")
        gsize = lib.fa_gqa_decode_args_size()
        if gsize != ctypes.sizeof(GqaArgs):
            raise RuntimeError(
                f"flagattention_amd: fa_gqa_decode_args is {gsize} bytes in the library, "
                f"{ctypes.sizeof(GqaArgs)} in the binding")
        _lib = lib
        return lib


def check(rc: int) -> None:
    """Map a non-zero C-ABI return code to RuntimeError(fa_last_error())."""
    if rc != FA_OK:
        msg = load().fa_last_error()
        raise RuntimeError(f"flagattention_amd error {rc}: {msg.decode() if msg else ''}")
