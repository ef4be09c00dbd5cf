"""flagattention_amd: attention decode for AMD MI355X (gfx950).

MLA decode -- dense and sparse top-k over a paged latent KV cache (576-dim QK, 512-dim V,
one shared latent KV head), split-KV scheduling and an LSE-weighted combine -- and
grouped-query decode over paged or contiguous caches, as hand-written HIP kernels behind
a C ABI (include/flagattention_amd.h).  This module is the Python operator surface; there
is no CPU fallback.
"""
from .errors import ArgumentError  # noqa: F401
from .gqa import flash_attention, flash_attention_split_kv, paged_attention  # noqa: F401
from .mla import (  # noqa: F401
    DecodeWorkspace,
    MLAArgumentError,
    flash_mla_with_kvcache,
    concat_and_cache_mla,
    get_mla_metadata,
    sparse_rows,
    topk_indices,
)

__all__ = ["get_mla_metadata", "flash_mla_with_kvcache", "concat_and_cache_mla", "topk_indices",
           "sparse_rows", "DecodeWorkspace",
           "MLAArgumentError", "ArgumentError", "paged_attention", "flash_attention_split_kv",
           "flash_attention"]
__version__ = "0.1.0"
