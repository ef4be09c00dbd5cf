"""MLA decode operators of the ``flag_attn`` namespace.

``get_mla_metadata(cache_seqlens, num_q_tokens_per_head_k, num_heads_k, num_heads_q=None,
is_fp8_kvcache=False, topk=None)`` returns ``(tile_scheduler_metadata, num_splits)``;
``flash_mla_with_kvcache(q, k_cache, block_table, cache_seqlens, head_dim_v,
tile_scheduler_metadata, num_splits, softmax_scale=None, causal=False,
is_fp8_kvcache=False, indices=None)`` returns ``(out, lse)``;
``concat_and_cache_mla(kv_c, k_pe, kv_cache, slot_mapping, is_fp8_kvcache=False)`` writes
new tokens into the paged cache (bf16 rows, or quantised fp8 rows);
``topk_indices(scores, cache_seqlens, topk, causal=False)`` turns per-key indexer scores
into the ``indices`` of sparse decode.  All are implemented in
``flagattention_amd.mla`` (validation, allocation, launch through the C ABI).
"""
from flagattention_amd.mla import (  # noqa: F401
    DecodeWorkspace,
    concat_and_cache_mla,
    MLAArgumentError,
    flash_mla_with_kvcache,
    get_mla_metadata,
    sparse_rows,
    topk_indices,
)

__all__ = ["get_mla_metadata", "flash_mla_with_kvcache", "concat_and_cache_mla", "topk_indices",
           "sparse_rows", "DecodeWorkspace", "MLAArgumentError"]
