"""flag_attn -- the FlagAttention operator namespace, backed by the MI355X (gfx950) HIP library.

Code written against the reference's ``flag_attn`` package imports its decode operators
from here.  The reference exports its operators from ``src/flag_attn/__init__.py:23-29``
in the same style (``from flag_attn.<module> import attention as <name>``); this package
exports the decode operators built for MI355X:

* ``get_mla_metadata`` / ``flash_mla_with_kvcache`` -- MLA decode (dense and sparse top-k
  over the paged latent KV cache, split-KV scheduling, LSE combine);
* ``concat_and_cache_mla`` -- the cache write path of those layouts (bf16 and fp8 rows);
* ``topk_indices`` -- the index producer of sparse decode (top-k positions per query token
  from per-key indexer scores);
* ``paged_attention`` -- MHA / GQA decode over a paged KV cache (``paged.py:20-177``);
* ``flash_attention_split_kv`` -- flash decoding over contiguous K/V (``split_kv.py:280-344``);
* ``flash_attention`` -- the forward of ``flash.py:269-300`` through its split-KV decode
  path (no dropout, no total attention, no backward).

Every operator runs in ``flagattention_amd/libflagattention_amd.so`` (hand-written HIP for
gfx950); there is no Triton and no CPU fallback.  The reference's training-path operators
(backward passes, ``piecewise_attention``, ``chunk_gated_delta_rule``) and its PyTorch
``testing`` oracles are not part of this package.
"""
from flag_attn.mla import (  # noqa: F401
    concat_and_cache_mla,
    flash_mla_with_kvcache,
    get_mla_metadata,
    topk_indices,
)
from flag_attn.paged import attention as paged_attention  # noqa: F401
from flag_attn.split_kv import attention as flash_attention_split_kv  # noqa: F401
from flag_attn.flash import attention as flash_attention  # noqa: F401

__all__ = ["get_mla_metadata", "flash_mla_with_kvcache", "concat_and_cache_mla", "topk_indices",
           "paged_attention",
           "flash_attention_split_kv", "flash_attention"]
__version__ = "0.2.0"
