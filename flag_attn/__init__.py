"""flag_attn -- the FlagAttention operator namespace, backed by the MI355X (gfx950) HIP library.

Code written against the reference's ``flag_attn`` package imports its decode operators
from here.  The reference exports its operators from ``src/flag_attn/__init__.py:23-29``
in the same style (``from flag_attn.<module> import attention as <name>``); this package
exports the decode operators built for MI355X:

* ``get_mla_metadata`` / ``flash_mla_with_kvcache`` -- MLA decode (dense and sparse top-k
  over the paged latent KV cache, split-KV scheduling, LSE combine);

Every operator runs in ``flagattention_amd/libflagattention_amd.so`` (hand-written HIP for
gfx950); there is no Triton and no CPU fallback.  The reference's training-path operators
(prefill ``flash_attention`` backward, ``piecewise_attention``, ``chunk_gated_delta_rule``)
and its PyTorch ``testing`` oracles are not part of this package.
"""
from flag_attn.mla import flash_mla_with_kvcache, get_mla_metadata  # noqa: F401

__all__ = ["get_mla_metadata", "flash_mla_with_kvcache"]
__version__ = "0.2.0"
