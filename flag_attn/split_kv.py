"""``flag_attn.split_kv`` -- ``attention`` is the flash decoding of
``src/flag_attn/split_kv.py:280`` (same signature), implemented in
``flagattention_amd.gqa.flash_attention_split_kv``."""
from flagattention_amd.gqa import flash_attention_split_kv as attention  # noqa: F401

__all__ = ["attention"]
