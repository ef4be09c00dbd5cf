"""``flag_attn.flash`` -- ``attention`` is the forward of ``src/flag_attn/flash.py:269``
(same signature) through its split-KV decode path, implemented in
``flagattention_amd.gqa.flash_attention``."""
from flagattention_amd.gqa import flash_attention as attention  # noqa: F401

__all__ = ["attention"]
