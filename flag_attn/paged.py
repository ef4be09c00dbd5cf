"""``flag_attn.paged`` -- ``attention`` is the paged decode of ``src/flag_attn/paged.py:20``
(same signature), implemented in ``flagattention_amd.gqa.paged_attention``."""
from flagattention_amd.gqa import paged_attention as attention  # noqa: F401

__all__ = ["attention"]
