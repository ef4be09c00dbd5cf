"""flagattention_amd: MLA decode for AMD MI355X (gfx950).

Dense and sparse top-k decode over a paged latent KV cache (576-dim QK, 512-dim V, one
shared latent KV head), split-KV scheduling and an LSE-weighted combine, as hand-written
HIP kernels behind a C ABI (include/flagattention_amd.h).  This module is the Python
operator surface; there is no CPU fallback.
"""
from .mla import (  # noqa: F401
    DecodeWorkspace,
    MLAArgumentError,
    flash_mla_with_kvcache,
    get_mla_metadata,
    sparse_rows,
)

__all__ = ["get_mla_metadata", "flash_mla_with_kvcache", "sparse_rows", "DecodeWorkspace",
           "MLAArgumentError"]
__version__ = "0.1.0"
