"""MLA decode operators: host side of the gfx950 HIP path.

Two calls make a decode step, in the shape of the public FlashMLA interface that the
operator surface of this package follows:

    tile_md, num_splits = get_mla_metadata(cache_seqlens, s_q * h_q // h_kv, h_kv)
    out, lse = flash_mla_with_kvcache(q, k_cache, block_table, cache_seqlens, 512,
                                      tile_md, num_splits, softmax_scale, causal,
                                      is_fp8_kvcache=..., indices=...)

Conventions kept from the reference decode operators (``src/flag_attn``):
  * outputs are allocated inside the call and returned, work is launched
    asynchronously on the current stream of the tensors' device, no host sync
    (``paged.py:30,69,177``; ``split_kv.py:331-344``);
  * the decode returns the pair ``(out, lse)`` with ``lse`` the fp32 natural-log
    normaliser, the return convention of ``flash.py:164-173``;
  * argument errors raise before any launch; the reference uses ``assert``
    (``paged.py:45-46``, ``split_kv.py:282-289``), so ``MLAArgumentError`` derives from
    both ``AssertionError`` and ``ValueError``.
  * the block table is addressed as in ``testing/paged.py:44-47``:
    token j lives in page ``block_table[b, j // 64]`` at row ``j % 64``.

All compute runs in libflagattention_amd.so; nothing here computes attention.
"""
from __future__ import annotations

import ctypes
import math
from typing import Optional, Tuple

import torch

from . import _lib
from .errors import ArgumentError

PAGE_SIZE = 64
D_QK = 576
D_V = 512
ROWS_PER_TILE = 128
MD_STRIDE = 8
FP8_ROW_BYTES = 656
MAX_BATCH = 4096
MAX_PARTS = 1024
# Scheduler cost, in 64-token blocks, charged once per sequence on the cost line
# (a sequence start inside a part adds a segment there: Q load, partial write-out and
# its share of the combine).
FIXED_OVERHEAD_BLOCKS = 4


def overhead_blocks(sparse: bool) -> int:
    """Per-sequence scheduler overhead for dense / sparse decode.

    Every part pays for its first segment whatever it holds, so the overhead only
    balances parts that hold a second one.  Sparse sequences all have ceil(topk / 64)
    blocks, and with the default part count (a multiple of the batch for the usual
    shapes) the cuts fall on sequence starts: charging the overhead there would shrink
    the first part of every sequence instead (18 vs 10 tiles per part at B = 64,
    topk = 2048, P = 256), so sparse decode charges none.
    """
    return 0 if sparse else FIXED_OVERHEAD_BLOCKS


class MLAArgumentError(ArgumentError):
    """Invalid argument to an MLA operator (raised before any kernel launch)."""


def _require(cond: bool, msg: str) -> None:
    if not cond:
        raise MLAArgumentError(msg)


_cu_counts: dict = {}


def device_cu_count(device: torch.device) -> int:
    """Compute units of a CUDA (HIP) device, cached per device index."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    if idx not in _cu_counts:
        _cu_counts[idx] = torch.cuda.get_device_properties(idx).multi_processor_count
    return _cu_counts[idx]


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def num_m_blocks(num_q_tokens_per_head_k: int, num_heads_q: Optional[int] = None,
                 sparse: bool = False) -> int:
    """Work-groups per KV head per part (query rows in tiles of 128).

    Dense decode tiles the flattened (token, head) rows; sparse decode gives every
    query token its own tiles (each token has its own key set), which needs
    ``num_heads_q`` to split the rows into tokens.
    """
    if sparse and num_heads_q:
        s_q = max(1, num_q_tokens_per_head_k // num_heads_q)
        return s_q * -(-num_heads_q // ROWS_PER_TILE)
    return -(-num_q_tokens_per_head_k // ROWS_PER_TILE)


def default_num_parts(cu_count: int, num_q_tokens_per_head_k: int, num_heads_k: int,
                      num_heads_q: Optional[int] = None, sparse: bool = False) -> int:
    """One work-group per CU: parts = CUs / (KV heads x row tiles)."""
    parts = cu_count // (num_heads_k * num_m_blocks(num_q_tokens_per_head_k, num_heads_q,
                                                    sparse))
    return max(1, min(MAX_PARTS, parts))


def get_mla_metadata(
    cache_seqlens: torch.Tensor,
    num_q_tokens_per_head_k: int,
    num_heads_k: int,
    num_heads_q: Optional[int] = None,
    is_fp8_kvcache: bool = False,
    topk: Optional[int] = None,
    num_sm_parts: Optional[int] = None,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Tile-scheduler metadata for one decode step.

    Returns ``(tile_scheduler_metadata int32[num_parts, 8], num_splits int32[B + 1])``.
    ``num_splits`` is the exclusive prefix sum of each sequence's segment count.
    For sparse decode pass ``topk`` (every sequence then has ``ceil(topk / 64)``
    blocks of index slots) together with ``num_heads_q``: sparse work-groups hold the
    heads of one query token, so the part count depends on the head count.
    ``num_sm_parts`` overrides the CU-derived part count.

    The returned tensors remember the batch and mode they were built for;
    ``flash_mla_with_kvcache`` rejects them in a call of another batch or mode (dense
    metadata drives a sparse decode into skipped segments, sparse metadata a dense one
    into attending only the first ``ceil(topk / 64)`` pages).
    """
    _require(isinstance(cache_seqlens, torch.Tensor), "cache_seqlens must be a tensor")
    _require(cache_seqlens.dtype == torch.int32, "cache_seqlens must be int32")
    _require(cache_seqlens.dim() == 1, "cache_seqlens must be 1-D [batch]")
    batch = cache_seqlens.shape[0]
    _require(1 <= batch <= MAX_BATCH, f"batch {batch} outside [1, {MAX_BATCH}]")
    _require(num_heads_k == 1, "MLA decode has exactly one latent KV head (num_heads_k == 1)")
    _require(num_q_tokens_per_head_k >= 1, "num_q_tokens_per_head_k must be >= 1")
    if num_heads_q is not None:
        _require(num_heads_q >= 1, "num_heads_q must be >= 1")
    _require(topk is None or topk >= 1, "topk must be >= 1")
    _require(topk is None or num_heads_q is not None,
             "sparse metadata (topk) needs num_heads_q: parts are sized per query token")
    _require(cache_seqlens.is_cuda, "cache_seqlens must be a CUDA (HIP) tensor")
    _require(cache_seqlens.is_contiguous(), "cache_seqlens must be contiguous")
    device = cache_seqlens.device
    if num_sm_parts is None:
        num_sm_parts = default_num_parts(device_cu_count(device), num_q_tokens_per_head_k,
                                         num_heads_k, num_heads_q, topk is not None)
    _require(1 <= num_sm_parts <= MAX_PARTS, f"num_sm_parts outside [1, {MAX_PARTS}]")
    tile_md = torch.empty((num_sm_parts, MD_STRIDE), dtype=torch.int32, device=device)
    num_splits = torch.empty((batch + 1,), dtype=torch.int32, device=device)
    lib = _lib.load()
    with torch.cuda.device(device):
        _lib.check(lib.fa_mla_get_metadata(
            _ptr(cache_seqlens), batch, int(topk or 0), num_sm_parts,
            overhead_blocks(topk is not None),
            _ptr(tile_md), _ptr(num_splits), _stream(device)))
    sig = (batch, int(topk or 0))
    tile_md._fa_mla_sig = sig
    num_splits._fa_mla_sig = sig
    return tile_md, num_splits


def _check_metadata_signature(tile_md, num_splits, batch, topk):
    """Metadata from get_mla_metadata carries (batch, topk); a decode of another batch or
    mode must not run on it.  Tensors built elsewhere carry no tag and are not checked."""
    want = (batch, int(topk or 0))
    for t in (tile_md, num_splits):
        sig = getattr(t, "_fa_mla_sig", None)
        _require(sig is None or sig == want,
                 f"scheduler metadata was built for (batch, topk) = {sig}, this call is {want}")


def _check_decode_args(q, k_cache, block_table, cache_seqlens, head_dim_v, tile_md,
                       num_splits, causal, is_fp8_kvcache, indices):
    _require(isinstance(q, torch.Tensor) and q.dim() == 4,
             "q must be a 4-D tensor [batch, s_q, h_q, 576]")
    batch, s_q, h_q, d = q.shape
    _require(q.dtype == torch.bfloat16, "q must be bfloat16")
    _require(d == D_QK, f"q head dim {d} != {D_QK}")
    _require(head_dim_v == D_V, f"head_dim_v {head_dim_v} != {D_V}")
    _require(1 <= batch <= MAX_BATCH, f"batch {batch} outside [1, {MAX_BATCH}]")
    _require(q.stride(3) == 1, "q last dim must be contiguous")
    _require(all(st % 8 == 0 for st in q.stride()[:3]) and q.data_ptr() % 16 == 0,
             "q rows must be 16-byte aligned")
    _require(isinstance(k_cache, torch.Tensor) and k_cache.dim() == 4,
             "k_cache must be [num_blocks, 64, 1, row]")
    nblk, page, hk, row = k_cache.shape
    _require(page == PAGE_SIZE, f"k_cache block size {page} != {PAGE_SIZE}")
    _require(hk == 1, "k_cache must have one latent KV head")
    if is_fp8_kvcache:
        _require(k_cache.dtype in (torch.uint8, torch.float8_e4m3fn),
                 "fp8 k_cache must be uint8 / float8_e4m3fn bytes")
        _require(row == FP8_ROW_BYTES, f"fp8 k_cache row {row} != {FP8_ROW_BYTES} bytes")
        _require(indices is not None, "the fp8 KV cache is supported by sparse decode (indices)")
    else:
        _require(k_cache.dtype == torch.bfloat16, "k_cache must be bfloat16")
        _require(row == D_QK, f"k_cache row {row} != {D_QK}")
    _require(k_cache.stride(3) == 1, "k_cache rows must be contiguous")
    esz = k_cache.element_size()
    _require((k_cache.stride(0) * esz) % 16 == 0 and (k_cache.stride(1) * esz) % 16 == 0
             and k_cache.data_ptr() % 16 == 0, "k_cache rows must be 16-byte aligned")
    _require(block_table.dtype == torch.int32 and block_table.dim() == 2,
             "block_table must be int32 [batch, max_blocks]")
    _require(block_table.shape[0] == batch, "block_table batch mismatch")
    _require(block_table.shape[1] >= 1, "block_table needs at least one column")
    _require(block_table.stride(1) == 1, "block_table rows must be contiguous")
    _require(cache_seqlens.dtype == torch.int32 and cache_seqlens.shape == (batch,)
             and cache_seqlens.is_contiguous(), "cache_seqlens must be contiguous int32 [batch]")
    _require(tile_md.dtype == torch.int32 and tile_md.dim() == 2
             and tile_md.shape[1] == MD_STRIDE and tile_md.is_contiguous(),
             "tile_scheduler_metadata must be contiguous int32 [num_parts, 8]")
    _require(1 <= tile_md.shape[0] <= MAX_PARTS, "tile_scheduler_metadata has too many parts")
    _require(num_splits.dtype == torch.int32 and num_splits.shape == (batch + 1,)
             and num_splits.is_contiguous(), "num_splits must be contiguous int32 [batch + 1]")
    if indices is not None:
        _require(indices.dtype == torch.int32 and indices.dim() == 3
                 and indices.shape[:2] == (batch, s_q), "indices must be int32 [batch, s_q, topk]")
        _require(indices.shape[2] >= 1 and indices.stride(2) == 1,
                 "indices last dim must be contiguous and non-empty")
        _require(not causal, "causal masking does not apply to sparse (indices) decode")
    _check_metadata_signature(tile_md, num_splits, batch,
                              None if indices is None else indices.shape[2])
    tensors = [q, k_cache, block_table, cache_seqlens, tile_md, num_splits]
    if indices is not None:
        tensors.append(indices)
    _require(all(t.is_cuda for t in tensors), "all tensors must be CUDA (HIP) tensors")
    _require(all(t.device == q.device for t in tensors), "all tensors must be on one device")
    return batch, s_q, h_q


def _decode_args(q, k_cache, block_table, cache_seqlens, tile_md, num_splits, out, lse,
                 softmax_scale, causal, o_accum=None, lse_accum=None) -> "_lib.DecodeArgs":
    """The C-ABI argument block of one decode call (indices are added by _set_indices)."""
    batch, s_q, h_q, _ = q.shape
    esz = k_cache.element_size()
    return _lib.DecodeArgs(
        q=q.data_ptr(), q_stride_b=q.stride(0), q_stride_s=q.stride(1),
        q_stride_h=q.stride(2), kv=k_cache.data_ptr(),
        kv_block_stride=k_cache.stride(0) * esz, kv_row_stride=k_cache.stride(1) * esz,
        num_kv_blocks=k_cache.shape[0], block_table=block_table.data_ptr(),
        bt_stride_b=block_table.stride(0), max_blocks_per_seq=block_table.shape[1],
        cache_seqlens=cache_seqlens.data_ptr(), indices=None, idx_stride_b=0,
        idx_stride_s=0, topk=0, sparse_rows=None,
        tile_md=tile_md.data_ptr(), num_splits=num_splits.data_ptr(),
        num_parts=tile_md.shape[0], out=out.data_ptr(), lse=lse.data_ptr(),
        o_accum=None if o_accum is None else o_accum.data_ptr(),
        lse_accum=None if lse_accum is None else lse_accum.data_ptr(),
        batch=batch, s_q=s_q, h_q=h_q, softmax_scale=float(softmax_scale),
        causal=int(bool(causal)))


def _set_indices(args, indices) -> None:
    args.indices = indices.data_ptr()
    args.idx_stride_b = indices.stride(0)
    args.idx_stride_s = indices.stride(1)
    args.topk = indices.shape[2]


class DecodeWorkspace:
    """Outputs and split workspace for decode steps of one shape, allocated once.

    ``flash_mla_with_kvcache`` builds a transient one per call; a serving loop (or a
    benchmark) can keep one and call :meth:`run` every step, so no allocation happens
    per step.  Buffers: ``out`` bf16 [B, s_q, h_q, 512], ``lse`` fp32 [B, h_q, s_q],
    ``o_accum`` bf16 [B + parts, s_q * h_q, 512], ``lse_accum`` fp32 [B + parts, s_q * h_q]
    and, for sparse decode, the gather rows int32 [B, s_q, ceil(topk / 64) * 64].
    """

    def __init__(self, batch: int, s_q: int, h_q: int, num_parts: int,
                 device: torch.device, topk: Optional[int] = None):
        _require(batch >= 1 and s_q >= 1 and h_q >= 1 and num_parts >= 1, "bad workspace shape")
        self.batch, self.s_q, self.h_q, self.num_parts, self.topk = batch, s_q, h_q, num_parts, topk
        rows = s_q * h_q
        self.out = torch.empty((batch, s_q, h_q, D_V), dtype=torch.bfloat16, device=device)
        self.lse = torch.empty((batch, h_q, s_q), dtype=torch.float32, device=device)
        self.o_accum = torch.empty((batch + num_parts, rows, D_V), dtype=torch.bfloat16,
                                   device=device)
        self.lse_accum = torch.empty((batch + num_parts, rows), dtype=torch.float32,
                                     device=device)
        self.rows = None
        if topk is not None:
            topk_pad = -(-topk // PAGE_SIZE) * PAGE_SIZE
            self.rows = torch.empty((batch, s_q, topk_pad), dtype=torch.int32, device=device)

    def run(self, q, k_cache, block_table, cache_seqlens, tile_scheduler_metadata, num_splits,
            softmax_scale: Optional[float] = None, causal: bool = False,
            is_fp8_kvcache: bool = False, indices: Optional[torch.Tensor] = None,
            decode_events=None) -> Tuple[torch.Tensor, torch.Tensor]:
        """One decode step into this workspace; returns its ``(out, lse)`` tensors.

        ``decode_events``: optional ``(start, end)`` CUDA events recorded on the launch
        stream immediately around the decode kernel (used to time that kernel alone).
        """
        batch, s_q, h_q = _check_decode_args(q, k_cache, block_table, cache_seqlens, D_V,
                                             tile_scheduler_metadata, num_splits, causal,
                                             is_fp8_kvcache, indices)
        _require((batch, s_q, h_q) == (self.batch, self.s_q, self.h_q),
                 "workspace shape does not match q")
        _require(tile_scheduler_metadata.shape[0] <= self.num_parts,
                 "workspace has fewer parts than the scheduler metadata")
        _require(self.out.device == q.device, "workspace is on another device")
        if indices is not None:
            _require(self.topk is not None and indices.shape[2] == self.topk,
                     "workspace topk does not match indices")
        if softmax_scale is None:
            softmax_scale = 1.0 / math.sqrt(D_QK)
        _require(math.isfinite(softmax_scale), "softmax_scale must be finite")
        device = q.device
        args = _decode_args(q, k_cache, block_table, cache_seqlens, tile_scheduler_metadata,
                            num_splits, self.out, self.lse, softmax_scale, causal,
                            self.o_accum, self.lse_accum)
        lib = _lib.load()
        with torch.cuda.device(device):
            stream = _stream(device)
            if indices is not None:
                _set_indices(args, indices)
                args.sparse_rows = self.rows.data_ptr()
                _lib.check(lib.fa_mla_sparse_rows(ctypes.byref(args), stream))
            if decode_events is not None:
                decode_events[0].record()
            if indices is None:
                _lib.check(lib.fa_mla_decode_dense(ctypes.byref(args), stream))
            else:
                _lib.check(lib.fa_mla_decode_sparse(ctypes.byref(args), int(is_fp8_kvcache),
                                                    stream))
            if decode_events is not None:
                decode_events[1].record()
            _lib.check(lib.fa_mla_combine(ctypes.byref(args), stream))
        return self.out, self.lse


def flash_mla_with_kvcache(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    block_table: torch.Tensor,
    cache_seqlens: torch.Tensor,
    head_dim_v: int,
    tile_scheduler_metadata: torch.Tensor,
    num_splits: torch.Tensor,
    softmax_scale: Optional[float] = None,
    causal: bool = False,
    is_fp8_kvcache: bool = False,
    indices: Optional[torch.Tensor] = None,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """MLA decode over a paged latent KV cache (dense, or sparse top-k with ``indices``).

    q               bf16 [B, s_q, h_q, 576]
    k_cache         bf16 [num_blocks, 64, 1, 576], or fp8 rows uint8 [num_blocks, 64, 1, 656]
                    (512 e4m3 codes | 4 fp32 scales, one per 128 dims | 64 bf16 rope dims)
    block_table     int32 [B, max_blocks]: page of token j is block_table[b, j // 64]
    cache_seqlens   int32 [B]
    indices         int32 [B, s_q, topk] logical token ids; entries < 0 or >= cache_seqlens[b]
                    are masked (sparse decode)
    causal          bottom-right aligned over the last s_q positions (dense only)

    Returns ``out`` bf16 [B, s_q, h_q, 512] and ``lse`` fp32 [B, h_q, s_q]; rows with no
    visible key get out = 0, lse = -inf.
    """
    batch, s_q, h_q = _check_decode_args(q, k_cache, block_table, cache_seqlens, head_dim_v,
                                         tile_scheduler_metadata, num_splits, causal,
                                         is_fp8_kvcache, indices)
    ws = DecodeWorkspace(batch, s_q, h_q, tile_scheduler_metadata.shape[0], q.device,
                         topk=None if indices is None else indices.shape[2])
    return ws.run(q, k_cache, block_table, cache_seqlens, tile_scheduler_metadata, num_splits,
                  softmax_scale, causal, is_fp8_kvcache, indices)


def sparse_rows(
    indices: torch.Tensor,
    block_table: torch.Tensor,
    cache_seqlens: torch.Tensor,
    num_kv_blocks: int,
) -> torch.Tensor:
    """Physical cache row of every sparse index slot (the gather addresses).

    rows[b, s, j] = block_table[b, i // 64] * 64 + i % 64 for i = indices[b, s, j] in
    [0, cache_seqlens[b]), else -1; j runs over topk rounded up to 64 (pad slots are -1).
    A page id outside [0, num_kv_blocks) also yields -1.
    """
    _require(num_kv_blocks >= 1, "num_kv_blocks must be >= 1")
    _require(indices.dtype == torch.int32 and indices.dim() == 3, "indices must be int32 3-D")
    batch, s_q, topk = indices.shape
    _require(indices.stride(2) == 1, "indices last dim must be contiguous")
    _require(block_table.dtype == torch.int32 and block_table.dim() == 2
             and block_table.shape[0] == batch and block_table.stride(1) == 1,
             "block_table must be int32 [batch, max_blocks]")
    _require(cache_seqlens.dtype == torch.int32 and cache_seqlens.shape == (batch,)
             and cache_seqlens.is_contiguous(), "cache_seqlens must be contiguous int32 [batch]")
    _require(all(t.is_cuda for t in (indices, block_table, cache_seqlens)),
             "all tensors must be CUDA (HIP) tensors")
    device = indices.device
    topk_pad = -(-topk // PAGE_SIZE) * PAGE_SIZE
    rows = torch.empty((batch, s_q, topk_pad), dtype=torch.int32, device=device)
    args = _lib.DecodeArgs(
        block_table=block_table.data_ptr(), bt_stride_b=block_table.stride(0),
        max_blocks_per_seq=block_table.shape[1], cache_seqlens=cache_seqlens.data_ptr(),
        indices=indices.data_ptr(), idx_stride_b=indices.stride(0),
        idx_stride_s=indices.stride(1), topk=topk, sparse_rows=rows.data_ptr(),
        num_kv_blocks=num_kv_blocks, batch=batch, s_q=s_q, h_q=1, num_parts=1)
    lib = _lib.load()
    with torch.cuda.device(device):
        _lib.check(lib.fa_mla_sparse_rows(ctypes.byref(args), _stream(device)))
    return rows


def decode_noalloc(
    out: torch.Tensor,
    lse: torch.Tensor,
    q: torch.Tensor,
    k_cache: torch.Tensor,
    block_table: torch.Tensor,
    cache_seqlens: torch.Tensor,
    tile_scheduler_metadata: torch.Tensor,
    num_splits: torch.Tensor,
    softmax_scale: Optional[float] = None,
    causal: bool = False,
    is_fp8_kvcache: bool = False,
    indices: Optional[torch.Tensor] = None,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """``flash_mla_with_kvcache`` into caller-owned ``out`` / ``lse`` through the C ABI's
    allocation-free entry point (``fa_mla_decode_noalloc``): the split partials and gather
    rows live in the library's own device array, so the step allocates no device memory.
    For callers that cannot allocate (graph capture, serving loops).  Calls that overlap on
    one device share that array and race; a shape whose workspace exceeds
    ``FA_MLA_NOALLOC_SCRATCH_BYTES`` (64 MiB) raises ``RuntimeError``."""
    batch, s_q, h_q = _check_decode_args(q, k_cache, block_table, cache_seqlens, D_V,
                                         tile_scheduler_metadata, num_splits, causal,
                                         is_fp8_kvcache, indices)
    _require(out.dtype == torch.bfloat16 and out.shape == (batch, s_q, h_q, D_V)
             and out.is_contiguous() and out.device == q.device,
             "out must be contiguous bf16 [batch, s_q, h_q, 512] on q's device")
    _require(lse.dtype == torch.float32 and lse.shape == (batch, h_q, s_q)
             and lse.is_contiguous() and lse.device == q.device,
             "lse must be contiguous fp32 [batch, h_q, s_q] on q's device")
    if softmax_scale is None:
        softmax_scale = 1.0 / math.sqrt(D_QK)
    _require(math.isfinite(softmax_scale), "softmax_scale must be finite")
    args = _decode_args(q, k_cache, block_table, cache_seqlens, tile_scheduler_metadata,
                        num_splits, out, lse, softmax_scale, causal)
    mode = 0
    if indices is not None:
        _set_indices(args, indices)
        mode = 2 if is_fp8_kvcache else 1
    lib = _lib.load()
    with torch.cuda.device(q.device):
        _lib.check(lib.fa_mla_decode_noalloc(ctypes.byref(args), mode, _stream(q.device)))
    return out, lse


def concat_and_cache_mla(
    kv_c: torch.Tensor,
    k_pe: torch.Tensor,
    kv_cache: torch.Tensor,
    slot_mapping: torch.Tensor,
    is_fp8_kvcache: bool = False,
) -> None:
    """Write new tokens into the paged latent cache (in place).

    kv_c          bf16 [T, 512] latent vectors, k_pe bf16 [T, 64] rope vectors
    kv_cache      bf16 [num_blocks, 64, 1, 576], or fp8 rows uint8 [num_blocks, 64, 1, 656]
    slot_mapping  int32 / int64 [T]: physical row page * 64 + row of each token; negative
                  slots (padding tokens) and slots past the cache are skipped

    fp8 rows get one scale per 128 latent dims, ``amax / 448``, and e4m3 codes of
    ``x / scale`` rounded to nearest even -- the layout ``flash_mla_with_kvcache(...,
    is_fp8_kvcache=True)`` reads.  Runs on the current stream; no host synchronisation.
    """
    _require(kv_c.dim() == 2 and kv_c.shape[1] == D_V and kv_c.dtype == torch.bfloat16,
             "kv_c must be bf16 [num_tokens, 512]")
    t = kv_c.shape[0]
    _require(k_pe.dim() == 2 and k_pe.shape == (t, D_QK - D_V) and k_pe.dtype == torch.bfloat16,
             "k_pe must be bf16 [num_tokens, 64]")
    _require(kv_c.stride(1) == 1 and k_pe.stride(1) == 1, "kv_c / k_pe rows must be contiguous")
    _require(kv_c.data_ptr() % 16 == 0 and k_pe.data_ptr() % 16 == 0
             and kv_c.stride(0) % 8 == 0 and k_pe.stride(0) % 8 == 0,
             "kv_c / k_pe rows must be 16-byte aligned")
    _require(kv_cache.dim() == 4 and kv_cache.shape[1] == PAGE_SIZE and kv_cache.shape[2] == 1,
             "kv_cache must be [num_blocks, 64, 1, row]")
    if is_fp8_kvcache:
        _require(kv_cache.dtype in (torch.uint8, torch.float8_e4m3fn)
                 and kv_cache.shape[3] == FP8_ROW_BYTES, "fp8 kv_cache must be uint8 [.., 656]")
    else:
        _require(kv_cache.dtype == torch.bfloat16 and kv_cache.shape[3] == D_QK,
                 "kv_cache must be bf16 [.., 576]")
    esz = kv_cache.element_size()
    _require(kv_cache.stride(3) == 1 and kv_cache.data_ptr() % 16 == 0
             and (kv_cache.stride(0) * esz) % 16 == 0 and (kv_cache.stride(1) * esz) % 16 == 0,
             "kv_cache rows must be contiguous and 16-byte aligned")
    _require(slot_mapping.dim() == 1 and slot_mapping.shape[0] == t
             and slot_mapping.dtype in (torch.int32, torch.int64),
             "slot_mapping must be int32 / int64 [num_tokens]")
    tensors = (kv_c, k_pe, kv_cache, slot_mapping)
    _require(all(x.is_cuda and x.device == kv_c.device for x in tensors),
             "all tensors must be CUDA (HIP) tensors on one device")
    if t == 0:
        return
    slots = slot_mapping.to(torch.int64).contiguous()
    lib = _lib.load()
    with torch.cuda.device(kv_c.device):
        _lib.check(lib.fa_mla_kvcache_write(
            kv_c.data_ptr(), kv_c.stride(0), k_pe.data_ptr(), k_pe.stride(0), slots.data_ptr(),
            t, kv_cache.data_ptr(), kv_cache.stride(0) * esz, kv_cache.stride(1) * esz,
            kv_cache.shape[0], int(bool(is_fp8_kvcache)), _stream(kv_c.device)))


TOPK_MAX_LEN = 65536
TOPK_MAX_K = 65536


def topk_indices(
    scores: torch.Tensor,
    cache_seqlens: torch.Tensor,
    topk: int,
    causal: bool = False,
    out: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Sparse-attention indices from per-key indexer scores.

    scores         fp32 [B, s_q, L]: score of key position l for query token t of
                   sequence b (last dim contiguous); L <= 65536
    cache_seqlens  int32 [B]
    topk           1..65536
    causal         query token t sees keys [0, cache_seqlens[b] - (s_q - 1 - t)) (bottom-
                   right aligned, as the dense decode's causal mask); else [0, cache_seqlens[b])
    out            optional int32 [B, s_q, topk] contiguous to write into

    Returns int32 [B, s_q, topk]: the positions of the min(topk, n) largest visible
    scores in ascending order, then -1 -- the ``indices`` argument of
    ``flash_mla_with_kvcache``.  Scores compare by the total order of their bit patterns
    (-NaN < -inf < -0 < +0 < +inf < +NaN), ties by lower position, so the result is
    deterministic.  Runs on the current stream; no host synchronisation.
    """
    _require(isinstance(scores, torch.Tensor) and scores.dim() == 3
             and scores.dtype == torch.float32, "scores must be float32 [batch, s_q, len]")
    batch, s_q, length = scores.shape
    _require(length <= TOPK_MAX_LEN, f"scores length {length} > {TOPK_MAX_LEN}")
    _require(isinstance(topk, int) and 1 <= topk <= TOPK_MAX_K,
             f"topk must be an int in [1, {TOPK_MAX_K}]")
    _require(scores.stride(2) == 1 or length <= 1, "scores last dim must be contiguous")
    _require(isinstance(cache_seqlens, torch.Tensor) and cache_seqlens.dtype == torch.int32
             and cache_seqlens.shape == (batch,), "cache_seqlens must be int32 [batch]")
    tensors = [scores, cache_seqlens]
    if out is None:
        out = torch.empty((batch, s_q, topk), dtype=torch.int32, device=scores.device)
    else:
        _require(out.dtype == torch.int32 and out.shape == (batch, s_q, topk)
                 and out.is_contiguous(), "out must be contiguous int32 [batch, s_q, topk]")
        tensors.append(out)
    _require(all(x.is_cuda and x.device == scores.device for x in tensors),
             "all tensors must be CUDA (HIP) tensors on one device")
    if batch == 0:
        return out
    seqlens = cache_seqlens.contiguous()
    lib = _lib.load()
    ws_bytes = int(lib.fa_mla_topk_workspace_bytes(batch, s_q, length, topk))
    _require(ws_bytes >= 0, "invalid top-k shape")
    ws = (torch.empty(ws_bytes, dtype=torch.uint8, device=scores.device) if ws_bytes > 0
          else None)
    with torch.cuda.device(scores.device):
        _lib.check(lib.fa_mla_topk_indices(
            scores.data_ptr(), scores.stride(0), scores.stride(1), seqlens.data_ptr(), batch, s_q,
            length, topk, int(bool(causal)), out.data_ptr(), _ptr(ws), ws_bytes,
            _stream(scores.device)))
    return out
