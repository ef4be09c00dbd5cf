"""Grouped-query decode operators (MHA / GQA / MQA): host side of the gfx950 HIP path.

These keep the reference's operator signatures and conventions (``src/flag_attn``):

* ``paged_attention(query, key_cache, value_cache, context_lens, block_tables, attn_scale,
  max_context_len, num_splits=0)`` -- ``paged.py:20-177``: query ``[num_seqs, H, D]``,
  caches ``[num_blocks, H_kv, block_size, D]``, out ``[num_seqs, H, D]`` like the query;
  ``num_splits`` 0 picks the split count, 1 disables splitting, ``s > 1`` uses partitions
  of ``next_pow2(cdiv(max_context_len, s))`` tokens (``paged.py:64-67``);
* ``flash_attention_split_kv(q, k, v, causal=False, sm_scale=None)`` -- ``split_kv.py:280-344``:
  ``q [B, H, M, D]``, ``k, v [B, H_kv, N, D]`` (any strides with a contiguous last dim),
  returns ``o`` like ``q``;
* ``flash_attention(q, k, v, causal=False, sm_scale=None, dropout_p=0.0,
  return_log_normalizer=False, return_total_attention=False, return_seed_offset=False)``
  -- the forward of ``flash.py:269-300`` through its split-KV decode branch
  (``flash.py:73-139,164-173``): returns ``o``, or ``(o, L, None, None, None)`` when an
  extra return is asked for, ``L`` the fp32 natural-log normaliser ``[B, H, M]``.

Causal masking is bottom-right aligned (query position ``i`` of ``M`` sees keys
``<= N - M + i``, ``testing/flash.py:47-55``).  Outputs are allocated inside the call and
work is queued on the current stream; argument errors raise ``ArgumentError`` (both a
``ValueError`` and, like the reference's ``assert`` checks, an ``AssertionError``) before
any launch.  Everything computes in ``libflagattention_amd.so``; there is no fallback.
"""
from __future__ import annotations

import ctypes
import math
from typing import Optional

import torch

from . import _lib
from .errors import ArgumentError

HEAD_DIMS = (16, 32, 64, 128, 256, 512)
ROWS_PER_WG = 16
MIN_SPLIT_TOKENS = 256

# Benchmark hook: a (start, end) pair of CUDA events recorded on the launch stream right
# around the next decode kernel launch (not the combine); cleared after that launch.
timing_events = None


def _require(cond: bool, msg: str) -> None:
    if not cond:
        raise ArgumentError(msg)


def _dtype_code(dt: torch.dtype) -> int:
    _require(dt in (torch.float16, torch.bfloat16), f"dtype {dt} is not float16 / bfloat16")
    return 0 if dt == torch.float16 else 1


def _next_pow2(x: int) -> int:
    return 1 if x <= 1 else 1 << (x - 1).bit_length()


_cu_counts: dict = {}


def _cu_count(device: torch.device) -> int:
    idx = device.index if device.index is not None else torch.cuda.current_device()
    if idx not in _cu_counts:
        _cu_counts[idx] = torch.cuda.get_device_properties(idx).multi_processor_count
    return _cu_counts[idx]


def choose_splits(batch: int, h_kv: int, rows_per_kv_head: int, max_len: int,
                  cu_count: int) -> int:
    """Split-KV count: none when batch x KV heads x row blocks already gives every CU a
    work-group, else enough splits for about two work-groups per CU, each at least
    MIN_SPLIT_TOKENS keys long."""
    base = batch * h_kv * -(-rows_per_kv_head // ROWS_PER_WG)
    if base >= cu_count or max_len <= MIN_SPLIT_TOKENS:
        return 1
    return max(1, min(-(-2 * cu_count // base), -(-max_len // MIN_SPLIT_TOKENS)))


def _launch(args: "_lib.GqaArgs", device: torch.device, o_dtype: torch.dtype, rows: int,
            head_dim: int, num_splits: int) -> None:
    global timing_events
    lib = _lib.load()
    events, timing_events = timing_events, None
    with torch.cuda.device(device):
        stream = torch.cuda.current_stream(device).cuda_stream
        if num_splits > 1:
            o_part = torch.empty((rows, num_splits, head_dim), dtype=torch.float32, device=device)
            lse_part = torch.empty((rows, num_splits), dtype=torch.float32, device=device)
            args.o_part = o_part.data_ptr()
            args.lse_part = lse_part.data_ptr()
        if events is not None:
            events[0].record()
        _lib.check(lib.fa_gqa_decode(ctypes.byref(args), stream))
        if events is not None:
            events[1].record()
        if num_splits > 1:
            _lib.check(lib.fa_gqa_combine(ctypes.byref(args), stream))


def _aligned(t: torch.Tensor, dims) -> bool:
    return t.data_ptr() % 16 == 0 and all(t.stride(d) % 8 == 0 for d in dims)


def paged_attention(
    query: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    context_lens: torch.Tensor,
    block_tables: torch.Tensor,
    attn_scale: float,
    max_context_len: int,
    num_splits: int = 0,
) -> torch.Tensor:
    """Decode attention of one query token per sequence over a paged KV cache.

    Token ``j`` of sequence ``s`` is row ``j % block_size`` of page
    ``block_tables[s, j // block_size]`` (``testing/paged.py:44-47``); a page id outside the
    cache reads as a masked key.  Returns ``out`` shaped and typed like ``query``.
    """
    _require(query.dim() == 3, "query must be [num_seqs, num_heads, head_size]")
    _require(key_cache.dim() == 4 and value_cache.shape == key_cache.shape,
             "key_cache / value_cache must be [num_blocks, num_kv_heads, block_size, head_size]")
    num_seqs, h_q, d = query.shape
    num_blocks, h_kv, block_size, d_k = key_cache.shape
    _require(d == d_k, f"query head_size {d} != cache head_size {d_k}")
    _require(d in HEAD_DIMS, f"head_size={d} not in {HEAD_DIMS}")
    _require(h_kv >= 1 and h_q % h_kv == 0, "num_heads must be a multiple of num_kv_heads")
    code = _dtype_code(query.dtype)
    _require(key_cache.dtype == query.dtype and value_cache.dtype == query.dtype,
             "query / key_cache / value_cache dtypes differ")
    _require(value_cache.stride() == key_cache.stride(),
             "value_cache must have the same strides as key_cache")
    _require(query.stride(2) == 1 and key_cache.stride(3) == 1, "head dims must be contiguous")
    _require(_aligned(query, (0, 1)) and _aligned(key_cache, (0, 1, 2))
             and _aligned(value_cache, (0, 1, 2)), "rows must be 16-byte aligned")
    _require(context_lens.dtype == torch.int32 and context_lens.shape == (num_seqs,)
             and context_lens.is_contiguous(), "context_lens must be contiguous int32 [num_seqs]")
    _require(block_tables.dtype == torch.int32 and block_tables.dim() == 2
             and block_tables.shape[0] == num_seqs and block_tables.stride(1) == 1,
             "block_tables must be int32 [num_seqs, max_num_blocks_per_seq]")
    _require(num_splits >= 0, "num_splits must be >= 0")
    _require(max_context_len >= 1, "max_context_len must be >= 1")
    tensors = (query, key_cache, value_cache, context_lens, block_tables)
    _require(all(t.is_cuda and t.device == query.device for t in tensors),
             "all tensors must be CUDA (HIP) tensors on one device")
    device = query.device
    out = torch.empty_like(query)
    if num_splits == 0:
        s = choose_splits(num_seqs, h_kv, h_q // h_kv, max_context_len, _cu_count(device))
        split_tokens = -(-max_context_len // s)
    elif num_splits == 1:
        split_tokens = max_context_len
    else:
        split_tokens = _next_pow2(-(-max_context_len // num_splits))
    s = -(-max_context_len // split_tokens)
    if s == 1:
        split_tokens = 1 << 30  # one split sees every key of its sequence
    args = _lib.GqaArgs(
        q=query.data_ptr(), q_stride_b=query.stride(0), q_stride_h=query.stride(1), q_stride_m=0,
        k=key_cache.data_ptr(), v=value_cache.data_ptr(),
        k_stride_0=key_cache.stride(0), k_stride_h=key_cache.stride(1),
        k_stride_t=key_cache.stride(2), v_stride_0=value_cache.stride(0),
        v_stride_h=value_cache.stride(1), v_stride_t=value_cache.stride(2),
        block_table=block_tables.data_ptr(), bt_stride_b=block_tables.stride(0),
        max_blocks_per_seq=block_tables.shape[1], block_size=block_size, num_blocks=num_blocks,
        seqlens=context_lens.data_ptr(), n=0, out=out.data_ptr(), o_stride_b=out.stride(0),
        o_stride_h=out.stride(1), o_stride_m=0, lse=None, o_part=None, lse_part=None,
        batch=num_seqs, h_q=h_q, h_kv=h_kv, m=1, d=d, num_splits=s, split_tokens=split_tokens,
        scale=float(attn_scale), causal=0, dtype=code)
    _launch(args, device, query.dtype, num_seqs * h_q, d, s)
    return out


def _dense_decode(q, k, v, causal, sm_scale, want_lse):
    _require(q.dim() == 4 and k.dim() == 4 and v.dim() == 4, "q, k, v must be [B, H, T, D]")
    batch, h_q, m, d = q.shape
    _require(k.shape[-1] == d and v.shape[-1] == d, "feature size of q, k, v should be equal")
    _require(d in HEAD_DIMS, f"head dim {d} not in {HEAD_DIMS}")
    _require(k.shape[0] == batch and v.shape[0] == batch, "batch sizes differ")
    h_kv, n = k.shape[1], k.shape[2]
    _require(v.shape[1] == h_kv and v.shape[2] == n, "k and v shapes differ")
    _require(h_kv >= 1 and h_q % h_kv == 0, "number of heads in q must be a multiple of that in k & v")
    code = _dtype_code(q.dtype)
    _require(k.dtype == q.dtype and v.dtype == q.dtype, "q, k, v dtypes differ")
    _require(all(t.is_cuda and t.device == q.device for t in (q, k, v)),
             "q, k, v must be CUDA (HIP) tensors on one device")
    q, k, v = (t if t.stride(-1) == 1 else t.contiguous() for t in (q, k, v))
    if not (_aligned(q, (0, 1, 2)) and _aligned(k, (0, 1, 2)) and _aligned(v, (0, 1, 2))):
        q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(d)
    _require(math.isfinite(sm_scale), "sm_scale must be finite")
    device = q.device
    o = torch.empty_like(q)
    if o.stride(-1) != 1 or not _aligned(o, (0, 1, 2)):
        o = torch.empty(q.shape, dtype=q.dtype, device=device)
    lse = torch.empty((batch, h_q, m), dtype=torch.float32, device=device) if want_lse else None
    s = choose_splits(batch, h_kv, (h_q // h_kv) * m, n, _cu_count(device))
    split_tokens = -(-n // s) if n > 0 else 1
    s = max(1, -(-n // split_tokens)) if n > 0 else 1
    if s == 1:
        split_tokens = 1 << 30
    args = _lib.GqaArgs(
        q=q.data_ptr(), q_stride_b=q.stride(0), q_stride_h=q.stride(1), q_stride_m=q.stride(2),
        k=k.data_ptr(), v=v.data_ptr(), k_stride_0=k.stride(0), k_stride_h=k.stride(1),
        k_stride_t=k.stride(2), v_stride_0=v.stride(0), v_stride_h=v.stride(1),
        v_stride_t=v.stride(2), block_table=None, bt_stride_b=0, max_blocks_per_seq=0,
        block_size=0, num_blocks=0, seqlens=None, n=n, out=o.data_ptr(), o_stride_b=o.stride(0),
        o_stride_h=o.stride(1), o_stride_m=o.stride(2),
        lse=None if lse is None else lse.data_ptr(), o_part=None, lse_part=None, batch=batch,
        h_q=h_q, h_kv=h_kv, m=m, d=d, num_splits=s, split_tokens=split_tokens,
        scale=float(sm_scale), causal=int(bool(causal)), dtype=code)
    _launch(args, device, q.dtype, batch * h_q * m, d, s)
    return o, lse


def flash_attention_split_kv(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                             causal: bool = False, sm_scale: Optional[float] = None
                             ) -> torch.Tensor:
    """Flash decoding over contiguous K/V (``split_kv.py:280-344``): returns ``o`` shaped and
    typed like ``q``."""
    o, _ = _dense_decode(q, k, v, causal, sm_scale, False)
    return o


def flash_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, causal: bool = False,
                    sm_scale: Optional[float] = None, dropout_p: float = 0.0,
                    return_log_normalizer: bool = False, return_total_attention: bool = False,
                    return_seed_offset: bool = False):
    """The forward of ``flag_attn.flash_attention`` (``flash.py:269-300``) through its
    split-KV decode path.  Dropout and total attention (training-path outputs) are not
    provided and raise; there is no backward."""
    _require(dropout_p == 0.0, "dropout is a training-path feature; dropout_p must be 0")
    _require(not return_total_attention, "return_total_attention is not supported")
    want_lse = return_log_normalizer
    o, lse = _dense_decode(q, k, v, causal, sm_scale, want_lse)
    if return_log_normalizer or return_total_attention or return_seed_offset:
        return o, lse, None, None, None
    return o
