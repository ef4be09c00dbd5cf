"""CPU oracle for the grouped-query decode paths.  TEST INFRASTRUCTURE ONLY.

Only ``tests/`` (and ``bench.py``'s ``cpu_baseline`` leg) may import this module, and only
as the checker; the product path (``flagattention_amd.gqa``) never calls it.

Restates, on the CPU:

* ``paged_attention_loop`` -- ``src/flag_attn/testing/paged.py:18-65`` as written: a
  per-sequence, per-token Python gather (token ``j`` from page ``block_table[j // bs]``,
  row ``j % bs``, ``:37-52``), GQA by ``repeat_interleave`` (``:53-56``), fp32 ``bmm`` ->
  ``softmax`` -> ``bmm`` (``:58-60``), cast to the cache dtype (``:61``);
* ``paged_attention_ref`` -- the same arithmetic with the gather vectorised (index tensors
  instead of the token loop); pinned to ``paged_attention_loop`` bit for bit;
* ``paged_attention_lowp`` -- the same gather with ``testing/flash.py``'s ``upcast=False``
  arithmetic: the low-precision leg of the three-way rule for the paged sweeps;
* ``flash_attention_ref`` -- ``src/flag_attn/testing/flash.py:19-84``: GQA by
  ``repeat_interleave`` (``:42-44``), ``S = q k^T * sm_scale`` in the working dtype
  (fp32 with ``upcast=True``, the input dtype otherwise), bottom-right causal mask
  ``m + (N - M) >= n`` (``:47-55``), ``logsumexp`` of ``S`` in fp32 (``:58-59``), fp32
  softmax (``:62``), ``P`` cast to ``v``'s dtype for ``P v`` (``:73``), output cast to the
  input dtype (``:74-75``).  ``upcast=False`` is the ``torch_lowp`` leg of the reference's
  accuracy rule (``tests/flag_attn/test_flash_attention.py:119-127``).
"""
from __future__ import annotations

import math
from typing import Optional, Tuple

import torch


def paged_attention_loop(query, key_cache, value_cache, block_tables, context_lens,
                         scale) -> torch.Tensor:
    """``testing/paged.py:18-65`` restated line for line (small inputs only)."""
    output = torch.empty_like(query)
    num_query_heads = query.shape[1]
    num_kv_heads = value_cache.shape[1]
    group = num_query_heads // num_kv_heads
    block_size = value_cache.shape[2]
    head_size = value_cache.shape[3]
    tables = block_tables.cpu().tolist()
    lens = context_lens.cpu().tolist()
    for i in range(query.shape[0]):
        q = query[i].unsqueeze(0)
        keys, values = [], []
        for j in range(int(lens[i])):
            blk = int(tables[i][j // block_size])
            off = j % block_size
            keys.append(key_cache[blk, :, off, :])
            values.append(value_cache[blk, :, off, :])
        keys = torch.stack(keys, dim=0)
        values = torch.stack(values, dim=0)
        if group > 1:
            keys = torch.repeat_interleave(keys, group, dim=1)
            values = torch.repeat_interleave(values, group, dim=1)
        s = torch.bmm(q.transpose(0, 1).float(), keys.permute(1, 2, 0).float()) * scale
        p = torch.softmax(s, dim=-1)
        out = torch.bmm(p, values.transpose(0, 1).float()).transpose(0, 1)
        out = out.to(values.dtype)
        output[i].copy_(out.view(num_query_heads, head_size))
    return output


def paged_attention_ref(query, key_cache, value_cache, block_tables, context_lens,
                        scale, out_fp32: bool = False) -> torch.Tensor:
    """``paged_attention_loop`` with the token gather vectorised (same fp32 arithmetic).
    ``out_fp32=True`` returns the fp32 result before the cast to the cache dtype
    (``testing/paged.py:61``), the reference point of the three-way accuracy rule."""
    output = torch.empty(query.shape, dtype=torch.float32) if out_fp32 else torch.empty_like(query)
    h_q = query.shape[1]
    h_kv = value_cache.shape[1]
    group = h_q // h_kv
    bs = value_cache.shape[2]
    d = value_cache.shape[3]
    for i in range(query.shape[0]):
        n = int(context_lens[i])
        pos = torch.arange(n)
        pages = block_tables[i].long()[pos // bs]
        keys = key_cache[pages, :, pos % bs, :]      # [n, h_kv, d]
        values = value_cache[pages, :, pos % bs, :]
        if group > 1:
            keys = torch.repeat_interleave(keys, group, dim=1)
            values = torch.repeat_interleave(values, group, dim=1)
        q = query[i].unsqueeze(0)
        s = torch.bmm(q.transpose(0, 1).float(), keys.permute(1, 2, 0).float()) * scale
        p = torch.softmax(s, dim=-1)
        out = torch.bmm(p, values.transpose(0, 1).float()).transpose(0, 1)
        output[i].copy_((out if out_fp32 else out.to(values.dtype)).view(h_q, d))
    return output


def paged_attention_lowp(query, key_cache, value_cache, block_tables, context_lens,
                         scale) -> torch.Tensor:
    """The paged gather of ``testing/paged.py:37-56`` followed by the ``upcast=False``
    arithmetic of ``testing/flash.py:47-75`` in the cache dtype: ``S = q k^T`` and
    ``* scale`` in the dtype, softmax in fp32, ``P`` cast to the dtype, ``P v`` in the
    dtype.  The reference's paged tests have no such leg (they use ``allclose`` against the
    fp32 oracle); this one gives the paged sweeps the ``torch_lowp`` side of the rule
    ``max|hyp - ref| <= 2 max|lowp - ref| + 1e-5`` of
    ``tests/flag_attn/test_flash_attention.py:119-127``.  Returns the dtype result."""
    dtype = query.dtype
    output = torch.empty_like(query)
    h_q = query.shape[1]
    h_kv = value_cache.shape[1]
    group = h_q // h_kv
    bs = value_cache.shape[2]
    d = value_cache.shape[3]
    for i in range(query.shape[0]):
        n = int(context_lens[i])
        pos = torch.arange(n)
        pages = block_tables[i].long()[pos // bs]
        keys = key_cache[pages, :, pos % bs, :].to(dtype)      # [n, h_kv, d]
        values = value_cache[pages, :, pos % bs, :].to(dtype)
        if group > 1:
            keys = torch.repeat_interleave(keys, group, dim=1)
            values = torch.repeat_interleave(values, group, dim=1)
        q = query[i].unsqueeze(1)                               # [h_q, 1, d]
        s = torch.bmm(q, keys.permute(1, 2, 0).contiguous()) * scale
        p = torch.softmax(s.float(), dim=-1, dtype=torch.float32)
        out = torch.bmm(p.to(dtype), values.transpose(0, 1).contiguous())  # [h_q, 1, d]
        output[i].copy_(out.view(h_q, d))
    return output


def flash_attention_ref(q, k, v, causal: bool, sm_scale: Optional[float] = None,
                        upcast: bool = True) -> Tuple[torch.Tensor, torch.Tensor]:
    """``testing/flash.py:19-84`` with ``return_log_normalizer=True``: returns
    ``(o in the input dtype, lse fp32 [B, H, M])``."""
    input_dtype = q.dtype
    if upcast:
        q, k, v = q.float(), k.float(), v.float()
    d = q.shape[-1]
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(d)
    group = q.shape[1] // k.shape[1]
    if group > 1:
        k = torch.repeat_interleave(k, repeats=group, dim=1)
        v = torch.repeat_interleave(v, repeats=group, dim=1)
    n = k.shape[-2]
    m = q.shape[-2]
    ms = torch.arange(m).unsqueeze(-1)
    ns = torch.arange(n)
    s = torch.matmul(q, k.transpose(2, 3).contiguous()) * sm_scale
    if causal:
        s = torch.where(ms + (n - m) >= ns, s, float("-inf"))
    s = s.to(torch.float32)
    lse = torch.logsumexp(s, dim=-1)
    p = torch.softmax(s, dim=-1, dtype=torch.float32)
    if causal:
        p = torch.where(ms + (n - m) >= ns, p, 0.0)
    o = torch.matmul(p.to(v.dtype), v).to(input_dtype)
    return o, lse
