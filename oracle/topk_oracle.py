"""CPU oracle for the top-k index producer.  TEST INFRASTRUCTURE ONLY.

Only ``tests/`` and ``bench.py``'s ``cpu_baseline`` leg may import this module, and only
as the checker; the product path (``flagattention_amd.mla.topk_indices``) never calls it.

The reference has no sparse attention and no index producer, so there is no reference
line to follow: this restates the definition of the ``indices`` tensor the sparse decode
consumes (logical token ids per query token, ``-1`` = no key) as produced from per-key
indexer scores:

* query token ``t`` of sequence ``b`` sees keys ``[0, n)``,
  ``n = cache_seqlens[b] - (s_q - 1 - t)`` when causal (the bottom-right alignment of
  ``src/flag_attn/testing/flash.py:47-55``), else ``cache_seqlens[b]``; clipped to
  ``[0, len]``;
* it keeps the ``min(topk, n)`` largest scores: scores compare by the total order of
  their float32 bit patterns (sign-flip map to uint32: ``-NaN < -inf < -0 < +0 < +inf <
  +NaN``), equal scores rank the lower position first;
* the kept positions come out in ascending order, then ``-1``.

Pins (``tests/test_topk_oracle.py``): ``torch.topk``'s index set on rows of distinct
finite scores (a library routine), closed forms (all-equal rows keep the first ``topk``
positions; rows with ``n <= topk`` keep ``0..n-1``), the float ordering of specials
against ``numpy``'s own comparisons, a brute-force exchange check (no kept score ranks
below a dropped one), and planted mistakes that must fail them.
"""
from __future__ import annotations

import numpy as np


def order_keys(scores: np.ndarray) -> np.ndarray:
    """float32 -> uint32 keys whose unsigned order is the total order of the floats."""
    u = np.ascontiguousarray(scores, dtype=np.float32).view(np.uint32)
    return np.where(u & np.uint32(0x80000000), ~u, u | np.uint32(0x80000000)).astype(np.uint32)


def visible_lengths(cache_seqlens, s_q: int, length: int, causal: bool) -> np.ndarray:
    """[B, s_q] count of keys each query token sees."""
    lens = np.asarray(cache_seqlens, dtype=np.int64).reshape(-1, 1)
    t = np.arange(s_q, dtype=np.int64).reshape(1, -1)
    n = lens - (s_q - 1 - t) if causal else np.broadcast_to(lens, (lens.shape[0], s_q))
    return np.clip(n, 0, length)


def topk_indices_ref(scores: np.ndarray, cache_seqlens, topk: int,
                     causal: bool = False) -> np.ndarray:
    """scores float32 [B, s_q, L] -> int32 [B, s_q, topk]."""
    scores = np.asarray(scores, dtype=np.float32)
    bsz, s_q, length = scores.shape
    n_vis = visible_lengths(cache_seqlens, s_q, length, causal)
    out = np.full((bsz, s_q, topk), -1, dtype=np.int32)
    for b in range(bsz):
        for t in range(s_q):
            n = int(n_vis[b, t])
            if n <= topk:
                out[b, t, :n] = np.arange(n, dtype=np.int32)
                continue
            keys = order_keys(scores[b, t, :n]).astype(np.int64)
            pos = np.arange(n, dtype=np.int64)
            order = np.lexsort((pos, -keys))  # key descending, then position ascending
            out[b, t] = np.sort(order[:topk]).astype(np.int32)
    return out
