"""CPU oracle for the MLA decode path.  TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py``
may import this module, and only as the checker; the product path
(``flagattention_amd``) never calls it.

It restates, in float32 PyTorch on the CPU, what the reference computes on this path:

* paged gather: ``src/flag_attn/testing/paged.py:37-52`` -- token ``j`` of sequence
  ``b`` is row ``j % block_size`` of page ``block_table[b, j // block_size]``;
  vectorised here with index tensors instead of the per-token Python loop;
* attention with log-normaliser: ``src/flag_attn/testing/flash.py:19-84`` with
  ``upcast=True, return_log_normalizer=True``: ``S = q k^T * sm_scale``; causal keeps
  ``m + (N - M) >= n`` (bottom-right aligned, ``:47-55``); ``lse = logsumexp(S)``
  (``:58-59``); ``P = softmax(S)`` in fp32 (``:62``); ``out = P v``.  The single latent KV
  head is broadcast over the query heads instead of ``repeat_interleave`` (``:42-44``),
  which is the same arithmetic without the 128x copy;
* rows with no visible key: ``out = 0``, ``lse = -inf``, the convention of the reference
  split-KV kernel for empty rows (``src/flag_attn/split_kv.py:161-164``);
* split combine in LSE form: ``src/flag_attn/split_kv.py:198-228``.

Pieces the reference does not have (it has no MLA, sparse or fp8 path) are restated from
their definitions: the sparse index -> cache row translation, the fp8-e4m3 row codec and the
tile-scheduler metadata spec.  How each function is pinned (golden vectors, closed forms,
brute force) is stated in its docstring; the pins live in ``tests/test_oracle*.py``.
"""
from __future__ import annotations

import math
from typing import List, Optional, Sequence, Tuple

import numpy as np
import torch

PAGE = 64
D_QK = 576
D_V = 512
FP8_ROW_BYTES = 656
MD_STRIDE = 8


# --------------------------------------------------------------------------- gather

def gather_rows(k_cache: torch.Tensor, block_table: torch.Tensor, b: int,
                positions: torch.Tensor) -> torch.Tensor:
    """Cache rows of logical positions of sequence ``b``: ``k_cache[bt[b, j // 64], j % 64]``.

    Restates ``testing/paged.py:44-50``.  Pinned by ``tests/golden`` (explicit-loop gather)
    and by the identity-table case (gather == contiguous slice).
    """
    pos = positions.long()
    pages = block_table[b].long()[pos // PAGE]
    return k_cache[pages, pos % PAGE, 0]


def sparse_rows_ref(indices: torch.Tensor, block_table: torch.Tensor,
                    cache_seqlens: torch.Tensor, num_kv_blocks: int) -> torch.Tensor:
    """Physical cache row of every sparse slot, -1 for an unused slot.

    ``rows[b, s, j] = block_table[b, i // 64] * 64 + i % 64`` for ``i = indices[b, s, j]``
    with ``0 <= i < cache_seqlens[b]`` and a page id inside ``[0, num_kv_blocks)``; slots
    past ``topk`` (padding to a multiple of 64) are -1.  Same page arithmetic as
    ``testing/paged.py:44-47``.  Pinned by explicit loops in ``tests/golden``.
    """
    bsz, s_q, topk = indices.shape
    topk_pad = -(-topk // PAGE) * PAGE
    out = torch.full((bsz, s_q, topk_pad), -1, dtype=torch.int32)
    idx = indices.long()
    lens = cache_seqlens.long().view(bsz, 1, 1)
    valid = (idx >= 0) & (idx < lens) & ((idx // PAGE) < block_table.shape[1])
    safe = torch.where(valid, idx, torch.zeros_like(idx))
    bt = block_table.long()
    pages = torch.gather(bt.unsqueeze(1).expand(bsz, s_q, bt.shape[1]), 2, safe // PAGE)
    valid &= (pages >= 0) & (pages < num_kv_blocks)
    rows = torch.where(valid, pages * PAGE + safe % PAGE, torch.full_like(idx, -1))
    out[:, :, :topk] = rows.to(torch.int32)
    return out


# --------------------------------------------------------------------------- fp8 codec

def fp8_e4m3fn_table() -> np.ndarray:
    """float32 value of each of the 256 OCP fp8-e4m3 ("fn") codes, from the bit layout.

    sign | 4 exponent bits (bias 7) | 3 mantissa bits; exponent 0 is subnormal
    (``2^-6 * m / 8``); ``0x7F`` / ``0xFF`` are NaN; there is no infinity (max 448).
    Pinned against ``torch.float8_e4m3fn`` (an independent library decoder) over all codes.
    """
    out = np.empty(256, dtype=np.float32)
    for c in range(256):
        s = -1.0 if c & 0x80 else 1.0
        e = (c >> 3) & 0xF
        m = c & 0x7
        if e == 0xF and m == 0x7:
            out[c] = np.nan
        elif e == 0:
            out[c] = s * (2.0 ** -6) * (m / 8.0)
        else:
            out[c] = s * (2.0 ** (e - 7)) * (1.0 + m / 8.0)
    return out


_FP8_TABLE = torch.from_numpy(fp8_e4m3fn_table())


def fp8_rows_dequant(raw: torch.Tensor) -> torch.Tensor:
    """Decode 656-byte fp8 cache rows to float32 ``[..., 576]``.

    Row layout: bytes ``[0, 512)`` e4m3 codes of the 512 latent dims, ``[512, 528)`` four
    little-endian fp32 scales (one per 128 dims), ``[528, 656)`` 64 bf16 rope dims.
    ``latent[d] = decode(code[d]) * scale[d // 128]`` in fp32.
    """
    assert raw.dtype == torch.uint8 and raw.shape[-1] == FP8_ROW_BYTES
    lead = raw.shape[:-1]
    flat = raw.reshape(-1, FP8_ROW_BYTES)
    codes = _FP8_TABLE[flat[:, :512].long()]
    scales = flat[:, 512:528].contiguous().view(torch.float32)
    latent = codes.view(-1, 4, 128) * scales.view(-1, 4, 1)
    rope = flat[:, 528:656].contiguous().view(torch.bfloat16).float()
    return torch.cat([latent.reshape(-1, 512), rope], dim=1).reshape(*lead, D_QK)


def fp8_rows_quantize(latent: torch.Tensor, rope: torch.Tensor,
                      scales: torch.Tensor) -> torch.Tensor:
    """Encode fp32 latent ``[..., 512]``, bf16 rope ``[..., 64]`` and fp32 scales
    ``[..., 4]`` into 656-byte rows: ``code = e4m3(clamp(latent / scale, +-448))``
    (round-to-nearest-even via ``torch.float8_e4m3fn``).  Test-data producer."""
    lead = latent.shape[:-1]
    lat = latent.reshape(-1, 4, 128).float() / scales.reshape(-1, 4, 1).float()
    codes = lat.clamp(-448.0, 448.0).to(torch.float8_e4m3fn).view(torch.uint8).reshape(-1, 512)
    sc = scales.reshape(-1, 4).float().contiguous().view(torch.uint8)
    rp = rope.reshape(-1, 64).to(torch.bfloat16).contiguous().view(torch.uint8)
    return torch.cat([codes, sc, rp], dim=1).reshape(*lead, FP8_ROW_BYTES)


def fp8_tile_scales(latent: torch.Tensor) -> torch.Tensor:
    """Per-128-dim scales of the fp8 row format as the cache writer picks them:
    ``scale = amax / 448`` in fp32 over each tile of 128 latent dims (so the largest value
    maps to the largest finite e4m3 code), ``1.0`` for an all-zero tile.  ``latent``
    ``[..., 512]`` -> scales ``[..., 4]``.  IEEE specials follow torch's arithmetic: a NaN
    makes the tile's amax NaN and its scale ``1.0`` (``NaN > 0`` is false); an infinity
    makes the scale infinite."""
    lat = latent.float().reshape(*latent.shape[:-1], 4, 128)
    amax = lat.abs().amax(dim=-1)
    return torch.where(amax > 0, amax / 448.0, torch.ones_like(amax))


def kvcache_write_ref(k_cache: torch.Tensor, latent: torch.Tensor, rope: torch.Tensor,
                      slot_mapping: torch.Tensor, is_fp8: bool) -> torch.Tensor:
    """A copy of ``k_cache`` with token ``i`` written to physical row ``slot_mapping[i]``
    (page ``slot // 64``, row ``slot % 64``; slots outside the cache are skipped):
    bf16 rows ``latent | rope`` (1152 B), or fp8 rows ``fp8_rows_quantize(latent, rope,
    fp8_tile_scales(latent))`` (656 B)."""
    out = k_cache.clone()
    flat = out.view(-1, out.shape[-1])
    nrows = flat.shape[0]
    if is_fp8:
        rows = fp8_rows_quantize(latent.float(), rope, fp8_tile_scales(latent))
    else:
        rows = torch.cat([latent, rope], dim=-1).to(out.dtype)
    for i, slot in enumerate(slot_mapping.tolist()):
        if 0 <= slot < nrows:
            flat[slot] = rows[i]
    return out


# --------------------------------------------------------------------------- attention

def attention_lse(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, sm_scale: float,
                  causal: bool) -> Tuple[torch.Tensor, torch.Tensor]:
    """fp32 attention of ``q [H, M, Dqk]`` over one shared KV head ``k [N, Dqk]``,
    ``v [N, Dv]``; returns ``out [H, M, Dv]`` and ``lse [H, M]``.

    Restates ``testing/flash.py:47-75`` (upcast path).  Rows with no visible key give
    ``out = 0, lse = -inf``.  Pinned by a float64 brute-force golden set and closed forms.
    """
    q = q.float()
    k = k.float()
    v = v.float()
    h, m, _ = q.shape
    n = k.shape[0]
    s = torch.matmul(q, k.t()) * sm_scale  # [H, M, N]
    if causal:
        ms = torch.arange(m).unsqueeze(-1)
        ns = torch.arange(n)
        s = torch.where(ms + (n - m) >= ns, s, torch.tensor(float("-inf")))
    lse = torch.logsumexp(s, dim=-1) if n > 0 else torch.full((h, m), float("-inf"))
    empty = torch.isneginf(lse)
    p = torch.exp(s - torch.where(empty, torch.zeros_like(lse), lse).unsqueeze(-1))
    p = torch.where(empty.unsqueeze(-1), torch.zeros_like(p), p)
    out = torch.matmul(p, v)
    return out, lse


def attention_lse_lowp(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, sm_scale: float,
                       causal: bool, dtype: torch.dtype = torch.bfloat16
                       ) -> Tuple[torch.Tensor, torch.Tensor]:
    """The same attention with the reference's ``upcast=False`` arithmetic
    (``testing/flash.py:47-75``): ``S = q k^T * sm_scale`` in ``dtype``, softmax in fp32,
    ``P`` cast back to ``dtype``, ``P v`` in ``dtype``.  This is the ``torch_lowp`` leg of
    the reference's accuracy rule ``max|hyp - ref| <= 2 max|lowp - ref| + 1e-5``
    (``tests/flag_attn/test_flash_attention.py:119-127``).  Returns ``out`` (fp32 view of
    the ``dtype`` result) and ``lse`` of the low-precision ``S``."""
    q = q.to(dtype)
    k = k.to(dtype)
    v = v.to(dtype)
    h, m, _ = q.shape
    n = k.shape[0]
    if n == 0:
        return (torch.zeros((h, m, v.shape[1]), dtype=torch.float32),
                torch.full((h, m), float("-inf")))
    s = torch.matmul(q, k.t().contiguous()) * sm_scale
    if causal:
        ms = torch.arange(m).unsqueeze(-1)
        ns = torch.arange(n)
        s = torch.where(ms + (n - m) >= ns, s, torch.tensor(float("-inf"), dtype=dtype))
    s = s.float()
    lse = torch.logsumexp(s, dim=-1)
    empty = torch.isneginf(lse)
    p = torch.softmax(s, dim=-1, dtype=torch.float32)
    p = torch.where(empty.unsqueeze(-1), torch.zeros_like(p), p)
    out = torch.matmul(p.to(dtype), v).float()
    return out, lse


def dense_decode_ref(q: torch.Tensor, k_cache: torch.Tensor, block_table: torch.Tensor,
                     cache_seqlens: torch.Tensor, sm_scale: float, causal: bool = False,
                     batches: Optional[Sequence[int]] = None, lowp: bool = False
                     ) -> Tuple[torch.Tensor, torch.Tensor]:
    """Dense paged MLA decode in fp32.  ``q [B, s_q, h_q, 576]``, bf16/fp32 cache
    ``[num_blocks, 64, 1, 576]``; returns ``out [B', s_q, h_q, 512]`` and
    ``lse [B', h_q, s_q]`` for the sequences in ``batches`` (default: all).
    ``lowp=True``: the bf16 arithmetic of ``attention_lse_lowp`` instead."""
    bsz, s_q, h_q, _ = q.shape
    bl = list(range(bsz)) if batches is None else list(batches)
    out = torch.zeros((len(bl), s_q, h_q, D_V), dtype=torch.float32)
    lse = torch.full((len(bl), h_q, s_q), float("-inf"), dtype=torch.float32)
    att = attention_lse_lowp if lowp else attention_lse
    for i, b in enumerate(bl):
        n = int(cache_seqlens[b])
        kv = gather_rows(k_cache, block_table, b, torch.arange(n)).float()
        o, l = att(q[b].float().permute(1, 0, 2), kv, kv[:, :D_V], sm_scale, causal)
        out[i] = o.permute(1, 0, 2)
        lse[i] = l
    return out, lse


def dense_decode_loop(q: torch.Tensor, k_cache: torch.Tensor, block_table: torch.Tensor,
                      cache_seqlens: torch.Tensor, sm_scale: float,
                      batches: Optional[Sequence[int]] = None
                      ) -> Tuple[torch.Tensor, torch.Tensor]:
    """``dense_decode_ref`` with the gather written as ``testing/paged.py:37-52`` writes it:
    a Python loop over the tokens of each sequence, each row taken from page
    ``block_table[b, j // 64]``, offset ``j % 64``, then stacked.  Same arithmetic, so the
    same bits (``tests/test_oracle.py``); kept only as the reference-shaped CPU baseline
    (small inputs: one Python iteration per token)."""
    bsz, s_q, h_q, _ = q.shape
    bl = list(range(bsz)) if batches is None else list(batches)
    out = torch.zeros((len(bl), s_q, h_q, D_V), dtype=torch.float32)
    lse = torch.full((len(bl), h_q, s_q), float("-inf"), dtype=torch.float32)
    tables = block_table.tolist()
    for i, b in enumerate(bl):
        n = int(cache_seqlens[b])
        rows = []
        for j in range(n):
            blk = int(tables[b][j // PAGE])
            rows.append(k_cache[blk, j % PAGE, 0])
        kv = (torch.stack(rows, dim=0) if rows else k_cache.new_zeros((0, D_QK))).float()
        o, l = attention_lse(q[b].float().permute(1, 0, 2), kv, kv[:, :D_V], sm_scale, False)
        out[i] = o.permute(1, 0, 2)
        lse[i] = l
    return out, lse


def sparse_decode_ref(q: torch.Tensor, k_cache: torch.Tensor, block_table: torch.Tensor,
                      cache_seqlens: torch.Tensor, indices: torch.Tensor, sm_scale: float,
                      is_fp8: bool = False, batches: Optional[Sequence[int]] = None,
                      lowp: bool = False) -> Tuple[torch.Tensor, torch.Tensor]:
    """Sparse top-k MLA decode in fp32: query token ``(b, s)`` attends to the valid
    entries of ``indices[b, s]`` (``0 <= i < cache_seqlens[b]``), each a cache row found
    through ``block_table``; fp8 rows are decoded with ``fp8_rows_dequant``.
    ``lowp=True``: the bf16 arithmetic of ``attention_lse_lowp`` instead."""
    bsz, s_q, h_q, _ = q.shape
    bl = list(range(bsz)) if batches is None else list(batches)
    nblk = k_cache.shape[0]
    rows = sparse_rows_ref(indices[bl], block_table[bl], cache_seqlens[bl], nblk)
    out = torch.zeros((len(bl), s_q, h_q, D_V), dtype=torch.float32)
    lse = torch.full((len(bl), h_q, s_q), float("-inf"), dtype=torch.float32)
    flat = k_cache.reshape(nblk * PAGE, -1)
    for i, b in enumerate(bl):
        for s in range(s_q):
            r = rows[i, s]
            r = r[r >= 0].long()
            kv = fp8_rows_dequant(flat[r]) if is_fp8 else flat[r].float()
            att = attention_lse_lowp if lowp else attention_lse
            o, l = att(q[b, s].float().unsqueeze(1), kv, kv[:, :D_V], sm_scale, False)
            out[i, s] = o[:, 0]
            lse[i, :, s] = l[:, 0]
    return out, lse


def combine_ref(o_parts: torch.Tensor, lse_parts: torch.Tensor
                ) -> Tuple[torch.Tensor, torch.Tensor]:
    """LSE combine of split partials ``o_parts [S, R, Dv]`` (each normalised by its own
    split) and ``lse_parts [S, R]``: ``lse = logsumexp_s lse_s``,
    ``out = sum_s exp(lse_s - lse) o_s`` (``split_kv.py:198-228``).  All-empty rows give
    ``out = 0, lse = -inf``.  Pinned by split invariance: combining the attention of any
    partition of the keys equals the attention of all keys."""
    o_parts = o_parts.float()
    lse_parts = lse_parts.float()
    lse = torch.logsumexp(lse_parts, dim=0)
    empty = torch.isneginf(lse)
    w = torch.exp(lse_parts - torch.where(empty, torch.zeros_like(lse), lse).unsqueeze(0))
    w = torch.where(empty.unsqueeze(0), torch.zeros_like(w), w)
    out = (w.unsqueeze(-1) * o_parts).sum(0)
    return out, lse


# --------------------------------------------------------------------------- metadata

def metadata_spec(cache_seqlens: Sequence[int], num_parts: int, fixed_overhead: int,
                  topk: int = 0) -> Tuple[List[List[int]], List[int]]:
    """Tile-scheduler metadata, written from its definition (no reference exists).

    ``nb[b] = ceil(len_b / 64)`` (``ceil(topk / 64)`` for sparse), cost
    ``c[b] = nb[b] + fixed_overhead`` for non-empty sequences, 0 otherwise; ``C``/``G`` are
    the exclusive prefix sums of ``c``/``nb``.  Part ``p`` starts at cost position
    ``x_p = ceil(p * W / P)`` mapped to the global block ``G[b] + max(0, x_p - C[b] -
    overhead)`` of the sequence ``b`` whose cost interval holds ``x_p`` (``NB`` when
    ``x_p >= W``), and covers global blocks ``[gs_p, gs_{p+1})``.  A segment is a non-empty
    part's intersection with one sequence.  Returns ``tile_md`` rows
    ``[begin_b, begin_blk, end_b, end_blk_excl, first_split_local, n_blocks, gs_p, 0]``
    (all zero except ``gs_p`` for an empty part) and ``num_splits`` (``B + 1`` prefix).
    """
    bsz = len(cache_seqlens)
    if topk > 0:
        nb = [-(-topk // PAGE)] * bsz
    else:
        nb = [-(-max(int(x), 0) // PAGE) for x in cache_seqlens]
    c = [n + fixed_overhead if n > 0 else 0 for n in nb]
    C = [0]
    G = [0]
    for b in range(bsz):
        C.append(C[-1] + c[b])
        G.append(G[-1] + nb[b])
    W, NB = C[-1], G[-1]
    gs = []
    for p in range(num_parts + 1):
        x = -(-p * W // num_parts)
        if x >= W:
            gs.append(NB)
            continue
        b = [i for i in range(bsz) if C[i] <= x < C[i + 1]][0]
        gs.append(G[b] + max(0, x - C[b] - fixed_overhead))

    def seq_of(gblk: int) -> int:
        return [i for i in range(bsz) if G[i] <= gblk < G[i + 1]][0]

    md = []
    for p in range(num_parts):
        g0, g1 = gs[p], gs[p + 1]
        if g0 == g1:
            md.append([0, 0, 0, 0, 0, 0, g0, 0])
            continue
        bb, eb = seq_of(g0), seq_of(g1 - 1)
        first = sum(1 for q in range(p)
                    if gs[q] < gs[q + 1] and gs[q + 1] > G[bb] and gs[q] < G[bb + 1])
        md.append([bb, g0 - G[bb], eb, g1 - G[eb], first, g1 - g0, g0, 0])
    num_splits = [0]
    for b in range(bsz):
        n = sum(1 for p in range(num_parts)
                if nb[b] > 0 and gs[p] < gs[p + 1] and gs[p] < G[b + 1] and gs[p + 1] > G[b])
        num_splits.append(num_splits[-1] + n)
    return md, num_splits


# --------------------------------------------------------------------------- workloads

def make_dense_inputs(batch: int, h_q: int, s_q: int, seqlens: Sequence[int], seed: int,
                      scale: float = 1.0, dtype: torch.dtype = torch.bfloat16,
                      extra_blocks: int = 0):
    """Synthetic dense workload: N(0,1)*scale q / cache, block_table = a random permutation
    of a pool sized to the blocks needed (+ ``extra_blocks``), rows padded with 0."""
    gen = torch.Generator().manual_seed(seed)
    nblocks = [-(-int(x) // PAGE) for x in seqlens]
    pool = sum(nblocks) + extra_blocks
    perm = torch.randperm(max(pool, 1), generator=gen).to(torch.int32)
    maxb = max(max(nblocks), 1)
    bt = torch.zeros((batch, maxb), dtype=torch.int32)
    off = 0
    for b, n in enumerate(nblocks):
        bt[b, :n] = perm[off:off + n]
        off += n
    q = (torch.randn((batch, s_q, h_q, D_QK), generator=gen) * scale).to(dtype)
    kc = (torch.randn((max(pool, 1), PAGE, 1, D_QK), generator=gen) * scale).to(dtype)
    lens = torch.tensor(list(seqlens), dtype=torch.int32)
    return q, kc, bt, lens


def make_sparse_indices(batch: int, s_q: int, topk: int, seqlens: Sequence[int], seed: int,
                        invalid_frac: float = 0.02) -> torch.Tensor:
    """``topk`` unique token ids per query token, sampled without replacement from
    ``[0, len_b)``, with a Bernoulli(``invalid_frac``) share set to -1."""
    gen = torch.Generator().manual_seed(seed)
    idx = torch.empty((batch, s_q, topk), dtype=torch.int32)
    for b in range(batch):
        n = int(seqlens[b])
        for s in range(s_q):
            if n >= topk:
                idx[b, s] = torch.randperm(n, generator=gen)[:topk].to(torch.int32)
            else:
                row = torch.full((topk,), -1, dtype=torch.int32)
                row[:n] = torch.randperm(n, generator=gen).to(torch.int32)
                idx[b, s] = row
    if invalid_frac > 0:
        drop = torch.rand(idx.shape, generator=gen) < invalid_frac
        idx[drop] = -1
    return idx


def make_fp8_cache(num_blocks: int, seed: int, lat_scale: float = 0.1):
    """fp8 cache rows: latent N(0,1)*lat_scale quantised with per-128-dim scales drawn
    log-uniform in [1e-3, 1e-1]; rope N(0,1)*lat_scale in bf16."""
    gen = torch.Generator().manual_seed(seed)
    lat = torch.randn((num_blocks, PAGE, 1, 512), generator=gen) * lat_scale
    u = torch.rand((num_blocks, PAGE, 1, 4), generator=gen)
    scales = torch.exp(math.log(1e-3) + u * (math.log(1e-1) - math.log(1e-3)))
    rope = (torch.randn((num_blocks, PAGE, 1, 64), generator=gen) * lat_scale).to(torch.bfloat16)
    return fp8_rows_quantize(lat, rope, scales)
