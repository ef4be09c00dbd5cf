"""GPU parity of the HIP MLA decode path against the CPU oracle (MI355X only).

Bars: scheduler metadata and sparse gather rows bit-exact; out within atol 2e-2 /
rtol 1e-2 and lse within 1e-3 of the fp32 oracle, and out within the reference's rule
max|hyp - ref| <= 2 max|bf16 oracle - ref| + 1e-5 (tolerances in tests/_helpers.py).
Every call goes through the ``flag_attn`` operators.
"""
import math
import os

import numpy as np
import pytest
import torch

import flag_attn
import flagattention_amd as fa
from oracle import mla_oracle as orc
from tests._helpers import (DEV, assert_close, dense_refs, need_gpu, run_dense, run_sparse,
                            say, sparse_refs)

pytestmark = pytest.mark.gpu
SCALE = 192 ** -0.5


def _npz(golden_dir, name):
    return np.load(os.path.join(golden_dir, name), allow_pickle=False)


def _t(a):
    return torch.from_numpy(np.ascontiguousarray(a))


# ---------------------------------------------------------------- metadata

@pytest.mark.parametrize("lens,parts,topk", [
    ([256, 384], 4, 0),
    ([100, 0, 65], 1, 0),
    ([64], 4, 0),
    ([0, 0, 0], 8, 0),
    ([5000] * 8, 16, 2048),
    (list(range(0, 64 * 37, 37)), 128, 0),
    ([4096 + (i * 977) % 4097 for i in range(64)], 128, 0),
    ([128 * (1 + (i * 7919) % 512) for i in range(32)], 64, 0),
    ([1 + (i * 31) % 100000 for i in range(1000)], 256, 0),
    # either side of the 256-thread launch's limits (P <= 256, B <= 1024)
    ([1 + (i * 97) % 7000 for i in range(1024)], 256, 0),
    ([1 + (i * 97) % 7000 for i in range(1025)], 200, 0),
    ([4000] * 16, 257, 0),
    # batch / part limits; p * W passes 2^32 (the block total itself stays an int32)
    ([(i * 2654435761) % 2**25 for i in range(4096)], 1024, 0),
    ([3000], 1024, 0),
    # batches of 128 / 129 / 256 / 257 with empty sequences, short sequences under many
    # parts (more parts than blocks), all-empty and tiny top-k batches
    ([(i * 7919) % 9000 if i % 5 else 0 for i in range(128)], 256, 0),
    ([(i * 7919) % 9000 if i % 5 else 0 for i in range(129)], 256, 0),
    ([(i * 7919) % 9000 if i % 7 else 0 for i in range(256)], 1000, 0),
    ([(i * 7919) % 9000 if i % 7 else 0 for i in range(257)], 1000, 0),
    ([1 + (i * 31) % 200 for i in range(100)], 1024, 0),
    ([0] * 40 + [70] + [0] * 40, 255, 0),
    ([0] * 200, 300, 2048),
    ([1] * 128, 256, 100),
])
def test_metadata_kernel_matches_spec(lens, parts, topk):
    need_gpu()
    say(f"metadata lens={len(lens)} parts={parts} topk={topk}")
    ld = torch.tensor(lens, dtype=torch.int32, device=DEV)
    md, ns = flag_attn.get_mla_metadata(ld, 128, 1, num_heads_q=128, topk=topk or None,
                                        num_sm_parts=parts)
    torch.cuda.synchronize()
    want_md, want_ns = orc.metadata_spec(lens, parts, fa.mla.overhead_blocks(bool(topk)), topk)
    assert md.cpu().tolist() == want_md
    assert ns.cpu().tolist() == want_ns


# ---------------------------------------------------------------- sparse gather rows

def test_sparse_rows_golden_bit_exact(golden_dir):
    need_gpu()
    g = _npz(golden_dir, "sparse_bf16.npz")
    rows = flag_attn.mla.sparse_rows(_t(g["indices"]).to(DEV), _t(g["block_table"]).to(DEV),
                                     _t(g["cache_seqlens"]).to(DEV), g["k_cache"].shape[0])
    assert torch.equal(rows.cpu(), _t(g["rows"]))


def test_sparse_rows_random_bit_exact():
    need_gpu()
    gen = torch.Generator().manual_seed(11)
    lens = torch.tensor([3000, 70, 1, 9000], dtype=torch.int32)
    bt = torch.randint(-2, 200, (4, 150), generator=gen, dtype=torch.int32)  # some bad pages
    idx = torch.randint(-3, 9500, (4, 3, 1000), generator=gen, dtype=torch.int32)
    rows = flag_attn.mla.sparse_rows(idx.to(DEV), bt.to(DEV), lens.to(DEV), 190)
    assert torch.equal(rows.cpu(), orc.sparse_rows_ref(idx, bt, lens, 190))


# ---------------------------------------------------------------- dense

@pytest.mark.parametrize("name", ["dense_cfg1.npz", "dense_causal_sq2.npz"])
@pytest.mark.parametrize("parts", [None, 1, 3])
def test_dense_golden(golden_dir, name, parts):
    need_gpu()
    say(f"dense golden {name} parts={parts}")
    g = _npz(golden_dir, name)
    q = _t(g["q"]).to(torch.bfloat16)
    kc = _t(g["k_cache"]).to(torch.bfloat16)
    bt, lens = _t(g["block_table"]), _t(g["cache_seqlens"])
    scale, causal = float(g["sm_scale"]), bool(g["causal"])
    out, lse, _, _ = run_dense(q, kc, bt, lens, scale, causal, parts)
    low, _ = orc.dense_decode_ref(q, kc, bt, lens, scale, causal, lowp=True)
    assert_close(out, lse, _t(g["out"]).float(), _t(g["lse"]).float(), low)


DENSE_CASES = [
    # (batch, h_q, s_q, lens, causal, parts)
    (2, 16, 1, [256, 384], False, None),
    (6, 128, 1, [1, 63, 64, 65, 1000, 4097], False, None),
    (6, 128, 1, [1, 63, 64, 65, 1000, 4097], False, 1),
    (6, 128, 1, [1, 63, 64, 65, 1000, 4097], False, 37),
    (4, 128, 2, [1, 2, 129, 3000], True, None),
    (4, 128, 2, [1, 2, 129, 3000], True, 5),
    (3, 64, 1, [0, 500, 0], False, None),
    (3, 16, 2, [65, 7, 200], True, 2),
    (2, 100, 1, [700, 300], False, None),  # h_q not a multiple of 64
    (2, 128, 3, [190, 64], True, None),
    (2, 64, 2, [300, 1000], False, None),  # several query tokens, no causal mask
    (2, 1, 1, [500, 70], False, None),  # one query head
    (3, 8, 4, [33, 512, 2], True, 3),  # four causal tokens, one shorter than s_q
]


@pytest.mark.parametrize("case", DENSE_CASES, ids=lambda c: f"B{c[0]}h{c[1]}s{c[2]}c{int(c[4])}p{c[5]}")
def test_dense_random(case):
    need_gpu()
    batch, h_q, s_q, lens, causal, parts = case
    say(f"dense random {case}")
    q, kc, bt, ld = orc.make_dense_inputs(batch, h_q, s_q, lens, seed=sum(lens) + h_q,
                                          scale=1.0, extra_blocks=3)
    out, lse, _, _ = run_dense(q, kc, bt, ld, SCALE, causal, parts)
    assert_close(out, lse, *dense_refs(q, kc, bt, ld, SCALE, causal))


@pytest.mark.parametrize("parts", [None, 7])
def test_dense_aliased_block_table(parts):
    """Block tables drawn with replacement, as the reference's paged tests draw them
    (tests/flag_attn/test_paged_attention.py:54): pages shared between sequences and
    repeated inside one sequence."""
    need_gpu()
    say(f"dense aliased block table parts={parts}")
    gen = torch.Generator().manual_seed(54)
    pool, lens = 40, [3000, 1, 640, 2050]
    kc = torch.randn((pool, 64, 1, 576), generator=gen).to(torch.bfloat16)
    q = torch.randn((4, 1, 128, 576), generator=gen).to(torch.bfloat16)
    bt = torch.randint(0, pool, (4, 47), generator=gen, dtype=torch.int32)
    bt[0, 5] = bt[0, 2]  # a repeated page inside one sequence
    bt[2, 3] = bt[0, 7]  # and one shared with another sequence
    ld = torch.tensor(lens, dtype=torch.int32)
    out, lse, _, _ = run_dense(q, kc, bt, ld, SCALE, False, parts)
    assert_close(out, lse, *dense_refs(q, kc, bt, ld, SCALE, False))


def test_dense_split_invariance():
    """The same decode with 1 part (no split) and 128 parts (heavy splitting) agrees."""
    need_gpu()
    lens = [5000, 3000, 129, 64]
    q, kc, bt, ld = orc.make_dense_inputs(4, 128, 1, lens, seed=5, scale=0.5)
    o1, l1, _, ns1 = run_dense(q, kc, bt, ld, SCALE, False, 1)
    o2, l2, _, ns2 = run_dense(q, kc, bt, ld, SCALE, False, 128)
    assert ns1[-1] == 4 and ns2[-1] > 4
    assert torch.allclose(o1.float(), o2.float(), atol=1e-2, rtol=1e-2)
    assert torch.allclose(l1, l2, atol=1e-4)


def test_dense_many_splits_vs_oracle():
    """A sequence cut into more than 64 splits (the combine reduces split weights in
    chunks of 64 lanes) against the oracle."""
    need_gpu()
    lens = [20000, 700]
    q, kc, bt, ld = orc.make_dense_inputs(2, 16, 1, lens, seed=31, scale=0.5)
    out, lse, _, ns = run_dense(q, kc, bt, ld, SCALE, False, 512)
    assert int(ns[1] - ns[0]) > 128
    assert_close(out, lse, *dense_refs(q, kc, bt, ld, SCALE, False))


def test_dense_bad_page_is_masked_not_faulting():
    """A block-table entry outside the cache reads as a masked page."""
    need_gpu()
    q, kc, bt, ld = orc.make_dense_inputs(1, 16, 1, [192], seed=9)
    good = bt.clone()
    bt[0, 1] = kc.shape[0] + 1000
    out, lse, _, _ = run_dense(q, kc, bt, ld, SCALE)
    keep = torch.cat([torch.arange(0, 64), torch.arange(128, 192)])
    kv = orc.gather_rows(kc, good, 0, keep).float()
    ref_o, ref_l = orc.attention_lse(q[0].float().permute(1, 0, 2), kv, kv[:, :512], SCALE, False)
    assert_close(out, lse, ref_o.permute(1, 0, 2).unsqueeze(0), ref_l.unsqueeze(0))



def _plant_key(kc, bt, b, j, value):
    """Set logical token j of sequence b to a constant row (all 576 dims)."""
    kc[int(bt[b, j // 64]), j % 64, 0, :] = value


@pytest.mark.parametrize("parts", [None, 3])
def test_dense_wide_score_spread(parts):
    """A key scoring > 2^64 above the first tile's row max forces the second pass
    (the reference is re-based on the row max); the result must still match."""
    need_gpu()
    say(f"dense wide score spread parts={parts}")
    lens = [700, 300]
    q, kc, bt, ld = orc.make_dense_inputs(2, 128, 1, lens, seed=77, scale=0.1)
    q.fill_(1.0)
    # score of the planted key: 576 * 1.5 * 192^-0.5 * log2(e) = 90 (log2 units),
    # the first tile's scores stay within a few units of 0
    _plant_key(kc, bt, 0, 500, 1.5)
    _plant_key(kc, bt, 1, 10, 1.5)  # in the first tile: no second pass needed
    out, lse, _, _ = run_dense(q, kc, bt, ld, SCALE, False, parts)
    ref_out, ref_lse, low = dense_refs(q, kc, bt, ld, SCALE, False)
    assert float(ref_lse[0].min()) > 60.0  # the planted key dominates
    assert_close(out, lse, ref_out, ref_lse, low)


def test_sparse_wide_score_spread():
    need_gpu()
    say("sparse wide score spread")
    lens = [3000, 3000]
    q, kc, bt, ld = orc.make_dense_inputs(2, 128, 1, lens, seed=78, scale=0.1)
    q.fill_(1.0)
    idx = orc.make_sparse_indices(2, 1, 1024, lens, seed=79, invalid_frac=0.0)
    _plant_key(kc, bt, 0, int(idx[0, 0, 900]), 1.5)  # index slot 900: a late tile
    out, lse = run_sparse(q, kc, bt, ld, idx, SCALE)
    ref_out, ref_lse, low, _ = sparse_refs(q, kc, bt, ld, idx, SCALE)
    assert float(ref_lse[0].min()) > 60.0
    assert_close(out, lse, ref_out, ref_lse, low)


def test_sparse_fp8_wide_score_spread():
    """The second pass through the fp8 pipeline (rows converted in place a step ahead):
    a planted fp8 row of 1.5s (scale 1, rope 1.5) scores ~90 log2 units above the first
    tile's row max, in a late tile of sequence 0 only."""
    need_gpu()
    say("sparse fp8 wide score spread")
    lens = [3000, 3000]
    q, kc, bt, ld = orc.make_dense_inputs(2, 128, 1, lens, seed=80, scale=0.1)
    q.fill_(1.0)
    kc8 = orc.make_fp8_cache(kc.shape[0], seed=81, lat_scale=0.1)
    idx = orc.make_sparse_indices(2, 1, 1024, lens, seed=82, invalid_frac=0.0)
    j = int(idx[0, 0, 900])  # index slot 900: tile 28 of 32
    row = orc.fp8_rows_quantize(torch.full((1, 512), 1.5),
                                torch.full((1, 64), 1.5, dtype=torch.bfloat16), torch.ones((1, 4)))
    kc8[int(bt[0, j // 64]), j % 64, 0, :] = row[0]
    out, lse = run_sparse(q, kc8, bt, ld, idx, SCALE, True)
    ref_out, ref_lse, low, low_lse = sparse_refs(q, kc8, bt, ld, idx, SCALE, True)
    assert float(ref_lse[0].min()) > 60.0  # the planted key dominates sequence 0
    assert float(ref_lse[1].max()) < 30.0  # sequence 1 keeps its first-tile reference
    assert_close(out, lse, ref_out, ref_lse, low, low_lse)


# ---------------------------------------------------------------- sparse

@pytest.mark.parametrize("name,fp8", [("sparse_bf16.npz", False), ("sparse_fp8.npz", True)])
def test_sparse_golden(golden_dir, name, fp8):
    need_gpu()
    say(f"sparse golden {name}")
    g = _npz(golden_dir, name)
    q = _t(g["q"]).to(torch.bfloat16)
    kc = _t(g["k_cache"])
    kc = kc if fp8 else kc.to(torch.bfloat16)
    bt, lens, idx = _t(g["block_table"]), _t(g["cache_seqlens"]), _t(g["indices"])
    scale = float(g["sm_scale"])
    out, lse = run_sparse(q, kc, bt, lens, idx, scale, fp8)
    low, low_lse = orc.sparse_decode_ref(q, kc, bt, lens, idx, scale, is_fp8=fp8, lowp=True)
    assert_close(out, lse, _t(g["out"]).float(), _t(g["lse"]).float(), low,
                 low_lse if fp8 else None)


def sparse_random_inputs(fp8, topk):
    """Inputs of test_sparse_random: N(0,1) q and cache (fp8: latent N(0,1) quantised with
    per-128-dim scales), 2% of the indices -1.  Outputs reach |out| ~ 0.5, so a shifted
    gather or a zero output fails the bars (tests/test_oracle.py checks that on the CPU)."""
    lens = [5000, 2100, 3000]
    q, kc, bt, ld = orc.make_dense_inputs(3, 128, 1, lens, seed=topk, scale=1.0, extra_blocks=2)
    if fp8:
        kc = orc.make_fp8_cache(kc.shape[0], seed=topk + 1, lat_scale=1.0)
    idx = orc.make_sparse_indices(3, 1, topk, lens, seed=topk + 2)
    return q, kc, bt, ld, idx


@pytest.mark.parametrize("fp8", [False, True])
@pytest.mark.parametrize("topk,parts", [(256, None), (2048, None), (100, 3), (2048, 1)])
def test_sparse_random(fp8, topk, parts):
    need_gpu()
    say(f"sparse random fp8={fp8} topk={topk} parts={parts}")
    q, kc, bt, ld, idx = sparse_random_inputs(fp8, topk)
    out, lse = run_sparse(q, kc, bt, ld, idx, SCALE, fp8, parts)
    assert_close(out, lse, *sparse_refs(q, kc, bt, ld, idx, SCALE, fp8))


@pytest.mark.parametrize("parts", [None, 1, 5])
def test_dense_segments_of_every_tile_count(parts):
    """Segments of 1..7 tiles of 32 tokens, full and one token into the next tile: every
    count modulo the three-buffer round (the steps after the last whole round request no
    tiles)."""
    need_gpu()
    lens = [1, 32, 33, 64, 65, 96, 97, 128, 129, 160, 161, 192, 193]
    say(f"dense tile counts parts={parts}")
    q, kc, bt, ld = orc.make_dense_inputs(len(lens), 128, 1, lens, seed=31, scale=1.0,
                                          extra_blocks=2)
    out, lse, _, _ = run_dense(q, kc, bt, ld, SCALE, False, parts)
    assert_close(out, lse, *dense_refs(q, kc, bt, ld, SCALE, False))


@pytest.mark.parametrize("fp8", [False, True])
@pytest.mark.parametrize("topk,parts", [(32, None), (64, 1), (96, None), (128, 1), (160, None),
                                        (160, 1)])
def test_sparse_segments_of_every_tile_count(fp8, topk, parts):
    """Sparse segments of 1..5 tiles (top-k 32..160): every count modulo the three-buffer
    round, with and without splits."""
    need_gpu()
    say(f"sparse tile counts fp8={fp8} topk={topk} parts={parts}")
    q, kc, bt, ld, idx = sparse_random_inputs(fp8, topk)
    out, lse = run_sparse(q, kc, bt, ld, idx, SCALE, fp8, parts)
    assert_close(out, lse, *sparse_refs(q, kc, bt, ld, idx, SCALE, fp8))


@pytest.mark.parametrize("fp8", [False, True])
@pytest.mark.parametrize("h_q,s_q,topk", [(100, 2, 300), (256, 1, 500), (16, 3, 64)])
def test_sparse_head_and_token_shapes(fp8, h_q, s_q, topk):
    """Head counts that are not a multiple of the 128-row work-group, several query
    tokens (each with its own top-k), and more than one head block per token."""
    need_gpu()
    say(f"sparse shapes fp8={fp8} h_q={h_q} s_q={s_q} topk={topk}")
    lens = [700, 1500]
    q, kc, bt, ld = orc.make_dense_inputs(2, h_q, s_q, lens, seed=h_q + topk, scale=1.0,
                                          extra_blocks=1)
    if fp8:
        kc = orc.make_fp8_cache(kc.shape[0], seed=topk + 7, lat_scale=1.0)
    idx = orc.make_sparse_indices(2, s_q, topk, lens, seed=topk + 3)
    out, lse = run_sparse(q, kc, bt, ld, idx, SCALE, fp8)
    assert_close(out, lse, *sparse_refs(q, kc, bt, ld, idx, SCALE, fp8))


@pytest.mark.parametrize("h_q,s_q,causal", [(256, 1, False), (128, 2, True), (64, 5, True)])
def test_dense_multi_row_block(h_q, s_q, causal):
    """More than 128 query rows per sequence: several row blocks per part."""
    need_gpu()
    say(f"dense row blocks h_q={h_q} s_q={s_q} causal={causal}")
    lens = [1000, 3000, 65]
    q, kc, bt, ld = orc.make_dense_inputs(3, h_q, s_q, lens, seed=h_q * s_q, scale=0.5)
    out, lse, _, _ = run_dense(q, kc, bt, ld, SCALE, causal)
    assert_close(out, lse, *dense_refs(q, kc, bt, ld, SCALE, causal))


@pytest.mark.parametrize("fp8", [False, True])
def test_sparse_valid_indices_past_the_cache_length(fp8):
    """A top-k list longer than the cache with its valid ids scattered over every slot:
    slot positions are not token positions, so slots at or past the cache length hold
    keys like any other (only -1 and ids >= the length are masked)."""
    need_gpu()
    lens = [100, 37]
    topk = 256
    q, kc, bt, ld = orc.make_dense_inputs(2, 128, 1, lens, seed=12, scale=1.0, extra_blocks=1)
    if fp8:
        kc = orc.make_fp8_cache(kc.shape[0], seed=13, lat_scale=1.0)
    gen = torch.Generator().manual_seed(14)
    idx = torch.full((2, 1, topk), -1, dtype=torch.int32)
    for b, n in enumerate(lens):
        slots = torch.randperm(topk, generator=gen)[:n]
        idx[b, 0, slots] = torch.randperm(n, generator=gen).to(torch.int32)
    idx[0, 0, 7] = 100  # == the cache length: masked
    assert int((idx[0, 0, lens[0]:] >= 0).sum()) > 30  # valid ids past slot len
    out, lse = run_sparse(q, kc, bt, ld, idx, SCALE, fp8)
    assert_close(out, lse, *sparse_refs(q, kc, bt, ld, idx, SCALE, fp8))


@pytest.mark.parametrize("fp8", [False, True])
def test_sparse_duplicate_ids(fp8):
    """Repeated ids count once per slot.  Row 0 lists one id in all 128 slots: its
    attention is that key's value exactly, with lse = its score + ln 128; row 1 repeats
    a few ids among distinct ones (checked against the oracle)."""
    need_gpu()
    lens = [300, 300]
    topk = 128
    q, kc, bt, ld = orc.make_dense_inputs(2, 64, 1, lens, seed=21, scale=1.0, extra_blocks=1)
    if fp8:
        kc = orc.make_fp8_cache(kc.shape[0], seed=22, lat_scale=1.0)
    idx = orc.make_sparse_indices(2, 1, topk, lens, seed=23, invalid_frac=0.0)
    idx[0] = 5
    idx[1, 0, 64:96] = idx[1, 0, :32]
    out, lse = run_sparse(q, kc, bt, ld, idx, SCALE, fp8)
    ref_out, ref_lse, low, low_lse = sparse_refs(q, kc, bt, ld, idx, SCALE, fp8)
    assert_close(out, lse, ref_out, ref_lse, low, low_lse)
    # closed form for row 0: the one key of id 5 (physical row through the table)
    row = int(bt[0, 0]) * 64 + 5
    flat = kc.reshape(-1, kc.shape[-1])
    kv = orc.fp8_rows_dequant(flat[row:row + 1]) if fp8 else flat[row:row + 1].float()
    kv = kv.to(torch.bfloat16).float()  # the MFMA input (fp8 rows become bf16 on chip)
    score = (q[0, 0].float() @ kv[0]) * SCALE
    torch.testing.assert_close(lse[0, :, 0], score + math.log(topk), atol=2e-2, rtol=0)
    torch.testing.assert_close(out[0, 0].float(), kv[0, :512].expand(64, 512), atol=2e-2,
                               rtol=1e-2)


def _padded_views(q, kc, bt, pad_row):
    """Views with non-default strides over the same values: q with its (s, h) axes
    stored transposed and padded rows, cache rows padded to pad_row elements, and the
    block table as a column slice of a wider table."""
    b, s_q, h_q, d = q.shape
    qb = torch.zeros((b, h_q, s_q, d + 64), dtype=q.dtype)
    qb[..., :d] = q.transpose(1, 2)
    qv = qb[..., :d].transpose(1, 2)
    kb = torch.zeros(kc.shape[:3] + (pad_row,), dtype=kc.dtype)
    kb[..., :kc.shape[3]] = kc
    kv = kb[..., :kc.shape[3]]
    tb = torch.full((bt.shape[0], bt.shape[1] + 5), -7, dtype=bt.dtype)
    tb[:, 2:2 + bt.shape[1]] = bt
    tv = tb[:, 2:2 + bt.shape[1]]
    assert not qv.is_contiguous() and not kv.is_contiguous() and not tv.is_contiguous()
    return qb, kb, tb, qv, kv, tv


def _dev_view(base, view):
    """The same view of base, on the GPU (strides kept)."""
    d = base.to(DEV)
    return torch.as_strided(d, view.shape, view.stride(), view.storage_offset())


@pytest.mark.parametrize("causal", [False, True])
def test_dense_strided_inputs(causal):
    need_gpu()
    lens = [900, 130, 2000]
    q, kc, bt, ld = orc.make_dense_inputs(3, 128, 2, lens, seed=41, scale=1.0, extra_blocks=2)
    qb, kb, tb, qv, kv, tv = _padded_views(q, kc, bt, 640)
    qd, kd, td = _dev_view(qb, qv), _dev_view(kb, kv), _dev_view(tb, tv)
    ldd = ld.to(DEV)
    md, ns = flag_attn.get_mla_metadata(ldd, 2 * 128, 1)
    out, lse = flag_attn.flash_mla_with_kvcache(qd, kd, td, ldd, 512, md, ns, SCALE, causal)
    torch.cuda.synchronize()
    assert_close(out.cpu(), lse.cpu(), *dense_refs(q, kc, bt, ld, SCALE, causal))


@pytest.mark.parametrize("fp8", [False, True])
def test_sparse_strided_inputs(fp8):
    need_gpu()
    lens = [1500, 800]
    q, kc, bt, ld = orc.make_dense_inputs(2, 128, 1, lens, seed=42, scale=1.0, extra_blocks=1)
    if fp8:
        kc = orc.make_fp8_cache(kc.shape[0], seed=43, lat_scale=1.0)
    idx = orc.make_sparse_indices(2, 1, 300, lens, seed=44)
    qb, kb, tb, qv, kv, tv = _padded_views(q, kc, bt, 672 if fp8 else 640)
    qd, kd, td = _dev_view(qb, qv), _dev_view(kb, kv), _dev_view(tb, tv)
    ldd = ld.to(DEV)
    md, ns = flag_attn.get_mla_metadata(ldd, 128, 1, num_heads_q=128, topk=300)
    out, lse = flag_attn.flash_mla_with_kvcache(qd, kd, td, ldd, 512, md, ns, SCALE, False,
                                                is_fp8_kvcache=fp8, indices=idx.to(DEV))
    torch.cuda.synchronize()
    assert_close(out.cpu(), lse.cpu(), *sparse_refs(q, kc, bt, ld, idx, SCALE, fp8))


def test_sparse_all_masked_row():
    need_gpu()
    q, kc, bt, ld = orc.make_dense_inputs(2, 64, 1, [300, 300], seed=4)
    idx = orc.make_sparse_indices(2, 1, 128, [300, 300], seed=5, invalid_frac=0.0)
    idx[1] = -1
    out, lse = run_sparse(q, kc, bt, ld, idx, SCALE)
    ref_out, ref_lse, low, _ = sparse_refs(q, kc, bt, ld, idx, SCALE)
    assert bool(torch.isneginf(lse[1]).all()) and bool((out[1] == 0).all())
    assert_close(out, lse, ref_out, ref_lse, low)


def test_fp8_codec_exhaustive():
    """Every e4m3 code through the kernel's dequantiser, in K (lse) and V (out).

    One valid key per query token makes P = 1, so out = bf16(code * scale) exactly and
    lse = k[d] * sm_scale for a one-hot query at dim d.
    """
    need_gpu()
    codes = torch.arange(256, dtype=torch.uint8)
    codes[0x7F] = 0
    codes[0xFF] = 0  # the two NaN codes are not data
    lat = torch.cat([codes, codes.flip(0)])
    scales = torch.tensor([1.0, 2.0, 0.5, 0.015625], dtype=torch.float32)
    rope = torch.linspace(-3, 3, 64).to(torch.bfloat16)
    row = torch.cat([lat, scales.view(torch.uint8), rope.view(torch.uint8)])
    kc = torch.zeros((2, 64, 1, 656), dtype=torch.uint8)
    kc[1, 5, 0] = row
    s_q, h_q = 5, 128
    q = torch.zeros((1, s_q, h_q, 576), dtype=torch.bfloat16)
    for s in range(s_q):
        for h in range(h_q):
            d = s * h_q + h
            if d < 576:
                q[0, s, h, d] = 1.0
    bt = torch.tensor([[0, 1]], dtype=torch.int32)
    lens = torch.tensor([128], dtype=torch.int32)
    idx = torch.full((1, s_q, 64), -1, dtype=torch.int32)
    idx[0, :, 17] = 64 + 5  # logical token 69 -> page 1 row 5
    out, lse = run_sparse(q, kc, bt, lens, idx, 1.0, fp8=True)
    dec = orc.fp8_rows_dequant(row.view(1, 656))[0]  # fp32 [576]
    want_v = dec[:512].to(torch.bfloat16)
    for s in range(s_q):
        for h in range(h_q):
            assert torch.equal(out[0, s, h], want_v), f"V dequant differs (s={s}, h={h})"
    for s in range(s_q):
        for h in range(h_q):
            d = s * h_q + h
            want = float(dec[d].to(torch.bfloat16)) if d < 576 else 0.0
            assert abs(float(lse[0, h, s]) - want) <= 1e-6 * max(1.0, abs(want)), (s, h, d)
