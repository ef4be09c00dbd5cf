"""GPU parity of the grouped-query decode path (flag_attn.paged_attention,
flag_attn.flash_attention_split_kv, flag_attn.flash_attention) against the CPU oracle.

The sweeps are the reference's own: ``tests/flag_attn/test_paged_attention.py:79-157``
(fp16, uniform(+-D^-0.5) inputs, block tables drawn with replacement, ``allclose(atol=2e-3,
rtol=1e-5)`` against ``testing.paged_attention``) and
``tests/flag_attn/test_flash_attention.py:82-127`` (``test_attention_splitkv``: scale 10,
BHTD / BTHD strides, fp16 / bf16, causal or not, the rule
``max|hyp - ref| <= 2 max|torch_lowp - ref| + 1e-5``).  The paged sweeps apply that rule
too (against ``gqa_oracle.paged_attention_lowp``) beside the reference's ``allclose``.  Inputs are seeded here (the
reference's paged tests are not).  Caches are generated on the GPU; the oracle gets CPU
copies of the pages the block tables name.
"""
import pytest
import torch

import flag_attn
from oracle import gqa_oracle as go
from tests._helpers import DEV, assert_lowp_rule, need_gpu, say

pytestmark = pytest.mark.gpu
NUM_BLOCKS = 1000
CACHE_BYTES = 256 << 20  # per cache; fewer pages than NUM_BLOCKS when they are large


def base_paged_attention(num_seqs, num_query_heads, query_group_size, head_size, block_size,
                         max_seq_len, num_splits=0, dtype=torch.float16, seed=0):
    need_gpu()
    say(f"paged seqs={num_seqs} H={num_query_heads} g={query_group_size} D={head_size} "
        f"bs={block_size} len={max_seq_len} splits={num_splits} {dtype}")
    gen = torch.Generator().manual_seed(seed)
    dgen = torch.Generator(device=DEV).manual_seed(seed)
    num_kv_heads = num_query_heads // query_group_size
    context_lens = torch.randint(1, max_seq_len, (num_seqs,), generator=gen, dtype=torch.int32)
    context_lens[0] = max_seq_len
    max_context_len = int(context_lens.max())
    max_blocks = (max_context_len + block_size - 1) // block_size
    page_bytes = num_kv_heads * block_size * head_size * 2
    nblocks = max(64, min(NUM_BLOCKS, CACHE_BYTES // page_bytes))
    scale = head_size ** -0.5
    q = torch.empty((num_seqs, num_query_heads, head_size), device=DEV, dtype=dtype)
    q.uniform_(-scale, scale, generator=dgen)
    k_cache = torch.empty((nblocks, num_kv_heads, block_size, head_size), device=DEV, dtype=dtype)
    k_cache.uniform_(-scale, scale, generator=dgen)
    v_cache = torch.empty_like(k_cache).uniform_(-scale, scale, generator=dgen)
    block_tables = torch.randint(0, nblocks, (num_seqs, max_blocks), generator=gen,
                                 dtype=torch.int32)
    out = flag_attn.paged_attention(q, k_cache, v_cache, context_lens.to(DEV),
                                    block_tables.to(DEV), scale, max_context_len, num_splits)
    torch.cuda.synchronize()
    # oracle on the pages the tables name (remapped onto a compact pool)
    need = torch.unique(block_tables.flatten()).long()
    remap = torch.full((nblocks,), -1, dtype=torch.long)
    remap[need] = torch.arange(need.numel())
    kc = k_cache[need.to(DEV)].cpu()
    vc = v_cache[need.to(DEV)].cpu()
    bt = remap[block_tables.long()].to(torch.int32)
    ref = go.paged_attention_ref(q.cpu(), kc, vc, bt, context_lens, scale)
    err = float((out.cpu().float() - ref.float()).abs().max())
    say(f"  max |out - ref| = {err:.3e}")
    assert torch.allclose(out.cpu(), ref, atol=2e-3, rtol=1e-5)
    # the reference's allclose alone passes a kernel that drops a page at these output
    # sizes; the three-way rule against the fp32 result and the low-precision leg does not
    ref32 = go.paged_attention_ref(q.cpu(), kc, vc, bt, context_lens, scale, out_fp32=True)
    low = go.paged_attention_lowp(q.cpu(), kc, vc, bt, context_lens, scale)
    assert_lowp_rule(out.cpu(), ref32, low)


@pytest.mark.parametrize("num_seqs", [1, 32])
@pytest.mark.parametrize("num_query_heads", [64])
@pytest.mark.parametrize("query_group_size", [1, 8])
@pytest.mark.parametrize("head_size", [64, 128])
@pytest.mark.parametrize("block_size", [16, 128, 256])
@pytest.mark.parametrize("max_seq_len", [512, 4096])
def test_paged_attention_default(num_seqs, num_query_heads, query_group_size, head_size,
                                 block_size, max_seq_len):
    base_paged_attention(num_seqs, num_query_heads, query_group_size, head_size, block_size,
                         max_seq_len, seed=num_seqs * 7 + head_size + block_size + max_seq_len)


@pytest.mark.parametrize("num_seqs", [1, 16])
@pytest.mark.parametrize("num_query_heads", [64])
@pytest.mark.parametrize("query_group_size", [1, 8])
@pytest.mark.parametrize("head_size", [32, 64])
@pytest.mark.parametrize("block_size", [16])
@pytest.mark.parametrize("max_seq_len", [2048])
@pytest.mark.parametrize("num_splits", [1, 2, 3, 4, 5, 6, 7, 8])
def test_paged_attention_by_num_splits(num_seqs, num_query_heads, query_group_size, head_size,
                                       block_size, max_seq_len, num_splits):
    base_paged_attention(num_seqs, num_query_heads, query_group_size, head_size, block_size,
                         max_seq_len, num_splits, seed=num_splits * 13 + num_seqs + head_size)


@pytest.mark.parametrize("num_seqs, num_query_heads, query_group_size, head_size, block_size, "
                         "max_seq_len, num_splits", [
                             (1, 12, 1, 64, 16, 2, 0),
                             (16, 64, 8, 32, 16, 2048, 2),
                             (16, 64, 1, 64, 16, 2048, 6),
                         ])
def test_paged_attention_by_case(num_seqs, num_query_heads, query_group_size, head_size,
                                 block_size, max_seq_len, num_splits):
    base_paged_attention(num_seqs, num_query_heads, query_group_size, head_size, block_size,
                         max_seq_len, num_splits, seed=5)


@pytest.mark.parametrize("head_size,group,dtype", [
    (16, 4, torch.float16), (256, 2, torch.float16), (128, 8, torch.bfloat16),
    (256, 1, torch.bfloat16), (32, 16, torch.bfloat16),
])
@pytest.mark.parametrize("num_splits", [0, 3])
def test_paged_attention_more_shapes(head_size, group, dtype, num_splits):
    """Head dims 16 and 256, bf16, and query groups beyond the reference's sweep (16 rows
    per work-group at group 16)."""
    base_paged_attention(8, 32, group, head_size, 16, 1500, num_splits, dtype=dtype,
                         seed=head_size + group)


@pytest.mark.parametrize("d", [64, 512])
def test_paged_attention_bad_page_is_masked(d):
    """A block-table entry outside the cache reads as a masked key instead of faulting."""
    need_gpu()
    gen = torch.Generator().manual_seed(3)
    h, bs = 8, 16
    kc = torch.randn((10, h, bs, d), generator=gen).half()
    vc = torch.randn((10, h, bs, d), generator=gen).half()
    q = torch.randn((1, h, d), generator=gen).half()
    bt = torch.tensor([[0, 1000, 2]], dtype=torch.int32)
    lens = torch.tensor([48], dtype=torch.int32)
    out = flag_attn.paged_attention(q.to(DEV), kc.to(DEV), vc.to(DEV), lens.to(DEV), bt.to(DEV),
                                    d ** -0.5, 48, 1)
    keep = torch.tensor([[0, 2]], dtype=torch.int32)  # the same keys without the bad page
    ref_lens = torch.tensor([32], dtype=torch.int32)
    ref = go.paged_attention_ref(q, kc, vc, keep, ref_lens, d ** -0.5)
    assert torch.allclose(out.cpu(), ref, atol=2e-3, rtol=1e-5)


SPLITKV_SHAPES = [
    (2, 4, 4, 1, 612, 128), (2, 4, 4, 1, 1034, 64), (2, 4, 4, 1, 2048, 32),
    (2, 4, 4, 1, 4096, 16), (2, 4, 4, 1, 4001, 32), (2, 4, 4, 1, 4096, 64),
    (2, 4, 4, 2, 4000, 128), (1, 2, 2, 4, 8202, 16), (1, 2, 2, 1, 8192, 32),
    (2, 4, 2, 1, 612, 128), (2, 4, 1, 1, 1034, 64), (2, 4, 2, 1, 2048, 32),
    (2, 4, 1, 1, 4096, 16), (2, 4, 2, 1, 4001, 32), (2, 4, 1, 1, 4096, 64),
    (2, 4, 2, 2, 4000, 128), (1, 2, 1, 4, 8202, 16), (1, 2, 1, 1, 8192, 32),
]


def _splitkv_inputs(B, Hq, Hk, M, N, D, dtype, stride_order, scale, seed):
    gen = torch.Generator().manual_seed(seed)
    if stride_order == "BHTD":
        q = torch.empty((B, Hq, M, D)).normal_(0.0, scale, generator=gen)
        k = torch.empty((B, Hk, N, D)).normal_(0.0, scale, generator=gen)
        v = torch.empty((B, Hk, N, D)).normal_(0.0, scale, generator=gen)
        return q.to(dtype), k.to(dtype), v.to(dtype)
    q = torch.empty((B, M, Hq, D)).normal_(0.0, scale, generator=gen).transpose(1, 2)
    k = torch.empty((B, N, Hk, D)).normal_(0.0, scale, generator=gen).transpose(1, 2)
    v = torch.empty((B, N, Hk, D)).normal_(0.0, scale, generator=gen).transpose(1, 2)
    return q.to(dtype), k.to(dtype), v.to(dtype)


def _max_diff(a, b):
    return float((a.float() - b.float()).abs().max())


@pytest.mark.parametrize("scale", [10.0])
@pytest.mark.parametrize("B, Hq, Hk, M, N, D", SPLITKV_SHAPES)
@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("stride_order", ["BHTD", "BTHD"])
def test_attention_splitkv(B, Hq, Hk, M, N, D, causal, stride_order, dtype, scale):
    need_gpu()
    q, k, v = _splitkv_inputs(B, Hq, Hk, M, N, D, dtype, stride_order, scale, 10086 + N + M)
    o_ref, _ = go.flash_attention_ref(q, k, v, causal, upcast=True)
    o_torch, _ = go.flash_attention_ref(q, k, v, causal, upcast=False)
    # the reference test calls flash_attention, which takes its split-KV path at these shapes
    o_hyp = flag_attn.flash_attention(q.to(DEV), k.to(DEV), v.to(DEV), causal).cpu()
    torch_max_diff = _max_diff(o_torch, o_ref)
    hyp_max_diff = _max_diff(o_hyp, o_ref)
    assert o_hyp.dtype == dtype and o_hyp.shape == q.shape
    assert hyp_max_diff <= 2 * torch_max_diff + 1e-5, (hyp_max_diff, torch_max_diff)


@pytest.mark.parametrize("B, Hq, Hk, M, N, D", SPLITKV_SHAPES[::3])
@pytest.mark.parametrize("causal", [True, False])
def test_flash_attention_split_kv_and_lse(B, Hq, Hk, M, N, D, causal):
    """flash_attention_split_kv gives the same o; flash_attention's log normaliser matches
    the oracle's logsumexp."""
    need_gpu()
    q, k, v = _splitkv_inputs(B, Hq, Hk, M, N, D, torch.bfloat16, "BHTD", 1.0, N)
    o_ref, lse_ref = go.flash_attention_ref(q, k, v, causal, upcast=True)
    o_torch, _ = go.flash_attention_ref(q, k, v, causal, upcast=False)
    o1 = flag_attn.flash_attention_split_kv(q.to(DEV), k.to(DEV), v.to(DEV), causal).cpu()
    o2, lse, tot, seed, off = flag_attn.flash_attention(q.to(DEV), k.to(DEV), v.to(DEV), causal,
                                                        return_log_normalizer=True)
    assert tot is None and seed is None and off is None
    assert torch.equal(o1, o2.cpu())
    assert _max_diff(o1, o_ref) <= 2 * _max_diff(o_torch, o_ref) + 1e-5
    assert lse.shape == (B, Hq, M) and lse.dtype == torch.float32
    assert torch.allclose(lse.cpu(), lse_ref, atol=1e-3, rtol=1e-4)


@pytest.mark.parametrize("block_size,group,num_splits", [
    (8, 1, 0), (8, 1, 3), (24, 1, 3), (24, 4, 0), (48, 8, 5), (48, 2, 1),
])
def test_paged_attention_odd_block_sizes(block_size, group, num_splits):
    """Pages below 16 tokens (the reference allows them at query group 1, paged.py:46) and
    page sizes that are not powers of two (the kernel divides instead of shifting, and looks
    pages up per lane), with split starts (next_pow2 partitions) that do not fall on page
    boundaries."""
    base_paged_attention(8, 16, group, 64, block_size, 1500, num_splits,
                         seed=block_size * 10 + group + num_splits)


def _oracle_chunked(q, k, v, causal, upcast, chunk=4):
    """flash_attention_ref over batch slices (the GQA repeat of a whole batch would not fit
    in host memory at these shapes)."""
    outs, lses = [], []
    for b0 in range(0, q.shape[0], chunk):
        o, lse = go.flash_attention_ref(q[b0:b0 + chunk], k[b0:b0 + chunk], v[b0:b0 + chunk],
                                        causal, upcast=upcast)
        outs.append(o)
        lses.append(lse)
    return torch.cat(outs), torch.cat(lses)


@pytest.mark.parametrize("B, Hq, Hk, M, N, D, causal", [
    (64, 32, 8, 1, 2048, 128, False),
    (32, 64, 64, 2, 1500, 64, True),
])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("stride_order", ["BHTD", "BTHD"])
def test_unsplit_contiguous_decode(B, Hq, Hk, M, N, D, causal, dtype, stride_order):
    """Shapes with enough (sequence, KV head, row block) work-groups to fill the GPU take no
    split: the decode kernel writes out and lse itself (no combine).  These are the shapes
    for which the reference's flash_attention takes its _fwd_kernel branch and returns L
    (flash.py:78-101, split_kv.py:249-251)."""
    from flagattention_amd import gqa
    need_gpu()
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    assert gqa.choose_splits(B, Hk, (Hq // Hk) * M, N, cus) == 1
    q, k, v = _splitkv_inputs(B, Hq, Hk, M, N, D, dtype, stride_order, 1.0, N + M)
    o_ref, lse_ref = _oracle_chunked(q, k, v, causal, True)
    o_low, _ = _oracle_chunked(q, k, v, causal, False)
    o1, lse, _, _, _ = flag_attn.flash_attention(q.to(DEV), k.to(DEV), v.to(DEV), causal,
                                                 return_log_normalizer=True)
    o2 = flag_attn.flash_attention_split_kv(q.to(DEV), k.to(DEV), v.to(DEV), causal)
    torch.cuda.synchronize()
    assert o1.dtype == dtype and o1.shape == q.shape
    assert torch.equal(o1.cpu(), o2.cpu())
    assert_lowp_rule(o1.cpu(), o_ref, o_low)
    assert lse.shape == (B, Hq, M) and lse.dtype == torch.float32
    assert float((lse.cpu() - lse_ref).abs().max()) <= 1e-3


@pytest.mark.parametrize("M, N, causal", [
    (16, 300, False), (64, 700, True), (200, 1000, True), (40, 24, True), (33, 33, True),
    (17, 5, False),
])
def test_flash_attention_many_queries(M, N, causal):
    """flash_attention with more query positions than a decode step (the reference's
    forward takes any M, flash.py:269-300): rows of 16 (head, position) pairs per
    work-group.  Causal with M > N leaves the first M - N positions no key: out 0,
    lse -inf (the LARGER_M convention of split_kv.py:161-164, flash.py's _fwd_kernel)."""
    need_gpu()
    q, k, v = _splitkv_inputs(2, 4, 2, M, N, 64, torch.float16, "BHTD", 1.0, M * 1000 + N)
    o_ref, lse_ref = go.flash_attention_ref(q, k, v, causal, upcast=True)
    o_low, _ = go.flash_attention_ref(q, k, v, causal, upcast=False)
    o, lse, _, _, _ = flag_attn.flash_attention(q.to(DEV), k.to(DEV), v.to(DEV), causal,
                                                return_log_normalizer=True)
    torch.cuda.synchronize()
    o, lse = o.cpu(), lse.cpu()
    assert bool(torch.isfinite(o).all())
    assert_lowp_rule(o, o_ref, o_low)
    assert torch.equal(torch.isneginf(lse), torch.isneginf(lse_ref))
    fin = ~torch.isneginf(lse_ref)
    assert float((lse[fin] - lse_ref[fin]).abs().max()) <= 1e-3
    if causal and M > N:
        assert float(o[:, :, : M - N].abs().max()) == 0.0


@pytest.mark.parametrize("num_seqs", [1, 8])
@pytest.mark.parametrize("query_group_size", [1, 8])
@pytest.mark.parametrize("block_size", [16, 128])
@pytest.mark.parametrize("max_seq_len", [512, 2048])
def test_paged_attention_head_size_512(num_seqs, query_group_size, block_size, max_seq_len):
    """head_size 512, which the reference's paged_attention accepts (paged.py:45): the
    reference sweep's inputs at that head size (the dims-split kernel)."""
    base_paged_attention(num_seqs, 64, query_group_size, 512, block_size, max_seq_len,
                         seed=num_seqs + query_group_size + block_size + max_seq_len)


@pytest.mark.parametrize("num_splits,dtype,block_size", [
    (1, torch.float16, 16), (3, torch.float16, 16), (8, torch.bfloat16, 16),
    (0, torch.bfloat16, 24), (5, torch.float16, 8),
])
def test_paged_attention_head_size_512_splits(num_splits, dtype, block_size):
    base_paged_attention(4, 16, 1 if block_size < 16 else 4, 512, block_size, 1500, num_splits,
                         dtype=dtype, seed=num_splits + block_size)


@pytest.mark.parametrize("M, N, causal", [(1, 3000, False), (3, 700, True)])
def test_flash_attention_head_size_512(M, N, causal):
    """The contiguous decode at head dim 512 (beyond the reference's flash_attention, which
    stops at 128): split and unsplit shapes through the dims-split kernel."""
    need_gpu()
    for B, Hq, Hk in ((2, 4, 2), (64, 16, 4)):
        q, k, v = _splitkv_inputs(B, Hq, Hk, M, N, 512, torch.bfloat16, "BTHD", 1.0, N + B)
        o_ref, lse_ref = _oracle_chunked(q, k, v, causal, True)
        o_low, _ = _oracle_chunked(q, k, v, causal, False)
        o, lse, _, _, _ = flag_attn.flash_attention(q.to(DEV), k.to(DEV), v.to(DEV), causal,
                                                    return_log_normalizer=True)
        torch.cuda.synchronize()
        assert_lowp_rule(o.cpu(), o_ref, o_low)
        assert float((lse.cpu() - lse_ref).abs().max()) <= 1e-3


@pytest.mark.parametrize("N", [1, 31, 32, 33, 64, 65, 96, 97, 128])
def test_flash_attention_head_size_512_few_tiles(N):
    """One to four 32-token tiles per work-group at head dim 512: the dims-split loop
    requests K two tiles ahead and V one, so these are its pipeline's start and end cases
    (no next tile, a next tile without the one after it)."""
    need_gpu()
    q, k, v = _splitkv_inputs(3, 8, 2, 1, N, 512, torch.float16, "BHTD", 1.0, 700 + N)
    o_ref, lse_ref = _oracle_chunked(q, k, v, False, True)
    o_low, _ = _oracle_chunked(q, k, v, False, False)
    o, lse, _, _, _ = flag_attn.flash_attention(q.to(DEV), k.to(DEV), v.to(DEV), False,
                                                return_log_normalizer=True)
    torch.cuda.synchronize()
    assert_lowp_rule(o.cpu(), o_ref, o_low)
    assert float((lse.cpu() - lse_ref).abs().max()) <= 1e-3


@pytest.mark.parametrize("head_size", [64, 512])
def test_paged_attention_split_longer_than_lds_table(head_size):
    """A split of more than 2,048 pages (8-token pages, one split over 20,000 tokens): the
    split's block-table slice does not fit in LDS and the pages are looked up in global
    memory (the other loop of both kernels)."""
    base_paged_attention(2, 4, 1, head_size, 8, 20000, 1, seed=head_size)
