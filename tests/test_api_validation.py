"""Argument validation of the Python operators -- CPU only.

Every check runs before any device work, so these run without a GPU.  Errors are
MLAArgumentError, which is both a ValueError and (like the reference's ``assert``-based
checks, src/flag_attn/paged.py:45-46, split_kv.py:282-289) an AssertionError.
"""
import pytest
import torch

import flagattention_amd as fa
from flagattention_amd.mla import MLAArgumentError


def _dense(batch=2, s_q=1, h_q=16, nblk=4):
    q = torch.zeros((batch, s_q, h_q, 576), dtype=torch.bfloat16)
    kc = torch.zeros((nblk, 64, 1, 576), dtype=torch.bfloat16)
    bt = torch.zeros((batch, 2), dtype=torch.int32)
    lens = torch.full((batch,), 100, dtype=torch.int32)
    md = torch.zeros((8, 8), dtype=torch.int32)
    ns = torch.zeros((batch + 1,), dtype=torch.int32)
    return dict(q=q, k_cache=kc, block_table=bt, cache_seqlens=lens, head_dim_v=512,
                tile_scheduler_metadata=md, num_splits=ns)


def _call(**kw):
    return fa.flash_mla_with_kvcache(**kw)


def test_error_type_is_value_and_assertion_error():
    assert issubclass(MLAArgumentError, ValueError)
    assert issubclass(MLAArgumentError, AssertionError)


@pytest.mark.parametrize("mutate,msg", [
    (lambda a: a.update(q=a["q"].float()), "bfloat16"),
    (lambda a: a.update(q=torch.zeros((2, 1, 16, 512), dtype=torch.bfloat16)), "head dim"),
    (lambda a: a.update(head_dim_v=576), "head_dim_v"),
    (lambda a: a.update(k_cache=torch.zeros((4, 32, 1, 576), dtype=torch.bfloat16)), "block size"),
    (lambda a: a.update(k_cache=torch.zeros((4, 64, 2, 576), dtype=torch.bfloat16)), "KV head"),
    (lambda a: a.update(block_table=a["block_table"].long()), "block_table"),
    (lambda a: a.update(block_table=a["block_table"][:, :0]), "at least one column"),
    (lambda a: a.update(cache_seqlens=a["cache_seqlens"].long()), "cache_seqlens"),
    (lambda a: a.update(num_splits=torch.zeros((2,), dtype=torch.int32)), "num_splits"),
    (lambda a: a.update(tile_scheduler_metadata=torch.zeros((8, 4), dtype=torch.int32)),
     "tile_scheduler_metadata"),
    (lambda a: a.update(is_fp8_kvcache=True), "fp8"),
    (lambda a: a.update(causal=True, indices=torch.zeros((2, 1, 8), dtype=torch.int32)),
     "causal"),
    (lambda a: a.update(indices=torch.zeros((2, 2, 8), dtype=torch.int32)), "indices"),
    (lambda a: None, "CUDA"),  # valid shapes, but CPU tensors
])
def test_decode_rejects(mutate, msg):
    args = _dense()
    mutate(args)
    with pytest.raises(MLAArgumentError, match=msg):
        _call(**args)


def test_fp8_cache_row_size():
    args = _dense()
    args.update(is_fp8_kvcache=True, k_cache=torch.zeros((4, 64, 1, 576), dtype=torch.uint8),
                indices=torch.zeros((2, 1, 8), dtype=torch.int32))
    with pytest.raises(MLAArgumentError, match="656"):
        _call(**args)


@pytest.mark.parametrize("kw,msg", [
    (dict(cache_seqlens=torch.zeros(3, dtype=torch.int64), num_q_tokens_per_head_k=128,
          num_heads_k=1), "int32"),
    (dict(cache_seqlens=torch.zeros(3, dtype=torch.int32), num_q_tokens_per_head_k=128,
          num_heads_k=2), "one latent KV head"),
    (dict(cache_seqlens=torch.zeros((0,), dtype=torch.int32), num_q_tokens_per_head_k=128,
          num_heads_k=1), "batch"),
    (dict(cache_seqlens=torch.zeros(3, dtype=torch.int32), num_q_tokens_per_head_k=128,
          num_heads_k=1, topk=0), "topk"),
    (dict(cache_seqlens=torch.zeros(3, dtype=torch.int32), num_q_tokens_per_head_k=128,
          num_heads_k=1, topk=2048), "num_heads_q"),
    (dict(cache_seqlens=torch.zeros(3, dtype=torch.int32), num_q_tokens_per_head_k=128,
          num_heads_k=1), "CUDA"),
])
def test_metadata_rejects(kw, msg):
    with pytest.raises(MLAArgumentError, match=msg):
        fa.get_mla_metadata(**kw)


def test_parts_derivation():
    from flagattention_amd.mla import default_num_parts, num_m_blocks
    assert num_m_blocks(128) == 1 and num_m_blocks(16) == 1 and num_m_blocks(256) == 2
    assert num_m_blocks(256, 128, sparse=True) == 2 and num_m_blocks(200, 100, sparse=True) == 2
    assert num_m_blocks(200, 100) == 2 and num_m_blocks(32, 16, sparse=True) == 2
    assert default_num_parts(256, 128, 1) == 256
    assert default_num_parts(256, 256, 1) == 128
    assert default_num_parts(4, 1024, 1) == 1


@pytest.mark.parametrize("sig,indices", [
    ((2, 2048), None),                                   # sparse metadata, dense call
    ((2, 0), torch.zeros((2, 1, 8), dtype=torch.int32)),  # dense metadata, sparse call
    ((3, 0), None),                                      # metadata of another batch
])
def test_decode_rejects_metadata_of_another_call(sig, indices):
    """get_mla_metadata tags its tensors with (batch, topk); the decode checks the tag
    before anything else touches the device."""
    args = _dense()
    args["tile_scheduler_metadata"]._fa_mla_sig = sig
    args["num_splits"]._fa_mla_sig = sig
    args["indices"] = indices
    with pytest.raises(MLAArgumentError, match="scheduler metadata was built for"):
        _call(**args)


def test_flag_attn_namespace_exports_the_mla_operators():
    """The drop-in surface: ``import flag_attn`` gives the MLA operators with the
    FlashMLA-style signatures (src/flag_attn/__init__.py:23-29 is the export style)."""
    import inspect

    import flag_attn
    import flag_attn.mla

    assert flag_attn.get_mla_metadata is fa.get_mla_metadata
    assert flag_attn.flash_mla_with_kvcache is fa.flash_mla_with_kvcache
    md = inspect.signature(flag_attn.get_mla_metadata).parameters
    assert list(md)[:6] == ["cache_seqlens", "num_q_tokens_per_head_k", "num_heads_k",
                            "num_heads_q", "is_fp8_kvcache", "topk"]
    dec = inspect.signature(flag_attn.flash_mla_with_kvcache).parameters
    assert list(dec) == ["q", "k_cache", "block_table", "cache_seqlens", "head_dim_v",
                         "tile_scheduler_metadata", "num_splits", "softmax_scale", "causal",
                         "is_fp8_kvcache", "indices"]
    assert dec["indices"].default is None and dec["causal"].default is False


@pytest.mark.parametrize("kw,msg", [
    (dict(scores=torch.zeros(2, 1, 10, dtype=torch.float16)), "float32"),
    (dict(scores=torch.zeros(2, 10)), "float32"),
    (dict(scores=torch.zeros(2, 1, 65537)), "length"),
    (dict(topk=0), "topk"),
    (dict(topk=65537), "topk"),
    (dict(cache_seqlens=torch.zeros(3, dtype=torch.int32)), "cache_seqlens"),
    (dict(cache_seqlens=torch.zeros(2, dtype=torch.int64)), "cache_seqlens"),
    (dict(scores=torch.zeros(2, 1, 20)[:, :, ::2]), "contiguous"),
    (dict(out=torch.zeros(2, 1, 8, dtype=torch.int64)), "out"),
    (dict(), "CUDA"),
])
def test_topk_indices_rejects(kw, msg):
    args = dict(scores=torch.zeros(2, 1, 10), cache_seqlens=torch.zeros(2, dtype=torch.int32),
                topk=8)
    args.update(kw)
    with pytest.raises(MLAArgumentError, match=msg):
        fa.topk_indices(**args)
    import flag_attn
    assert flag_attn.topk_indices is fa.topk_indices
