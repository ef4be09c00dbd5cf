"""The allocation-free decode entry point (fa_mla_decode_noalloc) against the workspace path.

Same kernels, same scheduler metadata: the outputs must be bit-identical to
``flash_mla_with_kvcache``'s.  Two calls in a row, the second with a smaller input, check
that the shared scratch array carries nothing from one call into the next.
"""
import pytest
import torch

import flag_attn
from flagattention_amd import _lib
from flagattention_amd.mla import decode_noalloc
from oracle import mla_oracle as orc
from tests._helpers import DEV, need_gpu, say

pytestmark = pytest.mark.gpu
SCALE = 192 ** -0.5


def _both(q, kc, bt, lens, idx=None, fp8=False, causal=False):
    qd, kd, btd, ld = (t.to(DEV) for t in (q, kc, bt, lens))
    idd = None if idx is None else idx.to(DEV)
    b, s_q, h_q, _ = q.shape
    md, ns = flag_attn.get_mla_metadata(ld, s_q * h_q, 1, num_heads_q=h_q,
                                        topk=None if idx is None else idx.shape[2])
    ref_out, ref_lse = flag_attn.flash_mla_with_kvcache(qd, kd, btd, ld, 512, md, ns, SCALE,
                                                        causal, is_fp8_kvcache=fp8,
                                                        indices=idd)
    out = torch.full((b, s_q, h_q, 512), float("nan"), dtype=torch.bfloat16, device=DEV)
    lse = torch.full((b, h_q, s_q), float("nan"), dtype=torch.float32, device=DEV)
    decode_noalloc(out, lse, qd, kd, btd, ld, md, ns, SCALE, causal, fp8, idd)
    torch.cuda.synchronize()
    return out.cpu(), lse.cpu(), ref_out.cpu(), ref_lse.cpu()


def _assert_same(out, lse, ref_out, ref_lse):
    assert torch.equal(out.view(torch.int16), ref_out.view(torch.int16)), "out differs"
    assert torch.equal(lse.view(torch.int32), ref_lse.view(torch.int32)), "lse differs"


def test_noalloc_dense_two_calls():
    need_gpu()
    say("noalloc dense: large then small")
    q, kc, bt, ld = orc.make_dense_inputs(6, 128, 2, [1, 63, 700, 4097, 3000, 65], seed=70,
                                          scale=1.0)
    _assert_same(*_both(q, kc, bt, ld, causal=True))
    q, kc, bt, ld = orc.make_dense_inputs(2, 16, 1, [300, 129], seed=71, scale=1.0)
    _assert_same(*_both(q, kc, bt, ld))


@pytest.mark.parametrize("fp8", [False, True])
def test_noalloc_sparse_two_calls(fp8):
    need_gpu()
    say(f"noalloc sparse fp8={fp8}: large then small")
    lens = [5000, 2100, 3000]
    q, kc, bt, ld = orc.make_dense_inputs(3, 128, 1, lens, seed=72, scale=1.0, extra_blocks=2)
    if fp8:
        kc = orc.make_fp8_cache(kc.shape[0], seed=73, lat_scale=1.0)
    idx = orc.make_sparse_indices(3, 1, 2048, lens, seed=74)
    _assert_same(*_both(q, kc, bt, ld, idx, fp8))
    lens = [700]
    q, kc, bt, ld = orc.make_dense_inputs(1, 64, 2, lens, seed=75, scale=1.0)
    if fp8:
        kc = orc.make_fp8_cache(kc.shape[0], seed=76, lat_scale=1.0)
    idx = orc.make_sparse_indices(1, 2, 300, lens, seed=77)
    _assert_same(*_both(q, kc, bt, ld, idx, fp8))


def test_noalloc_rejects_oversized_workspace():
    """A shape whose split workspace exceeds the scratch array fails before any launch."""
    need_gpu()
    b, h_q = 4096, 128
    lens = torch.full((b,), 64, dtype=torch.int32, device=DEV)
    md, ns = flag_attn.get_mla_metadata(lens, h_q, 1, num_sm_parts=256)
    q = torch.zeros((b, 1, h_q, 576), dtype=torch.bfloat16, device=DEV)
    kc = torch.zeros((b, 64, 1, 576), dtype=torch.bfloat16, device=DEV)
    bt = torch.arange(b, dtype=torch.int32, device=DEV).view(b, 1)
    out = torch.empty((b, 1, h_q, 512), dtype=torch.bfloat16, device=DEV)
    lse = torch.empty((b, h_q, 1), dtype=torch.float32, device=DEV)
    assert _lib.load().fa_mla_noalloc_scratch_bytes is not None
    with pytest.raises(RuntimeError, match="more than the"):
        decode_noalloc(out, lse, q, kc, bt, lens, md, ns, SCALE)


@pytest.mark.parametrize("mode", ["dense", "sparse", "sparse_fp8"])
def test_noalloc_graph_capture_and_replay(mode):
    """decode_noalloc captured in a HIP graph (the caller it exists for): replays after the
    query and cache contents change in place, with eager work and synchronisations between
    the replays, each bit-identical to an eager flash_mla_with_kvcache on the new data."""
    need_gpu()
    say(f"noalloc graph replay: {mode}")
    lens = [3000, 1000, 4500]
    fp8 = mode == "sparse_fp8"
    q, kc, bt, ld = orc.make_dense_inputs(3, 128, 1, lens, seed=80, scale=1.0)
    if fp8:
        kc = orc.make_fp8_cache(kc.shape[0], seed=81, lat_scale=1.0)
    idx = orc.make_sparse_indices(3, 1, 1024, lens, seed=82) if mode != "dense" else None
    qd, kd, btd, ldd = (t.to(DEV) for t in (q, kc, bt, ld))
    idd = None if idx is None else idx.to(DEV)
    md, ns = flag_attn.get_mla_metadata(ldd, 128, 1, num_heads_q=128,
                                        topk=None if idx is None else idx.shape[2])
    out = torch.empty((3, 1, 128, 512), dtype=torch.bfloat16, device=DEV)
    lse = torch.empty((3, 128, 1), dtype=torch.float32, device=DEV)
    # first call eagerly: resolves the scratch array's device address outside the capture
    decode_noalloc(out, lse, qd, kd, btd, ldd, md, ns, SCALE, False, fp8, idd)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        decode_noalloc(out, lse, qd, kd, btd, ldd, md, ns, SCALE, False, fp8, idd)
    gen = torch.Generator(device=DEV).manual_seed(83)
    for rep in range(3):
        qd.copy_(torch.randn(qd.shape, generator=gen, device=DEV).to(qd.dtype))
        if fp8:
            kd.copy_(orc.make_fp8_cache(kc.shape[0], seed=90 + rep, lat_scale=1.0).to(DEV))
        else:
            kd.copy_(torch.randn(kd.shape, generator=gen, device=DEV).to(kd.dtype))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        ref_out, ref_lse = flag_attn.flash_mla_with_kvcache(qd, kd, btd, ldd, 512, md, ns, SCALE,
                                                            False, is_fp8_kvcache=fp8,
                                                            indices=idd)
        torch.cuda.synchronize()
        _assert_same(out.cpu(), lse.cpu(), ref_out.cpu(), ref_lse.cpu())
