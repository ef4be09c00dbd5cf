"""Every operator captured in a HIP graph (``torch.cuda.graph``) and replayed.

A serving loop captures its decode step once and replays it, so that no launch, allocation
or host synchronisation happens per step.  The operators make no host synchronisation, the
C-ABI allocates nothing (outputs and workspaces are torch tensors: inside a capture they
come from the graph's pool), and no memset node is recorded.  Each test captures one call,
then three times changes the inputs in place, replays, runs eager work of its own, and
compares the replay's outputs bit for bit with an eager call on the same inputs (the
workspace path of ``flash_mla_with_kvcache``, the split-KV combines of the GQA operators, the
two-stage top-k with its workspace, the cache writer).
"""
import pytest
import torch

import flag_attn
from oracle import mla_oracle as orc
from tests._helpers import DEV, need_gpu, say

pytestmark = pytest.mark.gpu
SCALE = 192 ** -0.5


def _same(a, b, what):
    a, b = a.cpu(), b.cpu()
    assert a.shape == b.shape and a.dtype == b.dtype, what
    if a.dtype in (torch.bfloat16, torch.float16):
        a, b = a.view(torch.int16), b.view(torch.int16)
    elif a.dtype == torch.float32:
        a, b = a.view(torch.int32), b.view(torch.int32)
    assert torch.equal(a, b), f"{what}: replay differs from the eager call"


def _capture_and_replay(eager, update, names):
    """eager() -> tuple of output tensors; update(rep) changes the inputs in place."""
    eager()  # library load and per-device set-up happen outside the capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = eager()
    for rep in range(3):
        update(rep)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        got = [o.clone() for o in outs]
        torch.randn(4096, device=DEV).sum().item()  # eager work between replays
        want = eager()
        torch.cuda.synchronize()
        for g, w, name in zip(got, want, names):
            _same(g, w, f"{name}, replay {rep}")


@pytest.mark.parametrize("mode", ["dense", "sparse", "sparse_fp8"])
def test_graph_mla_decode_step(mode):
    """get_mla_metadata + flash_mla_with_kvcache in one graph; the replays see new queries,
    new cache contents and (dense) new sequence lengths, so the captured metadata kernel
    recomputes the split plan."""
    need_gpu()
    say(f"graph: MLA decode step {mode}")
    lens = [3000, 700, 4500, 64]
    fp8 = mode == "sparse_fp8"
    q, kc, bt, ld = orc.make_dense_inputs(4, 128, 1, lens, seed=120, scale=1.0, extra_blocks=2)
    if fp8:
        kc = orc.make_fp8_cache(kc.shape[0], seed=121, lat_scale=1.0)
    idx = orc.make_sparse_indices(4, 1, 1024, lens, seed=122) if mode != "dense" else None
    qd, kd, btd, ldd = (t.to(DEV) for t in (q, kc, bt, ld))
    idd = None if idx is None else idx.to(DEV)
    topk = None if idx is None else idx.shape[2]
    gen = torch.Generator(device=DEV).manual_seed(123)

    def eager():
        md, ns = flag_attn.get_mla_metadata(ldd, 128, 1, num_heads_q=128, topk=topk)
        return flag_attn.flash_mla_with_kvcache(qd, kd, btd, ldd, 512, md, ns, SCALE, False,
                                                is_fp8_kvcache=fp8, indices=idd)

    def update(rep):
        qd.copy_(torch.randn(qd.shape, generator=gen, device=DEV).to(qd.dtype))
        if fp8:
            kd.copy_(orc.make_fp8_cache(kc.shape[0], seed=130 + rep, lat_scale=1.0).to(DEV))
        else:
            kd.copy_(torch.randn(kd.shape, generator=gen, device=DEV).to(kd.dtype))
        if mode == "dense":  # new lengths within the block table's pages
            new = torch.tensor([[2000, 4500, 64, 3900], [1, 1, 1, 4544],
                                [4544, 3000, 1500, 700]][rep], dtype=torch.int32)
            ldd.copy_(new.to(DEV))
        else:
            idd.copy_(orc.make_sparse_indices(4, 1, 1024, lens, seed=140 + rep).to(DEV))

    _capture_and_replay(eager, update, ["out", "lse"])


@pytest.mark.parametrize("num_splits", [0, 1, 4])
def test_graph_paged_attention(num_splits):
    need_gpu()
    say(f"graph: paged_attention num_splits={num_splits}")
    gen = torch.Generator(device=DEV).manual_seed(150)
    b, h_q, h_kv, d, bs, nblk = 6, 32, 8, 128, 16, 400
    lens = torch.tensor([1000, 17, 3000, 2048, 1, 777], dtype=torch.int32, device=DEV)
    bt = torch.randint(0, nblk, (b, 3000 // bs + 1), generator=gen, device=DEV,
                       dtype=torch.int32)
    q = torch.randn((b, h_q, d), generator=gen, device=DEV).half()
    kc = torch.randn((nblk, h_kv, bs, d), generator=gen, device=DEV).half()
    vc = torch.randn((nblk, h_kv, bs, d), generator=gen, device=DEV).half()

    def eager():
        return (flag_attn.paged_attention(q, kc, vc, lens, bt, d ** -0.5, 3000, num_splits),)

    def update(rep):
        q.copy_(torch.randn(q.shape, generator=gen, device=DEV).half())
        kc.copy_(torch.randn(kc.shape, generator=gen, device=DEV).half())
        vc.copy_(torch.randn(vc.shape, generator=gen, device=DEV).half())

    _capture_and_replay(eager, update, ["out"])


@pytest.mark.parametrize("return_lse", [False, True])
def test_graph_flash_attention_decode(return_lse):
    need_gpu()
    say(f"graph: flash_attention decode, lse={return_lse}")
    gen = torch.Generator(device=DEV).manual_seed(160)
    q = torch.randn((2, 16, 1, 64), generator=gen, device=DEV).bfloat16()
    k = torch.randn((2, 4, 5000, 64), generator=gen, device=DEV).bfloat16()
    v = torch.randn((2, 4, 5000, 64), generator=gen, device=DEV).bfloat16()

    def eager():
        if return_lse:
            o, lse, *_ = flag_attn.flash_attention(q, k, v, causal=True,
                                                   return_log_normalizer=True)
            return o, lse
        return (flag_attn.flash_attention_split_kv(q, k, v, causal=False),)

    def update(rep):
        for t in (q, k, v):
            t.copy_(torch.randn(t.shape, generator=gen, device=DEV).bfloat16())

    _capture_and_replay(eager, update, ["out", "lse"])


def test_graph_topk_two_stage():
    need_gpu()
    say("graph: topk_indices, two stages (workspace allocated in the capture)")
    gen = torch.Generator(device=DEV).manual_seed(170)
    scores = torch.randn((4, 2, 65536), generator=gen, device=DEV)
    lens = torch.tensor([65536, 40000, 3000, 65536], dtype=torch.int32, device=DEV)

    def eager():
        return (flag_attn.topk_indices(scores, lens, 2048, causal=True),)

    def update(rep):
        scores.copy_(torch.randn(scores.shape, generator=gen, device=DEV))

    _capture_and_replay(eager, update, ["indices"])


@pytest.mark.parametrize("fp8", [False, True])
def test_graph_kvcache_write(fp8):
    """The cache writer updates its cache in place: before each replay the captured cache
    is reset (eagerly, outside the graph) to the contents an eager call starts from."""
    need_gpu()
    say(f"graph: concat_and_cache_mla fp8={fp8}")
    gen = torch.Generator(device=DEV).manual_seed(180)
    nblk, t = 16, 500
    row = 656 if fp8 else 576
    if fp8:
        base = torch.randint(0, 256, (nblk, 64, 1, row), generator=gen, device=DEV,
                             dtype=torch.uint8)
    else:
        base = torch.randn((nblk, 64, 1, row), generator=gen, device=DEV).bfloat16()
    cache = base.clone()
    lat = torch.randn((t, 512), generator=gen, device=DEV).bfloat16()
    rope = torch.randn((t, 64), generator=gen, device=DEV).bfloat16()
    slots = torch.randperm(nblk * 64, generator=gen, device=DEV)[:t].to(torch.int64)
    flag_attn.concat_and_cache_mla(lat, rope, cache, slots, fp8)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        flag_attn.concat_and_cache_mla(lat, rope, cache, slots, fp8)
    for rp in range(3):
        lat.copy_(torch.randn(lat.shape, generator=gen, device=DEV).bfloat16())
        rope.copy_(torch.randn(rope.shape, generator=gen, device=DEV).bfloat16())
        cache.copy_(base)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        torch.randn(4096, device=DEV).sum().item()
        want = base.clone()
        flag_attn.concat_and_cache_mla(lat, rope, want, slots, fp8)
        torch.cuda.synchronize()
        _same(cache, want, f"cache, replay {rp}")
