"""Seeded random shapes for every operator, against the oracle.

The other GPU tests pick their shapes by hand (edge counts, the reference's sweeps, the
benchmark configs).  These draw them: case i uses ``random.Random(seed + i)``, so a failure
names its case and reruns exactly.  The draws cover what the hand-picked cases combine
less often:
- zero-length and shorter-than-``s_q`` sequences in one batch;
- head counts that are not multiples of 16 or 128;
- split counts from 1 to more than the batch's tiles;
- top-k sizes that are not multiples of the 32-token tile;
- odd page sizes with split starts off page boundaries;
- rows with tied scores.
The bars are those of the hand-picked tests: the north-star tolerances plus the reference's
three-way rule for floating point, bit-exact for indices and cache bytes.
"""
import random

import numpy as np
import pytest
import torch

import flag_attn
from oracle import gqa_oracle as go
from oracle import mla_oracle as orc
from oracle import topk_oracle as tko
from tests._helpers import (DEV, assert_close, dense_refs, need_gpu, run_dense, run_sparse, say,
                            sparse_refs)
from tests.test_gpu_gqa import _max_diff, _splitkv_inputs, base_paged_attention

pytestmark = pytest.mark.gpu
SCALE = 192 ** -0.5


def _lens(rng, batch, hi, s_q=1):
    """Lengths in [0, hi]: mostly uniform, with zero and shorter-than-s_q ones mixed in."""
    out = []
    for _ in range(batch):
        r = rng.random()
        out.append(0 if r < 0.1 else rng.randint(1, max(1, s_q)) if r < 0.2 else rng.randint(1, hi))
    if max(out) == 0:
        out[0] = rng.randint(1, hi)
    return out


@pytest.mark.parametrize("i", range(40))
def test_fuzz_mla_dense(i):
    need_gpu()
    rng = random.Random(5000 + i)
    batch = rng.randint(1, 7)
    h_q = rng.choice([1, 3, 16, 40, 64, 100, 128, 130, 200, 256, 300])
    s_q = rng.randint(1, 6)
    causal = rng.random() < 0.5
    parts = rng.choice([None, None, 1, rng.randint(2, 60)])
    lens = _lens(rng, batch, rng.choice([300, 2500, 9000]), s_q)
    say(f"fuzz dense {i}: B={batch} h_q={h_q} s_q={s_q} causal={causal} parts={parts} lens={lens}")
    q, kc, bt, ld = orc.make_dense_inputs(batch, h_q, s_q, lens, seed=6000 + i, scale=1.0,
                                          extra_blocks=rng.randint(0, 3))
    out, lse, _, _ = run_dense(q, kc, bt, ld, SCALE, causal, parts)
    assert_close(out, lse, *dense_refs(q, kc, bt, ld, SCALE, causal))


@pytest.mark.parametrize("i", range(30))
def test_fuzz_mla_sparse(i):
    need_gpu()
    rng = random.Random(7000 + i)
    fp8 = i % 2 == 1
    batch = rng.randint(1, 4)
    h_q = rng.choice([16, 64, 100, 128, 160])
    s_q = rng.randint(1, 3)
    topk = rng.choice([1, 17, 32, 64, 100, 333, 1024, 2048, 3000])
    parts = rng.choice([None, None, 1, rng.randint(2, 40)])
    lens = [rng.randint(1, rng.choice([500, 4000, 12000])) for _ in range(batch)]
    say(f"fuzz sparse {i}: fp8={fp8} B={batch} h_q={h_q} s_q={s_q} topk={topk} parts={parts} "
        f"lens={lens}")
    q, kc, bt, ld = orc.make_dense_inputs(batch, h_q, s_q, lens, seed=8000 + i, scale=1.0,
                                          extra_blocks=rng.randint(0, 2))
    if fp8:
        kc = orc.make_fp8_cache(kc.shape[0], seed=8100 + i, lat_scale=1.0)
    idx = orc.make_sparse_indices(batch, s_q, topk, lens, seed=8200 + i,
                                  invalid_frac=rng.choice([0.0, 0.02, 0.3]))
    out, lse = run_sparse(q, kc, bt, ld, idx, SCALE, fp8, parts)
    assert_close(out, lse, *sparse_refs(q, kc, bt, ld, idx, SCALE, fp8))


@pytest.mark.parametrize("i", range(30))
def test_fuzz_paged_attention(i):
    rng = random.Random(9000 + i)
    group = rng.choice([1, 2, 4, 8])
    h_kv = rng.choice([1, 2, 4])
    head_size = rng.choice([16, 32, 64, 128, 256, 512])
    block_size = rng.choice([16, 32, 64, 128] + ([8, 24] if group == 1 else [24, 48]))
    base_paged_attention(rng.randint(1, 6), group * h_kv, group, head_size, block_size,
                         rng.randint(2, 2000), rng.choice([0, 0, 1, 2, 3, 8]),
                         dtype=rng.choice([torch.float16, torch.bfloat16]), seed=9100 + i)


@pytest.mark.parametrize("i", range(20))
def test_fuzz_flash_attention_decode(i):
    need_gpu()
    rng = random.Random(9500 + i)
    h_kv = rng.choice([1, 2, 4])
    hq = h_kv * rng.choice([1, 2, 4])
    m = rng.choice([1, 1, 2, 4, 16])
    n = rng.randint(1, 3000)
    d = rng.choice([16, 32, 64, 128, 256, 512])
    causal = rng.random() < 0.5
    b = rng.randint(1, 3)
    say(f"fuzz flash_attention {i}: B={b} Hq={hq} Hk={h_kv} M={m} N={n} D={d} causal={causal}")
    q, k, v = _splitkv_inputs(b, hq, h_kv, m, n, d, torch.bfloat16, rng.choice(["BHTD", "BTHD"]),
                              1.0, 9600 + i)
    o_ref, lse_ref = go.flash_attention_ref(q, k, v, causal, upcast=True)
    o_low, _ = go.flash_attention_ref(q, k, v, causal, upcast=False)
    o, lse, *_ = flag_attn.flash_attention(q.to(DEV), k.to(DEV), v.to(DEV), causal,
                                           return_log_normalizer=True)
    o, lse = o.cpu(), lse.cpu()
    assert o.dtype == q.dtype and o.shape == q.shape
    assert _max_diff(o, o_ref) <= 2 * _max_diff(o_low, o_ref) + 1e-5
    fin = torch.isfinite(lse_ref)
    assert torch.equal(torch.isneginf(lse), torch.isneginf(lse_ref))
    if bool(fin.any()):
        assert torch.allclose(lse[fin], lse_ref[fin], atol=1e-3, rtol=1e-4)


@pytest.mark.parametrize("i", range(30))
def test_fuzz_topk(i):
    need_gpu()
    rng = random.Random(9800 + i)
    b, s_q = rng.randint(1, 6), rng.randint(1, 3)
    length = rng.choice([rng.randint(1, 3000), rng.randint(3000, 20000), rng.randint(20000, 65536)])
    topk = rng.choice([1, 7, 64, 512, 2048, rng.randint(1, min(length, 8192))])
    causal = rng.random() < 0.5
    gen = torch.Generator().manual_seed(9900 + i)
    if rng.random() < 0.3:  # integer scores: many ties
        scores = torch.randint(-20, 20, (b, s_q, length), generator=gen).float()
    else:
        scores = torch.randn((b, s_q, length), generator=gen)
    lens = [rng.randint(0, length) for _ in range(b)]
    say(f"fuzz topk {i}: B={b} s_q={s_q} len={length} topk={topk} causal={causal} lens={lens}")
    got = flag_attn.topk_indices(scores.to(DEV), torch.tensor(lens, dtype=torch.int32).to(DEV),
                                 topk, causal=causal).cpu().numpy()
    want = tko.topk_indices_ref(scores.numpy(), lens, topk, causal)
    bad = np.argwhere(got != want)
    assert bad.size == 0, f"{bad.shape[0]} mismatches, first at {bad[0].tolist()}"


@pytest.mark.parametrize("i", range(12))
def test_fuzz_kvcache_write(i):
    need_gpu()
    rng = random.Random(9950 + i)
    fp8 = i % 2 == 1
    nblk = rng.randint(1, 12)
    t = rng.randint(1, nblk * 64)
    gen = torch.Generator().manual_seed(9960 + i)
    row = 656 if fp8 else 576
    if fp8:
        cache = torch.randint(0, 256, (nblk, 64, 1, row), generator=gen, dtype=torch.uint8)
    else:
        cache = torch.randn((nblk, 64, 1, row), generator=gen).to(torch.bfloat16)
    lat = (torch.randn((t, 512), generator=gen) * rng.choice([1e-3, 1.0, 300.0])).to(torch.bfloat16)
    rope = torch.randn((t, 64), generator=gen).to(torch.bfloat16)
    slots = torch.randperm(nblk * 64, generator=gen)[:t].to(torch.int64)
    if t > 2:
        slots[rng.randrange(t)] = -1  # a padding token
    say(f"fuzz kvcache {i}: fp8={fp8} blocks={nblk} tokens={t}")
    want = orc.kvcache_write_ref(cache, lat, rope, slots, fp8)
    dc = cache.to(DEV)
    flag_attn.concat_and_cache_mla(lat.to(DEV), rope.to(DEV), dc, slots.to(DEV), fp8)
    got = dc.cpu()
    if fp8:
        assert torch.equal(got, want)
    else:
        assert torch.equal(got.view(torch.int16), want.view(torch.int16))
