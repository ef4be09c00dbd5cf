"""GPU parity of the MLA cache write path (flag_attn.concat_and_cache_mla) -- bit-exact
against the oracle's writer (oracle.kvcache_write_ref), and a write -> decode round trip."""
import pytest
import torch

import flag_attn
from oracle import mla_oracle as orc
from tests._helpers import DEV, assert_close, need_gpu, run_sparse, say, sparse_refs

pytestmark = pytest.mark.gpu
SCALE = 192 ** -0.5


def _tokens(t, seed, scale=1.0):
    gen = torch.Generator().manual_seed(seed)
    lat = (torch.randn((t, 512), generator=gen) * scale).to(torch.bfloat16)
    rope = (torch.randn((t, 64), generator=gen) * scale).to(torch.bfloat16)
    return lat, rope


def _edge_tokens():
    """Tiles that pin the rounding: scale 1 (amax 448) with values at e4m3 midpoints
    (ties round to the even code), subnormal codes and their midpoints, negative values,
    an all-zero tile and a tile with one non-zero value."""
    lat = torch.zeros((3, 512))
    ties = torch.tensor([448.0, 1.0625, 1.1875, -1.0625, 0.0029296875, 0.0009765625,
                         -0.0029296875, 0.001953125, 3.25, 13.0, 26.0, -208.0, 224.0, 0.5625])
    lat[0, :ties.numel()] = ties
    lat[0, 128] = 1.0
    lat[0, 256:384] = torch.linspace(-3.0, 3.0, 128)
    lat[1, 5] = -7.5
    lat[2] = torch.linspace(-1e-3, 2e-3, 512)
    rope = torch.linspace(-2, 2, 3 * 64).view(3, 64)
    return lat.to(torch.bfloat16), rope.to(torch.bfloat16)


@pytest.mark.parametrize("fp8", [False, True])
def test_kvcache_write_bit_exact(fp8):
    need_gpu()
    say(f"kvcache write fp8={fp8}")
    nblk, t = 20, 700
    gen = torch.Generator().manual_seed(31)
    row = 656 if fp8 else 576
    if fp8:
        cache = torch.randint(0, 256, (nblk, 64, 1, row), generator=gen, dtype=torch.uint8)
        cache[..., 512:528] = 0  # keep the untouched rows' scales finite
    else:
        cache = torch.randn((nblk, 64, 1, row), generator=gen).to(torch.bfloat16)
    lat, rope = _tokens(t, 32)
    el, er = _edge_tokens()
    lat = torch.cat([el, lat])
    rope = torch.cat([er, rope])
    slots = torch.randperm(nblk * 64, generator=gen)[: lat.shape[0]].to(torch.int64)
    slots[7] = -1                 # a padding token
    slots[11] = nblk * 64 + 5     # a slot past the cache
    want = orc.kvcache_write_ref(cache, lat, rope, slots, fp8)
    dc = cache.to(DEV)
    flag_attn.concat_and_cache_mla(lat.to(DEV), rope.to(DEV), dc, slots.to(DEV), fp8)
    torch.cuda.synchronize()
    got = dc.cpu()
    if fp8:
        assert torch.equal(got, want)
    else:
        assert torch.equal(got.view(torch.int16), want.view(torch.int16))


def test_kvcache_write_fp8_ieee_specials():
    """NaN and infinities in the latent vectors: the writer follows the same arithmetic as the
    oracle (a NaN makes its tile's amax NaN and the scale 1; an infinity makes the scale
    infinite, finite values zeros and infinite ones NaN).  Scales and every non-NaN byte
    are bit-exact; a NaN code may carry either sign (0x7F / 0xFF), as NaN signs are a
    platform detail of the CPU oracle."""
    need_gpu()
    say("kvcache write fp8 specials")
    nan, inf = float("nan"), float("inf")
    lat, rope = _tokens(6, 45)
    lat = lat.float()
    lat[0, 3] = nan                      # tile 0: one NaN among normal values
    lat[1, 130] = inf                    # tile 1: +inf
    lat[1, 140] = -inf                   # (same tile) -inf
    lat[2, 300] = -inf                   # tile 2: -inf alone
    lat[3, 400], lat[3, 401] = nan, inf  # tile 3: NaN and +inf together
    lat[4, :128] = nan                   # tile 0 all NaN
    lat[4, 128:256] = 0.0                # an all-zero tile next to it
    lat = lat.to(torch.bfloat16)
    cache = torch.zeros((1, 64, 1, 656), dtype=torch.uint8)
    slots = torch.arange(6, dtype=torch.int64) * 3
    want = orc.kvcache_write_ref(cache, lat, rope, slots, True)
    dc = cache.to(DEV)
    flag_attn.concat_and_cache_mla(lat.to(DEV), rope.to(DEV), dc, slots.to(DEV), True)
    torch.cuda.synchronize()
    got = dc.cpu().view(64, 656)
    want = want.view(64, 656)
    assert torch.equal(got[:, 512:], want[:, 512:])  # scales and rope bytes
    w_nan = (want[:, :512] & 0x7F) == 0x7F
    g_nan = (got[:, :512] & 0x7F) == 0x7F
    assert torch.equal(w_nan, g_nan)
    assert int(w_nan.sum()) >= 128 + 4  # the NaN inputs and inf / inf
    assert torch.equal(got[:, :512][~w_nan], want[:, :512][~w_nan])


def test_kvcache_write_int32_slots_and_strided_inputs():
    need_gpu()
    lat, rope = _tokens(64, 40)
    both = torch.cat([lat, rope], dim=1)  # kv_c / k_pe as views of one [T, 576] tensor
    cache = torch.zeros((2, 64, 1, 576), dtype=torch.bfloat16)
    slots = torch.arange(64, 128, dtype=torch.int32)
    want = orc.kvcache_write_ref(cache, lat, rope, slots.long(), False)
    d = both.to(DEV)
    dc = cache.to(DEV)
    flag_attn.concat_and_cache_mla(d[:, :512], d[:, 512:], dc, slots.to(DEV))
    torch.cuda.synchronize()
    assert torch.equal(dc.cpu().view(torch.int16), want.view(torch.int16))


def test_kvcache_write_then_sparse_fp8_decode():
    """Tokens written by the GPU writer decode exactly as the oracle-written cache does."""
    need_gpu()
    say("kvcache write -> sparse fp8 decode")
    lens = [1500, 900]
    nblk = sum(-(-n // 64) for n in lens) + 1
    gen = torch.Generator().manual_seed(50)
    lat, rope = _tokens(nblk * 64, 51)
    slots = torch.arange(nblk * 64, dtype=torch.int64)
    cache = torch.zeros((nblk, 64, 1, 656), dtype=torch.uint8)
    ref_cache = orc.kvcache_write_ref(cache, lat, rope, slots, True)
    dc = cache.to(DEV)
    flag_attn.concat_and_cache_mla(lat.to(DEV), rope.to(DEV), dc, slots.to(DEV), True)
    torch.cuda.synchronize()
    assert torch.equal(dc.cpu(), ref_cache)
    perm = torch.randperm(nblk, generator=gen).to(torch.int32)
    bt = torch.stack([perm[:24], torch.cat([perm[24:], perm[:24 - (nblk - 24)]])])
    ld = torch.tensor(lens, dtype=torch.int32)
    q = torch.randn((2, 1, 128, 576), generator=gen).to(torch.bfloat16)
    idx = orc.make_sparse_indices(2, 1, 512, lens, seed=52)
    out, lse = run_sparse(q, dc.cpu(), bt, ld, idx, SCALE, fp8=True)
    assert_close(out, lse, *sparse_refs(q, ref_cache, bt, ld, idx, SCALE, fp8=True))
