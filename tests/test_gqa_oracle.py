"""Pins of the grouped-query oracle (oracle/gqa_oracle.py) -- CPU only.

The reference ships no golden vectors for its paged / split-KV decode (its tests are
randomised against its own PyTorch oracles), so the restatements are pinned by:
(1) the vectorised paged gather against the line-for-line restatement of
``testing/paged.py``, bit for bit; (2) float64 brute force; (3) closed forms that fix
the answer (causal first row, uniform keys, one visible key); (4) agreement between the
paged and the contiguous oracles on the same keys; (5) mutations -- a top-left causal
mask, a dropped scale, a wrong GQA head mapping -- that must fail (2)-(4).
"""
import math

import pytest
import torch

from oracle import gqa_oracle as go


def _paged_case(seed, num_seqs, h_q, group, d, bs, max_len, nblocks=50, dtype=torch.float16):
    gen = torch.Generator().manual_seed(seed)
    h_kv = h_q // group
    lens = torch.randint(1, max_len, (num_seqs,), generator=gen, dtype=torch.int32)
    lens[0] = max_len
    s = d ** -0.5
    q = (torch.rand((num_seqs, h_q, d), generator=gen) * 2 - 1).mul(s).to(dtype)
    kc = (torch.rand((nblocks, h_kv, bs, d), generator=gen) * 2 - 1).mul(s).to(dtype)
    vc = (torch.rand((nblocks, h_kv, bs, d), generator=gen) * 2 - 1).mul(s).to(dtype)
    bt = torch.randint(0, nblocks, (num_seqs, -(-max_len // bs)), generator=gen,
                       dtype=torch.int32)
    return q, kc, vc, bt, lens, s


@pytest.mark.parametrize("group,bs", [(1, 16), (4, 4), (8, 16)])
def test_paged_vectorised_equals_loop(group, bs):
    q, kc, vc, bt, lens, s = _paged_case(group * 10 + bs, 3, 8, group, 32, bs, 100)
    a = go.paged_attention_loop(q, kc, vc, bt, lens, s)
    b = go.paged_attention_ref(q, kc, vc, bt, lens, s)
    assert torch.equal(a, b)


def _brute(q, k, v, causal, scale):
    """float64 attention of q [B, H, M, D] over k, v [B, Hk, N, D], head h -> kv h // g."""
    b, h, m, d = q.shape
    hk, n = k.shape[1], k.shape[2]
    g = h // hk
    out = torch.zeros((b, h, m, d), dtype=torch.float64)
    lse = torch.zeros((b, h, m), dtype=torch.float64)
    for bi in range(b):
        for hi in range(h):
            kk = k[bi, hi // g].double()
            vv = v[bi, hi // g].double()
            for mi in range(m):
                lim = n - m + mi + 1 if causal else n
                sc = (kk[:lim] @ q[bi, hi, mi].double()) * scale
                mx = sc.max()
                w = torch.exp(sc - mx)
                out[bi, hi, mi] = (w[:, None] * vv[:lim]).sum(0) / w.sum()
                lse[bi, hi, mi] = mx + torch.log(w.sum())
    return out, lse


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("h,hk,m,n", [(4, 4, 1, 37), (4, 2, 3, 20), (6, 1, 4, 9)])
def test_flash_ref_matches_float64_brute_force(causal, h, hk, m, n):
    gen = torch.Generator().manual_seed(h * 100 + m * 10 + n)
    q = torch.randn((2, h, m, 16), generator=gen)
    k = torch.randn((2, hk, n, 16), generator=gen)
    v = torch.randn((2, hk, n, 16), generator=gen)
    o, lse = go.flash_attention_ref(q, k, v, causal, upcast=True)
    bo, bl = _brute(q, k, v, causal, 16 ** -0.5)
    assert torch.allclose(o.double(), bo, atol=1e-5)
    assert torch.allclose(lse.double(), bl, atol=1e-5)


def test_flash_ref_closed_forms():
    gen = torch.Generator().manual_seed(3)
    n = 7
    q = torch.randn((1, 2, n, 8), generator=gen)
    k = torch.randn((1, 2, n, 8), generator=gen)
    v = torch.randn((1, 2, n, 8), generator=gen)
    o, lse = go.flash_attention_ref(q, k, v, True)
    # causal with M == N: query 0 sees key 0 only -> out = v[0], lse = q0.k0 * scale
    assert torch.allclose(o[:, :, 0], v[:, :, 0], atol=1e-6)
    want = (q[0, :, 0] * k[0, :, 0]).sum(-1) * 8 ** -0.5
    assert torch.allclose(lse[0, :, 0], want, atol=1e-6)
    # a zero query: uniform weights over the visible keys, lse = log(count)
    qz = torch.zeros_like(q)
    o, lse = go.flash_attention_ref(qz, k, v, False)
    assert torch.allclose(o[0, :, 3], v[0].mean(1), atol=1e-6)
    assert torch.allclose(lse, torch.full_like(lse, math.log(n)), atol=1e-6)


def test_paged_ref_agrees_with_flash_ref():
    """The paged oracle over an identity block table equals the contiguous oracle."""
    gen = torch.Generator().manual_seed(5)
    h_q, h_kv, d, bs, n = 8, 2, 32, 16, 70
    kc = torch.randn((5, h_kv, bs, d), generator=gen).half()
    vc = torch.randn((5, h_kv, bs, d), generator=gen).half()
    q = torch.randn((1, h_q, d), generator=gen).half()
    bt = torch.arange(5, dtype=torch.int32).view(1, 5)
    lens = torch.tensor([n], dtype=torch.int32)
    a = go.paged_attention_ref(q, kc, vc, bt, lens, d ** -0.5)
    k = kc.permute(1, 0, 2, 3).reshape(h_kv, 5 * bs, d)[:, :n].unsqueeze(0)
    v = vc.permute(1, 0, 2, 3).reshape(h_kv, 5 * bs, d)[:, :n].unsqueeze(0)
    b, _ = go.flash_attention_ref(q.unsqueeze(2), k, v, False)
    assert torch.allclose(a.float(), b[:, :, 0].float(), atol=1e-3)


def test_mutations_fail_the_pins():
    """Plausible mistakes planted in copies of the oracle are caught."""
    gen = torch.Generator().manual_seed(9)
    q = torch.randn((1, 4, 3, 16), generator=gen)
    k = torch.randn((1, 2, 10, 16), generator=gen)
    v = torch.randn((1, 2, 10, 16), generator=gen)
    bo, bl = _brute(q, k, v, True, 16 ** -0.5)

    def top_left(q, k, v):
        s = torch.matmul(q, torch.repeat_interleave(k, 2, 1).transpose(2, 3)) * 16 ** -0.5
        m, n = s.shape[-2:]
        s = torch.where(torch.arange(m)[:, None] >= torch.arange(n), s, float("-inf"))
        return torch.softmax(s, -1) @ torch.repeat_interleave(v, 2, 1)

    def wrong_group(q, k, v):  # head h -> kv head h % hk instead of h // g
        kk = k.repeat(1, 2, 1, 1)
        vv = v.repeat(1, 2, 1, 1)
        return go.flash_attention_ref(q, kk, vv, True)[0]

    def no_scale(q, k, v):
        return go.flash_attention_ref(q * 4.0, k, v, True)[0]

    for mutant in (top_left, wrong_group, no_scale):
        assert not torch.allclose(mutant(q, k, v).double(), bo, atol=1e-3), mutant.__name__
