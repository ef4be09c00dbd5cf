"""Pins of the low-precision oracle legs (the ``torch_lowp`` side of the three-way rule) --
CPU only.

The reference's accuracy rule ``max|hyp - ref| <= 2 max|lowp - ref| + 1e-5``
(``tests/flag_attn/test_flash_attention.py:119-127``) takes its bar from the
``upcast=False`` arithmetic of ``testing/flash.py:19-84``: ``S = q k^T`` rounded to the
input dtype, ``* sm_scale`` rounded again, softmax in fp32, ``P`` rounded to the input
dtype (``:73``), ``P v`` rounded to the input dtype.  A slip in that leg (computing it in
fp32, say) would move every bar that the GPU tests draw from it, so the leg is checked here
against an independent float64 emulation: the same rounding points, with round-to-nearest-
even to the dtype's significand done by hand (numpy ``frexp`` / ``rint``), not by torch's
casts.  Products and sums run in float64, so the torch legs (fp32 accumulation) may differ
from it by at most one unit in the last place of the low dtype at a rounding boundary.

Legs pinned: ``gqa_oracle.flash_attention_ref(upcast=False)`` (the bar of the
``test_attention_splitkv`` sweep), ``gqa_oracle.paged_attention_lowp`` (the bar of the
paged sweeps) and ``mla_oracle.attention_lse_lowp`` (the bar of every MLA decode test).
Each check is shown to reject the leg computed in fp32 instead.
"""
import math

import numpy as np
import pytest
import torch

from oracle import gqa_oracle as go
from oracle import mla_oracle as orc

# (significand bits incl. the implicit one, frexp exponent of the smallest normal, max finite)
FORMATS = {
    torch.float16: (11, -13, 65504.0),
    torch.bfloat16: (8, -125, 3.3895313892515355e38),
}


def round_to(x, dtype) -> np.ndarray:
    """float64 -> nearest value of ``dtype`` (ties to even), as float64; subnormals keep
    fewer significand bits, values past the largest finite one become +-inf."""
    p, emin, vmax = FORMATS[dtype]
    x = np.asarray(x, dtype=np.float64)
    m, e = np.frexp(x)  # x = m * 2^e, 0.5 <= |m| < 1
    # subnormal range keeps fewer bits (none or fewer: |x| under half the smallest step -> 0)
    bits = np.where(e >= emin, p, p - (emin - e))
    r = np.ldexp(np.rint(np.ldexp(m, bits)), e - bits)
    r = np.where(np.abs(r) > vmax, np.copysign(np.inf, x), r)
    return np.where(np.isfinite(x), r, x)


def ulp(x, dtype) -> np.ndarray:
    p, emin, _ = FORMATS[dtype]
    _, e = np.frexp(np.abs(np.asarray(x, dtype=np.float64)))
    return np.ldexp(1.0, np.maximum(e, emin) - p)


def emulate_attention_lowp(q, k, v, scale, causal, dtype):
    """float64 emulation of ``testing/flash.py:47-75`` with ``upcast=False``.
    q [..., M, D], k [..., N, D], v [..., N, Dv] (heads already matched); returns
    (out [..., M, Dv] rounded to dtype, lse [..., M])."""
    q64 = np.asarray(q.to(dtype).double())
    k64 = np.asarray(k.to(dtype).double())
    v64 = np.asarray(v.to(dtype).double())
    s = round_to(q64 @ np.swapaxes(k64, -1, -2), dtype)   # q k^T in dtype
    s = round_to(s * scale, dtype)                        # * sm_scale in dtype
    m, n = s.shape[-2], s.shape[-1]
    if causal:
        vis = np.arange(m)[:, None] + (n - m) >= np.arange(n)[None, :]
        s = np.where(vis, s, -np.inf)
    mx = s.max(axis=-1, keepdims=True)
    mx_safe = np.where(np.isfinite(mx), mx, 0.0)
    w = np.exp(s - mx_safe)
    tot = w.sum(axis=-1, keepdims=True)
    with np.errstate(divide="ignore", invalid="ignore"):
        lse = np.where(tot > 0, np.log(tot) + mx_safe, -np.inf)[..., 0]
        p = np.where(tot > 0, w / tot, 0.0)
    p = round_to(p, dtype)                                # P.to(v.dtype)
    out = round_to(p @ v64, dtype)                        # P v in dtype
    return out, lse


def agreement(hyp, emu, dtype):
    """(share of elements equal to the emulation, max difference in units of the low dtype's
    last place)."""
    h = np.asarray(hyp.double())
    d = np.abs(h - emu)
    return float((d == 0).mean()), float((d / ulp(np.maximum(np.abs(h), np.abs(emu)), dtype)).max())


def assert_matches(hyp, emu, dtype):
    same, worst = agreement(hyp, emu, dtype)
    assert same >= 0.95 and worst <= 1.0, (same, worst)


def assert_rejected(hyp, emu, dtype):
    same, worst = agreement(hyp, emu, dtype)
    assert not (same >= 0.95 and worst <= 1.0), (same, worst)


def test_round_to_known_values():
    """The hand rounding against values fixed by the formats' definitions."""
    f16, bf = torch.float16, torch.bfloat16
    # ties to even at 1 + half an ulp, and just past it
    assert round_to(1 + 2 ** -11, f16) == 1.0
    assert round_to(1 + 3 * 2 ** -11, f16) == 1 + 2 ** -9
    assert round_to(1 + 2 ** -11 + 2 ** -30, f16) == 1 + 2 ** -10
    assert round_to(1 + 2 ** -8, bf) == 1.0
    assert round_to(1 + 3 * 2 ** -8, bf) == 1 + 2 ** -6
    # fp16 subnormals: step 2^-24; the smallest normal 2^-14; overflow past 65504
    assert round_to(3 * 2 ** -25, f16) == 2 ** -23
    assert round_to(2 ** -25, f16) == 0.0
    assert round_to(2 ** -14 * (1 + 2 ** -12), f16) == 2 ** -14
    assert round_to(65519.0, f16) == 65504.0 and np.isinf(round_to(65520.0, f16))
    # agreement with torch's own casts on random values (both are round-to-nearest-even)
    gen = torch.Generator().manual_seed(0)
    x = torch.randn(20000, generator=gen, dtype=torch.float64) * 10.0 ** torch.randint(
        -9, 5, (20000,), generator=gen)
    for dt in (f16, bf):
        want = x.float().to(dt).double().numpy()
        got = round_to(x.float().double().numpy(), dt)
        assert np.array_equal(got, want)


def _splitkv_case(b, hq, hk, m, n, d, dtype, scale, seed):
    gen = torch.Generator().manual_seed(seed)
    q = torch.empty((b, hq, m, d)).normal_(0.0, scale, generator=gen).to(dtype)
    k = torch.empty((b, hk, n, d)).normal_(0.0, scale, generator=gen).to(dtype)
    v = torch.empty((b, hk, n, d)).normal_(0.0, scale, generator=gen).to(dtype)
    return q, k, v


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("b,hq,hk,m,n,d,causal,scale", [
    # test_attention_splitkv's inputs (scale 10): scores spread so far that the softmax is
    # one-hot and both legs return the same rows; the emulation must still match
    (2, 4, 4, 1, 612, 128, False, 10.0),
    (1, 4, 2, 2, 400, 64, True, 10.0),
    # scale 1: the legs differ, and the fp32 one must be rejected
    (2, 4, 4, 1, 612, 128, False, 1.0),
    (1, 4, 2, 2, 400, 64, True, 1.0),
    (2, 4, 1, 4, 300, 16, True, 1.0),
])
def test_flash_lowp_leg_matches_emulation(dtype, b, hq, hk, m, n, d, causal, scale):
    q, k, v = _splitkv_case(b, hq, hk, m, n, d, dtype, scale, seed=n + m)
    g = hq // hk
    kk = torch.repeat_interleave(k, g, dim=1)
    vv = torch.repeat_interleave(v, g, dim=1)
    emu_o, emu_l = emulate_attention_lowp(q, kk, vv, d ** -0.5, causal, dtype)
    o_low, l_low = go.flash_attention_ref(q, k, v, causal, upcast=False)
    assert o_low.dtype == dtype
    assert_matches(o_low, emu_o, dtype)
    assert np.allclose(l_low.double().numpy(), emu_l, rtol=1e-6, atol=1e-5)
    # planted: the leg computed in fp32 (upcast=True) must not pass for the low one
    o_hi, _ = go.flash_attention_ref(q, k, v, causal, upcast=True)
    if scale == 1.0:
        assert_rejected(o_hi, emu_o, dtype)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_paged_lowp_leg_matches_emulation(dtype):
    """The low-precision leg of the paged oracle on the paged sweep's input distribution
    (uniform(+-D^-0.5)): the gathered keys through the same emulation."""
    gen = torch.Generator().manual_seed(4)
    h_q, h_kv, d, bs, nblk = 8, 2, 64, 16, 40
    s = d ** -0.5
    q = (torch.rand((3, h_q, d), generator=gen) * 2 - 1).mul(s).to(dtype)
    kc = (torch.rand((nblk, h_kv, bs, d), generator=gen) * 2 - 1).mul(s).to(dtype)
    vc = (torch.rand((nblk, h_kv, bs, d), generator=gen) * 2 - 1).mul(s).to(dtype)
    bt = torch.randint(0, nblk, (3, 20), generator=gen, dtype=torch.int32)
    lens = torch.tensor([300, 17, 129], dtype=torch.int32)
    low = go.paged_attention_lowp(q, kc, vc, bt, lens, s)
    hi = go.paged_attention_ref(q, kc, vc, bt, lens, s, out_fp32=True)
    for i in range(3):
        n = int(lens[i])
        pos = torch.arange(n)
        pages = bt[i].long()[pos // bs]
        k = kc[pages, :, pos % bs, :].permute(1, 0, 2)  # [h_kv, n, d]
        v = vc[pages, :, pos % bs, :].permute(1, 0, 2)
        g = h_q // h_kv
        kk = torch.repeat_interleave(k, g, dim=0)
        vv = torch.repeat_interleave(v, g, dim=0)
        emu_o, _ = emulate_attention_lowp(q[i].unsqueeze(1), kk, vv, s, False, dtype)
        assert_matches(low[i], emu_o[:, 0], dtype)
    # planted: the fp32 leg, rounded to the dtype at the end, is not the low one
    emu_all = []
    for i in range(3):
        n = int(lens[i])
        pos = torch.arange(n)
        pages = bt[i].long()[pos // bs]
        kk = torch.repeat_interleave(kc[pages, :, pos % bs, :].permute(1, 0, 2), h_q // h_kv, 0)
        vv = torch.repeat_interleave(vc[pages, :, pos % bs, :].permute(1, 0, 2), h_q // h_kv, 0)
        emu_all.append(emulate_attention_lowp(q[i].unsqueeze(1), kk, vv, s, False, dtype)[0][:, 0])
    assert_rejected(hi.to(dtype), np.stack(emu_all), dtype)


@pytest.mark.parametrize("m,n,causal", [(1, 700, False), (2, 333, True)])
def test_mla_lowp_leg_matches_emulation(m, n, causal):
    """``attention_lse_lowp`` on the MLA decode tests' unit-scale inputs (576-dim QK,
    512-dim V = the first 512 dims of the same rows, one shared KV head)."""
    gen = torch.Generator().manual_seed(n)
    h = 16
    q = torch.randn((h, m, 576), generator=gen).to(torch.bfloat16)
    kv = torch.randn((n, 576), generator=gen).to(torch.bfloat16)
    scale = 192 ** -0.5
    o_low, l_low = orc.attention_lse_lowp(q, kv, kv[:, :512], scale, causal)
    emu_o, emu_l = emulate_attention_lowp(q, kv.unsqueeze(0).expand(h, n, 576),
                                          kv[:, :512].unsqueeze(0).expand(h, n, 512), scale,
                                          causal, torch.bfloat16)
    assert_matches(o_low, emu_o, torch.bfloat16)
    assert np.allclose(l_low.double().numpy(), emu_l, rtol=1e-6, atol=1e-5)
    # planted: the fp32 leg (attention_lse) is rejected on both outputs
    o_hi, l_hi = orc.attention_lse(q, kv, kv[:, :512], scale, causal)
    assert_rejected(o_hi.to(torch.bfloat16), emu_o, torch.bfloat16)
    assert float(np.abs(l_hi.double().numpy() - emu_l).max()) > 1e-4
