"""The GPU parity bars can fail -- CPU only.

A parity test proves nothing if a wrong answer passes it.  These tests take the inputs of
the GPU tests (and data shaped like the benchmark configs, N(0,1)*0.1), build plausible
wrong answers on the CPU from the oracle itself -- every key gathered one position off,
an all-zero output -- and check that ``tests/_helpers.assert_close`` rejects each of them
while it accepts the oracle's own answer.
"""
import pytest
import torch

from oracle import gqa_oracle as go
from oracle import mla_oracle as orc
from tests._helpers import assert_close, assert_lowp_rule
from tests.test_gpu_decode import sparse_random_inputs

SCALE = 192 ** -0.5


def _shift_indices(idx, lens):
    """Every valid index moved to its neighbouring token (i + 1, or i - 1 at the end)."""
    out = idx.clone()
    for b in range(idx.shape[0]):
        n = int(lens[b])
        row = out[b]
        valid = (row >= 0) & (row < n)
        up = torch.where(row + 1 < n, row + 1, row - 1)
        out[b] = torch.where(valid, up, row)
    return out


def _rejects(out, lse, ref_out, ref_lse, low):
    with pytest.raises(AssertionError):
        assert_close(out, lse, ref_out, ref_lse, low)


@pytest.mark.parametrize("fp8", [False, True])
def test_sparse_random_bars_reject_wrong_answers(fp8):
    q, kc, bt, ld, idx = sparse_random_inputs(fp8, 2048)
    ref_out, ref_lse = orc.sparse_decode_ref(q, kc, bt, ld, idx, SCALE, is_fp8=fp8)
    low, _ = orc.sparse_decode_ref(q, kc, bt, ld, idx, SCALE, is_fp8=fp8, lowp=True)
    # the oracle's own bf16-rounded answer passes
    assert_close(ref_out.to(torch.bfloat16), ref_lse, ref_out, ref_lse, low)
    # a gather one token off
    sh_out, sh_lse = orc.sparse_decode_ref(q, kc, bt, ld, _shift_indices(idx, ld), SCALE,
                                           is_fp8=fp8)
    _rejects(sh_out.to(torch.bfloat16), sh_lse, ref_out, ref_lse, low)
    # an all-zero output with the right lse
    _rejects(torch.zeros_like(ref_out).to(torch.bfloat16), ref_lse, ref_out, ref_lse, low)


def test_bench_like_dense_bars_reject_wrong_answers():
    """Data like BASELINE configs 2-5 (N(0,1) * 0.1): outputs ~1e-3, far below the absolute
    bars, so only the bf16-arithmetic rule can tell right from wrong here."""
    lens = [6000, 4500]
    q, kc, bt, ld = orc.make_dense_inputs(2, 128, 1, lens, seed=2, scale=0.1)
    ref_out, ref_lse = orc.dense_decode_ref(q, kc, bt, ld, SCALE)
    low, _ = orc.dense_decode_ref(q, kc, bt, ld, SCALE, lowp=True)
    assert float(ref_out.abs().max()) < 2e-2  # below ATOL_OUT: the absolute bar is blind
    assert_close(ref_out.to(torch.bfloat16), ref_lse, ref_out, ref_lse, low)
    # keys one token off: token j takes row j + 1 (the last one keeps its own)
    bad_out = torch.zeros_like(ref_out)
    bad_lse = torch.zeros_like(ref_lse)
    for b in range(2):
        n = lens[b]
        pos = torch.clamp(torch.arange(n) + 1, max=n - 1)
        kv = orc.gather_rows(kc, bt, b, pos).float()
        o, l = orc.attention_lse(q[b].float().permute(1, 0, 2), kv, kv[:, :512], SCALE, False)
        bad_out[b] = o.permute(1, 0, 2)
        bad_lse[b] = l
    _rejects(bad_out.to(torch.bfloat16), bad_lse, ref_out, ref_lse, low)
    _rejects(torch.zeros_like(ref_out).to(torch.bfloat16), ref_lse, ref_out, ref_lse, low)


@pytest.mark.parametrize("group,d,bs,max_len,dtype", [
    (8, 128, 16, 4096, torch.float16), (1, 64, 128, 512, torch.float16),
    (2, 256, 16, 1500, torch.float16), (8, 128, 16, 1500, torch.bfloat16),
])
def test_paged_bars_reject_dropped_and_wrong_pages(group, d, bs, max_len, dtype):
    """The paged GQA sweep's inputs (uniform(+-D^-0.5), tables drawn with replacement):
    outputs stay below ~2e-2, so the reference's allclose(atol=2e-3) can pass a kernel
    that loses the last 16 keys of each sequence.  The three-way rule against the fp32 result
    and the low-precision leg rejects that, and a wrong page id for the last page, while
    the oracle's own rounded answer passes both."""
    gen = torch.Generator().manual_seed(group + d)
    ns, h, nb = 16, 32, 200
    s = d ** -0.5
    lens = torch.randint(1, max_len, (ns,), generator=gen, dtype=torch.int32)
    lens[0] = max_len
    q = (torch.rand((ns, h, d), generator=gen) * 2 - 1).mul(s).to(dtype)
    kc = (torch.rand((nb, h // group, bs, d), generator=gen) * 2 - 1).mul(s).to(dtype)
    vc = (torch.rand((nb, h // group, bs, d), generator=gen) * 2 - 1).mul(s).to(dtype)
    bt = torch.randint(0, nb, (ns, -(-max_len // bs)), generator=gen, dtype=torch.int32)
    ref32 = go.paged_attention_ref(q, kc, vc, bt, lens, s, out_fp32=True)
    low = go.paged_attention_lowp(q, kc, vc, bt, lens, s)
    own = go.paged_attention_ref(q, kc, vc, bt, lens, s)
    assert torch.allclose(own, ref32.to(dtype), atol=2e-3, rtol=1e-5)
    assert_lowp_rule(own, ref32, low)
    dropped = go.paged_attention_ref(q, kc, vc, bt, torch.clamp(lens - 16, min=1), s)
    wrong_bt = bt.clone()
    for i in range(ns):
        last = (int(lens[i]) - 1) // bs
        wrong_bt[i, last] = (wrong_bt[i, last] + 1) % nb
    wrong = go.paged_attention_ref(q, kc, vc, wrong_bt, lens, s)
    for bad in (dropped, wrong):
        with pytest.raises(AssertionError):
            assert_lowp_rule(bad, ref32, low)
