"""Pins of the top-k index oracle (oracle/topk_oracle.py) -- CPU only.

There is no reference index producer, so the restatement is pinned by: (1) ``torch.topk``
(a library routine) on rows of distinct finite scores; (2) closed forms -- rows that see
at most ``topk`` keys keep ``0..n-1``, all-equal rows keep the first ``topk`` positions,
causal visibility ``n = len - (s_q - 1 - t)``; (3) the uint32 key order against numpy's
own float comparisons, with the specials placed by hand; (4) an exchange check: no kept
score ranks below a dropped one, and the output is strictly ascending; (5) planted
mistakes (ties by higher position, a visible length one short, top-left causal, unsorted
output) that must fail (1)-(4).
"""
import numpy as np
import pytest
import torch

from oracle import topk_oracle as tko


@pytest.mark.parametrize("length,topk", [(100, 7), (5000, 2048), (4097, 4096), (70, 1)])
def test_matches_torch_topk_on_distinct_scores(length, topk):
    gen = torch.Generator().manual_seed(length + topk)
    scores = torch.randperm(length * 3, generator=gen)[:length].float().view(1, 1, length) / 7.0
    lens = [length - 3]
    got = tko.topk_indices_ref(scores.numpy(), lens, topk)
    n = lens[0]
    want = torch.topk(scores[0, 0, :n], min(topk, n)).indices.sort().values.numpy()
    assert np.array_equal(got[0, 0, :len(want)], want)
    assert (got[0, 0, len(want):] == -1).all()


def test_closed_forms():
    rng = np.random.default_rng(1)
    sc = rng.standard_normal((3, 2, 50)).astype(np.float32)
    got = tko.topk_indices_ref(sc, [10, 0, 64], 16)
    assert np.array_equal(got[0, 0], np.r_[np.arange(10), -np.ones(6)])
    assert (got[1] == -1).all()
    assert np.array_equal(got[2, 1], np.sort(np.argsort(-sc[2, 1], kind="stable")[:16]))
    flat = np.zeros((1, 1, 300), np.float32)
    assert np.array_equal(tko.topk_indices_ref(flat, [300], 40)[0, 0], np.arange(40))
    # causal: token t of s_q = 3 sees len - (2 - t) keys
    n = tko.visible_lengths([20], 3, 50, True)
    assert n.tolist() == [[18, 19, 20]]
    got = tko.topk_indices_ref(np.zeros((1, 3, 50), np.float32), [20], 32, causal=True)
    assert [int((r >= 0).sum()) for r in got[0]] == [18, 19, 20]


def test_key_order_matches_float_order_and_places_specials():
    rng = np.random.default_rng(2)
    x = np.concatenate([rng.standard_normal(2000), [0.0, np.inf, -np.inf, 1e-45, -1e-45,
                                                     3.4e38, -3.4e38]]).astype(np.float32)
    k = tko.order_keys(x)
    i, j = rng.integers(0, x.size, (2, 20000))
    both = (x[i] != x[j])
    assert np.array_equal((k[i] > k[j])[both], (x[i] > x[j])[both])
    bits = np.array([0xFFFFFFFF, 0xFF800000, 0x80000000, 0x00000000, 0x7F800000, 0x7FC00000],
                    np.uint32)  # -NaN, -inf, -0, +0, +inf, +NaN in ascending rank
    assert (np.diff(tko.order_keys(bits.view(np.float32)).astype(np.int64)) > 0).all()


def _exchange_ok(scores, n, row):
    kept = row[row >= 0]
    if kept.size and kept.max() >= n:
        return False
    if n <= row.size:
        return np.array_equal(kept, np.arange(n))
    if kept.size != row.size or not (np.diff(kept) > 0).all():
        return False
    keys = tko.order_keys(scores[:n]).astype(np.int64)
    mask = np.zeros(n, bool)
    mask[kept] = True
    kmin = keys[mask].min()
    dropped = keys[~mask]
    if (dropped > kmin).any():
        return False
    # among ties at the boundary, kept positions come first
    tie_kept = np.nonzero(mask & (keys == kmin))[0]
    tie_drop = np.nonzero(~mask & (keys == kmin))[0]
    return tie_drop.size == 0 or tie_kept.max() < tie_drop.min()


@pytest.mark.parametrize("seed", range(6))
def test_exchange_property(seed):
    rng = np.random.default_rng(seed)
    sc = rng.integers(-4, 4, (2, 3, 700)).astype(np.float32)  # heavy ties
    lens = [700, 333]
    got = tko.topk_indices_ref(sc, lens, 100, causal=True)
    n = tko.visible_lengths(lens, 3, 700, True)
    for b in range(2):
        for t in range(3):
            assert _exchange_ok(sc[b, t], int(n[b, t]), got[b, t])


def _mutant(scores, lens, topk, causal, ties_high=False, len_off=0, ignore_causal=False,
            ascending=True):
    """The oracle with one planted mistake."""
    bsz, s_q, length = scores.shape
    n_vis = tko.visible_lengths([x + len_off for x in lens], s_q, length,
                                causal and not ignore_causal)
    out = np.full((bsz, s_q, topk), -1, np.int32)
    for b in range(bsz):
        for t in range(s_q):
            n = int(n_vis[b, t])
            keys = tko.order_keys(scores[b, t, :n]).astype(np.int64)
            pos = np.arange(n)
            order = np.lexsort((-pos if ties_high else pos, -keys))[:topk]
            out[b, t, :order.size] = np.sort(order) if ascending else order
    return out


def test_planted_mistakes_fail():
    rng = np.random.default_rng(7)
    ties = rng.integers(-3, 3, (1, 2, 400)).astype(np.float32)
    distinct = rng.permutation(800)[:400].astype(np.float32).reshape(1, 1, 400)
    distinct = np.repeat(distinct, 2, 1)
    distinct[0, :, 399] = 1e6  # the last key scores highest
    lens = [400]
    for sc, kw in ((ties, dict(ties_high=True)), (distinct, dict(ascending=False)),
                   (distinct, dict(len_off=-1)), (distinct, dict(ignore_causal=True))):
        n = tko.visible_lengths(lens, 2, 400, True)
        good = tko.topk_indices_ref(sc, lens, 50, causal=True)
        assert all(_exchange_ok(sc[0, t], int(n[0, t]), good[0, t]) for t in range(2))
        bad = _mutant(sc, lens, 50, True, **kw)
        assert not all(_exchange_ok(sc[0, t], int(n[0, t]), bad[0, t]) for t in range(2)), kw
