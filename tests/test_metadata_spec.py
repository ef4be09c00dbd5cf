"""Tile-scheduler metadata spec (oracle.metadata_spec) -- CPU only.

No reference implements this scheduler (the reference picks one split count per launch,
src/flag_attn/paged.py:52-67, src/flag_attn/split_kv.py:248-276), so the spec is pinned by
hand-derived cases and by the invariants a valid partition must satisfy.
"""
import random

import pytest

from oracle.mla_oracle import metadata_spec

PAGE = 64


def _blocks(lens, topk):
    return [-(-topk // PAGE)] * len(lens) if topk else [-(-max(x, 0) // PAGE) for x in lens]


def _segments(md, num_parts):
    segs = []  # (part, b, lo, hi, local)
    for p in range(num_parts):
        bb, blo, eb, bhi, first, n, g0, _ = md[p]
        if n == 0:
            continue
        for b in range(bb, eb + 1):
            segs.append((p, b, blo if b == bb else 0, bhi if b == eb else None,
                         first if b == bb else 0))
    return segs


def check_invariants(lens, num_parts, overhead, topk=0):
    md, ns = metadata_spec(lens, num_parts, overhead, topk)
    nb = _blocks(lens, topk)
    bsz = len(lens)
    assert len(md) == num_parts and len(ns) == bsz + 1 and ns[0] == 0
    # parts tile the global block line contiguously, in order
    starts = [row[6] for row in md] + [sum(nb)]
    assert starts[0] == 0 and all(a <= b for a, b in zip(starts, starts[1:]))
    for p in range(num_parts):
        assert md[p][5] == starts[p + 1] - starts[p]
    # every (sequence, block) is covered exactly once, segments numbered 0..n-1 in order
    covered = {b: [] for b in range(bsz)}
    for p, b, lo, hi, local in _segments(md, num_parts):
        hi = nb[b] if hi is None else hi
        if hi <= lo:  # a middle sequence with no blocks is skipped by the kernel
            assert nb[b] == 0
            continue
        covered[b].append((lo, hi, local))
    for b in range(bsz):
        segs = sorted(covered[b])
        assert [s[2] for s in segs] == list(range(len(segs)))
        pos = 0
        for lo, hi, _ in segs:
            assert lo == pos and hi > lo
            pos = hi
        assert pos == nb[b]
        assert ns[b + 1] - ns[b] == len(segs)
    # balance: a part never holds more blocks than one cost share
    w = sum(n + overhead for n in nb if n > 0)
    share = -(-w // num_parts)
    assert all(row[5] <= share for row in md)
    return md, ns


def test_hand_case_two_sequences_four_parts():
    # lens 256/384 -> 4 + 6 blocks; overhead 4 -> costs 8, 10 (W = 18);
    # cuts at cost 0, 5, 9, 14 -> global blocks 0, 1, 4, 6 (end 10)
    md, ns = metadata_spec([256, 384], 4, 4)
    assert md == [[0, 0, 0, 1, 0, 1, 0, 0],
                  [0, 1, 0, 4, 1, 3, 1, 0],
                  [1, 0, 1, 2, 0, 2, 4, 0],
                  [1, 2, 1, 6, 1, 4, 6, 0]]
    assert ns == [0, 2, 4]


def test_hand_case_single_part_is_unsplit():
    md, ns = metadata_spec([100, 0, 65], 1, 5)
    # blocks 2, 0, 2 -> one part covering all 4 global blocks
    assert md == [[0, 0, 2, 2, 0, 4, 0, 0]]
    assert ns == [0, 1, 1, 2]


def test_hand_case_more_parts_than_work():
    md, ns = metadata_spec([64], 4, 0)
    # one block, cost 1: x_p = ceil(p/4) = 0,1,1,1 -> part 0 has the block, the rest empty
    assert md[0] == [0, 0, 0, 1, 0, 1, 0, 0]
    assert [row[5] for row in md[1:]] == [0, 0, 0]
    assert ns == [0, 1]


def test_sparse_topk_uniform():
    md, ns = check_invariants([5000] * 8, 16, 4, topk=2048)
    # 8 x 32 blocks, cost 8 x 36 = 288 -> 18 per part: every part gets 14..18 blocks
    assert all(14 <= row[5] <= 18 for row in md)
    assert ns[-1] <= 8 + 16 - 1


@pytest.mark.parametrize("seed", range(20))
def test_random_invariants(seed):
    rng = random.Random(seed)
    bsz = rng.randint(1, 40)
    lens = [rng.choice([0, 1, 63, 64, 65, rng.randint(0, 20000)]) for _ in range(bsz)]
    if all(x == 0 for x in lens):
        lens[0] = 1
    parts = rng.choice([1, 2, 7, 8, 64, 128, 256])
    overhead = rng.choice([0, 1, 4, 5, 16])
    check_invariants(lens, parts, overhead)


def test_all_empty():
    md, ns = metadata_spec([0, 0, 0], 8, 4)
    assert all(row[5] == 0 for row in md) and ns == [0, 0, 0, 0]
