"""GPU parity of the top-k index producer (flag_attn.topk_indices) against the CPU oracle,
bit for bit: the kept set is fixed by the score order and the tie rule, and the output
order is ascending, so any difference is a bug.

Cases: random rows over every register-tile size the kernel instantiates (lengths 1 to
65536), topk 1 to 65535, causal s_q = 1..3, sequences shorter than topk, empty and
longer-than-scores lengths, heavy ties (integer scores, constant rows), IEEE specials
(+-0, +-inf, +-NaN incl. the all-ones pattern), strided score rows, and the sparse
benchmark shape (B = 128, 65536 scores per row, top-2048).
"""
import numpy as np
import pytest
import torch

import flag_attn
from oracle import topk_oracle as tko
from tests._helpers import DEV, need_gpu, say

pytestmark = pytest.mark.gpu


def _run(scores, lens, topk, causal):
    need_gpu()
    say(f"topk scores={tuple(scores.shape)} topk={topk} causal={causal}")
    got = flag_attn.topk_indices(scores.to(DEV), torch.tensor(lens, dtype=torch.int32).to(DEV),
                                 topk, causal=causal).cpu().numpy()
    want = tko.topk_indices_ref(scores.numpy(), lens, topk, causal)
    assert got.dtype == np.int32 and got.shape == want.shape
    bad = np.argwhere(got != want)
    assert bad.size == 0, f"{bad.shape[0]} mismatches, first at {bad[0].tolist()}"


@pytest.mark.parametrize("length", [1, 100, 1024, 1025, 3000, 5000, 9000, 17000, 40000, 65536])
@pytest.mark.parametrize("topk", [1, 64, 2048])
def test_random_rows(length, topk):
    gen = torch.Generator().manual_seed(length * 7 + topk)
    b, s_q = 3, 2
    scores = torch.randn((b, s_q, length), generator=gen)
    lens = [length, max(0, length - 37), min(length + 5, 70000)]
    _run(scores, lens, topk, causal=True)


@pytest.mark.parametrize("length,topk", [(40000, 10000), (65536, 65535), (9000, 4097)])
def test_large_topk(length, topk):
    gen = torch.Generator().manual_seed(topk)
    scores = torch.randn((2, 2, length), generator=gen)
    _run(scores, [length, length - 1], topk, causal=True)


@pytest.mark.parametrize("topk", [100, 1000, 4096])
@pytest.mark.parametrize("kind", ["int", "const", "fp16", "specials"])
def test_ties_and_specials(topk, kind):
    gen = torch.Generator().manual_seed(topk)
    shape = (2, 3, 12000)
    if kind == "int":
        scores = torch.randint(-3, 3, shape, generator=gen).float()
    elif kind == "const":
        scores = torch.full(shape, -1.5)
    elif kind == "fp16":
        scores = (torch.randn(shape, generator=gen) * 1e-3).half().float()
    else:
        pool = np.array([0xFFFFFFFF, 0xFFFFFFFE, 0xFF800000, 0xFF000000, 0x80000000, 0x00000000,
                         0x00000001, 0x3F800000, 0x7F800000, 0x7FC00000, 0x7FFFFFFF], np.uint32)
        pick = torch.randint(0, pool.size, shape, generator=gen).numpy()
        scores = torch.from_numpy(pool[pick].view(np.float32).copy())
    _run(scores, [12000, 9000], topk, causal=kind != "const")


@pytest.mark.parametrize("kind", ["int", "const", "specials"])
def test_two_stage_ties_and_specials(kind):
    """Rows long enough for the chunked two-stage path (50000 scores, top-1000): ties
    that span chunks, constant rows, IEEE specials."""
    gen = torch.Generator().manual_seed(7)
    shape = (2, 2, 50000)
    if kind == "int":
        scores = torch.randint(-3, 3, shape, generator=gen).float()
    elif kind == "const":
        scores = torch.full(shape, 0.25)
    else:
        pool = np.array([0xFFFFFFFF, 0xFF800000, 0x80000000, 0x00000000, 0x3F800000,
                         0x7F800000, 0x7FC00000], np.uint32)
        pick = torch.randint(0, pool.size, shape, generator=gen).numpy()
        scores = torch.from_numpy(pool[pick].view(np.float32).copy())
    _run(scores, [50000, 33000], 1000, causal=True)


def test_two_stage_chunk_boundaries():
    """Sequence lengths that end inside, at, and just past chunk boundaries, and chunks
    with fewer scores than topk."""
    gen = torch.Generator().manual_seed(8)
    scores = torch.randn((6, 1, 65536), generator=gen)
    _run(scores, [16384, 16385, 2049, 32768 + 2047, 49152 + 5000, 65536], 2048, causal=False)


def test_all_ones_pattern_rows():
    """Every score is the bit pattern 0xFFFFFFFF (key 0, the same key the kernel's padding
    slots carry): ties resolve by position over the visible keys only."""
    need_gpu()
    scores = torch.from_numpy(np.full((2, 1, 5000), 0xFFFFFFFF, np.uint32).view(np.float32).copy())
    _run(scores, [4500, 3000], 2048, causal=False)


@pytest.mark.parametrize("topk", [7, 2048])
def test_short_and_empty_sequences(topk):
    gen = torch.Generator().manual_seed(11)
    scores = torch.randn((4, 3, 3000), generator=gen)
    _run(scores, [0, 1, topk, 2], topk, causal=True)


def test_strided_rows_and_out_argument():
    need_gpu()
    gen = torch.Generator().manual_seed(5)
    base = torch.randn((2, 4, 9000), generator=gen).to(DEV)
    view = base[:, 1:4, 100:7100]  # strides (36000, 9000, 1), 7000 scores per row
    lens = torch.tensor([7000, 5000], dtype=torch.int32, device=DEV)
    # the output sits inside a larger buffer whose other words must stay untouched
    big = torch.full((2 * 3 * 512 + 128,), 77, dtype=torch.int32, device=DEV)
    out = big[64:64 + 2 * 3 * 512].view(2, 3, 512)
    ret = flag_attn.topk_indices(view, lens, 512, causal=True, out=out)
    assert ret.data_ptr() == out.data_ptr()
    want = tko.topk_indices_ref(view.cpu().numpy(), [7000, 5000], 512, True)
    assert np.array_equal(out.cpu().numpy(), want)
    rest = big.cpu().numpy()
    assert (rest[:64] == 77).all() and (rest[64 + 2 * 3 * 512:] == 77).all()


def test_sparse_benchmark_shape():
    """B = 128, one query token, 65536 scores per row, top-2048 (the fp8 sparse benchmark's
    index shape), with a few sequences shorter than topk."""
    need_gpu()
    gen = torch.Generator().manual_seed(5)
    scores = torch.randn((128, 1, 65536), generator=gen)
    lens = [65536] * 120 + [65000, 40000, 2048, 2047, 100, 0, 65536, 30000]
    _run(scores, lens, 2048, causal=False)


def test_indices_drive_sparse_decode():
    """The produced indices are what flash_mla_with_kvcache(indices=...) takes: a decode over
    them equals one over the oracle's indices bit for bit (same kernel, same input)."""
    need_gpu()
    from oracle import mla_oracle as orc
    gen = torch.Generator().manual_seed(3)
    b, s_q, h_q, topk = 2, 2, 16, 256
    lens = [1500, 900]
    q, kc, bt, lens_t = orc.make_dense_inputs(b, h_q, s_q, lens, seed=3)
    scores = torch.randn((b, s_q, 1500), generator=gen)
    ld = torch.tensor(lens, dtype=torch.int32, device=DEV)
    idx = flag_attn.topk_indices(scores.to(DEV), ld, topk, causal=True)
    ref_idx = torch.from_numpy(tko.topk_indices_ref(scores.numpy(), lens, topk, True))
    assert torch.equal(idx.cpu(), ref_idx)
    md, ns = flag_attn.get_mla_metadata(ld, s_q * h_q, 1, num_heads_q=h_q, topk=topk)
    qd, kd, btd = q.to(DEV), kc.to(DEV), bt.to(DEV)
    o1, l1 = flag_attn.flash_mla_with_kvcache(qd, kd, btd, ld, 512, md, ns, 576 ** -0.5,
                                              indices=idx)
    ref_out, ref_lse = orc.sparse_decode_ref(q, kc, bt, lens_t, ref_idx, 576 ** -0.5)
    torch.cuda.synchronize()
    assert (o1.cpu().float() - ref_out).abs().max() < 2e-2
    assert (l1.cpu() - ref_lse).abs().max() < 1e-3


def test_c_abi_without_workspace_matches_two_stage():
    """fa_mla_topk_indices with no workspace runs the single-stage path; a long row gives
    the same indices as the two-stage path the Python operator takes."""
    need_gpu()
    from flagattention_amd import _lib
    lib = _lib.load()
    gen = torch.Generator().manual_seed(21)
    scores = torch.randn((3, 1, 65536), generator=gen).to(DEV)
    lens = torch.tensor([65536, 40000, 20000], dtype=torch.int32, device=DEV)
    assert lib.fa_mla_topk_workspace_bytes(3, 1, 65536, 2048) > 0
    two = flag_attn.topk_indices(scores, lens, 2048)
    one = torch.empty_like(two)
    _lib.check(lib.fa_mla_topk_indices(scores.data_ptr(), 65536, 65536, lens.data_ptr(), 3, 1,
                                       65536, 2048, 0, one.data_ptr(), None, 0,
                                       torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    assert torch.equal(one.cpu(), two.cpu())
    want = tko.topk_indices_ref(scores.cpu().numpy(), [65536, 40000, 20000], 2048, False)
    assert np.array_equal(one.cpu().numpy(), want)


@pytest.mark.parametrize("length,topk", [(65536, 8192), (40000, 6000), (20000, 5000)])
@pytest.mark.parametrize("kind", ["random", "int"])
def test_two_stage_large_topk(length, topk, kind):
    """Two-stage plans whose top-k exceeds what the chunk and merge kernels stage in LDS
    (4096 slots): both then take their range-checked direct-store paths."""
    from flagattention_amd import _lib
    need_gpu()
    assert _lib.load().fa_mla_topk_workspace_bytes(2, 2, length, topk) > 0  # two stages
    gen = torch.Generator().manual_seed(length + topk)
    if kind == "random":
        scores = torch.randn((2, 2, length), generator=gen)
    else:
        scores = torch.randint(-4, 4, (2, 2, length), generator=gen).float()
    _run(scores, [length, length - 3000], topk, causal=True)


@pytest.mark.parametrize("high", [[2], [0, 3], [1, 2, 3]])
@pytest.mark.parametrize("kind", ["shift", "const"])
def test_two_stage_concentrated_chunks(high, kind):
    """Whole chunks (16384 scores) of large scores -- shifted normal ones, or one constant:
    the row's top-k then lies in one to three chunks (with the constant, as the lowest
    positions of the first such chunk), and the other chunks' candidates all lose."""
    gen = torch.Generator().manual_seed(sum(high))
    scores = torch.randn((2, 1, 65536), generator=gen)
    for c in high:
        if kind == "shift":
            scores[:, 0, c * 16384:(c + 1) * 16384] += 50.0
        else:
            scores[:, 0, c * 16384:(c + 1) * 16384] = 50.0
    _run(scores, [65536, 60000], 2048, causal=False)
