"""Pins of the CPU oracle (oracle/mla_oracle.py) -- CPU only.

The reference ships no golden vectors for this path, so the oracle is pinned by
(1) the float64 brute-force fixtures in tests/golden (independent code),
(2) closed forms that fix the answer, and (3) a library decoder (torch.float8_e4m3fn).
Mutation tests plant a plausible mistake in a copy of an oracle step and check the pins
catch it.
"""
import math
import os

import numpy as np
import pytest
import torch

from oracle import mla_oracle as orc

SCALE = 192 ** -0.5


def _load(golden_dir, name):
    return np.load(os.path.join(golden_dir, name), allow_pickle=False)


def _t(a, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a))
    return t if dtype is None else t.to(dtype)


# ---------------------------------------------------------------- fp8 codec

def test_fp8_table_matches_golden_and_torch(golden_dir):
    g = _load(golden_dir, "fp8_e4m3fn_table.npz")
    tab = orc.fp8_e4m3fn_table()
    gv = g["values"].astype(np.float32)
    assert np.array_equal(np.isnan(tab), np.isnan(gv))
    m = ~np.isnan(gv)
    assert np.array_equal(tab[m], gv[m])
    lib = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float().numpy()
    assert np.array_equal(np.isnan(tab), np.isnan(lib))
    assert np.array_equal(tab[m], lib[m])
    # spot values of the OCP e4m3fn format
    assert tab[0x7E] == 448.0 and tab[0x01] == 2.0 ** -9 and tab[0x38] == 1.0
    assert np.isnan(tab[0x7F]) and np.isnan(tab[0xFF]) and tab[0x80] == 0.0


def test_fp8_row_roundtrip():
    gen = torch.Generator().manual_seed(0)
    lat = torch.randn((3, 512), generator=gen)
    scales = torch.tensor([[0.01, 0.02, 0.05, 0.1]] * 3)
    rope = torch.randn((3, 64), generator=gen).to(torch.bfloat16)
    raw = orc.fp8_rows_quantize(lat, rope, scales)
    assert raw.shape == (3, 656) and raw.dtype == torch.uint8
    dec = orc.fp8_rows_dequant(raw)
    # rope bytes pass through exactly
    assert torch.equal(dec[:, 512:], rope.float())
    # latent error <= half an e4m3 step (relative 2^-4) of |x|, times the scale
    s = scales.repeat_interleave(128, dim=1)
    err = (dec[:, :512] - lat).abs()
    bound = torch.maximum(lat.abs() * 2.0 ** -4, s * 2.0 ** -10)
    assert bool((err <= bound + 1e-7).all())


# ---------------------------------------------------------------- dense attention

def _dense_from_golden(g):
    q = _t(g["q"])
    kc = _t(g["k_cache"])
    bt = _t(g["block_table"])
    lens = _t(g["cache_seqlens"])
    return q, kc, bt, lens


@pytest.mark.parametrize("name", ["dense_cfg1.npz", "dense_causal_sq2.npz"])
def test_dense_oracle_matches_golden(golden_dir, name):
    g = _load(golden_dir, name)
    q, kc, bt, lens = _dense_from_golden(g)
    out, lse = orc.dense_decode_ref(q, kc, bt, lens, float(g["sm_scale"]), bool(g["causal"]))
    assert np.allclose(out.numpy(), g["out"], atol=2e-5, rtol=1e-4)
    gl = g["lse"]
    assert np.array_equal(np.isinf(lse.numpy()), np.isinf(gl))
    fin = np.isfinite(gl)
    assert np.allclose(lse.numpy()[fin], gl[fin], atol=2e-5)


def test_dense_mutation_causal_alignment_is_caught(golden_dir):
    """Top-left instead of bottom-right causal alignment must fail the golden pin."""
    g = _load(golden_dir, "dense_causal_sq2.npz")
    q, kc, bt, lens = _dense_from_golden(g)
    b = 0
    n = int(lens[b])
    kv = orc.gather_rows(kc, bt, b, torch.arange(n)).float()
    qb = q[b].float().permute(1, 0, 2)
    s = torch.matmul(qb, kv.t()) * float(g["sm_scale"])
    m = qb.shape[1]
    wrong = torch.arange(m).unsqueeze(-1) >= torch.arange(n)  # top-left
    lse_wrong = torch.logsumexp(torch.where(wrong, s, torch.tensor(-math.inf)), -1)
    assert not np.allclose(lse_wrong.numpy(), g["lse"][b], atol=1e-3)


def test_dense_mutation_gather_offset_is_caught(golden_dir):
    """Reading page row j % 64 of page j // 64 of the *unpermuted* pool must fail."""
    g = _load(golden_dir, "dense_cfg1.npz")
    q, kc, bt, lens = _dense_from_golden(g)
    ident = torch.zeros_like(bt)
    off = 0
    for b, n in enumerate(lens.tolist()):
        nb = -(-n // 64)
        ident[b, :nb] = torch.arange(off, off + nb, dtype=torch.int32)
        off += nb
    out, _ = orc.dense_decode_ref(q, kc, ident, lens, float(g["sm_scale"]))
    assert not np.allclose(out.numpy(), g["out"], atol=1e-2)


def test_dense_mutation_missing_scale_is_caught(golden_dir):
    g = _load(golden_dir, "dense_cfg1.npz")
    q, kc, bt, lens = _dense_from_golden(g)
    _, lse = orc.dense_decode_ref(q, kc, bt, lens, 1.0)
    assert not np.allclose(lse.numpy(), g["lse"], atol=1e-2)


def test_identity_table_gather_is_contiguous_slice():
    kc = torch.randn((4, 64, 1, 576))
    bt = torch.arange(4, dtype=torch.int32).view(1, 4)
    rows = orc.gather_rows(kc, bt, 0, torch.arange(200))
    assert torch.equal(rows, kc.reshape(256, 576)[:200])


def test_closed_form_equal_keys():
    """All keys equal: out = v, lse = q.k * scale + ln N."""
    q = torch.randn((3, 1, 576), dtype=torch.float64)
    k = torch.randn((576,), dtype=torch.float64).repeat(37, 1)
    out, lse = orc.attention_lse(q, k, k[:, :512], SCALE, False)
    assert torch.allclose(out[:, 0], k[0, :512].float().expand(3, 512), atol=1e-5)
    want = (q[:, 0].float() @ k[0].float()) * SCALE + math.log(37)
    assert torch.allclose(lse[:, 0], want, atol=1e-4)


def test_closed_form_zero_query_is_mean():
    k = torch.randn((50, 576))
    q = torch.zeros((2, 1, 576))
    out, lse = orc.attention_lse(q, k, k[:, :512], SCALE, False)
    assert torch.allclose(out[:, 0], k[:, :512].mean(0).expand(2, 512), atol=1e-5)
    assert torch.allclose(lse, torch.full_like(lse, math.log(50)), atol=1e-6)


def test_closed_form_single_key_and_empty():
    k = torch.randn((1, 576))
    q = torch.randn((2, 1, 576))
    out, lse = orc.attention_lse(q, k, k[:, :512], SCALE, False)
    assert torch.allclose(out[:, 0], k[0, :512].expand(2, 512))
    assert torch.allclose(lse[:, 0], (q[:, 0] @ k[0]) * SCALE, atol=1e-5)
    out, lse = orc.attention_lse(q, k[:0], k[:0, :512], SCALE, False)
    assert torch.equal(out, torch.zeros_like(out)) and bool(torch.isneginf(lse).all())


def test_causal_equals_truncated_keys():
    k = torch.randn((40, 576))
    q = torch.randn((4, 3, 576))
    out, lse = orc.attention_lse(q, k, k[:, :512], SCALE, True)
    for m in range(3):
        n = 40 - 3 + 1 + m
        o2, l2 = orc.attention_lse(q[:, m:m + 1], k[:n], k[:n, :512], SCALE, False)
        assert torch.allclose(out[:, m], o2[:, 0], atol=1e-5)
        assert torch.allclose(lse[:, m], l2[:, 0], atol=1e-5)


def test_attention_matches_library_sdpa():
    """A textbook-routine special case: torch's scaled_dot_product_attention in float64."""
    q = torch.randn((4, 2, 576), dtype=torch.float64)
    k = torch.randn((70, 576), dtype=torch.float64)
    out, _ = orc.attention_lse(q, k, k[:, :512], SCALE, False)
    ref = torch.nn.functional.scaled_dot_product_attention(
        q.unsqueeze(0), k.unsqueeze(0).unsqueeze(0).expand(1, 4, 70, 576),
        k[:, :512].unsqueeze(0).unsqueeze(0).expand(1, 4, 70, 512), scale=SCALE)[0]
    assert torch.allclose(out.double(), ref, atol=1e-5)


# ---------------------------------------------------------------- sparse

@pytest.mark.parametrize("name,fp8", [("sparse_bf16.npz", False), ("sparse_fp8.npz", True)])
def test_sparse_oracle_matches_golden(golden_dir, name, fp8):
    g = _load(golden_dir, name)
    q = _t(g["q"])
    kc = _t(g["k_cache"])
    bt = _t(g["block_table"])
    lens = _t(g["cache_seqlens"])
    idx = _t(g["indices"])
    rows = orc.sparse_rows_ref(idx, bt, lens, kc.shape[0])
    assert torch.equal(rows, _t(g["rows"]))
    out, lse = orc.sparse_decode_ref(q, kc, bt, lens, idx, float(g["sm_scale"]), is_fp8=fp8)
    assert np.allclose(out.numpy(), g["out"], atol=2e-5, rtol=1e-4)
    assert np.allclose(lse.numpy(), g["lse"], atol=2e-5)


def test_sparse_full_index_set_equals_dense():
    q, kc, bt, lens = orc.make_dense_inputs(2, 8, 1, [100, 130], seed=7, dtype=torch.float32)
    idx = torch.full((2, 1, 130), -1, dtype=torch.int32)
    for b, n in enumerate([100, 130]):
        idx[b, 0, :n] = torch.randperm(n).to(torch.int32)
    o1, l1 = orc.sparse_decode_ref(q, kc, bt, lens, idx, SCALE)
    o2, l2 = orc.dense_decode_ref(q, kc, bt, lens, SCALE)
    assert torch.allclose(o1, o2, atol=1e-5) and torch.allclose(l1, l2, atol=1e-5)


def test_sparse_rows_masks_bad_pages():
    bt = torch.tensor([[0, 5, 99]], dtype=torch.int32)  # page 99 outside a 6-page cache
    lens = torch.tensor([192], dtype=torch.int32)
    idx = torch.tensor([[[0, 70, 130, 191, 192, -1]]], dtype=torch.int32)
    rows = orc.sparse_rows_ref(idx, bt, lens, 6)
    assert rows.shape == (1, 1, 64)
    assert rows[0, 0, :6].tolist() == [0, 5 * 64 + 6, -1, -1, -1, -1]
    assert bool((rows[0, 0, 6:] == -1).all())


# ---------------------------------------------------------------- combine

def test_combine_matches_golden_and_unsplit(golden_dir):
    g = _load(golden_dir, "combine_3way.npz")
    out, lse = orc.combine_ref(_t(g["o_parts"]), _t(g["lse_parts"]))
    assert np.allclose(out.numpy(), g["out"], atol=1e-5)
    assert np.allclose(lse.numpy(), g["lse"], atol=1e-5)


def test_combine_split_invariance_random_partitions():
    gen = torch.Generator().manual_seed(3)
    k = torch.randn((300, 576), generator=gen)
    q = torch.randn((5, 1, 576), generator=gen)
    full_o, full_l = orc.attention_lse(q, k, k[:, :512], SCALE, False)
    for cuts in ([0, 300], [0, 1, 300], [0, 64, 128, 299, 300], [0, 100, 100, 300]):
        parts_o, parts_l = [], []
        for a, b in zip(cuts[:-1], cuts[1:]):
            o, l = orc.attention_lse(q, k[a:b], k[a:b, :512], SCALE, False)
            parts_o.append(o[:, 0])
            parts_l.append(l[:, 0])
        o, l = orc.combine_ref(torch.stack(parts_o), torch.stack(parts_l))
        assert torch.allclose(o, full_o[:, 0], atol=1e-5)
        assert torch.allclose(l, full_l[:, 0], atol=1e-5)


def test_combine_all_empty():
    o, l = orc.combine_ref(torch.zeros((2, 3, 512)), torch.full((2, 3), -math.inf))
    assert torch.equal(o, torch.zeros_like(o)) and bool(torch.isneginf(l).all())


# ---------------------------------------------------------------- cache writer

def test_fp8_tile_scales_and_write_ref():
    """The writer's scale maps each tile's largest magnitude to the largest e4m3 code
    (0x7E / 0xFE = +-448), an all-zero tile gets scale 1 and zero codes, and the written
    row decodes to within half an e4m3 step of the input."""
    gen = torch.Generator().manual_seed(21)
    lat = torch.randn((5, 512), generator=gen).to(torch.bfloat16)
    lat[2, 128:256] = 0
    rope = torch.randn((5, 64), generator=gen).to(torch.bfloat16)
    sc = orc.fp8_tile_scales(lat)
    assert sc.shape == (5, 4) and float(sc[2, 1]) == 1.0
    cache = torch.zeros((1, 64, 1, 656), dtype=torch.uint8)
    slots = torch.tensor([3, 0, 63, -1, 7])
    out = orc.kvcache_write_ref(cache, lat, rope, slots, True)
    flat = out.view(64, 656)
    for i, s in enumerate(slots.tolist()):
        if s < 0:
            continue
        row = flat[s]
        codes = row[:512].view(4, 128)
        for t in range(4):
            tile = lat[i].float().view(4, 128)[t]
            if float(tile.abs().max()) > 0:
                assert int(codes[t, int(tile.abs().argmax())]) & 0x7F == 0x7E
        dec = orc.fp8_rows_dequant(row.view(1, 656))[0]
        assert torch.equal(dec[512:], rope[i].float())
        err = (dec[:512] - lat[i].float()).abs()
        bound = lat[i].float().abs() * 2.0 ** -4 + sc[i].repeat_interleave(128) * 2.0 ** -10
        assert bool((err <= bound).all())
    assert int(flat[1].sum()) == 0  # an unwritten row stays as it was
    # token 2 (slot 63) has its second tile all zero: codes zero, scale 1
    assert bool((flat[63][128:256] == 0).all())
    assert float(flat[63][512:528].view(torch.float32)[1]) == 1.0
    bf = orc.kvcache_write_ref(torch.zeros((1, 64, 1, 576), dtype=torch.bfloat16), lat, rope,
                               slots, False)
    assert torch.equal(bf.view(64, 576)[7], torch.cat([lat[4], rope[4]]))


def test_loop_gather_equals_vectorised_bit_for_bit(golden_dir):
    """The per-token loop restatement (the reference's testing/paged.py gather shape, used
    only as a CPU baseline) gives the vectorised oracle's bits, and both match the float64
    golden of the config-1 shape."""
    q, kc, bt, lens = orc.make_dense_inputs(3, 16, 1, [256, 1, 700], seed=11, scale=1.0)
    a_out, a_lse = orc.dense_decode_ref(q, kc, bt, lens, 192 ** -0.5)
    b_out, b_lse = orc.dense_decode_loop(q, kc, bt, lens, 192 ** -0.5)
    assert torch.equal(a_out, b_out) and torch.equal(a_lse, b_lse)
    g = _load(golden_dir, "dense_cfg1.npz")
    q, kc, bt, lens = _dense_from_golden(g)
    out, lse = orc.dense_decode_loop(q, kc, bt, lens, float(g["sm_scale"]))
    assert np.allclose(out.numpy(), g["out"], atol=2e-5, rtol=1e-4)
    assert np.allclose(lse.numpy(), g["lse"], atol=2e-5)
