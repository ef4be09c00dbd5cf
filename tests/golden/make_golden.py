"""Generate the golden fixtures under tests/golden/ (run from the repo root:
``python tests/golden/make_golden.py``).

The expected outputs are computed by a float64 brute force written independently of
``oracle/mla_oracle.py``: explicit Python loops over sequences, query rows and keys, a
per-token page walk for the gather (the loop form of ``src/flag_attn/testing/paged.py:37-50``),
textbook softmax attention (``src/flag_attn/testing/flash.py:47-75``: causal keeps
``m + (N - M) >= n``; lse is the natural-log normaliser), and the fp8-e4m3 decode from the
bit layout.  The oracle is then tested against these files, so a slip in either shows up.

Inputs are drawn from fixed seeds with numpy's PCG64 and stored in the files, so the
fixtures do not depend on any RNG at test time.
"""
from __future__ import annotations

import math
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
PAGE = 64


def bf16_round(x: np.ndarray) -> np.ndarray:
    """Round float32 values to the nearest bfloat16 (ties to even), kept as float32."""
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32)


def fp8_decode(code: int) -> float:
    s = -1.0 if code & 0x80 else 1.0
    e = (code >> 3) & 0xF
    m = code & 7
    if e == 0xF and m == 7:
        return math.nan
    if e == 0:
        return s * m / 8.0 * 2.0 ** -6
    return s * (1.0 + m / 8.0) * 2.0 ** (e - 7)


def fp8_encode(x: float) -> int:
    """Nearest e4m3 code (ties to even code), saturating at +-448."""
    best, bestd = 0, math.inf
    for c in range(256):
        v = fp8_decode(c)
        if math.isnan(v):
            continue
        d = abs(v - x)
        if d < bestd or (d == bestd and (c & 1) == 0 and (best & 1) == 1):
            best, bestd = c, d
    return best


def attend(qrow: np.ndarray, keys: list, vals: list, scale: float):
    """float64 softmax attention of one query row over explicit key/value lists."""
    if not keys:
        return np.zeros(512), -math.inf
    sc = [float(np.dot(qrow, k)) * scale for k in keys]
    mx = max(sc)
    w = [math.exp(x - mx) for x in sc]
    tot = sum(w)
    out = np.zeros(512)
    for wi, v in zip(w, vals):
        out += wi * v
    return out / tot, mx + math.log(tot)


def page_walk(cache: np.ndarray, bt: np.ndarray, b: int, j: int) -> np.ndarray:
    return cache[int(bt[b, j // PAGE]), j % PAGE, 0]


def dense_case(name, batch, h_q, s_q, lens, causal, seed, scale, extra_blocks=2):
    rng = np.random.Generator(np.random.PCG64(seed))
    nblk = [-(-n // PAGE) for n in lens]
    pool = sum(nblk) + extra_blocks
    perm = rng.permutation(pool).astype(np.int32)
    bt = np.zeros((batch, max(nblk)), dtype=np.int32)
    off = 0
    for b, n in enumerate(nblk):
        bt[b, :n] = perm[off:off + n]
        off += n
    q = bf16_round(rng.standard_normal((batch, s_q, h_q, 576)).astype(np.float32))
    cache = bf16_round(rng.standard_normal((pool, PAGE, 1, 576)).astype(np.float32))
    out = np.zeros((batch, s_q, h_q, 512))
    lse = np.full((batch, h_q, s_q), -math.inf)
    for b in range(batch):
        n = lens[b]
        rows = [page_walk(cache, bt, b, j).astype(np.float64) for j in range(n)]
        for s in range(s_q):
            vis = n - s_q + 1 + s if causal else n
            keys = rows[:max(vis, 0)]
            vals = [r[:512] for r in keys]
            for h in range(h_q):
                o, l = attend(q[b, s, h].astype(np.float64), keys, vals, scale)
                out[b, s, h] = o
                lse[b, h, s] = l
    np.savez_compressed(os.path.join(HERE, name), q=q, k_cache=cache, block_table=bt,
                        cache_seqlens=np.array(lens, dtype=np.int32), causal=np.array(causal),
                        sm_scale=np.array(scale), out=out, lse=lse)


def sparse_case(name, batch, h_q, s_q, lens, topk, seed, scale, fp8):
    rng = np.random.Generator(np.random.PCG64(seed))
    nblk = [-(-n // PAGE) for n in lens]
    pool = sum(nblk) + 1
    perm = rng.permutation(pool).astype(np.int32)
    bt = np.zeros((batch, max(nblk)), dtype=np.int32)
    off = 0
    for b, n in enumerate(nblk):
        bt[b, :n] = perm[off:off + n]
        off += n
    q = bf16_round(rng.standard_normal((batch, s_q, h_q, 576)).astype(np.float32))
    if fp8:
        raw = np.zeros((pool, PAGE, 1, 656), dtype=np.uint8)
        lat = rng.standard_normal((pool, PAGE, 512)) * 0.5
        sc = np.exp(rng.uniform(math.log(1e-2), math.log(1.0), (pool, PAGE, 4))).astype(np.float32)
        rope = bf16_round(rng.standard_normal((pool, PAGE, 64)).astype(np.float32))
        dec = np.zeros((pool, PAGE, 1, 576))
        for pg in range(pool):
            for r in range(PAGE):
                for d in range(512):
                    c = fp8_encode(float(lat[pg, r, d]) / float(sc[pg, r, d // 128]))
                    raw[pg, r, 0, d] = c
                    dec[pg, r, 0, d] = fp8_decode(c) * float(sc[pg, r, d // 128])
                raw[pg, r, 0, 512:528] = np.frombuffer(sc[pg, r].tobytes(), dtype=np.uint8)
                bits = (rope[pg, r].view(np.uint32) >> 16).astype(np.uint16)
                raw[pg, r, 0, 528:656] = np.frombuffer(bits.tobytes(), dtype=np.uint8)
                dec[pg, r, 0, 512:] = rope[pg, r]
        cache_store, cache_val = raw, dec
    else:
        cache_store = bf16_round(rng.standard_normal((pool, PAGE, 1, 576)).astype(np.float32))
        cache_val = cache_store.astype(np.float64)
    idx = np.full((batch, s_q, topk), -1, dtype=np.int32)
    for b in range(batch):
        for s in range(s_q):
            pick = rng.permutation(lens[b])[:topk]
            idx[b, s, :len(pick)] = pick
    drop = rng.random(idx.shape) < 0.1
    idx[drop] = -1
    idx[0, 0, 0] = lens[0]  # out of range -> masked
    idx[0, 0, 1] = -7       # negative -> masked
    topk_pad = -(-topk // PAGE) * PAGE
    rows = np.full((batch, s_q, topk_pad), -1, dtype=np.int32)
    out = np.zeros((batch, s_q, h_q, 512))
    lse = np.full((batch, h_q, s_q), -math.inf)
    for b in range(batch):
        for s in range(s_q):
            keys = []
            for j in range(topk):
                i = int(idx[b, s, j])
                if 0 <= i < lens[b]:
                    rows[b, s, j] = int(bt[b, i // PAGE]) * PAGE + i % PAGE
                    keys.append(page_walk(cache_val, bt, b, i))
            vals = [k[:512] for k in keys]
            for h in range(h_q):
                o, l = attend(q[b, s, h].astype(np.float64), keys, vals, scale)
                out[b, s, h] = o
                lse[b, h, s] = l
    np.savez_compressed(os.path.join(HERE, name), q=q, k_cache=cache_store, block_table=bt,
                        cache_seqlens=np.array(lens, dtype=np.int32), indices=idx, rows=rows,
                        sm_scale=np.array(scale), out=out, lse=lse)


def fp8_table_case(name):
    codes = np.arange(256)
    vals = np.array([fp8_decode(int(c)) for c in codes])
    np.savez_compressed(os.path.join(HERE, name), codes=codes, values=vals)


def combine_case(name, seed):
    """Split partials of a 3-way key partition and the unsplit attention they combine to."""
    rng = np.random.Generator(np.random.PCG64(seed))
    q = rng.standard_normal((4, 576))
    keys = rng.standard_normal((50, 576))
    scale = 192 ** -0.5
    cuts = [0, 13, 13, 50]  # middle split is empty
    o_parts = np.zeros((3, 4, 512))
    lse_parts = np.zeros((3, 4))
    for si in range(3):
        kk = [keys[j] for j in range(cuts[si], cuts[si + 1])]
        for r in range(4):
            o, l = attend(q[r], kk, [k[:512] for k in kk], scale)
            o_parts[si, r] = o
            lse_parts[si, r] = l
    out = np.zeros((4, 512))
    lse = np.zeros(4)
    for r in range(4):
        o, l = attend(q[r], list(keys), [k[:512] for k in keys], scale)
        out[r] = o
        lse[r] = l
    np.savez_compressed(os.path.join(HERE, name), o_parts=o_parts, lse_parts=lse_parts,
                        out=out, lse=lse)


if __name__ == "__main__":
    # B=2, h_q=16, s_q=1, lens 256 / 384, sm_scale 192^-0.5
    dense_case("dense_cfg1.npz", 2, 16, 1, [256, 384], False, 1, 192 ** -0.5, extra_blocks=0)
    # causal multi-token (s_q = 2) with ragged lengths, a 1-token and a 65-token sequence
    dense_case("dense_causal_sq2.npz", 3, 8, 2, [70, 1, 129], True, 2, 192 ** -0.5)
    sparse_case("sparse_bf16.npz", 2, 8, 2, [150, 300], 100, 3, 192 ** -0.5, fp8=False)
    sparse_case("sparse_fp8.npz", 2, 8, 1, [100, 70], 80, 4, 192 ** -0.5, fp8=True)
    fp8_table_case("fp8_e4m3fn_table.npz")
    combine_case("combine_3way.npz", 5)
    print("golden fixtures written to", HERE)
