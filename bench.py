"""MLA decode benchmark on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload dense|skew|sparse|sparse_fp8]
    python bench.py --workload gqa_paged|gqa_splitkv|gqa_paged_d512|topk|kvcache|kvcache_fp8
                                                           # the other decode-path kernels
    python bench.py --traffic-calibrate [--workload ...]   # driver for rocprofv3 --pmc passes

A step is one decode of the whole batch through the public path: scheduler metadata
(get_mla_metadata) + [sparse row translation] + decode + split combine, with every input
already resident in HBM (the line's ``step_kernels`` lists the launches).
The default workload is BASELINE config 2 (dense bf16, B=64, h_q=128, s_q=1, lengths
U[4096, 8192], 64-token pages through a permuted block table).  KV pools are rotated
between steps so consecutive steps do not hit the 256 MB last-level cache.  After the W
warm-up steps a settle phase runs further untimed steps until at least SETTLE_S seconds of
steps have run since the start of the warm-up (reported as ``settle_s``): with only a few
warm-up steps the GPU has not reached its steady clocks and the decode kernel runs ~20%
slower.

With no --workload (the default invocation) the line also carries `other_workloads`: every
other workload above, measured briefly in the same process after the flagship (OTHER_STEPS
timed steps each, no CPU baseline, an OTHER_SETTLE_S settle phase) -- its µs/step, its
kernel's mean time by events and roofline fraction -- so that one default run records every
workload; --no-extras skips it.

Prints one JSON line: value = wall-clock us/step (lower is better); `roofline` is the
decode kernel alone (HIP events around its launch on the launch stream, on every k-th
timed step, k = min(EVENT_EVERY, steps // MIN_EVENT_LAUNCHES) so that at least
MIN_EVENT_LAUNCHES launches are bracketed: an event pair costs each step it brackets a few
us of dispatch gap, which is charged to `value`), algorithmic bytes / FLOPs
per launch over its mean duration; `cpu_baseline` is the CPU oracle
(the reference's PyTorch math restated) timed on a bounded sample of the same workload.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

import torch  # noqa: E402

METRIC = "MLA decode µs/step + achieved HBM GB/s & MFMA TFLOPS (% of roofline), B=64 h=128"
PEAK_HBM_GBS = 8000.0      # MI355X HBM3E
PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 MFMA
SCALE = 192 ** -0.5
PAGE = 64
EVENT_EVERY = 8  # at most this many timed steps per decode launch bracketed by events
MIN_EVENT_LAUNCHES = 10  # ...and at least this many bracketed launches
SETTLE_S = 0.25  # seconds of untimed steps (warm-up included) before the timed region
# ... for the other workloads of the default run: right after the compute-bound MLA steps a
# memory-bound one needs ~0.5 s of its own steps to reach its sustained rate (paged GQA
# measured 5% slow with 0.25 s, at its standalone rate with 0.5 s)
OTHER_SETTLE_S = 1.0
COPY_BYTES = 512 << 20  # calibration copy of --traffic-calibrate
# the default run (no --workload) also measures these, briefly, into `other_workloads`
OTHER_WORKLOADS = ("skew", "sparse", "sparse_fp8", "gqa_paged", "gqa_splitkv", "gqa_paged_d512",
                   "topk", "kvcache", "kvcache_fp8")
OTHER_STEPS, OTHER_WARMUP = 200, 100


def workload_spec(name: str) -> dict:
    if name == "dense":
        return dict(name="dense_bf16_cfg2", batch=64, h_q=128, s_q=1, causal=False,
                    lens=("uniform", 4096, 8192), topk=None, fp8=False, seed=2)
    if name == "skew":
        return dict(name="dense_bf16_skew_cfg3", batch=32, h_q=128, s_q=2, causal=True,
                    lens=("lognormal", 4096, 1.0, 128, 65536), topk=None, fp8=False, seed=3)
    if name == "sparse":
        return dict(name="sparse_bf16_top2048_cfg4", batch=64, h_q=128, s_q=1, causal=False,
                    lens=("const", 32768), topk=2048, fp8=False, seed=4)
    if name == "sparse_fp8":
        return dict(name="sparse_fp8_top2048_cfg5", batch=128, h_q=128, s_q=1, causal=False,
                    lens=("const", 65536), topk=2048, fp8=True, seed=5)
    raise SystemExit(f"unknown workload {name}")


def make_lens(spec, gen) -> torch.Tensor:
    kind = spec["lens"][0]
    b = spec["batch"]
    if kind == "uniform":
        return torch.randint(spec["lens"][1], spec["lens"][2] + 1, (b,), generator=gen,
                             dtype=torch.int32)
    if kind == "lognormal":
        _, med, sigma, lo, hi = spec["lens"]
        x = torch.exp(math.log(med) + sigma * torch.randn((b,), generator=gen))
        return x.round().clamp(lo, hi).to(torch.int32)
    return torch.full((b,), spec["lens"][1], dtype=torch.int32)


def build_inputs(spec, dev, copies):
    """Synthetic inputs on the GPU: q, `copies` KV pools (+ their block tables), lens,
    indices.  Values N(0,1)*0.1 in bf16 (fp8: quantised per 128-dim tile)."""
    gen = torch.Generator().manual_seed(spec["seed"])
    lens = make_lens(spec, gen)
    nblk = [-(-int(x) // PAGE) for x in lens]
    pool = sum(nblk)
    maxb = max(nblk)
    dgen = torch.Generator(device=dev).manual_seed(spec["seed"])
    q = (torch.randn((spec["batch"], spec["s_q"], spec["h_q"], 576), generator=dgen,
                     device=dev) * 0.1).to(torch.bfloat16)
    pools, tables = [], []
    for _ in range(copies):
        perm = torch.randperm(pool, generator=gen).to(torch.int32)
        bt = torch.zeros((spec["batch"], maxb), dtype=torch.int32)
        off = 0
        for b, n in enumerate(nblk):
            bt[b, :n] = perm[off:off + n]
            off += n
        tables.append(bt.to(dev))
        if spec["fp8"]:
            kc = torch.empty((pool, PAGE, 1, 656), dtype=torch.uint8, device=dev)
            chunk = 1024
            for c0 in range(0, pool, chunk):
                c1 = min(pool, c0 + chunk)
                lat = torch.randn((c1 - c0, PAGE, 1, 512), generator=dgen, device=dev) * 0.1
                u = torch.rand((c1 - c0, PAGE, 1, 4), generator=dgen, device=dev)
                sc = torch.exp(math.log(1e-3) + u * (math.log(1e-1) - math.log(1e-3)))
                codes = (lat.view(c1 - c0, PAGE, 1, 4, 128) / sc.unsqueeze(-1)).clamp(-448, 448)
                codes = codes.to(torch.float8_e4m3fn).view(torch.uint8).view(c1 - c0, PAGE, 1, 512)
                rope = (torch.randn((c1 - c0, PAGE, 1, 64), generator=dgen, device=dev)
                        * 0.1).to(torch.bfloat16)
                kc[c0:c1] = torch.cat([codes, sc.contiguous().view(torch.uint8),
                                       rope.view(torch.uint8)], dim=-1)
        else:
            kc = (torch.randn((pool, PAGE, 1, 576), generator=dgen, device=dev) * 0.1).to(
                torch.bfloat16)
        pools.append(kc)
    indices = None
    if spec["topk"]:
        topk = spec["topk"]
        b, s_q = spec["batch"], spec["s_q"]
        n = int(lens[0])
        r = torch.rand((b * s_q, n), generator=dgen, device=dev)
        indices = torch.topk(r, topk, dim=1).indices.to(torch.int32).view(b, s_q, topk)
        drop = torch.rand((b, s_q, topk), generator=dgen, device=dev) < 0.02
        indices = torch.where(drop, torch.full_like(indices, -1), indices).contiguous()
    return q, pools, tables, lens.to(dev), indices


def algorithmic_work(spec, lens_cpu, indices) -> tuple:
    """HBM bytes and FLOPs one decode launch must move / compute: every KV row it
    attends to once, q in, out (or the split partial) and lse out, and the block-table
    words (dense) or translated row ids (sparse) that address the rows; FLOPs of QK (576)
    and PV (512) per row and head."""
    b, s_q, h_q = spec["batch"], spec["s_q"], spec["h_q"]
    row_bytes = 656 if spec["fp8"] else 1152
    if spec["topk"]:
        n_valid = int((indices >= 0).sum())  # per (b, s) token lists
        kv_rows = n_valid
        table = indices.numel() * 4  # the translated row ids
        flops_rows = n_valid  # each valid (b, s, token) pair meets h_q heads once
    else:
        kv_rows = int(lens_cpu.sum())
        table = sum(-(-int(x) // PAGE) for x in lens_cpu) * 4
        flops_rows = kv_rows * s_q
    nbytes = kv_rows * row_bytes + b * s_q * h_q * (576 * 2 + 512 * 2 + 4) + table
    flops = flops_rows * h_q * 2 * (576 + 512)
    return nbytes, flops


# The sources each timed kernel is compiled from (its translation unit and the headers
# it includes); a traffic record holds only while these are unchanged.
_SHARED = ("flagattention_amd/csrc/fa_common.h", "flagattention_amd/csrc/fa_wave.h",
           "include/flagattention_amd.h")
DECODE_SOURCES = ("flagattention_amd/csrc/fa_decode.hip",) + _SHARED
KERNEL_SOURCES = {
    "mla_decode": DECODE_SOURCES,
    "gqa_decode": ("flagattention_amd/csrc/fa_gqa_decode.hip",) + _SHARED,
    "topk": ("flagattention_amd/csrc/fa_topk.hip",) + _SHARED,
    "kvcache": ("flagattention_amd/csrc/fa_kvcache.hip",) + _SHARED,
}


def kernel_sources_sha(family: str = "mla_decode") -> str:
    """sha256 (16 hex) over a kernel family's sources, as recorded in profiles/."""
    import hashlib
    h = hashlib.sha256()
    for rel in KERNEL_SOURCES[family]:
        h.update(rel.encode())
        with open(os.path.join(ROOT, rel), "rb") as fh:
            h.update(fh.read())
    return h.hexdigest()[:16]


def recorded_traffic(workload_name: str, family: str = "mla_decode"):
    """HBM bytes per launch of the timed kernel(s) measured with rocprofv3 FETCH_SIZE +
    WRITE_SIZE (copy-calibrated, profiles/traffic.json) -- only if recorded for these exact
    kernel sources; otherwise None."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    if not os.path.exists(path):
        return None
    with open(path) as fh:
        rec = json.load(fh).get(workload_name)
    if not rec or rec.get("csrc_sha") != kernel_sources_sha(family):
        return None
    return int(rec["hbm_read_bytes"]) + int(rec["hbm_write_bytes"])


TRAFFIC_SOURCE = "profiles/traffic.json (rocprofv3 FETCH_SIZE+WRITE_SIZE, copy-calibrated)"


def with_traffic_source(rec: dict) -> dict:
    """Names where a measured `traffic` comes from."""
    if rec["roofline"].get("traffic") is not None:
        rec["roofline"]["traffic_source"] = TRAFFIC_SOURCE
    return rec


def settle_seconds(args) -> float:
    """The settle phase's length: SETTLE_S, or the run's own (other workloads)."""
    return getattr(args, "settle_s", SETTLE_S)


def calibrate_then(step, args, name: str) -> None:
    """--traffic-calibrate: the 512 MiB device copy whose counter values scale the kernel's,
    then --settle-launches + --launches steps (the profiler's counter passes)."""
    dev = torch.device("cuda:0")
    src = torch.empty(COPY_BYTES // 4, dtype=torch.float32, device=dev).normal_()
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    for i in range(args.settle_launches + args.launches):
        step(i)
    torch.cuda.synchronize()
    print(f"copy_bytes={COPY_BYTES} workload={name} settle_launches={args.settle_launches} "
          f"launches={args.launches}", flush=True)


def cpu_baseline(spec, q, pool, table, lens, indices) -> dict:
    """The oracle (fp32 PyTorch restatement of the reference's CPU path) on a bounded
    sample of the workload's sequences, scaled to a full step."""
    from oracle import mla_oracle as orc

    torch.set_num_threads(os.cpu_count() or 1)
    b = spec["batch"]
    sample = 1
    lens_c = lens.cpu()
    sel = list(range(b))

    def run(nseq):
        idx = sel[:nseq]
        need = torch.unique(table[idx].flatten()).long()
        # copy only the pages these sequences use, then remap the table
        remap = torch.full((pool.shape[0],), -1, dtype=torch.long, device=pool.device)
        remap[need] = torch.arange(need.numel(), device=pool.device)
        kc = pool[need].cpu()
        bt = remap[table[idx].long()].to(torch.int32).cpu()
        qc = q[idx].cpu()
        t0 = time.perf_counter()
        if spec["topk"]:
            orc.sparse_decode_ref(qc, kc, bt, lens_c[idx], indices[idx].cpu(), SCALE,
                                  is_fp8=spec["fp8"])
        else:
            orc.dense_decode_ref(qc, kc, bt, lens_c[idx], SCALE, spec["causal"])
        return time.perf_counter() - t0

    t1 = run(1)
    sample = max(1, min(b, int(15.0 / max(t1, 1e-3))))
    times = [run(sample) for _ in range(3)]
    t = sorted(times)[1]
    us_step = t / sample * b * 1e6
    rec = {"value": round(us_step, 1), "unit": "µs/step", "cores": torch.get_num_threads(),
           "kind": "port",
           "sample": f"{sample} of {b} sequences of {spec['name']}, median of 3, "
                     f"scaled x{b / sample:.2f} to the full step"}
    if not spec["topk"] and not spec["causal"]:
        rec["loop_variant"] = cpu_loop_baseline(spec, q, pool, table, lens)
    return rec


def cpu_loop_baseline(spec, q, pool, table, lens) -> dict:
    """The same oracle with the gather written as the reference's testing/paged.py:37-52
    writes it (one Python iteration per token): on one sequence of the workload, scaled to
    the full batch, and on BASELINE config 1's shape (B=2, 16 heads, lengths 256 and 384)."""
    from oracle import mla_oracle as orc

    b = spec["batch"]
    need = torch.unique(table[:1].flatten()).long()
    remap = torch.full((pool.shape[0],), -1, dtype=torch.long, device=pool.device)
    remap[need] = torch.arange(need.numel(), device=pool.device)
    args = (q[:1].cpu(), pool[need].cpu(), remap[table[:1].long()].to(torch.int32).cpu(),
            lens[:1].cpu(), SCALE)
    orc.dense_decode_loop(*args)
    t0 = time.perf_counter()
    orc.dense_decode_loop(*args)
    t_seq = time.perf_counter() - t0
    c1 = orc.make_dense_inputs(2, 16, 1, [256, 384], seed=1, scale=1.0, dtype=torch.float32)
    orc.dense_decode_loop(*c1, SCALE)
    t0 = time.perf_counter()
    orc.dense_decode_loop(*c1, SCALE)
    t_c1 = time.perf_counter() - t0
    return {"value": round(t_seq * b * 1e6, 1), "unit": "µs/step",
            "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"1 of {b} sequences ({int(lens[0])} tokens), per-token loop gather, "
                      f"scaled x{b}",
            "config1_us": round(t_c1 * 1e6, 1)}


# Grouped-query decode workloads (flag_attn.paged_attention / flash_attention decode), the
# shapes of the reference's benchmark/paged_benchmark.py (64 query heads, group 8, head dim
# 128, 16-token blocks, fp16; the largest batch, context 8192) and
# benchmark/flash_decoding_benchmark.py (batch 2, 2048 / D heads, one query, long context).
GQA_WORKLOADS = {
    "gqa_paged": dict(name="gqa_paged_b64_h64_g8_d128_ctx8192", kind="paged", batch=64, h_q=64,
                      group=8, d=128, block=16, ctx=8192, seed=11),
    "gqa_splitkv": dict(name="gqa_splitkv_b2_h16_d128_ctx262144", kind="splitkv", batch=2,
                        h_q=16, group=1, d=128, ctx=262144, seed=12),
    # head size 512 (the reference's largest paged_attention head size)
    "gqa_paged_d512": dict(name="gqa_paged_b64_h32_g8_d512_ctx4096", kind="paged", batch=64,
                           h_q=32, group=8, d=512, block=16, ctx=4096, seed=16),
}
GQA_METRIC = "GQA decode µs/step + achieved HBM GB/s (% of roofline)"


def run_gqa(args) -> dict:
    """Grouped-query decode bench: inputs resident in HBM, the KV pool sized to the keys
    the step reads (a permuted block table for the paged cache) and rotated between two
    copies; the roofline kernel is the decode kernel alone (events around its launch)."""
    import flag_attn
    from flagattention_amd import gqa

    spec = GQA_WORKLOADS[args.workload]
    dev = torch.device("cuda:0")
    gen = torch.Generator().manual_seed(spec["seed"])
    dgen = torch.Generator(device=dev).manual_seed(spec["seed"])
    b, h_q, d, ctx = spec["batch"], spec["h_q"], spec["d"], spec["ctx"]
    h_kv = h_q // spec["group"]
    dt = torch.float16
    scale = d ** -0.5
    copies = []
    for _ in range(2):
        if spec["kind"] == "paged":
            bs = spec["block"]
            nblk = -(-ctx // bs)
            pool = b * nblk
            q = torch.empty((b, h_q, d), dtype=dt, device=dev).uniform_(-scale, scale,
                                                                        generator=dgen)
            kc = torch.empty((pool, h_kv, bs, d), dtype=dt, device=dev).uniform_(
                -scale, scale, generator=dgen)
            vc = torch.empty_like(kc).uniform_(-scale, scale, generator=dgen)
            bt = torch.randperm(pool, generator=gen).to(torch.int32).view(b, nblk).to(dev)
            lens = torch.full((b,), ctx, dtype=torch.int32, device=dev)
            copies.append((q, kc, vc, lens, bt))
        else:
            q = torch.randn((b, h_q, 1, d), generator=dgen, device=dev).to(dt)
            k = torch.randn((b, h_kv, ctx, d), generator=dgen, device=dev).to(dt)
            v = torch.randn((b, h_kv, ctx, d), generator=dgen, device=dev).to(dt)
            copies.append((q, k, v))

    def step(i, events=None):
        gqa.timing_events = events
        c = copies[i % 2]
        if spec["kind"] == "paged":
            q, kc, vc, lens, bt = c
            return flag_attn.paged_attention(q, kc, vc, lens, bt, scale, ctx)
        q, k, v = c
        return flag_attn.flash_attention(q, k, v, False)

    if args.traffic_calibrate:
        calibrate_then(step, args, spec["name"])
        return None
    t_warm = time.perf_counter()
    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    settle_steps = 0
    while time.perf_counter() - t_warm < settle_seconds(args):
        for _ in range(20):
            step(settle_steps)
            settle_steps += 1
        torch.cuda.synchronize()
    settle_s = time.perf_counter() - t_warm
    every = max(1, min(EVENT_EVERY, args.steps // MIN_EVENT_LAUNCHES))
    evs = {i: (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for i in range(0, args.steps, every)}
    t0 = time.perf_counter()
    for i in range(args.steps):
        step(i, evs.get(i))
    torch.cuda.synchronize()
    us_step = (time.perf_counter() - t0) / args.steps * 1e6
    dec = sorted(s.elapsed_time(e) for s, e in evs.values())
    dec_us = sum(dec) / len(dec) * 1e3
    kv_bytes = b * ctx * h_kv * d * 2 * 2
    nbytes = kv_bytes + 2 * b * h_q * d * 2 + (b * (-(-ctx // spec.get("block", ctx))) * 4
                                                  if spec["kind"] == "paged" else 0)
    flops = 2.0 * b * h_q * 2 * ctx * d  # QK and PV, as benchmark/paged_benchmark.py:198
    gbs = nbytes / (dec_us * 1e-6) / 1e9
    cpu = None
    if not args.no_cpu_baseline:
        cpu = gqa_cpu_baseline(spec, copies[0], scale)
    rec = {
        "metric": GQA_METRIC, "value": round(us_step, 2), "unit": "µs/step", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "settle_s": round(settle_s, 3),
        "settle_steps": settle_steps, "ms_per_step": round(us_step / 1e3, 5),
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None, "dtype": "fp16",
        "data": "synthetic",
        "config": {"workload": spec["name"], "batch": b, "h_q": h_q, "h_kv": h_kv, "d": d,
                   "ctx": ctx, "block_size": spec.get("block")},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS,
                     "unit": "GB/s", "frac": round(gbs / PEAK_HBM_GBS, 4),
                     "traffic": recorded_traffic(spec["name"], "gqa_decode"),
                     "kernel": "gqa_decode_wide_kernel" if d == 512 else "gqa_decode_kernel", "kernel_launches_timed": len(dec),
                     "kernel_us_mean": round(dec_us, 2), "bytes_per_launch": nbytes,
                     "flops_per_launch": flops,
                     "tflops": round(flops / (dec_us * 1e-6) / 1e12, 2)},
        "cpu_baseline": cpu,
    }
    return with_traffic_source(rec)


def gqa_cpu_baseline(spec, inputs, scale) -> dict:
    """The oracle (the reference's testing/paged.py and testing/flash.py math, restated)
    on one sequence of the workload, scaled to the full step."""
    from oracle import gqa_oracle as go

    torch.set_num_threads(os.cpu_count() or 1)
    b = spec["batch"]
    if spec["kind"] == "paged":
        q, kc, vc, lens, bt = inputs
        need = torch.unique(bt[:1].flatten()).long()
        remap = torch.full((kc.shape[0],), -1, dtype=torch.long, device=kc.device)
        remap[need] = torch.arange(need.numel(), device=kc.device)
        args = (q[:1].cpu(), kc[need].cpu(), vc[need].cpu(),
                remap[bt[:1].long()].to(torch.int32).cpu(), lens[:1].cpu(), scale)
        fn = lambda: go.paged_attention_ref(*args)  # noqa: E731
    else:
        q, k, v = inputs
        args = (q[:1].cpu(), k[:1].cpu(), v[:1].cpu())
        fn = lambda: go.flash_attention_ref(*args, False, upcast=True)  # noqa: E731
    fn()
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    t = sorted(times)[1]
    return {"value": round(t * b * 1e6, 1), "unit": "µs/step", "cores": torch.get_num_threads(),
            "kind": "port", "sample": f"1 of {b} sequences of {spec['name']}, median of 3, "
                                      f"scaled x{b} to the full step"}


# Top-k index producer workload (flag_attn.topk_indices): the index shape of the fp8 sparse
# benchmark -- 128 sequences, one query token, 65536 indexer scores each, top-2048.
TOPK_WORKLOADS = {
    "topk": dict(name="topk_b128_len65536_top2048", batch=128, s_q=1, length=65536,
                 topk=2048, seed=13),
}
TOPK_METRIC = "top-k index producer µs/step + achieved HBM GB/s (% of roofline)"


def run_topk(args) -> dict:
    """Index producer bench: fp32 scores resident in HBM (two copies rotated); a step is
    one flag_attn.topk_indices launch, timed with events around it on its stream."""
    import flag_attn

    spec = TOPK_WORKLOADS[args.workload]
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(spec["seed"])
    b, s_q, length, topk = spec["batch"], spec["s_q"], spec["length"], spec["topk"]
    scores = [torch.randn((b, s_q, length), generator=gen, device=dev) for _ in range(2)]
    lens = torch.full((b,), length, dtype=torch.int32, device=dev)
    out = torch.empty((b, s_q, topk), dtype=torch.int32, device=dev)

    def step(i):
        return flag_attn.topk_indices(scores[i % 2], lens, topk, out=out)

    if args.traffic_calibrate:
        calibrate_then(step, args, spec["name"])
        return None
    t_warm = time.perf_counter()
    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    settle_steps = 0
    while time.perf_counter() - t_warm < settle_seconds(args):
        for _ in range(20):
            step(settle_steps)
            settle_steps += 1
        torch.cuda.synchronize()
    settle_s = time.perf_counter() - t_warm
    every = max(1, min(EVENT_EVERY, args.steps // MIN_EVENT_LAUNCHES))
    stream = torch.cuda.current_stream()
    evs = {i: (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for i in range(0, args.steps, every)}
    t0 = time.perf_counter()
    for i in range(args.steps):
        ev = evs.get(i)
        if ev:
            ev[0].record(stream)
        step(i)
        if ev:
            ev[1].record(stream)
    torch.cuda.synchronize()
    us_step = (time.perf_counter() - t0) / args.steps * 1e6
    dec = sorted(s.elapsed_time(e) for s, e in evs.values())
    k_us = sum(dec) / len(dec) * 1e3
    nbytes = b * s_q * (length * 4 + topk * 4) + b * 4
    gbs = nbytes / (k_us * 1e-6) / 1e9
    cpu = None
    if not args.no_cpu_baseline:
        from oracle import topk_oracle as tko
        rows = 8
        sample = scores[0][:rows].cpu().numpy()
        lens_cpu = [length] * rows
        tko.topk_indices_ref(sample[:1], lens_cpu[:1], topk)
        t1 = time.perf_counter()
        tko.topk_indices_ref(sample, lens_cpu, topk)
        t_cpu = time.perf_counter() - t1
        cpu = {"value": round(t_cpu * (b * s_q / rows) * 1e6, 1), "unit": "µs/step", "cores": 1,
               "kind": "port", "sample": f"{rows} of {b * s_q} rows (numpy lexsort), scaled "
                                         f"x{b * s_q // rows} to the full step"}
    rec = {
        "metric": TOPK_METRIC, "value": round(us_step, 2), "unit": "µs/step", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "settle_s": round(settle_s, 3),
        "settle_steps": settle_steps, "ms_per_step": round(us_step / 1e3, 5),
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None, "dtype": "fp32",
        "data": "synthetic",
        "config": {"workload": spec["name"], "batch": b, "s_q": s_q, "length": length,
                   "topk": topk},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS,
                     "unit": "GB/s", "frac": round(gbs / PEAK_HBM_GBS, 4),
                     "traffic": recorded_traffic(spec["name"], "topk"),
                     # one topk_indices call: the chunk and merge kernels of the two-stage plan
                     "kernel": "topk_chunk_kernel+topk_merge_kernel",
                     "kernel_launches_timed": len(dec),
                     "kernel_us_mean": round(k_us, 2), "bytes_per_launch": nbytes},
        "cpu_baseline": cpu,
    }
    return with_traffic_source(rec)


KVC_WORKLOADS = {
    "kvcache": dict(name="kvcache_write_bf16_t131072", tokens=131072, fp8=False, seed=14),
    "kvcache_fp8": dict(name="kvcache_write_fp8_t131072", tokens=131072, fp8=True, seed=15),
}
KVC_METRIC = "MLA cache write µs/step + achieved HBM GB/s (% of roofline)"


def run_kvcache(args) -> dict:
    """Cache write path bench (concat_and_cache_mla): a prefill-sized batch of new tokens
    (latent + rope, bf16) written into shuffled pages of the paged cache; two input copies
    rotated.  A step is one launch, timed with events around it on its stream."""
    import flag_attn

    spec = KVC_WORKLOADS[args.workload]
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(spec["seed"])
    t, fp8 = spec["tokens"], spec["fp8"]
    pages = t // 64
    row = 656 if fp8 else 576
    dt = torch.uint8 if fp8 else torch.bfloat16
    cache = torch.zeros((pages, 64, 1, row), dtype=dt, device=dev)
    lat = [torch.randn((t, 512), generator=gen, device=dev).to(torch.bfloat16) for _ in range(2)]
    rope = [torch.randn((t, 64), generator=gen, device=dev).to(torch.bfloat16) for _ in range(2)]
    # int64 slots, the usual slot_mapping type (int32 ones are widened per call)
    perm = torch.randperm(pages, generator=gen, device=dev)
    tok = torch.arange(t, device=dev, dtype=torch.int64)
    slots = perm[tok // 64] * 64 + tok % 64

    def step(i):
        flag_attn.concat_and_cache_mla(lat[i % 2], rope[i % 2], cache, slots, fp8)

    if args.traffic_calibrate:
        calibrate_then(step, args, spec["name"])
        return None
    t_warm = time.perf_counter()
    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    settle_steps = 0
    while time.perf_counter() - t_warm < settle_seconds(args):
        for _ in range(20):
            step(settle_steps)
            settle_steps += 1
        torch.cuda.synchronize()
    settle_s = time.perf_counter() - t_warm
    every = max(1, min(EVENT_EVERY, args.steps // MIN_EVENT_LAUNCHES))
    stream = torch.cuda.current_stream()
    evs = {i: (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for i in range(0, args.steps, every)}
    t0 = time.perf_counter()
    for i in range(args.steps):
        ev = evs.get(i)
        if ev:
            ev[0].record(stream)
        step(i)
        if ev:
            ev[1].record(stream)
    torch.cuda.synchronize()
    us_step = (time.perf_counter() - t0) / args.steps * 1e6
    dec = sorted(s.elapsed_time(e) for s, e in evs.values())
    k_us = sum(dec) / len(dec) * 1e3
    # tokens read (latent + rope, bf16), rows written, one int32 slot per token
    nbytes = t * (1152 + (656 if fp8 else 1152) + 4)
    gbs = nbytes / (k_us * 1e-6) / 1e9
    cpu = None
    if not args.no_cpu_baseline:
        from oracle import mla_oracle as orc
        n = 4096
        sample_cache = torch.zeros((n // 64, 64, 1, row), dtype=dt)
        sl, sr = lat[0][:n].cpu(), rope[0][:n].cpu()
        sslots = torch.arange(n, dtype=torch.int64)
        t1 = time.perf_counter()
        orc.kvcache_write_ref(sample_cache, sl, sr, sslots, fp8)
        t_cpu = time.perf_counter() - t1
        cpu = {"value": round(t_cpu * (t / n) * 1e6, 1), "unit": "µs/step",
               "cores": torch.get_num_threads(), "kind": "port",
               "sample": f"{n} of {t} tokens (oracle writer), scaled x{t // n} to the full step"}
    rec = {
        "metric": KVC_METRIC, "value": round(us_step, 2), "unit": "µs/step", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "settle_s": round(settle_s, 3),
        "settle_steps": settle_steps, "ms_per_step": round(us_step / 1e3, 5),
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "fp8-e4m3" if fp8 else "bf16", "data": "synthetic",
        "config": {"workload": spec["name"], "tokens": t, "pages": pages,
                   "row_bytes": 656 if fp8 else 1152},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS,
                     "unit": "GB/s", "frac": round(gbs / PEAK_HBM_GBS, 4),
                     "traffic": recorded_traffic(spec["name"], "kvcache"),
                     "kernel": "mla_kvcache_write_kernel", "kernel_launches_timed": len(dec),
                     "kernel_us_mean": round(k_us, 2), "bytes_per_launch": nbytes},
        "cpu_baseline": cpu,
    }
    return with_traffic_source(rec)


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=500)
    ap.add_argument("--warmup", type=int, default=500)
    ap.add_argument("--workload", default=None,
                    choices=["dense", "skew", "sparse", "sparse_fp8"] + list(GQA_WORKLOADS)
                    + list(TOPK_WORKLOADS) + list(KVC_WORKLOADS))
    ap.add_argument("--copies", type=int, default=2, help="rotated KV pools (cache defeat)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extras", action="store_true",
                    help="default run: skip the other workloads' summary (other_workloads)")
    ap.add_argument("--traffic-calibrate", action="store_true",
                    help="profiling driver: a 512 MiB device copy, then --launches decode "
                         "steps (rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE passes)")
    ap.add_argument("--launches", type=int, default=5)
    ap.add_argument("--settle-launches", type=int, default=0,
                    help="--traffic-calibrate: untimed steps after the copy and before the "
                         "measured launches (with rocprofv3 --kernel-iteration-range, the "
                         "counters then come from launches at the sustained clock state)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported "
              "(batch sharding across GPUs needs no exchange: run one process per GPU).",
              file=sys.stderr)
        raise SystemExit(2)

    extras = args.workload is None and not args.traffic_calibrate and not args.no_extras
    if args.workload is None:
        args.workload = "dense"
    rec = run_workload(args)
    if rec is None:  # --traffic-calibrate
        return
    if extras:
        rec["other_workloads"] = other_workloads(args)
    print(json.dumps(rec), flush=True)


def run_workload(args):
    """The record of args.workload (None for --traffic-calibrate, which only drives the
    profiler's counter passes)."""
    if args.workload in GQA_WORKLOADS:
        return run_gqa(args)
    if args.workload in TOPK_WORKLOADS:
        return run_topk(args)
    if args.workload in KVC_WORKLOADS:
        return run_kvcache(args)
    return run_mla(args)


def other_workloads(args) -> dict:
    """Every other workload, each with OTHER_STEPS timed steps after OTHER_WARMUP warm-up
    steps and the settle phase, no CPU baseline: the value, the kernel's mean time by
    events and its roofline fraction, so that one default run records every workload's
    numbers.  A workload that fails records its error instead."""
    out = {}
    for w in OTHER_WORKLOADS:
        sub = argparse.Namespace(**vars(args))
        sub.workload, sub.steps, sub.warmup, sub.no_cpu_baseline = w, OTHER_STEPS, OTHER_WARMUP, True
        sub.settle_s = OTHER_SETTLE_S
        try:
            r = run_workload(sub)
            ro = r["roofline"]
            out[w] = {"config": r["config"]["workload"], "value": r["value"], "unit": r["unit"],
                      "kernel": ro["kernel"], "kernel_us_mean": ro["kernel_us_mean"],
                      "bound": ro["bound"], "frac": ro["frac"]}
            for k in ("hbm_frac", "mfma_frac"):
                if k in ro:
                    out[w][k] = ro[k]
        except Exception as e:  # noqa: BLE001 -- recorded, the flagship line still prints
            out[w] = {"error": f"{type(e).__name__}: {e}"[:300]}
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
    return out


def run_mla(args) -> dict | None:
    import flag_attn.mla as fa

    dev = torch.device("cuda:0")
    spec = workload_spec(args.workload)
    q, pools, tables, lens, indices = build_inputs(spec, dev, args.copies)
    s_q, h_q, b = spec["s_q"], spec["h_q"], spec["batch"]
    md, ns = fa.get_mla_metadata(lens, s_q * h_q, 1, num_heads_q=h_q, topk=spec["topk"])
    ws = fa.DecodeWorkspace(b, s_q, h_q, md.shape[0], dev, topk=spec["topk"])

    def step(i, events=None):
        md, ns = fa.get_mla_metadata(lens, s_q * h_q, 1, num_heads_q=h_q, topk=spec["topk"])
        c = i % len(pools)
        return ws.run(q, pools[c], tables[c], lens, md, ns, SCALE, spec["causal"],
                      spec["fp8"], indices, decode_events=events)

    if args.traffic_calibrate:
        # the copy's counter value over its known byte count scales the decode's values
        calibrate_then(step, args, spec["name"])
        return None

    t_warm = time.perf_counter()
    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    settle_steps = 0
    while time.perf_counter() - t_warm < settle_seconds(args):
        for _ in range(20):
            step(settle_steps)
            settle_steps += 1
        torch.cuda.synchronize()
    settle_s = time.perf_counter() - t_warm
    every = max(1, min(EVENT_EVERY, args.steps // MIN_EVENT_LAUNCHES))
    evs = {i: (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for i in range(0, args.steps, every)}
    t0 = time.perf_counter()
    for i in range(args.steps):
        step(i, evs.get(i))
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    us_step = (t1 - t0) / args.steps * 1e6
    dec_ms = sorted(s.elapsed_time(e) for s, e in evs.values())
    dec_us_mean = sum(dec_ms) / len(dec_ms) * 1e3
    dec_us_med = dec_ms[len(dec_ms) // 2] * 1e3

    lens_cpu = lens.cpu()
    nbytes, flops = algorithmic_work(spec, lens_cpu, indices.cpu() if indices is not None else None)
    gbs = nbytes / (dec_us_mean * 1e-6) / 1e9
    tflops = flops / (dec_us_mean * 1e-6) / 1e12
    hbm_frac = gbs / PEAK_HBM_GBS
    mfma_frac = tflops / PEAK_BF16_TFLOPS
    # the bound is the roof with the larger required time at peak
    bound = "hbm" if nbytes / PEAK_HBM_GBS >= flops / (PEAK_BF16_TFLOPS * 1e3) else "mfma"
    traffic = recorded_traffic(spec["name"])
    if bound == "hbm":
        roof = {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                "frac": round(hbm_frac, 4), "traffic": traffic}
    else:
        roof = {"bound": "mfma", "achieved": round(tflops, 1), "peak": PEAK_BF16_TFLOPS,
                "unit": "TFLOP/s", "frac": round(mfma_frac, 4), "traffic": traffic}
    if traffic is not None:
        roof["traffic_source"] = TRAFFIC_SOURCE
    roof.update({"kernel": "mla_decode_kernel", "kernel_launches_timed": len(dec_ms),
                 "kernel_us_mean": round(dec_us_mean, 2),
                 "kernel_us_median": round(dec_us_med, 2), "bytes_per_launch": nbytes,
                 "flops_per_launch": flops, "hbm_gbs": round(gbs, 1),
                 "hbm_frac": round(hbm_frac, 4), "mfma_tflops": round(tflops, 1),
                 "mfma_frac": round(mfma_frac, 4)})

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(spec, q, pools[0], tables[0], lens, indices)

    step_kernels = ["mla_metadata_kernel"] + (["mla_sparse_rows_kernel"] if spec["topk"] else [])
    step_kernels += ["mla_decode_kernel", "mla_combine_kernel"]
    rec = {
        "metric": METRIC,
        "value": round(us_step, 2),
        "unit": "µs/step",
        # what one timed step launches, in order: the scheduler metadata is recomputed every
        # step (a model computes it once per forward pass and reuses it in every layer)
        "step_kernels": step_kernels,
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "settle_s": round(settle_s, 3),
        "settle_steps": settle_steps,
        "ms_per_step": round(us_step / 1e3, 5),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16" if not spec["fp8"] else "fp8-e4m3 KV, bf16 MFMA",
        "data": "synthetic",
        "config": {"workload": spec["name"], "batch": b, "h_q": h_q, "s_q": s_q,
                   "d_qk": 576, "d_v": 512, "page": PAGE, "causal": spec["causal"],
                   "topk": spec["topk"], "mean_seqlen": float(lens_cpu.float().mean()),
                   "num_parts": int(md.shape[0]), "kv_pool_copies": len(pools)},
        "roofline": roof,
        "cpu_baseline": cpu,
    }
    return rec


if __name__ == "__main__":
    main()
