"""HBM-traffic profiling driver for rocprofv3 --pmc runs (FETCH_SIZE / WRITE_SIZE).

Runs a plain device copy of a known size (the calibration kernel) and then the decode
of one bench workload, so one counter pass measures both; the copy's counter value
divided by its known byte count is the scale factor applied to the decode's value.

    rocprofv3 --pmc FETCH_SIZE --output-format csv -d OUT -o pmc -- \
        python flagattention_amd/profile_traffic.py --workload dense
"""
from __future__ import annotations

import argparse
import os
import sys

import torch

COPY_BYTES = 512 << 20


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--workload", default="dense")
    ap.add_argument("--launches", type=int, default=5)
    args = ap.parse_args()
    sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
    import bench
    import flagattention_amd as fa

    dev = torch.device("cuda:0")
    src = torch.empty(COPY_BYTES // 4, dtype=torch.float32, device=dev).normal_()
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    spec = bench.workload_spec(args.workload)
    q, pools, tables, lens, indices = bench.build_inputs(spec, dev, 2)
    s_q, h_q, b = spec["s_q"], spec["h_q"], spec["batch"]
    md, ns = fa.get_mla_metadata(lens, s_q * h_q, 1, topk=spec["topk"])
    ws = fa.DecodeWorkspace(b, s_q, h_q, md.shape[0], dev, topk=spec["topk"])
    for i in range(args.launches):
        ws.run(q, pools[i % 2], tables[i % 2], lens, md, ns, bench.SCALE, spec["causal"],
               spec["fp8"], indices)
    torch.cuda.synchronize()
    print(f"copy_bytes={COPY_BYTES} workload={spec['name']} launches={args.launches}", flush=True)


if __name__ == "__main__":
    main()
