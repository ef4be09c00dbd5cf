"""Parity at the benchmark workloads through ``flag_attn``.

Each test builds the workload exactly as ``bench.py`` does (same seed, shapes, lengths,
block tables and indices, resident on the GPU) and runs the decode the benchmark times,
then checks:

* scheduler metadata bit-exact against ``oracle.metadata_spec`` over the whole batch;
* sparse gather rows bit-exact against ``oracle.sparse_rows_ref`` over the whole batch;
* out / lse against the oracle on sampled sequences (the longest, the one cut into the
  most splits, the first, the last and the middle one), under the north-star bars and the
  reference's bf16-arithmetic rule.  The benchmark data is N(0,1) * 0.1, where |out| stays
  ~5e-3, far below the absolute bars: the rule is the bar that can fail there
  (``tests/test_bars.py`` shows a one-token gather shift fails it on such data).
"""
import pytest
import torch

import bench
import flag_attn
from flagattention_amd.mla import overhead_blocks
from oracle import mla_oracle as orc
from tests._helpers import assert_close, need_gpu, say

pytestmark = pytest.mark.gpu


def _sample(spec, q, pool, table, lens, indices, batches):
    """CPU copies of the sampled sequences' inputs: only the pages their block-table rows
    name, with the rows remapped onto that compact pool."""
    sel = torch.tensor(batches, device=table.device)
    bt_sel = table[sel]
    need = torch.unique(bt_sel.flatten()).long()
    remap = torch.full((pool.shape[0],), -1, dtype=torch.long, device=pool.device)
    remap[need] = torch.arange(need.numel(), device=pool.device)
    kc = pool[need].cpu()
    bt = remap[bt_sel.long()].to(torch.int32).cpu()
    idx = None if indices is None else indices[sel].cpu()
    return q[sel].cpu(), kc, bt, lens[sel].cpu(), idx


@pytest.mark.parametrize("workload", ["dense", "skew", "sparse", "sparse_fp8"])
def test_benchmark_workload(workload):
    need_gpu()
    spec = bench.workload_spec(workload)
    say(f"benchmark workload {spec['name']}: building inputs")
    dev = torch.device("cuda:0")
    q, pools, tables, lens, indices = bench.build_inputs(spec, dev, 1)
    pool, table = pools[0], tables[0]
    b, s_q, h_q, topk = spec["batch"], spec["s_q"], spec["h_q"], spec["topk"]

    md, ns = flag_attn.get_mla_metadata(lens, s_q * h_q, 1, num_heads_q=h_q, topk=topk)
    out, lse = flag_attn.flash_mla_with_kvcache(q, pool, table, lens, 512, md, ns, bench.SCALE,
                                                spec["causal"], is_fp8_kvcache=spec["fp8"],
                                                indices=indices)
    torch.cuda.synchronize()
    lens_c = lens.cpu()
    parts = md.shape[0]
    say(f"{spec['name']}: parts={parts} splits={int(ns[-1])}")

    want_md, want_ns = orc.metadata_spec(lens_c.tolist(), parts, overhead_blocks(bool(topk)),
                                         topk or 0)
    assert md.cpu().tolist() == want_md
    assert ns.cpu().tolist() == want_ns

    if topk:
        rows = flag_attn.mla.sparse_rows(indices, table, lens, pool.shape[0])
        want_rows = orc.sparse_rows_ref(indices.cpu(), table.cpu(), lens_c, pool.shape[0])
        assert torch.equal(rows.cpu(), want_rows)

    nsplit = (ns[1:] - ns[:-1]).cpu()
    picks = [int(torch.argmax(lens_c)), int(torch.argmax(nsplit)), 0, b - 1, b // 2]
    batches = sorted(set(picks))
    say(f"{spec['name']}: checking sequences {batches} (splits {nsplit[batches].tolist()})")
    qs, kc, bt, ls, idx = _sample(spec, q, pool, table, lens, indices, batches)
    if topk:
        ref_out, ref_lse = orc.sparse_decode_ref(qs, kc, bt, ls, idx, bench.SCALE,
                                                 is_fp8=spec["fp8"])
        low, low_lse = orc.sparse_decode_ref(qs, kc, bt, ls, idx, bench.SCALE,
                                             is_fp8=spec["fp8"], lowp=True)
    else:
        ref_out, ref_lse = orc.dense_decode_ref(qs, kc, bt, ls, bench.SCALE, spec["causal"])
        low, _ = orc.dense_decode_ref(qs, kc, bt, ls, bench.SCALE, spec["causal"], lowp=True)
        low_lse = None
    sel = torch.tensor(batches)
    assert_close(out.cpu()[sel], lse.cpu()[sel], ref_out, ref_lse, low,
                 low_lse if spec["fp8"] else None)
    # every row of the batch was written (finite; an unwritten split would leave garbage)
    assert bool(torch.isfinite(out).all()) and bool(torch.isfinite(lse).all())
