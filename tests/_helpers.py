"""Shared helpers for the GPU parity tests (run the HIP path, compare with the oracle)."""
import sys

import torch

import flagattention_amd as fa

DEV = "cuda"
# bf16 out vs the fp32 oracle, fp32 lse absolute.
ATOL_OUT = 2e-2
RTOL_OUT = 1e-2
ATOL_LSE = 1e-3


def need_gpu():
    assert torch.cuda.is_available(), "GPU tests need an MI355X; none is visible"


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def run_dense(q, kc, bt, lens, scale, causal=False, parts=None):
    qd, kd, btd, ld = (t.to(DEV) for t in (q, kc, bt, lens))
    s_q, h_q = q.shape[1], q.shape[2]
    md, ns = fa.get_mla_metadata(ld, s_q * h_q, 1, num_sm_parts=parts)
    out, lse = fa.flash_mla_with_kvcache(qd, kd, btd, ld, 512, md, ns, scale, causal)
    torch.cuda.synchronize()
    return out.cpu(), lse.cpu(), md.cpu(), ns.cpu()


def run_sparse(q, kc, bt, lens, idx, scale, fp8=False, parts=None):
    qd, kd, btd, ld, idd = (t.to(DEV) for t in (q, kc, bt, lens, idx))
    s_q, h_q, topk = q.shape[1], q.shape[2], idx.shape[2]
    md, ns = fa.get_mla_metadata(ld, s_q * h_q, 1, num_heads_q=h_q, topk=topk, num_sm_parts=parts)
    out, lse = fa.flash_mla_with_kvcache(qd, kd, btd, ld, 512, md, ns, scale, False,
                                         is_fp8_kvcache=fp8, indices=idd)
    torch.cuda.synchronize()
    return out.cpu(), lse.cpu()


def assert_close(out, lse, ref_out, ref_lse, atol=ATOL_OUT, rtol=RTOL_OUT, atol_lse=ATOL_LSE):
    """out (bf16) within atol/rtol of the fp32 oracle; lse -inf where the oracle's is,
    finite ones within atol_lse."""
    out = out.float()
    assert out.shape == ref_out.shape and lse.shape == ref_lse.shape
    assert bool(torch.isfinite(out).all()), "non-finite output"
    err = (out - ref_out).abs()
    tol = atol + rtol * ref_out.abs()
    bad = err > tol
    assert not bool(bad.any()), (
        f"out mismatch: {int(bad.sum())} elems, max err {float(err.max()):.3e}")
    inf_ref = torch.isneginf(ref_lse)
    assert torch.equal(torch.isneginf(lse), inf_ref), "lse -inf pattern differs"
    fin = ~inf_ref
    if bool(fin.any()):
        lerr = (lse[fin] - ref_lse[fin]).abs().max()
        assert float(lerr) <= atol_lse, f"lse max err {float(lerr):.3e}"
