"""Shared helpers for the GPU parity tests (run the HIP path, compare with the oracle)."""
import sys

import torch

import flag_attn
from oracle import mla_oracle as orc

DEV = "cuda"
# bf16 out vs the fp32 oracle, fp32 lse absolute.
ATOL_OUT = 2e-2
RTOL_OUT = 1e-2
ATOL_LSE = 1e-3
# The reference's accuracy rule (tests/flag_attn/test_flash_attention.py:119-127,
# README.md:111-117): max|hyp - ref_fp32| <= LOWP_FACTOR * max|ref_lowp - ref_fp32| + LOWP_ABS.
LOWP_FACTOR = 2.0
LOWP_ABS = 1e-5


def assert_lowp_rule(hyp, ref, low):
    """The reference's rule max|hyp - ref| <= 2 max|low - ref| + 1e-5 (ref: the fp32 oracle,
    low: the oracle in the inputs' low-precision arithmetic)."""
    e_hyp = float((hyp.float() - ref.float()).abs().max()) if ref.numel() else 0.0
    e_low = float((low.float() - ref.float()).abs().max()) if ref.numel() else 0.0
    assert e_hyp <= LOWP_FACTOR * e_low + LOWP_ABS, (
        f"error {e_hyp:.3e} > {LOWP_FACTOR} x low-precision error {e_low:.3e} + {LOWP_ABS}")


def need_gpu():
    assert torch.cuda.is_available(), "GPU tests need an MI355X; none is visible"


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def run_dense(q, kc, bt, lens, scale, causal=False, parts=None):
    qd, kd, btd, ld = (t.to(DEV) for t in (q, kc, bt, lens))
    s_q, h_q = q.shape[1], q.shape[2]
    md, ns = flag_attn.get_mla_metadata(ld, s_q * h_q, 1, num_sm_parts=parts)
    out, lse = flag_attn.flash_mla_with_kvcache(qd, kd, btd, ld, 512, md, ns, scale, causal)
    torch.cuda.synchronize()
    return out.cpu(), lse.cpu(), md.cpu(), ns.cpu()


def run_sparse(q, kc, bt, lens, idx, scale, fp8=False, parts=None):
    qd, kd, btd, ld, idd = (t.to(DEV) for t in (q, kc, bt, lens, idx))
    s_q, h_q, topk = q.shape[1], q.shape[2], idx.shape[2]
    md, ns = flag_attn.get_mla_metadata(ld, s_q * h_q, 1, num_heads_q=h_q, topk=topk,
                                        num_sm_parts=parts)
    out, lse = flag_attn.flash_mla_with_kvcache(qd, kd, btd, ld, 512, md, ns, scale, False,
                                                is_fp8_kvcache=fp8, indices=idd)
    torch.cuda.synchronize()
    return out.cpu(), lse.cpu()


def dense_refs(q, kc, bt, lens, scale, causal=False, batches=None):
    """(fp32 out, fp32 lse, bf16-arithmetic out) of the oracle for a dense decode."""
    ref_out, ref_lse = orc.dense_decode_ref(q, kc, bt, lens, scale, causal, batches=batches)
    low_out, _ = orc.dense_decode_ref(q, kc, bt, lens, scale, causal, batches=batches, lowp=True)
    return ref_out, ref_lse, low_out


def sparse_refs(q, kc, bt, lens, idx, scale, fp8=False, batches=None):
    """(fp32 out, fp32 lse, bf16-arithmetic out, bf16-arithmetic lse or None) of the oracle
    for a sparse decode.  The fp8 cache is dequantised to bf16 on chip (the MFMA input
    type), which moves S by up to ~2^-9 |q||k|; against the fp32-dequant oracle the lse of
    unit-scale data then needs the bf16-arithmetic rule rather than the fixed 1e-3, so the
    bf16-arithmetic lse is returned for fp8 (and only for fp8)."""
    ref_out, ref_lse = orc.sparse_decode_ref(q, kc, bt, lens, idx, scale, is_fp8=fp8,
                                             batches=batches)
    low_out, low_lse = orc.sparse_decode_ref(q, kc, bt, lens, idx, scale, is_fp8=fp8,
                                             batches=batches, lowp=True)
    return ref_out, ref_lse, low_out, (low_lse if fp8 else None)


def assert_close(out, lse, ref_out, ref_lse, low_out=None, low_lse=None, atol=ATOL_OUT,
                 rtol=RTOL_OUT, atol_lse=ATOL_LSE):
    """out (bf16) within atol/rtol of the fp32 oracle; lse -inf where the oracle's is,
    finite ones within atol_lse; and, given the oracle's bf16-arithmetic output
    ``low_out``, the reference's rule max|out - ref| <= 2 max|low_out - ref| + 1e-5
    (the bar that scales with the data: the absolute bars alone pass any answer when
    the outputs are small).  Given ``low_lse`` (fp8 cache only), the lse bar is
    max(atol_lse, 2 max|low_lse - ref_lse| + 1e-5)."""
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
        bar = atol_lse
        if low_lse is not None:
            e_low = float((low_lse[fin] - ref_lse[fin]).abs().max())
            bar = max(atol_lse, LOWP_FACTOR * e_low + LOWP_ABS)
        assert float(lerr) <= bar, f"lse max err {float(lerr):.3e} > {bar:.3e}"
    if low_out is not None:
        assert low_out.shape == ref_out.shape
        e_hyp = float(err.max()) if err.numel() else 0.0
        e_low = float((low_out.float() - ref_out).abs().max()) if err.numel() else 0.0
        assert e_hyp <= LOWP_FACTOR * e_low + LOWP_ABS, (
            f"out error {e_hyp:.3e} > {LOWP_FACTOR} x bf16-arithmetic error {e_low:.3e} "
            f"+ {LOWP_ABS}")
