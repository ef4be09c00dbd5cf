"""Static check of the generated gfx950 code: no scalar select or branch on a stale SCC.

hipcc has emitted, for a uniform early exit tested on vector values (the top-k radix
search), an ``s_cselect_b32`` whose condition code was last written by an unrelated
``s_or_b64 exec, exec, ...`` (an exec restore, which sets SCC = exec != 0).  The select
then always took its first operand, and every search that ran all its passes got a
wrong threshold; only one parity case showed it.  The kernels now keep such values in
scalars.  This test compiles every kernel source to assembly and fails if any SCC reader
(``s_cselect``, ``s_cbranch_scc``, ``s_addc`` / ``s_subb``, ``s_cmov``) takes its SCC,
within its basic block, from an instruction that writes exec.  Planted-mistake check:
the same scan flags the miscompiled form (the search results read as vectors).
"""
import concurrent.futures as cf
import os
import re
import shutil
import subprocess
import tempfile

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "flagattention_amd", "csrc")
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"

_READER = re.compile(r"^\s*(s_cselect_b(32|64)|s_cbranch_scc[01]|s_addc_u32|s_subb_u32|s_cmovk?_[bi]32)\b")
_WRITER = re.compile(
    r"^\s*(s_(add|sub|addk)_[ui]32|s_(and|or|xor|andn2|orn2|nand|nor|xnor)_b(32|64)"
    r"|s_\w*saveexec_b64|s_\w*wrexec\w*|s_cmpk?_\w+|s_bitcmp\w*|s_(lshl|lshr|ashr)\w*|s_bfe\w*"
    r"|s_(min|max)_[ui]32|s_abs_i32|s_absdiff_i32|s_not_b(32|64)|s_bcnt\w*|s_wqm\w*"
    r"|s_quadmask\w*|s_addc_u32|s_subb_u32)\b")
_EXEC_DEST = re.compile(r"^\s*s_\w+\s+exec\b|^\s*s_\w*saveexec|^\s*s_\w*wrexec")


def stale_scc_sites(asm: str):
    """(line, reader, writer) for each SCC reader fed by an exec-writing instruction."""
    out = []
    last = None
    for i, line in enumerate(asm.splitlines()):
        if re.match(r"^\S+:", line):  # a label starts a block: SCC unknown
            last = None
            continue
        if _READER.match(line) and last is not None and _EXEC_DEST.match(last[1]):
            out.append((i + 1, line.strip(), last[1].strip()))
        if _WRITER.match(line):
            last = (i, line)
    return out


def _asm(src: str, workdir: str, text=None) -> str:
    if text is not None:
        path = os.path.join(workdir, os.path.basename(src))
        with open(path, "w") as f:
            f.write(text)
        src = path
    out = os.path.join(workdir, os.path.basename(src) + ".s")
    subprocess.run([HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang", "-target-feature",
                    "-Xclang", "-packed-fp32-ops", f"-I{ROOT}/include", f"-I{CSRC}", "--cuda-device-only",
                    "-S", src, "-o", out], check=True, capture_output=True)
    with open(out) as f:
        return f.read()


needs_hipcc = pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not available")


def test_scan_flags_a_stale_select():
    """The scan itself: a select after an exec restore is flagged, after a compare it is not."""
    bad = "\ts_or_b64 exec, exec, s[14:15]\n\tv_or_b32_e32 v3, v32, v3\n\ts_cselect_b32 s16, 8, 0\n"
    good = "\ts_cmp_eq_u32 s50, s16\n\ts_cselect_b64 s[16:17], -1, 0\n\ts_and_b64 vcc, exec, s[16:17]\n" \
           "\ts_cselect_b32 s16, 8, 0\n"
    across = "\ts_or_b64 exec, exec, s[14:15]\n.LBB0_5:\n\ts_cselect_b32 s16, 8, 0\n"
    assert len(stale_scc_sites(bad)) == 1
    assert stale_scc_sites(good) == []
    assert stale_scc_sites(across) == []


@needs_hipcc
def test_no_stale_scc_in_kernels():
    srcs = sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))
    with tempfile.TemporaryDirectory() as d, cf.ThreadPoolExecutor(max_workers=8) as ex:
        asms = list(ex.map(lambda s: _asm(s, d), srcs))
    found = {os.path.basename(s): stale_scc_sites(a) for s, a in zip(srcs, asms)}
    found = {k: v for k, v in found.items() if v}
    assert not found, f"SCC readers fed by exec writes: {found}"


@needs_hipcc
def test_scan_catches_the_miscompiled_search():
    """Planted mistake: the top-k search results read as vector values again."""
    src = os.path.join(CSRC, "fa_topk.hip")
    with open(src) as f:
        text = f.read()
    planted = (text.replace("static_cast<unsigned int>(__builtin_amdgcn_readfirstlane(sm.info[0]))",
                            "static_cast<unsigned int>(sm.info[0])")
                   .replace("need -= __builtin_amdgcn_readfirstlane(sm.info[1]);", "need -= sm.info[1];")
                   .replace("eq = __builtin_amdgcn_readfirstlane(sm.info[2]);", "eq = sm.info[2];"))
    assert planted != text
    with tempfile.TemporaryDirectory() as d:
        assert stale_scc_sites(_asm(src, d, planted)), "the planted form should miscompile and be flagged"
