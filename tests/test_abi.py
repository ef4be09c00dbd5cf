"""The C-ABI library loads and exports every symbol include/*.h declares -- CPU only
(no compute calls: this container has no GPU)."""
import ctypes
import glob
import os
import re

import pytest

from flagattention_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared_functions():
    names = set()
    for hdr in glob.glob(os.path.join(ROOT, "include", "*.h")):
        text = open(hdr).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"^\s*[A-Za-z_][\w\s\*]*?\b(fa_\w+)\s*\(", text, flags=re.M):
            names.add(m.group(1))
    return names


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(_lib.LIB_PATH):
        from flagattention_amd import build
        build.build()
    return _lib.load()


def test_header_declares_expected_entry_points():
    names = _declared_functions()
    assert {"fa_abi_version", "fa_last_error", "fa_mla_get_metadata", "fa_mla_decode_dense",
            "fa_mla_decode_sparse", "fa_mla_sparse_rows", "fa_mla_combine"} <= names


def test_library_exports_every_declared_symbol(lib):
    for name in _declared_functions():
        assert hasattr(lib, name), f"{name} declared in include/ but not exported"
        assert name in _lib.SIGNATURES, f"{name} has no ctypes signature in _lib.py"


def test_abi_version_and_struct_size(lib):
    assert lib.fa_abi_version() == _lib.ABI_VERSION
    assert lib.fa_mla_decode_args_size() == ctypes.sizeof(_lib.DecodeArgs)


def test_argument_errors_need_no_gpu(lib):
    # rejected on the host side of the ABI before any HIP call
    rc = lib.fa_mla_get_metadata(None, 0, 0, 1, 4, None, None, None)
    assert rc == -1 and b"batch" in lib.fa_last_error()
    rc = lib.fa_mla_decode_dense(None, None)
    assert rc == -1 and b"NULL" in lib.fa_last_error()
    args = _lib.DecodeArgs(batch=1, s_q=1, h_q=1, num_parts=1, topk=0)
    rc = lib.fa_mla_sparse_rows(ctypes.byref(args), None)
    assert rc == -1
    with pytest.raises(RuntimeError, match="flagattention_amd error -1"):
        _lib.check(rc)
