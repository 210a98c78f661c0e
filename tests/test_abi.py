"""The C-ABI library loads without a GPU and exports every function that
include/turboquant_amd.h declares (no compute call is made here)."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "turboquant_amd", "libturboquant_amd.so")


def declared_functions():
    names = []
    for hdr in sorted(os.listdir(os.path.join(ROOT, "include"))):
        if hdr.endswith(".h"):
            text = open(os.path.join(ROOT, "include", hdr)).read()
            text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
            names += re.findall(r"\b(tq_[a-z0-9_]+)\s*\(", text)
    return sorted(set(names))


@pytest.mark.skipif(not os.path.exists(LIB), reason="library not built (run __graft_entry__.build())")
def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(LIB)
    names = declared_functions()
    assert len(names) >= 11
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


@pytest.mark.skipif(not os.path.exists(LIB), reason="library not built")
def test_host_only_entry_points():
    lib = ctypes.CDLL(LIB)
    lib.tq_version.restype = ctypes.c_char_p
    assert b"gfx950" in lib.tq_version()
    lib.tq_attention_workspace_size.restype = ctypes.c_size_t
    # 1 x 16 heads x 32K: partials for 32 chunks of 1024 plus counters
    n = lib.tq_attention_workspace_size(1, 16, 8, 128, 32768)
    assert n >= 16 * 32 * 130 * 4
    assert lib.tq_attention_workspace_size(0, 16, 8, 128, 32768) == 0  # invalid shape -> 0
