"""The C-ABI library loads on a CPU-only host and exports exactly what
include/relux_kv.h declares (no compute calls: there is no GPU here)."""
import ctypes
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "relux_kv.h")
LIB = os.path.join(ROOT, "relux_amd", "librelux_kv.so")


def _declared():
    text = open(HEADER).read()
    decls = re.findall(r"int32_t\s+(rlx_\w+)\s*\(([^;]*?)\);", text, re.S)
    return {name: args for name, args in decls}


def test_header_declares_entry_points():
    decl = _declared()
    for name in ["rlx_init", "rlx_kv_create", "rlx_mla_create", "rlx_kv_append", "rlx_mla_append",
                 "rlx_kv_gather", "rlx_gqa_attend", "rlx_mla_attend", "rlx_rollback",
                 "rlx_evict", "rlx_compact", "rlx_page_table"]:
        assert name in decl


def test_library_exports_every_declared_symbol():
    if not os.path.exists(LIB):
        pytest.fail("librelux_kv.so is not built (run __graft_entry__.build())")
    out = subprocess.run(["nm", "-D", "--defined-only", LIB], capture_output=True, text=True,
                         check=True).stdout
    exported = set(re.findall(r"\bT (rlx_\w+)", out))
    assert set(_declared()) <= exported
    ctypes.CDLL(LIB)  # loads without a GPU


def test_python_binding_matches_header():
    from relux_amd import _lib
    decl = _declared()
    assert set(_lib.SIGNATURES) == set(decl)
    for name, args in decl.items():
        n = 0 if args.strip() in ("", "void") else args.count(",") + 1
        assert len(_lib.SIGNATURES[name]) == n, name
    lib = _lib.load()
    for name in decl:
        assert getattr(lib, name).restype is ctypes.c_int32
