"""The C-ABI library loads on a machine without a GPU and exports every
function that include/helix_paged.h declares (no compute calls here)."""

import ctypes
import os
import re

import helix_runtime_amd as hx
from helix_runtime_amd import _native

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    text = open(os.path.join(ROOT, "include", "helix_paged.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(helix_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_boundary():
    names = declared_functions()
    assert "helix_paged_decode_attention" in names
    assert "helix_paged_attention_with_tail_out" in names
    assert len(names) >= 50


def test_library_exports_every_declared_symbol():
    lib = hx.load()
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert missing == []


def test_python_binding_covers_every_declared_symbol():
    assert sorted(_native.SIGNATURES) == declared_functions()


def test_status_names_and_last_error():
    lib = hx.load()
    assert lib.helix_status_name(0) == b"ok"
    assert lib.helix_status_name(4) == b"resource_exhausted"
    out = ctypes.c_void_p()
    rc = lib.helix_block_manager_create(None, ctypes.byref(out))
    assert rc == hx.INVALID_ARGUMENT
    assert b"config" in lib.helix_last_error()


def test_library_is_gfx950_code_object():
    blob = open(_native.LIB_PATH, "rb").read()
    assert b"gfx950" in blob
