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


def declared_arities():
    text = open(os.path.join(ROOT, "include", "helix_paged.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    out = {}
    for name, params in re.findall(r"\b(helix_[a-z0-9_]+)\s*\(([^;{]*?)\)\s*;", text, flags=re.S):
        params = params.strip()
        out[name] = 0 if params in ("", "void") else params.count(",") + 1
    return out


def test_python_binding_arities_match_the_header():
    arity = declared_arities()
    assert set(arity) == set(_native.SIGNATURES)
    wrong = {n: (len(a), arity[n]) for n, (_, a) in _native.SIGNATURES.items()
             if len(a) != arity[n]}
    assert wrong == {}


def test_batched_entry_points_reject_other_geometries_before_launch():
    """A pool of head_dim 64 or 32-token pages is refused with
    HELIX_UNSUPPORTED before any pointer is read or kernel launched (the
    pointers here are NULL and no GPU is needed)."""
    lib = hx.load()
    for head_dim, block_tokens in ((64, 16), (128, 32), (256, 16)):
        rc = lib.helix_paged_decode_attention(None, 4, 32, 8, head_dim, None, None, 100,
                                              block_tokens, None, 8, None, None, None, None,
                                              None, 1 << 20, 0, None)
        assert rc == hx.UNSUPPORTED
        assert b"head_dim 128 and 16-token pages" in lib.helix_last_error()
        rc = lib.helix_paged_prefill_attention(None, 4, 32, 8, 16, head_dim, None, None, 100,
                                               block_tokens, None, 8, None, None, None, None,
                                               None)
        assert rc == hx.UNSUPPORTED


def test_cache_creation_rejects_bad_page_formats_before_any_allocation():
    """helix_paged_cache_create_fp8 refuses zero, negative and non-finite
    scales and helix_paged_cache_create_typed an unknown element type with
    HELIX_INVALID_ARGUMENT, leaving *out NULL; both checks run before the
    device is touched (no GPU here)."""
    lib = hx.load()
    cfg = _native.Config(layers=2, kv_heads=8, head_dimension=128, block_tokens=16,
                         physical_blocks=64)
    out = ctypes.c_void_p(12345)
    for ks, vs in ((0.0, 1.0), (1.0, -2.0), (float("inf"), 1.0), (1.0, float("nan")),
                   (-0.0, 1.0)):
        rc = lib.helix_paged_cache_create_fp8(ctypes.byref(cfg), 0, ks, vs, ctypes.byref(out))
        assert rc == hx.INVALID_ARGUMENT, (ks, vs)
        assert out.value is None
        assert b"fp8 page scales must be finite and positive" in lib.helix_last_error()
        out = ctypes.c_void_p(12345)
    for dtype in (-1, 3, 4):
        rc = lib.helix_paged_cache_create_typed(ctypes.byref(cfg), 0, dtype, ctypes.byref(out))
        assert rc == hx.INVALID_ARGUMENT, dtype
        assert out.value is None
        assert b"page dtype must be" in lib.helix_last_error()
        out = ctypes.c_void_p(12345)
    rc = lib.helix_paged_cache_create_fp8(ctypes.byref(cfg), 0, 1.0, 1.0, None)
    assert rc == hx.INVALID_ARGUMENT


def test_python_cache_rejects_bad_page_formats_before_any_allocation():
    """The Python PagedKvCache refuses an unknown page type, scales on a
    page type without them, and bad fp8 scales (the C check) with
    INVALID_ARGUMENT before the device is touched."""
    import pytest
    geometry = dict(layers=2, kv_heads=8, head_dimension=128, block_tokens=16,
                    physical_blocks=64)
    cases = (dict(page_dtype="fp4"), dict(page_dtype="bf16", k_scale=2.0),
             dict(page_dtype="f32", v_scale=0.5), dict(page_dtype="fp8", k_scale=0.0),
             dict(page_dtype="fp8", v_scale=float("inf")))
    for kw in cases:
        with pytest.raises(hx.HelixError) as e:
            hx.PagedKvCache(**geometry, **kw)
        assert e.value.status == hx.INVALID_ARGUMENT, kw


def test_typed_entry_points_reject_bad_formats_before_launch():
    """The typed stateless decode and prefill refuse an unknown page dtype
    and a non-finite or non-positive fp8 scale with HELIX_INVALID_ARGUMENT,
    and bf16 / fp8 pools with an explicit split size with
    HELIX_UNSUPPORTED, before any pointer is read (NULL pointers, no GPU)."""
    lib = hx.load()

    def decode(dtype, ks=1.0, vs=1.0, split=0):
        return lib.helix_paged_decode_attention_typed(
            None, 4, 32, 8, 128, None, None, 100, 16, None, 8, None, None, None, None, None,
            1 << 20, split, dtype, ks, vs, None)

    def prefill(dtype, ks=1.0, vs=1.0):
        return lib.helix_paged_prefill_attention_typed(
            None, 4, 32, 8, 64, 128, None, None, 100, 16, None, 8, None, None, None, None,
            dtype, ks, vs, None)

    for call in (decode, prefill):
        assert call(3) == hx.INVALID_ARGUMENT
        assert b"page dtype" in lib.helix_last_error()
        assert call(-1) == hx.INVALID_ARGUMENT
        for ks, vs in ((0.0, 1.0), (1.0, -2.0), (float("nan"), 1.0), (1.0, float("inf"))):
            assert call(2, ks, vs) == hx.INVALID_ARGUMENT
            assert b"fp8 page scales" in lib.helix_last_error()
    assert decode(1, split=4) == hx.UNSUPPORTED
    assert decode(2, 0.5, 0.5, split=1) == hx.UNSUPPORTED
    assert b"stream kernel only" in lib.helix_last_error()
