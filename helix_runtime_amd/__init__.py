"""MI355X-native paged-KV hot path of helix-runtime.

Python front end over the C ABI in ``include/helix_paged.h``.  The names and
argument meaning follow the reference's C++ interface
(``include/helix/kv_cache/cuda_paged.hpp``, ``include/helix/kv_cache/paged.hpp``,
``include/helix/attention/cuda_paged.hpp``); errors surface as
:class:`HelixError` carrying the reference's error code.  PyTorch is used
only for device memory and streams: every computation runs in the HIP
kernels of ``libhelix_paged.so``.
"""

from __future__ import annotations

import ctypes
import sys
import os
import subprocess

from . import _native
from ._native import (HelixError, Sequence, INVALID_ARGUMENT, OUT_OF_RANGE, UNSUPPORTED,
                      RESOURCE_EXHAUSTED, RUNTIME, INTERNAL, check)

__all__ = [
    "build", "load", "HelixError", "Sequence", "BlockManager", "PagedKvCache", "DecodeBatch",
    "PagedBlockTable", "paged_attention_out", "paged_attention_with_tail_out",
    "paged_decode_attention", "decode_workspace_bytes", "decode_workspace", "append_slots",
    "PagedPrefixCache", "PREFIX_INSERTED", "PREFIX_ALREADY_PRESENT", "PREFIX_REJECTED_TOO_LARGE",
    "INVALID_ARGUMENT", "OUT_OF_RANGE", "UNSUPPORTED", "RESOURCE_EXHAUSTED", "RUNTIME", "INTERNAL",
]


def build(jobs: int = 8) -> str:
    """Compile libhelix_paged.so for gfx950 with the in-tree Makefile."""
    subprocess.run(["make", "-s", "-C", _native.HERE, f"-j{jobs}", "libhelix_paged.so"],
                   check=True)
    return _native.LIB_PATH


def load():
    return _native.load()


def _lib():
    return _native.load()


def _ptr(t):
    """Device (or host) address of a tensor, or None."""
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(stream):
    import torch
    if stream is None:
        stream = torch.cuda.current_stream()
    return ctypes.c_void_p(stream.cuda_stream)


def _require_f32(t, name):
    import torch
    if t.dtype != torch.float32 or not t.is_contiguous():
        raise HelixError(INVALID_ARGUMENT, f"{name} must be a contiguous float32 tensor")


def _cfg(layers, kv_heads, head_dimension, block_tokens, physical_blocks):
    return _native.Config(layers, kv_heads, head_dimension, block_tokens, physical_blocks)


# ------------------------------------------------------------------ host ----
class BlockManager:
    """Host page bookkeeping of the paged pool (no device memory)."""

    def __init__(self, layers, kv_heads, head_dimension, block_tokens, physical_blocks):
        h = ctypes.c_void_p()
        cfg = _cfg(layers, kv_heads, head_dimension, block_tokens, physical_blocks)
        check(_lib().helix_block_manager_create(ctypes.byref(cfg), ctypes.byref(h)))
        self._h = h
        self.block_tokens = block_tokens
        self.physical_blocks = physical_blocks

    def __del__(self, _finalizing=sys.is_finalizing):
        if _finalizing():
            return  # the process is exiting; the driver reclaims device memory
        h = getattr(self, "_h", None)
        if h:
            _lib().helix_block_manager_destroy(h)
            self._h = None

    def create_sequence(self) -> Sequence:
        s = Sequence()
        check(_lib().helix_block_manager_create_sequence(self._h, ctypes.byref(s)))
        return s

    def fork_sequence(self, source, prefix_tokens, allow_cow=False):
        s, c = Sequence(), _native.CowCopy()
        check(_lib().helix_block_manager_fork_sequence(self._h, source, prefix_tokens,
                                                       int(allow_cow), ctypes.byref(s),
                                                       ctypes.byref(c)))
        return s, (c.from_block, c.to_block, c.tokens)

    def append(self, seq, tokens=1):
        slots = (ctypes.c_uint64 * tokens)()
        check(_lib().helix_block_manager_append(self._h, seq, tokens, slots))
        return list(slots)

    def release_sequence(self, seq):
        check(_lib().helix_block_manager_release_sequence(self._h, seq))

    def contains(self, seq):
        out = ctypes.c_int()
        check(_lib().helix_block_manager_contains(self._h, seq, ctypes.byref(out)))
        return bool(out.value)

    def length(self, seq):
        out = ctypes.c_size_t()
        check(_lib().helix_block_manager_length(self._h, seq, ctypes.byref(out)))
        return out.value

    def block_table(self, seq):
        n = ctypes.c_size_t()
        buf = (ctypes.c_uint32 * self.physical_blocks)()
        check(_lib().helix_block_manager_block_table(self._h, seq, buf, self.physical_blocks,
                                                     ctypes.byref(n)))
        return list(buf[: n.value])

    def stats(self):
        s = _native.Stats()
        check(_lib().helix_block_manager_stats(self._h, ctypes.byref(s)))
        return s.as_dict()

    def block_info(self, block):
        r, t = ctypes.c_size_t(), ctypes.c_size_t()
        check(_lib().helix_block_manager_block_info(self._h, block, ctypes.byref(r),
                                                    ctypes.byref(t)))
        return r.value, t.value

    def validate(self):
        check(_lib().helix_block_manager_validate(self._h))

    def geometry(self):
        a, b, c = ctypes.c_size_t(), ctypes.c_size_t(), ctypes.c_size_t()
        check(_lib().helix_block_manager_geometry(self._h, ctypes.byref(a), ctypes.byref(b),
                                                  ctypes.byref(c)))
        return a.value, b.value, c.value


PAGE_DTYPES = {"f32": 0, "bf16": 1, "fp8": 2}

# ---------------------------------------------------------- prefix cache ----
PREFIX_INSERTED, PREFIX_ALREADY_PRESENT, PREFIX_REJECTED_TOO_LARGE = 0, 1, 2


def _tokens(tokens):
    arr = (ctypes.c_uint32 * max(len(tokens), 1))(*[int(t) for t in tokens])
    return arr, len(tokens)


class PagedPrefixCache:
    """helix::kv_cache::PagedPrefixCache (include/helix/kv_cache/prefix.hpp:
    66-112) over a ``PagedKvCache`` (device pool) or a ``BlockManager`` (host
    bookkeeping only).  ``insert`` returns one of PREFIX_INSERTED,
    PREFIX_ALREADY_PRESENT, PREFIX_REJECTED_TOO_LARGE; ``lookup_longest``
    returns ``(sequence, matched_tokens)`` or None, and the caller releases
    the sequence."""

    def __init__(self, pool, maximum_entries, maximum_block_references):
        h = ctypes.c_void_p()
        cfg = _native.PrefixConfig(maximum_entries, maximum_block_references)
        if isinstance(pool, BlockManager):
            check(_lib().helix_prefix_cache_create_host(pool._h, ctypes.byref(cfg),
                                                        ctypes.byref(h)))
        elif isinstance(pool, PagedKvCache):
            check(_lib().helix_prefix_cache_create(pool._h, ctypes.byref(cfg), ctypes.byref(h)))
        else:
            check(_lib().helix_prefix_cache_create(None, ctypes.byref(cfg), ctypes.byref(h)))
        self._h = h
        self._pool = pool  # the host manager must outlive the index

    def close(self):
        h = getattr(self, "_h", None)
        if h:
            _lib().helix_prefix_cache_destroy(h)
            self._h = None

    def __del__(self, _finalizing=sys.is_finalizing):
        if _finalizing():
            return  # the process is exiting; the driver reclaims device memory
        self.close()

    def insert(self, namespace_id, tokens, source):
        arr, n = _tokens(tokens)
        out = ctypes.c_int()
        check(_lib().helix_prefix_cache_insert(self._h, namespace_id, arr, n, source,
                                               ctypes.byref(out)))
        return out.value

    def lookup_longest(self, namespace_id, tokens, maximum_prefix_tokens=None):
        arr, n = _tokens(tokens)
        limit = (1 << 64) - 1 if maximum_prefix_tokens is None else maximum_prefix_tokens
        hit, seq, matched = ctypes.c_int(), Sequence(), ctypes.c_size_t()
        check(_lib().helix_prefix_cache_lookup_longest(self._h, namespace_id, arr, n, limit,
                                                       ctypes.byref(hit), ctypes.byref(seq),
                                                       ctypes.byref(matched)))
        return (seq, matched.value) if hit.value else None

    def contains(self, namespace_id, tokens):
        arr, n = _tokens(tokens)
        out = ctypes.c_int()
        check(_lib().helix_prefix_cache_contains(self._h, namespace_id, arr, n,
                                                 ctypes.byref(out)))
        return bool(out.value)

    def erase(self, namespace_id, tokens):
        arr, n = _tokens(tokens)
        out = ctypes.c_int()
        check(_lib().helix_prefix_cache_erase(self._h, namespace_id, arr, n, ctypes.byref(out)))
        return bool(out.value)

    def evict_lru(self):
        out = ctypes.c_int()
        check(_lib().helix_prefix_cache_evict_lru(self._h, ctypes.byref(out)))
        return bool(out.value)

    def clear(self):
        check(_lib().helix_prefix_cache_clear(self._h))

    def stats(self):
        s = _native.PrefixStats()
        check(_lib().helix_prefix_cache_stats(self._h, ctypes.byref(s)))
        return s.as_dict()

    def config(self):
        c = _native.PrefixConfig()
        check(_lib().helix_prefix_cache_config(self._h, ctypes.byref(c)))
        return c.maximum_entries, c.maximum_block_references

    def block_tokens(self):
        out = ctypes.c_size_t()
        check(_lib().helix_prefix_cache_block_tokens(self._h, ctypes.byref(out)))
        return out.value


# ---------------------------------------------------------------- device ----
class PagedKvCache:
    """GPU paged KV pool (CudaPagedKvCache + the CPU cache's fork/bulk append)."""

    def __init__(self, layers, kv_heads, head_dimension, block_tokens, physical_blocks,
                 device=0, page_dtype="f32", k_scale=1.0, v_scale=1.0):
        """``page_dtype`` "bf16" stores pages as bf16 (extension: appended
        fp32 rows rounded to nearest even, gathers widen back to fp32);
        "fp8" stores OCP E4M3 codes of x / k_scale (keys) and x / v_scale
        (values), rounded to nearest even and saturating at +-448; gathers
        return decode(code) * scale."""
        h = ctypes.c_void_p()
        cfg = _cfg(layers, kv_heads, head_dimension, block_tokens, physical_blocks)
        if page_dtype not in PAGE_DTYPES:
            raise HelixError(INVALID_ARGUMENT, f"page_dtype must be one of {sorted(PAGE_DTYPES)}")
        if page_dtype != "fp8" and (k_scale != 1.0 or v_scale != 1.0):
            raise HelixError(INVALID_ARGUMENT, "k_scale and v_scale apply to fp8 pages only")
        if page_dtype == "fp8":
            check(_lib().helix_paged_cache_create_fp8(ctypes.byref(cfg), device, float(k_scale),
                                                      float(v_scale), ctypes.byref(h)))
        else:
            check(_lib().helix_paged_cache_create_typed(ctypes.byref(cfg), device,
                                                        PAGE_DTYPES[page_dtype], ctypes.byref(h)))
        self._h = h
        self.page_dtype = page_dtype
        ks, vs = ctypes.c_float(), ctypes.c_float()
        check(_lib().helix_paged_cache_fp8_scales(h, ctypes.byref(ks), ctypes.byref(vs)))
        self.k_scale, self.v_scale = ks.value, vs.value
        self.layers, self.kv_heads, self.head_dimension = layers, kv_heads, head_dimension
        self.block_tokens, self.physical_blocks, self.device = block_tokens, physical_blocks, device

    def close(self):
        h = getattr(self, "_h", None)
        if h:
            _lib().helix_paged_cache_destroy(h)
            self._h = None

    def __del__(self, _finalizing=sys.is_finalizing):
        if _finalizing():
            return  # the process is exiting; the driver reclaims device memory
        self.close()

    def create_sequence(self) -> Sequence:
        s = Sequence()
        check(_lib().helix_paged_cache_create_sequence(self._h, ctypes.byref(s)))
        return s

    def fork_sequence(self, source, prefix_tokens, allow_cow=False, stream=None):
        s = Sequence()
        check(_lib().helix_paged_cache_fork_sequence(self._h, source, prefix_tokens,
                                                     int(allow_cow), _stream(stream),
                                                     ctypes.byref(s)))
        return s

    def append(self, seq, token_keys, token_values, stream=None):
        """token_keys/values: device [layers, kv_heads, head_dimension]."""
        for t, n in ((token_keys, "token keys"), (token_values, "token values")):
            _require_f32(t, n)
            if tuple(t.shape) != (self.layers, self.kv_heads, self.head_dimension):
                raise HelixError(INVALID_ARGUMENT,
                                 f"{n} shape does not match [layers, heads, dimension]")
        check(_lib().helix_paged_cache_append(self._h, seq, _ptr(token_keys), _ptr(token_values),
                                              _stream(stream)))

    def append_layer_major(self, seq, layer_keys, layer_values, stream=None):
        """One device [kv_heads, tokens, head_dimension] tensor per layer."""
        if len(layer_keys) != self.layers or len(layer_values) != self.layers:
            raise HelixError(INVALID_ARGUMENT, "requires one key/value tensor per layer")
        tokens = layer_keys[0].shape[1]
        for t in list(layer_keys) + list(layer_values):
            _require_f32(t, "layer tensor")
            if tuple(t.shape) != (self.kv_heads, tokens, self.head_dimension):
                raise HelixError(INVALID_ARGUMENT, "layer tensor shape mismatch")
        kp = (ctypes.c_void_p * self.layers)(*[t.data_ptr() for t in layer_keys])
        vp = (ctypes.c_void_p * self.layers)(*[t.data_ptr() for t in layer_values])
        check(_lib().helix_paged_cache_append_layer_major(self._h, seq, kp, vp, tokens,
                                                          _stream(stream)))

    def release_sequence(self, seq):
        check(_lib().helix_paged_cache_release_sequence(self._h, seq))

    def retrieve_layer(self, seq, layer):
        """Allocating gather: returns device (keys, values) [kv_heads, length, dim]."""
        import torch
        n = self.length(seq)
        shape = (self.kv_heads, n, self.head_dimension)
        k = torch.empty(shape, dtype=torch.float32, device=f"cuda:{self.device}")
        v = torch.empty(shape, dtype=torch.float32, device=f"cuda:{self.device}")
        self.copy_layer_out(seq, layer, k, v)
        return k, v

    def copy_layer_out(self, seq, layer, keys, values, stream=None):
        check(_lib().helix_paged_cache_copy_layer_out(self._h, seq, layer, _ptr(keys),
                                                      _ptr(values), _stream(stream)))

    def copy_layer_prefix_out(self, seq, layer, expected_length, keys, values, stream=None):
        check(_lib().helix_paged_cache_copy_layer_prefix_out(
            self._h, seq, layer, expected_length, _ptr(keys), _ptr(values), keys.shape[1],
            _stream(stream)))

    def contains(self, seq):
        out = ctypes.c_int()
        check(_lib().helix_paged_cache_contains(self._h, seq, ctypes.byref(out)))
        return bool(out.value)

    def length(self, seq):
        out = ctypes.c_size_t()
        check(_lib().helix_paged_cache_length(self._h, seq, ctypes.byref(out)))
        return out.value

    def block_table(self, seq):
        n = ctypes.c_size_t()
        buf = (ctypes.c_uint32 * self.physical_blocks)()
        check(_lib().helix_paged_cache_block_table(self._h, seq, buf, self.physical_blocks,
                                                   ctypes.byref(n)))
        return list(buf[: n.value])

    def stats(self):
        s = _native.Stats()
        check(_lib().helix_paged_cache_stats(self._h, ctypes.byref(s)))
        return s.as_dict()

    def is_healthy(self):
        out = ctypes.c_int()
        check(_lib().helix_paged_cache_is_healthy(self._h, ctypes.byref(out)))
        return bool(out.value)

    def geometry(self):
        a, b, c = ctypes.c_size_t(), ctypes.c_size_t(), ctypes.c_size_t()
        check(_lib().helix_paged_cache_geometry(self._h, ctypes.byref(a), ctypes.byref(b),
                                                ctypes.byref(c)))
        return a.value, b.value, c.value

    def layer_pool_pointers(self, layer):
        k, v = ctypes.c_void_p(), ctypes.c_void_p()
        check(_lib().helix_paged_cache_layer_pools(self._h, layer, ctypes.byref(k),
                                                   ctypes.byref(v)))
        return k.value, v.value

    def layer_pools(self, layer):
        """Device copies of layer `layer`'s pools [physical, kv_heads, block_tokens, dim]
        (float32, bfloat16 for a bf16 cache, uint8 E4M3 codes for an fp8 cache)."""
        import torch
        kp, vp = self.layer_pool_pointers(layer)
        shape = (self.physical_blocks, self.kv_heads, self.block_tokens, self.head_dimension)
        dtype = {"bf16": torch.bfloat16, "fp8": torch.uint8}.get(self.page_dtype, torch.float32)
        out = []
        for p in (kp, vp):
            t = torch.empty(shape, dtype=dtype, device=f"cuda:{self.device}")
            device_copy(t.data_ptr(), p, t.numel() * t.element_size())
            out.append(t)
        return out[0], out[1]

    def read_sequence(self, seq):
        return DecodeView(self, seq)


class DecodeView:
    """Read lease on one sequence; holds the cache lock until released."""

    def __init__(self, cache, seq):
        h = ctypes.c_void_p()
        check(_lib().helix_paged_cache_read_sequence(cache._h, seq, ctypes.byref(h)))
        self._h = h
        self._cache = cache

    def release(self):
        if getattr(self, "_h", None):
            _lib().helix_decode_view_release(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.release()

    def __del__(self, _finalizing=sys.is_finalizing):
        if _finalizing():
            return  # the process is exiting; the driver reclaims device memory
        self.release()

    def length(self):
        out = ctypes.c_size_t()
        check(_lib().helix_decode_view_length(self._h, ctypes.byref(out)))
        return out.value

    def physical_blocks(self):
        p, n = ctypes.POINTER(ctypes.c_uint32)(), ctypes.c_size_t()
        check(_lib().helix_decode_view_physical_blocks(self._h, ctypes.byref(p), ctypes.byref(n)))
        return [p[i] for i in range(n.value)]

    def block_table(self):
        p = ctypes.c_void_p()
        check(_lib().helix_decode_view_block_table(self._h, ctypes.byref(p)))
        return p.value

    def layer_pool_pointers(self, layer):
        k, v = ctypes.c_void_p(), ctypes.c_void_p()
        check(_lib().helix_decode_view_layer_pools(self._h, layer, ctypes.byref(k),
                                                   ctypes.byref(v)))
        return k.value, v.value

    def poison(self):
        _lib().helix_decode_view_poison(self._h)


class PagedBlockTable:
    """Validated device copy of a logical->physical page mapping."""

    def __init__(self, physical_blocks, physical_block_count, device=0):
        ids = (ctypes.c_uint32 * max(1, len(physical_blocks)))(*physical_blocks)
        h = ctypes.c_void_p()
        check(_lib().helix_block_table_create(ids, len(physical_blocks), physical_block_count,
                                              device, ctypes.byref(h)))
        self._h = h
        self.logical_block_count = len(physical_blocks)
        self.physical_block_count = physical_block_count

    def data(self):
        return _lib().helix_block_table_data(self._h)

    def __del__(self, _finalizing=sys.is_finalizing):
        if _finalizing():
            return  # the process is exiting; the driver reclaims device memory
        h = getattr(self, "_h", None)
        if h:
            _lib().helix_block_table_destroy(h)
            self._h = None


# ------------------------------------------------------------- attention ----
def rope_out(input, cosine, sine, output, positions=None, stream=None):
    """kernels::rope / cpu::rope_out (src/kernels/cpu/reference.cpp:490-533) on
    device tensors: input/output [tokens, ..., head_dim] float32 (output may
    be input), cosine/sine [rows, head_dim / 2].  Without positions token t
    uses row t (rows must equal tokens); with int32 positions [tokens] it uses
    row positions[t]."""
    tokens, head_dim = input.shape[0], input.shape[-1]
    vectors = input.numel() // (tokens * head_dim) if tokens and head_dim else 0
    check(_lib().helix_rope(_ptr(input), _ptr(output), tokens, vectors, head_dim, _ptr(cosine),
                            _ptr(sine), cosine.shape[0],
                            None if positions is None else _ptr(positions), _stream(stream)))
    return output


def rope(input, cosine, sine, positions=None, stream=None):
    import torch
    return rope_out(input, cosine, sine, torch.empty_like(input), positions, stream)


def paged_attention_out(query, key_blocks, value_blocks, block_table, kv_tokens,
                        query_position_offset, output, score_workspace, stream=None):
    """paged_scaled_dot_product_attention_out; block_table: device uint32 pointer or tensor."""
    hq, nq, kd = query.shape
    n, hkv, p, vd = value_blocks.shape
    table_ptr = block_table.data_ptr() if hasattr(block_table, "data_ptr") else block_table
    logical = 0 if kv_tokens == 0 else (kv_tokens - 1) // p + 1
    check(_lib().helix_paged_attention_out(
        _ptr(query), hq, nq, kd, _ptr(key_blocks), _ptr(value_blocks), n, hkv, p, vd,
        ctypes.c_void_p(table_ptr), logical, kv_tokens, query_position_offset, _ptr(output),
        _ptr(score_workspace), score_workspace.numel(), _stream(stream)))


def paged_attention_with_tail_out(query, key_blocks, value_blocks, block_table, history_tokens,
                                  tail_key, tail_value, output, score_workspace, stream=None,
                                  logical_blocks=None, probabilities=False):
    """paged_scaled_dot_product_attention_with_tail_out; score_workspace
    [q_heads, tail, history + tail] receives the softmax probabilities, as
    the reference's contract says.  probabilities=True selects the exact
    scalar kernel for every shape
    (helix_paged_attention_with_tail_probabilities_out)."""
    hq, t, kd = query.shape
    n, hkv, p, vd = value_blocks.shape
    table_ptr = block_table.data_ptr() if hasattr(block_table, "data_ptr") else block_table
    if logical_blocks is None:
        logical_blocks = 0 if history_tokens == 0 else (history_tokens - 1) // p + 1
    fn = (_lib().helix_paged_attention_with_tail_probabilities_out if probabilities
          else _lib().helix_paged_attention_with_tail_out)
    check(fn(_ptr(query), hq, t, kd, _ptr(key_blocks), _ptr(value_blocks), n, hkv, p, vd,
             ctypes.c_void_p(table_ptr), logical_blocks, history_tokens, _ptr(tail_key),
             _ptr(tail_value), _ptr(output), _ptr(score_workspace), score_workspace.numel(),
             _stream(stream)))


def decode_workspace_bytes(batch, q_heads, kv_heads, max_blocks, pages_per_split=0):
    out = ctypes.c_size_t()
    check(_lib().helix_paged_decode_workspace_bytes(batch, q_heads, kv_heads, max_blocks,
                                                    pages_per_split, ctypes.byref(out)))
    return out.value


def decode_workspace(batch, q_heads, kv_heads, max_blocks, pages_per_split=0, device="cuda:0",
                     stream=None):
    """Allocate and zero a decode workspace (torch uint8 tensor)."""
    import torch
    n = decode_workspace_bytes(batch, q_heads, kv_heads, max_blocks, pages_per_split)
    ws = torch.empty(max(n, 16), dtype=torch.uint8, device=device)
    check(_lib().helix_paged_decode_workspace_init(_ptr(ws), ws.numel(), _stream(stream)))
    return ws


_PAGE_DTYPES = {"f32": 0, "bf16": 1, "fp8": 2}


def paged_decode_attention(query, key_pool, value_pool, tables, lengths, tail_key, tail_value,
                           output, workspace, pages_per_split=0, stream=None, pool_shape=None,
                           page_dtype="f32", k_scale=1.0, v_scale=1.0):
    """Batched decode: query [B, Hq, 128]; pools [N, Hkv, 16, 128] tensors (or raw
    device addresses with pool_shape) of page_dtype "f32", "bf16" or "fp8"
    (E4M3 codes with scales k_scale / v_scale, pools as uint8 / int16 / any
    tensor whose bytes are the pages); tables [B, max_blocks] int32/uint32;
    lengths [B] int32; tail [B, Hkv, 128]; output [B, Hq, 128]."""
    b, hq, _ = query.shape
    if pool_shape is None:
        pool_shape = tuple(key_pool.shape)
        key_pool, value_pool = key_pool.data_ptr(), value_pool.data_ptr()
    n, hkv, p, d = pool_shape
    dtype = _PAGE_DTYPES.get(page_dtype, page_dtype)
    check(_lib().helix_paged_decode_attention_typed(
        _ptr(query), b, hq, hkv, d, ctypes.c_void_p(key_pool), ctypes.c_void_p(value_pool), n,
        p, _ptr(tables),
        tables.shape[1], _ptr(lengths), _ptr(tail_key), _ptr(tail_value), _ptr(output),
        _ptr(workspace), workspace.numel() * workspace.element_size(), pages_per_split,
        dtype, k_scale, v_scale, _stream(stream)))


def append_slots(keys, values, key_pool, value_pool, slots, stream=None):
    """Write rows [count, Hkv, D] into one layer's pools at int64 slots."""
    n, hkv, p, d = key_pool.shape
    check(_lib().helix_paged_append_slots(_ptr(keys), _ptr(values), _ptr(key_pool),
                                          _ptr(value_pool), n, hkv, p, d, _ptr(slots),
                                          slots.numel(), _stream(stream)))


def paged_prefill_attention(query, key_pool, value_pool, tables, lengths, chunk_key,
                            chunk_value, output, stream=None, pool_shape=None,
                            page_dtype="f32", k_scale=1.0, v_scale=1.0):
    """Batched chunked prefill (MFMA): query [B, Hq, T, 128]; pools [N, Hkv, 16,
    128] tensors (or raw device addresses with pool_shape) of page_dtype
    "f32", "bf16" or "fp8" (scales k_scale / v_scale); tables [B,
    max_blocks] int32/uint32; lengths [B] int32 history tokens; chunk_key /
    chunk_value [B, Hkv, T, 128] fp32; output [B, Hq, T, 128]."""
    b, hq, t, _ = query.shape
    if pool_shape is None:
        pool_shape = tuple(key_pool.shape)
        key_pool, value_pool = key_pool.data_ptr(), value_pool.data_ptr()
    n, hkv, p, d = pool_shape
    dtype = _PAGE_DTYPES.get(page_dtype, page_dtype)
    check(_lib().helix_paged_prefill_attention_typed(
        _ptr(query), b, hq, hkv, t, d, ctypes.c_void_p(key_pool), ctypes.c_void_p(value_pool),
        n, p, _ptr(tables), tables.shape[1], _ptr(lengths), _ptr(chunk_key), _ptr(chunk_value),
        _ptr(output), dtype, k_scale, v_scale, _stream(stream)))


def append_chunk(keys, values, key_pool, value_pool, slots, stream=None):
    """Write rows [B, Hkv, T, D] into one layer's pools at int64 slots [B, T]."""
    n, hkv, p, d = key_pool.shape
    b, t = slots.shape
    check(_lib().helix_paged_append_chunk(_ptr(keys), _ptr(values), _ptr(key_pool),
                                          _ptr(value_pool), n, hkv, p, d, _ptr(slots), b, t,
                                          _stream(stream)))


class DecodeBatch:
    """Batched decode driver over a PagedKvCache (persistent device tables)."""

    def __init__(self, cache, sequences, q_heads, max_tokens, pages_per_split=0):
        arr = (Sequence * len(sequences))(*sequences)
        h = ctypes.c_void_p()
        check(_lib().helix_decode_batch_create(cache._h, arr, len(sequences), q_heads, max_tokens,
                                               pages_per_split, ctypes.byref(h)))
        self._h = h
        self._cache = cache
        self.batch = len(sequences)

    def close(self):
        h = getattr(self, "_h", None)
        if h:
            _lib().helix_decode_batch_destroy(h)
            self._h = None

    def __del__(self, _finalizing=sys.is_finalizing):
        if _finalizing():
            return  # the process is exiting; the driver reclaims device memory
        self.close()

    def prepare(self, stream=None):
        check(_lib().helix_decode_batch_prepare(self._h, _stream(stream)))

    def append_attention_layer(self, layer, query, keys, values, output, stream=None):
        """append_layer + attention_layer in one decode launch (the new token
        rows are the attention tail and are written to their slots)."""
        check(_lib().helix_decode_batch_append_attention_layer(
            self._h, layer, _ptr(query), _ptr(keys), _ptr(values), _ptr(output),
            _stream(stream)))

    def prepare_chunk(self, tokens, stream=None):
        """Reserve `tokens` slots per sequence (chunked prefill step)."""
        check(_lib().helix_decode_batch_prepare_chunk(self._h, tokens, _stream(stream)))

    def prefill_layer(self, layer, query, chunk_key, chunk_value, output, stream=None):
        check(_lib().helix_decode_batch_prefill_layer(self._h, layer, _ptr(query),
                                                      _ptr(chunk_key), _ptr(chunk_value),
                                                      _ptr(output), _stream(stream)))

    def append_layer(self, layer, keys, values, stream=None):
        check(_lib().helix_decode_batch_append_layer(self._h, layer, _ptr(keys), _ptr(values),
                                                     _stream(stream)))

    def append_all_layers(self, keys, values, stream=None):
        """append_layer for every layer in one launch: rows [layers, batch,
        kv_heads, tokens, head_dim] (the step's token committed after the
        forward pass, as CudaPagedKvCache::append commits [layers, kv_heads,
        head_dim] for one sequence)."""
        check(_lib().helix_decode_batch_append_all_layers(self._h, _ptr(keys), _ptr(values),
                                                          _stream(stream)))

    def rope(self, query, key, cosine, sine, stream=None):
        """Rotary embedding of the step's query [batch, q_heads, dim] and key
        [batch, kv_heads, dim] in place, each sequence at its position (its
        length before the step); cosine/sine [rows, dim / 2]."""
        check(_lib().helix_decode_batch_rope(self._h, _ptr(query), _ptr(key), _ptr(cosine),
                                             _ptr(sine), cosine.shape[0], _stream(stream)))

    def attention_layer(self, layer, query, tail_key, tail_value, output, stream=None):
        check(_lib().helix_decode_batch_attention_layer(self._h, layer, _ptr(query),
                                                        _ptr(tail_key), _ptr(tail_value),
                                                        _ptr(output), _stream(stream)))

    def shared_pages(self):
        """Leading pages the prepared decode step attends once for the batch."""
        n = ctypes.c_size_t()
        check(_lib().helix_decode_batch_shared_pages(self._h, ctypes.byref(n)))
        return n.value

    def set_timing_event(self, event):
        """Record `event` (a torch.cuda.Event or None) between the main decode
        kernel and the merge kernel of every attention_layer()."""
        if event is not None:
            event = ctypes.c_void_p(event.cuda_event if hasattr(event, "cuda_event") else event)
        check(_lib().helix_decode_batch_set_timing_event(self._h, event))

    def device_state(self):
        t, l, s = ctypes.c_void_p(), ctypes.c_void_p(), ctypes.c_void_p()
        mb, ps = ctypes.c_size_t(), ctypes.c_size_t()
        check(_lib().helix_decode_batch_tables(self._h, ctypes.byref(t), ctypes.byref(l),
                                               ctypes.byref(s), ctypes.byref(mb),
                                               ctypes.byref(ps)))
        return {"tables": t.value, "lengths": l.value, "slots": s.value,
                "max_blocks": mb.value, "pages_per_split": ps.value}


# ---------------------------------------------------------------- plumbing ----
_hip = None


def device_copy(dst: int, src: int, nbytes: int):
    """hipMemcpy device-to-device (plumbing for reading raw pool memory)."""
    global _hip
    if _hip is None:
        _hip = ctypes.CDLL("libamdhip64.so")
        _hip.hipMemcpy.restype = ctypes.c_int
        _hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    rc = _hip.hipMemcpy(ctypes.c_void_p(dst), ctypes.c_void_p(src), nbytes, 3)
    if rc != 0:
        raise HelixError(RUNTIME, f"hipMemcpy failed with {rc}")
