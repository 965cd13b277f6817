"""ctypes declarations of ``include/helix_paged.h`` (libhelix_paged.so).

The library is built in-tree by ``helix_runtime_amd/Makefile`` (see
``helix_runtime_amd.build``).  Loading fails loudly when it is missing: there
is no fallback implementation of any entry point.
"""

from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libhelix_paged.so")

c_size = ctypes.c_size_t
c_int = ctypes.c_int
c_u32 = ctypes.c_uint32
c_u64 = ctypes.c_uint64
c_float = ctypes.c_float
vp = ctypes.c_void_p


class Config(ctypes.Structure):
    _fields_ = [("layers", c_size), ("kv_heads", c_size), ("head_dimension", c_size),
                ("block_tokens", c_size), ("physical_blocks", c_size)]


STAT_FIELDS = (
    "bytes_reserved", "bytes_used", "bytes_free", "peak_bytes_used",
    "total_blocks", "used_blocks", "free_blocks", "active_sequence_count",
    "active_tokens", "resident_tokens", "allocated_token_slots",
    "block_reference_count", "shared_blocks",
    "sequence_create_count", "sequence_fork_count", "append_count", "release_count",
    "block_allocation_count", "block_reuse_count")


class Stats(ctypes.Structure):
    _fields_ = [(n, c_u64) for n in STAT_FIELDS]

    def as_dict(self):
        return {n: int(getattr(self, n)) for n in STAT_FIELDS}


class Sequence(ctypes.Structure):
    _fields_ = [("id", c_u64), ("cache_id", c_u64)]

    def __eq__(self, other):
        return isinstance(other, Sequence) and (self.id, self.cache_id) == (other.id, other.cache_id)

    def __hash__(self):
        return hash((self.id, self.cache_id))

    def __bool__(self):
        return self.id != 0

    def __repr__(self):
        return f"Sequence(id={self.id}, cache_id={self.cache_id})"


class CowCopy(ctypes.Structure):
    _fields_ = [("from_block", c_u32), ("to_block", c_u32), ("tokens", c_size)]


PREFIX_STAT_FIELDS = (
    "maximum_entries", "maximum_block_references", "entry_count", "retained_tokens",
    "retained_block_references", "peak_entries", "peak_block_references",
    "lookup_count", "hit_count", "miss_count", "insertion_count", "duplicate_insertion_count",
    "rejected_insertion_count", "eviction_count", "erase_count")


class PrefixStats(ctypes.Structure):
    _fields_ = [(n, c_u64) for n in PREFIX_STAT_FIELDS]

    def as_dict(self):
        return {n: int(getattr(self, n)) for n in PREFIX_STAT_FIELDS}


class PrefixConfig(ctypes.Structure):
    _fields_ = [("maximum_entries", c_size), ("maximum_block_references", c_size)]


P = ctypes.POINTER

# name -> (restype, argtypes)
SIGNATURES = {
    "helix_last_error": (ctypes.c_char_p, []),
    "helix_status_name": (ctypes.c_char_p, [c_int]),
    # block manager
    "helix_block_manager_create": (c_int, [P(Config), P(vp)]),
    "helix_block_manager_destroy": (None, [vp]),
    "helix_block_manager_create_sequence": (c_int, [vp, P(Sequence)]),
    "helix_block_manager_fork_sequence": (c_int, [vp, Sequence, c_size, c_int, P(Sequence), P(CowCopy)]),
    "helix_block_manager_append": (c_int, [vp, Sequence, c_size, P(c_u64)]),
    "helix_block_manager_release_sequence": (c_int, [vp, Sequence]),
    "helix_block_manager_contains": (c_int, [vp, Sequence, P(c_int)]),
    "helix_block_manager_length": (c_int, [vp, Sequence, P(c_size)]),
    "helix_block_manager_block_table": (c_int, [vp, Sequence, P(c_u32), c_size, P(c_size)]),
    "helix_block_manager_stats": (c_int, [vp, P(Stats)]),
    "helix_block_manager_block_info": (c_int, [vp, c_u32, P(c_size), P(c_size)]),
    "helix_block_manager_validate": (c_int, [vp]),
    "helix_block_manager_geometry": (c_int, [vp, P(c_size), P(c_size), P(c_size)]),
    # device cache
    "helix_paged_cache_create": (c_int, [P(Config), c_int, P(vp)]),
    "helix_paged_cache_destroy": (None, [vp]),
    "helix_paged_cache_create_sequence": (c_int, [vp, P(Sequence)]),
    "helix_paged_cache_fork_sequence": (c_int, [vp, Sequence, c_size, c_int, vp, P(Sequence)]),
    "helix_paged_cache_append": (c_int, [vp, Sequence, vp, vp, vp]),
    "helix_paged_cache_append_layer_major": (c_int, [vp, Sequence, P(vp), P(vp), c_size, vp]),
    "helix_paged_cache_release_sequence": (c_int, [vp, Sequence]),
    "helix_paged_cache_copy_layer_out": (c_int, [vp, Sequence, c_size, vp, vp, vp]),
    "helix_paged_cache_copy_layer_prefix_out": (c_int, [vp, Sequence, c_size, c_size, vp, vp, c_size, vp]),
    "helix_paged_cache_contains": (c_int, [vp, Sequence, P(c_int)]),
    "helix_paged_cache_length": (c_int, [vp, Sequence, P(c_size)]),
    "helix_paged_cache_block_table": (c_int, [vp, Sequence, P(c_u32), c_size, P(c_size)]),
    "helix_paged_cache_stats": (c_int, [vp, P(Stats)]),
    "helix_paged_cache_is_healthy": (c_int, [vp, P(c_int)]),
    "helix_paged_cache_geometry": (c_int, [vp, P(c_size), P(c_size), P(c_size)]),
    "helix_paged_cache_layer_pools": (c_int, [vp, c_size, P(vp), P(vp)]),
    "helix_paged_cache_read_sequence": (c_int, [vp, Sequence, P(vp)]),
    "helix_decode_view_length": (c_int, [vp, P(c_size)]),
    "helix_decode_view_physical_blocks": (c_int, [vp, P(P(c_u32)), P(c_size)]),
    "helix_decode_view_block_table": (c_int, [vp, P(vp)]),
    "helix_decode_view_layer_pools": (c_int, [vp, c_size, P(vp), P(vp)]),
    "helix_decode_view_poison": (None, [vp]),
    "helix_decode_view_release": (None, [vp]),
    "helix_block_table_create": (c_int, [P(c_u32), c_size, c_size, c_int, P(vp)]),
    "helix_block_table_data": (vp, [vp]),
    "helix_block_table_logical_block_count": (c_size, [vp]),
    "helix_block_table_destroy": (None, [vp]),
    # attention
    "helix_paged_score_workspace_bytes": (c_int, [c_size] * 7 + [P(c_size)]),
    "helix_paged_tail_score_workspace_bytes": (c_int, [c_size] * 7 + [P(c_size)]),
    "helix_paged_attention_out": (
        c_int, [vp, c_size, c_size, c_size, vp, vp, c_size, c_size, c_size, c_size, vp, c_size,
                c_size, c_size, vp, vp, c_size, vp]),
    "helix_paged_attention_with_tail_out": (
        c_int, [vp, c_size, c_size, c_size, vp, vp, c_size, c_size, c_size, c_size, vp, c_size,
                c_size, vp, vp, vp, vp, c_size, vp]),
    "helix_paged_attention_with_tail_probabilities_out": (
        c_int, [vp, c_size, c_size, c_size, vp, vp, c_size, c_size, c_size, c_size, vp, c_size,
                c_size, vp, vp, vp, vp, c_size, vp]),
    "helix_paged_decode_attention_noalloc": (
        c_int, [vp, c_size, c_size, c_size, c_size, vp, vp, c_size, c_size, vp, c_size, vp, vp,
                vp, vp, c_int, c_float, c_float, vp]),
    "helix_paged_decode_workspace_bytes": (c_int, [c_size] * 5 + [P(c_size)]),
    "helix_paged_decode_workspace_init": (c_int, [vp, c_size, vp]),
    "helix_paged_decode_attention": (
        c_int, [vp, c_size, c_size, c_size, c_size, vp, vp, c_size, c_size, vp, c_size, vp, vp,
                vp, vp, vp, c_size, c_size, vp]),
    "helix_paged_decode_attention_typed": (
        c_int, [vp, c_size, c_size, c_size, c_size, vp, vp, c_size, c_size, vp, c_size, vp, vp,
                vp, vp, vp, c_size, c_size, c_int, c_float, c_float, vp]),
    "helix_paged_prefill_attention_typed": (
        c_int, [vp, c_size, c_size, c_size, c_size, c_size, vp, vp, c_size, c_size, vp, c_size,
                vp, vp, vp, vp, c_int, c_float, c_float, vp]),
    "helix_paged_append_slots": (
        c_int, [vp, vp, vp, vp, c_size, c_size, c_size, c_size, vp, c_size, vp]),
    "helix_paged_prefill_attention": (
        c_int, [vp, c_size, c_size, c_size, c_size, c_size, vp, vp, c_size, c_size, vp, c_size,
                vp, vp, vp, vp, vp]),
    "helix_paged_append_chunk": (
        c_int, [vp, vp, vp, vp, c_size, c_size, c_size, c_size, vp, c_size, c_size, vp]),
    "helix_decode_batch_prepare_chunk": (c_int, [vp, c_size, vp]),
    "helix_decode_batch_append_attention_layer": (c_int, [vp, c_size, vp, vp, vp, vp, vp]),
    "helix_decode_batch_prefill_layer": (c_int, [vp, c_size, vp, vp, vp, vp, vp]),
    "helix_decode_batch_create": (c_int, [vp, P(Sequence), c_size, c_size, c_size, c_size, P(vp)]),
    "helix_decode_batch_prepare": (c_int, [vp, vp]),
    "helix_decode_batch_append_layer": (c_int, [vp, c_size, vp, vp, vp]),
    "helix_decode_batch_append_all_layers": (c_int, [vp, vp, vp, vp]),
    "helix_decode_batch_rope": (c_int, [vp, vp, vp, vp, vp, c_size, vp]),
    "helix_rope": (c_int, [vp, vp, c_size, c_size, c_size, vp, vp, c_size, vp, vp]),
    "helix_decode_batch_attention_layer": (c_int, [vp, c_size, vp, vp, vp, vp, vp]),
    "helix_decode_batch_tables": (c_int, [vp, P(vp), P(vp), P(vp), P(c_size), P(c_size)]),
    "helix_decode_batch_set_timing_event": (c_int, [vp, vp]),
    "helix_decode_batch_shared_pages": (c_int, [vp, P(c_size)]),
    "helix_decode_batch_destroy": (None, [vp]),
    "helix_paged_cache_create_typed": (c_int, [P(Config), c_int, c_int, P(vp)]),
    "helix_paged_cache_create_fp8": (c_int, [P(Config), c_int, c_float, c_float, P(vp)]),
    "helix_paged_cache_page_dtype": (c_int, [vp, P(c_int)]),
    "helix_paged_cache_fp8_scales": (c_int, [vp, P(c_float), P(c_float)]),
    # prefix cache
    "helix_prefix_cache_create": (c_int, [vp, P(PrefixConfig), P(vp)]),
    "helix_prefix_cache_create_host": (c_int, [vp, P(PrefixConfig), P(vp)]),
    "helix_prefix_cache_destroy": (None, [vp]),
    "helix_prefix_cache_insert": (c_int, [vp, c_u64, P(c_u32), c_size, Sequence, P(c_int)]),
    "helix_prefix_cache_lookup_longest": (c_int, [vp, c_u64, P(c_u32), c_size, c_size, P(c_int),
                                                  P(Sequence), P(c_size)]),
    "helix_prefix_cache_contains": (c_int, [vp, c_u64, P(c_u32), c_size, P(c_int)]),
    "helix_prefix_cache_erase": (c_int, [vp, c_u64, P(c_u32), c_size, P(c_int)]),
    "helix_prefix_cache_evict_lru": (c_int, [vp, P(c_int)]),
    "helix_prefix_cache_clear": (c_int, [vp]),
    "helix_prefix_cache_stats": (c_int, [vp, P(PrefixStats)]),
    "helix_prefix_cache_config": (c_int, [vp, P(PrefixConfig)]),
    "helix_prefix_cache_block_tokens": (c_int, [vp, P(c_size)]),
}

_lib = None


def load():
    """Load libhelix_paged.so; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with helix_runtime_amd.build() "
                "(there is no non-HIP implementation)")
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


class HelixError(RuntimeError):
    """A non-zero helix_status with the library's message."""

    def __init__(self, status: int, message: str):
        self.status = status
        super().__init__(f"[{status}] {message}")


INVALID_ARGUMENT = 1
OUT_OF_RANGE = 2
UNSUPPORTED = 3
RESOURCE_EXHAUSTED = 4
RUNTIME = 5
INTERNAL = 6


def check(status: int):
    if status != 0:
        msg = load().helix_last_error().decode(errors="replace")
        raise HelixError(status, msg)
