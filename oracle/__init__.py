"""CPU oracle for the paged-KV hot path -- TEST INFRASTRUCTURE ONLY.

numpy/ctypes front end of ``oracle/paged_oracle.cpp``, a C++ restatement of
the reference's CPU paged KV cache (``src/kv_cache/paged.cpp``) and CPU paged
attention (``src/attention/paged_reference.cpp:173-384`` with the softmax of
``src/kernels/cpu/reference.cpp:264-316``).  Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import this package, and only as the checker / CPU baseline: the product path
(``helix_runtime_amd``) never calls it.

Parity pinning of each oracle function is recorded in ``tests/test_oracle.py``.
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")

STATUS_OK = 0
INVALID_ARGUMENT = 1
OUT_OF_RANGE = 2
UNSUPPORTED = 3
RESOURCE_EXHAUSTED = 4


class OracleError(RuntimeError):
    def __init__(self, code: int, what: str):
        super().__init__(f"{what}: oracle status {code}")
        self.code = code


def build() -> str:
    """Compile the oracle library with its Makefile (g++ only)."""
    subprocess.run(["make", "-s", "-C", _HERE, "liboracle.so"], check=True)
    return _LIB_PATH


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        _declare(_lib)
    return _lib


_fp = ctypes.POINTER(ctypes.c_float)
_u32p = ctypes.POINTER(ctypes.c_uint32)
_i32p = ctypes.POINTER(ctypes.c_int32)
_sz = ctypes.c_size_t
_u64 = ctypes.c_uint64


class Stats(ctypes.Structure):
    _fields_ = [(name, ctypes.c_uint64) for name in (
        "bytes_reserved", "bytes_used", "bytes_free", "peak_bytes_used",
        "total_blocks", "used_blocks", "free_blocks", "active_sequence_count",
        "active_tokens", "resident_tokens", "allocated_token_slots",
        "block_reference_count", "shared_blocks",
        "sequence_create_count", "sequence_fork_count", "append_count", "release_count",
        "block_allocation_count", "block_reuse_count")]

    def as_dict(self):
        return {name: getattr(self, name) for name, _ in self._fields_}


def _declare(l):
    l.oracle_pool_create.restype = ctypes.c_void_p
    l.oracle_pool_create.argtypes = [_sz, _sz, _sz, _sz, _sz, ctypes.POINTER(ctypes.c_int)]
    l.oracle_pool_destroy.argtypes = [ctypes.c_void_p]
    l.oracle_bytes_per_token.restype = _sz
    l.oracle_bytes_per_token.argtypes = [ctypes.c_void_p]
    l.oracle_block_bytes.restype = _sz
    l.oracle_block_bytes.argtypes = [ctypes.c_void_p]
    l.oracle_create_sequence.restype = _u64
    l.oracle_create_sequence.argtypes = [ctypes.c_void_p]
    l.oracle_fork_sequence.argtypes = [ctypes.c_void_p, _u64, _sz, ctypes.c_int,
                                       ctypes.POINTER(_u64)]
    l.oracle_append.argtypes = [ctypes.c_void_p, _u64, _fp, _fp]
    l.oracle_append_layer_major.argtypes = [ctypes.c_void_p, _u64, _fp, _fp, _sz]
    l.oracle_release_sequence.argtypes = [ctypes.c_void_p, _u64]
    l.oracle_length.restype = _sz
    l.oracle_length.argtypes = [ctypes.c_void_p, _u64]
    l.oracle_block_table.restype = _sz
    l.oracle_block_table.argtypes = [ctypes.c_void_p, _u64, _u32p, _sz]
    l.oracle_stats.argtypes = [ctypes.c_void_p, ctypes.POINTER(Stats)]
    l.oracle_copy_layer.argtypes = [ctypes.c_void_p, _u64, _sz, _fp, _fp, _sz]
    l.oracle_layer_pages.argtypes = [ctypes.c_void_p, _sz, _fp, _fp]
    l.oracle_block_token_count.restype = _sz
    l.oracle_block_token_count.argtypes = [ctypes.c_void_p, ctypes.c_uint32]
    l.oracle_block_refcount.restype = _sz
    l.oracle_block_refcount.argtypes = [ctypes.c_void_p, ctypes.c_uint32]
    l.oracle_paged_attention.argtypes = [_fp, _sz, _sz, _sz, _sz, _sz, _fp, _fp, _sz, _u32p,
                                         _sz, _fp, _fp, _sz, _sz, _fp, _fp]
    l.oracle_batched_decode.argtypes = [_fp, _sz, _sz, _sz, _sz, _fp, _fp, _sz, _u32p, _sz,
                                        _i32p, _fp, _fp, _fp, ctypes.c_int]
    l.oracle_sdpa.argtypes = [_fp, _fp, _fp, _sz, _sz, _sz, _sz, _sz, _sz, _fp, _fp]
    l.oracle_softmax_rows.argtypes = [_fp, _sz, _sz]
    l.oracle_random_uniform.argtypes = [_u64, ctypes.c_float, ctypes.c_float, _fp, _sz]
    l.oracle_random_normal.argtypes = [_u64, _fp, _sz]
    l.oracle_mt19937_64_nth.restype = _u64
    l.oracle_mt19937_64_nth.argtypes = [_u64, _sz]


def _f(a):
    if a is None:
        return None
    assert a.dtype == np.float32 and a.flags.c_contiguous
    return a.ctypes.data_as(_fp)


def _u(a):
    if a is None:
        return None
    assert a.dtype == np.uint32 and a.flags.c_contiguous
    return a.ctypes.data_as(_u32p)


def _check(code, what):
    if code != STATUS_OK:
        raise OracleError(code, what)


# ------------------------------------------------------------------ inputs --
def random_uniform(shape, seed, lower=-1.0, upper=1.0):
    """Tensor::random_uniform(shape, seed, lower, upper) of the reference."""
    out = np.empty(shape, dtype=np.float32)
    lib().oracle_random_uniform(seed, lower, upper, _f(out), out.size)
    return out


def random_normal(shape, seed):
    out = np.empty(shape, dtype=np.float32)
    lib().oracle_random_normal(seed, _f(out), out.size)
    return out


# ------------------------------------------------------------ bf16 pages --
# Extension (no reference counterpart: the reference stores fp32 only,
# docs/KV_CACHE.md:531).  The contract of bf16 pages: a page element is the
# fp32 value rounded to nearest, ties to even (IEEE 754 roundTiesToEven onto
# the 8-bit-mantissa grid); NaN stays NaN with the sign and top payload bits
# kept and the quiet bit set; finite values that round past the largest bf16
# become inf.  Attention over bf16 pages is the fp32 reference evaluated on
# those rounded values.
def bf16_bits(x):
    """uint16 bf16 encodings of float32 values."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    rounded = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return np.where(nan, (u >> 16) | 0x40, rounded).astype(np.uint16)


def round_bf16(x):
    """float32 values moved onto the bf16 grid."""
    return (bf16_bits(x).astype(np.uint32) << 16).view(np.float32)


# ------------------------------------------------------------- fp8 pages --
# Extension (no reference counterpart, as bf16 above).  fp8 pages hold OCP
# FP8 E4M3 ("e4m3fn": 1 sign, 4 exponent bits of bias 7, 3 mantissa bits; no
# infinities; 0x7f / 0xff are NaN; largest finite 448) with one fp32 scale per
# cache for keys and one for values.  The contract: a page element is the
# code of x / scale (an fp32 division) rounded to nearest, ties to even,
# saturating: values past 448 (infinities included) become +-448, NaN
# stays NaN (0x7f with the sign).  Its value is decode(code) * scale (an
# fp32 product).  Attention over fp8 pages is the fp32 reference evaluated
# on those values; the step's fp32 tail rows and chunk rows go through the
# same rounding (they are the values their pages hold once appended).
FP8_MAX = 448.0


def fp8_decode(codes):
    """float32 values of E4M3 codes (uint8), from the format's definition."""
    c = np.asarray(codes, dtype=np.uint8).astype(np.int64)
    sign = np.where(c & 0x80, -1.0, 1.0)
    e = (c >> 3) & 0xF
    m = c & 0x7
    mag = np.where(e == 0, m * 2.0 ** -9, (1.0 + m / 8.0) * 2.0 ** (e - 7))
    mag = np.where((c & 0x7F) == 0x7F, np.nan, mag)
    return (sign * mag).astype(np.float32)


_FP8_TABLE = fp8_decode(np.arange(128, dtype=np.uint8)[:127]).astype(np.float64)  # 0 .. 448


def fp8_bits(x, scale=1.0):
    """uint8 E4M3 codes of float32 values divided by ``scale`` (saturating,
    ties to even), by nearest search over the 127 non-negative finite codes."""
    with np.errstate(invalid="ignore"):
        y = np.ascontiguousarray(x, dtype=np.float32) / np.float32(scale)
    a = np.abs(y.astype(np.float64)).ravel()
    nan = np.isnan(a)
    a = np.where(nan, 0.0, np.minimum(a, FP8_MAX))
    hi = np.searchsorted(_FP8_TABLE, a, side="left")          # first code >= a
    hi = np.minimum(hi, 126)
    lo = np.maximum(hi - 1, 0)
    dlo = a - _FP8_TABLE[lo]
    dhi = _FP8_TABLE[hi] - a
    pick_hi = (dhi < dlo) | ((dhi == dlo) & (hi % 2 == 0))
    code = np.where(a == _FP8_TABLE[hi], hi, np.where(pick_hi, hi, lo))
    code = np.where(nan, 0x7F, code)
    sign = (y.view(np.uint32).ravel() >> 31).astype(np.int64) << 7
    return (code | sign).astype(np.uint8).reshape(np.shape(y))


def round_fp8(x, scale=1.0):
    """float32 values moved onto the scaled fp8 grid: decode(code) * scale."""
    return fp8_decode(fp8_bits(x, scale)) * np.float32(scale)


def mt19937_64_nth(seed, n):
    return int(lib().oracle_mt19937_64_nth(seed, n))


# ---------------------------------------------------------------- the pool --
class PagedPool:
    """Restatement of the reference's CPU ``PagedKvCache`` (paged.cpp)."""

    def __init__(self, layers, kv_heads, head_dim, block_tokens, physical_blocks):
        status = ctypes.c_int(0)
        self.layers, self.kv_heads, self.head_dim = layers, kv_heads, head_dim
        self.block_tokens, self.physical_blocks = block_tokens, physical_blocks
        self._p = lib().oracle_pool_create(layers, kv_heads, head_dim, block_tokens,
                                           physical_blocks, ctypes.byref(status))
        _check(status.value, "PagedPool")

    def __del__(self):
        p = getattr(self, "_p", None)
        if p:
            lib().oracle_pool_destroy(p)
            self._p = None

    def bytes_per_token(self):
        return lib().oracle_bytes_per_token(self._p)

    def block_bytes(self):
        return lib().oracle_block_bytes(self._p)

    def create_sequence(self):
        return lib().oracle_create_sequence(self._p)

    def fork_sequence(self, source, prefix, allow_cow=False):
        out = _u64(0)
        _check(lib().oracle_fork_sequence(self._p, source, prefix, int(allow_cow),
                                          ctypes.byref(out)), "fork_sequence")
        return out.value

    def append(self, seq, keys, values):
        keys = np.ascontiguousarray(keys, dtype=np.float32)
        values = np.ascontiguousarray(values, dtype=np.float32)
        assert keys.shape == (self.layers, self.kv_heads, self.head_dim)
        _check(lib().oracle_append(self._p, seq, _f(keys), _f(values)), "append")

    def append_layer_major(self, seq, keys, values):
        """keys/values: [L, H, T, D]."""
        keys = np.ascontiguousarray(keys, dtype=np.float32)
        values = np.ascontiguousarray(values, dtype=np.float32)
        _check(lib().oracle_append_layer_major(self._p, seq, _f(keys), _f(values),
                                               keys.shape[2]), "append_layer_major")

    def release_sequence(self, seq):
        _check(lib().oracle_release_sequence(self._p, seq), "release_sequence")

    def length(self, seq):
        return lib().oracle_length(self._p, seq)

    def block_table(self, seq):
        cap = self.physical_blocks
        out = np.zeros(cap, dtype=np.uint32)
        n = lib().oracle_block_table(self._p, seq, _u(out), cap)
        return out[:n].copy()

    def stats(self):
        s = Stats()
        lib().oracle_stats(self._p, ctypes.byref(s))
        return s.as_dict()

    def copy_layer(self, seq, layer, dest_tokens=None, fill=0.0):
        n = self.length(seq)
        dest = n if dest_tokens is None else dest_tokens
        k = np.full((self.kv_heads, dest, self.head_dim), fill, dtype=np.float32)
        v = np.full((self.kv_heads, dest, self.head_dim), fill, dtype=np.float32)
        _check(lib().oracle_copy_layer(self._p, seq, layer, _f(k), _f(v), dest), "copy_layer")
        return k, v

    def layer_pages(self, layer):
        shape = (self.physical_blocks, self.kv_heads, self.block_tokens, self.head_dim)
        k = np.empty(shape, dtype=np.float32)
        v = np.empty(shape, dtype=np.float32)
        lib().oracle_layer_pages(self._p, layer, _f(k), _f(v))
        return k, v

    def block_token_count(self, block):
        return lib().oracle_block_token_count(self._p, block)

    def block_refcount(self, block):
        return lib().oracle_block_refcount(self._p, block)


# ---------------------------------------------------------------- attention --
def paged_attention(query, key_blocks, value_blocks, block_table, history,
                    tail_key=None, tail_value=None, query_position_offset=None):
    """Paged SDPA: query [Hq, T, D]; blocks [N, Hkv, P, D|DV]; tail [Hkv, T, D|DV].

    Returns (output [Hq, T, DV], probabilities [Hq, T, history + tail]).
    """
    query = np.ascontiguousarray(query, dtype=np.float32)
    key_blocks = np.ascontiguousarray(key_blocks, dtype=np.float32)
    value_blocks = np.ascontiguousarray(value_blocks, dtype=np.float32)
    table = np.ascontiguousarray(block_table, dtype=np.uint32)
    hq, t, d = query.shape
    _, hkv, p, dv = value_blocks.shape
    tail = 0 if tail_key is None else tail_key.shape[1]
    if tail:
        tail_key = np.ascontiguousarray(tail_key, dtype=np.float32)
        tail_value = np.ascontiguousarray(tail_value, dtype=np.float32)
        offset = history
    else:
        offset = query_position_offset
    out = np.zeros((hq, t, dv), dtype=np.float32)
    ws = np.zeros((hq, t, history + tail), dtype=np.float32)
    _check(lib().oracle_paged_attention(_f(query), hq, hkv, t, d, dv, _f(key_blocks),
                                        _f(value_blocks), p, _u(table), history,
                                        _f(tail_key), _f(tail_value), tail, offset,
                                        _f(out), _f(ws)), "paged_attention")
    return out, ws


def batched_decode(query, key_blocks, value_blocks, tables, lengths, tail_key, tail_value,
                   threads=1):
    """Per-sequence loop of the decode-with-tail oracle.

    query [B, Hq, D]; blocks [N, Hkv, P, D]; tables [B, max_blocks] uint32;
    lengths [B] int32 (history tokens); tail [B, Hkv, D].  Returns [B, Hq, D].
    """
    query = np.ascontiguousarray(query, dtype=np.float32)
    b, hq, d = query.shape
    _, hkv, p, _ = key_blocks.shape
    tables = np.ascontiguousarray(tables, dtype=np.uint32)
    lengths = np.ascontiguousarray(lengths, dtype=np.int32)
    out = np.zeros((b, hq, d), dtype=np.float32)
    _check(lib().oracle_batched_decode(
        _f(query), b, hq, hkv, d, _f(np.ascontiguousarray(key_blocks)),
        _f(np.ascontiguousarray(value_blocks)), p, _u(tables), tables.shape[1],
        lengths.ctypes.data_as(_i32p), _f(np.ascontiguousarray(tail_key)),
        _f(np.ascontiguousarray(tail_value)), _f(out), threads), "batched_decode")
    return out


def sdpa(query, key, value, query_position_offset):
    """Contiguous SDPA of src/attention/reference.cpp; returns (out, probabilities)."""
    query = np.ascontiguousarray(query, dtype=np.float32)
    key = np.ascontiguousarray(key, dtype=np.float32)
    value = np.ascontiguousarray(value, dtype=np.float32)
    h, q, d = query.shape
    k = key.shape[1]
    dv = value.shape[2]
    out = np.zeros((h, q, dv), dtype=np.float32)
    ws = np.zeros((h, q, k), dtype=np.float32)
    _check(lib().oracle_sdpa(_f(query), _f(key), _f(value), h, q, k, d, dv,
                             query_position_offset, _f(out), _f(ws)), "sdpa")
    return out, ws


def softmax_rows(x):
    x = np.array(x, dtype=np.float32, copy=True)
    width = x.shape[-1]
    lib().oracle_softmax_rows(_f(x), x.size // width, width)
    return x


def pack_logical_blocks(logical, table, physical_blocks, block_tokens, padding):
    """Scatter a logical [H, tokens, W] tensor into [N, H, P, W] pages.

    Same fixture construction as the reference's ``pack_logical_blocks``
    (tests/cuda_attention_test.cpp:32-54): untouched slots hold ``padding``.
    """
    h, tokens, w = logical.shape
    packed = np.full((physical_blocks, h, block_tokens, w), padding, dtype=np.float32)
    for t in range(tokens):
        packed[table[t // block_tokens], :, t % block_tokens, :] = logical[:, t, :]
    return packed
