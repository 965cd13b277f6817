"""Replays the golden fixtures of tests/golden/ (the reference's own known
answers, transcribed by tests/golden/make_fixtures.py) on a paged-cache
backend: the CPU oracle pool or the HIP library's device cache."""

from __future__ import annotations

import json
import os

import numpy as np

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
STATUS = {"invalid_argument": 1, "out_of_range": 2, "resource_exhausted": 4}


def load(name):
    with open(os.path.join(GOLDEN, name)) as f:
        return json.load(f)


def make_token(layers, heads, dim, base):
    """tests/paged_kv_cache_test.cpp:18-27: base + flat index, [L, H, D]."""
    return (base + np.arange(layers * heads * dim, dtype=np.float64)).astype(
        np.float32).reshape(layers, heads, dim)


def make_layer_major(layers, heads, begin, count, dim, base):
    """tests/paged_kv_cache_test.cpp:29-49: [L, H, count, D] with value
    base + (begin + t) * 100 + (l * H + h) * D + c."""
    out = np.empty((layers, heads, count, dim), np.float32)
    for l in range(layers):
        for h in range(heads):
            for t in range(count):
                for c in range(dim):
                    out[l, h, t, c] = base + (begin + t) * 100 + (l * heads + h) * dim + c
    return out


class OracleBackend:
    def __init__(self, config):
        import oracle
        self.mod = oracle
        self.pool = oracle.PagedPool(*config)

    def create(self):
        return self.pool.create_sequence()

    def append(self, seq, keys, values):
        self.pool.append(seq, keys, values)

    def append_layer_major(self, seq, keys, values):
        self.pool.append_layer_major(seq, keys, values)

    def fork(self, seq, prefix):
        return self.pool.fork_sequence(seq, prefix)

    def release(self, seq):
        self.pool.release_sequence(seq)

    def length(self, seq):
        return self.pool.length(seq)

    def table(self, seq):
        return [int(x) for x in self.pool.block_table(seq)]

    def layer(self, seq, layer):
        return self.pool.copy_layer(seq, layer)

    def stats(self):
        return self.pool.stats()

    def error_status(self, exc):
        return exc.code if isinstance(exc, self.mod.OracleError) else None


class LibraryBackend:
    def __init__(self, config):
        import helix_runtime_amd as hx
        self.hx = hx
        self.cache = hx.PagedKvCache(*config)

    @staticmethod
    def _dev(a):
        import torch
        return torch.from_numpy(np.ascontiguousarray(a)).to("cuda:0")

    def create(self):
        return self.cache.create_sequence()

    def append(self, seq, keys, values):
        self.cache.append(seq, self._dev(keys), self._dev(values))

    def append_layer_major(self, seq, keys, values):
        self.cache.append_layer_major(seq, [self._dev(k) for k in keys],
                                      [self._dev(v) for v in values])

    def fork(self, seq, prefix):
        return self.cache.fork_sequence(seq, prefix)

    def release(self, seq):
        self.cache.release_sequence(seq)

    def length(self, seq):
        return self.cache.length(seq)

    def table(self, seq):
        return list(self.cache.block_table(seq))

    def layer(self, seq, layer):
        import torch
        k, v = self.cache.retrieve_layer(seq, layer)
        torch.cuda.synchronize()
        return k.cpu().numpy(), v.cpu().numpy()

    def stats(self):
        return self.cache.stats()

    def error_status(self, exc):
        return exc.status if isinstance(exc, self.hx.HelixError) else None


def run_scenario(scenario, backend_cls):
    """Executes one scenario; every expectation is asserted on the backend."""
    L, H, D, P, N = scenario["config"]
    b = backend_cls(scenario["config"])
    seqs = {}

    def run(op):
        kind = op["op"]
        if kind == "create":
            seqs[op["seq"]] = b.create()
        elif kind == "append_encoded":
            b.append(seqs[op["seq"]], make_token(L, H, D, op["key_base"]),
                     make_token(L, H, D, op["value_base"]))
        elif kind == "append_values":
            b.append(seqs[op["seq"]], np.array(op["keys"], np.float32).reshape(L, H, D),
                     np.array(op["values"], np.float32).reshape(L, H, D))
        elif kind == "append_layer_major_encoded":
            args = (L, H, op["token_begin"], op["count"], D)
            b.append_layer_major(seqs[op["seq"]], make_layer_major(*args, op["key_base"]),
                                 make_layer_major(*args, op["value_base"]))
        elif kind == "fork":
            seqs[op["new"]] = b.fork(seqs[op["seq"]], op["prefix"])
        elif kind == "release":
            b.release(seqs[op["seq"]])
        elif kind == "expect_error":
            try:
                run(op["inner"])
            except Exception as exc:  # noqa: BLE001 - the backend's own error type
                status = b.error_status(exc)
                assert status is not None, f"unexpected exception {exc!r}"
                if op["status"] != "any":
                    assert status == STATUS[op["status"]], (status, op)
            else:
                raise AssertionError(f"expected an error from {op['inner']}")
        elif kind == "expect_table":
            assert b.table(seqs[op["seq"]]) == op["table"], op
        elif kind == "expect_table_size":
            assert len(b.table(seqs[op["seq"]])) == op["size"], op
        elif kind == "expect_table_last":
            assert b.table(seqs[op["seq"]])[-1] == op["block"], op
        elif kind == "expect_tables_share":
            ta, tb = b.table(seqs[op["a"]]), b.table(seqs[op["b"]])
            assert ta[: op["count"]] == tb[: op["count"]], (ta, tb)
        elif kind == "expect_tables_differ_at":
            ta, tb = b.table(seqs[op["a"]]), b.table(seqs[op["b"]])
            assert ta[op["index"]] != tb[op["index"]], (ta, tb)
        elif kind == "expect_length":
            assert b.length(seqs[op["seq"]]) == op["length"], op
        elif kind == "expect_layer":
            k, v = b.layer(seqs[op["seq"]], op["layer"])
            np.testing.assert_array_equal(k.ravel(), np.array(op["keys"], np.float32))
            np.testing.assert_array_equal(v.ravel(), np.array(op["values"], np.float32))
        elif kind == "expect_layer_element":
            k, v = b.layer(seqs[op["seq"]], op["layer"])
            assert k.ravel()[op["index"]] == op["key"] and v.ravel()[op["index"]] == op["value"]
        elif kind == "expect_stats":
            st = b.stats()
            for name, value in op["stats"].items():
                assert st[name] == value, (name, st[name], value)
        else:
            raise ValueError(f"unknown fixture op {kind}")

    for op in scenario["ops"]:
        run(op)


def pack_pages(logical, table, physical_blocks, block_tokens, padding):
    """[H, tokens, D] history -> pool [physical, H, block_tokens, D] through
    the block table, unused slots set to padding
    (tests/cuda_attention_test.cpp:32-54 builds its pools the same way)."""
    h, t, d = logical.shape
    pool = np.full((physical_blocks, h, block_tokens, d), padding, np.float32)
    for tok in range(t):
        pool[table[tok // block_tokens], :, tok % block_tokens] = logical[:, tok]
    return pool
