"""Writes the golden fixtures of this directory.

The data are the explicit expected values of the reference's own tests,
transcribed by hand from their source files (cited per fixture), plus
closed-form expectations where the reference test computes its expectation
at run time: those are evaluated here in float64 from the definition of
scaled-dot-product attention (softmax(q k^T / sqrt(d)) v with the causal
rule key <= offset + row), never from reference code.  Nothing here imports
or runs the reference.  Run from the repo root:

    python tests/golden/make_fixtures.py
"""

import json
import math
import os

HERE = os.path.dirname(os.path.abspath(__file__))


def layer1_encoded(tokens, base):
    """Keys (or values) of layer 1 of a [2 layers, 2 heads, 2 dims] cache
    filled by make_token(2, 2, 2, base + token * 100) for tokens 0..tokens-1
    (tests/paged_kv_cache_test.cpp:18-27), retrieved head-major."""
    out = []
    for head in range(2):
        for token in range(tokens):
            for coord in range(2):
                out.append(base + token * 100 + (1 * 2 + head) * 2 + coord)
    return out


# tests/paged_kv_cache_test.cpp:78-84 spells these arrays out.
L1_KEYS_5 = [4.0, 5.0, 104.0, 105.0, 204.0, 205.0, 304.0, 305.0, 404.0, 405.0,
             6.0, 7.0, 106.0, 107.0, 206.0, 207.0, 306.0, 307.0, 406.0, 407.0]
L1_VALUES_5 = [1004.0, 1005.0, 1104.0, 1105.0, 1204.0, 1205.0, 1304.0, 1305.0, 1404.0,
               1405.0, 1006.0, 1007.0, 1106.0, 1107.0, 1206.0, 1207.0, 1306.0, 1307.0,
               1406.0, 1407.0]
assert layer1_encoded(5, 0) == L1_KEYS_5 and layer1_encoded(5, 1000) == L1_VALUES_5


def enc(seq, token, key_base=0, value_base=1000):
    return {"op": "append_encoded", "seq": seq, "key_base": key_base + token * 100,
            "value_base": value_base + token * 100}


SCENARIOS = [
    {
        "name": "maps logical history across physical block boundaries",
        "source": "tests/paged_kv_cache_test.cpp:60-121",
        "config": [2, 2, 2, 2, 4],
        "ops": [{"op": "create", "seq": "s"}] + [enc("s", t) for t in range(5)] + [
            {"op": "expect_table", "seq": "s", "table": [0, 1, 2]},
            {"op": "expect_layer", "seq": "s", "layer": 1, "keys": L1_KEYS_5,
             "values": L1_VALUES_5},
            {"op": "expect_stats", "stats": {
                "bytes_reserved": 512, "bytes_used": 384, "bytes_free": 128,
                "peak_bytes_used": 384, "total_blocks": 4, "used_blocks": 3, "free_blocks": 1,
                "active_sequence_count": 1, "active_tokens": 5, "allocated_token_slots": 6,
                "block_allocation_count": 3, "block_reuse_count": 0}},
        ],
    },
    {
        "name": "block exhaustion is transactional and partial blocks remain writable",
        "source": "tests/paged_kv_cache_test.cpp:144-175",
        "config": [1, 1, 2, 2, 1],
        "ops": [
            {"op": "create", "seq": "first"}, {"op": "create", "seq": "second"},
            {"op": "append_values", "seq": "first", "keys": [1.0, 2.0], "values": [1.0, 2.0]},
            {"op": "expect_error", "status": "resource_exhausted",
             "inner": {"op": "append_values", "seq": "second", "keys": [1.0, 2.0],
                       "values": [1.0, 2.0]}},
            {"op": "expect_length", "seq": "second", "length": 0},
            {"op": "expect_table", "seq": "second", "table": []},
            {"op": "expect_stats", "stats": {"append_count": 1}},
            {"op": "append_values", "seq": "first", "keys": [1.0, 2.0], "values": [1.0, 2.0]},
            {"op": "expect_length", "seq": "first", "length": 2},
            {"op": "expect_error", "status": "any",
             "inner": {"op": "append_values", "seq": "first", "keys": [1.0, 2.0],
                       "values": [1.0, 2.0]}},
            {"op": "expect_length", "seq": "first", "length": 2},
            {"op": "expect_table_size", "seq": "first", "size": 1},
            {"op": "expect_stats", "stats": {"active_tokens": 2}},
            {"op": "release", "seq": "first"},
            {"op": "append_values", "seq": "second", "keys": [9.0, 8.0], "values": [9.0, 8.0]},
            {"op": "expect_table", "seq": "second", "table": [0]},
            {"op": "expect_stats", "stats": {"block_reuse_count": 1}},
            {"op": "expect_layer", "seq": "second", "layer": 0, "keys": [9.0, 8.0],
             "values": [9.0, 8.0]},
        ],
    },
    {
        "name": "bulk layer-major append spans partial and whole blocks",
        "source": "tests/paged_kv_cache_test.cpp:177-199",
        "config": [2, 2, 2, 2, 3],
        "ops": [
            {"op": "create", "seq": "s"}, enc("s", 0),
            {"op": "append_layer_major_encoded", "seq": "s", "token_begin": 1, "count": 4,
             "key_base": 0, "value_base": 1000},
            {"op": "expect_length", "seq": "s", "length": 5},
            {"op": "expect_layer", "seq": "s", "layer": 1, "keys": L1_KEYS_5,
             "values": L1_VALUES_5},
            {"op": "expect_stats", "stats": {"append_count": 5, "block_allocation_count": 3}},
        ],
    },
    {
        "name": "bulk append beyond the pool is transactional",
        "source": "tests/paged_kv_cache_test.cpp:201-220",
        "config": [2, 2, 2, 2, 2],
        "ops": [
            {"op": "create", "seq": "s"},
            {"op": "expect_error", "status": "any",
             "inner": {"op": "append_layer_major_encoded", "seq": "s", "token_begin": 0,
                       "count": 5, "key_base": 0, "value_base": 1000}},
            {"op": "expect_length", "seq": "s", "length": 0},
            {"op": "expect_table", "seq": "s", "table": []},
            {"op": "expect_stats", "stats": {"append_count": 0}},
        ],
    },
    {
        "name": "free pool is a deterministic FIFO and release reclaims every block",
        "source": "tests/paged_kv_cache_test.cpp:222-256",
        "config": [1, 1, 1, 1, 3],
        "ops": [{"op": "create", "seq": n} for n in ("a", "b", "c")] + [
            {"op": "append_values", "seq": n, "keys": [1.0], "values": [1.0]}
            for n in ("a", "b", "c")] + [
            {"op": "expect_table", "seq": "a", "table": [0]},
            {"op": "expect_table", "seq": "b", "table": [1]},
            {"op": "expect_table", "seq": "c", "table": [2]},
            {"op": "release", "seq": "b"}, {"op": "release", "seq": "a"},
            {"op": "create", "seq": "d"}, {"op": "create", "seq": "e"},
            {"op": "append_values", "seq": "d", "keys": [1.0], "values": [1.0]},
            {"op": "append_values", "seq": "e", "keys": [1.0], "values": [1.0]},
            {"op": "expect_table", "seq": "d", "table": [1]},
            {"op": "expect_table", "seq": "e", "table": [0]},
            {"op": "expect_stats", "stats": {"block_reuse_count": 2}},
            {"op": "release", "seq": "c"}, {"op": "release", "seq": "d"},
            {"op": "release", "seq": "e"},
            {"op": "expect_stats", "stats": {"bytes_used": 0, "used_blocks": 0, "free_blocks": 3,
                                             "active_tokens": 0, "allocated_token_slots": 0}},
        ],
    },
    {
        "name": "block-aligned fork shares the immutable prefix and branches diverge",
        "source": "tests/paged_kv_cache_test.cpp:365-462",
        "config": [2, 2, 2, 2, 6],
        "ops": [{"op": "create", "seq": "src"}] + [enc("src", t) for t in range(5)] + [
            {"op": "fork", "seq": "src", "new": "fork", "prefix": 4},
            {"op": "expect_table_size", "seq": "src", "size": 3},
            {"op": "expect_table_size", "seq": "fork", "size": 2},
            {"op": "expect_tables_share", "a": "src", "b": "fork", "count": 2},
            {"op": "expect_layer", "seq": "fork", "layer": 1,
             "keys": [v for h in range(2) for v in L1_KEYS_5[h * 10: h * 10 + 8]],
             "values": [v for h in range(2) for v in L1_VALUES_5[h * 10: h * 10 + 8]]},
            {"op": "expect_stats", "stats": {
                "active_sequence_count": 2, "active_tokens": 9, "resident_tokens": 5,
                "used_blocks": 3, "block_reference_count": 5, "shared_blocks": 2,
                "sequence_create_count": 2, "sequence_fork_count": 1,
                "block_allocation_count": 3}},
            {"op": "append_layer_major_encoded", "seq": "fork", "token_begin": 4, "count": 1,
             "key_base": 9000, "value_base": 19000},
            enc("src", 0, 8000, 18000),
            {"op": "expect_tables_share", "a": "src", "b": "fork", "count": 2},
            {"op": "expect_tables_differ_at", "a": "src", "b": "fork", "index": 2},
            {"op": "expect_layer_element", "seq": "src", "layer": 1, "index": 10,
             "key": 8004.0, "value": 18004.0},
            {"op": "expect_layer_element", "seq": "fork", "layer": 1, "index": 8,
             "key": 9404.0, "value": 19404.0},
            {"op": "expect_stats", "stats": {"active_tokens": 11, "resident_tokens": 7,
                                             "used_blocks": 4, "block_reference_count": 6,
                                             "shared_blocks": 2}},
            {"op": "release", "seq": "src"},
            {"op": "expect_length", "seq": "fork", "length": 5},
            {"op": "expect_stats", "stats": {"active_tokens": 5, "resident_tokens": 5,
                                             "used_blocks": 3, "block_reference_count": 3,
                                             "shared_blocks": 0}},
            {"op": "release", "seq": "fork"},
            {"op": "expect_stats", "stats": {"active_sequence_count": 0, "active_tokens": 0,
                                             "resident_tokens": 0, "used_blocks": 0,
                                             "free_blocks": 6, "block_reference_count": 0}},
        ],
    },
    {
        "name": "fork validation and exhaustion are transactional",
        "source": "tests/paged_kv_cache_test.cpp:464-513",
        "config": [1, 1, 2, 2, 3],
        "ops": [{"op": "create", "seq": "src"}] + [
            {"op": "append_values", "seq": "src", "keys": [1.0, 2.0], "values": [1.0, 2.0]}
            for _ in range(5)] + [
            {"op": "expect_error", "status": "any",
             "inner": {"op": "fork", "seq": "src", "new": "x", "prefix": p}} for p in (0, 3, 6)] + [
            {"op": "expect_stats", "stats": {"active_sequence_count": 1, "active_tokens": 5,
                                             "resident_tokens": 5, "used_blocks": 3,
                                             "block_reference_count": 3,
                                             "sequence_create_count": 1,
                                             "sequence_fork_count": 0}},
            {"op": "fork", "seq": "src", "new": "fork", "prefix": 4},
            {"op": "expect_stats", "stats": {"free_blocks": 0}},
            {"op": "expect_error", "status": "any",
             "inner": {"op": "append_values", "seq": "fork", "keys": [1.0, 2.0],
                       "values": [1.0, 2.0]}},
            {"op": "expect_length", "seq": "fork", "length": 4},
            {"op": "expect_table_size", "seq": "fork", "size": 2},
            {"op": "expect_stats", "stats": {"append_count": 5}},
            {"op": "release", "seq": "src"},
            {"op": "expect_stats", "stats": {"free_blocks": 1, "used_blocks": 2,
                                             "active_tokens": 4, "resident_tokens": 4}},
            {"op": "append_values", "seq": "fork", "keys": [9.0, 8.0], "values": [7.0, 6.0]},
            {"op": "expect_table_last", "seq": "fork", "block": 2},
            {"op": "expect_stats", "stats": {"block_reuse_count": 1}},
            {"op": "release", "seq": "fork"},
            {"op": "expect_stats", "stats": {"used_blocks": 0, "free_blocks": 3,
                                             "active_tokens": 0, "resident_tokens": 0}},
        ],
    },
]


def sdpa_closed_form(q, k, v, offset):
    """softmax(q k^T / sqrt(d)) v over one head, keys <= offset + row, float64."""
    d = len(q[0])
    out, probs = [], []
    for r, qr in enumerate(q):
        vis = offset + r + 1
        s = [sum(a * b for a, b in zip(qr, k[j])) / math.sqrt(d) for j in range(vis)]
        m = max(s)
        e = [math.exp(x - m) for x in s]
        z = sum(e)
        p = [x / z for x in e] + [0.0] * (len(k) - vis)
        probs.append(p)
        out.append([sum(p[j] * v[j][c] for j in range(len(k))) for c in range(len(v[0]))])
    return out, probs


def attention_cases():
    cases = []
    # tests/cuda_attention_test.cpp:196-228: two queries at offset 1 over three
    # keys packed into blocks {2, 0} of a 3-block pool (2 tokens per block),
    # the unused slot of the last block padded with +-10000.
    q = [[1.0, 0.0], [0.0, 1.0]]
    k = [[1.0, 0.0], [0.0, 1.0], [1.0, 1.0]]
    v = [[10.0, 1.0, -1.0], [20.0, 2.0, -2.0], [30.0, 3.0, -3.0]]
    out, probs = sdpa_closed_form(q, k, v, 1)
    cases.append({"name": "known reordered blocks, tail padding ignored",
                  "source": "tests/cuda_attention_test.cpp:196-228",
                  "query": q, "keys": k, "values": v, "table": [2, 0], "physical_blocks": 3,
                  "block_tokens": 2, "offset": 1, "key_padding": 10000.0,
                  "value_padding": -10000.0, "output": out, "probabilities": probs})
    # tests/paged_attention_test.cpp:44-78: causal prefill of three queries
    # over the same keys appended token by token.
    q3 = [[1.0, 0.0], [0.0, 1.0], [1.0, 1.0]]
    v2 = [[10.0, 1.0], [20.0, 2.0], [30.0, 3.0]]
    out, probs = sdpa_closed_form(q3, k, v2, 0)
    cases.append({"name": "causal prefill across block boundaries",
                  "source": "tests/paged_attention_test.cpp:44-78",
                  "query": q3, "keys": k, "values": v2, "table": [0, 1], "physical_blocks": 2,
                  "block_tokens": 2, "offset": 0, "key_padding": 0.0, "value_padding": 0.0,
                  "output": out, "probabilities": probs})
    # tests/paged_kv_cache_test.cpp:123-142: one decode query at offset 2.
    out, probs = sdpa_closed_form([[1.0, 1.0]], k, v2, 2)
    cases.append({"name": "decode query over retrieved blocks",
                  "source": "tests/paged_kv_cache_test.cpp:123-142",
                  "query": [[1.0, 1.0]], "keys": k, "values": v2, "table": [0, 1],
                  "physical_blocks": 2, "block_tokens": 2, "offset": 2, "key_padding": 0.0,
                  "value_padding": 0.0, "output": out, "probabilities": probs})
    return cases


MODEL_KERNELS = {
    "source": "tests/cpu_kernels_test.cpp",
    "rope": {"source": "tests/cpu_kernels_test.cpp:379-389",
             "input": [[[1, 2, 3, 4], [5, 6, 7, 8]], [[9, 10, 11, 12], [13, 14, 15, 16]]],
             "cosine": [[1, 1], [0, 0]], "sine": [[0, 0], [1, 1]],
             "output": [[[1, 2, 3, 4], [5, 6, 7, 8]], [[-10, 9, -12, 11], [-14, 13, -16, 15]]]},
    "silu": {"source": "tests/cpu_kernels_test.cpp:32-46",
             "input": [-100.0, -2.0, -0.0, 0.0, 1.0, 2.0, 100.0],
             "output": [0.0, -0.23840584, 0.0, 0.0, 0.7310586, 1.7615942, 100.0],
             "tolerance": 1.0e-5},
    "swiglu": {"source": "tests/cpu_kernels_test.cpp:246-255",
               "gate": [-2.0, 0.0, 1.0, 3.0], "up": [0.5, 2.0, -1.0, 4.0],
               "output": [-0.11920292, 0.0, -0.7310586, 11.43089], "tolerance": 2.0e-5},
}


def main():
    with open(os.path.join(HERE, "paged_cache_scenarios.json"), "w") as f:
        json.dump(SCENARIOS, f, indent=1)
    with open(os.path.join(HERE, "attention_known_answers.json"), "w") as f:
        json.dump(attention_cases(), f, indent=1)
    with open(os.path.join(HERE, "model_kernel_known_answers.json"), "w") as f:
        json.dump(MODEL_KERNELS, f, indent=1)


if __name__ == "__main__":
    main()
