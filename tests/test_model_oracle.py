"""Pins the CPU oracle of the reference's Llama model (oracle/llama.py)
against the known answers of the reference's kernel tests
(tests/cpu_kernels_test.cpp), closed forms and the forward/decode
invariant of tests/cuda_llama_model_test.cpp:293-334."""

import math

import numpy as np
import pytest

from oracle import llama as L

f32 = np.float32


def test_rope_known_answer():
    """cpu_kernels_test.cpp:379-389 (RotatesAdjacentPairsForEveryTokenAndHead)."""
    x = np.arange(1, 17, dtype=f32).reshape(2, 2, 4)
    cos = np.array([[1, 1], [0, 0]], f32)
    sin = np.array([[0, 0], [1, 1]], f32)
    out = L.rope(x, cos, sin)
    np.testing.assert_array_equal(out.reshape(-1), np.array(
        [1, 2, 3, 4, 5, 6, 7, 8, -10, 9, -12, 11, -14, 13, -16, 15], f32))


def test_rope_rounds_each_operation_in_float32():
    """out[2i] = fl(fl(a*c) - fl(b*s)): a plain double evaluation rounded once
    differs on some inputs, the float32 sequence is what the reference's CPU
    code computes without fused multiply-add."""
    rng = np.random.default_rng(0)
    a, b = rng.standard_normal(4096).astype(f32), rng.standard_normal(4096).astype(f32)
    th = rng.uniform(0, 6.3, 4096)
    c, s = np.cos(th).astype(f32), np.sin(th).astype(f32)
    out = L.rope(np.stack([a, b], -1).reshape(4096, 1, 2), c[:, None], s[:, None]).reshape(4096, 2)
    seq0 = f32(f32(a * c) - f32(b * s))
    seq1 = f32(f32(a * s) + f32(b * c))
    np.testing.assert_array_equal(out[:, 0], seq0)
    np.testing.assert_array_equal(out[:, 1], seq1)
    once = ((a.astype(np.float64) * c - b.astype(np.float64) * s)).astype(f32)
    assert np.any(once != seq0)  # the check above can tell the two apart


def test_rope_is_a_rotation():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((5, 3, 8)).astype(f32)
    c, s = L.make_rope_cache(5, 8, 10000.0, 7)
    y = L.rope(x, c, s)
    n0 = np.hypot(x[..., 0::2].astype(np.float64), x[..., 1::2])
    n1 = np.hypot(y[..., 0::2].astype(np.float64), y[..., 1::2])
    np.testing.assert_allclose(n1, n0, rtol=1e-6)
    back = L.rope(y, c, -s)
    np.testing.assert_allclose(back, x, atol=1e-5)


def test_rope_cache_closed_form():
    c, s = L.make_rope_cache(4, 8, 10000.0, 3)
    # pair 0 has frequency 1: angle = position
    np.testing.assert_array_equal(c[:, 0], np.cos(np.arange(3, 7, dtype=np.float64)).astype(f32))
    np.testing.assert_array_equal(s[:, 0], np.sin(np.arange(3, 7, dtype=np.float64)).astype(f32))
    # pair i: theta^(-2i/D)
    ang = 5 * 10000.0 ** (-2 * 3 / 8)
    assert c[2, 3] == f32(math.cos(ang)) and s[2, 3] == f32(math.sin(ang))
    c0, s0 = L.make_rope_cache(1, 8, 10000.0, 0)
    assert np.all(c0 == 1) and np.all(s0 == 0)


def test_rms_norm_known_answers():
    """cpu_kernels_test.cpp:205-233."""
    x = np.array([[1, 2, 3], [-2, 0.5, 4]], f32)
    w = np.array([1, 0.5, 2], f32)
    out = L.rms_norm(x, w, 1e-5)
    for r in range(2):
        scale = 1.0 / math.sqrt(sum(float(v) ** 2 for v in x[r]) / 3.0 + float(f32(1e-5)))
        exp = [f32(float(x[r, c]) * scale * float(w[c])) for c in range(3)]
        np.testing.assert_array_equal(out[r], np.array(exp, f32))
    out = L.rms_norm(np.array([[3, 4]], f32), np.ones(2, f32), 1e-5)
    scale = f32(1.0) / np.sqrt(f32(12.5) + f32(1e-5))
    np.testing.assert_allclose(out[0], [3 * scale, 4 * scale], atol=1e-6)


def test_silu_and_swiglu_known_answers():
    """cpu_kernels_test.cpp:32-46 and 246-255."""
    v = L.stable_silu(np.array([-100, -2, -0.0, 0, 1, 2, 100], f32))
    np.testing.assert_allclose(v, [0, -0.23840584, 0, 0, 0.7310586, 1.7615942, 100], atol=1e-5)
    assert v[2] == 0 and v[3] == 0
    out = L.swiglu(np.array([-2, 0, 1, 3], f32), np.array([0.5, 2, -1, 4], f32))
    np.testing.assert_allclose(out, [-0.11920292, 0, -0.7310586, 11.43089], atol=2e-5)


def test_linear_accumulates_in_double():
    rng = np.random.default_rng(2)
    x = rng.standard_normal((3, 37)).astype(f32)
    w = rng.standard_normal((37, 5)).astype(f32)
    out = L.linear(x, w)
    for i in range(3):
        for j in range(5):
            acc = 0.0
            for k in range(37):
                acc += float(x[i, k]) * float(w[k, j])
            assert abs(float(out[i, j]) - float(f32(acc))) <= 1e-7 * max(1.0, abs(acc))


@pytest.mark.parametrize("kv_heads", [0, 1])
def test_decode_with_cache_equals_full_prefix_forward(kv_heads):
    """The invariant of cuda_llama_model_test.cpp:293-334: decoding token by
    token with the per-layer K/V committed after each step gives the logits
    of recomputing the whole prefix.  kv_heads=1 is the GQA form (two query
    heads per kv head)."""
    cfg = L.LlamaConfig(11, 8, 12, 2, 2, 8, kv_heads=kv_heads)
    w = L.random_weights(cfg, seed=5)
    tokens = [1, 5, 3, 7, 2]
    kvh, d = cfg.kv_head_count, cfg.head_dimension
    keys = [np.zeros((kvh, 0, d), f32) for _ in range(cfg.layer_count)]
    values = [np.zeros((kvh, 0, d), f32) for _ in range(cfg.layer_count)]
    for pos, tok in enumerate(tokens):
        logits, tk, tv = L.decode_one(cfg, w, tok, pos, keys, values)
        full = L.forward(cfg, w, tokens[: pos + 1])
        np.testing.assert_allclose(logits, full[-1], atol=1e-6, rtol=1e-5)
        keys = [np.concatenate([keys[l], tk[l][:, None]], axis=1) for l in range(cfg.layer_count)]
        values = [np.concatenate([values[l], tv[l][:, None]], axis=1) for l in range(cfg.layer_count)]
    _, fk, fv = L.forward(cfg, w, tokens, capture_kv=True)
    for l in range(cfg.layer_count):
        np.testing.assert_allclose(keys[l], fk[l], atol=1e-6)
        np.testing.assert_allclose(values[l], fv[l], atol=1e-6)


def test_gqa_equals_mha_with_repeated_kv_weights():
    """A GQA model equals the MHA model whose key/value weights repeat each
    kv head's columns for its query heads."""
    g = L.LlamaConfig(13, 16, 20, 2, 4, 8, kv_heads=2)
    w = L.random_weights(g, seed=9)
    m = L.LlamaConfig(13, 16, 20, 2, 4, 8)
    d = g.head_dimension
    mw = L.random_weights(m, seed=9)
    mw.token_embedding, mw.final_norm, mw.lm_head = w.token_embedding, w.final_norm, w.lm_head
    for lg, lm in zip(w.layers, mw.layers):
        for name in ("attention_norm", "query", "attention_output", "ffn_norm", "gate", "up", "down"):
            setattr(lm, name, getattr(lg, name))
        lm.key = np.concatenate([lg.key[:, (h // 2) * d:(h // 2 + 1) * d] for h in range(4)], 1)
        lm.value = np.concatenate([lg.value[:, (h // 2) * d:(h // 2 + 1) * d] for h in range(4)], 1)
    toks = [3, 1, 4, 1, 5]
    np.testing.assert_allclose(L.forward(g, w, toks), L.forward(m, mw, toks), atol=1e-6)
