"""CPU oracle of the reference's Llama forward and decode -- TEST
INFRASTRUCTURE ONLY.

A numpy restatement of ``CpuLlamaModel`` (``src/model/cpu_llama.cpp``) and the
CPU kernels it calls (``src/kernels/cpu/reference.cpp``), used to check the
model-side integration of the paged decode path: a decode step whose
attention, rotary embedding and K/V commit run through the HIP library must
produce the logits that recomputing the whole prefix on the CPU produces
(the reference's own check, ``tests/cuda_llama_model_test.cpp:293-334``).
Attention itself is the oracle's C++ restatement (``oracle.sdpa``,
``src/attention/reference.cpp:124-228``).  Only ``tests/`` imports this.

The reference model is multi-head (key/value weights [hidden, hidden]); the
restatement also takes ``kv_heads`` < heads (grouped-query attention), where
each kv head serves ``heads / kv_heads`` consecutive query heads -- the same
as repeating the kv heads, which is how the GQA invariant is stated.

Arithmetic follows the reference's cast sequence: float64 accumulation in
linear and RMSNorm, rounding to float32 at each tensor boundary, and the
rotary embedding in float32 with every product and sum rounded on its own.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from . import sdpa

f32 = np.float32
f64 = np.float64


@dataclass
class LlamaConfig:
    """include/helix/model/llama.hpp:14-26 (plus kv_heads for GQA)."""
    vocabulary_size: int
    hidden_size: int
    intermediate_size: int
    layer_count: int
    attention_head_count: int
    max_sequence_length: int
    rms_norm_epsilon: float = 1.0e-5
    rope_theta: float = 10000.0
    kv_heads: int = 0  # 0: attention_head_count (the reference's MHA)

    @property
    def head_dimension(self):
        return self.hidden_size // self.attention_head_count

    @property
    def kv_head_count(self):
        return self.kv_heads or self.attention_head_count


def make_rope_cache(tokens, head_dimension, theta, position_offset=0):
    """detail::make_rope_cache (src/model/llama_common.cpp:22-47): angle =
    (offset + t) * theta^(-2i/D) in double, cos/sin rounded to float32."""
    pairs = head_dimension // 2
    pair = np.arange(pairs, dtype=f64)
    exponent = -2.0 * pair / f64(head_dimension)
    frequency = np.power(f64(f32(theta)), exponent)
    position = (position_offset + np.arange(tokens, dtype=f64))[:, None]
    angle = position * frequency[None, :]
    return np.cos(angle).astype(f32), np.sin(angle).astype(f32)


def rope(x, cosine, sine):
    """cpu::rope_out (src/kernels/cpu/reference.cpp:490-533): x [T, ..., D]
    float32, token t uses row t; float32 products and differences, each
    rounded (numpy float32 arithmetic rounds every operation)."""
    x = np.asarray(x, dtype=f32)
    t = x.shape[0]
    v = x.reshape(t, -1, x.shape[-1])
    first, second = v[..., 0::2], v[..., 1::2]
    c = np.asarray(cosine, dtype=f32)[:t, None, :]
    s = np.asarray(sine, dtype=f32)[:t, None, :]
    out = np.empty_like(v)
    out[..., 0::2] = first * c - second * s
    out[..., 1::2] = first * s + second * c
    return out.reshape(x.shape)


def rms_norm(x, weight, epsilon):
    """cpu::rms_norm_out (src/kernels/cpu/reference.cpp:369-407): per row,
    inverse_rms = 1 / sqrt(sum(x^2) / width + eps) in double, output =
    float(x * inverse_rms * w)."""
    xd = np.asarray(x, dtype=f32).astype(f64)
    width = xd.shape[-1]
    ss = np.sum(xd * xd, axis=-1, keepdims=True)
    inverse = 1.0 / np.sqrt(ss / f64(width) + f64(f32(epsilon)))
    return (xd * inverse * np.asarray(weight, dtype=f32).astype(f64)).astype(f32)


def linear(x, weight):
    """cpu::linear / matmul_out (src/kernels/cpu/reference.cpp:324-359,
    541-552): x [rows, in] @ W [in, out] with float64 accumulation, then
    float32."""
    return (np.asarray(x, dtype=f32).astype(f64) @ np.asarray(weight, dtype=f32).astype(f64)
            ).astype(f32)


def stable_silu(x):
    """stable_silu (src/kernels/cpu/reference.cpp:98-108) in double."""
    xd = np.asarray(x, dtype=f32).astype(f64)
    with np.errstate(over="ignore"):
        pos = 1.0 / (1.0 + np.exp(-np.where(xd >= 0, xd, 0.0)))
        e = np.exp(np.where(xd < 0, xd, 0.0))
    sigmoid = np.where(xd >= 0, pos, e / (1.0 + e))
    return (xd * sigmoid).astype(f32)


def swiglu(gate, up):
    """cpu::swiglu_out (src/kernels/cpu/reference.cpp:415-418):
    float(stable_silu(gate)) * up in float32."""
    return stable_silu(gate) * np.asarray(up, dtype=f32)


@dataclass
class LayerWeights:
    """LlamaLayerWeights (include/helix/model/llama.hpp:28-48); matrices are
    [in, out] as cpu::linear takes them."""
    attention_norm: np.ndarray
    query: np.ndarray
    key: np.ndarray
    value: np.ndarray
    attention_output: np.ndarray
    ffn_norm: np.ndarray
    gate: np.ndarray
    up: np.ndarray
    down: np.ndarray


@dataclass
class Weights:
    token_embedding: np.ndarray  # [vocab, hidden]
    layers: list
    final_norm: np.ndarray       # [hidden]
    lm_head: np.ndarray          # [hidden, vocab]


def random_weights(config: LlamaConfig, seed=0):
    """Seeded weights in the ranges of tests/cuda_llama_model_test.cpp:27-48
    (norm gains U[0.8, 1.2], projections U[-0.2, 0.2], embedding
    U[-0.25, 0.25])."""
    rng = np.random.default_rng(seed)
    h, i, v = config.hidden_size, config.intermediate_size, config.vocabulary_size
    kv = config.kv_head_count * config.head_dimension

    def u(shape, lo, hi):
        return rng.uniform(lo, hi, size=shape).astype(f32)

    layers = [LayerWeights(u((h,), 0.8, 1.2), u((h, h), -0.2, 0.2), u((h, kv), -0.2, 0.2),
                           u((h, kv), -0.2, 0.2), u((h, h), -0.2, 0.2), u((h,), 0.8, 1.2),
                           u((h, i), -0.2, 0.2), u((h, i), -0.2, 0.2), u((i, h), -0.2, 0.2))
              for _ in range(config.layer_count)]
    return Weights(u((v, h), -0.25, 0.25), layers, u((h,), 0.8, 1.2), u((h, v), -0.2, 0.2))


def _attention(query, key, value, offset, group):
    """attention::cpu::scaled_dot_product_attention over head-major
    [heads, T, D] (oracle.sdpa), kv heads repeated for GQA."""
    if group > 1:
        key = np.repeat(key, group, axis=0)
        value = np.repeat(value, group, axis=0)
    out, _ = sdpa(query, key, value, offset)
    return out


def forward(config: LlamaConfig, weights: Weights, token_ids, capture_kv=False):
    """execute_forward (src/model/cpu_llama.cpp:37-110): causal forward of a
    whole token sequence; returns logits [T, vocab] and, with capture_kv, the
    rotated keys and the values per layer, head-major [kv_heads, T, D]."""
    tokens = len(token_ids)
    heads, kvh, d = config.attention_head_count, config.kv_head_count, config.head_dimension
    cosine, sine = make_rope_cache(tokens, d, config.rope_theta)
    hidden = weights.token_embedding[np.asarray(token_ids, dtype=np.int64)].astype(f32)
    keys, values = [], []
    for layer in weights.layers:
        x = rms_norm(hidden, layer.attention_norm, config.rms_norm_epsilon)
        q = rope(linear(x, layer.query).reshape(tokens, heads, d), cosine, sine)
        k = rope(linear(x, layer.key).reshape(tokens, kvh, d), cosine, sine)
        v = linear(x, layer.value).reshape(tokens, kvh, d)
        qh, kh, vh = (np.ascontiguousarray(a.transpose(1, 0, 2)) for a in (q, k, v))
        if capture_kv:
            keys.append(kh)
            values.append(vh)
        ctx = _attention(qh, kh, vh, 0, heads // kvh)
        merged = np.ascontiguousarray(ctx.transpose(1, 0, 2)).reshape(tokens, heads * d)
        hidden = hidden + linear(merged, layer.attention_output)
        f = rms_norm(hidden, layer.ffn_norm, config.rms_norm_epsilon)
        hidden = hidden + linear(swiglu(linear(f, layer.gate), linear(f, layer.up)), layer.down)
    logits = linear(rms_norm(hidden, weights.final_norm, config.rms_norm_epsilon), weights.lm_head)
    return (logits, keys, values) if capture_kv else logits


def decode_one(config: LlamaConfig, weights: Weights, token_id, position, layer_keys,
               layer_values):
    """execute_decode_one (src/model/cpu_llama.cpp:190-268) with the compact
    cache path: one token at `position` attends to the cached history
    (layer_keys[l], layer_values[l]: [kv_heads, position, D]) plus itself.
    Returns (logits [vocab], token_keys [L, kv_heads, D], token_values)."""
    heads, kvh, d = config.attention_head_count, config.kv_head_count, config.head_dimension
    cosine, sine = make_rope_cache(1, d, config.rope_theta, position)
    hidden = weights.token_embedding[np.asarray([token_id], dtype=np.int64)].astype(f32)
    token_keys, token_values = [], []
    for li, layer in enumerate(weights.layers):
        x = rms_norm(hidden, layer.attention_norm, config.rms_norm_epsilon)
        q = rope(linear(x, layer.query).reshape(1, heads, d), cosine, sine)
        k = rope(linear(x, layer.key).reshape(1, kvh, d), cosine, sine)
        v = linear(x, layer.value).reshape(1, kvh, d)
        qh, kh, vh = (np.ascontiguousarray(a.transpose(1, 0, 2)) for a in (q, k, v))
        token_keys.append(kh[:, 0])
        token_values.append(vh[:, 0])
        ck = np.concatenate([layer_keys[li], kh], axis=1)
        cv = np.concatenate([layer_values[li], vh], axis=1)
        ctx = _attention(qh, ck, cv, position, heads // kvh)
        merged = np.ascontiguousarray(ctx.transpose(1, 0, 2)).reshape(1, heads * d)
        hidden = hidden + linear(merged, layer.attention_output)
        f = rms_norm(hidden, layer.ffn_norm, config.rms_norm_epsilon)
        hidden = hidden + linear(swiglu(linear(f, layer.gate), linear(f, layer.up)), layer.down)
    logits = linear(rms_norm(hidden, weights.final_norm, config.rms_norm_epsilon), weights.lm_head)
    return logits[0], np.stack(token_keys), np.stack(token_values)
