"""Model-side integration of the paged decode path on the GPU.

The rotary-embedding kernel against the CPU oracle bit-exactly, then a tiny
Llama (the reference model's structure, head_dim 128) decoding a batch of
sequences with ragged histories: the model's own dense work (RMSNorm,
projections, SwiGLU) in torch, and everything on the KV path through the
library -- RoPE of the step's query and key in one launch, attention over the
pages plus the uncommitted tail with no per-layer synchronisation, and the
token's K/V committed for all layers in one launch after the forward pass
(or written by the fused decode kernel).  Each step's logits must equal the
oracle's recomputation of the whole prefix within the reference's model
tolerance (tests/cuda_llama_model_test.cpp:20-21, 293-334)."""

import numpy as np
import pytest
import torch

import helix_runtime_amd as hx
from oracle import llama as L

pytestmark = pytest.mark.gpu

D, P = 128, 16
ATOL, RTOL = 2.0e-4, 2.0e-3  # tests/cuda_llama_model_test.cpp:20-21


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda:0")


def host(t):
    return t.detach().cpu().numpy()


# ------------------------------------------------------------------ rope ----

@pytest.mark.parametrize("shape", [(7, 5, 128), (3, 3, 6), (1, 1, 2), (64, 8, 128)])
def test_rope_bit_exact_with_positions(device, shape):
    rng = np.random.default_rng(shape[0])
    x = rng.standard_normal(shape).astype(np.float32) * 3
    cos, sin = L.make_rope_cache(200, shape[-1], 10000.0)
    pos = rng.integers(0, 200, size=shape[0]).astype(np.int32)
    out = hx.rope(dev(x), dev(cos), dev(sin), positions=dev(pos))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(host(out), L.rope(x, cos[pos], sin[pos]))


def test_rope_rows_in_order_and_in_place(device):
    """Without positions token t uses row t (the reference's contract); the
    output may be the input itself (cpu_kernels_test.cpp:391-411)."""
    rng = np.random.default_rng(3)
    x = rng.uniform(-2, 2, size=(3, 3, 6)).astype(np.float32)
    ang = np.arange(9, dtype=np.float32).reshape(3, 3) * np.float32(0.17)
    cos, sin = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    t = dev(x)
    hx.rope_out(t, dev(cos), dev(sin), t)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(host(t), L.rope(x, cos, sin))
    # the known answer of cpu_kernels_test.cpp:379-389
    k = dev(np.arange(1, 17, dtype=np.float32).reshape(2, 2, 4))
    out = hx.rope(k, dev(np.array([[1, 1], [0, 0]], np.float32)),
                  dev(np.array([[0, 0], [1, 1]], np.float32)))
    np.testing.assert_array_equal(host(out).reshape(-1), np.array(
        [1, 2, 3, 4, 5, 6, 7, 8, -10, 9, -12, 11, -14, 13, -16, 15], np.float32))


def test_rope_rejects_and_poisons(device):
    x = torch.ones(4, 2, 8, device=device)
    cos, sin = L.make_rope_cache(5, 8, 10000.0)
    with pytest.raises(hx.HelixError):
        hx.rope(x, dev(cos), dev(sin))  # 5 table rows for 4 tokens, no positions
    with pytest.raises(hx.HelixError):
        hx.rope(torch.ones(2, 2, 7, device=device), dev(cos[:2, :3]), dev(sin[:2, :3]))
    pos = dev(np.array([0, 5, -1, 4], np.int32))  # rows 1 and 2 out of range
    out = host(hx.rope(x, dev(cos), dev(sin), positions=pos))
    assert np.isnan(out[1]).all() and np.isnan(out[2]).all()
    np.testing.assert_array_equal(out[0], L.rope(host(x)[:1], cos[:1], sin[:1])[0])
    np.testing.assert_array_equal(out[3], L.rope(host(x)[3:], cos[4:5], sin[4:5])[0])


def test_decode_batch_rope_uses_each_sequence_position(device):
    H, HQ = 2, 8
    cache = hx.PagedKvCache(1, H, D, P, 32)
    lengths = [0, 1, 16, 45]
    seqs = []
    for n in lengths:
        s = cache.create_sequence()
        if n:
            cache.append_layer_major(s, [torch.zeros(H, n, D, device=device)],
                                     [torch.zeros(H, n, D, device=device)])
        seqs.append(s)
    batch = hx.DecodeBatch(cache, seqs, HQ, max_tokens=64)
    batch.prepare()
    rng = np.random.default_rng(11)
    q = rng.standard_normal((4, HQ, D)).astype(np.float32)
    k = rng.standard_normal((4, H, D)).astype(np.float32)
    cos, sin = L.make_rope_cache(64, D, 500000.0)
    tq, tk = dev(q), dev(k)
    batch.rope(tq, tk, dev(cos), dev(sin))
    torch.cuda.synchronize()
    pos = np.array(lengths)
    np.testing.assert_array_equal(host(tq), L.rope(q, cos[pos], sin[pos]))
    np.testing.assert_array_equal(host(tk), L.rope(k, cos[pos], sin[pos]))
    batch.close()


# ------------------------------------------------------- model decode ----

class TorchLlama:
    """The model's side of a decode step on the GPU: dense ops in torch fp32
    (the caller's own kernels), the KV path through the library."""

    def __init__(self, cfg, weights):
        self.cfg = cfg
        t = lambda a: dev(a)  # noqa: E731
        self.emb = t(weights.token_embedding)
        self.final = t(weights.final_norm)
        self.head = t(weights.lm_head)
        self.layers = [{k: t(getattr(lw, k)) for k in (
            "attention_norm", "query", "key", "value", "attention_output", "ffn_norm", "gate",
            "up", "down")} for lw in weights.layers]
        cos, sin = L.make_rope_cache(cfg.max_sequence_length, cfg.head_dimension, cfg.rope_theta)
        self.cos, self.sin = t(cos), t(sin)

    def norm(self, x, w):
        eps = self.cfg.rms_norm_epsilon
        return x * torch.rsqrt(torch.mean(x * x, dim=-1, keepdim=True) + eps) * w

    def decode_step(self, batch, token_ids, mode):
        cfg = self.cfg
        B, heads, kvh = len(token_ids), cfg.attention_head_count, cfg.kv_head_count
        batch.prepare()
        hidden = self.emb[torch.as_tensor(token_ids, device="cuda:0")]
        # The step's K/V for all layers: each layer's projections are written
        # straight into their slice (the reference copies them there).
        k_all = torch.empty(cfg.layer_count, B, kvh, D, device="cuda:0")
        v_all = torch.empty_like(k_all)
        for l, w in enumerate(self.layers):
            x = self.norm(hidden, w["attention_norm"])
            q = (x @ w["query"]).view(B, heads, D)
            torch.matmul(x, w["key"], out=k_all[l].view(B, kvh * D))
            torch.matmul(x, w["value"], out=v_all[l].view(B, kvh * D))
            batch.rope(q, k_all[l], self.cos, self.sin)
            ctx = torch.empty(B, heads, D, device="cuda:0")
            if mode == "fused":
                batch.append_attention_layer(l, q, k_all[l], v_all[l], ctx)
            else:
                batch.attention_layer(l, q, k_all[l], v_all[l], ctx)
            hidden = hidden + ctx.view(B, heads * D) @ w["attention_output"]
            f = self.norm(hidden, w["ffn_norm"])
            act = torch.nn.functional.silu(f @ w["gate"]) * (f @ w["up"])
            hidden = hidden + act @ w["down"]
        if mode == "commit":
            batch.append_all_layers(k_all, v_all)
        return self.norm(hidden, self.final) @ self.head


@pytest.mark.parametrize("mode", ["commit", "fused"])
@pytest.mark.parametrize("heads,kv_heads", [(4, 4), (8, 2)])
def test_llama_decode_matches_full_prefix_recomputation(device, mode, heads, kv_heads):
    torch.backends.cuda.matmul.allow_tf32 = False
    cfg = L.LlamaConfig(64, heads * D, 384, 2, heads, 96, kv_heads=kv_heads)
    weights = L.random_weights(cfg, seed=heads + kv_heads)
    model = TorchLlama(cfg, weights)
    rng = np.random.default_rng(kv_heads)
    prompts = [list(rng.integers(0, 64, size=n)) for n in (0, 5, 17, 33)]
    kvh = cfg.kv_head_count
    cache = hx.PagedKvCache(cfg.layer_count, kvh, D, P, 64)
    seqs = []
    for prompt in prompts:
        s = cache.create_sequence()
        if prompt:
            _, keys, values = L.forward(cfg, weights, prompt, capture_kv=True)
            cache.append_layer_major(s, [dev(k) for k in keys], [dev(v) for v in values])
        seqs.append(s)
    batch = hx.DecodeBatch(cache, seqs, heads, max_tokens=cfg.max_sequence_length)
    texts = [list(p) for p in prompts]
    for step in range(3):
        tokens = [int(t) for t in rng.integers(0, 64, size=len(seqs))]
        logits = host(model.decode_step(batch, tokens, mode))
        for b, tok in enumerate(tokens):
            texts[b].append(tok)
            expected = L.forward(cfg, weights, texts[b])[-1]
            np.testing.assert_allclose(logits[b], expected, atol=ATOL, rtol=RTOL,
                                       err_msg=f"step {step} sequence {b}")
    # The committed pages hold every token's rotated key and value.
    for b, s in enumerate(seqs):
        assert cache.length(s) == len(texts[b])
        _, keys, values = L.forward(cfg, weights, texts[b], capture_kv=True)
        for l in range(cfg.layer_count):
            gk, gv = cache.retrieve_layer(s, l)
            np.testing.assert_allclose(host(gk), keys[l], atol=ATOL, rtol=RTOL)
            np.testing.assert_allclose(host(gv), values[l], atol=ATOL, rtol=RTOL)
    batch.close()
    cache.close()
