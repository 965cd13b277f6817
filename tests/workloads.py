"""Builders of the BASELINE workloads at their real shapes, for the GPU parity
tests: a device cache whose free queue is shuffled (so every sequence's pages
scatter over the pool, as the configs ask), filled with N(0, 1) histories,
plus helpers that read back what the oracle needs (host pools, tables,
lengths).  The oracle is evaluated on the cache's own page contents; the
page writes themselves are pinned bit-exactly by the cache tests."""

from __future__ import annotations

import math

import numpy as np
import torch

import helix_runtime_amd as hx

D, P = 128, 16


def shuffled_cache(layers, kv_heads, physical_blocks, seed, page_dtype="f32",
                   head_dim=D, block_tokens=P):
    """A cache whose FIFO free queue holds every block in a seeded random
    order: each block is allocated once and the holders are released in a
    permuted order."""
    cache = hx.PagedKvCache(layers, kv_heads, head_dim, block_tokens, physical_blocks,
                            page_dtype=page_dtype)
    rng = np.random.default_rng(seed)
    tok = torch.zeros(layers, kv_heads, head_dim, device="cuda:0")
    holders = []
    for _ in range(physical_blocks):
        s = cache.create_sequence()
        cache.append(s, tok, tok)
        holders.append(s)
    for i in rng.permutation(len(holders)):
        cache.release_sequence(holders[int(i)])
    return cache


def fill(cache, seq, tokens, gen):
    """Appends `tokens` N(0, 1) tokens to every layer of `seq` in one bulk
    append."""
    if tokens == 0:
        return
    L, H, Dh = cache.layers, cache.kv_heads, cache.head_dimension
    k = [torch.randn(H, tokens, Dh, device="cuda:0", generator=gen) for _ in range(L)]
    v = [torch.randn(H, tokens, Dh, device="cuda:0", generator=gen) for _ in range(L)]
    cache.append_layer_major(seq, k, v)


def generator(seed):
    g = torch.Generator(device="cuda:0")
    g.manual_seed(seed)
    return g


def config2(layers=1, seed=2):
    """Llama-2-7B MHA: 8 sequences, 32/32 heads, contexts U[128, 2048], pool
    1.25x the pages needed, shuffled."""
    rng = np.random.default_rng(seed)
    lengths = rng.integers(128, 2049, size=8)
    need = int(((lengths + P) // P + 1).sum())
    cache = shuffled_cache(layers, 32, int(math.ceil(1.25 * need)), seed)
    gen = generator(seed)
    seqs = []
    for n in lengths:
        s = cache.create_sequence()
        fill(cache, s, int(n), gen)
        seqs.append(s)
    return cache, seqs, 32


def config3(layers=1, seed=3, batch=64, page_dtype="f32"):
    """Llama-3-8B GQA: 64 sequences, 32/8 heads, contexts log-uniform in
    [512, 8192], shuffled pages."""
    rng = np.random.default_rng(seed)
    lengths = np.exp(rng.uniform(math.log(512), math.log(8192), size=batch)).astype(np.int64)
    need = int(((lengths + P) // P + 2).sum()) + 16
    cache = shuffled_cache(layers, 8, need, seed, page_dtype=page_dtype)
    gen = generator(seed)
    seqs = []
    for n in lengths:
        s = cache.create_sequence()
        fill(cache, s, int(n), gen)
        seqs.append(s)
    return cache, seqs, 32


def config4(layers=1, seed=4, steps=2, page_dtype="f32"):
    """Prefix sharing: 128 forks of a root of 1024 + 8 tokens (64 full pages
    shared at refcount 128, the 8-token partial page copied on write by
    every fork), then unique suffixes of U[64, 512] tokens; 32/8 heads."""
    rng = np.random.default_rng(seed)
    batch, prefix, partial = 128, 1024, 8
    suffix = rng.integers(64, 513, size=batch)
    own = (partial + suffix + steps + P - 1) // P + 1
    cache = shuffled_cache(layers, 8, int((prefix + partial) // P + 1 + own.sum() + 16), seed,
                           page_dtype=page_dtype)
    gen = generator(seed)
    root = cache.create_sequence()
    fill(cache, root, prefix + partial, gen)
    seqs = [cache.fork_sequence(root, prefix + partial, allow_cow=True) for _ in range(batch)]
    cache.release_sequence(root)
    for s, n in zip(seqs, suffix):
        fill(cache, s, int(n), gen)
    return cache, seqs, 32


def page_values(cache, pool, scale):
    """fp32 values of a host copy of a raw pool: the pool itself for fp32
    pages, bf16 bits widened, fp8 codes decoded times the cache's scale."""
    import oracle
    if cache.page_dtype == "bf16":
        return (pool.view(np.uint16).astype(np.uint32) << 16).view(np.float32)
    if cache.page_dtype == "fp8":
        return oracle.fp8_decode(pool) * np.float32(scale)
    return pool


def round_rows(cache, rows, scale):
    """Step rows (tail / chunk) on the cache's page grid."""
    import oracle
    if cache.page_dtype == "bf16":
        return oracle.round_bf16(rows)
    if cache.page_dtype == "fp8":
        return oracle.round_fp8(rows, scale)
    return rows


def oracle_inputs(cache, seqs, layer):
    """Host copies of one layer's pools (as fp32 values) and the batch's
    tables and lengths."""
    kr, vr = cache.layer_pools(layer)
    if cache.page_dtype == "bf16":
        kr, vr = kr.view(torch.int16), vr.view(torch.int16)
    kp = page_values(cache, kr.cpu().numpy(), cache.k_scale)
    vp = page_values(cache, vr.cpu().numpy(), cache.v_scale)
    tabs = [cache.block_table(s) for s in seqs]
    tables = np.zeros((len(seqs), max(len(t) for t in tabs) + 1), np.uint32)
    for b, t in enumerate(tabs):
        tables[b, : len(t)] = t
    lengths = np.array([cache.length(s) for s in seqs], np.int32)
    return kp, vp, tables, lengths
