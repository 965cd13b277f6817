"""Prefix cache over the device pool: the payload checks of the reference's
tests/prefix_cache_test.cpp (pages a lookup returns hold the anchored
source's K/V, anchors keep them alive after the source is released), and a
decode step over sequences forked from one cached prompt (the cascade path)
against the CPU oracle."""

import numpy as np
import pytest
import torch

import helix_runtime_amd as hx
import oracle

pytestmark = pytest.mark.gpu


def append_tokens(cache, seq, count, base):
    # prefix_cache_test.cpp:19-27: key base + t, value base + 1000 + t.
    for t in range(count):
        k = torch.full((1, 1, 1), base + t, dtype=torch.float32, device="cuda:0")
        v = torch.full((1, 1, 1), base + 1000.0 + t, dtype=torch.float32, device="cuda:0")
        cache.append(seq, k, v)


def expect_payload(cache, seq, count, base):
    # prefix_cache_test.cpp:29-39.
    k, v = cache.retrieve_layer(seq, 0)
    torch.cuda.synchronize()
    assert tuple(k.shape) == (1, count, 1)
    want = base + np.arange(count, dtype=np.float32)
    assert np.array_equal(k.cpu().numpy()[0, :, 0], want)
    assert np.array_equal(v.cpu().numpy()[0, :, 0], want + 1000.0)


def test_lookups_return_the_anchored_payload(device):
    """prefix_cache_test.cpp:116-164."""
    cache = hx.PagedKvCache(1, 1, 1, 2, 6)
    srcs = [cache.create_sequence() for _ in range(3)]
    for s, base in zip(srcs, (100.0, 200.0, 300.0)):
        append_tokens(cache, s, 2, base)
    prefixes = hx.PagedPrefixCache(cache, 4, 4)
    assert prefixes.insert(1, [7, 8], srcs[0]) == hx.PREFIX_INSERTED
    assert prefixes.insert(1, [7, 9], srcs[1]) == hx.PREFIX_INSERTED
    assert prefixes.insert(2, [7, 8], srcs[2]) == hx.PREFIX_INSERTED
    assert prefixes.insert(1, [7, 8], srcs[1]) == hx.PREFIX_ALREADY_PRESENT
    got = [prefixes.lookup_longest(1, [7, 8]), prefixes.lookup_longest(1, [7, 9]),
           prefixes.lookup_longest(2, [7, 8])]
    for (seq, matched), src, base in zip(got, srcs, (100.0, 200.0, 300.0)):
        assert matched == 2
        assert cache.block_table(seq)[0] == cache.block_table(src)[0]
        expect_payload(cache, seq, 2, base)
    for seq, _ in got:
        cache.release_sequence(seq)
    prefixes.close()
    for s in srcs:
        cache.release_sequence(s)
    assert cache.stats()["used_blocks"] == 0


def test_anchor_keeps_payload_alive(device):
    """prefix_cache_test.cpp:279-303."""
    cache = hx.PagedKvCache(1, 1, 1, 2, 2)
    source = cache.create_sequence()
    append_tokens(cache, source, 4, 50.0)
    tokens = [40, 41, 42, 43]
    prefixes = hx.PagedPrefixCache(cache, 1, 2)
    assert prefixes.insert(5, tokens, source) == hx.PREFIX_INSERTED
    cache.release_sequence(source)
    assert cache.stats()["active_sequence_count"] == 1 and cache.stats()["free_blocks"] == 0
    match, matched = prefixes.lookup_longest(5, tokens)
    assert matched == 4
    prefixes.clear()
    assert prefixes.stats()["erase_count"] == 1
    assert cache.stats()["active_sequence_count"] == 1 and cache.stats()["free_blocks"] == 0
    expect_payload(cache, match, 4, 50.0)
    cache.release_sequence(match)
    c = cache.stats()
    assert (c["active_sequence_count"], c["used_blocks"], c["free_blocks"]) == (0, 0, 2)


def test_index_outlives_the_cache_handle(device):
    """The index keeps the device pool alive: anchors are released into it
    after the cache handle is closed."""
    cache = hx.PagedKvCache(1, 1, 1, 2, 4)
    source = cache.create_sequence()
    append_tokens(cache, source, 2, 1.0)
    prefixes = hx.PagedPrefixCache(cache, 2, 4)
    assert prefixes.insert(3, [1, 2], source) == hx.PREFIX_INSERTED
    cache.close()
    assert prefixes.contains(3, [1, 2])
    prefixes.close()


def test_cached_prompt_forks_decode_like_the_oracle(device):
    """A prompt cached once, looked up by 6 requests; each fork appends its
    own tokens and the batch decodes through the cascade path.  Outputs
    match the oracle's paged attention on the oracle pool that replayed the
    same operations."""
    L, H, HQ, D, P, N = 1, 2, 8, 128, 16, 64
    rng = np.random.default_rng(11)
    cache, pool = hx.PagedKvCache(L, H, D, P, N), oracle.PagedPool(L, H, D, P, N)
    prompt_len = 5 * P
    src, osrc = cache.create_sequence(), pool.create_sequence()
    k = rng.standard_normal((L, H, prompt_len, D), dtype=np.float32)
    v = rng.standard_normal((L, H, prompt_len, D), dtype=np.float32)
    cache.append_layer_major(src, [torch.from_numpy(k[0]).cuda()], [torch.from_numpy(v[0]).cuda()])
    pool.append_layer_major(osrc, k, v)
    prompt = [int(t) for t in rng.integers(0, 50000, prompt_len)]
    prefixes = hx.PagedPrefixCache(cache, 8, 32)
    assert prefixes.insert(1, prompt, src) == hx.PREFIX_INSERTED
    seqs, oseqs = [], []
    for r in range(6):
        query = prompt + [int(t) for t in rng.integers(0, 50000, 7)]
        seq, matched = prefixes.lookup_longest(1, query)
        assert matched == prompt_len
        oseq = pool.fork_sequence(osrc, matched)
        extra = 3 + 5 * r
        ke = rng.standard_normal((L, H, extra, D), dtype=np.float32)
        ve = rng.standard_normal((L, H, extra, D), dtype=np.float32)
        cache.append_layer_major(seq, [torch.from_numpy(ke[0]).cuda()],
                                 [torch.from_numpy(ve[0]).cuda()])
        pool.append_layer_major(oseq, ke, ve)
        assert cache.block_table(seq) == list(pool.block_table(oseq))
        seqs.append(seq)
        oseqs.append(oseq)
    batch = hx.DecodeBatch(cache, seqs, HQ, max_tokens=prompt_len + 64)
    batch.prepare()
    assert batch.shared_pages() == 5
    q = rng.standard_normal((6, HQ, D), dtype=np.float32)
    tk = rng.standard_normal((6, H, D), dtype=np.float32)
    tv = rng.standard_normal((6, H, D), dtype=np.float32)
    out = torch.empty(6, HQ, D, device="cuda:0")
    dq, dk, dv = (torch.from_numpy(a).cuda() for a in (q, tk, tv))
    batch.append_attention_layer(0, dq, dk, dv, out)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    kp, vp = pool.layer_pages(0)
    for b, oseq in enumerate(oseqs):
        tab = np.array(pool.block_table(oseq), np.uint32)
        want = oracle.paged_attention(q[b][:, None], kp, vp, tab, pool.length(oseq),
                                      tk[b][:, None], tv[b][:, None])[0][:, 0]
        diff = np.abs(got[b].astype(np.float64) - want)
        assert (diff <= 2e-5 + 1e-4 * np.abs(want)).all(), f"sequence {b}: {diff.max()}"
    batch.close()
    for s in seqs:
        cache.release_sequence(s)
    prefixes.close()
    cache.release_sequence(src)
    assert cache.stats()["used_blocks"] == 0
