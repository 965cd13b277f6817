"""The batched decode driver end to end: per step prepare (slot reservation
and incremental device tables), per layer append of the current token and
attention over the pre-step history plus the tail.  Outputs are checked
against the oracle per step and layer; the pages written by the appends are
checked bit-exactly against the oracle pool afterwards."""

import numpy as np
import pytest
import torch

import helix_runtime_amd as hx
import oracle

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-5, 1e-4
D, P = 128, 16


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda:0")


def host(t):
    return t.detach().cpu().numpy()


@pytest.mark.parametrize("mode", ["separate", "fused", "commit"])
@pytest.mark.parametrize("hq", [8, 32])
def test_decode_batch_steps_match_oracle(device, hq, mode):
    """separate: append_layer then attention_layer per layer; fused: one
    launch per layer; commit: attention over the uncommitted tail for every
    layer, then one append_all_layers launch (the reference's flow: the
    token is appended for all layers after the forward pass)."""
    L, H, D, P = 2, 8, 128, 16
    rng = np.random.default_rng(hq)
    lengths = [1, 15, 16, 31, 47, 200]
    N = sum((n + 8) // P + 2 for n in lengths) + 8
    cache = hx.PagedKvCache(L, H, D, P, N)
    pool = oracle.PagedPool(L, H, D, P, N)
    seqs = []
    for n in lengths:
        s, so = cache.create_sequence(), pool.create_sequence()
        k = rng.standard_normal((L, H, n, D), dtype=np.float32)
        v = rng.standard_normal((L, H, n, D), dtype=np.float32)
        cache.append_layer_major(s, [dev(k[l]) for l in range(L)], [dev(v[l]) for l in range(L)])
        pool.append_layer_major(so, k, v)
        seqs.append((s, so))
    # a bystander sequence keeps allocating between steps (FIFO interleaving)
    other, other_o = cache.create_sequence(), pool.create_sequence()
    B = len(seqs)
    batch = hx.DecodeBatch(cache, [s for s, _ in seqs], hq, max_tokens=256)
    for step in range(3):
        tok = np.zeros((1, L, H, 1, D), np.float32)
        cache.append_layer_major(other, [dev(tok[0, l]) for l in range(L)],
                                 [dev(tok[0, l]) for l in range(L)])
        pool.append_layer_major(other_o, tok[0], tok[0])
        batch.prepare()
        hist = np.array([pool.length(so) for _, so in seqs], np.int32)
        max_blocks = batch.device_state()["max_blocks"]
        tables = np.zeros((B, max_blocks), np.uint32)
        keys = rng.standard_normal((L, B, H, D), dtype=np.float32)
        values = rng.standard_normal((L, B, H, D), dtype=np.float32)
        for layer in range(L):
            q = rng.standard_normal((B, hq, D), dtype=np.float32)
            out = torch.empty(B, hq, D, device=device)
            if mode == "fused":
                batch.append_attention_layer(layer, dev(q), dev(keys[layer]), dev(values[layer]),
                                             out)
            elif mode == "separate":
                batch.append_layer(layer, dev(keys[layer]), dev(values[layer]))
                batch.attention_layer(layer, dev(q), dev(keys[layer]), dev(values[layer]), out)
            else:
                batch.attention_layer(layer, dev(q), dev(keys[layer]), dev(values[layer]), out)
            torch.cuda.synchronize()
            kp, vp = pool.layer_pages(layer)
            for b, (_, so) in enumerate(seqs):
                t = pool.block_table(so)
                tables[b, : len(t)] = t
            ref = oracle.batched_decode(q, kp, vp, tables, hist, keys[layer], values[layer],
                                        threads=8)
            np.testing.assert_allclose(host(out), ref, atol=ATOL, rtol=RTOL)
        if mode == "commit":
            batch.append_all_layers(dev(keys), dev(values))
        for b, (_, so) in enumerate(seqs):
            pool.append(so, keys[:, b], values[:, b])
        assert cache.stats() == pool.stats()
    for s, so in seqs:
        assert cache.block_table(s) == pool.block_table(so).tolist()
        for layer in range(L):
            gk, gv = cache.retrieve_layer(s, layer)
            ok, ov = pool.copy_layer(so, layer)
            np.testing.assert_array_equal(host(gk), ok)
            np.testing.assert_array_equal(host(gv), ov)
    batch.close()


@pytest.mark.parametrize("tokens", [1, 5, 16, 37])
def test_append_all_layers_chunk_bit_exact(device, tokens):
    """One append_all_layers launch writes a step of `tokens` tokens for every
    layer (rows [layers, batch, kv_heads, tokens, dim]) exactly as the oracle's
    layer-major append does, across page boundaries and mid-page starts."""
    L, H = 3, 4
    rng = np.random.default_rng(tokens)
    lengths = [0, 7, 16, 33]
    N = sum((n + tokens) // P + 2 for n in lengths) + 4
    cache = hx.PagedKvCache(L, H, D, P, N)
    pool = oracle.PagedPool(L, H, D, P, N)
    seqs = []
    for n in lengths:
        s, so = cache.create_sequence(), pool.create_sequence()
        if n:
            k = rng.standard_normal((L, H, n, D), dtype=np.float32)
            v = rng.standard_normal((L, H, n, D), dtype=np.float32)
            cache.append_layer_major(s, [dev(k[l]) for l in range(L)],
                                     [dev(v[l]) for l in range(L)])
            pool.append_layer_major(so, k, v)
        seqs.append((s, so))
    B = len(seqs)
    batch = hx.DecodeBatch(cache, [s for s, _ in seqs], H, max_tokens=128)
    if tokens == 1:
        batch.prepare()
    else:
        batch.prepare_chunk(tokens)
    keys = rng.standard_normal((L, B, H, tokens, D), dtype=np.float32)
    values = rng.standard_normal((L, B, H, tokens, D), dtype=np.float32)
    batch.append_all_layers(dev(keys), dev(values))
    torch.cuda.synchronize()
    for b, (_, so) in enumerate(seqs):
        pool.append_layer_major(so, keys[:, b], values[:, b])
    for s, so in seqs:
        assert cache.block_table(s) == pool.block_table(so).tolist()
        for layer in range(L):
            gk, gv = cache.retrieve_layer(s, layer)
            ok, ov = pool.copy_layer(so, layer)
            np.testing.assert_array_equal(host(gk), ok)
            np.testing.assert_array_equal(host(gv), ov)
    batch.close()


def test_decode_batch_validates(device):
    cache = hx.PagedKvCache(1, 2, 128, 16, 8)
    s = cache.create_sequence()
    with pytest.raises(hx.HelixError) as e:
        hx.DecodeBatch(cache, [s], 6, max_tokens=64)
    assert e.value.status == hx.UNSUPPORTED
    with pytest.raises(hx.HelixError):
        hx.DecodeBatch(cache, [s, s], 4, max_tokens=64)
    odd = hx.PagedKvCache(1, 2, 64, 16, 8)
    with pytest.raises(hx.HelixError) as e:
        hx.DecodeBatch(odd, [odd.create_sequence()], 4, max_tokens=64)
    assert e.value.status == hx.UNSUPPORTED
    b = hx.DecodeBatch(cache, [s], 4, max_tokens=17)
    x = torch.zeros(1, 2, 128, device=device)
    with pytest.raises(hx.HelixError):
        b.append_layer(0, x, x)  # before prepare
    b.prepare()
    with pytest.raises(hx.HelixError):
        b.append_layer(1, x, x)  # layer out of range
    b.close()


def test_prefix_sharing_decode_with_cow_forks(device):
    """Config-4 shape in small: forks share the full prefix pages (refcount =
    number of forks once the root is released) and copy the partial page on
    write, so each first suffix token lands mid-page in a private copy.
    Decode steps over the shared pages match the oracle; pages and stats
    match the oracle pool bit-exactly."""
    L, H, HQ = 2, 4, 16
    rng = np.random.default_rng(44)
    prefix, forks = 3 * P + 5, 6
    suffix = [3, 11, 16, 27, 40, 64]
    N = 64
    cache = hx.PagedKvCache(L, H, D, P, N)
    pool = oracle.PagedPool(L, H, D, P, N)
    root, root_o = cache.create_sequence(), pool.create_sequence()
    k = rng.standard_normal((L, H, prefix, D), dtype=np.float32)
    v = rng.standard_normal((L, H, prefix, D), dtype=np.float32)
    cache.append_layer_major(root, [dev(k[l]) for l in range(L)], [dev(v[l]) for l in range(L)])
    pool.append_layer_major(root_o, k, v)
    seqs = []
    for _ in range(forks):
        s = cache.fork_sequence(root, prefix, allow_cow=True)
        so = pool.fork_sequence(root_o, prefix, allow_cow=True)
        seqs.append((s, so))
    cache.release_sequence(root)
    pool.release_sequence(root_o)
    st = cache.stats()
    assert st == pool.stats()
    assert st["shared_blocks"] == prefix // P
    for b, (s, so) in enumerate(seqs):
        n = suffix[b]
        k = rng.standard_normal((L, H, n, D), dtype=np.float32)
        v = rng.standard_normal((L, H, n, D), dtype=np.float32)
        cache.append_layer_major(s, [dev(k[l]) for l in range(L)],
                                 [dev(v[l]) for l in range(L)])
        pool.append_layer_major(so, k, v)
    B = len(seqs)
    batch = hx.DecodeBatch(cache, [s for s, _ in seqs], HQ, max_tokens=prefix + max(suffix) + 8)
    for step in range(2):
        batch.prepare()
        hist = np.array([pool.length(so) for _, so in seqs], np.int32)
        tables = np.zeros((B, batch.device_state()["max_blocks"]), np.uint32)
        for b, (_, so) in enumerate(seqs):
            t = pool.block_table(so)
            tables[b, : len(t)] = t
        keys = rng.standard_normal((L, B, H, D), dtype=np.float32)
        values = rng.standard_normal((L, B, H, D), dtype=np.float32)
        for layer in range(L):
            q = rng.standard_normal((B, HQ, D), dtype=np.float32)
            out = torch.empty(B, HQ, D, device=device)
            batch.append_layer(layer, dev(keys[layer]), dev(values[layer]))
            batch.attention_layer(layer, dev(q), dev(keys[layer]), dev(values[layer]), out)
            torch.cuda.synchronize()
            kp, vp = pool.layer_pages(layer)
            ref = oracle.batched_decode(q, kp, vp, tables, hist, keys[layer], values[layer],
                                        threads=8)
            np.testing.assert_allclose(host(out), ref, atol=ATOL, rtol=RTOL)
        for b, (_, so) in enumerate(seqs):
            pool.append(so, keys[:, b], values[:, b])
    assert cache.stats() == pool.stats()
    for s, so in seqs:
        assert cache.block_table(s) == pool.block_table(so).tolist()
        for layer in range(L):
            gk, gv = cache.retrieve_layer(s, layer)
            ok, ov = pool.copy_layer(so, layer)
            np.testing.assert_array_equal(host(gk), ok)
            np.testing.assert_array_equal(host(gv), ov)
    batch.close()


@pytest.mark.parametrize("mode", ["separate", "fused", "commit"])
@pytest.mark.parametrize("hq", [4, 8, 32])
def test_cascade_shared_prefix_decode(device, hq, mode):
    """Sequences forked from one root share its full leading pages; the decode
    step attends them once for the batch (cascade) and the per-sequence rest
    through the stream kernel.  Outputs match the oracle over several steps,
    including a sequence whose history is exactly the shared prefix."""
    L, H = 2, 4
    rng = np.random.default_rng(77 + hq)
    prefix, forks = 10 * P, 8
    suffix = [0, 1, 5, 16, 17, 40, 100, 3]
    N = 128
    cache = hx.PagedKvCache(L, H, D, P, N)
    pool = oracle.PagedPool(L, H, D, P, N)
    root, root_o = cache.create_sequence(), pool.create_sequence()
    k = rng.standard_normal((L, H, prefix, D), dtype=np.float32)
    v = rng.standard_normal((L, H, prefix, D), dtype=np.float32)
    cache.append_layer_major(root, [dev(k[l]) for l in range(L)], [dev(v[l]) for l in range(L)])
    pool.append_layer_major(root_o, k, v)
    seqs = []
    for b in range(forks):
        s = cache.fork_sequence(root, prefix)
        so = pool.fork_sequence(root_o, prefix)
        n = suffix[b]
        if n:
            k = rng.standard_normal((L, H, n, D), dtype=np.float32)
            v = rng.standard_normal((L, H, n, D), dtype=np.float32)
            cache.append_layer_major(s, [dev(k[l]) for l in range(L)],
                                     [dev(v[l]) for l in range(L)])
            pool.append_layer_major(so, k, v)
        seqs.append((s, so))
    B = len(seqs)
    batch = hx.DecodeBatch(cache, [s for s, _ in seqs], hq, max_tokens=prefix + max(suffix) + 8)
    for step in range(3):
        batch.prepare()
        assert batch.shared_pages() == prefix // P
        hist = np.array([pool.length(so) for _, so in seqs], np.int32)
        tables = np.zeros((B, batch.device_state()["max_blocks"]), np.uint32)
        for b, (_, so) in enumerate(seqs):
            t = pool.block_table(so)
            tables[b, : len(t)] = t
        keys = rng.standard_normal((L, B, H, D), dtype=np.float32)
        values = rng.standard_normal((L, B, H, D), dtype=np.float32)
        for layer in range(L):
            q = rng.standard_normal((B, hq, D), dtype=np.float32)
            out = torch.empty(B, hq, D, device=device)
            if mode == "fused":
                batch.append_attention_layer(layer, dev(q), dev(keys[layer]), dev(values[layer]),
                                             out)
            elif mode == "separate":
                batch.append_layer(layer, dev(keys[layer]), dev(values[layer]))
                batch.attention_layer(layer, dev(q), dev(keys[layer]), dev(values[layer]), out)
            else:
                batch.attention_layer(layer, dev(q), dev(keys[layer]), dev(values[layer]), out)
            torch.cuda.synchronize()
            kp, vp = pool.layer_pages(layer)
            ref = oracle.batched_decode(q, kp, vp, tables, hist, keys[layer], values[layer],
                                        threads=8)
            np.testing.assert_allclose(host(out), ref, atol=ATOL, rtol=RTOL)
        if mode == "commit":
            batch.append_all_layers(dev(keys), dev(values))
        for b, (_, so) in enumerate(seqs):
            pool.append(so, keys[:, b], values[:, b])
    assert cache.stats() == pool.stats()
    for s, so in seqs:
        for layer in range(L):
            gk, gv = cache.retrieve_layer(s, layer)
            ok, ov = pool.copy_layer(so, layer)
            np.testing.assert_array_equal(host(gk), ok)
            np.testing.assert_array_equal(host(gv), ov)
    batch.close()


def _fill(cache, pool, s, so, n, rng):
    L, H = cache.layers, cache.kv_heads
    k = rng.standard_normal((L, H, n, D), dtype=np.float32)
    v = rng.standard_normal((L, H, n, D), dtype=np.float32)
    cache.append_layer_major(s, [dev(k[l]) for l in range(L)], [dev(v[l]) for l in range(L)])
    pool.append_layer_major(so, k, v)


def _step_checked(batch, cache, pool, seqs, hq, rng, device, stream=None):
    """One decode step (append_layer + attention_layer per layer) checked
    against the oracle; the oracle pool takes the same tokens."""
    L, H, B = cache.layers, cache.kv_heads, len(seqs)
    batch.prepare(stream)
    hist = np.array([pool.length(so) for _, so in seqs], np.int32)
    tables = np.zeros((B, batch.device_state()["max_blocks"]), np.uint32)
    for b, (_, so) in enumerate(seqs):
        t = pool.block_table(so)
        tables[b, : len(t)] = t
    keys = rng.standard_normal((L, B, H, D), dtype=np.float32)
    values = rng.standard_normal((L, B, H, D), dtype=np.float32)
    for layer in range(L):
        q = rng.standard_normal((B, hq, D), dtype=np.float32)
        out = torch.empty(B, hq, D, device=device)
        batch.append_layer(layer, dev(keys[layer]), dev(values[layer]), stream)
        batch.attention_layer(layer, dev(q), dev(keys[layer]), dev(values[layer]), out, stream)
        torch.cuda.synchronize()
        kp, vp = pool.layer_pages(layer)
        ref = oracle.batched_decode(q, kp, vp, tables, hist, keys[layer], values[layer],
                                    threads=8)
        np.testing.assert_allclose(host(out), ref, atol=ATOL, rtol=RTOL)
    for b, (_, so) in enumerate(seqs):
        pool.append(so, keys[:, b], values[:, b])


def test_outside_append_between_steps_reaches_device_tables(device):
    """A member appended to through the cache between steps (crossing page
    boundaries) has its new pages in the device tables at the next
    prepare(): attention reads the right pages and the fused step writes
    into the right slot."""
    L, H, HQ = 2, 4, 16
    rng = np.random.default_rng(91)
    N = 96
    cache = hx.PagedKvCache(L, H, D, P, N)
    pool = oracle.PagedPool(L, H, D, P, N)
    seqs = []
    for n in (5, 16, 30):
        s, so = cache.create_sequence(), pool.create_sequence()
        _fill(cache, pool, s, so, n, rng)
        seqs.append((s, so))
    batch = hx.DecodeBatch(cache, [s for s, _ in seqs], HQ, max_tokens=256)
    _step_checked(batch, cache, pool, seqs, HQ, rng, device)
    # 40 tokens outside the batch: member 1 (17 tokens) gains three pages.
    _fill(cache, pool, seqs[1][0], seqs[1][1], 40, rng)
    # A bystander takes pages in between so a stale entry would point at
    # someone else's data.
    other, other_o = cache.create_sequence(), pool.create_sequence()
    _fill(cache, pool, other, other_o, 33, rng)
    _step_checked(batch, cache, pool, seqs, HQ, rng, device)
    _step_checked(batch, cache, pool, seqs, HQ, rng, device)
    assert cache.stats() == pool.stats()
    for s, so in seqs:
        assert cache.block_table(s) == pool.block_table(so).tolist()
        for layer in range(L):
            gk, gv = cache.retrieve_layer(s, layer)
            ok, ov = pool.copy_layer(so, layer)
            np.testing.assert_array_equal(host(gk), ok)
            np.testing.assert_array_equal(host(gv), ov)
    batch.close()


def test_release_after_prepare_is_rejected(device):
    """Releasing a member between prepare() and the step's calls makes every
    later call of the step, and the next prepare(), fail instead of writing
    into freed pages; releasing a bystander does not."""
    cache = hx.PagedKvCache(1, 2, D, P, 32)
    a, b, c = (cache.create_sequence() for _ in range(3))
    x = torch.zeros(1, 2, D, device=device)
    for s in (a, b, c):
        cache.append(s, x, x)
    batch = hx.DecodeBatch(cache, [a, b], 4, max_tokens=64)
    q = torch.zeros(2, 4, D, device=device)
    rows = torch.zeros(2, 2, D, device=device)
    out = torch.empty(2, 4, D, device=device)
    batch.prepare()
    cache.release_sequence(c)  # not a member: the step stays valid
    batch.append_attention_layer(0, q, rows, rows, out)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    cache.release_sequence(b)
    for call in (lambda: batch.append_layer(0, rows, rows),
                 lambda: batch.attention_layer(0, q, rows, rows, out),
                 lambda: batch.append_attention_layer(0, q, rows, rows, out)):
        with pytest.raises(hx.HelixError) as e:
            call()
        assert e.value.status == hx.INVALID_ARGUMENT
        assert "released" in str(e.value)
    with pytest.raises(hx.HelixError):
        batch.prepare()
    batch.close()


def test_failed_prepare_leaves_batch_unprepared(device):
    """A prepare() that fails (the pool has no free page for the step) does
    not leave the previous step usable."""
    cache = hx.PagedKvCache(1, 2, D, P, 2)
    s = cache.create_sequence()
    x = torch.zeros(1, 2, D, device=device)
    for _ in range(16):
        cache.append(s, x, x)
    filler = cache.create_sequence()
    cache.append(filler, x, x)  # takes the last free page
    batch = hx.DecodeBatch(cache, [s], 4, max_tokens=64)
    rows = torch.zeros(1, 2, D, device=device)
    with pytest.raises(hx.HelixError) as e:
        batch.prepare()
    assert e.value.status == hx.RESOURCE_EXHAUSTED
    with pytest.raises(hx.HelixError) as e:
        batch.append_layer(0, rows, rows)
    assert "before prepare" in str(e.value)
    cache.release_sequence(filler)
    batch.prepare()
    batch.append_layer(0, rows, rows)
    torch.cuda.synchronize()
    batch.close()


def test_step_calls_on_other_streams(device):
    """prepare() on one stream and the step's calls on another: the calls
    wait for the step upload, and the next prepare() on the first stream
    waits for them."""
    L, H, HQ = 2, 4, 8
    rng = np.random.default_rng(93)
    cache = hx.PagedKvCache(L, H, D, P, 64)
    pool = oracle.PagedPool(L, H, D, P, 64)
    seqs = []
    for n in (15, 16, 17, 100):
        s, so = cache.create_sequence(), pool.create_sequence()
        _fill(cache, pool, s, so, n, rng)
        seqs.append((s, so))
    batch = hx.DecodeBatch(cache, [s for s, _ in seqs], HQ, max_tokens=256)
    side = torch.cuda.Stream()
    B = len(seqs)
    for step in range(3):
        hist = np.array([pool.length(so) for _, so in seqs], np.int32)
        keys = rng.standard_normal((L, B, H, D), dtype=np.float32)
        values = rng.standard_normal((L, B, H, D), dtype=np.float32)
        qs = rng.standard_normal((L, B, HQ, D), dtype=np.float32)
        dk, dvv, dq = dev(keys), dev(values), dev(qs)
        outs = [torch.empty(B, HQ, D, device=device) for _ in range(L)]
        torch.cuda.synchronize()
        # No host synchronisation between the upload and the side stream's
        # launches: only the library's stream ordering separates them.
        batch.prepare(torch.cuda.current_stream())
        for layer in range(L):
            batch.append_attention_layer(layer, dq[layer], dk[layer], dvv[layer], outs[layer],
                                         side)
        side.synchronize()
        tables = np.zeros((B, batch.device_state()["max_blocks"]), np.uint32)
        for b, (_, so) in enumerate(seqs):
            t = pool.block_table(so)
            tables[b, : len(t)] = t
        for layer in range(L):
            kp, vp = pool.layer_pages(layer)
            ref = oracle.batched_decode(qs[layer], kp, vp, tables, hist, keys[layer],
                                        values[layer], threads=8)
            np.testing.assert_allclose(host(outs[layer]), ref, atol=ATOL, rtol=RTOL)
        for b, (_, so) in enumerate(seqs):
            pool.append(so, keys[:, b], values[:, b])
    batch.close()


@pytest.mark.parametrize("page_dtype", ["f32", "bf16"])
@pytest.mark.parametrize("hq", [8, 32])
def test_decode_over_many_short_sequences(device, hq, page_dtype):
    """1024 sequences of 0-40 tokens (a quarter empty: their unit is the
    tail alone).  Past 256 sequences the stream kernel finds each
    wavefront's first unit by scanning the lengths chunk by chunk beyond its
    preloaded four, and each wavefront runs through several short units."""
    L, H, B = 1, 8, 1024
    rnd = (lambda x: x) if page_dtype == "f32" else oracle.round_bf16
    rng = np.random.default_rng(31 + hq)
    lengths = rng.integers(0, 41, size=B)
    lengths[rng.random(B) < 0.25] = 0
    N = int(sum((n + P - 1) // P + 1 for n in lengths)) + 8
    cache = hx.PagedKvCache(L, H, D, P, N, page_dtype=page_dtype)
    pool = oracle.PagedPool(L, H, D, P, N)
    seqs = []
    for n in lengths:
        s, so = cache.create_sequence(), pool.create_sequence()
        if n:
            k = rng.standard_normal((L, H, n, D), dtype=np.float32)
            v = rng.standard_normal((L, H, n, D), dtype=np.float32)
            cache.append_layer_major(s, [dev(k[0])], [dev(v[0])])
            pool.append_layer_major(so, rnd(k), rnd(v))
        seqs.append((s, so))
    batch = hx.DecodeBatch(cache, [s for s, _ in seqs], hq, max_tokens=64)
    batch.prepare()
    hist = np.array([pool.length(so) for _, so in seqs], np.int32)
    tables = np.zeros((B, batch.device_state()["max_blocks"]), np.uint32)
    for b, (_, so) in enumerate(seqs):
        t = pool.block_table(so)
        tables[b, : len(t)] = t
    keys = rng.standard_normal((B, H, D), dtype=np.float32)
    values = rng.standard_normal((B, H, D), dtype=np.float32)
    q = rng.standard_normal((B, hq, D), dtype=np.float32)
    out = torch.empty(B, hq, D, device=device)
    batch.attention_layer(0, dev(q), dev(keys), dev(values), out)
    torch.cuda.synchronize()
    kp, vp = pool.layer_pages(0)
    ref = oracle.batched_decode(q, kp, vp, tables, hist, rnd(keys), rnd(values), threads=8)
    np.testing.assert_allclose(host(out), ref, atol=ATOL, rtol=RTOL)
    batch.close()


def test_stateless_decode_of_1000_sequences(device):
    """The batched C-ABI entry (caller workspace) at 1000 sequences, not a
    multiple of the 64-sequence scan chunk, with ragged contexts."""
    rng = np.random.default_rng(41)
    B, hkv, hq = 1000, 8, 32
    lengths = rng.integers(0, 300, size=B).astype(np.int32)
    pages = (lengths + P - 1) // P
    phys = int(pages.sum()) + 4
    perm = rng.permutation(phys).astype(np.uint32)
    max_blocks = int(pages.max()) + 1
    tables = np.zeros((B, max_blocks), np.uint32)
    at = 0
    for b, n in enumerate(pages):
        tables[b, :n] = perm[at: at + n]
        at += n
    kp = rng.standard_normal((phys, hkv, P, D), dtype=np.float32)
    vp = rng.standard_normal((phys, hkv, P, D), dtype=np.float32)
    q = rng.standard_normal((B, hq, D), dtype=np.float32)
    tk = rng.standard_normal((B, hkv, D), dtype=np.float32)
    tv = rng.standard_normal((B, hkv, D), dtype=np.float32)
    out = torch.empty(B, hq, D, device=device)
    ws = hx.decode_workspace(B, hq, hkv, max_blocks)
    hx.paged_decode_attention(dev(q), dev(kp), dev(vp), dev(tables.view(np.int32)), dev(lengths),
                              dev(tk), dev(tv), out, ws)
    torch.cuda.synchronize()
    ref = oracle.batched_decode(q, kp, vp, tables, lengths, tk, tv, threads=8)
    np.testing.assert_allclose(host(out), ref, atol=ATOL, rtol=RTOL)
