"""bf16 pages (extension; the reference stores fp32 only, docs/KV_CACHE.md:531).

Contract, checked here through the C ABI:
- a page element is the appended fp32 value rounded to nearest even
  (oracle.bf16_bits, pinned in test_oracle.py), bit-exact, for the token,
  bulk, slot and fused appends and through copy-on-write forks; gathers widen
  it back exactly;
- attention over a bf16 cache equals the fp32 oracle evaluated on the
  rounded pages and the rounded step rows (tail / chunk), within the fp32
  tolerance: max-abs 2e-5 plus rel 1e-4.
The oracle pool is fed the rounded values, so its pages are the bf16 pages
widened."""

import numpy as np
import pytest
import torch

import helix_runtime_amd as hx
import oracle

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-5, 1e-4
D, P = 128, 16
R = oracle.round_bf16


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda:0")


def host(t):
    return t.detach().cpu().numpy()


def bits_equal(got, want):
    return np.array_equal(np.asarray(got, np.float32).view(np.uint32),
                          np.asarray(want, np.float32).view(np.uint32))


def byte_free(stats):
    return {k: v for k, v in stats.items() if not k.startswith("bytes") and k != "peak_bytes_used"}


def test_pages_hold_rounded_values_and_halve_the_bytes(device):
    L, H, N = 2, 3, 8
    cache = hx.PagedKvCache(L, H, D, P, N, page_dtype="bf16")
    f32 = hx.PagedKvCache(L, H, D, P, N)
    assert cache.stats()["bytes_reserved"] * 2 == f32.stats()["bytes_reserved"]
    f32.close()
    rng = np.random.default_rng(1)
    s = cache.create_sequence()
    k = rng.standard_normal((L, H, 21, D), dtype=np.float32) * 50
    v = rng.standard_normal((L, H, 21, D), dtype=np.float32)
    special = np.array([np.nan, -np.nan, np.inf, -np.inf, 0.0, -0.0, 3.4e38, -3.4e38, 1e-40,
                        np.uint32(0x3F808000).view(np.float32),
                        np.uint32(0x3F818000).view(np.float32)], np.float32)
    k[0, 0, 3, : special.size] = special
    v[1, 2, 20, : special.size] = special
    cache.append_layer_major(s, [dev(k[l]) for l in range(L)], [dev(v[l]) for l in range(L)])
    tok_k = rng.standard_normal((L, H, D), dtype=np.float32)
    tok_v = rng.standard_normal((L, H, D), dtype=np.float32)
    tok_k[1, 1, :4] = [np.nan, 1.00390625, -np.inf, 65504.5]
    cache.append(s, dev(tok_k), dev(tok_v))
    want_k = np.concatenate([k, tok_k[:, :, None]], axis=2)
    want_v = np.concatenate([v, tok_v[:, :, None]], axis=2)
    table = cache.block_table(s)
    for layer in range(L):
        gk, gv = cache.retrieve_layer(s, layer)
        torch.cuda.synchronize()
        got_k, got_v = host(gk), host(gv)
        # Widening is exact, NaN payloads included.
        assert bits_equal(got_k, R(want_k[layer])) and bits_equal(got_v, R(want_v[layer]))
        # Raw page bits: oracle encodings at the right positions.
        kp, vp = cache.layer_pools(layer)
        raw = kp.view(torch.int16).cpu().numpy().view(np.uint16)
        for t in range(22):
            blk = table[t // P]
            assert np.array_equal(raw[blk, :, t % P], oracle.bf16_bits(want_k[layer, :, t]))
    cache.release_sequence(s)


@pytest.mark.parametrize("seed", [0, 1])
def test_random_program_pages_match_rounded_oracle(device, seed):
    """create / token append / bulk append / aligned and copy-on-write forks /
    release on a bf16 cache against the oracle pool fed rounded rows."""
    L, H, N = 2, 2, 40
    rng = np.random.default_rng(100 + seed)
    cache = hx.PagedKvCache(L, H, D, P, N, page_dtype="bf16")
    pool = oracle.PagedPool(L, H, D, P, N)
    live = []
    for step in range(60):
        op = rng.integers(0, 6)
        if op == 0 or not live:
            live.append((cache.create_sequence(), pool.create_sequence()))
        elif op == 1:
            s, so = live[rng.integers(len(live))]
            if pool.stats()["free_blocks"] > 2:
                k = rng.standard_normal((L, H, D), dtype=np.float32)
                v = rng.standard_normal((L, H, D), dtype=np.float32)
                cache.append(s, dev(k), dev(v))
                pool.append(so, R(k), R(v))
        elif op == 2:
            s, so = live[rng.integers(len(live))]
            n = int(rng.integers(1, 30))
            if pool.stats()["free_blocks"] * P > n + P:
                k = rng.standard_normal((L, H, n, D), dtype=np.float32)
                v = rng.standard_normal((L, H, n, D), dtype=np.float32)
                cache.append_layer_major(s, [dev(k[l]) for l in range(L)],
                                         [dev(v[l]) for l in range(L)])
                pool.append_layer_major(so, R(k), R(v))
        elif op == 3:
            s, so = live[rng.integers(len(live))]
            n = pool.length(so)
            if n and pool.stats()["free_blocks"] > 1:
                cut = int(rng.integers(1, n + 1))
                live.append((cache.fork_sequence(s, cut, allow_cow=True),
                             pool.fork_sequence(so, cut, allow_cow=True)))
        elif len(live) > 1:
            s, so = live.pop(int(rng.integers(len(live))))
            cache.release_sequence(s)
            pool.release_sequence(so)
        assert byte_free(cache.stats()) == byte_free(pool.stats()), f"step {step}"
    for s, so in live:
        assert cache.block_table(s) == pool.block_table(so).tolist()
        for layer in range(L):
            gk, gv = cache.retrieve_layer(s, layer)
            ok, ov = pool.copy_layer(so, layer)
            assert bits_equal(host(gk), ok) and bits_equal(host(gv), ov)


@pytest.mark.parametrize("fused", [False, True])
@pytest.mark.parametrize("hq", [8, 32])
def test_decode_steps_match_oracle_on_rounded_values(device, hq, fused):
    L, H = 2, 8
    rng = np.random.default_rng(7 + hq)
    lengths = [1, 15, 16, 31, 47, 200, 600]
    N = sum((n + 8) // P + 2 for n in lengths) + 8
    cache = hx.PagedKvCache(L, H, D, P, N, page_dtype="bf16")
    pool = oracle.PagedPool(L, H, D, P, N)
    seqs = []
    for n in lengths:
        s, so = cache.create_sequence(), pool.create_sequence()
        k = rng.standard_normal((L, H, n, D), dtype=np.float32)
        v = rng.standard_normal((L, H, n, D), dtype=np.float32)
        cache.append_layer_major(s, [dev(k[l]) for l in range(L)], [dev(v[l]) for l in range(L)])
        pool.append_layer_major(so, R(k), R(v))
        seqs.append((s, so))
    B = len(seqs)
    batch = hx.DecodeBatch(cache, [s for s, _ in seqs], hq, max_tokens=700)
    for step in range(2):
        batch.prepare()
        hist = np.array([pool.length(so) for _, so in seqs], np.int32)
        tables = np.zeros((B, batch.device_state()["max_blocks"]), np.uint32)
        keys = rng.standard_normal((L, B, H, D), dtype=np.float32)
        values = rng.standard_normal((L, B, H, D), dtype=np.float32)
        for layer in range(L):
            q = rng.standard_normal((B, hq, D), dtype=np.float32)
            out = torch.empty(B, hq, D, device=device)
            if fused:
                batch.append_attention_layer(layer, dev(q), dev(keys[layer]), dev(values[layer]),
                                             out)
            else:
                batch.append_layer(layer, dev(keys[layer]), dev(values[layer]))
                batch.attention_layer(layer, dev(q), dev(keys[layer]), dev(values[layer]), out)
            torch.cuda.synchronize()
            kp, vp = pool.layer_pages(layer)
            for b, (_, so) in enumerate(seqs):
                t = pool.block_table(so)
                tables[b, : len(t)] = t
            ref = oracle.batched_decode(q, kp, vp, tables, hist, R(keys[layer]),
                                        R(values[layer]), threads=8)
            np.testing.assert_allclose(host(out), ref, atol=ATOL, rtol=RTOL)
        for b, (_, so) in enumerate(seqs):
            pool.append(so, R(keys[:, b]), R(values[:, b]))
    for s, so in seqs:
        for layer in range(L):
            gk, gv = cache.retrieve_layer(s, layer)
            ok, ov = pool.copy_layer(so, layer)
            assert bits_equal(host(gk), ok) and bits_equal(host(gv), ov)
    batch.close()


def test_cascade_decode_on_bf16_pages(device):
    """Forks of one prompt share its pages; the decode step attends them once
    (cascade prefix pass, bf16 staging) plus each fork's own pages."""
    L, H, HQ = 1, 4, 16
    rng = np.random.default_rng(21)
    N = 64
    cache = hx.PagedKvCache(L, H, D, P, N, page_dtype="bf16")
    pool = oracle.PagedPool(L, H, D, P, N)
    root, root_o = cache.create_sequence(), pool.create_sequence()
    k = rng.standard_normal((L, H, 6 * P, D), dtype=np.float32)
    v = rng.standard_normal((L, H, 6 * P, D), dtype=np.float32)
    cache.append_layer_major(root, [dev(k[0])], [dev(v[0])])
    pool.append_layer_major(root_o, R(k), R(v))
    seqs = []
    for i in range(5):
        s, so = cache.fork_sequence(root, 6 * P), pool.fork_sequence(root_o, 6 * P)
        n = 3 + 7 * i
        ke = rng.standard_normal((L, H, n, D), dtype=np.float32)
        ve = rng.standard_normal((L, H, n, D), dtype=np.float32)
        cache.append_layer_major(s, [dev(ke[0])], [dev(ve[0])])
        pool.append_layer_major(so, R(ke), R(ve))
        seqs.append((s, so))
    batch = hx.DecodeBatch(cache, [s for s, _ in seqs], HQ, max_tokens=200)
    batch.prepare()
    assert batch.shared_pages() == 6
    q = rng.standard_normal((5, HQ, D), dtype=np.float32)
    tk = rng.standard_normal((5, H, D), dtype=np.float32)
    tv = rng.standard_normal((5, H, D), dtype=np.float32)
    out = torch.empty(5, HQ, D, device=device)
    batch.append_attention_layer(0, dev(q), dev(tk), dev(tv), out)
    torch.cuda.synchronize()
    kp, vp = pool.layer_pages(0)
    for b, (_, so) in enumerate(seqs):
        tab = np.array(pool.block_table(so), np.uint32)
        want = oracle.paged_attention(q[b][:, None], kp, vp, tab, pool.length(so),
                                      R(tk[b])[:, None], R(tv[b])[:, None])[0][:, 0]
        np.testing.assert_allclose(host(out)[b], want, atol=ATOL, rtol=RTOL)
    batch.close()


def test_chunked_prefill_on_bf16_pages(device):
    L, H, HQ = 2, 4, 16
    rng = np.random.default_rng(31)
    hists = [0, 5, 16, 70, 300]
    T = 40
    N = sum((h + T + 1) // P + 2 for h in hists) + 4
    cache = hx.PagedKvCache(L, H, D, P, N, page_dtype="bf16")
    pool = oracle.PagedPool(L, H, D, P, N)
    seqs = []
    for h in hists:
        s, so = cache.create_sequence(), pool.create_sequence()
        if h:
            k = rng.standard_normal((L, H, h, D), dtype=np.float32)
            v = rng.standard_normal((L, H, h, D), dtype=np.float32)
            cache.append_layer_major(s, [dev(k[l]) for l in range(L)], [dev(v[l]) for l in range(L)])
            pool.append_layer_major(so, R(k), R(v))
        seqs.append((s, so))
    B = len(seqs)
    batch = hx.DecodeBatch(cache, [s for s, _ in seqs], HQ, max_tokens=max(hists) + T + 8)
    batch.prepare_chunk(T)
    ck = rng.standard_normal((L, B, H, T, D), dtype=np.float32)
    cv = rng.standard_normal((L, B, H, T, D), dtype=np.float32)
    for layer in range(L):
        q = rng.standard_normal((B, HQ, T, D), dtype=np.float32)
        out = torch.empty(B, HQ, T, D, device=device)
        batch.append_layer(layer, dev(ck[layer]), dev(cv[layer]))
        batch.prefill_layer(layer, dev(q), dev(ck[layer]), dev(cv[layer]), out)
        torch.cuda.synchronize()
        kp, vp = pool.layer_pages(layer)
        for b, (_, so) in enumerate(seqs):
            tab = np.array(pool.block_table(so), np.uint32)
            want = oracle.paged_attention(q[b], kp, vp, tab, pool.length(so), R(ck[layer, b]),
                                          R(cv[layer, b]))[0]
            np.testing.assert_allclose(host(out)[b], want, atol=ATOL, rtol=RTOL)
    for b, (s, so) in enumerate(seqs):
        pool.append_layer_major(so, R(ck[:, b]), R(cv[:, b]))
        for layer in range(L):
            gk, gv = cache.retrieve_layer(s, layer)
            ok, ov = pool.copy_layer(so, layer)
            assert bits_equal(host(gk), ok) and bits_equal(host(gv), ov)
    batch.close()


def test_bf16_validation(device):
    with pytest.raises(hx.HelixError) as e:
        hx.PagedKvCache(1, 1, D, P, 4, page_dtype="fp4")
    assert e.value.status == hx.INVALID_ARGUMENT
    cache = hx.PagedKvCache(1, 2, D, P, 8, page_dtype="bf16")
    s = cache.create_sequence()
    with pytest.raises(hx.HelixError) as e:  # the split path reads fp32 pages only
        hx.DecodeBatch(cache, [s], 8, max_tokens=64, pages_per_split=4)
    assert e.value.status == hx.UNSUPPORTED


@pytest.mark.parametrize("hq", [8, 32])
def test_decode_with_infinite_keys_matches_oracle(device, hq):
    """Keys of +-inf in bf16 pages: a page holding one takes fp32 dot
    products, so scores are +-inf (or NaN) exactly as in the oracle; pages
    without one are unaffected."""
    L, H = 1, 8
    rng = np.random.default_rng(61 + hq)
    lengths = [40, 70, 5]
    N = sum((n + 8) // P + 2 for n in lengths) + 4
    cache = hx.PagedKvCache(L, H, D, P, N, page_dtype="bf16")
    pool = oracle.PagedPool(L, H, D, P, N)
    seqs = []
    for i, n in enumerate(lengths):
        s, so = cache.create_sequence(), pool.create_sequence()
        k = rng.standard_normal((L, H, n, D), dtype=np.float32)
        v = rng.standard_normal((L, H, n, D), dtype=np.float32)
        if i == 0:
            k[0, 1, 5, 3] = np.inf      # one +inf dim: score +-inf by the query's sign
            k[0, 2, 20, 7] = -np.inf
        if i == 1:
            k[0, 0, 33, :] = np.inf     # a whole +inf row
            k[0, 5, 64, 0] = np.inf
            k[0, 5, 64, 1] = -np.inf    # inf - inf: NaN score
        cache.append_layer_major(s, [dev(k[0])], [dev(v[0])])
        pool.append_layer_major(so, R(k), R(v))
        seqs.append((s, so))
    B = len(seqs)
    batch = hx.DecodeBatch(cache, [s for s, _ in seqs], hq, max_tokens=200)
    batch.prepare()
    q = rng.standard_normal((B, hq, D), dtype=np.float32)
    tk = rng.standard_normal((B, H, D), dtype=np.float32)
    tv = rng.standard_normal((B, H, D), dtype=np.float32)
    out = torch.empty(B, hq, D, device=device)
    batch.attention_layer(0, dev(q), dev(tk), dev(tv), out)
    torch.cuda.synchronize()
    kp, vp = pool.layer_pages(0)
    hist = np.array([pool.length(so) for _, so in seqs], np.int32)
    tables = np.zeros((B, batch.device_state()["max_blocks"]), np.uint32)
    for b, (_, so) in enumerate(seqs):
        t = pool.block_table(so)
        tables[b, : len(t)] = t
    ref = oracle.batched_decode(q, kp, vp, tables, hist, R(tk), R(tv), threads=8)
    got = host(out)
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    np.testing.assert_allclose(got, ref, atol=ATOL, rtol=RTOL)
    batch.close()
