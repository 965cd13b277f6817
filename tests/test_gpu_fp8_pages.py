"""fp8 E4M3 pages (extension; the reference stores fp32 only,
docs/KV_CACHE.md:531).

Contract, checked here through the C ABI:
- a page element is the OCP E4M3 code of x / scale (key or value scale of
  the cache) rounded to nearest even, saturating at +-448, NaN kept
  (oracle.fp8_bits, pinned in test_oracle.py), bit-exact for the token, bulk,
  slot and fused appends and through copy-on-write forks; gathers return
  decode(code) * scale exactly;
- attention over an fp8 cache equals the fp32 oracle evaluated on those
  values and on the step rows (tail / chunk) rounded the same way, within
  the fp32 tolerance: max-abs 2e-5 plus rel 1e-4.
The oracle pool is fed the rounded values, so its pages are the fp8 pages
decoded."""

import numpy as np
import pytest
import torch

import helix_runtime_amd as hx
import oracle

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-5, 1e-4
D, P = 128, 16
KS, VS = 0.037, 0.011  # scales that are not powers of two: the division rounds


def RK(x):
    return oracle.round_fp8(x, KS)


def RV(x):
    return oracle.round_fp8(x, VS)


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda:0")


def host(t):
    return t.detach().cpu().numpy()


def bits_equal(got, want):
    """Bit-exact on every non-NaN value (signed zeros included), NaN where
    the oracle has NaN: a NaN code widens to a NaN whose payload the
    contract leaves open (its code, sign included, is checked raw)."""
    g, w = np.asarray(got, np.float32), np.asarray(want, np.float32)
    nan = np.isnan(w)
    return (np.array_equal(np.isnan(g), nan)
            and np.array_equal(g[~nan].view(np.uint32), w[~nan].view(np.uint32)))


def byte_free(stats):
    return {k: v for k, v in stats.items() if not k.startswith("bytes") and k != "peak_bytes_used"}


def fp8_cache(L, H, N):
    return hx.PagedKvCache(L, H, D, P, N, page_dtype="fp8", k_scale=KS, v_scale=VS)


def test_every_code_round_trips_through_append_and_gather(device):
    """Scale 1: appending decode(c) stores c for every finite code c, NaN
    stores 0x7f / 0xff, and the gather widens each code to its exact value
    (the device's conversion against the format's definition)."""
    codes = np.arange(256, dtype=np.uint8)
    vals = oracle.fp8_decode(codes)
    vals[0xFF] = -np.nan
    row = vals.reshape(2, D)  # two token rows of 128 codes
    cache = hx.PagedKvCache(1, 1, D, P, 4, page_dtype="fp8")
    assert (cache.k_scale, cache.v_scale) == (1.0, 1.0)
    s = cache.create_sequence()
    k = row[None, None]          # [L, H, 2, D]
    v = row[::-1].copy()[None, None]
    cache.append_layer_major(s, [dev(k[0])], [dev(v[0])])
    kp, vp = cache.layer_pools(0)
    blk = cache.block_table(s)[0]
    raw_k = kp.cpu().numpy()[blk, 0, :2].reshape(-1)
    raw_v = vp.cpu().numpy()[blk, 0, :2].reshape(-1)
    assert np.array_equal(raw_k, codes)
    assert np.array_equal(raw_v, codes.reshape(2, D)[::-1].reshape(-1))
    gk, gv = cache.retrieve_layer(s, 0)
    torch.cuda.synchronize()
    got = host(gk)[0].reshape(-1)
    want = oracle.fp8_decode(codes)
    assert bits_equal(got, want)   # signed zero and subnormals included
    cache.release_sequence(s)


def test_pages_hold_scaled_codes_and_quarter_the_bytes(device):
    L, H, N = 2, 3, 8
    cache = fp8_cache(L, H, N)
    assert (cache.k_scale, cache.v_scale) == (np.float32(KS), np.float32(VS))
    f32 = hx.PagedKvCache(L, H, D, P, N)
    assert cache.stats()["bytes_reserved"] * 4 == f32.stats()["bytes_reserved"]
    f32.close()
    rng = np.random.default_rng(1)
    s = cache.create_sequence()
    k = rng.standard_normal((L, H, 21, D), dtype=np.float32)
    v = rng.standard_normal((L, H, 21, D), dtype=np.float32) * 0.5
    special = np.array([np.nan, -np.nan, np.inf, -np.inf, 0.0, -0.0, 3.4e38, -3.4e38, 1e-40,
                        448 * KS, 464 * KS, 1.0625 * KS, 2.0 ** -10 * KS], np.float32)
    k[0, 0, 3, : special.size] = special
    v[1, 2, 20, : special.size] = special
    cache.append_layer_major(s, [dev(k[l]) for l in range(L)], [dev(v[l]) for l in range(L)])
    tok_k = rng.standard_normal((L, H, D), dtype=np.float32)
    tok_v = rng.standard_normal((L, H, D), dtype=np.float32)
    tok_k[1, 1, :4] = [np.nan, 1e9, -np.inf, 5e-3 * KS]
    cache.append(s, dev(tok_k), dev(tok_v))
    want_k = np.concatenate([k, tok_k[:, :, None]], axis=2)
    want_v = np.concatenate([v, tok_v[:, :, None]], axis=2)
    table = cache.block_table(s)
    for layer in range(L):
        gk, gv = cache.retrieve_layer(s, layer)
        torch.cuda.synchronize()
        assert bits_equal(host(gk), RK(want_k[layer])) and bits_equal(host(gv), RV(want_v[layer]))
        kp, vp = cache.layer_pools(layer)
        raw_k, raw_v = kp.cpu().numpy(), vp.cpu().numpy()
        for t in range(22):
            blk = table[t // P]
            assert np.array_equal(raw_k[blk, :, t % P], oracle.fp8_bits(want_k[layer, :, t], KS))
            assert np.array_equal(raw_v[blk, :, t % P], oracle.fp8_bits(want_v[layer, :, t], VS))
    cache.release_sequence(s)


@pytest.mark.parametrize("seed", [0, 1])
def test_random_program_pages_match_rounded_oracle(device, seed):
    """create / token append / bulk append / aligned and copy-on-write forks /
    release on an fp8 cache against the oracle pool fed rounded rows."""
    L, H, N = 2, 2, 40
    rng = np.random.default_rng(200 + seed)
    cache = fp8_cache(L, H, N)
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
                pool.append(so, RK(k), RV(v))
        elif op == 2:
            s, so = live[rng.integers(len(live))]
            n = int(rng.integers(1, 30))
            if pool.stats()["free_blocks"] * P > n + P:
                k = rng.standard_normal((L, H, n, D), dtype=np.float32)
                v = rng.standard_normal((L, H, n, D), dtype=np.float32)
                cache.append_layer_major(s, [dev(k[l]) for l in range(L)],
                                         [dev(v[l]) for l in range(L)])
                pool.append_layer_major(so, RK(k), RV(v))
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
@pytest.mark.parametrize("hq", [8, 16, 32, 64])
def test_decode_steps_match_oracle_on_rounded_values(device, hq, fused):
    """Query groups 1, 2, 4 and 8 over ragged histories, two steps, with the
    new token appended separately or by the decode launch itself."""
    L, H = 2, 8
    rng = np.random.default_rng(17 + hq)
    lengths = [1, 15, 16, 31, 47, 200, 600]
    N = sum((n + 8) // P + 2 for n in lengths) + 8
    cache = fp8_cache(L, H, N)
    pool = oracle.PagedPool(L, H, D, P, N)
    seqs = []
    for n in lengths:
        s, so = cache.create_sequence(), pool.create_sequence()
        k = rng.standard_normal((L, H, n, D), dtype=np.float32)
        v = rng.standard_normal((L, H, n, D), dtype=np.float32)
        cache.append_layer_major(s, [dev(k[l]) for l in range(L)], [dev(v[l]) for l in range(L)])
        pool.append_layer_major(so, RK(k), RV(v))
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
            ref = oracle.batched_decode(q, kp, vp, tables, hist, RK(keys[layer]),
                                        RV(values[layer]), threads=8)
            np.testing.assert_allclose(host(out), ref, atol=ATOL, rtol=RTOL)
        for b, (_, so) in enumerate(seqs):
            pool.append(so, RK(keys[:, b]), RV(values[:, b]))
    for s, so in seqs:
        for layer in range(L):
            gk, gv = cache.retrieve_layer(s, layer)
            ok, ov = pool.copy_layer(so, layer)
            assert bits_equal(host(gk), ok) and bits_equal(host(gv), ov)
    batch.close()


@pytest.mark.parametrize("hq", [8, 32])
def test_decode_over_many_short_units_matches_oracle(device, hq):
    """1024 sequences of 0-40 tokens (a quarter of them empty, so their
    unit is the tail alone): each stream wavefront runs through several
    one- and two-page units in a row, so the query rows of up to three units
    are in LDS at once (one being attended, two loading) and every area is
    reused many times (about 16 K pages over the 4096 fp8 stream wavefronts
    of a 256-CU GPU: four pages each)."""
    L, H, B = 1, 8, 1024
    rng = np.random.default_rng(29 + hq)
    lengths = rng.integers(0, 41, size=B)
    lengths[rng.random(B) < 0.25] = 0
    N = int(sum((n + P - 1) // P + 1 for n in lengths)) + 8
    cache = fp8_cache(L, H, N)
    pool = oracle.PagedPool(L, H, D, P, N)
    seqs = []
    for n in lengths:
        s, so = cache.create_sequence(), pool.create_sequence()
        if n:
            k = rng.standard_normal((L, H, n, D), dtype=np.float32)
            v = rng.standard_normal((L, H, n, D), dtype=np.float32)
            cache.append_layer_major(s, [dev(k[0])], [dev(v[0])])
            pool.append_layer_major(so, RK(k), RV(v))
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
    ref = oracle.batched_decode(q, kp, vp, tables, hist, RK(keys), RV(values), threads=8)
    np.testing.assert_allclose(host(out), ref, atol=ATOL, rtol=RTOL)
    batch.close()


@pytest.mark.parametrize("hq", [16, 32])
def test_cascade_decode_on_fp8_pages(device, hq):
    """Forks of one prompt share its pages; the decode step attends them once
    (cascade prefix pass with fp8 staging: the fused launch at G 4, the side
    stream at G 8) plus each fork's own pages."""
    L, H = 1, 4
    rng = np.random.default_rng(23 + hq)
    N = 64
    cache = fp8_cache(L, H, N)
    pool = oracle.PagedPool(L, H, D, P, N)
    root, root_o = cache.create_sequence(), pool.create_sequence()
    k = rng.standard_normal((L, H, 6 * P, D), dtype=np.float32)
    v = rng.standard_normal((L, H, 6 * P, D), dtype=np.float32)
    cache.append_layer_major(root, [dev(k[0])], [dev(v[0])])
    pool.append_layer_major(root_o, RK(k), RV(v))
    seqs = []
    for i in range(5):
        s, so = cache.fork_sequence(root, 6 * P), pool.fork_sequence(root_o, 6 * P)
        n = 3 + 7 * i
        ke = rng.standard_normal((L, H, n, D), dtype=np.float32)
        ve = rng.standard_normal((L, H, n, D), dtype=np.float32)
        cache.append_layer_major(s, [dev(ke[0])], [dev(ve[0])])
        pool.append_layer_major(so, RK(ke), RV(ve))
        seqs.append((s, so))
    batch = hx.DecodeBatch(cache, [s for s, _ in seqs], hq, max_tokens=200)
    batch.prepare()
    assert batch.shared_pages() == 6
    q = rng.standard_normal((5, hq, D), dtype=np.float32)
    tk = rng.standard_normal((5, H, D), dtype=np.float32)
    tv = rng.standard_normal((5, H, D), dtype=np.float32)
    out = torch.empty(5, hq, D, device=device)
    batch.append_attention_layer(0, dev(q), dev(tk), dev(tv), out)
    torch.cuda.synchronize()
    kp, vp = pool.layer_pages(0)
    for b, (_, so) in enumerate(seqs):
        tab = np.array(pool.block_table(so), np.uint32)
        want = oracle.paged_attention(q[b][:, None], kp, vp, tab, pool.length(so),
                                      RK(tk[b])[:, None], RV(tv[b])[:, None])[0][:, 0]
        np.testing.assert_allclose(host(out)[b], want, atol=ATOL, rtol=RTOL)
    batch.close()


def test_chunked_prefill_on_fp8_pages(device):
    L, H, HQ = 2, 4, 16
    rng = np.random.default_rng(41)
    hists = [0, 5, 16, 70, 300]
    T = 40
    N = sum((h + T + 1) // P + 2 for h in hists) + 4
    cache = fp8_cache(L, H, N)
    pool = oracle.PagedPool(L, H, D, P, N)
    seqs = []
    for h in hists:
        s, so = cache.create_sequence(), pool.create_sequence()
        if h:
            k = rng.standard_normal((L, H, h, D), dtype=np.float32)
            v = rng.standard_normal((L, H, h, D), dtype=np.float32)
            cache.append_layer_major(s, [dev(k[l]) for l in range(L)], [dev(v[l]) for l in range(L)])
            pool.append_layer_major(so, RK(k), RV(v))
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
            want = oracle.paged_attention(q[b], kp, vp, tab, pool.length(so), RK(ck[layer, b]),
                                          RV(cv[layer, b]))[0]
            np.testing.assert_allclose(host(out)[b], want, atol=ATOL, rtol=RTOL)
    for b, (s, so) in enumerate(seqs):
        pool.append_layer_major(so, RK(ck[:, b]), RV(cv[:, b]))
        for layer in range(L):
            gk, gv = cache.retrieve_layer(s, layer)
            ok, ov = pool.copy_layer(so, layer)
            assert bits_equal(host(gk), ok) and bits_equal(host(gv), ov)
    batch.close()


def test_fp8_validation(device):
    for ks, vs in ((0.0, 1.0), (1.0, -1.0), (float("inf"), 1.0), (1.0, float("nan"))):
        with pytest.raises(hx.HelixError) as e:
            hx.PagedKvCache(1, 1, D, P, 4, page_dtype="fp8", k_scale=ks, v_scale=vs)
        assert e.value.status == hx.INVALID_ARGUMENT
    cache = fp8_cache(1, 2, 8)
    s = cache.create_sequence()
    with pytest.raises(hx.HelixError) as e:  # the split path reads fp32 pages only
        hx.DecodeBatch(cache, [s], 8, max_tokens=64, pages_per_split=4)
    assert e.value.status == hx.UNSUPPORTED
