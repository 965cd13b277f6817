"""GPU paged cache: append, bulk append, gather, fork / copy-on-write and
release must match the CPU oracle bit-exactly (reference tests
tests/cuda_paged_kv_cache_test.cpp and tests/paged_kv_cache_test.cpp)."""

import numpy as np
import pytest
import torch

import helix_runtime_amd as hx
import oracle

pytestmark = pytest.mark.gpu


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda:0")


def host(t):
    return t.detach().cpu().numpy()


def encoded_token(cfg, token):
    # tests/cuda_paged_kv_cache_test.cpp:40-66
    L, H, D = cfg[0], cfg[1], cfg[2]
    k = np.empty((L, H, D), np.float32)
    for l in range(L):
        for h in range(H):
            for c in range(D):
                k[l, h, c] = float(token * 1000 + l * 100 + h * 10 + c)
    return k + np.float32(0.25), -k - np.float32(0.5)


def test_encoded_tokens_land_on_their_pages(device):
    # tests/cuda_paged_kv_cache_test.cpp:77-152
    cfg = (2, 3, 5, 2, 3)
    cache = hx.PagedKvCache(*cfg)
    assert cache.is_healthy()
    seq = cache.create_sequence()
    with cache.read_sequence(seq) as view:
        assert view.length() == 0 and view.physical_blocks() == [] and view.block_table() is None
    for t in range(5):
        k, v = encoded_token(cfg, t)
        cache.append(seq, dev(k), dev(v))
    with cache.read_sequence(seq) as view:
        assert view.length() == 5 and view.physical_blocks() == [0, 1, 2]
    for layer in range(2):
        kp, vp = (host(x) for x in cache.layer_pools(layer))
        for t in range(5):
            for h in range(3):
                for c in range(5):
                    enc = float(t * 1000 + layer * 100 + h * 10 + c)
                    assert kp[t // 2, h, t % 2, c] == np.float32(enc + 0.25)
                    assert vp[t // 2, h, t % 2, c] == np.float32(-enc - 0.5)
    bpt, bb, cap = cache.geometry()
    assert bpt == 2 * 2 * 3 * 5 * 4 and bb == bpt * 2 and cap == 6
    s = cache.stats()
    assert s["bytes_reserved"] == bb * 3 and s["bytes_used"] == s["bytes_reserved"]
    assert (s["bytes_free"], s["total_blocks"], s["used_blocks"], s["free_blocks"]) == (0, 3, 3, 0)
    assert (s["active_tokens"], s["resident_tokens"], s["allocated_token_slots"]) == (5, 5, 6)
    assert (s["block_reference_count"], s["shared_blocks"], s["append_count"]) == (3, 0, 5)
    assert (s["block_allocation_count"], s["block_reuse_count"]) == (3, 0)


def test_exhaustion_is_transactional_and_reuse_is_fifo(device):
    # tests/cuda_paged_kv_cache_test.cpp:154-192
    cfg = (1, 2, 3, 2, 3)
    cache = hx.PagedKvCache(*cfg)
    first, second = cache.create_sequence(), cache.create_sequence()
    for t in range(4):
        cache.append(first, *map(dev, encoded_token(cfg, t)))
    cache.append(second, *map(dev, encoded_token(cfg, 10)))
    cache.append(second, *map(dev, encoded_token(cfg, 11)))
    before = cache.stats()
    rk, rv = map(dev, encoded_token(cfg, 12))
    with pytest.raises(hx.HelixError) as e:
        cache.append(second, rk, rv)
    assert e.value.status == hx.RESOURCE_EXHAUSTED
    assert cache.length(second) == 2 and cache.stats() == before
    cache.release_sequence(first)
    assert not cache.contains(first) and cache.stats()["free_blocks"] == 2
    cache.append(second, rk, rv)
    assert cache.block_table(second) == [2, 0]
    assert cache.stats()["block_reuse_count"] == 1 and cache.stats()["release_count"] == 1


def test_rejects_invalid_handles_shapes_and_aliasing(device):
    # tests/cuda_paged_kv_cache_test.cpp:194-234
    for cfg in [(0, 1, 1, 1, 1), (1, 0, 1, 1, 1), (1, 1, 0, 1, 1), (1, 1, 1, 0, 1), (1, 1, 1, 1, 0)]:
        with pytest.raises(hx.HelixError):
            hx.PagedKvCache(*cfg)
    with pytest.raises(hx.HelixError):
        hx.PagedKvCache(1, 1, 1, 1, 1, device=-1)
    cfg = (1, 1, 2, 1, 1)
    first, second = hx.PagedKvCache(*cfg), hx.PagedKvCache(*cfg)
    seq, foreign = first.create_sequence(), second.create_sequence()
    k, v = map(dev, encoded_token(cfg, 0))
    with pytest.raises(hx.HelixError):
        first.append(foreign, k, v)
    with pytest.raises(hx.HelixError):
        first.append(hx.Sequence(), k, v)
    with pytest.raises(hx.HelixError):
        first.append(seq, torch.zeros(1, 2, device=device), v)
    with pytest.raises(hx.HelixError):
        first.append(seq, torch.zeros(1, 1, 2, dtype=torch.int32, device=device), v)
    # A device pointer inside the pool is rejected before any launch.
    kp, _ = first.layer_pool_pointers(0)
    rc = hx.load().helix_paged_cache_append(first._h, seq, kp, v.data_ptr(), None)
    assert rc == hx.INVALID_ARGUMENT
    first.append(seq, k, v)
    first.release_sequence(seq)
    with pytest.raises(hx.HelixError):
        first.release_sequence(seq)
    with pytest.raises(hx.HelixError):
        first.read_sequence(seq)


def test_poisoned_view_quarantines_the_cache(device):
    # tests/cuda_paged_kv_cache_test.cpp:295-322
    cfg = (1, 1, 2, 2, 1)
    cache = hx.PagedKvCache(*cfg)
    seq = cache.create_sequence()
    k, v = map(dev, encoded_token(cfg, 0))
    cache.append(seq, k, v)
    view = cache.read_sequence(seq)
    assert view.block_table() is not None
    view.poison()
    with pytest.raises(hx.HelixError):
        view.length()
    view.release()
    assert not cache.is_healthy() and cache.contains(seq) and cache.length(seq) == 1
    for call in (cache.create_sequence, lambda: cache.read_sequence(seq),
                 lambda: cache.append(seq, k, v)):
        with pytest.raises(hx.HelixError) as e:
            call()
        assert e.value.status == hx.RUNTIME
    cache.release_sequence(seq)
    assert not cache.contains(seq) and cache.stats()["free_blocks"] == 1


def test_gather_and_prefix_out_match_oracle_bit_exactly(device):
    # tests/paged_kv_cache_test.cpp:60-121 values
    cache = hx.PagedKvCache(2, 2, 2, 2, 4)
    pool = oracle.PagedPool(2, 2, 2, 2, 4)
    seq, so = cache.create_sequence(), pool.create_sequence()
    for t in range(5):
        k = (t * 100.0 + np.arange(8, dtype=np.float32)).reshape(2, 2, 2)
        v = (1000.0 + t * 100 + np.arange(8, dtype=np.float32)).reshape(2, 2, 2)
        cache.append(seq, dev(k), dev(v))
        pool.append(so, k, v)
    gk, gv = cache.retrieve_layer(seq, 1)
    np.testing.assert_array_equal(host(gk).ravel(), [4, 5, 104, 105, 204, 205, 304, 305, 404, 405,
                                                     6, 7, 106, 107, 206, 207, 306, 307, 406, 407])
    ok, ov = pool.copy_layer(so, 1)
    np.testing.assert_array_equal(host(gv), ov)
    pk = torch.full((2, 6, 2), -99.0, device=device)
    pv = torch.full((2, 6, 2), 99.0, device=device)
    cache.copy_layer_prefix_out(seq, 1, 5, pk, pv)
    np.testing.assert_array_equal(host(pk)[:, :5], ok)
    assert (host(pk)[:, 5] == -99.0).all() and (host(pv)[:, 5] == 99.0).all()
    with pytest.raises(hx.HelixError):
        cache.copy_layer_prefix_out(seq, 1, 4, pk, pv)
    with pytest.raises(hx.HelixError):
        cache.copy_layer_out(seq, 1, pk, pk)


@pytest.mark.parametrize("seed", range(4))
def test_random_program_pages_match_oracle_bit_exactly(device, seed):
    """Appends, bulk appends, aligned and copy-on-write forks and releases in
    random order: every live sequence's gather and the raw layer pages equal
    the oracle's, bit for bit."""
    rng = np.random.default_rng(100 + seed)
    L, H, D, P, N = 3, 2, 8 if seed % 2 == 0 else 6, 4, 48
    cache = hx.PagedKvCache(L, H, D, P, N)
    pool = oracle.PagedPool(L, H, D, P, N)
    live = []
    for step in range(120):
        op = rng.integers(0, 5)
        if op == 0 or not live:
            live.append((cache.create_sequence(), pool.create_sequence()))
        elif op in (1, 4):
            s, so = live[rng.integers(len(live))]
            if op == 1:
                k = rng.standard_normal((L, H, D)).astype(np.float32)
                v = rng.standard_normal((L, H, D)).astype(np.float32)
                try:
                    pool.append(so, k, v)
                    ok = True
                except oracle.OracleError:
                    ok = False
                if ok:
                    cache.append(s, dev(k), dev(v))
                else:
                    with pytest.raises(hx.HelixError):
                        cache.append(s, dev(k), dev(v))
            else:
                n = int(rng.integers(1, 3 * P))
                k = rng.standard_normal((L, H, n, D)).astype(np.float32)
                v = rng.standard_normal((L, H, n, D)).astype(np.float32)
                try:
                    pool.append_layer_major(so, k, v)
                    ok = True
                except oracle.OracleError:
                    ok = False
                lk = [dev(k[l]) for l in range(L)]
                lv = [dev(v[l]) for l in range(L)]
                if ok:
                    cache.append_layer_major(s, lk, lv)
                else:
                    with pytest.raises(hx.HelixError):
                        cache.append_layer_major(s, lk, lv)
        elif op == 2:
            s, so = live[rng.integers(len(live))]
            n = cache.length(s)
            if n:
                prefix = int(rng.integers(1, n + 1))
                try:
                    fo = pool.fork_sequence(so, prefix, allow_cow=True)
                except oracle.OracleError:
                    fo = None
                if fo is None:
                    with pytest.raises(hx.HelixError):
                        cache.fork_sequence(s, prefix, allow_cow=True)
                else:
                    live.append((cache.fork_sequence(s, prefix, allow_cow=True), fo))
        else:
            s, so = live.pop(int(rng.integers(len(live))))
            cache.release_sequence(s)
            pool.release_sequence(so)
        assert cache.stats() == pool.stats()
    for s, so in live:
        assert cache.block_table(s) == pool.block_table(so).tolist()
        for layer in range(L):
            gk, gv = cache.retrieve_layer(s, layer)
            ok, ov = pool.copy_layer(so, layer)
            np.testing.assert_array_equal(host(gk), ok)
            np.testing.assert_array_equal(host(gv), ov)
    for layer in range(L):
        kp, vp = (host(x) for x in cache.layer_pools(layer))
        ok, ov = pool.layer_pages(layer)
        for b in range(N):
            n = pool.block_token_count(b)
            if n:
                np.testing.assert_array_equal(kp[b, :, :n], ok[b, :, :n])
                np.testing.assert_array_equal(vp[b, :, :n], ov[b, :, :n])


def test_append_slots_writes_rows_and_skips_negative_slots(device):
    n, h, p, d = 6, 2, 16, 128
    kp = torch.zeros(n, h, p, d, device=device)
    vp = torch.zeros(n, h, p, d, device=device)
    keys = torch.randn(4, h, d, device=device)
    values = torch.randn(4, h, d, device=device)
    slots = torch.tensor([5, -1, 16 * 3 + 15, 0], dtype=torch.int64, device=device)
    hx.append_slots(keys, values, kp, vp, slots)
    torch.cuda.synchronize()
    assert torch.equal(kp[0, :, 5], keys[0]) and torch.equal(vp[3, :, 15], values[2])
    assert torch.equal(kp[0, :, 0], keys[3])
    assert int((kp != 0).any(dim=-1).sum()) == 3 * h
