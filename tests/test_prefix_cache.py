"""Prefix cache (PagedPrefixCache) on host page bookkeeping, CPU only.

Every scenario of the reference's tests/prefix_cache_test.cpp runs twice:
against the oracle restatement (oracle/prefix_cache.py over the oracle
pool), which pins the oracle to the reference's own expected values, and
against libhelix_paged's trie-based index over the host BlockManager through
the C ABI.  A seeded random program then checks the library against the
oracle operation by operation: statuses, matched lengths, statistics, pool
statistics and the block tables of every sequence a lookup returns."""

import threading

import numpy as np
import pytest

import helix_runtime_amd as hx
import oracle
from oracle.prefix_cache import (ALREADY_PRESENT, INSERTED, REJECTED_TOO_LARGE,
                                 PrefixCacheOracle)


# ------------------------------------------------------------- drivers ----
class CppDriver:
    """libhelix_paged: BlockManager + PagedPrefixCache."""
    error = hx.HelixError

    def pool(self, layers, kv_heads, head_dim, block_tokens, blocks):
        return hx.BlockManager(layers, kv_heads, head_dim, block_tokens, blocks)

    def append(self, pool, seq, n):
        pool.append(seq, n)

    def prefixes(self, pool, entries, blocks):
        return hx.PagedPrefixCache(pool, entries, blocks)

    def insert(self, prefixes, pool, ns, tokens, source):
        return prefixes.insert(ns, tokens, source)

    def code(self, err):
        return err.status


class _OraclePool(oracle.PagedPool):
    def __init__(self, *a):
        super().__init__(*a)
        self.live = set()

    def create_sequence(self):
        s = super().create_sequence()
        self.live.add(s)
        return s

    def fork_sequence(self, source, prefix, allow_cow=False):
        s = super().fork_sequence(source, prefix, allow_cow)
        self.live.add(s)
        return s

    def release_sequence(self, seq):
        super().release_sequence(seq)
        self.live.discard(seq)


class OracleDriver:
    error = oracle.OracleError

    def pool(self, layers, kv_heads, head_dim, block_tokens, blocks):
        return _OraclePool(layers, kv_heads, head_dim, block_tokens, blocks)

    def append(self, pool, seq, n):
        z = np.zeros((pool.layers, pool.kv_heads, pool.head_dim), np.float32)
        for _ in range(n):
            pool.append(seq, z, z)

    def prefixes(self, pool, entries, blocks):
        return PrefixCacheOracle(pool, entries, blocks)

    def insert(self, prefixes, pool, ns, tokens, source):
        if source not in pool.live:  # cache->length(source) throws (prefix.cpp:301)
            raise oracle.OracleError(oracle.INVALID_ARGUMENT, "unknown source")
        return prefixes.insert(ns, tokens, source, pool.length(source))

    def code(self, err):
        return err.code


DRIVERS = [pytest.param(OracleDriver(), id="oracle"), pytest.param(CppDriver(), id="library")]


def code_of(drv, fn):
    with pytest.raises(drv.error) as e:
        fn()
    return drv.code(e.value)


# ------------------------------------- scenarios of prefix_cache_test.cpp ----
@pytest.mark.parametrize("drv", DRIVERS)
def test_longest_aligned_exact_prefix_and_references(drv):
    """prefix_cache_test.cpp:41-114."""
    cache = drv.pool(1, 1, 1, 2, 8)
    source = cache.create_sequence()
    drv.append(cache, source, 6)
    tokens = [10, 11, 12, 13, 14, 15]
    prefixes = drv.prefixes(cache, 4, 8)
    assert drv.insert(prefixes, cache, 7, tokens[:2], source) == INSERTED
    assert drv.insert(prefixes, cache, 7, tokens[:4], source) == INSERTED
    assert prefixes.contains(7, tokens[:2]) and prefixes.contains(7, tokens[:4])
    s = prefixes.stats()
    assert (s["entry_count"], s["retained_tokens"], s["retained_block_references"],
            s["peak_entries"], s["peak_block_references"], s["insertion_count"]) == (2, 6, 3, 2,
                                                                                     3, 2)
    c = cache.stats()
    assert (c["active_sequence_count"], c["active_tokens"], c["resident_tokens"],
            c["block_reference_count"], c["shared_blocks"]) == (3, 12, 6, 6, 2)

    extended = [10, 11, 12, 13, 99]
    seq, matched = prefixes.lookup_longest(7, extended)
    assert matched == 4
    assert list(cache.block_table(seq)) == list(cache.block_table(source))[:2]
    bounded, bmatched = prefixes.lookup_longest(7, extended, 3)
    assert bmatched == 2 and cache.length(bounded) == 2
    assert prefixes.lookup_longest(7, [10, 90, 12, 13, 99]) is None
    assert prefixes.lookup_longest(8, extended) is None
    cache.release_sequence(seq)
    cache.release_sequence(bounded)

    assert drv.insert(prefixes, cache, 7, tokens[:2], source) == ALREADY_PRESENT
    s = prefixes.stats()
    assert (s["entry_count"], s["lookup_count"], s["hit_count"], s["miss_count"],
            s["duplicate_insertion_count"]) == (2, 4, 2, 2, 1)
    prefixes.clear()
    cache.release_sequence(source)
    c = cache.stats()
    assert (c["active_sequence_count"], c["used_blocks"], c["block_reference_count"]) == (0, 0, 0)


@pytest.mark.parametrize("drv", DRIVERS)
def test_exact_keys_separate_content_and_namespaces(drv):
    """prefix_cache_test.cpp:116-164 (payload checks: the GPU test)."""
    cache = drv.pool(1, 1, 1, 2, 6)
    srcs = [cache.create_sequence() for _ in range(3)]
    for s in srcs:
        drv.append(cache, s, 2)
    prefixes = drv.prefixes(cache, 4, 4)
    assert drv.insert(prefixes, cache, 1, [7, 8], srcs[0]) == INSERTED
    assert drv.insert(prefixes, cache, 1, [7, 9], srcs[1]) == INSERTED
    assert drv.insert(prefixes, cache, 2, [7, 8], srcs[2]) == INSERTED
    assert drv.insert(prefixes, cache, 1, [7, 8], srcs[1]) == ALREADY_PRESENT
    got = [prefixes.lookup_longest(1, [7, 8]), prefixes.lookup_longest(1, [7, 9]),
           prefixes.lookup_longest(2, [7, 8])]
    for (seq, _), src in zip(got, srcs):
        assert cache.block_table(seq)[0] == cache.block_table(src)[0]
    assert prefixes.stats()["duplicate_insertion_count"] == 1
    for seq, _ in got:
        cache.release_sequence(seq)
    prefixes.clear()
    for s in srcs:
        cache.release_sequence(s)
    assert cache.stats()["used_blocks"] == 0


@pytest.mark.parametrize("drv", DRIVERS)
def test_block_budget_with_deterministic_lru_eviction(drv):
    """prefix_cache_test.cpp:166-222."""
    cache = drv.pool(1, 1, 1, 2, 8)
    a, b, c = (cache.create_sequence() for _ in range(3))
    drv.append(cache, a, 2)
    drv.append(cache, b, 4)
    drv.append(cache, c, 2)
    k1, k2, k3 = [1, 2], [3, 4, 5, 6], [7, 8]
    prefixes = drv.prefixes(cache, 4, 3)
    assert drv.insert(prefixes, cache, 9, k1, a) == INSERTED
    assert drv.insert(prefixes, cache, 9, k2, b) == INSERTED
    touched, _ = prefixes.lookup_longest(9, k1)
    cache.release_sequence(touched)
    assert drv.insert(prefixes, cache, 9, k3, c) == INSERTED
    assert prefixes.contains(9, k1) and not prefixes.contains(9, k2) and prefixes.contains(9, k3)
    s = prefixes.stats()
    assert (s["entry_count"], s["retained_block_references"], s["peak_block_references"],
            s["eviction_count"]) == (2, 2, 3, 1)
    assert prefixes.evict_lru()
    assert not prefixes.contains(9, k1) and prefixes.contains(9, k3)
    assert prefixes.evict_lru() and not prefixes.evict_lru()
    s = prefixes.stats()
    assert (s["entry_count"], s["retained_tokens"], s["retained_block_references"],
            s["eviction_count"]) == (0, 0, 0, 3)

    bounded = drv.prefixes(cache, 2, 8)
    assert drv.insert(bounded, cache, 9, k1, a) == INSERTED
    assert drv.insert(bounded, cache, 9, k2, b) == INSERTED
    assert drv.insert(bounded, cache, 9, k1, c) == ALREADY_PRESENT
    assert drv.insert(bounded, cache, 9, k3, c) == INSERTED
    assert bounded.contains(9, k1) and not bounded.contains(9, k2) and bounded.contains(9, k3)
    s = bounded.stats()
    assert (s["entry_count"], s["peak_entries"], s["eviction_count"],
            s["duplicate_insertion_count"]) == (2, 2, 1, 1)
    assert not bounded.erase(9, k2)
    assert bounded.erase(9, k1)
    assert bounded.stats()["erase_count"] == 1
    bounded.clear()
    for s_ in (a, b, c):
        cache.release_sequence(s_)
    assert cache.stats()["used_blocks"] == 0


@pytest.mark.parametrize("drv", DRIVERS)
def test_rejects_invalid_keys_sources_and_oversized_entries(drv):
    """prefix_cache_test.cpp:224-277."""
    cache = drv.pool(1, 1, 1, 2, 4)
    assert code_of(drv, lambda: drv.prefixes(cache, 0, 1)) == hx.INVALID_ARGUMENT
    assert code_of(drv, lambda: drv.prefixes(cache, 1, 0)) == hx.INVALID_ARGUMENT
    source = cache.create_sequence()
    drv.append(cache, source, 4)
    tokens = [1, 2, 3, 4, 5, 6]
    prefixes = drv.prefixes(cache, 4, 1)
    assert drv.insert(prefixes, cache, 1, tokens[:4], source) == REJECTED_TOO_LARGE
    assert prefixes.stats()["entry_count"] == 0
    assert prefixes.stats()["rejected_insertion_count"] == 1
    assert cache.stats()["sequence_fork_count"] == 0
    assert cache.stats()["active_sequence_count"] == 1

    invalid = hx.INVALID_ARGUMENT
    assert code_of(drv, lambda: drv.insert(prefixes, cache, 0, tokens[:2], source)) == invalid
    assert code_of(drv, lambda: drv.insert(prefixes, cache, 1, [], source)) == invalid
    assert code_of(drv, lambda: drv.insert(prefixes, cache, 1, tokens[:3], source)) == invalid
    assert code_of(drv, lambda: drv.insert(prefixes, cache, 1, tokens, source)) == hx.OUT_OF_RANGE
    assert code_of(drv, lambda: prefixes.contains(0, tokens[:2])) == invalid
    assert code_of(drv, lambda: prefixes.contains(1, tokens[:3])) == invalid
    assert prefixes.lookup_longest(1, []) is None
    assert prefixes.lookup_longest(1, tokens, 0) is None

    foreign = drv.pool(1, 1, 1, 2, 2)
    fsrc = foreign.create_sequence()
    drv.append(foreign, fsrc, 2)
    if isinstance(drv, CppDriver):  # the oracle pool's handles carry no cache identity
        assert code_of(drv, lambda: drv.insert(prefixes, cache, 1, tokens[:2], fsrc)) == invalid
    cache.release_sequence(source)
    assert code_of(drv, lambda: drv.insert(prefixes, cache, 1, tokens[:2], source)) == invalid
    assert prefixes.stats()["entry_count"] == 0 and prefixes.stats()["insertion_count"] == 0
    assert cache.stats()["active_sequence_count"] == 0
    foreign.release_sequence(fsrc)


@pytest.mark.parametrize("drv", DRIVERS)
def test_anchors_keep_pages_until_last_owner_releases(drv):
    """prefix_cache_test.cpp:279-303 (pages; payload in the GPU test)."""
    cache = drv.pool(1, 1, 1, 2, 2)
    source = cache.create_sequence()
    drv.append(cache, source, 4)
    tokens = [40, 41, 42, 43]
    prefixes = drv.prefixes(cache, 1, 2)
    assert drv.insert(prefixes, cache, 5, tokens, source) == INSERTED
    cache.release_sequence(source)
    assert cache.stats()["active_sequence_count"] == 1 and cache.stats()["free_blocks"] == 0
    match, _ = prefixes.lookup_longest(5, tokens)
    prefixes.clear()
    s = prefixes.stats()
    assert s["entry_count"] == 0 and s["erase_count"] == 1
    assert cache.stats()["active_sequence_count"] == 1 and cache.stats()["free_blocks"] == 0
    cache.release_sequence(match)
    c = cache.stats()
    assert (c["active_sequence_count"], c["used_blocks"], c["free_blocks"]) == (0, 0, 2)


def test_destructor_releases_anchors():
    """prefix_cache_test.cpp:305-321."""
    cache = hx.BlockManager(1, 1, 1, 2, 2)
    source = cache.create_sequence()
    cache.append(source, 4)
    prefixes = hx.PagedPrefixCache(cache, 1, 2)
    assert prefixes.insert(1, [1, 2, 3, 4], source) == INSERTED
    cache.release_sequence(source)
    assert cache.stats()["active_sequence_count"] == 1
    prefixes.close()
    c = cache.stats()
    assert (c["active_sequence_count"], c["used_blocks"], c["block_reference_count"]) == (0, 0, 0)


def test_concurrent_lookup_fork_release():
    """prefix_cache_test.cpp:323-369: 8 threads x 32 lookups; ctypes drops
    the GIL around each call, so the calls do run concurrently."""
    cache = hx.BlockManager(1, 1, 1, 2, 4)
    source = cache.create_sequence()
    cache.append(source, 8)
    tokens = list(range(10, 18))
    prefixes = hx.PagedPrefixCache(cache, 1, 4)
    assert prefixes.insert(1, tokens, source) == INSERTED
    failures = []

    def worker():
        try:
            for _ in range(32):
                hit = prefixes.lookup_longest(1, tokens)
                if hit is None or hit[1] != len(tokens):
                    raise RuntimeError("concurrent prefix lookup unexpectedly missed")
                cache.release_sequence(hit[0])
        except Exception as e:  # noqa: BLE001
            failures.append(e)

    threads = [threading.Thread(target=worker) for _ in range(8)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not failures
    s = prefixes.stats()
    assert (s["lookup_count"], s["hit_count"], s["miss_count"], s["entry_count"]) == (256, 256,
                                                                                     0, 1)
    assert cache.stats()["active_sequence_count"] == 2
    assert cache.stats()["block_reference_count"] == 8
    prefixes.clear()
    cache.release_sequence(source)
    assert cache.stats()["used_blocks"] == 0


def test_constructor_and_accessors():
    cache = hx.BlockManager(1, 1, 1, 4, 8)
    prefixes = hx.PagedPrefixCache(cache, 3, 5)
    assert prefixes.block_tokens() == 4 and prefixes.config() == (3, 5)
    s = prefixes.stats()
    assert s["maximum_entries"] == 3 and s["maximum_block_references"] == 5
    with pytest.raises(hx.HelixError) as e:
        hx.PagedPrefixCache(None, 1, 1)  # prefix_cache_test.cpp:225
    assert e.value.status == hx.INVALID_ARGUMENT
    with pytest.raises(hx.HelixError) as e:
        hx.PagedPrefixCache(cache, 1, (1 << 64) // 2)  # token accounting overflow
    assert e.value.status == hx.OUT_OF_RANGE


# ------------------------------------------------- random program parity ----
@pytest.mark.parametrize("seed", range(10))
def test_random_program_matches_oracle(seed):
    """Random inserts (sources of random lengths over a 3-token alphabet, so
    keys share prefixes), lookups with random bounds, erases, evictions and
    clears; both sides must agree on every result and both pools on every
    statistic and block table."""
    rng = np.random.default_rng(seed)
    page, blocks = int(rng.choice([1, 2, 4])), 64
    entries, budget = int(rng.integers(2, 9)), int(rng.integers(4, 25))
    lib_pool, ora_pool = hx.BlockManager(1, 1, 1, page, blocks), _OraclePool(1, 1, 1, page,
                                                                           blocks)
    lib, ora = hx.PagedPrefixCache(lib_pool, entries, budget), PrefixCacheOracle(ora_pool,
                                                                                entries, budget)
    drv = OracleDriver()
    sources = []  # (lib seq, oracle seq, tokens)
    held = []     # lookups still held: (lib seq, oracle seq)
    for step in range(300):
        op = rng.integers(0, 10)
        if op <= 2 or not sources:
            if len(sources) < 6 and lib_pool.stats()["free_blocks"] >= 8:
                n = int(rng.integers(1, 8)) * page
                toks = [int(t) for t in rng.integers(0, 3, n)]
                ls, os_ = lib_pool.create_sequence(), ora_pool.create_sequence()
                lib_pool.append(ls, n)
                drv.append(ora_pool, os_, n)
                sources.append((ls, os_, toks))
        elif op <= 4:
            ls, os_, toks = sources[rng.integers(len(sources))]
            n = int(rng.integers(1, len(toks) // page + 1)) * page
            ns = int(rng.integers(1, 3))
            assert lib.insert(ns, toks[:n], ls) == ora.insert(ns, toks[:n], os_, len(toks))
        elif op <= 7:
            ls, os_, toks = sources[rng.integers(len(sources))]
            q = toks + [int(t) for t in rng.integers(0, 3, int(rng.integers(0, 4)))]
            bound = None if rng.random() < 0.5 else int(rng.integers(0, len(q) + 1))
            ns = int(rng.integers(1, 3))
            a, b = lib.lookup_longest(ns, q, bound), ora.lookup_longest(ns, q, bound)
            assert (a is None) == (b is None), f"step {step}"
            if a is not None:
                assert a[1] == b[1]
                assert list(lib_pool.block_table(a[0])) == list(ora_pool.block_table(b[0]))
                held.append((a[0], b[0]))
        elif op == 8:
            ls, os_, toks = sources[rng.integers(len(sources))]
            n = int(rng.integers(1, len(toks) // page + 1)) * page
            ns = int(rng.integers(1, 3))
            if rng.random() < 0.5:
                assert lib.erase(ns, toks[:n]) == ora.erase(ns, toks[:n])
            else:
                assert lib.contains(ns, toks[:n]) == ora.contains(ns, toks[:n])
        else:
            r = rng.random()
            if r < 0.6:
                assert lib.evict_lru() == ora.evict_lru()
            elif r < 0.7:
                lib.clear()
                ora.clear()
            elif held:
                a, b = held.pop(int(rng.integers(len(held))))
                lib_pool.release_sequence(a)
                ora_pool.release_sequence(b)
            elif sources:
                ls, os_, _ = sources.pop(int(rng.integers(len(sources))))
                lib_pool.release_sequence(ls)
                ora_pool.release_sequence(os_)
        assert lib.stats() == ora.stats(), f"step {step}"
        assert lib_pool.stats() == ora_pool.stats(), f"step {step}"
    lib_pool.validate()
