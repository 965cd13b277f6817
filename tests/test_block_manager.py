"""Host page bookkeeping (product C++ code, via the C ABI) against the
reference's own expectations and, on random operation sequences, against the
oracle pool: block tables, slots, reference counts and every statistic must
match exactly.  No GPU is needed."""

import numpy as np
import pytest

import helix_runtime_amd as hx
import oracle


def test_fifo_tables_and_stats_of_reference_test():
    # tests/paged_kv_cache_test.cpp:60-121 (metadata part)
    m = hx.BlockManager(2, 2, 2, 2, 4)
    assert m.geometry() == (64, 128, 8)
    s = m.create_sequence()
    slots = [m.append(s)[0] for _ in range(5)]
    assert slots == [0, 1, 2, 3, 4]
    assert m.block_table(s) == [0, 1, 2]
    st = m.stats()
    assert (st["bytes_reserved"], st["bytes_used"], st["bytes_free"], st["peak_bytes_used"]) == (512, 384, 128, 384)
    assert (st["used_blocks"], st["free_blocks"], st["active_tokens"], st["allocated_token_slots"]) == (3, 1, 5, 6)
    assert (st["block_allocation_count"], st["block_reuse_count"]) == (3, 0)
    m.validate()


def test_exhaustion_is_transactional():
    m = hx.BlockManager(1, 1, 2, 2, 1)
    a, b = m.create_sequence(), m.create_sequence()
    m.append(a)
    with pytest.raises(hx.HelixError) as e:
        m.append(b)
    assert e.value.status == hx.RESOURCE_EXHAUSTED
    assert m.length(b) == 0 and m.block_table(b) == [] and m.stats()["append_count"] == 1
    m.append(a)
    with pytest.raises(hx.HelixError):
        m.append(a)
    assert m.length(a) == 2
    with pytest.raises(hx.HelixError):
        m.append(b, 3)
    m.release_sequence(a)
    assert m.append(b) == [0] and m.stats()["block_reuse_count"] == 1
    m.validate()


def test_fifo_reuse_order():
    # tests/paged_kv_cache_test.cpp:222-256
    m = hx.BlockManager(1, 1, 1, 1, 3)
    seqs = [m.create_sequence() for _ in range(3)]
    for s in seqs:
        m.append(s)
    m.release_sequence(seqs[1])
    m.release_sequence(seqs[0])
    d, e = m.create_sequence(), m.create_sequence()
    assert m.append(d) == [1] and m.append(e) == [0]
    with pytest.raises(hx.HelixError) as err:
        m.release_sequence(seqs[0])
    assert err.value.status == hx.INVALID_ARGUMENT


def test_handles_of_another_manager_are_rejected():
    a = hx.BlockManager(1, 1, 2, 2, 2)
    b = hx.BlockManager(1, 1, 2, 2, 2)
    sa, sb = a.create_sequence(), b.create_sequence()
    assert sa.id == sb.id and sa.cache_id != sb.cache_id
    assert not a.contains(sb)
    with pytest.raises(hx.HelixError):
        a.append(sb)
    with pytest.raises(hx.HelixError):
        a.release_sequence(hx.Sequence())


@pytest.mark.parametrize("cfg", [(0, 1, 2, 2, 2), (1, 0, 2, 2, 2), (1, 1, 0, 2, 2), (1, 1, 2, 0, 2),
                                 (1, 1, 2, 2, 0), (1, 1, 1, 1, 2**32), (1, 1, 2**62, 2, 1)])
def test_invalid_configurations(cfg):
    # tests/paged_kv_cache_test.cpp:258-272
    with pytest.raises(hx.HelixError):
        hx.BlockManager(*cfg)


def test_fork_stats_match_reference():
    # tests/paged_kv_cache_test.cpp:365-462 (metadata part)
    m = hx.BlockManager(2, 2, 2, 2, 6)
    src = m.create_sequence()
    for _ in range(5):
        m.append(src)
    fork, cow = m.fork_sequence(src, 4)
    assert cow[2] == 0
    assert m.block_table(fork) == m.block_table(src)[:2]
    st = m.stats()
    assert (st["active_sequence_count"], st["active_tokens"], st["resident_tokens"]) == (2, 9, 5)
    assert (st["used_blocks"], st["block_reference_count"], st["shared_blocks"]) == (3, 5, 2)
    assert (st["sequence_create_count"], st["sequence_fork_count"]) == (2, 1)
    m.append(fork)
    m.append(src)
    st = m.stats()
    assert (st["active_tokens"], st["resident_tokens"], st["used_blocks"]) == (11, 7, 4)
    m.release_sequence(src)
    st = m.stats()
    assert (st["block_reference_count"], st["shared_blocks"], st["used_blocks"]) == (3, 0, 3)
    m.validate()
    for prefix in (0, 3, 6):
        with pytest.raises(hx.HelixError):
            m.fork_sequence(fork, prefix)


def test_copy_on_write_fork_plan():
    m = hx.BlockManager(1, 1, 4, 4, 6)
    src = m.create_sequence()
    m.append(src, 10)
    fork, (frm, to, n) = m.fork_sequence(src, 6, allow_cow=True)
    st_tab, f_tab = m.block_table(src), m.block_table(fork)
    assert f_tab[0] == st_tab[0] and (frm, n) == (st_tab[1], 2) and f_tab[1] == to
    assert m.block_info(st_tab[0]) == (2, 4) and m.block_info(to) == (1, 2)
    assert m.length(fork) == 6
    m.append(fork)
    m.validate()


def _run_random_program(seed, steps=400):
    rng = np.random.default_rng(seed)
    L, H, D, P, N = 2, 2, 2, int(rng.integers(1, 6)), int(rng.integers(4, 40))
    m = hx.BlockManager(L, H, D, P, N)
    o = oracle.PagedPool(L, H, D, P, N)
    live = []  # (manager handle, oracle id)
    tok = np.zeros((L, H, D), np.float32)
    for _ in range(steps):
        op = rng.integers(0, 5)
        if op == 0 or not live:
            live.append((m.create_sequence(), o.create_sequence()))
        elif op == 1:
            s, so = live[rng.integers(len(live))]
            n = int(rng.integers(1, 2 * P + 2))
            ok_o = True
            try:
                o.append_layer_major(so, np.zeros((L, H, n, D), np.float32),
                                     np.zeros((L, H, n, D), np.float32))
            except oracle.OracleError:
                ok_o = False
            try:
                m.append(s, n)
                ok_m = True
            except hx.HelixError:
                ok_m = False
            assert ok_m == ok_o
        elif op == 2:
            s, so = live[rng.integers(len(live))]
            ln = m.length(s)
            if ln:
                prefix = int(rng.integers(1, ln + 1))
                cow = bool(rng.integers(0, 2))
                try:
                    fo = o.fork_sequence(so, prefix, cow)
                except oracle.OracleError:
                    fo = None
                try:
                    fm, _ = m.fork_sequence(s, prefix, cow)
                except hx.HelixError:
                    fm = None
                assert (fm is None) == (fo is None)
                if fm is not None:
                    live.append((fm, fo))
        elif op == 3:
            i = int(rng.integers(len(live)))
            s, so = live.pop(i)
            m.release_sequence(s)
            o.release_sequence(so)
        else:
            s, so = live[rng.integers(len(live))]
            try:
                o.append(so, tok, tok)
                ok_o = True
            except oracle.OracleError:
                ok_o = False
            try:
                m.append(s)
                ok_m = True
            except hx.HelixError:
                ok_m = False
            assert ok_m == ok_o
        assert m.stats() == o.stats()
        for s, so in live:
            assert m.block_table(s) == o.block_table(so).tolist()
            assert m.length(s) == o.length(so)
    m.validate()


@pytest.mark.parametrize("seed", range(12))
def test_random_programs_match_oracle(seed):
    _run_random_program(seed)
