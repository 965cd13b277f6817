"""Pins the CPU oracle before it is trusted as the checker.

Every oracle function is checked against something it does not itself
compute: the golden arrays and exact statistics written inline in the
reference's own tests, closed forms, a textbook float64 attention written
independently here with numpy, invariants (paged == contiguous, GQA ==
replicated MHA, batch == per-sequence loop) and the C++ standard's known
answer for mt19937_64.  Citations are to the reference's test files.
"""

import math

import numpy as np
import pytest

import oracle
from oracle import PagedPool


def make_token(layers, heads, dim, base):
    # tests/paged_kv_cache_test.cpp:19-28
    return (base + np.arange(layers * heads * dim, dtype=np.float32)).reshape(layers, heads, dim)


def make_layer_major(layers, heads, token_begin, count, dim, base):
    # tests/paged_kv_cache_test.cpp:30-51, stacked to [L, H, T, D]
    out = np.empty((layers, heads, count, dim), dtype=np.float32)
    for l in range(layers):
        for h in range(heads):
            for t in range(count):
                for c in range(dim):
                    out[l, h, t, c] = base + float((token_begin + t) * 100 + (l * heads + h) * dim + c)
    return out


def textbook_attention(q, k, v, offset):
    """float64 softmax(QK^T/sqrt(D) + causal mask) V, per head (numpy only)."""
    q = q.astype(np.float64)
    k = k.astype(np.float64)
    v = v.astype(np.float64)
    h, nq, d = q.shape
    nk = k.shape[1]
    s = np.einsum("hqd,hkd->hqk", q, k) / math.sqrt(d)
    mask = np.arange(nk)[None, :] > (offset + np.arange(nq))[:, None]
    s = np.where(mask[None], -np.inf, s)
    s = s - s.max(axis=-1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(axis=-1, keepdims=True)
    return np.einsum("hqk,hkd->hqd", p, v), p


# ------------------------------------------------------------------ RNG ----
def test_mt19937_64_known_answer():
    # C++ standard [rand.predef]: the 10000th invocation of a default
    # constructed mt19937_64 (seed 5489) produces 9981545732273789042.
    assert oracle.mt19937_64_nth(5489, 10000) == 9981545732273789042


def test_random_uniform_formula_and_range():
    # src/tensor/tensor.cpp:169-189: values are lower + range * (k / 2^24).
    x = oracle.random_uniform((4096,), 8101, -1.0, 1.0)
    assert x.min() >= -1.0 and x.max() < 1.0
    k = (x.astype(np.float64) + 1.0) / 2.0 * 16777216.0
    assert np.allclose(k, np.round(k), atol=1e-3 * 2)  # on the 2^-24 lattice (float rounding)
    y = oracle.random_uniform((4096,), 8101, -1.0, 1.0)
    assert np.array_equal(x, y)
    assert not np.array_equal(x, oracle.random_uniform((4096,), 8102, -1.0, 1.0))


def test_random_normal_moments():
    x = oracle.random_normal((1 << 20,), 1234).astype(np.float64)
    assert abs(x.mean()) < 5e-3
    assert abs(x.var() - 1.0) < 5e-3
    assert abs((x > 1.0).mean() - 0.158655) < 2e-3


# ----------------------------------------------------------- pool golden ----
def test_maps_logical_history_across_block_boundaries():
    # tests/paged_kv_cache_test.cpp:60-121
    pool = PagedPool(2, 2, 2, 2, 4)
    assert pool.bytes_per_token() == 64
    assert pool.block_bytes() == 128
    seq = pool.create_sequence()
    for t in range(5):
        pool.append(seq, make_token(2, 2, 2, t * 100.0), make_token(2, 2, 2, 1000.0 + t * 100))
    assert pool.block_table(seq).tolist() == [0, 1, 2]
    k, v = pool.copy_layer(seq, 1)
    assert k.shape == (2, 5, 2)
    np.testing.assert_array_equal(k.ravel(), [4, 5, 104, 105, 204, 205, 304, 305, 404, 405,
                                              6, 7, 106, 107, 206, 207, 306, 307, 406, 407])
    np.testing.assert_array_equal(v.ravel(), [1004, 1005, 1104, 1105, 1204, 1205, 1304, 1305,
                                              1404, 1405, 1006, 1007, 1106, 1107, 1206, 1207,
                                              1306, 1307, 1406, 1407])
    pk, pv = pool.copy_layer(seq, 1, dest_tokens=6, fill=-99.0)
    np.testing.assert_array_equal(pk[:, :5], k)
    np.testing.assert_array_equal(pv[:, :5], v)
    assert (pk[:, 5] == -99.0).all()
    s = pool.stats()
    assert s["bytes_reserved"] == 512 and s["bytes_used"] == 384 and s["bytes_free"] == 128
    assert s["peak_bytes_used"] == 384 and s["total_blocks"] == 4 and s["used_blocks"] == 3
    assert s["free_blocks"] == 1 and s["active_sequence_count"] == 1 and s["active_tokens"] == 5
    assert s["allocated_token_slots"] == 6 and s["allocated_token_slots"] - s["resident_tokens"] == 1
    assert s["block_allocation_count"] == 3 and s["block_reuse_count"] == 0


def test_exhaustion_is_transactional_and_partial_blocks_writable():
    # tests/paged_kv_cache_test.cpp:144-175
    pool = PagedPool(1, 1, 2, 2, 1)
    first, second = pool.create_sequence(), pool.create_sequence()
    tok = np.array([[[1.0, 2.0]]], dtype=np.float32)
    pool.append(first, tok, tok)
    with pytest.raises(oracle.OracleError) as e:
        pool.append(second, tok, tok)
    assert e.value.code == oracle.RESOURCE_EXHAUSTED
    assert pool.length(second) == 0 and pool.block_table(second).size == 0
    assert pool.stats()["append_count"] == 1
    pool.append(first, tok, tok)
    assert pool.length(first) == 2
    with pytest.raises(oracle.OracleError):
        pool.append(first, tok, tok)
    assert pool.length(first) == 2 and pool.stats()["active_tokens"] == 2
    pool.release_sequence(first)
    rep = np.array([[[9.0, 8.0]]], dtype=np.float32)
    pool.append(second, rep, rep)
    assert pool.block_table(second).tolist() == [0]
    assert pool.stats()["block_reuse_count"] == 1
    np.testing.assert_array_equal(pool.copy_layer(second, 0)[0].ravel(), [9.0, 8.0])


def test_bulk_layer_major_matches_scalar_appends():
    # tests/paged_kv_cache_test.cpp:177-220
    bulk, scalar = PagedPool(2, 2, 2, 2, 3), PagedPool(2, 2, 2, 2, 3)
    bs, ss = bulk.create_sequence(), scalar.create_sequence()
    bulk.append(bs, make_token(2, 2, 2, 0.0), make_token(2, 2, 2, 1000.0))
    bulk.append_layer_major(bs, make_layer_major(2, 2, 1, 4, 2, 0.0),
                            make_layer_major(2, 2, 1, 4, 2, 1000.0))
    for t in range(5):
        scalar.append(ss, make_token(2, 2, 2, t * 100.0), make_token(2, 2, 2, 1000.0 + t * 100))
    for layer in range(2):
        for a, b in zip(bulk.copy_layer(bs, layer), scalar.copy_layer(ss, layer)):
            np.testing.assert_array_equal(a, b)
    assert bulk.length(bs) == 5
    assert bulk.stats()["append_count"] == 5 and bulk.stats()["block_allocation_count"] == 3
    ex = PagedPool(2, 2, 2, 2, 2)
    es = ex.create_sequence()
    with pytest.raises(oracle.OracleError):
        ex.append_layer_major(es, make_layer_major(2, 2, 0, 5, 2, 0.0),
                              make_layer_major(2, 2, 0, 5, 2, 1000.0))
    assert ex.length(es) == 0 and ex.block_table(es).size == 0 and ex.stats()["append_count"] == 0


def test_free_pool_is_deterministic_fifo():
    # tests/paged_kv_cache_test.cpp:222-256
    pool = PagedPool(1, 1, 1, 1, 3)
    tok = np.ones((1, 1, 1), dtype=np.float32)
    a, b, c = (pool.create_sequence() for _ in range(3))
    for s in (a, b, c):
        pool.append(s, tok, tok)
    assert [pool.block_table(s)[0] for s in (a, b, c)] == [0, 1, 2]
    pool.release_sequence(b)
    pool.release_sequence(a)
    d, e = pool.create_sequence(), pool.create_sequence()
    pool.append(d, tok, tok)
    pool.append(e, tok, tok)
    assert pool.block_table(d)[0] == 1 and pool.block_table(e)[0] == 0
    assert pool.stats()["block_reuse_count"] == 2
    for s in (c, d, e):
        pool.release_sequence(s)
    st = pool.stats()
    assert st["bytes_used"] == 0 and st["bytes_free"] == st["bytes_reserved"]
    assert st["used_blocks"] == 0 and st["free_blocks"] == 3 and st["allocated_token_slots"] == 0
    with pytest.raises(oracle.OracleError):
        pool.release_sequence(a)


def test_interleaved_appends_account_exactly():
    # tests/paged_kv_cache_test.cpp:331-363 (threads replaced by a round robin)
    pool = PagedPool(1, 1, 2, 7, 16)
    seqs = [pool.create_sequence() for _ in range(4)]
    tok = np.array([[[3.0, 4.0]]], dtype=np.float32)
    for _ in range(25):
        for s in seqs:
            pool.append(s, tok, tok)
    st = pool.stats()
    assert st["active_tokens"] == 100 and st["used_blocks"] == 16
    assert st["allocated_token_slots"] - st["resident_tokens"] == 12
    for s in seqs:
        assert pool.length(s) == 25 and pool.block_table(s).size == 4
        pool.release_sequence(s)
    st = pool.stats()
    assert st["free_blocks"] == 16 and st["active_sequence_count"] == 0 and st["active_tokens"] == 0


def test_tail_slack_bound():
    # tests/paged_kv_cache_test.cpp:304-329 (paged side)
    pool = PagedPool(1, 1, 1, 4, 3)
    a, b = pool.create_sequence(), pool.create_sequence()
    tok = np.full((1, 1, 1), 2.0, dtype=np.float32)
    pool.append(a, tok, tok)
    for _ in range(5):
        pool.append(b, tok, tok)
    st = pool.stats()
    assert st["allocated_token_slots"] == 12
    assert st["allocated_token_slots"] - st["resident_tokens"] == 6
    assert st["bytes_used"] == 96


def test_block_aligned_fork_shares_prefix_and_diverges():
    # tests/paged_kv_cache_test.cpp:365-462
    pool = PagedPool(2, 2, 2, 2, 6)
    src = pool.create_sequence()
    for t in range(5):
        pool.append(src, make_token(2, 2, 2, t * 100.0), make_token(2, 2, 2, 1000.0 + t * 100))
    fork = pool.fork_sequence(src, 4)
    st_, ft = pool.block_table(src), pool.block_table(fork)
    assert st_.size == 3 and ft.size == 2 and (ft == st_[:2]).all()
    sk, sv = pool.copy_layer(src, 1)
    fk, fv = pool.copy_layer(fork, 1)
    np.testing.assert_array_equal(sk[:, :4], fk)
    np.testing.assert_array_equal(sv[:, :4], fv)
    s = pool.stats()
    assert (s["active_sequence_count"], s["active_tokens"], s["resident_tokens"]) == (2, 9, 5)
    assert s["active_tokens"] - s["resident_tokens"] == 4
    assert (s["used_blocks"], s["block_reference_count"], s["shared_blocks"]) == (3, 5, 2)
    assert (s["sequence_create_count"], s["sequence_fork_count"]) == (2, 1)
    assert s["block_allocation_count"] == 3
    assert s["allocated_token_slots"] - s["resident_tokens"] == 1
    pool.append_layer_major(fork, make_layer_major(2, 2, 4, 1, 2, 9000.0),
                            make_layer_major(2, 2, 4, 1, 2, 19000.0))
    pool.append(src, make_token(2, 2, 2, 8000.0), make_token(2, 2, 2, 18000.0))
    ds, df = pool.block_table(src), pool.block_table(fork)
    assert ds[0] == df[0] and ds[1] == df[1] and ds[2] != df[2]
    dk, dv = pool.copy_layer(src, 1)
    assert dk.ravel()[10] == 8004.0 and dv.ravel()[10] == 18004.0
    gk, gv = pool.copy_layer(fork, 1)
    assert gk.ravel()[8] == 9404.0 and gv.ravel()[8] == 19404.0
    s = pool.stats()
    assert (s["active_tokens"], s["resident_tokens"], s["used_blocks"]) == (11, 7, 4)
    assert (s["block_reference_count"], s["shared_blocks"]) == (6, 2)
    pool.release_sequence(src)
    assert pool.length(fork) == 5
    np.testing.assert_array_equal(pool.copy_layer(fork, 1)[0][:, :4], fk)
    s = pool.stats()
    assert (s["active_tokens"], s["resident_tokens"], s["used_blocks"]) == (5, 5, 3)
    assert (s["block_reference_count"], s["shared_blocks"]) == (3, 0)
    pool.release_sequence(fork)
    s = pool.stats()
    assert (s["active_sequence_count"], s["active_tokens"], s["resident_tokens"]) == (0, 0, 0)
    assert (s["used_blocks"], s["free_blocks"], s["block_reference_count"]) == (0, 6, 0)


def test_fork_validation_and_exhaustion():
    # tests/paged_kv_cache_test.cpp:464-513
    pool = PagedPool(1, 1, 2, 2, 3)
    src = pool.create_sequence()
    tok = np.array([[[1.0, 2.0]]], dtype=np.float32)
    for _ in range(5):
        pool.append(src, tok, tok)
    before = pool.stats()
    for prefix in (0, 3, 6):
        with pytest.raises(oracle.OracleError):
            pool.fork_sequence(src, prefix)
    assert pool.stats() == before
    fork = pool.fork_sequence(src, 4)
    assert pool.stats()["free_blocks"] == 0
    with pytest.raises(oracle.OracleError):
        pool.append(fork, tok, tok)
    assert pool.length(fork) == 4 and pool.block_table(fork).size == 2
    assert pool.stats()["append_count"] == 5
    pool.release_sequence(src)
    s = pool.stats()
    assert (s["free_blocks"], s["used_blocks"], s["active_tokens"], s["resident_tokens"]) == (1, 2, 4, 4)
    pool.append(fork, np.array([[[9.0, 8.0]]], np.float32), np.array([[[7.0, 6.0]]], np.float32))
    assert pool.block_table(fork)[-1] == 2 and pool.stats()["block_reuse_count"] == 1
    with pytest.raises(oracle.OracleError):
        pool.fork_sequence(src, 2)
    pool.release_sequence(fork)
    s = pool.stats()
    assert (s["used_blocks"], s["free_blocks"], s["active_tokens"], s["resident_tokens"]) == (0, 3, 0, 0)


def test_prefix_fork_fanout_stats():
    # tests/paged_kv_cache_test.cpp:515-602 (threads replaced by sequential order)
    pool = PagedPool(1, 1, 2, 4, 6)
    src = pool.create_sequence()
    pool.append_layer_major(src, make_layer_major(1, 1, 0, 8, 2, 10.0),
                            make_layer_major(1, 1, 0, 8, 2, 1000.0))
    forks = []
    for t in range(4):
        f = pool.fork_sequence(src, 8)
        tail = make_token(1, 1, 2, 10000.0 + t * 100)
        pool.append(f, tail, tail)
        forks.append(f)
    sk, _ = pool.copy_layer(src, 0)
    for t, f in enumerate(forks):
        fk, _ = pool.copy_layer(f, 0)
        assert fk.shape == (1, 9, 2)
        np.testing.assert_array_equal(fk.ravel()[:16], sk.ravel())
        assert fk.ravel()[16] == 10000 + t * 100 and fk.ravel()[17] == 10001 + t * 100
    s = pool.stats()
    assert (s["active_sequence_count"], s["active_tokens"], s["resident_tokens"]) == (5, 44, 12)
    assert s["active_tokens"] - s["resident_tokens"] == 32
    assert (s["used_blocks"], s["free_blocks"], s["block_reference_count"]) == (6, 0, 14)
    assert (s["shared_blocks"], s["sequence_fork_count"]) == (2, 4)
    for f in forks:
        pool.release_sequence(f)
    s = pool.stats()
    assert (s["active_sequence_count"], s["active_tokens"], s["resident_tokens"]) == (1, 8, 8)
    assert (s["used_blocks"], s["free_blocks"], s["block_reference_count"], s["shared_blocks"]) == (2, 4, 2, 0)
    pool.release_sequence(src)
    s = pool.stats()
    assert (s["active_sequence_count"], s["used_blocks"], s["free_blocks"], s["block_reference_count"]) == (0, 0, 6, 0)


def test_layer_view_spans():
    # tests/paged_kv_cache_test.cpp:604-636: key_block(lb, head) is the valid
    # prefix of page lb in the per-layer page layout.
    pool = PagedPool(2, 2, 2, 2, 2)
    seq = pool.create_sequence()
    for t in range(3):
        pool.append(seq, make_token(2, 2, 2, t * 100.0), make_token(2, 2, 2, 1000.0 + t * 100))
    table = pool.block_table(seq)
    assert table.tolist() == [0, 1]
    kp, vp = pool.layer_pages(1)
    assert kp[table[0], 0].ravel().tolist() == [4.0, 5.0, 104.0, 105.0]
    assert kp[table[1], 0, :1].ravel().tolist() == [204.0, 205.0]
    assert vp[table[1], 1, :1].ravel().tolist() == [1206.0, 1207.0]
    assert pool.block_token_count(int(table[1])) == 1


def test_cow_fork_extension_invariants():
    # No reference counterpart (docs/KV_CACHE.md:247): pinned by invariants --
    # shared pages untouched, the new page's prefix equals the source page's
    # prefix, the logical gather of the fork equals the source prefix.
    pool = PagedPool(2, 2, 3, 4, 8)
    src = pool.create_sequence()
    data_k = oracle.random_uniform((2, 2, 10, 3), 5)
    data_v = oracle.random_uniform((2, 2, 10, 3), 6)
    pool.append_layer_major(src, data_k, data_v)
    before_pages = pool.layer_pages(0)
    with pytest.raises(oracle.OracleError):
        pool.fork_sequence(src, 6)
    fork = pool.fork_sequence(src, 6, allow_cow=True)
    st, ft = pool.block_table(src), pool.block_table(fork)
    assert ft[0] == st[0] and ft[1] != st[1]
    assert pool.block_refcount(int(st[0])) == 2 and pool.block_refcount(int(ft[1])) == 1
    after_pages = pool.layer_pages(0)
    for b in st:
        np.testing.assert_array_equal(after_pages[0][b], before_pages[0][b])
    for layer in range(2):
        sk, sv = pool.copy_layer(src, layer)
        fk, fv = pool.copy_layer(fork, layer)
        np.testing.assert_array_equal(fk, sk[:, :6])
        np.testing.assert_array_equal(fv, sv[:, :6])
    tok = np.full((2, 2, 3), 7.0, np.float32)
    pool.append(fork, tok, tok)
    np.testing.assert_array_equal(pool.copy_layer(src, 0)[0], data_k[0])
    assert pool.copy_layer(fork, 0)[0][0, 6].tolist() == [7.0, 7.0, 7.0]


# ----------------------------------------------------------- attention -----
def test_known_causal_attention_closed_form():
    # tests/attention_test.cpp:22-48
    q = np.array([[[1, 0], [0, 1]]], np.float32)
    v = np.array([[[10, 0], [0, 20]]], np.float32)
    out, ws = oracle.sdpa(q, q, v, 0)
    e = math.exp(1.0 / math.sqrt(2.0))
    p1, p2 = 1.0 / (1.0 + e), e / (1.0 + e)
    np.testing.assert_allclose(ws.ravel(), [1, 0, p1, p2], atol=1e-5)
    np.testing.assert_allclose(out.ravel(), [10, 0, 10 * p1, 20 * p2], atol=1e-5)


def test_query_offset_decode_closed_form():
    # tests/attention_test.cpp:50-63
    q = np.array([[[1.0]]], np.float32)
    k = np.array([[[0.0], [1.0], [2.0]]], np.float32)
    v = np.array([[[1, 2], [10, 20], [100, 200]]], np.float32)
    out, _ = oracle.sdpa(q, k, v, 2)
    den = 1 + math.exp(1) + math.exp(2)
    np.testing.assert_allclose(out.ravel(), [(1 + 10 * math.exp(1) + 100 * math.exp(2)) / den,
                                             (2 + 20 * math.exp(1) + 200 * math.exp(2)) / den],
                               atol=2e-5)


def test_softmax_special_cases():
    # src/kernels/cpu/reference.cpp:264-316 semantics
    inf, nan = np.inf, np.nan
    x = np.array([[0.0, nan, 1.0], [-inf, -inf, -inf], [inf, 1.0, inf], [0.0, 0.0, -inf]],
                 np.float32)
    y = oracle.softmax_rows(x)
    assert np.isnan(y[0]).all() and np.isnan(y[1]).all()
    assert y[2].tolist() == [0.5, 0.0, 0.5]
    assert y[3].tolist() == [0.5, 0.5, 0.0]


def test_causal_mask_does_not_read_future_nan():
    # tests/attention_test.cpp:65-79 and tests/paged_attention_test.cpp:186-220
    nan = np.nan
    out, ws = oracle.sdpa(np.array([[[1.0]]], np.float32), np.array([[[0.0], [nan]]], np.float32),
                          np.array([[[3, 4], [nan, nan]]], np.float32), 0)
    assert out.ravel().tolist() == [3.0, 4.0] and ws.ravel().tolist() == [1.0, 0.0]
    empty = np.zeros((1, 1, 2, 1), np.float32)
    out, ws = oracle.paged_attention(np.zeros((1, 2, 1), np.float32), empty, empty,
                                     np.zeros(0, np.uint32), 0,
                                     np.array([[[0.0], [nan]]], np.float32),
                                     np.array([[[3.0], [nan]]], np.float32))
    assert out.ravel()[0] == 3.0 and np.isnan(out.ravel()[1])
    assert ws.ravel()[0] == 1.0 and ws.ravel()[1] == 0.0
    # history-only: a NaN value after the visible prefix is not read
    pool = PagedPool(1, 1, 1, 1, 2)
    s = pool.create_sequence()
    pool.append(s, np.zeros((1, 1, 1), np.float32), np.full((1, 1, 1), 3.0, np.float32))
    pool.append(s, np.zeros((1, 1, 1), np.float32), np.full((1, 1, 1), nan, np.float32))
    kp, vp = pool.layer_pages(0)
    out, _ = oracle.paged_attention(np.zeros((1, 1, 1), np.float32), kp, vp,
                                    pool.block_table(s), 2, query_position_offset=0)
    assert out.ravel()[0] == 3.0


def test_paged_matches_contiguous_across_block_boundaries():
    # tests/paged_attention_test.cpp:44-78
    pool = PagedPool(1, 1, 2, 2, 2)
    s = pool.create_sequence()
    for k, v in (([1, 0], [10, 1]), ([0, 1], [20, 2]), ([1, 1], [30, 3])):
        pool.append(s, np.array([[k]], np.float32), np.array([[v]], np.float32))
    ck, cv = pool.copy_layer(s, 0)
    q = np.array([[[1, 0], [0, 1], [1, 1]]], np.float32)
    exp_out, exp_ws = oracle.sdpa(q, ck, cv, 0)
    kp, vp = pool.layer_pages(0)
    out, ws = oracle.paged_attention(q, kp, vp, pool.block_table(s), 3, query_position_offset=0)
    assert ws.nbytes == 36
    np.testing.assert_allclose(out, exp_out, atol=1e-5)
    np.testing.assert_allclose(ws, exp_ws, atol=1e-5)
    tb, tp = textbook_attention(q, ck, cv, 0)
    np.testing.assert_allclose(out, tb, atol=1e-5)
    np.testing.assert_allclose(ws, tp, atol=1e-6)


def test_odd_multihead_chunked_history():
    # tests/paged_attention_test.cpp:80-103 (seeds 91000+t, 92000+t, 93000)
    pool = PagedPool(2, 3, 5, 4, 3)
    s = pool.create_sequence()
    for t in range(9):
        pool.append(s, oracle.random_uniform((2, 3, 5), 91000 + t),
                    oracle.random_uniform((2, 3, 5), 92000 + t))
    ck, cv = pool.copy_layer(s, 1)
    q = oracle.random_uniform((3, 3, 5), 93000)
    expected, _ = oracle.sdpa(q, ck, cv, 6)
    kp, vp = pool.layer_pages(1)
    out, _ = oracle.paged_attention(q, kp, vp, pool.block_table(s), 9, query_position_offset=6)
    np.testing.assert_allclose(out, expected, atol=2e-5)
    np.testing.assert_allclose(out, textbook_attention(q, ck, cv, 6)[0], atol=2e-5)


def test_tail_continuation_matches_compacted_history():
    # tests/paged_attention_test.cpp:105-144 (seeds 94000.., 95000.., 96000-96002)
    pool = PagedPool(1, 2, 3, 2, 2)
    s = pool.create_sequence()
    for t in range(3):
        pool.append(s, oracle.random_uniform((1, 2, 3), 94000 + t),
                    oracle.random_uniform((1, 2, 3), 95000 + t))
    q = oracle.random_uniform((2, 2, 3), 96000)
    tk = oracle.random_uniform((2, 2, 3), 96001)
    tv = oracle.random_uniform((2, 2, 3), 96002)
    ck, cv = pool.copy_layer(s, 0)
    exp_out, exp_ws = oracle.sdpa(q, np.concatenate([ck, tk], 1), np.concatenate([cv, tv], 1), 3)
    kp, vp = pool.layer_pages(0)
    out, ws = oracle.paged_attention(q, kp, vp, pool.block_table(s), 3, tk, tv)
    assert ws.nbytes == 80
    np.testing.assert_allclose(out, exp_out, atol=2e-5)
    np.testing.assert_allclose(ws, exp_ws, atol=2e-5)
    tb, tp = textbook_attention(q, np.concatenate([ck, tk], 1), np.concatenate([cv, tv], 1), 3)
    np.testing.assert_allclose(out, tb, atol=2e-5)


def test_tail_with_empty_history():
    # tests/paged_attention_test.cpp:146-156 (seeds 97000-97002)
    q = oracle.random_uniform((2, 1, 3), 97000)
    tk = oracle.random_uniform((2, 1, 3), 97001)
    tv = oracle.random_uniform((2, 1, 3), 97002)
    empty = np.zeros((1, 2, 2, 3), np.float32)
    out, _ = oracle.paged_attention(q, empty, empty, np.zeros(0, np.uint32), 0, tk, tv)
    np.testing.assert_allclose(out, oracle.sdpa(q, tk, tv, 0)[0], atol=1e-5)
    np.testing.assert_allclose(out, tv, atol=1e-6)  # one visible key: output == its value


def test_known_reordered_blocks_with_poisoned_padding():
    # tests/cuda_attention_test.cpp:196-228: table {2, 0}, padding +-10000
    table = np.array([2, 0], np.uint32)
    q = np.array([[[1, 0], [0, 1]]], np.float32)
    k = np.array([[[1, 0], [0, 1], [1, 1]]], np.float32)
    v = np.array([[[10, 1, -1], [20, 2, -2], [30, 3, -3]]], np.float32)
    kp = oracle.pack_logical_blocks(k, table, 3, 2, 10000.0)
    vp = oracle.pack_logical_blocks(v, table, 3, 2, -10000.0)
    out, ws = oracle.paged_attention(q, kp, vp, table, 3, query_position_offset=1)
    exp_out, exp_ws = oracle.sdpa(q, k, v, 1)
    np.testing.assert_allclose(out, exp_out, atol=2e-5)
    np.testing.assert_allclose(ws, exp_ws, atol=2e-6)
    tb, tp = textbook_attention(q, k, v, 1)
    np.testing.assert_allclose(out, tb, atol=2e-5)
    np.testing.assert_allclose(ws, tp, atol=2e-6)


@pytest.mark.parametrize("h,nq,nk,d,dv,p", [(1, 1, 3, 1, 2, 2), (2, 3, 5, 5, 7, 2),
                                             (3, 7, 11, 37, 41, 4)])
def test_odd_shapes_reversed_tables(h, nq, nk, d, dv, p):
    # tests/cuda_attention_test.cpp:230-273 (seeds 8101-8103, padding +-77)
    blocks = (nk - 1) // p + 1
    phys = blocks + 2
    table = np.array([phys - 1 - i for i in range(blocks)], np.uint32)
    q = oracle.random_uniform((h, nq, d), 8101)
    k = oracle.random_uniform((h, nk, d), 8102)
    v = oracle.random_uniform((h, nk, dv), 8103)
    off = nk - nq
    expected, _ = oracle.sdpa(q, k, v, off)
    out, _ = oracle.paged_attention(q, oracle.pack_logical_blocks(k, table, phys, p, 77.0),
                                    oracle.pack_logical_blocks(v, table, phys, p, -77.0),
                                    table, nk, query_position_offset=off)
    tol = 2e-5 + d * 1e-6
    np.testing.assert_allclose(out, expected, atol=tol)
    np.testing.assert_allclose(out, textbook_attention(q, k, v, off)[0], atol=tol)


@pytest.mark.parametrize("h,hist,tail,d,dv,p", [(1, 0, 1, 1, 2, 2), (2, 3, 1, 5, 7, 2),
                                                 (3, 5, 3, 37, 41, 4)])
def test_tail_odd_shapes(h, hist, tail, d, dv, p):
    # tests/cuda_attention_test.cpp:376-449 (seeds 8201-8205, padding +-10000)
    blocks = 0 if hist == 0 else (hist - 1) // p + 1
    phys = blocks + 2
    table = np.array([phys - 1 - i for i in range(blocks)], np.uint32)
    q = oracle.random_uniform((h, tail, d), 8201)
    hk = oracle.random_uniform((h, hist, d), 8202)
    hv = oracle.random_uniform((h, hist, dv), 8203)
    tk = oracle.random_uniform((h, tail, d), 8204)
    tv = oracle.random_uniform((h, tail, dv), 8205)
    ck, cv = np.concatenate([hk, tk], 1), np.concatenate([hv, tv], 1)
    exp_out, exp_ws = oracle.sdpa(q, ck, cv, hist)
    out, ws = oracle.paged_attention(q, oracle.pack_logical_blocks(hk, table, phys, p, 1e4),
                                     oracle.pack_logical_blocks(hv, table, phys, p, -1e4),
                                     table, hist, tk, tv)
    tol = 2e-5 + d * 1e-6
    np.testing.assert_allclose(out, exp_out, atol=tol)
    np.testing.assert_allclose(ws, exp_ws, atol=2e-6)
    np.testing.assert_allclose(out, textbook_attention(q, ck, cv, hist)[0], atol=tol)


def test_gqa_equals_replicated_mha():
    # Extension invariant: GQA == MHA over KV heads repeated Hq / Hkv times.
    hq, hkv, d, p, hist = 8, 2, 16, 4, 13
    blocks = (hist - 1) // p + 1
    table = np.array([5, 0, 3, 1], np.uint32)[:blocks]
    kp = oracle.random_normal((6, hkv, p, d), 1)
    vp = oracle.random_normal((6, hkv, p, d), 2)
    q = oracle.random_normal((hq, 1, d), 3)
    tk = oracle.random_normal((hkv, 1, d), 4)
    tv = oracle.random_normal((hkv, 1, d), 5)
    g = hq // hkv
    out, _ = oracle.paged_attention(q, kp, vp, table, hist, tk, tv)
    rep, _ = oracle.paged_attention(q, np.repeat(kp, g, axis=1), np.repeat(vp, g, axis=1), table,
                                    hist, np.repeat(tk, g, axis=0), np.repeat(tv, g, axis=0))
    np.testing.assert_array_equal(out, rep)
    # and against the textbook on the gathered history
    hk = np.concatenate([kp[table[i]] for i in range(blocks)], 1)[:, :hist]
    hv = np.concatenate([vp[table[i]] for i in range(blocks)], 1)[:, :hist]
    ck = np.repeat(np.concatenate([hk, tk], 1), g, axis=0)
    cv = np.repeat(np.concatenate([hv, tv], 1), g, axis=0)
    np.testing.assert_allclose(out, textbook_attention(q, ck, cv, hist)[0], atol=2e-5)


def test_batched_decode_equals_per_sequence_loop():
    # Extension invariant: batch == loop of single-sequence calls, any thread count.
    b, hq, hkv, d, p = 5, 4, 2, 8, 4
    lengths = np.array([1, 4, 9, 0, 16], np.int32)
    n = 40
    kp = oracle.random_normal((n, hkv, p, d), 11)
    vp = oracle.random_normal((n, hkv, p, d), 12)
    rng = np.random.default_rng(0)
    tables = rng.permutation(n)[: b * 5].reshape(b, 5).astype(np.uint32)
    q = oracle.random_normal((b, hq, d), 13)
    tk = oracle.random_normal((b, hkv, d), 14)
    tv = oracle.random_normal((b, hkv, d), 15)
    out1 = oracle.batched_decode(q, kp, vp, tables, lengths, tk, tv, threads=1)
    out3 = oracle.batched_decode(q, kp, vp, tables, lengths, tk, tv, threads=3)
    np.testing.assert_array_equal(out1, out3)
    for i in range(b):
        o, _ = oracle.paged_attention(q[i][:, None], kp, vp, tables[i], int(lengths[i]),
                                      tk[i][:, None], tv[i][:, None])
        np.testing.assert_array_equal(out1[i], o[:, 0])


# ------------------------------------------------------------ bf16 pages ----
def test_bf16_rounding_known_answers():
    """Round-to-nearest-even onto the bf16 grid, case by case."""
    f = np.float32
    cases = [
        (1.0, 0x3F80), (-2.0, 0xC000), (0.0, 0x0000), (-0.0, 0x8000),
        (np.inf, 0x7F80), (-np.inf, 0xFF80),
        # exactly representable: unchanged
        (1.0078125, 0x3F81),
        # halfway between 0x3F80 and 0x3F81: ties to even (down)
        (np.uint32(0x3F808000).view(np.float32), 0x3F80),
        # halfway between 0x3F81 and 0x3F82: ties to even (up)
        (np.uint32(0x3F818000).view(np.float32), 0x3F82),
        # just above halfway: up; just below: down
        (np.uint32(0x3F808001).view(np.float32), 0x3F81),
        (np.uint32(0x3F807FFF).view(np.float32), 0x3F80),
        # largest float32 rounds past the largest bf16: inf
        (np.finfo(np.float32).max, 0x7F80),
        # largest bf16 stays finite
        (np.uint32(0x7F7F0000).view(np.float32), 0x7F7F),
        # subnormals round on the same grid
        (np.uint32(0x00018000).view(np.float32), 0x0002),
        (np.uint32(0x00008000).view(np.float32), 0x0000),
    ]
    for x, want in cases:
        got = int(oracle.bf16_bits(np.array([x], f))[0])
        assert got == want, (x, hex(got), hex(want))
    nan = oracle.bf16_bits(np.array([np.nan, -np.nan], f))
    assert np.isnan(oracle.round_bf16(np.array([np.nan, -np.nan], f))).all()
    assert (nan[0] & 0x8000) == 0 and (nan[1] & 0x8000) != 0  # sign kept


def test_bf16_rounding_matches_torch():
    """torch's CPU float32 -> bfloat16 conversion rounds to nearest even; it
    must agree bit for bit on every non-NaN value, across magnitudes."""
    import torch
    rng = np.random.default_rng(3)
    bits = rng.integers(0, 1 << 32, 200000, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    x = x[~np.isnan(x)]
    x = np.concatenate([x, rng.standard_normal(50000).astype(np.float32) * 1e3])
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(oracle.bf16_bits(x), want)
    assert np.array_equal(oracle.round_bf16(x), torch.from_numpy(x).to(torch.bfloat16).float().numpy())


# ------------------------------------------------------------- fp8 pages ----
def test_fp8_decode_matches_torch_on_every_code():
    """The E4M3 value table from the format's definition against torch's
    float8_e4m3fn -> float32 widening, all 256 codes (NaN codes as NaN)."""
    import torch
    codes = np.arange(256, dtype=np.uint8)
    want = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    got = oracle.fp8_decode(codes)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    ok = ~np.isnan(want)
    assert np.array_equal(got[ok].view(np.uint32), want[ok].view(np.uint32))  # signed zeros too
    assert np.isnan(got[[0x7F, 0xFF]]).all() and np.isnan(got).sum() == 2
    assert got[0x7E] == 448.0 and got[0x01] == 2.0 ** -9 and got[0x08] == 2.0 ** -6


def test_fp8_rounding_known_answers():
    """Ties to even on the E4M3 grid, the subnormal step, saturation and NaN."""
    f = np.float32
    cases = [
        (1.0, 0x38), (-2.0, 0xC0), (0.0, 0x00), (-0.0, 0x80),
        (1.0625, 0x38),   # halfway 1.0 / 1.125: even (down)
        (1.1875, 0x3A),   # halfway 1.125 / 1.25: even (up)
        (1.0626, 0x39), (1.0624, 0x38),
        (448.0, 0x7E), (449.0, 0x7E), (464.0, 0x7E), (465.0, 0x7E), (1e30, 0x7E),
        (np.inf, 0x7E), (-np.inf, 0xFE),   # saturating: no infinities in E4M3
        (2.0 ** -9, 0x01), (2.0 ** -10, 0x00),  # halfway 0 / 2^-9: even (zero)
        (3 * 2.0 ** -10, 0x02),                 # halfway 2^-9 / 2^-8: even (up)
        (2.0 ** -6, 0x08), (15 * 2.0 ** -10, 0x08),  # last subnormal step rounds up to 2^-6
        (np.uint32(1).view(np.float32), 0x00),  # fp32 subnormal: zero
    ]
    for x, want in cases:
        got = int(oracle.fp8_bits(np.array([x], f))[0])
        assert got == want, (x, hex(got), hex(want))
    nan = oracle.fp8_bits(np.array([np.nan, -np.nan], f))
    assert nan.tolist() == [0x7F, 0xFF]


def test_fp8_rounding_matches_torch_in_range():
    """torch's float32 -> float8_e4m3fn conversion rounds to nearest even and
    turns what rounds past 448 into NaN; this contract saturates instead.
    Below that boundary (|x| < 464) the two agree bit for bit; above it
    every value saturates."""
    import torch
    rng = np.random.default_rng(11)
    bits = rng.integers(0, 1 << 32, 300000, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    x = x[~np.isnan(x)]
    x = np.concatenate([x, rng.standard_normal(100000).astype(np.float32),
                        rng.standard_normal(50000).astype(np.float32) * 100,
                        rng.standard_normal(50000).astype(np.float32) * 1e-3])
    small = np.abs(x) < 464.0
    want = torch.from_numpy(x[small]).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(oracle.fp8_bits(x[small]), want)
    big = x[~small]
    assert big.size > 1000
    assert np.array_equal(oracle.fp8_bits(big), np.where(big > 0, 0x7E, 0xFE).astype(np.uint8))


def test_fp8_scale_divides_before_rounding():
    """code = round(x / scale); value = decode(code) * scale, both in fp32."""
    rng = np.random.default_rng(5)
    x = rng.standard_normal(20000).astype(np.float32) * 7
    for scale in (1.0, 0.25, 0.0371, 3.0):
        s = np.float32(scale)
        assert np.array_equal(oracle.fp8_bits(x, scale), oracle.fp8_bits(x / s))
        want = oracle.fp8_decode(oracle.fp8_bits(x / s)) * s
        assert np.array_equal(oracle.round_fp8(x, scale), want)
        # relative error of the grid: at most half a mantissa step (2^-4) in range
        v = oracle.round_fp8(x, scale)
        normal = np.abs(x / s) >= 2.0 ** -6
        inrange = np.abs(x / s) <= 448
        m = normal & inrange
        assert (np.abs(v[m] - x[m]) <= np.abs(x[m]) * 2.0 ** -4 * (1 + 1e-6)).all()
