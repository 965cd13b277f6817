"""Chunked-prefill attention (fp32 MFMA) against the CPU oracle.

The oracle is the restatement of the reference's CPU paged attention with a
T-token tail (src/attention/paged_reference.cpp:173-384): query row t sees
the whole paged history and chunk rows 0..t.  GQA is checked as replicated
MHA, the batch as a per-sequence loop.  Tolerance: max-abs 2e-5 plus
rel 1e-4, per element."""

import concurrent.futures as cf

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


def make_case(rng, hq, hkv, hists, T, spare=3):
    """Pool with every sequence's pages scattered by a seeded permutation."""
    pages = [(h + P - 1) // P for h in hists]
    n = sum(pages) + spare
    kp = rng.standard_normal((n, hkv, P, D), dtype=np.float32)
    vp = rng.standard_normal((n, hkv, P, D), dtype=np.float32)
    perm = rng.permutation(n)
    max_blocks = max(max(pages), 1)
    tables = np.zeros((len(hists), max_blocks), np.uint32)
    at = 0
    for b, c in enumerate(pages):
        tables[b, :c] = perm[at: at + c]
        at += c
    B = len(hists)
    q = rng.standard_normal((B, hq, T, D), dtype=np.float32)
    ck = rng.standard_normal((B, hkv, T, D), dtype=np.float32)
    cv = rng.standard_normal((B, hkv, T, D), dtype=np.float32)
    return kp, vp, tables, np.array(hists, np.int32), q, ck, cv


def oracle_prefill(kp, vp, tables, lengths, q, ck, cv, workers=8):
    def one(b):
        return oracle.paged_attention(q[b], kp, vp, tables[b], int(lengths[b]), ck[b], cv[b])[0]

    with cf.ThreadPoolExecutor(workers) as ex:
        return np.stack(list(ex.map(one, range(len(lengths)))))


def run_gpu(kp, vp, tables, lengths, q, ck, cv):
    out = torch.full(q.shape, float("nan"), device="cuda:0")
    hx.paged_prefill_attention(dev(q), dev(kp), dev(vp), dev(tables), dev(lengths), dev(ck),
                               dev(cv), out)
    torch.cuda.synchronize()
    return host(out)


def assert_close(got, want, what=""):
    both_nan = np.isnan(got) & np.isnan(want)
    same_inf = np.isinf(got) & np.isinf(want) & (np.sign(got) == np.sign(want))
    diff = np.abs(got.astype(np.float64) - want.astype(np.float64))
    ok = both_nan | same_inf | (diff <= ATOL + RTOL * np.abs(want))
    if not ok.all():
        idx = np.argwhere(~ok)[0]
        raise AssertionError(f"{what}: {(~ok).sum()} elements off, first at {tuple(idx)}: "
                             f"got {got[tuple(idx)]}, want {want[tuple(idx)]}")


@pytest.mark.parametrize("hq,hkv", [(4, 4), (8, 4), (16, 4), (32, 4)])
@pytest.mark.parametrize("T", [1, 5, 16, 37, 130])
def test_prefill_matches_oracle(device, hq, hkv, T):
    rng = np.random.default_rng(1000 * hq + T)
    case = make_case(rng, hq, hkv, [0, 1, 15, 16, 17, 100, 257], T)
    assert_close(run_gpu(*case), oracle_prefill(*case), f"hq={hq} hkv={hkv} T={T}")


def test_prefill_config5_sample(device):
    """Config-5 geometry (32q / 8kv heads, 512-token chunk) on 3 sequences."""
    rng = np.random.default_rng(5)
    case = make_case(rng, 32, 8, [0, 700, 1311], 512)
    assert_close(run_gpu(*case), oracle_prefill(*case), "config5 sample")


def test_prefill_long_history_small_chunk(device):
    rng = np.random.default_rng(6)
    case = make_case(rng, 8, 2, [4096, 3001], 24)
    assert_close(run_gpu(*case), oracle_prefill(*case), "long history")


def test_prefill_future_nonfinite_values_do_not_leak(device):
    """A non-finite value row in the chunk reaches only the rows that see it
    (the reference skips masked keys in P.V)."""
    rng = np.random.default_rng(7)
    kp, vp, tables, lengths, q, ck, cv = make_case(rng, 8, 4, [40, 0], 40)
    cv[0, 1, 20, 5] = np.inf
    cv[0, 2, 33, :] = np.nan
    cv[1, 0, 3, 7] = -np.inf
    ck[1, 3, 11, :] = np.nan  # masked key rows never produce scores either
    case = (kp, vp, tables, lengths, q, ck, cv)
    got, want = run_gpu(*case), oracle_prefill(*case)
    assert np.isfinite(want[0, :, :20]).all()  # rows before the bad row stay finite
    assert_close(got, want, "non-finite future rows")


def test_prefill_special_scores(device):
    rng = np.random.default_rng(8)
    kp, vp, tables, lengths, q, ck, cv = make_case(rng, 4, 4, [33, 16], 9)
    q[0, 0, 3, :] = np.nan          # NaN query row -> NaN output row
    ck[0, 1, 2, 0] = np.inf         # +inf score for rows of head 1 that see it
    q[0, 1, :, 0] = 1.0
    kp[:, 2, :, :] = -1e30          # huge negative history scores
    q[1, 3, :, :] *= 1e20           # overflowing scores
    case = (kp, vp, tables, lengths, q, ck, cv)
    assert_close(run_gpu(*case), oracle_prefill(*case), "special scores")


def test_prefill_bad_page_and_length_give_nan(device):
    rng = np.random.default_rng(9)
    kp, vp, tables, lengths, q, ck, cv = make_case(rng, 8, 4, [50, 20, 30], 12)
    tables[0, 1] = kp.shape[0] + 5           # page ID out of range
    lengths[2] = tables.shape[1] * P + 1     # history the table row cannot cover
    got = run_gpu(kp, vp, tables, lengths, q, ck, cv)
    assert np.isnan(got[0]).all() and np.isnan(got[2]).all()
    want = oracle.paged_attention(q[1], kp, vp, tables[1], int(lengths[1]), ck[1], cv[1])[0]
    assert_close(got[1], want, "untouched sequence")


def test_prefill_rejects_bad_arguments(device):
    q = torch.zeros(1, 6, 4, D, device=device)
    pool = torch.zeros(4, 2, P, D, device=device)
    tables = torch.zeros(1, 2, dtype=torch.int32, device=device)
    lengths = torch.zeros(1, dtype=torch.int32, device=device)
    chunk = torch.zeros(1, 2, 4, D, device=device)
    out = torch.zeros_like(q)
    with pytest.raises(hx.HelixError):  # group 3 unsupported
        hx.paged_prefill_attention(q, pool, pool, tables, lengths, chunk, chunk, out)
    q2 = torch.zeros(1, 4, 4, D, device=device)
    with pytest.raises(hx.HelixError):  # output aliases the query
        hx.paged_prefill_attention(q2, pool, pool, tables, lengths, chunk, chunk, q2)


def test_batch_chunk_steps_append_and_attend(device):
    """prepare_chunk + per-layer chunk append + prefill, then a decode step;
    pages are bit-exact against the oracle pool and outputs within
    tolerance."""
    L, H, HQ = 2, 4, 16
    rng = np.random.default_rng(10)
    hists = [0, 5, 16, 70]
    T = 40
    N = sum((h + T + 1) // P + 2 for h in hists) + 4
    cache = hx.PagedKvCache(L, H, D, P, N)
    pool = oracle.PagedPool(L, H, D, P, N)
    seqs = []
    for h in hists:
        s, so = cache.create_sequence(), pool.create_sequence()
        if h:
            k = rng.standard_normal((L, H, h, D), dtype=np.float32)
            v = rng.standard_normal((L, H, h, D), dtype=np.float32)
            cache.append_layer_major(s, [dev(k[l]) for l in range(L)],
                                     [dev(v[l]) for l in range(L)])
            pool.append_layer_major(so, k, v)
        seqs.append((s, so))
    B = len(seqs)
    batch = hx.DecodeBatch(cache, [s for s, _ in seqs], HQ, max_tokens=max(hists) + T + 8)
    batch.prepare_chunk(T)
    ck = rng.standard_normal((L, B, H, T, D), dtype=np.float32)
    cv = rng.standard_normal((L, B, H, T, D), dtype=np.float32)
    for layer in range(L):
        q = rng.standard_normal((B, HQ, T, D), dtype=np.float32)
        out = torch.empty(B, HQ, T, D, device=device)
        dk, dvv = dev(ck[layer]), dev(cv[layer])
        batch.append_layer(layer, dk, dvv)
        batch.prefill_layer(layer, dev(q), dk, dvv, out)
        torch.cuda.synchronize()
        got = host(out)
        for b, (_, so) in enumerate(seqs):
            tab = np.array(pool.block_table(so), np.uint32)
            kp_o, vp_o = pool.layer_pages(layer)
            want = oracle.paged_attention(q[b], kp_o, vp_o, tab, pool.length(so), ck[layer, b],
                                          cv[layer, b])[0]
            assert_close(got[b], want, f"layer {layer} seq {b}")
    for b, (_, so) in enumerate(seqs):
        pool.append_layer_major(so, ck[:, b], cv[:, b])
    # The chunk landed in the pages exactly where the oracle pool put it.
    for b, (s, so) in enumerate(seqs):
        assert cache.block_table(s) == list(pool.block_table(so))
        for layer in range(L):
            k_gpu, v_gpu = cache.retrieve_layer(s, layer)
            k_o, v_o = pool.copy_layer(so, layer)
            assert np.array_equal(host(k_gpu), k_o) and np.array_equal(host(v_gpu), v_o)
    # A decode step after the chunk uses the grown tables.
    batch.prepare()
    tk = rng.standard_normal((B, H, D), dtype=np.float32)
    tv = rng.standard_normal((B, H, D), dtype=np.float32)
    q = rng.standard_normal((B, HQ, D), dtype=np.float32)
    out = torch.empty(B, HQ, D, device=device)
    batch.append_layer(0, dev(tk), dev(tv))
    batch.attention_layer(0, dev(q), dev(tk), dev(tv), out)
    torch.cuda.synchronize()
    kp_o, vp_o = pool.layer_pages(0)
    for b, (_, so) in enumerate(seqs):
        tab = np.array(pool.block_table(so), np.uint32)
        want = oracle.paged_attention(q[b][:, None], kp_o, vp_o, tab, pool.length(so),
                                      tk[b][:, None], tv[b][:, None])[0][:, 0]
        assert_close(host(out)[b], want, f"decode after chunk seq {b}")
    with pytest.raises(hx.HelixError):  # decode attention needs a one-token step
        batch.prepare_chunk(2)
        batch.attention_layer(0, dev(q), dev(tk), dev(tv), out)
    batch.close()
