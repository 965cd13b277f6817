"""Config 5 at its real size against the CPU oracle.

16 sequences, each appending a 512-token chunk onto a paged history drawn
U[0, 4096] from a fixed seed (one history pinned to 0 and one to >= 4000),
32 query heads / 8 kv heads, head_dim 128, 16-token pages scattered across
the pool by the cache's shuffled free queue; one layer.  The chunk goes
through the production flow: DecodeBatch.prepare_chunk -> append_layer ->
prefill_layer (the fast matrix-core kernel plus the exact redo of flagged
work items).  Every output row of every sequence is compared with the
oracle's restatement of the reference's paged SDPA with a T-token tail
(src/attention/paged_reference.cpp:210-384) within max-abs 2e-5 plus rel
1e-4; the appended pages are compared bit-exactly with the oracle pool.
bf16 pages run the same workload against the oracle on the rounded values.
"""

import concurrent.futures as cf
import os

import numpy as np
import pytest
import torch

import helix_runtime_amd as hx
import oracle

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-5, 1e-4
D, P, HQ, HKV, T, B = 128, 16, 32, 8, 512, 16


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda:0")


def host(t):
    return t.detach().cpu().numpy()


def config5_histories(seed=55):
    rng = np.random.default_rng(seed)
    hists = rng.integers(0, 4097, size=B)
    hists[3] = 0
    hists[11] = max(int(hists[11]), 4000 + int(rng.integers(0, 97)))
    return [int(h) for h in hists]


def run_config5(page_dtype, seed):
    hists = config5_histories()
    assert 0 in hists and max(hists) >= 4000
    rk = oracle.round_bf16 if page_dtype == "bf16" else (lambda x: x)
    rng = np.random.default_rng(seed)
    N = sum((h + T) // P + 2 for h in hists) + 16
    cache = hx.PagedKvCache(1, HKV, D, P, N, page_dtype=page_dtype)
    pool = oracle.PagedPool(1, HKV, D, P, N)
    seqs = []
    for h in hists:
        s, so = cache.create_sequence(), pool.create_sequence()
        if h:
            k = rng.standard_normal((1, HKV, h, D), dtype=np.float32)
            v = rng.standard_normal((1, HKV, h, D), dtype=np.float32)
            cache.append_layer_major(s, [dev(k[0])], [dev(v[0])])
            pool.append_layer_major(so, rk(k), rk(v))
        seqs.append((s, so))
    ck = rng.standard_normal((B, HKV, T, D), dtype=np.float32)
    cv = rng.standard_normal((B, HKV, T, D), dtype=np.float32)
    q = rng.standard_normal((B, HQ, T, D), dtype=np.float32)
    batch = hx.DecodeBatch(cache, [s for s, _ in seqs], HQ, max_tokens=max(hists) + T + 8)
    batch.prepare_chunk(T)
    out = torch.full((B, HQ, T, D), float("nan"), device="cuda:0")
    dk, dv_ = dev(ck), dev(cv)
    print(f"config5 {page_dtype}: histories {hists}", flush=True)
    batch.append_layer(0, dk, dv_)
    batch.prefill_layer(0, dev(q), dk, dv_, out)
    torch.cuda.synchronize()
    got = host(out)
    kp, vp = pool.layer_pages(0)

    def want(b):
        so = seqs[b][1]
        tab = np.array(pool.block_table(so), np.uint32)
        return oracle.paged_attention(q[b], kp, vp, tab, pool.length(so), rk(ck[b]),
                                      rk(cv[b]))[0]

    workers = min(16, os.cpu_count() or 1)
    with cf.ThreadPoolExecutor(workers) as ex:
        wants = list(ex.map(want, range(B)))
    for b in range(B):
        np.testing.assert_allclose(got[b], wants[b], atol=ATOL, rtol=RTOL,
                                   err_msg=f"config5 {page_dtype} sequence {b} hist {hists[b]}")
    # The chunk landed in the pages where the oracle pool puts it.
    for b, (s, so) in enumerate(seqs):
        pool.append_layer_major(so, rk(ck[b][None]), rk(cv[b][None]))
        assert cache.block_table(s) == list(pool.block_table(so))
    if page_dtype == "f32":
        for b in (3, 11, 0):
            s, so = seqs[b]
            k_gpu, v_gpu = cache.retrieve_layer(s, 0)
            k_o, v_o = pool.copy_layer(so, 0)
            assert np.array_equal(host(k_gpu), k_o) and np.array_equal(host(v_gpu), v_o)
    batch.close()


def test_config5_full_size_fp32_pages(device):
    run_config5("f32", 5005)


def test_config5_full_size_bf16_pages(device):
    run_config5("bf16", 5006)
