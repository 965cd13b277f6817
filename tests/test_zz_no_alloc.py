"""helix_paged_decode_attention_noalloc (the entry point that allocates
nothing; its partials live in a library-owned device array) against
helix_paged_decode_attention(_typed) with a caller workspace: identical
outputs, bit for bit, on two calls in a row, the second with a smaller
input, on fp32, bf16 and fp8 pools, and within the north-star tolerance of
the oracle."""

import ctypes

import numpy as np
import pytest
import torch

import helix_runtime_amd as hx
import oracle

pytestmark = pytest.mark.gpu

D, P = 128, 16


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda:0")


def problem(seed, batch, hkv, g, max_len):
    rng = np.random.default_rng(seed)
    lengths = rng.integers(0, max_len + 1, size=batch).astype(np.int32)
    lengths[0] = max_len
    pages = (lengths + P - 1) // P
    phys = int(pages.sum()) + 4
    perm = rng.permutation(phys).astype(np.uint32)
    max_blocks = int(pages.max()) + 1
    tables = np.zeros((batch, max_blocks), np.uint32)
    at = 0
    for b, n in enumerate(pages):
        tables[b, :n] = perm[at: at + n]
        at += n
    kp = rng.standard_normal((phys, hkv, P, D), dtype=np.float32)
    vp = rng.standard_normal((phys, hkv, P, D), dtype=np.float32)
    q = rng.standard_normal((batch, hkv * g, D), dtype=np.float32)
    tk = rng.standard_normal((batch, hkv, D), dtype=np.float32)
    tv = rng.standard_normal((batch, hkv, D), dtype=np.float32)
    return q, kp, vp, tables, lengths, tk, tv


def noalloc(q, kp, vp, tables, lengths, tk, tv, out, pool_shape=None, dtype=0, ks=1.0, vs=1.0):
    b, hq, _ = q.shape
    n, hkv, p, d = kp.shape if pool_shape is None else pool_shape
    p_ = lambda t: ctypes.c_void_p(t if isinstance(t, int) else t.data_ptr())  # noqa: E731
    return hx.load().helix_paged_decode_attention_noalloc(
        p_(q), b, hq, hkv, d, p_(kp), p_(vp), n, p, p_(tables), tables.shape[1], p_(lengths),
        p_(tk), p_(tv), p_(out), dtype, ks, vs,
        ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))


def test_noalloc_matches_workspace_entry_twice_shrinking(device):
    # Two calls in a row, the second smaller; then a larger one and an MHA
    # one, so the array's partial layout moves under a fixed count region.
    for seed, batch, hkv, g, max_len in ((1, 24, 8, 4, 3000), (2, 5, 8, 4, 700),
                                         (3, 40, 8, 4, 1500), (4, 6, 32, 1, 900)):
        print(f"noalloc case seed={seed} batch={batch} hkv={hkv} g={g} max_len={max_len}",
              flush=True)
        q, kp, vp, tables, lengths, tk, tv = problem(seed, batch, hkv, g, max_len)
        dq, dkp, dvp, dtab, dlen, dtk, dtv = (dev(x) for x in (q, kp, vp, tables.view(np.int32),
                                                               lengths, tk, tv))
        want = torch.empty(batch, hkv * g, D, device=device)
        ws = hx.decode_workspace(batch, hkv * g, hkv, tables.shape[1])
        hx.paged_decode_attention(dq, dkp, dvp, dtab, dlen, dtk, dtv, want, ws)
        got = torch.full((batch, hkv * g, D), 7.0, device=device)
        assert noalloc(dq, dkp, dvp, dtab, dlen, dtk, dtv, got) == 0, \
            hx.load().helix_last_error()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(got.cpu().numpy(), want.cpu().numpy())
        ref = oracle.batched_decode(q, kp, vp, tables, lengths, tk, tv, threads=8)
        np.testing.assert_allclose(got.cpu().numpy(), ref, atol=2e-5, rtol=1e-4)


def test_noalloc_calls_queued_on_one_stream_do_not_race(device):
    """Two calls of different sizes queued back to back on one stream, with
    no host synchronisation between them, share the library's array
    correctly: calls ordered on one stream are the supported way to reuse
    it (calls that overlap on one GPU race, as the header states)."""
    cases = [problem(11, 30, 8, 4, 2500), problem(12, 7, 8, 4, 400)]
    outs, wants = [], []
    for q, kp, vp, tables, lengths, tk, tv in cases:
        args = [dev(x) for x in (q, kp, vp, tables.view(np.int32), lengths, tk, tv)]
        want = torch.empty(q.shape, device=device)
        ws = hx.decode_workspace(q.shape[0], q.shape[1], kp.shape[1], tables.shape[1])
        hx.paged_decode_attention(*args, want, ws)
        outs.append((args, torch.full(q.shape, 7.0, device=device)))
        wants.append(want)
    torch.cuda.synchronize()
    for args, got in outs:  # queued, no synchronisation in between
        assert noalloc(*args, got) == 0, hx.load().helix_last_error()
    torch.cuda.synchronize()
    for (_, got), want in zip(outs, wants):
        np.testing.assert_array_equal(got.cpu().numpy(), want.cpu().numpy())


@pytest.mark.parametrize("dtype", ["bf16", "fp8"])
def test_noalloc_typed_pools_match_the_typed_workspace_entry(device, dtype):
    """bf16 and fp8 pools (a typed cache's layer pools) through the entry
    point, two calls in a row, the second smaller: bit-identical to
    helix_paged_decode_attention_typed with a workspace."""
    ks, vs = (0.037, 0.011) if dtype == "fp8" else (1.0, 1.0)
    code = {"bf16": 1, "fp8": 2}[dtype]
    kw = dict(k_scale=ks, v_scale=vs) if dtype == "fp8" else {}
    for seed, batch, max_len in ((21, 20, 2500), (22, 6, 600)):
        print(f"noalloc typed case {dtype} seed={seed} batch={batch}", flush=True)
        rng = np.random.default_rng(seed)
        H, HQ = 8, 32
        hists = [int(x) for x in rng.integers(0, max_len + 1, size=batch)]
        N = sum((h + P - 1) // P for h in hists) + 8
        cache = hx.PagedKvCache(1, H, D, P, N, page_dtype=dtype, **kw)
        tables = np.zeros((batch, max(1, max((h + P - 1) // P for h in hists))), np.uint32)
        for b, h in enumerate(hists):
            s = cache.create_sequence()
            if h:
                cache.append_layer_major(s, [dev(rng.standard_normal((H, h, D), dtype=np.float32))],
                                         [dev(rng.standard_normal((H, h, D), dtype=np.float32))])
            tab = cache.block_table(s)
            tables[b, :len(tab)] = tab
        kptr, vptr = cache.layer_pool_pointers(0)
        q = dev(rng.standard_normal((batch, HQ, D), dtype=np.float32))
        tk = dev(rng.standard_normal((batch, H, D), dtype=np.float32))
        tv = dev(rng.standard_normal((batch, H, D), dtype=np.float32))
        dtab, dlen = dev(tables.view(np.int32)), dev(np.array(hists, np.int32))
        want = torch.empty(batch, HQ, D, device=device)
        ws = hx.decode_workspace(batch, HQ, H, tables.shape[1])
        hx.paged_decode_attention(q, kptr, vptr, dtab, dlen, tk, tv, want, ws,
                                  pool_shape=(N, H, P, D), page_dtype=dtype, **kw)
        got = torch.full((batch, HQ, D), 7.0, device=device)
        assert noalloc(q, kptr, vptr, dtab, dlen, tk, tv, got, pool_shape=(N, H, P, D),
                       dtype=code, ks=ks, vs=vs) == 0, hx.load().helix_last_error()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(got.cpu().numpy(), want.cpu().numpy())
        cache.close()


def test_noalloc_rejects_batches_beyond_its_scratch(device):
    """More (sequence, kv head) units than the 16 MiB scratch holds are
    refused before any launch."""
    q = torch.zeros(4096, 32, D, device=device)
    out = torch.zeros(4096, 32, D, device=device)
    x = torch.zeros(16, device=device)
    p_ = ctypes.c_void_p(x.data_ptr())
    rc = hx.load().helix_paged_decode_attention_noalloc(
        ctypes.c_void_p(q.data_ptr()), 4096, 32, 8, D, p_, p_, 100, P, p_, 4, p_, p_, p_,
        ctypes.c_void_p(out.data_ptr()), 0, 1.0, 1.0,
        ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert rc == hx.OUT_OF_RANGE
    assert b"16 MiB scratch" in hx.load().helix_last_error()
