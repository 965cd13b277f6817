"""The stateless batched entry points over bf16 and fp8 E4M3 pools
(helix_paged_decode_attention_typed / helix_paged_prefill_attention_typed,
extension: the reference's pools are fp32 only, docs/KV_CACHE.md:531).

A caller that keeps reduced-precision pools without a DecodeBatch passes the
pools of a typed cache, its own tables and lengths.  The result must equal
the fp32 oracle on the values the pages hold (and on the tail / chunk rows
rounded onto the same grid, the values their pages will hold) within max-abs
2e-5 plus rel 1e-4.  The fp32 format through the typed entry is the untyped
entry (every other test of the batched kernels runs it)."""

import numpy as np
import pytest
import torch

import helix_runtime_amd as hx
import oracle

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-5, 1e-4
D, P, H = 128, 16, 8
KS, VS = 0.037, 0.011


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda:0")


def host(t):
    return t.detach().cpu().numpy()


def rounders(dtype):
    if dtype == "bf16":
        return oracle.round_bf16, oracle.round_bf16
    return (lambda x: oracle.round_fp8(x, KS)), (lambda x: oracle.round_fp8(x, VS))


def build(dtype, hists, seed):
    rk, rv = rounders(dtype)
    rng = np.random.default_rng(seed)
    N = sum((h + P - 1) // P for h in hists) + 8
    kw = dict(k_scale=KS, v_scale=VS) if dtype == "fp8" else {}
    cache = hx.PagedKvCache(1, H, D, P, N, page_dtype=dtype, **kw)
    pool = oracle.PagedPool(1, H, D, P, N)
    seqs = []
    for h in hists:
        s, so = cache.create_sequence(), pool.create_sequence()
        if h:
            k = rng.standard_normal((1, H, h, D), dtype=np.float32)
            v = rng.standard_normal((1, H, h, D), dtype=np.float32)
            cache.append_layer_major(s, [dev(k[0])], [dev(v[0])])
            pool.append_layer_major(so, rk(k), rv(v))
        seqs.append((s, so))
    max_blocks = max(1, max((h + P - 1) // P for h in hists))
    tables = np.zeros((len(hists), max_blocks), np.uint32)
    for b, (s, so) in enumerate(seqs):
        tab = cache.block_table(s)
        assert tab == list(pool.block_table(so))
        tables[b, :len(tab)] = tab
    return cache, pool, tables, N, rng


@pytest.mark.parametrize("dtype", ["bf16", "fp8"])
@pytest.mark.parametrize("hq", [8, 16, 32, 64])
def test_typed_stateless_decode_matches_oracle(device, dtype, hq):
    hists = [0, 5, 16, 300, 1000, 2100]
    cache, pool, tables, N, rng = build(dtype, hists, 71 + hq)
    rk, rv = rounders(dtype)
    B = len(hists)
    HQ = hq
    q = rng.standard_normal((B, HQ, D), dtype=np.float32)
    tk = rng.standard_normal((B, H, D), dtype=np.float32)
    tv = rng.standard_normal((B, H, D), dtype=np.float32)
    lengths = np.array(hists, np.int32)
    kptr, vptr = cache.layer_pool_pointers(0)
    out = torch.full((B, HQ, D), 7.0, device=device)
    ws = hx.decode_workspace(B, HQ, H, tables.shape[1])
    kw = dict(k_scale=KS, v_scale=VS) if dtype == "fp8" else {}
    hx.paged_decode_attention(dev(q), kptr, vptr, dev(tables.view(np.int32)), dev(lengths),
                              dev(tk), dev(tv), out, ws, pool_shape=(N, H, P, D),
                              page_dtype=dtype, **kw)
    torch.cuda.synchronize()
    kp, vp = pool.layer_pages(0)
    want = oracle.batched_decode(q, kp, vp, tables, lengths, rk(tk), rv(tv), threads=8)
    np.testing.assert_allclose(host(out), want, atol=ATOL, rtol=RTOL)
    with pytest.raises(hx.HelixError) as e:  # no explicit split size on reduced pages
        hx.paged_decode_attention(dev(q), kptr, vptr, dev(tables.view(np.int32)), dev(lengths),
                                  dev(tk), dev(tv), out, ws, pages_per_split=4,
                                  pool_shape=(N, H, P, D), page_dtype=dtype, **kw)
    assert e.value.status == hx.UNSUPPORTED


@pytest.mark.parametrize("dtype", ["bf16", "fp8"])
@pytest.mark.parametrize("hq", [8, 16, 32, 64])
def test_typed_stateless_prefill_matches_oracle(device, dtype, hq):
    hists = [0, 7, 64, 333, 1200]
    cache, pool, tables, N, rng = build(dtype, hists, 72 + hq)
    rk, rv = rounders(dtype)
    B, T = len(hists), 40
    HQ = hq
    q = rng.standard_normal((B, HQ, T, D), dtype=np.float32)
    ck = rng.standard_normal((B, H, T, D), dtype=np.float32)
    cv = rng.standard_normal((B, H, T, D), dtype=np.float32)
    kptr, vptr = cache.layer_pool_pointers(0)
    out = torch.full((B, HQ, T, D), 7.0, device=device)
    kw = dict(k_scale=KS, v_scale=VS) if dtype == "fp8" else {}
    hx.paged_prefill_attention(dev(q), kptr, vptr, dev(tables.view(np.int32)),
                               dev(np.array(hists, np.int32)), dev(ck), dev(cv), out,
                               pool_shape=(N, H, P, D), page_dtype=dtype, **kw)
    torch.cuda.synchronize()
    kp, vp = pool.layer_pages(0)
    got = host(out)
    for b, h in enumerate(hists):
        tab = tables[b, : (h + P - 1) // P]
        want = oracle.paged_attention(q[b], kp, vp, tab, h, rk(ck[b]), rv(cv[b]))[0]
        np.testing.assert_allclose(got[b], want, atol=ATOL, rtol=RTOL,
                                   err_msg=f"{dtype} sequence {b}")
