"""Chunked prefill through DecodeBatch, which runs a fast kernel and then
redoes exactly, with the fp32 kernel, every work item that met a special
value: on bf16 and fp8 pages the bf16 matrix-core kernel (the fp32 operand
of each product split into three exact bf16 terms), on fp32 pages the fp32
kernel without its exact paths (one tile per wavefront).  Checked against
the fp32 oracle on the rounded values within the fp32 tolerance (2e-5 abs +
1e-4 rel):
- every query group (1, 2, 4, 8 query heads per kv head), ragged histories;
- the two special cases the matrix-core kernel hands to the exact kernel:
  a NaN score (here from NaN key rows, and from an infinite bf16 key whose
  query term splits with a zero middle part, where the split alone would
  give NaN instead of inf) and a non-finite value row in a chunk position
  that earlier rows mask;
- a config-5-shaped chunk (512 tokens over histories of ~1000);
- every finite fp8 code in a history (the staging's hardware fp8-to-bf16
  move);
- chunk lengths and histories around the 32-key staging blocks."""

import numpy as np
import pytest
import torch

import helix_runtime_amd as hx
import oracle

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-5, 1e-4
D, P = 128, 16
KS, VS = 0.037, 0.011  # fp8 scales that are not powers of two


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda:0")


def host(t):
    return t.detach().cpu().numpy()


def rounder(page_dtype):
    if page_dtype == "f32":
        return (lambda x: x), (lambda x: x)
    if page_dtype == "bf16":
        return oracle.round_bf16, oracle.round_bf16
    return (lambda x: oracle.round_fp8(x, KS)), (lambda x: oracle.round_fp8(x, VS))


def make_cache(page_dtype, L, H, N):
    if page_dtype == "fp8":
        return hx.PagedKvCache(L, H, D, P, N, page_dtype="fp8", k_scale=KS, v_scale=VS)
    return hx.PagedKvCache(L, H, D, P, N, page_dtype=page_dtype)


def run_prefill(page_dtype, hq, hists, T, seed, edit=None, H=4):
    """Builds the histories, prepares a T-token chunk, runs append + prefill
    for one layer and returns (output, oracle output) per sequence.  edit(k,
    v, ck, cv, q) may plant special values (all float32 host arrays)."""
    L = 1
    RK, RV = rounder(page_dtype)
    rng = np.random.default_rng(seed)
    N = sum((h + T) // P + 2 for h in hists) + 4
    cache = make_cache(page_dtype, L, H, N)
    pool = oracle.PagedPool(L, H, D, P, N)
    B = len(hists)
    ks = [rng.standard_normal((L, H, h, D), dtype=np.float32) for h in hists]
    vs = [rng.standard_normal((L, H, h, D), dtype=np.float32) for h in hists]
    ck = rng.standard_normal((B, H, T, D), dtype=np.float32)
    cv = rng.standard_normal((B, H, T, D), dtype=np.float32)
    q = rng.standard_normal((B, hq, T, D), dtype=np.float32)
    if edit is not None:
        edit(ks, vs, ck, cv, q)
    seqs = []
    for b, h in enumerate(hists):
        s, so = cache.create_sequence(), pool.create_sequence()
        if h:
            cache.append_layer_major(s, [dev(ks[b][0])], [dev(vs[b][0])])
            pool.append_layer_major(so, RK(ks[b]), RV(vs[b]))
        seqs.append((s, so))
    batch = hx.DecodeBatch(cache, [s for s, _ in seqs], hq, max_tokens=max(hists) + T + 8)
    batch.prepare_chunk(T)
    out = torch.empty(B, hq, T, D, device="cuda:0")
    batch.append_layer(0, dev(ck), dev(cv))
    batch.prefill_layer(0, dev(q), dev(ck), dev(cv), out)
    torch.cuda.synchronize()
    kp, vp = pool.layer_pages(0)
    got = host(out)
    wants = []
    for b, (_, so) in enumerate(seqs):
        tab = np.array(pool.block_table(so), np.uint32)
        wants.append(oracle.paged_attention(q[b], kp, vp, tab, pool.length(so), RK(ck[b]),
                                            RV(cv[b]))[0])
    batch.close()
    return got, wants


def check(got, wants):
    for b, want in enumerate(wants):
        np.testing.assert_allclose(got[b], want, atol=ATOL, rtol=RTOL)


@pytest.mark.parametrize("page_dtype", ["f32", "bf16", "fp8"])
@pytest.mark.parametrize("hq", [4, 8, 16, 32])
def test_prefill_every_group_matches_oracle(device, page_dtype, hq):
    got, wants = run_prefill(page_dtype, hq, [0, 5, 16, 70, 300], 40, 11 + hq)
    check(got, wants)


@pytest.mark.parametrize("page_dtype", ["f32", "bf16", "fp8"])
def test_prefill_special_values_are_redone_exactly(device, page_dtype):
    """NaN key rows in a history (every row's scores NaN there), non-finite
    value rows at chunk positions 7 and 25 (rows before them must not see
    them: 0 * inf would leak NaN) and one value dim infinite (fp8: NaN) over
    a whole history page (every row's first maximum there has p = 1,
    whose middle and low bf16 terms are 0: the split gives 0 * inf = NaN
    where fp32 gives inf)."""
    bad = np.float32("nan") if page_dtype == "fp8" else np.float32("inf")

    def edit(ks, vs, ck, cv, q):
        ks[2][0, 1, 33, 5] = np.float32("nan")
        vs[1][0, 3, :16, 77] = bad
        cv[1, 0, 7, 100] = bad
        cv[3, 2, 25, :4] = bad

    got, wants = run_prefill(page_dtype, 16, [3, 40, 90, 16], 32, 5, edit)
    check(got, wants)


def test_prefill_infinite_bf16_key_with_zero_middle_query_term(device):
    """An infinite key element (bf16 holds inf) against query entries whose
    scaled value is exact in bf16: the split's middle term is zero, so the
    matrix cores give 0 * inf = NaN where fp32 gives inf; the exact redo
    must restore the fp32 result."""
    qs = np.float32(1.4426950408889634) / np.sqrt(np.float32(128.0))
    c = None
    for k in np.linspace(0.25, 4.0, 61, dtype=np.float32):
        cand = np.float32(k / qs)
        for _ in range(64):
            if (np.array(cand * qs, np.float32).view(np.uint32) & 0xFFFF) == 0:
                c = cand
                break
            cand = np.nextafter(cand, np.float32(np.inf), dtype=np.float32)
        if c is not None:
            break
    assert c is not None, "no query value with a zero middle bf16 term found"

    def edit(ks, vs, ck, cv, q):
        ks[1][0, 2, 17, 9] = np.float32("inf")
        q[1, 8:12, :, 9] = c  # kv head 2's four query heads

    got, wants = run_prefill("bf16", 16, [20, 50, 8], 24, 9, edit)
    check(got, wants)


@pytest.mark.parametrize("page_dtype", ["f32", "bf16", "fp8"])
def test_prefill_config5_shaped_chunk(device, page_dtype):
    """512-token chunks over histories of ~1000 tokens, 32 query and 8 kv
    heads: four position blocks per (sequence, kv head) in longest-first
    order."""
    got, wants = run_prefill(page_dtype, 32, [1000, 777, 1210], 512, 23, H=8)
    check(got, wants)


def test_prefill_every_fp8_code_in_history(device):
    """Every finite E4M3 code (subnormals, the largest values and both signs)
    in the history keys and values, each at several dims and heads: the
    staging moves the page codes to bf16 in hardware, which must keep every
    code value exact."""
    codes = np.array([c for c in range(256) if c & 0x7F != 0x7F], np.uint8)  # 254 codes
    vals = oracle.fp8_decode(codes)

    def edit(ks, vs, ck, cv, q):
        for b, (k, v) in enumerate(zip(ks, vs)):
            _, H, n, _ = k.shape
            idx = (np.arange(H)[:, None, None] * 7 + np.arange(n)[None, :, None] * D
                   + np.arange(D)[None, None, :] + 13 * b)
            k[0] = vals[idx % len(codes)] * np.float32(KS)
            v[0] = vals[(idx + 101) % len(codes)] * np.float32(VS)
        q *= np.float32(0.05)  # keys reach 448 * KS: keep the scores moderate

    got, wants = run_prefill("fp8", 16, [254, 300], 24, 31, edit)
    check(got, wants)


@pytest.mark.parametrize("page_dtype", ["bf16", "fp8"])
@pytest.mark.parametrize("T", [1, 31, 33, 64])
def test_prefill_chunk_lengths_across_key_blocks(device, page_dtype, T):
    """Chunks of 1, 31, 33 and 64 tokens over histories that end just before,
    on and just after a 32-key staging block (and one that ends mid-page),
    so the last block of each work item is partial in every way."""
    got, wants = run_prefill(page_dtype, 8, [31, 32, 33, 47, 64], T, 40 + T)
    check(got, wants)
