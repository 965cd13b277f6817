"""Every BASELINE decode configuration at its real size, on the GPU, against
the oracle (the C++ restatement of the reference's CPU paged attention,
src/attention/paged_reference.cpp:173-384; GQA as replicated MHA, the batch as
a per-sequence loop).

- config 1: exactly the tiny reference-shaped case (1 sequence, 4/4 heads,
  head_dim 16, 64-token history in 4 pages drawn by seeded permutation from
  an 8-page pool, one-token tail), outputs and probabilities;
- config 2: 8 MHA sequences of U[128, 2048] tokens, 32/32 heads;
- config 3: 64 sequences of log-uniform [512, 8192] tokens, 32/8 heads;
- config 4: 128 copy-on-write forks of a 1032-token root, suffixes
  U[64, 512]; the decode step attends the 64 shared pages once for the
  batch, so the cascade's prefix pass runs 4 query-row blocks per kv head.

Pages of every config are scattered over a pool whose free queue was
shuffled.  Tolerance: max-abs 2e-5 plus rel 1e-4."""

import numpy as np
import pytest
import torch

import helix_runtime_amd as hx
import oracle
import workloads

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-5, 1e-4
D = 128


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda:0")


def close(out, ref):
    np.testing.assert_allclose(out.cpu().numpy(), ref, atol=ATOL, rtol=RTOL)


def test_config1_tiny_reference_shape(device):
    rng = np.random.default_rng(1)
    table = rng.permutation(8)[:4].astype(np.uint32)
    kp = oracle.random_normal((8, 4, 16, 16), 11)
    vp = oracle.random_normal((8, 4, 16, 16), 12)
    q = oracle.random_normal((4, 1, 16), 13)
    tk = oracle.random_normal((4, 1, 16), 14)
    tv = oracle.random_normal((4, 1, 16), 15)
    out = torch.empty(4, 1, 16, device=device)
    ws = torch.empty(4, 1, 65, device=device)
    hx.paged_attention_with_tail_out(dev(q), dev(kp), dev(vp), dev(table.astype(np.int32)), 64,
                                     dev(tk), dev(tv), out, ws)
    torch.cuda.synchronize()
    exp_out, exp_ws = oracle.paged_attention(q, kp, vp, table, 64, tk, tv)
    close(out, exp_out)
    np.testing.assert_allclose(ws.cpu().numpy(), exp_ws, atol=2e-6, rtol=0)
    # The same case as a one-sequence batch through a cache and DecodeBatch
    # is impossible (head_dim 16): the batched entry points reject it.
    cache = hx.PagedKvCache(1, 4, 16, 16, 8)
    with pytest.raises(hx.HelixError) as e:
        hx.DecodeBatch(cache, [cache.create_sequence()], 4, max_tokens=80)
    assert e.value.status == hx.UNSUPPORTED


def run_steps(cache, seqs, hq, steps, seed, expect_shared=None):
    """`steps` decode steps through DecodeBatch (append and attention fused
    in one launch per layer), every layer checked against the oracle."""
    rng = np.random.default_rng(seed)
    B, H, L = len(seqs), cache.kv_heads, cache.layers
    max_tokens = max(cache.length(s) for s in seqs) + steps + 1
    batch = hx.DecodeBatch(cache, seqs, hq, max_tokens=max_tokens)
    try:
        for _ in range(steps):
            batch.prepare()
            if expect_shared is not None:
                assert batch.shared_pages() == expect_shared
            for layer in range(L):
                q = rng.standard_normal((B, hq, D), dtype=np.float32)
                tk = rng.standard_normal((B, H, D), dtype=np.float32)
                tv = rng.standard_normal((B, H, D), dtype=np.float32)
                # Pre-step pages: read before the fused append writes the token.
                kp, vp, tables, hist = workloads.oracle_inputs(cache, seqs, layer)
                hist = hist - 1  # prepare() already counts the step's token
                out = torch.empty(B, hq, D, device="cuda:0")
                batch.append_attention_layer(layer, dev(q), dev(tk), dev(tv), out)
                torch.cuda.synchronize()
                rtk = workloads.round_rows(cache, tk, cache.k_scale)
                rtv = workloads.round_rows(cache, tv, cache.v_scale)
                ref = oracle.batched_decode(q, kp, vp, tables, hist, rtk, rtv, threads=16)
                close(out, ref)
                # The fused append wrote the token into its slot.
                for b in (0, B - 1):
                    gk, gv = cache.retrieve_layer(seqs[b], layer)
                    np.testing.assert_array_equal(gk[:, -1].cpu().numpy(), rtk[b])
                    np.testing.assert_array_equal(gv[:, -1].cpu().numpy(), rtv[b])
                del kp, vp
    finally:
        batch.close()


def test_config2_mha_full_size(device):
    cache, seqs, hq = workloads.config2(layers=1)
    run_steps(cache, seqs, hq, steps=2, seed=20)
    cache.close()


@pytest.mark.parametrize("page_dtype", ["f32", "bf16", "fp8"])
def test_config3_gqa_full_size(device, page_dtype):
    """fp32 pages, and the reduced-precision extensions (bf16, fp8 E4M3 at
    scale 1): the oracle reads the pages' own values and the step rows
    rounded onto the page grid."""
    cache, seqs, hq = workloads.config3(layers=1, page_dtype=page_dtype)
    run_steps(cache, seqs, hq, steps=1, seed=30)
    cache.close()


@pytest.mark.parametrize("page_dtype", ["f32", "bf16", "fp8"])
def test_config4_prefix_sharing_full_size(device, page_dtype):
    cache, seqs, hq = workloads.config4(layers=1, steps=2, page_dtype=page_dtype)
    st = cache.stats()
    assert st["shared_blocks"] == 64
    run_steps(cache, seqs, hq, steps=2, seed=40, expect_shared=64)
    cache.close()
