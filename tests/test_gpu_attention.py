"""GPU paged attention against the CPU oracle.

Tolerance: the north-star bound, max-abs 2e-5 plus rel 1e-4, for outputs of
the batched decode kernel; the reference's own GPU-test bound 2e-5 + D * 1e-6
on outputs and 2e-6 on probabilities for the reference-shaped entry points
(tests/cuda_attention_test.cpp:227,270,441-443)."""

import math

import numpy as np
import pytest
import torch

import helix_runtime_amd as hx
import oracle

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-5, 1e-4


def dev(a, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a))
    if dtype is not None:
        t = t.to(dtype)
    return t.to("cuda:0")


def host(t):
    return t.detach().cpu().numpy()


def reversed_table(logical, physical):
    return np.array([physical - 1 - i for i in range(logical)], np.uint32)


def run_tail(q, kp, vp, table, hist, tk, tv):
    hq, t, _ = q.shape
    dv = vp.shape[-1]
    out = torch.empty(hq, t, dv, device="cuda:0")
    ws = torch.empty(hq, t, hist + t, device="cuda:0")
    tab = dev(table.astype(np.int32)) if len(table) else torch.zeros(1, dtype=torch.int32,
                                                                      device="cuda:0")
    hx.paged_attention_with_tail_out(dev(q), dev(kp), dev(vp), tab if len(table) else 0, hist,
                                     dev(tk), dev(tv), out, ws)
    torch.cuda.synchronize()
    return host(out), host(ws)


def run_history(q, kp, vp, table, kv_tokens, offset):
    hq, nq, _ = q.shape
    dv = vp.shape[-1]
    out = torch.empty(hq, nq, dv, device="cuda:0")
    ws = torch.empty(hq, nq, kv_tokens, device="cuda:0")
    hx.paged_attention_out(dev(q), dev(kp), dev(vp), dev(table.astype(np.int32)), kv_tokens,
                           offset, out, ws)
    torch.cuda.synchronize()
    return host(out), host(ws)


# ------------------------------------------------ reference-shaped API ----
def test_known_reordered_blocks_ignore_poisoned_padding(device):
    # tests/cuda_attention_test.cpp:196-228
    table = np.array([2, 0], np.uint32)
    q = np.array([[[1, 0], [0, 1]]], np.float32)
    k = np.array([[[1, 0], [0, 1], [1, 1]]], np.float32)
    v = np.array([[[10, 1, -1], [20, 2, -2], [30, 3, -3]]], np.float32)
    kp = oracle.pack_logical_blocks(k, table, 3, 2, 10000.0)
    vp = oracle.pack_logical_blocks(v, table, 3, 2, -10000.0)
    out, ws = run_history(q, kp, vp, table, 3, 1)
    exp_out, exp_ws = oracle.sdpa(q, k, v, 1)
    np.testing.assert_allclose(out, exp_out, atol=2e-5, rtol=0)
    np.testing.assert_allclose(ws, exp_ws, atol=2e-6, rtol=0)


@pytest.mark.parametrize("h,nq,nk,d,dv,p", [(1, 1, 3, 1, 2, 2), (2, 3, 5, 5, 7, 2),
                                             (3, 7, 11, 37, 41, 4)])
def test_history_odd_shapes(device, h, nq, nk, d, dv, p):
    # tests/cuda_attention_test.cpp:230-273 (seeds 8101-8103, padding +-77)
    logical = (nk - 1) // p + 1
    phys = logical + 2
    table = reversed_table(logical, phys)
    q = oracle.random_uniform((h, nq, d), 8101)
    k = oracle.random_uniform((h, nk, d), 8102)
    v = oracle.random_uniform((h, nk, dv), 8103)
    kp = oracle.pack_logical_blocks(k, table, phys, p, 77.0)
    vp = oracle.pack_logical_blocks(v, table, phys, p, -77.0)
    out, ws = run_history(q, kp, vp, table, nk, nk - nq)
    exp_out, exp_ws = oracle.paged_attention(q, kp, vp, table, nk, query_position_offset=nk - nq)
    np.testing.assert_allclose(out, exp_out, atol=2e-5 + d * 1e-6, rtol=0)
    np.testing.assert_allclose(ws, exp_ws, atol=2e-6, rtol=0)


@pytest.mark.parametrize("h,hist,tail,d,dv,p", [(1, 0, 1, 1, 2, 2), (2, 3, 1, 5, 7, 2),
                                                 (3, 5, 3, 37, 41, 4)])
def test_tail_odd_shapes(device, h, hist, tail, d, dv, p):
    # tests/cuda_attention_test.cpp:376-449 (seeds 8201-8205, padding +-10000)
    logical = 0 if hist == 0 else (hist - 1) // p + 1
    phys = logical + 2
    table = reversed_table(logical, phys)
    q = oracle.random_uniform((h, tail, d), 8201)
    hk = oracle.random_uniform((h, hist, d), 8202)
    hv = oracle.random_uniform((h, hist, dv), 8203)
    tk = oracle.random_uniform((h, tail, d), 8204)
    tv = oracle.random_uniform((h, tail, dv), 8205)
    kp = oracle.pack_logical_blocks(hk, table, phys, p, 1e4)
    vp = oracle.pack_logical_blocks(hv, table, phys, p, -1e4)
    out, ws = run_tail(q, kp, vp, table, hist, tk, tv)
    exp_out, exp_ws = oracle.paged_attention(q, kp, vp, table, hist, tk, tv)
    np.testing.assert_allclose(out, exp_out, atol=2e-5 + d * 1e-6, rtol=0)
    np.testing.assert_allclose(ws, exp_ws, atol=2e-6, rtol=0)


def test_tail_causal_mask_does_not_read_future_nan(device):
    # tests/cuda_attention_test.cpp:533-554
    nan = np.nan
    q = np.zeros((1, 2, 1), np.float32)
    kp = np.zeros((1, 1, 2, 1), np.float32)
    tk = np.array([[[0.0], [nan]]], np.float32)
    tv = np.array([[[3.0], [nan]]], np.float32)
    out, ws = run_tail(q, kp, kp, np.zeros(0, np.uint32), 0, tk, tv)
    assert out.ravel()[0] == 3.0 and np.isnan(out.ravel()[1])
    assert ws.ravel()[0] == 1.0 and ws.ravel()[1] == 0.0


def test_gqa_generic_matches_oracle(device):
    hq, hkv, d, p, hist, t = 8, 2, 24, 4, 19, 3
    logical = (hist - 1) // p + 1
    table = np.random.default_rng(3).permutation(logical + 3)[:logical].astype(np.uint32)
    kp = oracle.random_normal((logical + 3, hkv, p, d), 1)
    vp = oracle.random_normal((logical + 3, hkv, p, d), 2)
    q = oracle.random_normal((hq, t, d), 3)
    tk = oracle.random_normal((hkv, t, d), 4)
    tv = oracle.random_normal((hkv, t, d), 5)
    out, ws = run_tail(q, kp, vp, table, hist, tk, tv)
    exp_out, exp_ws = oracle.paged_attention(q, kp, vp, table, hist, tk, tv)
    np.testing.assert_allclose(out, exp_out, atol=ATOL, rtol=RTOL)
    np.testing.assert_allclose(ws, exp_ws, atol=2e-6, rtol=0)


def test_reference_contract_errors(device):
    # tests/cuda_attention_test.cpp:290-374 (the checks that survive the
    # pointer-and-size boundary)
    q = torch.zeros(1, 2, 2, device=device)
    kb = torch.zeros(3, 1, 2, 2, device=device)
    vb = torch.zeros(3, 1, 2, 2, device=device)
    out = torch.zeros(1, 2, 2, device=device)
    ws = torch.zeros(1, 2, 3, device=device)
    table = dev(np.array([2, 0], np.int32))
    lib = hx.load()
    base = dict(query=q, key_blocks=kb, value_blocks=vb, block_table=table)

    def call(kv_tokens=3, offset=1, output=out, workspace=ws, logical=2, key_blocks=kb,
             value_blocks=vb, query=q):
        return lib.helix_paged_attention_out(
            query.data_ptr(), query.shape[0], query.shape[1], query.shape[2],
            key_blocks.data_ptr(), value_blocks.data_ptr(), key_blocks.shape[0],
            key_blocks.shape[1], key_blocks.shape[2], value_blocks.shape[3], table.data_ptr(),
            logical, kv_tokens, offset, output.data_ptr(), workspace.data_ptr(),
            workspace.numel(), None)

    assert call() == 0
    assert call(logical=1) == hx.INVALID_ARGUMENT          # short table
    assert call(kv_tokens=0, offset=0, logical=0) == hx.INVALID_ARGUMENT
    assert call(offset=2) == hx.INVALID_ARGUMENT          # query range past the keys
    assert call(output=q) == hx.INVALID_ARGUMENT          # output aliases query
    ws5 = torch.zeros(1, 2, 3, device=device)
    assert call(output=ws5, workspace=ws5) == hx.INVALID_ARGUMENT
    assert call(workspace=torch.zeros(1, 2, 2, device=device)) == hx.INVALID_ARGUMENT
    torch.cuda.synchronize()
    bad = hx.PagedBlockTable([2, 0], 3)
    assert bad.logical_block_count == 2
    with pytest.raises(hx.HelixError) as e:
        hx.PagedBlockTable([3], 3)
    assert e.value.status == hx.OUT_OF_RANGE
    with pytest.raises(hx.HelixError):
        hx.PagedBlockTable([], 0)
    empty = hx.PagedBlockTable([], 3)
    assert empty.data() is None


def test_zero_queries_launch_nothing(device):
    # tests/cuda_attention_test.cpp:275-288
    q = torch.zeros(2, 0, 5, device=device)
    kb = torch.zeros(4, 2, 3, 5, device=device)
    vb = torch.zeros(4, 2, 3, 7, device=device)
    out = torch.zeros(2, 0, 7, device=device)
    ws = torch.zeros(2, 0, 7, device=device)
    table = dev(np.array([3, 1, 0], np.int32))
    hx.paged_attention_out(q, kb, vb, table, 7, 7, out, ws)
    n = ctypes_size()
    assert hx.load().helix_paged_score_workspace_bytes(2, 0, 2, 4, 3, 3, 7, n) == 0
    assert n._obj.value == 0


def ctypes_size():
    import ctypes
    return ctypes.byref(ctypes.c_size_t())


# -------------------------------------------------------- batched decode ----
def make_decode_problem(seed, batch, hq, hkv, lengths, spare=1.25, d=128, p=16):
    rng = np.random.default_rng(seed)
    pages = [(int(n) + p - 1) // p for n in lengths]
    need = sum(pages)
    n_phys = max(1, int(math.ceil(need * spare)))
    perm = rng.permutation(n_phys).astype(np.uint32)
    max_blocks = max(1, max(pages))
    tables = np.zeros((batch, max_blocks), np.uint32)
    off = 0
    for b in range(batch):
        tables[b, : pages[b]] = perm[off: off + pages[b]]
        off += pages[b]
    kp = rng.standard_normal((n_phys, hkv, p, d), dtype=np.float32)
    vp = rng.standard_normal((n_phys, hkv, p, d), dtype=np.float32)
    q = rng.standard_normal((batch, hq, d), dtype=np.float32)
    tk = rng.standard_normal((batch, hkv, d), dtype=np.float32)
    tv = rng.standard_normal((batch, hkv, d), dtype=np.float32)
    return q, kp, vp, tables, np.asarray(lengths, np.int32), tk, tv


def run_decode(q, kp, vp, tables, lengths, tk, tv, pages_per_split=0, ws=None):
    b, hq, d = q.shape
    out = torch.empty(b, hq, d, device="cuda:0")
    if ws is None:
        ws = hx.decode_workspace(b, hq, kp.shape[1], tables.shape[1], pages_per_split)
    hx.paged_decode_attention(dev(q), dev(kp), dev(vp), dev(tables.astype(np.int32)),
                              dev(lengths), dev(tk), dev(tv), out, ws, pages_per_split)
    torch.cuda.synchronize()
    return host(out)


@pytest.mark.parametrize("hq,hkv", [(4, 4), (8, 4), (32, 8), (64, 8)])
def test_decode_groups_match_oracle(device, hq, hkv):
    lengths = [0, 1, 15, 16, 17, 100, 255, 256, 1000]
    prob = make_decode_problem(7, len(lengths), hq, hkv, lengths)
    out = run_decode(*prob)
    ref = oracle.batched_decode(*prob, threads=8)
    np.testing.assert_allclose(out, ref, atol=ATOL, rtol=RTOL)


@pytest.mark.parametrize("split", [1, 2, 3, 8, 64, 0])
def test_decode_split_sizes_agree(device, split):
    lengths = [5, 33, 160, 481, 1500, 2049]
    prob = make_decode_problem(11, len(lengths), 32, 8, lengths)
    out = run_decode(*prob, pages_per_split=split)
    ref = oracle.batched_decode(*prob, threads=8)
    np.testing.assert_allclose(out, ref, atol=ATOL, rtol=RTOL)


def test_config2_llama2_mha_decode(device):
    # B8, 32/32 heads, D128, P16, ctx ~U[128, 2048], pool 1.25x.
    rng = np.random.default_rng(2)
    lengths = rng.integers(128, 2049, size=8)
    prob = make_decode_problem(2, 8, 32, 32, lengths)
    out = run_decode(*prob)
    ref = oracle.batched_decode(*prob, threads=8)
    np.testing.assert_allclose(out, ref, atol=ATOL, rtol=RTOL)


def test_config3_shape_sampled_decode(device):
    # BASELINE config 3 shape (32/8 heads, ctx log-uniform [512, 8192]) on 8 sequences.
    rng = np.random.default_rng(3)
    lengths = np.exp(rng.uniform(np.log(512), np.log(8192), size=8)).astype(np.int64)
    prob = make_decode_problem(3, 8, 32, 8, lengths)
    out = run_decode(*prob)
    ref = oracle.batched_decode(*prob, threads=8)
    np.testing.assert_allclose(out, ref, atol=ATOL, rtol=RTOL)


def test_decode_is_deterministic_and_workspace_reusable(device):
    # The per-unit arrival counters reset themselves: repeated calls on one
    # workspace give bit-identical results.
    prob = make_decode_problem(5, 4, 32, 8, [700, 3000, 64, 1])
    ws = hx.decode_workspace(4, 32, 8, prob[3].shape[1], 4)
    runs = [run_decode(*prob, pages_per_split=4, ws=ws) for _ in range(3)]
    assert np.array_equal(runs[0], runs[1]) and np.array_equal(runs[1], runs[2])
    np.testing.assert_allclose(runs[0], oracle.batched_decode(*prob), atol=ATOL, rtol=RTOL)


def test_decode_special_values_follow_reference_softmax(device):
    # src/kernels/cpu/reference.cpp:264-316 -- +inf scores share the mass,
    # NaN scores poison the row, out-of-range pages give NaN.
    q, kp, vp, tables, lengths, tk, tv = make_decode_problem(9, 4, 4, 4, [40, 40, 40, 40])
    q[:] = 1.0
    kp = kp.copy()
    # sequence 0 head 0: two +inf keys (tokens 3 and 20)
    for tok in (3, 20):
        kp[tables[0, tok // 16], 0, tok % 16, 0] = np.inf
        kp[tables[0, tok // 16], 0, tok % 16, 1:] = 0.0
    # sequence 1 head 1: a NaN key at token 30
    kp[tables[1, 30 // 16], 1, 30 % 16, 5] = np.nan
    # sequence 2: a corrupt page ID
    tables = tables.copy()
    tables[2, 1] = 10_000
    out = run_decode(q, kp, vp, tables, lengths, tk, tv)
    tables_ok = tables.copy()
    tables_ok[2, 1] = tables[3, 0]
    ref = oracle.batched_decode(q, kp, vp, tables_ok, lengths, tk, tv)
    expected0 = 0.5 * (vp[tables[0, 0], 0, 3] + vp[tables[0, 1], 0, 4])
    np.testing.assert_allclose(out[0, 0], expected0, atol=ATOL, rtol=RTOL)
    np.testing.assert_allclose(ref[0, 0], expected0, atol=ATOL, rtol=RTOL)
    assert np.isnan(out[1, 1]).all() and np.isnan(ref[1, 1]).all()
    assert np.isnan(out[2]).all()
    np.testing.assert_allclose(out[3], ref[3], atol=ATOL, rtol=RTOL)
    np.testing.assert_allclose(out[1, [0, 2, 3]], ref[1, [0, 2, 3]], atol=ATOL, rtol=RTOL)


def test_decode_rejects_bad_arguments(device):
    q, kp, vp, tables, lengths, tk, tv = make_decode_problem(1, 2, 12, 4, [10, 20])
    with pytest.raises(hx.HelixError) as e:
        run_decode(q, kp, vp, tables, lengths, tk, tv)  # group of 3
    assert e.value.status == hx.UNSUPPORTED
    q, kp, vp, tables, lengths, tk, tv = make_decode_problem(1, 2, 8, 4, [10, 20])
    out = torch.empty(2, 8, 128, device=device)
    small = torch.empty(4, device=device)
    with pytest.raises(hx.HelixError):
        hx.paged_decode_attention(dev(q), dev(kp), dev(vp), dev(tables.astype(np.int32)),
                                  dev(lengths), dev(tk), dev(tv), out, small, 1)


# ------------------------------ reference-shaped entry, single-sequence decode route ----
# One query row per head at head_dim 128 and 16-token pages (the reference
# model's per-layer call, src/model/cuda_llama.cpp:361-367) runs the
# single-sequence decode kernel; the score workspace still ends up holding the
# softmax probabilities, as the reference's contract says
# (tests/cuda_attention_test.cpp:441-443).  Outputs within 2e-5 + 1e-4 rel
# of the oracle, probabilities within the reference's 2e-6.
PROB_ATOL = 2e-6


def single_decode_problem(seed, hkv, g, hist, spare=3):
    rng = np.random.default_rng(seed)
    logical = (hist + 15) // 16
    phys = logical + spare
    table = rng.permutation(phys)[:logical].astype(np.uint32)
    kp = rng.standard_normal((phys, hkv, 16, 128), dtype=np.float32)
    vp = rng.standard_normal((phys, hkv, 16, 128), dtype=np.float32)
    q = rng.standard_normal((hkv * g, 1, 128), dtype=np.float32)
    tk = rng.standard_normal((hkv, 1, 128), dtype=np.float32)
    tv = rng.standard_normal((hkv, 1, 128), dtype=np.float32)
    return table, kp, vp, q, tk, tv


def run_single(q, kp, vp, table, hist, tk, tv, stream=None, probabilities=False, ws_fill=7.0):
    out = torch.full((q.shape[0], 1, 128), 5.0, device="cuda:0")
    ws = torch.full((q.shape[0], 1, hist + 1), ws_fill, device="cuda:0")
    tab = dev(table.astype(np.int32)) if len(table) else 0
    args = (dev(q), dev(kp), dev(vp), tab, hist, dev(tk), dev(tv), out, ws)
    torch.cuda.synchronize()  # the inputs are ready for a call on another stream
    hx.paged_attention_with_tail_out(*args, stream=stream, probabilities=probabilities)
    torch.cuda.synchronize()
    return host(out), host(ws)


@pytest.mark.parametrize("hkv,g", [(8, 4), (32, 1), (4, 2), (2, 8)])
@pytest.mark.parametrize("hist", [0, 1, 15, 16, 150, 257, 1000, 2770, 8192])
def test_with_tail_decode_route_matches_oracle(device, hkv, g, hist):
    """Output and probabilities against the oracle for every query group and
    history lengths around page edges; a second call on the same buffers is
    bit-identical (the kernel's per-kv-head tickets reset themselves), and
    the exact probability variant agrees."""
    table, kp, vp, q, tk, tv = single_decode_problem(hist + 7 * g, hkv, g, hist)
    exp_out, exp_ws = oracle.paged_attention(q, kp, vp, table, hist, tk, tv)
    out, ws = run_single(q, kp, vp, table, hist, tk, tv)
    np.testing.assert_allclose(out, exp_out, atol=ATOL, rtol=RTOL)
    np.testing.assert_allclose(ws, exp_ws, atol=PROB_ATOL, rtol=0)
    out2, ws2 = run_single(q, kp, vp, table, hist, tk, tv, ws_fill=-3.0)
    np.testing.assert_array_equal(out2, out)
    np.testing.assert_array_equal(ws2, ws)
    if hist <= 1000:
        out3, ws3 = run_single(q, kp, vp, table, hist, tk, tv, probabilities=True)
        np.testing.assert_allclose(out3, exp_out, atol=2e-5 + 128e-6, rtol=0)
        np.testing.assert_allclose(ws3, exp_ws, atol=PROB_ATOL, rtol=0)


@pytest.mark.parametrize("kv,offset", [(1, 0), (40, 0), (40, 17), (1000, 999), (1000, 500),
                                       (3001, 1234)])
def test_history_decode_route_matches_oracle(device, kv, offset):
    """paged_scaled_dot_product_attention_out with one query row at position
    `offset` of kv_tokens keys: keys past the position get probability 0."""
    table, kp, vp, q, _, _ = single_decode_problem(kv + offset, 8, 4, kv)
    exp_out, exp_ws = oracle.paged_attention(q, kp, vp, table, kv, query_position_offset=offset)
    out = torch.full((32, 1, 128), 5.0, device=device)
    ws = torch.full((32, 1, kv), 7.0, device=device)
    hx.paged_attention_out(dev(q), dev(kp), dev(vp), dev(table.astype(np.int32)), kv, offset,
                           out, ws)
    torch.cuda.synchronize()
    np.testing.assert_allclose(host(out), exp_out, atol=ATOL, rtol=RTOL)
    np.testing.assert_allclose(host(ws), exp_ws, atol=PROB_ATOL, rtol=0)


def test_decode_route_special_values(device):
    """The reference softmax rules on the single-sequence decode route
    (src/kernels/cpu/reference.cpp:264-316): +inf scores share the mass, a
    NaN score makes its row NaN, other rows are untouched."""
    hist = 700
    table, kp, vp, q, tk, tv = single_decode_problem(41, 8, 4, hist)
    kp = kp.copy()
    q[:, 0, :] = np.abs(q[:, 0, :]) + 0.1
    for tok in (3, 650):  # kv head 0: two +inf keys
        kp[table[tok // 16], 0, tok % 16, :] = np.inf
    kp[table[321 // 16], 2, 321 % 16, 9] = np.nan  # kv head 2: one NaN key element
    exp_out, exp_ws = oracle.paged_attention(q, kp, vp, table, hist, tk, tv)
    out, ws = run_single(q, kp, vp, table, hist, tk, tv)
    assert np.isnan(out[8:12]).all() and np.isnan(ws[8:12]).all()
    assert (ws[0:4, 0, 3] == 0.5).all() and (ws[0:4, 0, 650] == 0.5).all()
    np.testing.assert_allclose(out, exp_out, atol=ATOL, rtol=RTOL)
    np.testing.assert_allclose(ws, exp_ws, atol=PROB_ATOL, rtol=0)


def test_with_tail_decode_route_bad_page_is_nan(device):
    """A page ID past the pool yields NaN output and probabilities, and is
    never dereferenced (cuda_paged.cu:58-61); other kv heads are unaffected
    only through the output shape (the reference poisons the whole call's
    rows that read the page: every kv head reads it)."""
    hist = 1000
    table, kp, vp, q, tk, tv = single_decode_problem(5, 8, 4, hist)
    table = table.copy()
    table[17] = kp.shape[0] + 5
    out, ws = run_single(q, kp, vp, table, hist, tk, tv)
    assert np.isnan(out).all() and np.isnan(ws).all()


def test_decode_route_calls_on_two_streams_and_changing_sizes(device):
    """Alternating history lengths on one stream, then the same calls on a
    second stream: each call's scratch (partials and tickets) is its
    stream's own and left clean for the next call."""
    s2 = torch.cuda.Stream()
    cases = [single_decode_problem(60 + i, 8, 4, h) + (h,) for i, h in
             enumerate([5000, 40, 8192, 700, 0, 3333])]
    for stream in (None, s2):
        for table, kp, vp, q, tk, tv, hist in cases:
            exp_out, exp_ws = oracle.paged_attention(q, kp, vp, table, hist, tk, tv)
            out, ws = run_single(q, kp, vp, table, hist, tk, tv, stream=stream)
            np.testing.assert_allclose(out, exp_out, atol=ATOL, rtol=RTOL)
            np.testing.assert_allclose(ws, exp_ws, atol=PROB_ATOL, rtol=0)


def test_with_tail_decode_route_config3_batch_as_calls(device):
    """The reference's one-call-per-sequence flow at config-3 shape (8 of
    the 64 sequences, contexts log-uniform in [512, 8192]) through the
    reference-shaped entry point matches the oracle."""
    rng = np.random.default_rng(33)
    for i in range(8):
        hist = int(np.exp(rng.uniform(math.log(512), math.log(8192))))
        table, kp, vp, q, tk, tv = single_decode_problem(300 + i, 8, 4, hist)
        exp_out, exp_ws = oracle.paged_attention(q, kp, vp, table, hist, tk, tv)
        out, ws = run_single(q, kp, vp, table, hist, tk, tv)
        np.testing.assert_allclose(out, exp_out, atol=ATOL, rtol=RTOL)
        np.testing.assert_allclose(ws, exp_ws, atol=PROB_ATOL, rtol=0)


# ------------------------------ reference-shaped entry, matrix-core chunk route ----
# Several query rows at head_dim 128 and 16-token pages (the reference's
# chunked-prefill call through the same entry points) run the exact fp32
# matrix-core prefill kernel, which also leaves the probabilities.
def chunk_problem(seed, hkv, g, hist, T, spare=3):
    rng = np.random.default_rng(seed)
    logical = (hist + 15) // 16
    phys = logical + spare
    table = rng.permutation(phys)[:logical].astype(np.uint32)
    kp = rng.standard_normal((phys, hkv, 16, 128), dtype=np.float32)
    vp = rng.standard_normal((phys, hkv, 16, 128), dtype=np.float32)
    q = rng.standard_normal((hkv * g, T, 128), dtype=np.float32)
    tk = rng.standard_normal((hkv, T, 128), dtype=np.float32)
    tv = rng.standard_normal((hkv, T, 128), dtype=np.float32)
    return table, kp, vp, q, tk, tv


def run_chunk(q, kp, vp, table, hist, tk, tv, probabilities=False):
    hq, T, _ = q.shape
    out = torch.full((hq, T, 128), 5.0, device="cuda:0")
    ws = torch.full((hq, T, hist + T), 7.0, device="cuda:0")
    tab = dev(table.astype(np.int32)) if len(table) else 0
    hx.paged_attention_with_tail_out(dev(q), dev(kp), dev(vp), tab, hist, dev(tk), dev(tv), out,
                                     ws, probabilities=probabilities)
    torch.cuda.synchronize()
    return host(out), host(ws)


@pytest.mark.parametrize("T,hist", [(2, 0), (2, 1000), (2, 4096), (37, 0), (37, 1000),
                                    (37, 4096), (512, 0), (512, 1000), (512, 4096)])
def test_with_tail_chunk_route_matches_oracle(device, T, hist):
    """Config-5 geometry (32 query / 8 kv heads) chunks of 2, 37 and 512 rows
    over histories of 0, 1000 and 4096 tokens: outputs and the probability
    workspace against the oracle."""
    table, kp, vp, q, tk, tv = chunk_problem(T * 7 + hist, 8, 4, hist, T)
    exp_out, exp_ws = oracle.paged_attention(q, kp, vp, table, hist, tk, tv)
    out, ws = run_chunk(q, kp, vp, table, hist, tk, tv)
    np.testing.assert_allclose(out, exp_out, atol=ATOL, rtol=RTOL)
    np.testing.assert_allclose(ws, exp_ws, atol=PROB_ATOL, rtol=0)


@pytest.mark.parametrize("hkv,g", [(32, 1), (4, 2), (2, 8)])
def test_with_tail_chunk_route_every_group(device, hkv, g):
    table, kp, vp, q, tk, tv = chunk_problem(90 + g, hkv, g, 333, 70)
    exp_out, exp_ws = oracle.paged_attention(q, kp, vp, table, 333, tk, tv)
    out, ws = run_chunk(q, kp, vp, table, 333, tk, tv)
    np.testing.assert_allclose(out, exp_out, atol=ATOL, rtol=RTOL)
    np.testing.assert_allclose(ws, exp_ws, atol=PROB_ATOL, rtol=0)
    out2, ws2 = run_chunk(q, kp, vp, table, 333, tk, tv, probabilities=True)
    np.testing.assert_allclose(out2, exp_out, atol=2e-5 + 128e-6, rtol=0)
    np.testing.assert_allclose(ws2, ws, atol=PROB_ATOL, rtol=0)


@pytest.mark.parametrize("kv,offset,nq", [(40, 0, 40), (300, 100, 37), (1000, 488, 512),
                                          (2000, 16, 2), (700, 650, 50)])
def test_history_chunk_route_matches_oracle(device, kv, offset, nq):
    """paged_scaled_dot_product_attention_out with several query rows at
    positions offset .. offset + nq - 1 of kv_tokens keys: the rows' own
    keys come from the pages, keys past a row's position get 0."""
    table, kp, vp, q, _, _ = chunk_problem(kv + offset + nq, 8, 4, kv, nq)
    exp_out, exp_ws = oracle.paged_attention(q, kp, vp, table, kv, query_position_offset=offset)
    out = torch.full((32, nq, 128), 5.0, device=device)
    ws = torch.full((32, nq, kv), 7.0, device=device)
    hx.paged_attention_out(dev(q), dev(kp), dev(vp), dev(table.astype(np.int32)), kv, offset,
                           out, ws)
    torch.cuda.synchronize()
    np.testing.assert_allclose(host(out), exp_out, atol=ATOL, rtol=RTOL)
    np.testing.assert_allclose(host(ws), exp_ws, atol=PROB_ATOL, rtol=0)


def test_chunk_route_special_values(device):
    """+inf and NaN keys in the history, a non-finite value row in the chunk
    that earlier rows mask, and a bad page ID in a second call."""
    hist, T = 300, 40
    table, kp, vp, q, tk, tv = chunk_problem(17, 8, 4, hist, T)
    kp = kp.copy()
    q[:4] = np.abs(q[:4]) + 0.1
    for tok in (7, 250):  # kv head 0: two +inf keys every row sees
        kp[table[tok // 16], 0, tok % 16, :] = np.inf
    kp[table[100 // 16], 3, 100 % 16, 2] = np.nan  # kv head 3: NaN rows
    tv[5, 20, 7] = np.inf                           # kv head 5: rows 0-19 must not see it
    exp_out, exp_ws = oracle.paged_attention(q, kp, vp, table, hist, tk, tv)
    out, ws = run_chunk(q, kp, vp, table, hist, tk, tv)
    assert np.isnan(out[12:16]).all() and np.isnan(ws[12:16]).all()
    assert np.isfinite(out[20:24, :20]).all()
    np.testing.assert_allclose(out, exp_out, atol=ATOL, rtol=RTOL)
    np.testing.assert_allclose(ws, exp_ws, atol=PROB_ATOL, rtol=0)
    table = table.copy()
    table[5] = kp.shape[0] + 9
    out, ws = run_chunk(q, kp, vp, table, hist, tk, tv)
    assert np.isnan(out).all() and np.isnan(ws).all()


def test_reference_routes_seeded_random_calls(device):
    """Seeded random calls of both reference-shaped entry points at head_dim
    128 and 16-token pages: query groups 1/2/4/8, one or several query rows,
    histories from 0 (tail form) or offsets anywhere in the keys (history
    form), so every route (single-sequence decode with and without a merge,
    matrix-core chunk with its key ranges, the gathered-chunk history form)
    meets ragged edges; outputs and probabilities against the oracle."""
    rng = np.random.default_rng(2024)
    for case in range(24):
        g = int(rng.choice([1, 2, 4, 8]))
        hkv = int(rng.choice([1, 2, 4, 8])) if g < 8 else int(rng.choice([1, 2, 4]))
        T = int(rng.choice([1, 1, 2, 3, 17, 64, 130]))
        tail_form = case % 2 == 0
        hist = int(rng.integers(0, 1500))
        print(f"case {case}: g={g} hkv={hkv} T={T} hist={hist} tail={tail_form}", flush=True)
        if tail_form:
            table, kp, vp, q, tk, tv = chunk_problem(7000 + case, hkv, g, hist, T)
            exp_out, exp_ws = oracle.paged_attention(q, kp, vp, table, hist, tk, tv)
            out, ws = run_chunk(q, kp, vp, table, hist, tk, tv)
        else:
            kv = hist + T + int(rng.integers(0, 40))
            offset = int(rng.integers(0, kv - T + 1))
            table, kp, vp, q, _, _ = chunk_problem(7000 + case, hkv, g, kv, T)
            exp_out, exp_ws = oracle.paged_attention(q, kp, vp, table, kv,
                                                     query_position_offset=offset)
            o = torch.full((hkv * g, T, 128), 5.0, device=device)
            w = torch.full((hkv * g, T, kv), 7.0, device=device)
            hx.paged_attention_out(dev(q), dev(kp), dev(vp), dev(table.astype(np.int32)), kv,
                                   offset, o, w)
            torch.cuda.synchronize()
            out, ws = host(o), host(w)
        np.testing.assert_allclose(out, exp_out, atol=ATOL, rtol=RTOL, err_msg=f"case {case}")
        np.testing.assert_allclose(ws, exp_ws, atol=PROB_ATOL, rtol=0, err_msg=f"case {case}")


def test_reference_routes_from_four_host_threads_on_their_own_streams(device):
    """Four host threads, each issuing decode and chunk calls of changing
    sizes on its own stream: every stream gets its own route scratch
    (grown as its calls grow), so the calls never share partials and all
    results match the oracle."""
    import threading

    cases = []
    for i in range(8):
        T = [1, 40, 1, 3][i % 4]
        hist = [900, 300, 4000, 17][i % 4] + 13 * i
        table, kp, vp, q, tk, tv = chunk_problem(8800 + i, 8, 4, hist, T)
        exp_out, exp_ws = oracle.paged_attention(q, kp, vp, table, hist, tk, tv)
        args = (dev(q), dev(kp), dev(vp), dev(table.astype(np.int32)), hist, dev(tk), dev(tv))
        cases.append((args, hist, T, exp_out, exp_ws))
    torch.cuda.synchronize()
    results = {}
    errors = []

    def worker(w):
        try:
            stream = torch.cuda.Stream()
            outs = []
            with torch.cuda.stream(stream):
                for rep in range(3):
                    for i in range(w, len(cases) + w):
                        args, hist, T, _, _ = cases[i % len(cases)]
                        o = torch.empty(32, T, 128, device="cuda:0")
                        s = torch.empty(32, T, hist + T, device="cuda:0")
                        hx.paged_attention_with_tail_out(*args, o, s, stream=stream)
                        outs.append((i % len(cases), o, s))
            stream.synchronize()
            results[w] = outs
        except Exception as e:  # reported below
            errors.append(repr(e))

    threads = [threading.Thread(target=worker, args=(w,)) for w in range(4)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert errors == []
    for w, outs in results.items():
        for i, o, s in outs:
            _, _, _, exp_out, exp_ws = cases[i]
            np.testing.assert_allclose(host(o), exp_out, atol=ATOL, rtol=RTOL,
                                       err_msg=f"thread {w} case {i}")
            np.testing.assert_allclose(host(s), exp_ws, atol=PROB_ATOL, rtol=0,
                                       err_msg=f"thread {w} case {i}")
