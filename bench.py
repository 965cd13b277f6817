"""Benchmark of the paged-KV hot path on one MI355X.

Default workload: Llama-3-8B-shaped GQA decode across all
32 layers, batch 64, 32 query / 8 KV heads, head_dim 128, 16-token pages,
context lengths log-uniform in [512, 8192], physical pages shuffled across
the pool, float32 K/V/Q ~ N(0, 1).  One step = reserve one slot per sequence,
then per layer: append the current K/V token into its page and run paged
decode attention over the pre-step history plus that uncommitted tail.

Printed JSON line: ``value`` is the whole step's algorithmic bytes (decode
attention + append, all layers) divided by the wall time of a step.  The
``roofline`` object is the decode attention kernel's own rate, timed with HIP
events on the stream the kernels run on.  ``cpu_baseline`` times the CPU
oracle (the C++ restatement of the reference's CPU paged attention) on a
bounded sample of the same workload on this host's cores.
"""

from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import sys
import time

import numpy as np
import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

import helix_runtime_amd as hx  # noqa: E402

HBM_PEAK_GBPS = 8000.0
LAYERS, HQ, HKV, D, P, BATCH = 32, 32, 8, 128, 16, 64
# Page element type (--page-dtype): "f32" is the reference's format and the
# headline; "bf16" and "fp8" (E4M3, scales 1) are the reduced-precision
# extension.
PAGE_DTYPE, PAGE_BYTES = "f32", 4


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def decode_bytes(lengths, hq=None, hkv=None, d=D, p=P):
    """Algorithmic HBM bytes of one decode-attention launch (one layer):
    sum over sequences of K+V history (each byte once per KV head), the K/V
    tail, Q in and O out, and the block-table entries."""
    hq, hkv = hq or HQ, hkv or HKV
    lengths = np.asarray(lengths, np.int64)
    return int(np.sum(2 * hkv * lengths * d * PAGE_BYTES + 2 * hkv * d * 4 + 2 * hq * d * 4 +
                      ((lengths + p - 1) // p) * 4))


def append_bytes(batch, hkv=None, d=D):
    """Read the fp32 source row + write the page row, keys and values, one
    token per sequence."""
    hkv = hkv or HKV
    return 2 * hkv * d * (4 + PAGE_BYTES) * batch


def append_write_bytes(batch, hkv=None, d=D):
    """The page writes of append_bytes alone."""
    hkv = hkv or HKV
    return 2 * hkv * d * PAGE_BYTES * batch


def build_workload(seed, batch, layers, steps_total, shuffle=True, config=3):
    """Config 3: contexts log-uniform in [512, 8192], pool sized to the need.
    Config 2: contexts uniform in [128, 2048], pool 1.25x the need."""
    rng = np.random.default_rng(seed)
    if config == 2:
        lengths = rng.integers(128, 2049, size=batch).astype(np.int64)
    else:
        lengths = np.exp(rng.uniform(math.log(512), math.log(8192), size=batch)).astype(np.int64)
    pages = (lengths + P - 1) // P
    grow = (steps_total + P) // P + 1
    n_phys = int(pages.sum() + batch * grow + 16)
    if config == 2:
        n_phys = int(math.ceil(1.25 * n_phys))
    cache = hx.PagedKvCache(layers, HKV, D, P, n_phys, page_dtype=PAGE_DTYPE)
    log(f"pool: {n_phys} blocks x {layers} layers "
        f"({n_phys * layers * 2 * HKV * P * D * PAGE_BYTES / 1e9:.1f} GB)")
    # Shuffle the free queue: allocate every block once, release in a seeded
    # random order, so later allocations scatter each sequence over the pool.
    tok = torch.zeros(layers, HKV, D, device="cuda:0")
    dummies = []
    for _ in range(n_phys if shuffle else 0):
        s = cache.create_sequence()
        cache.append(s, tok, tok)
        dummies.append(s)
    for i in rng.permutation(len(dummies)):
        cache.release_sequence(dummies[int(i)])
    # Fill the histories with N(0, 1) data in one bulk append per sequence.
    gen = torch.Generator(device="cuda:0")
    gen.manual_seed(seed)
    src_elems = HKV * int(lengths.max()) * D
    src_k = torch.randn(layers, src_elems + 4096, device="cuda:0", generator=gen)
    src_v = torch.randn(layers, src_elems + 4096, device="cuda:0", generator=gen)
    seqs = []
    for b in range(batch):
        s = cache.create_sequence()
        n = int(lengths[b])
        off = int(rng.integers(0, 1024)) * 4
        lk = [src_k[l, off: off + HKV * n * D].view(HKV, n, D) for l in range(layers)]
        lv = [src_v[l, off: off + HKV * n * D].view(HKV, n, D) for l in range(layers)]
        cache.append_layer_major(s, lk, lv)
        seqs.append(s)
    del src_k, src_v
    torch.cuda.empty_cache()
    return cache, seqs, lengths


PREFIX_BATCH, PREFIX_TOKENS, PREFIX_PARTIAL = 128, 1024, 8


def build_prefix_workload(seed, layers, steps_total):
    """Config 4: 128 sequences share a 1024-token prefix (64 full pages at
    refcount 128) plus an 8-token partial page that every fork copies on
    write, so each sequence's first suffix token lands mid-page in its own
    copy; then unique suffixes of uniform [64, 512] tokens."""
    rng = np.random.default_rng(seed + 40)
    root_len = PREFIX_TOKENS + PREFIX_PARTIAL
    suffix = rng.integers(64, 513, size=PREFIX_BATCH)
    own_pages = (PREFIX_PARTIAL + suffix + steps_total + P - 1) // P + 1
    n_phys = int(root_len // P + 1 + own_pages.sum() + 16)
    cache = hx.PagedKvCache(layers, HKV, D, P, n_phys, page_dtype=PAGE_DTYPE)
    log(f"pool: {n_phys} blocks x {layers} layers "
        f"({n_phys * layers * 2 * HKV * P * D * PAGE_BYTES / 1e9:.1f} GB)")
    tok = torch.zeros(layers, HKV, D, device="cuda:0")
    dummies = []
    for _ in range(n_phys):
        s = cache.create_sequence()
        cache.append(s, tok, tok)
        dummies.append(s)
    for i in rng.permutation(len(dummies)):
        cache.release_sequence(dummies[int(i)])
    gen = torch.Generator(device="cuda:0")
    gen.manual_seed(seed)
    n_src = HKV * max(root_len, int(suffix.max())) * D + 4096
    src_k = torch.randn(layers, n_src, device="cuda:0", generator=gen)
    src_v = torch.randn(layers, n_src, device="cuda:0", generator=gen)

    def rows(src, n, off):
        return [src[l, off: off + HKV * n * D].view(HKV, n, D) for l in range(layers)]

    root = cache.create_sequence()
    cache.append_layer_major(root, rows(src_k, root_len, 0), rows(src_v, root_len, 0))
    seqs = [cache.fork_sequence(root, root_len, allow_cow=True) for _ in range(PREFIX_BATCH)]
    cache.release_sequence(root)
    for b, s in enumerate(seqs):
        off = int(rng.integers(0, 1024)) * 4
        n = int(suffix[b])
        cache.append_layer_major(s, rows(src_k, n, off), rows(src_v, n, off))
    del src_k, src_v
    torch.cuda.empty_cache()
    lengths = np.array([cache.length(s) for s in seqs], np.int64)
    st = cache.stats()
    log(f"prefix workload: shared blocks {st['shared_blocks']}, "
        f"block references {st['block_reference_count']}")
    return cache, seqs, lengths


def unique_decode_bytes(lengths, shared_tokens=PREFIX_TOKENS, hq=None, hkv=None, d=D, p=P):
    """HBM bytes of one config-4 decode launch when every shared prefix page
    is read from HBM once: the logical formula with the shared tokens counted
    once instead of once per sequence."""
    hq, hkv = hq or HQ, hkv or HKV
    lengths = np.asarray(lengths, np.int64)
    shared = 2 * hkv * shared_tokens * d * PAGE_BYTES
    own = 2 * hkv * (lengths - shared_tokens) * d * PAGE_BYTES
    return int(shared + np.sum(own + 2 * hkv * d * 4 + 2 * hq * d * 4 +
                               ((lengths + p - 1) // p) * 4))


# Worker threads of the CPU baseline: one per host core this process may use,
# at most the GPU box's CPU share per GPU (16; the box may report more cores
# than one job is given).
CPU_SHARE = 16


def host_cpu():
    """The host the CPU baseline runs on: logical CPUs, the CPUs this process
    may run on, the CPU model, and the thread count the baseline uses."""
    nproc = os.cpu_count() or 1
    try:
        usable = len(os.sched_getaffinity(0))
    except AttributeError:  # pragma: no cover
        usable = nproc
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:  # pragma: no cover
        pass
    return {"nproc": nproc, "usable_cpus": usable, "cpu_model": model,
            "threads": min(CPU_SHARE, usable)}


def cpu_baseline(cache, seqs, layers_multi, layers_single, threads, seed):
    """Times the CPU oracle (C++ restatement of the reference CPU paged
    attention, fp64 accumulation, GQA as replicated MHA) on the bench's own
    cache contents: one thread per core over `layers_multi` layers and a
    single thread (the reference's own mode) over `layers_single` layers,
    all sequences each.  The GPU kernel is checked against every sampled
    layer at full size."""
    import oracle

    rng = np.random.default_rng(seed + 7)
    batch = len(seqs)
    tables_list = [cache.block_table(s) for s in seqs]
    lengths = np.array([cache.length(s) for s in seqs], np.int32)
    max_blocks = max(len(t) for t in tables_list)
    tables = np.zeros((batch, max_blocks), np.uint32)
    for b, t in enumerate(tables_list):
        tables[b, : len(t)] = t
    timed = {threads: [0, 0.0], 1: [0, 0.0]}
    max_err = 0.0
    plan = [(layer, threads) for layer in range(layers_multi)]
    plan += [(layers_multi + i, 1) for i in range(layers_single)]
    for layer, nthreads in plan:
        layer %= cache.layers
        kp, vp = (x.cpu().numpy() for x in cache.layer_pools(layer))
        q = rng.standard_normal((batch, HQ, D), dtype=np.float32)
        tk = rng.standard_normal((batch, HKV, D), dtype=np.float32)
        tv = rng.standard_normal((batch, HKV, D), dtype=np.float32)
        t0 = time.perf_counter()
        ref = oracle.batched_decode(q, kp, vp, tables, lengths, tk, tv, threads=nthreads)
        timed[nthreads][1] += time.perf_counter() - t0
        timed[nthreads][0] += decode_bytes(lengths)
        # Full-size parity of the GPU kernel on the same inputs.
        dv = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to("cuda:0")  # noqa: E731
        out = torch.empty(batch, HQ, D, device="cuda:0")
        ws = hx.decode_workspace(batch, HQ, HKV, max_blocks)
        kpool, vpool = cache.layer_pool_pointers(layer)
        hx.paged_decode_attention(dv(q), kpool, vpool, dv(tables.astype(np.int32)), dv(lengths),
                                  dv(tk), dv(tv), out, ws,
                                  pool_shape=(cache.physical_blocks, HKV, P, D))
        torch.cuda.synchronize()
        diff = np.abs(out.cpu().numpy() - ref)
        tol = 2e-5 + 1e-4 * np.abs(ref)
        max_err = max(max_err, float(diff.max()))
        if not (diff <= tol).all():
            raise SystemExit(f"parity failure on layer {layer}: max abs err {diff.max()}")
        del kp, vp
    rate = {n: (b / t / 1e9 if t > 0 else None, t) for n, (b, t) in timed.items()}
    return rate, max_err


_probe_lib = None


def probe_lib():
    """The bench-only probe kernels (libhelix_probe.so, built beside the
    product library but not part of it)."""
    global _probe_lib
    if _probe_lib is None:
        path = os.path.join(ROOT, "helix_runtime_amd", "libhelix_probe.so")
        if not os.path.exists(path):
            raise SystemExit(f"{path} is missing: run `make -C helix_runtime_amd libhelix_probe.so`")
        _probe_lib = ctypes.CDLL(path)
        for name in ("helix_probe_stream_read", "helix_probe_page_read"):
            getattr(_probe_lib, name).restype = ctypes.c_int
    return _probe_lib


def probe_check(rc):
    if rc != 0:
        raise SystemExit(f"probe kernel failed with status {rc}")


def copy_probe(nbytes=1 << 30, reps=10):
    """Streaming copy of a known size: reads nbytes and writes nbytes per launch."""
    src = torch.randn(nbytes // 4, device="cuda:0")
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        dst.copy_(src)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / reps
    big = torch.randn(4 * nbytes // 4, device="cuda:0")
    del src, dst
    props = torch.cuda.get_device_properties(0)
    best = (0.0, 0, 0.0)
    for per_cu in (2, 4, 8, 16, 32):
        blocks = props.multi_processor_count * per_cu
        sink = torch.empty(blocks * 256, device="cuda:0")
        args = (ctypes.c_void_p(big.data_ptr()), ctypes.c_size_t(big.numel()),
                ctypes.c_void_p(sink.data_ptr()), ctypes.c_uint(blocks),
                ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
        probe_check(probe_lib().helix_probe_stream_read(*args))
        e0.record()
        for _ in range(reps):
            probe_check(probe_lib().helix_probe_stream_read(*args))
        e1.record()
        torch.cuda.synchronize()
        ms_r = e0.elapsed_time(e1) / reps
        gbps = 4 * nbytes / ms_r / 1e6
        log(f"stream-read probe: {blocks} workgroups: {gbps:.0f} GB/s")
        if gbps > best[0]:
            best = (gbps, blocks, ms_r)
    ms_read = best[2]
    print(json.dumps({"copy_probe_bytes_read": nbytes, "copy_probe_bytes_written": nbytes,
                      "avg_ms": round(ms, 4), "gbps_read_plus_write": round(2 * nbytes / ms / 1e6, 1),
                      "read_probe_bytes": 4 * nbytes, "read_probe_ms": round(ms_read, 4),
                      "read_probe_gbps": round(4 * nbytes / ms_read / 1e6, 1)}), flush=True)


def page_probe(seed, reps=10, order="head"):
    """Reads the config-3 decode's pages in the stream kernel's order (kv-head
    major, each wavefront a contiguous range of the page list, two K/V page
    pairs in flight) with loads only: the attainable rate for this access
    pattern, with default and with non-temporal (streaming) loads.  Pages of
    the --page-dtype element size; order "sequence" lists the units
    sequence-major instead (the kv heads of one sequence in turn)."""
    rng = np.random.default_rng(seed)
    lengths = np.exp(rng.uniform(math.log(512), math.log(8192), size=BATCH)).astype(np.int64)
    pages = (lengths + P - 1) // P
    n_phys = int(pages.sum() + 64)
    perm = rng.permutation(n_phys).astype(np.int64)
    tables, at = [], 0
    for n in pages:
        tables.append(perm[at: at + n])
        at += n
    if order == "sequence":
        kv = [(ph * HKV + h, n_phys * HKV + ph * HKV + h)
              for t in tables for h in range(HKV) for ph in t]
    else:
        kv = [(ph * HKV + h, n_phys * HKV + ph * HKV + h)
              for h in range(HKV) for t in tables for ph in t]
    props = torch.cuda.get_device_properties(0)
    waves = props.multi_processor_count * 8
    steps = len(kv) // waves
    pairs = np.array(kv[: waves * steps], np.uint32).reshape(-1)
    pool = torch.zeros(2 * n_phys * HKV * P * D * PAGE_BYTES, dtype=torch.uint8, device="cuda:0")
    dpairs = torch.from_numpy(pairs.view(np.int32)).to("cuda:0")
    sink = torch.empty(waves * 64, device="cuda:0")
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    out = {"page_probe_pairs": waves * steps, "page_dtype": PAGE_DTYPE, "order": order,
           "page_probe_bytes": waves * steps * 2 * P * D * PAGE_BYTES}
    for nt in (0, 1):
        args = (ctypes.c_void_p(pool.data_ptr()), ctypes.c_void_p(dpairs.data_ptr()),
                ctypes.c_size_t(steps), ctypes.c_uint(waves), ctypes.c_int(nt),
                ctypes.c_int(PAGE_BYTES), ctypes.c_void_p(sink.data_ptr()),
                ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
        probe_check(probe_lib().helix_probe_page_read(*args))
        e0.record()
        for _ in range(reps):
            probe_check(probe_lib().helix_probe_page_read(*args))
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / reps
        out["page_probe_gbps" + ("_nontemporal" if nt else "")] = round(
            out["page_probe_bytes"] / ms / 1e6, 1)
    print(json.dumps(out), flush=True)


def run_reference_entry(args):
    """The reference-shaped decode entry point at config-3 shape: the
    reference model attends one sequence per call
    (attention::cuda::paged_scaled_dot_product_attention_with_tail_out,
    src/model/cuda_llama.cpp:365-367), so a layer of the batch-64 step is 64
    calls, each with that sequence's device block table, its [32, 1, 128]
    query, [8, 1, 128] tail and a [32, 1, history + 1] score workspace.
    Here those calls take the single-sequence decode route (ref_decode_kernel,
    plus its merge launch when a kv head takes several workgroups), which
    also leaves the probabilities in the workspace as the reference does.
    Each layer's 64 calls are queued behind a short device-side sleep so the
    events time the device work, not Python's call overhead.  The exact
    scalar route (helix_paged_attention_with_tail_probabilities_out) is
    timed on a few layers beside it."""
    L = args.layers
    cache, seqs, lengths = build_workload(args.seed, BATCH, L, 2)
    gen = torch.Generator(device="cuda:0")
    gen.manual_seed(args.seed + 1)
    q = torch.randn(L, BATCH, HQ, 1, D, device="cuda:0", generator=gen)
    tk = torch.randn(L, BATCH, HKV, 1, D, device="cuda:0", generator=gen)
    tv = torch.randn(L, BATCH, HKV, 1, D, device="cuda:0", generator=gen)
    out = torch.empty(BATCH, HQ, 1, D, device="cuda:0")
    tables = [torch.tensor(cache.block_table(s), dtype=torch.int32, device="cuda:0")
              for s in seqs]
    ws = [torch.empty(HQ, 1, int(n) + 1, device="cuda:0") for n in lengths]
    pools = [cache.layer_pool_pointers(l) for l in range(L)]
    shape = (cache.physical_blocks, HKV, P, D)
    kpool = [_DevicePointer(k) for k, _ in pools]
    vpool = [_DevicePointer(v) for _, v in pools]

    class _Pool(_DevicePointer):
        shape = None

    def pool(ptr):
        t = _Pool(ptr.address)
        t.shape = shape
        return t

    stream = torch.cuda.current_stream()

    def layer(l, probabilities, e0, e1):
        torch.cuda._sleep(20_000_000)  # holds the queue while the calls are enqueued
        e0.record(stream)
        for b in range(BATCH):
            hx.paged_attention_with_tail_out(q[l, b], pool(kpool[l]), pool(vpool[l]), tables[b],
                                             int(lengths[b]), tk[l, b], tv[l, b], out[b], ws[b],
                                             stream, probabilities=probabilities)
        e1.record(stream)

    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(2)] for _ in range(L)]
    for l in range(L):  # warmup
        layer(l, False, *ev[l])
    torch.cuda.synchronize()
    layer_ms = []
    for _ in range(args.steps):
        for l in range(L):
            layer(l, False, *ev[l])
        torch.cuda.synchronize()
        layer_ms += [e[0].elapsed_time(e[1]) for e in ev]
    exact_layers = min(2, L)
    exact_ms = []
    for l in range(exact_layers):
        layer(l, True, *ev[l])
    torch.cuda.synchronize()
    exact_ms = [ev[l][0].elapsed_time(ev[l][1]) for l in range(exact_layers)]
    per_layer = decode_bytes(lengths)
    ms = float(np.mean(layer_ms))
    gbps = per_layer / (ms * 1e-3) / 1e9
    exact_gbps = per_layer / (float(np.mean(exact_ms)) * 1e-3) / 1e9
    line = {
        "metric": "reference-shaped decode entry (one call per sequence) attn GB/s, 8B-GQA "
                  "batch 64",
        "value": round(gbps, 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": 1, "ms_per_step": round(ms * L, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic N(0,1) K/V/Q, seeded; pages shuffled across the pool",
        "config": {"workload": "config3 pages and contexts, attended through "
                               "paged_scaled_dot_product_attention_with_tail_out: 64 calls "
                               "per layer, 32q/8kv heads, head_dim 128, page 16",
                   "batch": BATCH, "layers": L, "mean_context": float(lengths.mean())},
        "layer_avg_us": round(ms * 1e3, 2),
        "call_avg_us": round(ms * 1e3 / BATCH, 2),
        "hbm_frac": round(gbps / HBM_PEAK_GBPS, 4),
        "exact_route_layer_avg_us": round(float(np.mean(exact_ms)) * 1e3, 2),
        "exact_route_gbps": round(exact_gbps, 2),
        "exact_route_note": "probabilities materialised "
                            "(helix_paged_attention_with_tail_probabilities_out)",
    }
    print(json.dumps(line), flush=True)
    cache.close()


def run_reference_chunk(args):
    """The reference-shaped chunk call at config-5 shape: the reference runs
    chunked prefill through the same entry point as decode
    (attention::cuda::paged_scaled_dot_product_attention_with_tail_out with a
    T-token tail, include/helix/attention/cuda_paged.hpp:49-53), one sequence
    per call, so a layer of config 5 is 16 calls, each with that sequence's
    block table, its [32, 512, 128] query, [8, 512, 128] chunk and a
    [32, 512, history + 512] score workspace that receives the
    probabilities.  Here those calls run the exact fp32 matrix-core prefill
    kernel (prefill_probs_kernel).  The exact scalar route
    (helix_paged_attention_with_tail_probabilities_out, the generic kernel)
    is timed on two of the calls beside it."""
    rng = np.random.default_rng(args.seed + 50)
    hists = rng.integers(0, 4097, size=CHUNK_BATCH)
    T = CHUNK_TOKENS
    n_phys = int(((hists + P - 1) // P).sum() + 16)
    cache = hx.PagedKvCache(1, HKV, D, P, n_phys)
    tok = torch.zeros(1, HKV, D, device="cuda:0")
    dummies = []
    for _ in range(n_phys):
        s = cache.create_sequence()
        cache.append(s, tok, tok)
        dummies.append(s)
    for i in rng.permutation(len(dummies)):
        cache.release_sequence(dummies[int(i)])
    gen = torch.Generator(device="cuda:0")
    gen.manual_seed(args.seed)
    seqs = []
    for b in range(CHUNK_BATCH):
        s = cache.create_sequence()
        n = int(hists[b])
        if n:
            cache.append_layer_major(s, [torch.randn(HKV, n, D, device="cuda:0", generator=gen)],
                                     [torch.randn(HKV, n, D, device="cuda:0", generator=gen)])
        seqs.append(s)
    kptr, vptr = cache.layer_pool_pointers(0)

    class _Pool(_DevicePointer):
        shape = (cache.physical_blocks, HKV, P, D)

    kpool, vpool = _Pool(kptr), _Pool(vptr)
    tables = [torch.tensor(cache.block_table(s) or [0], dtype=torch.int32, device="cuda:0")
              for s in seqs]
    q = torch.randn(CHUNK_BATCH, HQ, T, D, device="cuda:0", generator=gen)
    ck = torch.randn(CHUNK_BATCH, HKV, T, D, device="cuda:0", generator=gen)
    cv = torch.randn(CHUNK_BATCH, HKV, T, D, device="cuda:0", generator=gen)
    out = torch.empty(CHUNK_BATCH, HQ, T, D, device="cuda:0")
    ws = [torch.empty(HQ, T, int(n) + T, device="cuda:0") for n in hists]
    stream = torch.cuda.current_stream()

    def call(b, probabilities=False):
        hx.paged_attention_with_tail_out(q[b], kpool, vpool, tables[b], int(hists[b]), ck[b],
                                         cv[b], out[b], ws[b], stream,
                                         probabilities=probabilities)

    def layer(e0, e1, which=range(CHUNK_BATCH), probabilities=False):
        torch.cuda._sleep(20_000_000)
        e0.record(stream)
        for b in which:
            call(b, probabilities)
        e1.record(stream)

    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    for _ in range(args.warmup):
        layer(e0, e1)
    torch.cuda.synchronize()
    layer_ms = []
    for _ in range(args.steps):
        layer(e0, e1)
        torch.cuda.synchronize()
        layer_ms.append(e0.elapsed_time(e1))
    ms = float(np.mean(layer_ms))
    flops = prefill_flops(hists)
    tflops = flops / (ms * 1e-3) / 1e12
    exact = [int(np.argmin(hists)), int(np.argsort(hists)[CHUNK_BATCH // 2])]
    layer(e0, e1, exact, True)
    torch.cuda.synchronize()
    exact_ms = e0.elapsed_time(e1)
    exact_tflops = prefill_flops(hists[exact]) / (exact_ms * 1e-3) / 1e12
    prob_bytes = float(sum(HQ * T * (int(n) + T) * 4 for n in hists))
    line = {
        "metric": "reference-shaped chunk call (one call per sequence) TFLOP/s (fp32 MFMA, "
                  "probabilities written), 8B-GQA 16 x 512-token chunks",
        "value": round(tflops, 3), "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic N(0,1) K/V/Q, seeded; pages shuffled across the pool",
        "config": {"workload": "config5 chunks attended through "
                               "paged_scaled_dot_product_attention_with_tail_out: 16 calls per "
                               "layer, 32q/8kv heads, head_dim 128, page 16, 512-token tails",
                   "batch": CHUNK_BATCH, "chunk_tokens": T,
                   "mean_history": float(hists.mean())},
        "layer_avg_us": round(ms * 1e3, 2),
        "call_avg_us": round(ms * 1e3 / CHUNK_BATCH, 2),
        "roofline": {"bound": "mfma", "achieved": round(tflops, 3),
                     "peak": MFMA_F32_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(tflops / MFMA_F32_PEAK_TFLOPS, 4), "traffic": None},
        "probability_bytes_per_layer": prob_bytes,
        "exact_route_calls": exact,
        "exact_route_us": round(exact_ms * 1e3, 2),
        "exact_route_tflops": round(exact_tflops, 4),
        "exact_route_note": "generic kernel (helix_paged_attention_with_tail_probabilities_out) "
                            "on the shortest and the median history",
    }
    print(json.dumps(line), flush=True)
    cache.close()


def run_tiny(args):
    """Config 1: the tiny reference-shaped decode (1 sequence, 4/4 heads,
    head_dim 16, 16-token pages, a 64-token history in 4 pages drawn by a
    seeded permutation from an 8-page pool, one-token tail), through
    paged_scaled_dot_product_attention_with_tail_out.  head_dim 16 is outside
    the batched kernels' geometry, so the call runs the exact kernel and
    writes the probabilities.  A latency measurement: `value` is the device
    time per call (calls queued back to back behind a device-side sleep so
    host overhead is hidden); `call_wall_us` is the host-inclusive rate of
    calls issued one after another."""
    rng = np.random.default_rng(1)
    table = rng.permutation(8)[:4].astype(np.int32)
    dv = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to("cuda:0")  # noqa: E731
    kp_h = rng.standard_normal((8, 4, 16, 16), dtype=np.float32)
    vp_h = rng.standard_normal((8, 4, 16, 16), dtype=np.float32)
    q_h = rng.standard_normal((4, 1, 16), dtype=np.float32)
    tk_h = rng.standard_normal((4, 1, 16), dtype=np.float32)
    tv_h = rng.standard_normal((4, 1, 16), dtype=np.float32)
    kp, vp, q, tk, tv, tab = dv(kp_h), dv(vp_h), dv(q_h), dv(tk_h), dv(tv_h), dv(table)
    out = torch.empty(4, 1, 16, device="cuda:0")
    ws = torch.empty(4, 1, 65, device="cuda:0")
    stream = torch.cuda.current_stream()

    def call():
        hx.paged_attention_with_tail_out(q, kp, vp, tab, 64, tk, tv, out, ws, stream)

    for _ in range(args.warmup + 5):
        call()
    torch.cuda.synchronize()
    reps = max(200, args.steps * 20)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda._sleep(50_000_000)
    e0.record(stream)
    for _ in range(reps):
        call()
    e1.record(stream)
    torch.cuda.synchronize()
    dev_us = e0.elapsed_time(e1) * 1e3 / reps
    t0 = time.perf_counter()
    for _ in range(reps):
        call()
    torch.cuda.synchronize()
    wall_us = (time.perf_counter() - t0) * 1e6 / reps
    # Algorithmic bytes: the 4 history pages of K and V (4 heads x 16 tokens
    # x 16 dims), tail K/V, query, output, table, probability workspace.
    nbytes = 2 * 4 * 64 * 16 * 4 + 2 * 4 * 16 * 4 + 2 * 4 * 16 * 4 + 4 * 4 + 4 * 65 * 4
    gbps = nbytes / (dev_us * 1e-6) / 1e9
    cpu = None
    if not args.no_cpu:
        import oracle
        got = out.cpu().numpy()
        n = 2000
        t0 = time.perf_counter()
        for _ in range(n):
            ref, _ = oracle.paged_attention(q_h, kp_h, vp_h, table.astype(np.uint32), 64, tk_h,
                                            tv_h)
        cpu_us = (time.perf_counter() - t0) * 1e6 / n
        err = float(np.abs(got - ref).max())
        if not (np.abs(got - ref) <= 2e-5 + 1e-4 * np.abs(ref)).all():
            raise SystemExit(f"config 1 parity failure: max abs err {err}")
        hostinfo = host_cpu()
        cpu = {"value": round(cpu_us, 3), "unit": "us per call", "cores": 1, "kind": "port",
               "threads": 1, "nproc": hostinfo["nproc"], "usable_cpus": hostinfo["usable_cpus"],
               "cpu_model": hostinfo["cpu_model"],
               "sample": f"CPU oracle (C++ restatement of the reference CPU paged attention, "
                         f"fp64 accumulation) on the same inputs, {n} calls on one thread "
                         f"including the ctypes call; GPU output matched it to max abs err "
                         f"{err:.2e}"}
    line = {
        "metric": "tiny paged decode latency (config 1, reference-shaped entry point)",
        "value": round(dev_us, 3), "unit": "us per call", "n_gpus": 1, "steps": reps,
        "warmup": args.warmup + 5, "ms_per_step": round(dev_us * 1e-3, 6),
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic N(0,1) K/V/Q, seeded (numpy default_rng(1))",
        "config": {"workload": "config1: 1 sequence, 1 layer, 4/4 heads, head_dim 16, page 16, "
                               "64-token history in 4 of 8 pages (seeded permutation), "
                               "one-token tail", "q_heads": 4, "kv_heads": 4, "head_dim": 16,
                   "block_tokens": 16, "history": 64},
        "call_wall_us": round(wall_us, 3),
        "roofline": {"bound": "hbm", "achieved": round(gbps, 3), "peak": HBM_PEAK_GBPS,
                     "unit": "GB/s", "frac": round(gbps / HBM_PEAK_GBPS, 8),
                     "traffic": None,
                     "note": "latency-bound: 35 KB per call; the time is the kernel's launch "
                             "and its three dependent passes, not HBM bandwidth"},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


# Llama-3-8B decoder shapes for --model-step.
MODEL_HIDDEN, MODEL_INTER, MODEL_VOCAB, ROPE_THETA = 4096, 14336, 128256, 500000.0


class _DevicePointer:
    """A raw device address passed where the wrappers take a tensor."""

    def __init__(self, address):
        self.address = address

    def data_ptr(self):
        return self.address


def run_model_step(args):
    """A whole Llama-3-8B-shaped decode step (batch 64, config-3 contexts, 32
    layers, random fp32 weights): the model's dense work (RMSNorm,
    projections, SwiGLU, LM head) in torch (hipBLASLt GEMMs), the KV path in
    the library.  Two flows over the same pages, alternating step by step:

    * reference: the order of CudaLlamaModel::decode_one_paged_device
      (src/model/cuda_llama.cpp:311-400) -- per layer two RoPE launches,
      attention over the uncommitted tail, copies of the token's K/V into
      the step's [L, B, Hkv, D] buffers and a stream synchronisation; the
      token committed for all layers after the forward pass;
    * integrated: one RoPE launch for query and key, K/V projected straight
      into the step buffers, the append fused into each decode launch, no
      synchronisation inside the step.

    value = tokens per second of the integrated flow."""
    steps_total = args.warmup + 2 * args.steps + 2
    cache, seqs, lengths0 = build_workload(args.seed, BATCH, LAYERS, steps_total)
    nseq = len(seqs)
    batch = hx.DecodeBatch(cache, seqs, HQ, max_tokens=int(lengths0.max()) + steps_total + P)
    gen = torch.Generator(device="cuda:0")
    gen.manual_seed(args.seed + 7)

    def w(*shape):
        return torch.randn(*shape, device="cuda:0", generator=gen) * 0.02

    layers = [{"an": 1 + w(MODEL_HIDDEN), "q": w(MODEL_HIDDEN, HQ * D),
               "k": w(MODEL_HIDDEN, HKV * D), "v": w(MODEL_HIDDEN, HKV * D),
               "o": w(HQ * D, MODEL_HIDDEN), "fn": 1 + w(MODEL_HIDDEN),
               "g": w(MODEL_HIDDEN, MODEL_INTER), "u": w(MODEL_HIDDEN, MODEL_INTER),
               "d": w(MODEL_INTER, MODEL_HIDDEN)} for _ in range(LAYERS)]
    emb = w(MODEL_VOCAB, MODEL_HIDDEN)
    final = 1 + w(MODEL_HIDDEN)
    head = w(MODEL_HIDDEN, MODEL_VOCAB)
    weight_bytes = sum(t.numel() for lw in layers for t in lw.values()) * 4 + head.numel() * 4
    positions = int(lengths0.max()) + steps_total + 1
    pair = torch.arange(D // 2, dtype=torch.float64)
    ang = torch.arange(positions, dtype=torch.float64)[:, None] * (
        ROPE_THETA ** (-2.0 * pair / D))[None, :]
    cos = torch.cos(ang).float().to("cuda:0")
    sin = torch.sin(ang).float().to("cuda:0")
    torch.backends.cuda.matmul.allow_tf32 = False
    stream = torch.cuda.current_stream()
    k_all = torch.empty(LAYERS, nseq, HKV, D, device="cuda:0")
    v_all = torch.empty_like(k_all)
    ctx = torch.empty(nseq, HQ, D, device="cuda:0")
    token_ids = torch.randint(0, MODEL_VOCAB, (nseq,), device="cuda:0", generator=gen)
    step_lengths = _DevicePointer(batch.device_state()["lengths"])

    def norm(x, g):
        return x * torch.rsqrt(torch.mean(x * x, dim=-1, keepdim=True) + 1e-5) * g

    def step(integrated):
        batch.prepare(stream)
        hidden = emb[token_ids]
        for l, lw in enumerate(layers):
            x = norm(hidden, lw["an"])
            q = (x @ lw["q"]).view(nseq, HQ, D)
            if integrated:
                torch.matmul(x, lw["k"], out=k_all[l].view(nseq, HKV * D))
                torch.matmul(x, lw["v"], out=v_all[l].view(nseq, HKV * D))
                batch.rope(q, k_all[l], cos, sin, stream)
                batch.append_attention_layer(l, q, k_all[l], v_all[l], ctx, stream)
            else:
                k = (x @ lw["k"]).view(nseq, HKV, D)
                v = (x @ lw["v"]).view(nseq, HKV, D)
                hx.rope_out(q, cos, sin, q, positions=step_lengths, stream=stream)
                hx.rope_out(k, cos, sin, k, positions=step_lengths, stream=stream)
                batch.attention_layer(l, q, k, v, ctx, stream)
                k_all[l].copy_(k)
                v_all[l].copy_(v)
            hidden = hidden + ctx.view(nseq, HQ * D) @ lw["o"]
            f = norm(hidden, lw["fn"])
            hidden = hidden + (torch.nn.functional.silu(f @ lw["g"]) * (f @ lw["u"])) @ lw["d"]
            if not integrated:
                stream.synchronize()
        if not integrated:
            batch.append_all_layers(k_all, v_all, stream)
        return norm(hidden, final) @ head

    times = {True: [], False: []}
    for i in range(2 * (args.warmup + args.steps)):
        integrated = i % 2 == 0
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        step(integrated)
        torch.cuda.synchronize()
        if i >= 2 * args.warmup:
            times[integrated].append(time.perf_counter() - t0)
    ms = {k: float(np.mean(v)) * 1e3 for k, v in times.items()}
    # Attention alone in the same state: the decode launches of one step.
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
    batch.prepare(stream)
    q = torch.randn(nseq, HQ, D, device="cuda:0", generator=gen)
    ev[0].record(stream)
    for l in range(LAYERS):
        batch.append_attention_layer(l, q, k_all[l], v_all[l], ctx, stream)
    ev[1].record(stream)
    torch.cuda.synchronize()
    attn_ms = ev[0].elapsed_time(ev[1])
    line = {
        "metric": "Llama-3-8B-shaped decode step tokens/s (dense ops in torch, paged KV path "
                  "in the library), batch 64",
        "value": round(nseq / (ms[True] * 1e-3), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms[True], 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: random fp32 weights, N(0,1) cache contents, seeded",
        "config": {"workload": "config3 contexts under a Llama-3-8B-shaped decoder: 32 layers, "
                               "hidden 4096, 32q/8kv heads, intermediate 14336, vocab 128256",
                   "batch": nseq, "mean_context": float(lengths0.mean())},
        "reference_flow_ms_per_step": round(ms[False], 3),
        "reference_flow_tokens_per_s": round(nseq / (ms[False] * 1e-3), 1),
        "attention_ms_per_step": round(attn_ms, 3),
        "attention_share": round(attn_ms / ms[True], 4),
        "dense_weight_bytes": weight_bytes,
        "roofline": None,
        "cpu_baseline": None,
    }
    print(json.dumps(line), flush=True)
    batch.close()
    cache.close()


MFMA_F32_PEAK_TFLOPS = 157.3
MFMA_BF16_PEAK_TFLOPS = 2500.0  # dense
CHUNK_BATCH, CHUNK_TOKENS = 16, 512


def prefill_flops(hists, t=CHUNK_TOKENS, hq=None, d=D):
    """Algorithmic FLOPs of one chunked-prefill launch (one layer): QK^T and
    P.V over the history plus the causal triangle of the chunk."""
    hq = hq or HQ
    hists = np.asarray(hists, np.float64)
    return float(np.sum(4.0 * hq * d * (t * hists + t * (t + 1) / 2.0)))


def measured_traffic(workload):
    """HBM bytes per launch of a workload's dominant kernel(s), measured with
    the FETCH_SIZE / WRITE_SIZE counters and recorded under profiles/ (the
    counters cannot be read from inside this process); None when absent."""
    path = os.path.join(ROOT, "profiles", f"{workload}_traffic.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        return json.load(f).get("hbm_bytes_per_launch")


def run_prefill(args):
    """Config 5: 16 sequences each append a 512-token chunk onto a paged
    history of uniform [0, 4096] tokens, then attend causally (MFMA path).
    The chunk's slots are reserved once; every timed step re-runs the same
    per-layer chunk append + prefill attention, so the histories stay at
    their drawn lengths."""
    import oracle

    rng = np.random.default_rng(args.seed + 50)
    L = args.layers
    hists = rng.integers(0, 4097, size=CHUNK_BATCH)
    T = CHUNK_TOKENS
    n_phys = int(((hists + T + P - 1) // P).sum() + CHUNK_BATCH + 16)
    cache = hx.PagedKvCache(L, HKV, D, P, n_phys, page_dtype=PAGE_DTYPE)
    log(f"pool: {n_phys} blocks x {L} layers ({n_phys * L * 2 * HKV * P * D * PAGE_BYTES / 1e9:.1f} GB)")
    tok = torch.zeros(L, HKV, D, device="cuda:0")
    dummies = []
    for _ in range(n_phys):
        s = cache.create_sequence()
        cache.append(s, tok, tok)
        dummies.append(s)
    for i in rng.permutation(len(dummies)):
        cache.release_sequence(dummies[int(i)])
    gen = torch.Generator(device="cuda:0")
    gen.manual_seed(args.seed)
    src_elems = HKV * 4096 * D
    src_k = torch.randn(L, src_elems + 4096, device="cuda:0", generator=gen)
    src_v = torch.randn(L, src_elems + 4096, device="cuda:0", generator=gen)
    seqs = []
    for b in range(CHUNK_BATCH):
        s = cache.create_sequence()
        n = int(hists[b])
        if n:
            off = int(rng.integers(0, 1024)) * 4
            cache.append_layer_major(s, [src_k[l, off: off + HKV * n * D].view(HKV, n, D)
                                         for l in range(L)],
                                     [src_v[l, off: off + HKV * n * D].view(HKV, n, D)
                                      for l in range(L)])
        seqs.append(s)
    del src_k, src_v
    torch.cuda.empty_cache()
    batch = hx.DecodeBatch(cache, seqs, HQ, max_tokens=int(hists.max()) + T + P)
    stream = torch.cuda.current_stream()
    batch.prepare_chunk(T, stream)
    q = torch.randn(L, CHUNK_BATCH, HQ, T, D, device="cuda:0", generator=gen)
    ck = torch.randn(L, CHUNK_BATCH, HKV, T, D, device="cuda:0", generator=gen)
    cv = torch.randn(L, CHUNK_BATCH, HKV, T, D, device="cuda:0", generator=gen)
    out = torch.empty(CHUNK_BATCH, HQ, T, D, device="cuda:0")
    ev = [[[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(L)]
          for _ in range(args.steps)]

    def step(events):
        for l in range(L):
            if events is not None:
                events[l][0].record(stream)
            batch.append_layer(l, ck[l], cv[l], stream)
            if events is not None:
                events[l][1].record(stream)
            batch.prefill_layer(l, q[l], ck[l], cv[l], out, stream)
            if events is not None:
                events[l][2].record(stream)

    for _ in range(args.warmup):
        step(None)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        step(ev[i])
    torch.cuda.synchronize()
    ms_per_step = (time.perf_counter() - t0) * 1e3 / args.steps
    append_ms = [ev[i][l][0].elapsed_time(ev[i][l][1]) for i in range(args.steps) for l in range(L)]
    attn_ms = [ev[i][l][1].elapsed_time(ev[i][l][2]) for i in range(args.steps) for l in range(L)]
    flops = prefill_flops(hists)
    attn_avg = float(np.mean(attn_ms))
    tflops = flops / (attn_avg * 1e-3) / 1e12
    chunk_bytes = 2 * CHUNK_BATCH * HKV * T * D * (4 + PAGE_BYTES)
    append_gbps = chunk_bytes / (float(np.mean(append_ms)) * 1e-3) / 1e9

    cpu = None
    if not args.no_cpu and PAGE_DTYPE == "f32":
        # Bounded sample: layer 0 of the first `cpu_seqs` sequences, one
        # thread per sequence, checked against the GPU output of that layer.
        nseq = min(args.cpu_seqs, CHUNK_BATCH)
        batch.append_layer(0, ck[0], cv[0], stream)
        batch.prefill_layer(0, q[0], ck[0], cv[0], out, stream)
        torch.cuda.synchronize()
        got = out.cpu().numpy()
        kp, vp = (x.cpu().numpy() for x in cache.layer_pools(0))
        qh, ckh, cvh = q[0].cpu().numpy(), ck[0].cpu().numpy(), cv[0].cpu().numpy()
        st = batch.device_state()
        mb = st["max_blocks"]
        tables = [np.array(cache.block_table(s), np.uint32) for s in seqs]

        def one(b):
            return oracle.paged_attention(qh[b], kp, vp, tables[b], int(hists[b]), ckh[b],
                                          cvh[b])[0]

        import concurrent.futures as cf
        t0 = time.perf_counter()
        with cf.ThreadPoolExecutor(nseq) as ex:
            refs = list(ex.map(one, range(nseq)))
        secs = time.perf_counter() - t0
        err = 0.0
        for b in range(nseq):
            diff = np.abs(got[b] - refs[b])
            if not (diff <= 2e-5 + 1e-4 * np.abs(refs[b])).all():
                raise SystemExit(f"prefill parity failure on sequence {b}: max {diff.max()}")
            err = max(err, float(diff.max()))
        cpu_flops = prefill_flops(hists[:nseq])
        hostinfo = host_cpu()
        cpu = {"value": round(cpu_flops / secs / 1e12, 5), "unit": "TFLOP/s", "cores": nseq,
               "kind": "port", "threads": nseq, "nproc": hostinfo["nproc"],
               "usable_cpus": hostinfo["usable_cpus"], "cpu_model": hostinfo["cpu_model"],
               "sample": f"CPU oracle (fp64 accumulation) on layer 0 of {nseq} of "
                         f"{CHUNK_BATCH} sequences, one thread each, {secs:.1f} s; the reference "
                         f"has no GQA, so the CPU runs GQA as MHA with replicated KV heads (the "
                         f"FLOP count is the same, each K/V byte is read {HQ // HKV}x); GPU "
                         f"matched it to max abs err {err:.2e}"}
        del kp, vp, mb
    metric = "chunked-prefill attention TFLOP/s (fp32 MFMA), 8B-GQA 16 x 512-token chunks"
    roofline = {"bound": "mfma", "achieved": round(tflops, 3), "peak": MFMA_F32_PEAK_TFLOPS,
                "unit": "TFLOP/s", "frac": round(tflops / MFMA_F32_PEAK_TFLOPS, 4)}
    if PAGE_DTYPE != "f32":
        # bf16 / fp8 pages run on the bf16 matrix cores: page values are exact
        # in bf16 and the fp32 operand of each product is split into three
        # exact bf16 terms, so each algorithmic FLOP costs three bf16 MFMA
        # FLOPs.  Priced against the dense bf16 peak.
        metric = ("chunked-prefill attention TFLOP/s (bf16 MFMA, fp32 operand split into three "
                  f"exact bf16 terms), 8B-GQA 16 x 512-token chunks [{PAGE_DTYPE} pages]")
        roofline = {"bound": "mfma", "achieved": round(tflops, 3), "peak": MFMA_BF16_PEAK_TFLOPS,
                    "unit": "TFLOP/s", "frac": round(tflops / MFMA_BF16_PEAK_TFLOPS, 4),
                    "mfma_flops_per_flop": 3,
                    "mfma_frac": round(3 * tflops / MFMA_BF16_PEAK_TFLOPS, 4)}
    line = {
        "metric": metric,
        "value": round(tflops, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic N(0,1) Q/K/V, seeded; pages shuffled across the pool",
        "config": {"workload": "config5: chunked prefill, 16 sequences x 512-token chunk onto "
                               "history U[0, 4096], 32q/8kv heads, head_dim 128, page 16",
                   "batch": CHUNK_BATCH, "chunk_tokens": T, "layers": L, "q_heads": HQ,
                   "kv_heads": HKV, "head_dim": D, "block_tokens": P,
                   "mean_history": float(hists.mean()), "page_dtype": PAGE_DTYPE},
        "prefill_avg_us": round(attn_avg * 1e3, 2),
        "prefill_median_us": round(float(np.median(attn_ms)) * 1e3, 2),
        "append_gbps": round(append_gbps, 2),
        "append_avg_us": round(float(np.mean(append_ms)) * 1e3, 2),
        "roofline": dict(roofline, traffic=measured_traffic("prefill_config5" + (
            "" if PAGE_DTYPE == "f32" else f"_{PAGE_DTYPE}"))),
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    batch.close()
    cache.close()


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--seed", type=int, default=3)
    ap.add_argument("--layers", type=int, default=None,
                    help="layers of the pool and step (default: 32; config 2: 1, the "
                         "single-layer MHA decode BASELINE names)")
    ap.add_argument("--pages-per-split", type=int, default=0,
                    help="decode split size in pages (0: library default)")
    ap.add_argument("--cpu-layers", type=int, default=32,
                    help="layers timed on the CPU oracle with one thread per core")
    ap.add_argument("--cpu-single-layers", type=int, default=8,
                    help="layers timed on the CPU oracle with one thread")
    ap.add_argument("--cpu-threads", type=int, default=0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--separate-append", action="store_true",
                    help="the reference's flow: attention over the uncommitted tail for every "
                         "layer, then one launch appending the token for all layers (instead "
                         "of the append fused into each layer's decode launch)")
    ap.add_argument("--no-shuffle", action="store_true",
                    help="allocate pages in pool order instead of scattering them")
    ap.add_argument("--config", type=int, default=3, choices=(1, 2, 3, 4, 5),
                    help="3: batched GQA decode (default, the headline metric); 1: the tiny "
                         "reference-shaped decode (latency); 2: batch-8 MHA decode; "
                         "4: prefix-sharing decode; 5: chunked prefill on the matrix cores")
    ap.add_argument("--cpu-seqs", type=int, default=4,
                    help="config 5: sequences of layer 0 timed on the CPU oracle")
    ap.add_argument("--page-dtype", default="f32", choices=("f32", "bf16", "fp8"),
                    help="page element type (bf16, fp8: the reduced-precision extension; the CPU "
                         "baseline is reported for f32 pages only)")
    ap.add_argument("--page-probe", action="store_true",
                    help="only read the config-3 pages in the decode order with loads only "
                         "(the attainable rate for the access pattern)")
    ap.add_argument("--probe-order", default="head", choices=("head", "sequence"),
                    help="--page-probe: unit order of the page list")
    ap.add_argument("--model-step", action="store_true",
                    help="a whole Llama-3-8B-shaped decode step (torch dense ops, library KV "
                         "path): the integrated flow against the reference's per-layer order")
    ap.add_argument("--chunk", action="store_true",
                    help="with --reference-entry: the config-5 chunk call through the "
                         "reference-shaped entry point")
    ap.add_argument("--reference-entry", action="store_true",
                    help="time the reference-shaped per-sequence decode entry point at config-3 "
                         "shape (64 calls per layer) instead of the batched step")
    ap.add_argument("--copy-probe", action="store_true",
                    help="only run a 1 GiB device-to-device copy (HBM probe / counter calibration)")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (the paged-KV "
              "hot path shards by KV head or by sequence with no exchange). "
              "Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    global PAGE_DTYPE, PAGE_BYTES, HQ, HKV, BATCH
    PAGE_DTYPE, PAGE_BYTES = args.page_dtype, {"bf16": 2, "fp8": 1}.get(args.page_dtype, 4)
    if args.layers is None:
        args.layers = 1 if args.config == 2 else LAYERS
    if args.config == 2:
        HQ, HKV, BATCH = 32, 32, 8
    torch.cuda.set_device(0)
    if args.copy_probe:
        copy_probe()
        return
    if args.page_probe:
        page_probe(args.seed, order=args.probe_order)
        return
    if args.model_step:
        run_model_step(args)
        return
    if args.reference_entry and args.chunk:
        run_reference_chunk(args)
        return
    if args.reference_entry:
        run_reference_entry(args)
        return
    if args.config == 5:
        run_prefill(args)
        return
    if args.config == 1:
        run_tiny(args)
        return
    # warmup, the timed steps, then as many instrumented steps (per-kernel events)
    steps_total = args.warmup + 2 * args.steps + 2
    t_setup = time.perf_counter()
    if args.config == 4:
        cache, seqs, lengths0 = build_prefix_workload(args.seed, args.layers, steps_total)
    else:
        cache, seqs, lengths0 = build_workload(args.seed, BATCH, args.layers, steps_total,
                                                 shuffle=not args.no_shuffle, config=args.config)
    nseq = len(seqs)
    log(f"setup {time.perf_counter() - t_setup:.1f}s; mean context {lengths0.mean():.0f}")

    batch = hx.DecodeBatch(cache, seqs, HQ, max_tokens=int(lengths0.max()) + steps_total + P,
                           pages_per_split=args.pages_per_split)
    split = batch.device_state()["pages_per_split"]
    gen = torch.Generator(device="cuda:0")
    gen.manual_seed(args.seed + 1)
    L = args.layers
    q = torch.randn(L, nseq, HQ, D, device="cuda:0", generator=gen)
    k = torch.randn(L, nseq, HKV, D, device="cuda:0", generator=gen)
    v = torch.randn(L, nseq, HKV, D, device="cuda:0", generator=gen)
    out = torch.empty(L, nseq, HQ, D, device="cuda:0")
    stream = torch.cuda.current_stream()
    # Per (step, layer): before append, before attention, between the main
    # decode kernel and its merge (recorded by the library), after attention.
    ev = [[[torch.cuda.Event(enable_timing=True) for _ in range(4)] for _ in range(L)]
          for _ in range(args.steps)]
    for per_step in ev:
        for e in per_step:
            e[3].record(stream)  # creates the event handle the library records
    torch.cuda.synchronize()

    fused = not args.separate_append

    def step(events):
        batch.prepare(stream)
        for l in range(L):
            if events is not None:
                events[l][0].record(stream)
                events[l][1].record(stream)
                batch.set_timing_event(events[l][3])
            if fused:
                batch.append_attention_layer(l, q[l], k[l], v[l], out[l], stream)
            else:
                batch.attention_layer(l, q[l], k[l], v[l], out[l], stream)
            if events is not None:
                events[l][2].record(stream)
        if events is not None:
            batch.set_timing_event(None)
        if not fused:
            # The reference's flow: the token is committed for every layer
            # after the forward pass has attended to it as the tail.
            batch.append_all_layers(k, v, stream)

    for _ in range(args.warmup):
        step(None)
    # Timed steps: no per-layer events (event records between launches add
    # their own gaps); `value` and ms_per_step come from these.
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        step(None)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    ms_per_step = elapsed * 1e3 / args.steps
    # Instrumented steps (same work, the next K steps): per-launch events for
    # the kernel breakdown and the roofline.
    for i in range(args.steps):
        step(ev[i])
    torch.cuda.synchronize()
    # Append rates, timed separately: the all-layer commit (one launch moves
    # the step's token for all layers) and the single-layer append.
    reps = 3 * L
    aev = [[torch.cuda.Event(enable_timing=True) for _ in range(2)] for _ in range(reps)]
    lev = [[torch.cuda.Event(enable_timing=True) for _ in range(2)] for _ in range(reps)]
    for r in range(reps):
        aev[r][0].record(stream)
        batch.append_all_layers(k, v, stream)
        aev[r][1].record(stream)
    for r in range(reps):
        lev[r][0].record(stream)
        batch.append_layer(r % L, k[r % L], v[r % L], stream)
        lev[r][1].record(stream)
    torch.cuda.synchronize()
    append_ms = [e[0].elapsed_time(e[1]) for e in aev]
    append_layer_ms = [e[0].elapsed_time(e[1]) for e in lev]
    attn_ms = [ev[i][l][1].elapsed_time(ev[i][l][2]) for i in range(args.steps) for l in range(L)]
    kern_ms = [ev[i][l][1].elapsed_time(ev[i][l][3]) for i in range(args.steps) for l in range(L)]
    merge_ms = [ev[i][l][3].elapsed_time(ev[i][l][2]) for i in range(args.steps) for l in range(L)]

    # History of timed step i is the initial length plus the tokens of the
    # warmup and earlier timed steps; the instrumented steps follow them.
    timed_hist = [lengths0 + args.warmup + i for i in range(args.steps)]
    inst_hist = [lengths0 + args.warmup + args.steps + i for i in range(args.steps)]
    # Config 4's roofline is on unique HBM bytes: shared prefix pages are
    # read from HBM once per launch and served from cache to the other
    # sequences.
    roof_fn = unique_decode_bytes if args.config == 4 else decode_bytes
    step_roof_bytes = float(np.mean([roof_fn(h) for h in timed_hist]))
    roof_bytes = float(np.mean([roof_fn(h) for h in inst_hist]))
    launch_bytes = float(np.mean([decode_bytes(h) for h in inst_hist]))
    if fused:
        # The decode kernel also writes the new token rows into their pages.
        step_roof_bytes += append_write_bytes(nseq)
        roof_bytes += append_write_bytes(nseq)
        launch_bytes += append_write_bytes(nseq)
    step_decode = step_roof_bytes * L
    # Fused: the append's writes are counted with the decode and its source
    # rows are the attention tail, already counted there.  Otherwise the
    # all-layer commit reads the rows and writes the pages.
    step_append = 0 if fused else append_bytes(nseq) * L
    value = (step_decode + step_append) / (ms_per_step * 1e-3) / 1e9
    attn_avg_ms = float(np.mean(attn_ms))
    kern_avg_ms = float(np.mean(kern_ms))
    append_avg_ms = float(np.mean(append_ms))
    # The roofline is the dominant kernel's (timed alone): the stream decode
    # kernel, or at config 4 the fused cascade kernel (prefix pass and
    # stream in one launch); decode_attn_gbps is the whole attention launch
    # including the merge.
    roof_ms = kern_avg_ms
    achieved = roof_bytes / (roof_ms * 1e-3) / 1e9
    pair_gbps = roof_bytes / (attn_avg_ms * 1e-3) / 1e9
    logical_gbps = launch_bytes / (attn_avg_ms * 1e-3) / 1e9
    # The all-layer commit moves every layer's row of the step's token.
    append_gbps = append_bytes(nseq) * L / (append_avg_ms * 1e-3) / 1e9
    append_layer_avg_ms = float(np.mean(append_layer_ms))

    suffix = "" if PAGE_DTYPE == "f32" else f"_{PAGE_DTYPE}"
    traffic = measured_traffic(f"decode_config{args.config}{suffix}")

    cpu = None
    if not args.no_cpu and PAGE_DTYPE == "f32":
        hostinfo = host_cpu()
        threads = args.cpu_threads or hostinfo["threads"]
        rate, err = cpu_baseline(cache, seqs, args.cpu_layers, args.cpu_single_layers, threads,
                                 args.seed)
        (gbps, secs), (gbps1, secs1) = rate[threads], rate[1]
        cpu = {"value": round(gbps, 3), "unit": "GB/s", "cores": threads, "kind": "port",
               "threads": threads, "nproc": hostinfo["nproc"],
               "usable_cpus": hostinfo["usable_cpus"], "cpu_model": hostinfo["cpu_model"],
               "single_thread_value": None if gbps1 is None else round(gbps1, 3),
               "sample": f"CPU oracle (C++ restatement of the reference CPU paged attention, "
                         f"fp64 accumulation), {threads} threads (one per usable host CPU, "
                         f"capped at the GPU box's {CPU_SHARE}-CPU share per GPU; host has "
                         f"{hostinfo['nproc']} logical CPUs, {hostinfo['usable_cpus']} usable) "
                         f"over {args.cpu_layers} layer passes (the cache's {cache.layers} "
                         f"layer(s) in turn) x all {nseq} sequences "
                         f"({secs:.1f} s wall), plus 1 thread (the reference's own mode) over "
                         f"{args.cpu_single_layers} layer(s) ({secs1:.1f} s). The reference has "
                         f"no GQA, so the CPU runs GQA as MHA with each KV head replicated for "
                         f"its {HQ // HKV} query heads: it does {HQ // HKV}x the work per counted "
                         f"byte, whose formula (each K/V byte once per KV head) is the GPU's. "
                         f"GPU kernel matched it on every sampled layer, max abs err {err:.2e}"}

    if args.config == 2:
        metric = "paged decode attn GB/s (% of HBM peak) + append GB/s, 7B-MHA batch 8"
        workload = {"workload": "config2: Llama-2-7B MHA decode, batch 8, 32q/32kv heads, "
                                "head_dim 128, page 16, ctx uniform [128, 2048], pool 1.25x "
                                "need, shuffled",
                    "batch": nseq, "layers": L, "q_heads": HQ, "kv_heads": HKV, "head_dim": D,
                    "block_tokens": P, "mean_context": float(lengths0.mean()),
                    "pages_per_split": split}
    elif args.config == 4:
        metric = ("prefix-sharing paged decode attn GB/s on unique HBM bytes + append GB/s, "
                  "8B-GQA batch 128")
        workload = {"workload": "config4: prefix-sharing decode, 128 sequences share a 1024-token "
                                "prefix (refcount 128) + an 8-token copy-on-write partial page, "
                                "unique suffixes U[64, 512], 32q/8kv heads, head_dim 128, page 16",
                    "batch": nseq, "layers": L, "q_heads": HQ, "kv_heads": HKV, "head_dim": D,
                    "block_tokens": P, "mean_context": float(lengths0.mean()),
                    "pages_per_split": split}
    else:
        metric = "paged decode attn GB/s (% of HBM peak) + append GB/s, 8B-GQA batch 64"
        workload = {"workload": "config3: Llama-3-8B GQA decode, 32 layers, batch 64, "
                                "32q/8kv heads, head_dim 128, page 16, ctx log-uniform "
                                "[512, 8192]",
                    "batch": nseq, "layers": L, "q_heads": HQ, "kv_heads": HKV,
                    "head_dim": D, "block_tokens": P, "mean_context": float(lengths0.mean()),
                    "pages_per_split": split}
    if PAGE_DTYPE != "f32":
        metric += f" [{PAGE_DTYPE} pages]"
        workload["page_dtype"] = PAGE_DTYPE
    line = {
        "metric": metric,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic N(0,1) K/V/Q, seeded; pages shuffled across the pool",
        "config": workload,
        "decode_attn_gbps": round(pair_gbps, 2),
        "decode_attn_hbm_frac": round(pair_gbps / HBM_PEAK_GBPS, 4),
        "decode_attn_logical_gbps": round(logical_gbps, 2),
        "append_gbps": round(append_gbps, 2),
        "append_avg_us": round(append_avg_ms * 1e3, 2),
        "append_layer_avg_us": round(append_layer_avg_ms * 1e3, 2),
        "append_mode": ("fused into each layer's decode launch; append_gbps is the all-layer "
                        "commit (one launch writes the step's token for all layers, the "
                        "batched CudaPagedKvCache::append), timed separately"
                        if fused else "attention over the uncommitted tail for every layer, "
                                      "then one all-layer commit launch per step"),
        "decode_avg_us": round(attn_avg_ms * 1e3, 2),
        "decode_median_us": round(float(np.median(attn_ms)) * 1e3, 2),
        "decode_kernel_avg_us": round(kern_avg_ms * 1e3, 2),
        "decode_merge_avg_us": round(float(np.mean(merge_ms)) * 1e3, 2),
        "decode_kernel": ("decode_split_kernel" if split != 0 else
                          "cascade_decode_kernel" if batch.shared_pages() > 0 else
                          "decode_stream_kernel"),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBPS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBPS, 4),
                     "traffic": traffic},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    batch.close()
    cache.close()


if __name__ == "__main__":
    main()
