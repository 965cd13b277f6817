"""The HIP library replays the golden fixtures of tests/golden/ on the GPU:
the reference's paged-cache scenarios on the device cache (tables, page
contents and statistics bit-exact), its attention known answers through the
reference-shaped entry points (history-only with a query offset, and
history plus tail), and the RoPE known answer."""

import numpy as np
import pytest
import torch

import helix_runtime_amd as hx
from golden_runner import LibraryBackend, load, pack_pages, run_scenario

pytestmark = pytest.mark.gpu

SCENARIOS = load("paged_cache_scenarios.json")
ATTENTION = load("attention_known_answers.json")
KERNELS = load("model_kernel_known_answers.json")


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda:0")


@pytest.mark.parametrize("scenario", SCENARIOS, ids=[s["name"] for s in SCENARIOS])
def test_library_cache_replays_reference_scenarios(device, scenario):
    run_scenario(scenario, LibraryBackend)


@pytest.mark.parametrize("case", ATTENTION, ids=[c["name"] for c in ATTENTION])
def test_library_attention_known_answers(device, case):
    q = np.array(case["query"], np.float32)[None]
    k = np.array(case["keys"], np.float32)[None]
    v = np.array(case["values"], np.float32)[None]
    bt = case["block_tokens"]
    kp = dev(pack_pages(k, case["table"], case["physical_blocks"], bt, case["key_padding"]))
    vp = dev(pack_pages(v, case["table"], case["physical_blocks"], bt, case["value_padding"]))
    table = dev(np.array(case["table"], np.int32))
    nq, nk = q.shape[1], k.shape[1]
    # history-only form: all keys in pages, queries at the fixture's offset
    out = torch.empty(1, nq, v.shape[2], device=device)
    ws = torch.empty(1, nq, nk, device=device)
    hx.paged_attention_out(dev(q), kp, vp, table, nk, case["offset"], out, ws)
    torch.cuda.synchronize()
    np.testing.assert_allclose(out.cpu().numpy()[0], case["output"], atol=2e-5, rtol=1e-4)
    np.testing.assert_allclose(ws.cpu().numpy()[0], case["probabilities"], atol=2e-6)
    # history plus tail: the last nq keys are the uncommitted tail
    hist = nk - nq
    if case["offset"] == hist:
        out2 = torch.empty_like(out)
        ws2 = torch.empty_like(ws)
        hx.paged_attention_with_tail_out(dev(q), kp, vp, table, hist, dev(k[:, hist:]),
                                         dev(v[:, hist:]), out2, ws2)
        torch.cuda.synchronize()
        np.testing.assert_allclose(out2.cpu().numpy()[0], case["output"], atol=2e-5, rtol=1e-4)
        np.testing.assert_allclose(ws2.cpu().numpy()[0], case["probabilities"], atol=2e-6)


def test_library_rope_known_answer(device):
    r = KERNELS["rope"]
    out = hx.rope(dev(np.array(r["input"], np.float32)), dev(np.array(r["cosine"], np.float32)),
                  dev(np.array(r["sine"], np.float32)))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(out.cpu().numpy(), np.array(r["output"], np.float32))
