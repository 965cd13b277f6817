"""The CPU oracle replays the golden fixtures of tests/golden/: the paged
cache scenarios and attention known answers of the reference's own tests
(tables, values and statistics bit-exact; attention within 2e-5 of the
closed form) and the model kernels' known answers."""

import numpy as np
import pytest

import oracle
from oracle import llama
from golden_runner import OracleBackend, load, pack_pages, run_scenario

SCENARIOS = load("paged_cache_scenarios.json")
ATTENTION = load("attention_known_answers.json")
KERNELS = load("model_kernel_known_answers.json")


@pytest.mark.parametrize("scenario", SCENARIOS, ids=[s["name"] for s in SCENARIOS])
def test_oracle_pool_replays_reference_scenarios(scenario):
    run_scenario(scenario, OracleBackend)


@pytest.mark.parametrize("case", ATTENTION, ids=[c["name"] for c in ATTENTION])
def test_oracle_attention_known_answers(case):
    q = np.array(case["query"], np.float32)[None]
    k = np.array(case["keys"], np.float32)[None]
    v = np.array(case["values"], np.float32)[None]
    out, probs = oracle.sdpa(q, k, v, case["offset"])
    np.testing.assert_allclose(out[0], case["output"], atol=2e-5, rtol=1e-4)
    np.testing.assert_allclose(probs[0], case["probabilities"], atol=2e-6)
    # the paged form over the fixture's block table, padding never read
    kp = pack_pages(k, case["table"], case["physical_blocks"], case["block_tokens"],
                    case["key_padding"])
    vp = pack_pages(v, case["table"], case["physical_blocks"], case["block_tokens"],
                    case["value_padding"])
    hist = k.shape[1] - q.shape[1]
    if hist >= 0 and case["offset"] == hist:
        tail = slice(hist, None)
        tab = np.array(case["table"][: -(-hist // case["block_tokens"]) or 0], np.uint32)
        pout, _ = oracle.paged_attention(q, kp, vp, tab, hist, k[:, tail], v[:, tail])
        np.testing.assert_allclose(pout[0], case["output"], atol=2e-5, rtol=1e-4)


def test_oracle_model_kernel_known_answers():
    r = KERNELS["rope"]
    out = llama.rope(np.array(r["input"], np.float32), np.array(r["cosine"], np.float32),
                     np.array(r["sine"], np.float32))
    np.testing.assert_array_equal(out, np.array(r["output"], np.float32))
    s = KERNELS["silu"]
    np.testing.assert_allclose(llama.stable_silu(np.array(s["input"], np.float32)), s["output"],
                               atol=s["tolerance"])
    g = KERNELS["swiglu"]
    np.testing.assert_allclose(llama.swiglu(np.array(g["gate"], np.float32),
                                            np.array(g["up"], np.float32)), g["output"],
                               atol=g["tolerance"])
