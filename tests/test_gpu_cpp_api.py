"""The reference's own CUDA cache and paged-attention tests
(tests/cuda_paged_kv_cache_test.cpp, tests/cuda_attention_test.cpp:196-556),
restated in C++ against include/helix_paged.hpp and run on the GPU, plus the
extensions (fork with copy-on-write, bulk append, gather, prefix cache,
DecodeBatch against the oracle).  One process runs every case; the binary
prints each case's name before it runs."""

import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BINARY = os.path.join(ROOT, "tests", "cpp", "paged_api_test")


def test_cpp_api_suite_passes_on_gpu():
    if not os.path.exists(BINARY):
        pytest.skip("tests/cpp/paged_api_test is not built (make -C tests/cpp)")
    r = subprocess.run([BINARY], capture_output=True, text=True, timeout=110)
    print(r.stdout[-4000:])
    print(r.stderr[-4000:])
    assert r.returncode == 0, r.stdout[-4000:] + r.stderr[-4000:]
    assert "20 ran, 0 skipped, 0 failed" in r.stdout
