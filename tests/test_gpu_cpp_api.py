"""The C++ API suite (tests/cpp/paged_api_test.cpp) on the GPU: the golden
fixtures of tests/golden/ replayed through include/helix_paged.hpp, random
operation programs against the oracle pool, invalid-call tables, the read
lease, seeded attention sweeps, the single-sequence decode route of the decode entry point
and the extensions.  One process runs every case; the binary prints each
case's name before it runs."""

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
