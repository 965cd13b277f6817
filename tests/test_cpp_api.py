"""The C++ mirror (include/helix_paged.hpp) on the CPU: the header compiles
on its own as C++20; the C++ API test binary links against the library and
the oracle, runs its host-contract cases (validation before any device work,
the status -> helix_amd::Error mapping, host tensors) and skips the GPU
cases."""

import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BINARY = os.path.join(ROOT, "tests", "cpp", "paged_api_test")


def test_header_compiles_standalone(tmp_path):
    src = tmp_path / "use.cpp"
    src.write_text('#include "helix_paged.hpp"\n'
                   "int main() { helix_amd::kv_cache::PagedKvCacheConfig c{1, 1, 1, 1, 1};\n"
                   "  return static_cast<int>(c.layers) - 1; }\n")
    subprocess.run(["g++", "-std=c++20", "-Wall", "-Wextra", "-Werror", "-fsyntax-only",
                    "-D__HIP_PLATFORM_AMD__", "-I", os.path.join(ROOT, "include"),
                    "-I", "/opt/rocm/include", str(src)], check=True)


def test_api_binary_runs_host_cases_and_skips_gpu_cases():
    if not os.path.exists(BINARY):
        pytest.skip("tests/cpp/paged_api_test is not built (run __graft_entry__.build())")
    env = dict(os.environ, HIP_VISIBLE_DEVICES="")  # no device here; make it explicit
    r = subprocess.run([BINARY], capture_output=True, text=True, timeout=120, env=env)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "5 ran, 15 skipped, 0 failed" in r.stdout, r.stdout[-2000:]
