"""The host part of the library under the sanitizers (CPU only).

`make -C tests/cpp sanitize` compiles the block manager, the prefix cache
and their C ABI (helix_runtime_amd/csrc/{block_manager,prefix_cache,
host_api}.cpp) together with the oracle pool and the host-only cases of
tests/cpp/host_programs.hpp twice with g++: under AddressSanitizer plus
UndefinedBehaviorSanitizer, and under ThreadSanitizer.  The cases are eight
threads running create / append / fork / release programs on one block
manager, seeded random programs against the oracle pool, and eight threads
on one host prefix cache.  Both builds must run clean: every case passes
and no sanitizer reports anything.  (The reference builds its tests with
-fsanitize=address,undefined: cmake/HelixCompilerOptions.cmake:33-39.)"""

import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CPP = os.path.join(ROOT, "tests", "cpp")


@pytest.fixture(scope="module")
def built():
    subprocess.run(["make", "-s", "-C", CPP, "-j2", "sanitize"], check=True,
                   capture_output=True, text=True)
    return CPP


@pytest.mark.parametrize("binary,env", [
    ("host_sanitize_asan", {"ASAN_OPTIONS": "detect_leaks=1:abort_on_error=0",
                            "UBSAN_OPTIONS": "print_stacktrace=1:halt_on_error=1"}),
    ("host_sanitize_tsan", {"TSAN_OPTIONS": "halt_on_error=1:second_deadlock_stack=1"}),
])
def test_host_code_runs_clean_under_sanitizer(built, binary, env):
    r = subprocess.run([os.path.join(built, binary)], capture_output=True, text=True,
                       env={**os.environ, **env}, timeout=600)
    report = r.stdout + r.stderr
    assert r.returncode == 0, report[-4000:]
    assert "3 ran, 0 skipped, 0 failed" in r.stdout, report[-4000:]
    for marker in ("AddressSanitizer", "LeakSanitizer", "ThreadSanitizer", "runtime error:"):
        assert marker not in report, report[-4000:]
