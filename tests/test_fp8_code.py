"""The device's fp8 rounding (fp8_code in helix_runtime_amd/csrc/fp8.hpp,
bit arithmetic) against the oracle's (nearest code by search over the value
table, pinned to torch in test_oracle.py), through a host build of the same
function: random bit patterns, normals at several scales, every code value
and every midpoint between neighbouring codes (the ties)."""

import os
import shutil
import subprocess

import numpy as np
import pytest

import oracle

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HIPCC = "/opt/rocm/bin/hipcc"


def test_host_build_of_device_rounding_matches_oracle(tmp_path):
    if not os.path.exists(HIPCC) and shutil.which("hipcc") is None:
        pytest.skip("hipcc is not available")
    exe = tmp_path / "fp8_code_check"
    subprocess.run([HIPCC if os.path.exists(HIPCC) else "hipcc", "-x", "hip",
                    "--offload-arch=gfx950", "-O2", "-std=c++17",
                    os.path.join(ROOT, "tests", "cpp", "fp8_code_check.cpp"), "-o", str(exe)],
                   check=True, capture_output=True, timeout=300)
    rng = np.random.default_rng(9)
    table = oracle.fp8_decode(np.arange(256, dtype=np.uint8))
    finite = table[~np.isnan(table)].astype(np.float64)
    pos = np.unique(np.abs(finite))
    mids = ((pos[:-1] + pos[1:]) / 2).astype(np.float32)  # exact in fp32
    x = np.concatenate([
        rng.integers(0, 1 << 32, 1_000_000, dtype=np.uint64).astype(np.uint32).view(np.float32),
        rng.standard_normal(300_000).astype(np.float32)
        * np.float32(10.0) ** rng.integers(-4, 4, 300_000).astype(np.float32),
        table, mids, -mids, np.nextafter(mids, np.float32(0)), np.nextafter(mids, np.float32(1e9)),
    ]).astype(np.float32)
    src, dst = tmp_path / "in.bin", tmp_path / "out.bin"
    x.tofile(src)
    subprocess.run([str(exe), str(src), str(dst)], check=True, timeout=120)
    got = np.fromfile(dst, np.uint8)
    want = oracle.fp8_bits(x)
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, (x[bad[:5]], got[bad[:5]], want[bad[:5]])
