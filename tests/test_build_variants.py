"""Compile-only checks of the kernel configurations the default build leaves out.

gemm_mfma.hip keeps a second wave layout behind NOMAS_GEMM_WAVE_ROWS (4: eight
waves per block, two per SIMD, 64 token rows x 128 weight rows each; the
default is 2).  It is not what the library ships, but it must still build
for gfx950 with the same flags.
"""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HIPCC = "/opt/rocm/bin/hipcc"


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not installed")
def test_eight_wave_gemm_layout_compiles(tmp_path):
    src = os.path.join(ROOT, "hy-nomas-rs_amd", "csrc", "gemm_mfma.hip")
    out = tmp_path / "gemm_mfma_w4.o"
    cmd = [HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "-Wall", "-Werror=unused-variable",
           "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
           "-DNOMAS_GEMM_WAVE_ROWS=4", "-c", src, "-o", str(out)]
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stderr[-2000:]
    assert out.stat().st_size > 0
