"""The CPU suite again, against AddressSanitizer + UndefinedBehaviorSanitizer
builds of the host library and the oracle -- CPU only.

`make sanitize` builds libnomas_moe_san.so (the C ABI, safetensors reader,
generator and layer host code instrumented; the device code as usual) and
liboracle_san.so, both with ROCm's clang.  A child pytest loads them instead
of the normal builds, with clang's ASan runtime preloaded: any out-of-bounds
access, use after free or undefined behaviour (overflow, bad shift, misaligned
access ...) in the host code reached by the CPU tests aborts the child, and
this test fails with its report.  Leak detection is off (the interpreter and
torch hold memory until exit).
"""
import glob
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")


def _asan_runtime():
    hits = sorted(glob.glob(os.path.join(ROCM, "llvm/lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so")))
    return hits[-1] if hits else None


@pytest.mark.skipif(_asan_runtime() is None, reason="clang's ASan runtime is not installed")
def test_cpu_suite_under_asan_and_ubsan():
    pkg, orc = os.path.join(ROOT, "hy-nomas-rs_amd"), os.path.join(ROOT, "oracle")
    for d in (pkg, orc):
        subprocess.run(["make", "-s", "-j8", "-C", d, "sanitize"], check=True)
    env = dict(os.environ)
    env.update({
        "LD_PRELOAD": _asan_runtime(),
        "ASAN_OPTIONS": "detect_leaks=0:abort_on_error=1:detect_odr_violation=0",
        "UBSAN_OPTIONS": "print_stacktrace=1:halt_on_error=1",
        "NOMAS_MOE_LIB": os.path.join(pkg, "libnomas_moe_san.so"),
        "NOMAS_ORACLE_LIB": os.path.join(orc, "liboracle_san.so"),
        "CUDA_VISIBLE_DEVICES": "", "HIP_VISIBLE_DEVICES": "",  # host code only
    })
    # the child really loads the instrumented builds, under the ASan runtime
    probe = ("import ctypes, nomas_moe._lib as L, oracle as O; L.lib(); O.lib(); "
             "ctypes.CDLL(None).__asan_init; print(L.LIB_PATH); print(O._LIB_PATH)")
    r = subprocess.run([sys.executable, "-c", probe], env=dict(env, PYTHONPATH=os.pathsep.join(
        [pkg, orc, env.get("PYTHONPATH", "")])), cwd=ROOT, capture_output=True, text=True,
        timeout=300)
    assert r.returncode == 0, r.stderr[-3000:]
    assert r.stdout.split() == [env["NOMAS_MOE_LIB"], env["NOMAS_ORACLE_LIB"]], r.stdout
    cmd = [sys.executable, "-m", "pytest", "-q", "-x", "-m", "not gpu", "-p", "no:cacheprovider",
           "--ignore", os.path.join(ROOT, "tests", "test_sanitized.py"), os.path.join(ROOT, "tests")]
    r = subprocess.run(cmd, env=env, cwd=ROOT, capture_output=True, text=True, timeout=900)
    tail = (r.stdout + r.stderr)[-6000:]
    print(tail)
    assert r.returncode == 0, tail
    assert "ERROR: AddressSanitizer" not in tail and "runtime error" not in tail
