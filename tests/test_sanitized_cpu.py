"""The oracle and the host build of the kernels' integer arithmetic under AddressSanitizer and
UndefinedBehaviorSanitizer: their CPU tests re-run in a child process against the sanitizer
builds (make -C oracle sanitize -> oracle/lib_san/, make -C uor-r4_amd/csrc sanitize ->
uor-r4_amd/lib_san/), with the shared sanitizer runtime preloaded. Any out-of-bounds access, use
after free, signed overflow, bad shift or misaligned access aborts the child and fails here.
"""

import glob
import os
import subprocess
import sys

import pytest

from conftest import ROOT

RUNTIME = sorted(glob.glob("/opt/rocm/llvm/lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so"))
# The oracle's own tests (golden vectors, mathematics, index, copy read, discrete scorer) and
# the host arithmetic's (tests/test_cabi_host.py).
SUBSET = ["tests/test_oracle_math.py", "tests/test_oracle_golden.py", "tests/test_cabi_host.py",
          "tests/test_index_oracle.py", "tests/test_copy_oracle.py", "tests/test_d11_oracle.py"]


@pytest.mark.skipif(not RUNTIME, reason="ROCm's clang sanitizer runtime is absent")
def test_oracle_and_host_arithmetic_under_asan_and_ubsan():
    for d in (os.path.join(ROOT, "oracle"), os.path.join(ROOT, "uor-r4_amd", "csrc")):
        subprocess.run(["make", "-C", d, "sanitize"], check=True, capture_output=True)
    preload = os.environ.get("LD_PRELOAD")
    env = dict(os.environ,
               LD_PRELOAD=RUNTIME[-1] + (":" + preload if preload else ""),
               ASAN_OPTIONS="detect_leaks=0:abort_on_error=1:verify_asan_link_order=0",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1",
               UOR_ORACLE_LIB_DIR=os.path.join(ROOT, "oracle", "lib_san"),
               UOR_HOSTPRIMS_LIB=os.path.join(ROOT, "uor-r4_amd", "lib_san",
                                              "libuor_fbs_hostprims.so"))
    r = subprocess.run([sys.executable, "-m", "pytest", "-x", "-q", "-m", "not gpu",
                        "-p", "no:cacheprovider", *SUBSET],
                       cwd=ROOT, env=env, capture_output=True, text=True, timeout=1200)
    tail = (r.stdout[-4000:] + "\n" + r.stderr[-4000:]).strip()
    assert r.returncode == 0, tail
    assert " passed" in r.stdout and "error" not in r.stdout.splitlines()[-1], tail
