"""The kernels' reciprocal and reciprocal-square-root estimates (fbs_int.h rsqrt_q46, recip_q63),
checked over every input they take by tests/seed_bounds.cpp: the error bounds the exact
corrections downstream rely on, and equality with the same Newton steps in 64-bit products (the
32-bit forms the kernels use)."""

import os
import subprocess

from conftest import ROOT


def test_seed_estimates_over_every_input(tmp_path):
    exe = str(tmp_path / "seed_bounds")
    subprocess.run(["g++", "-O2", "-std=c++20", "-pthread", "-x", "c++", "-D__HIP_PLATFORM_AMD__",
                    "-I/opt/rocm/include", os.path.join(ROOT, "tests", "seed_bounds.cpp"), "-o", exe],
                   check=True, capture_output=True)
    r = subprocess.run([exe], capture_output=True, text=True, timeout=600)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
