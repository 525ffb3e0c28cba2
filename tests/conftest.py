"""Shared test setup: import paths, the `gpu` marker, and the built libraries."""

import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (os.path.join(ROOT, "uor-r4_amd"), os.path.join(ROOT, "oracle"), ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")
    config.addinivalue_line("markers", "slow: a longer CPU test")


@pytest.fixture(params=["one-wave", "paired"])
def block_waves(request, monkeypatch):
    """Both kernel families: one wavefront per sequence, and paired blocks (two wavefronts per
    sequence, the library's default). The library reads UOR_FBS_BLOCK_WAVES when a model is
    created."""
    monkeypatch.setenv("UOR_FBS_BLOCK_WAVES", "1" if request.param == "one-wave" else "2")
    return request.param


@pytest.fixture(scope="session", autouse=True)
def _oracle_built():
    """The oracle is test infrastructure: build it if a fresh checkout lacks it."""
    libs = [os.path.join(ROOT, "oracle", "lib", n) for n in ("libfbs_oracle.so", "libd11_oracle.so", "libcopy_oracle.so")]
    if not all(os.path.exists(so) for so in libs):
        subprocess.run(["make", "-C", os.path.join(ROOT, "oracle")], check=True,
                       stdout=subprocess.DEVNULL)
