"""CPU checks of bench.py's own arithmetic and contract (no GPU): the algorithmic bytes per
token against the per-config figures the path's definition gives (c d input row + L (W d 4 +
d 4) window read and history write + c d per candidate row + 4), the counter-summary lookup
that feeds `roofline.traffic`, the config shapes, and the refusal of more than one GPU."""

import os
import subprocess
import sys
from dataclasses import replace

import pytest

from conftest import ROOT

sys.path.insert(0, ROOT)
import bench  # noqa: E402
from uor_fbs import synth  # noqa: E402


@pytest.mark.parametrize("config,candidates,expected", [
    ("c1", 512, 158_980),    # 4 probes x 128 rows (8,192 tokens over 64 drawers)
    ("c2", 512, 158_980),
    ("c3", 1024, 629_252),   # the uniform-drawer estimate: 8 probes x 128 rows
    ("c5", 1024, 930_308),   # int8 rows: one byte per channel
])
def test_algorithmic_bytes_per_token(config, candidates, expected):
    assert bench.algorithmic_bytes_per_token(synth.CONFIGS[config], candidates) == expected


def test_bytes_formula_terms():
    spec = replace(synth.CONFIGS["c3"], window=3, layers=1)
    d = spec.width
    # input row 2d, window 3 rows of 4-byte drives + one history row, no candidates, the token
    assert bench.algorithmic_bytes_per_token(spec, 0) == 2 * d + (3 * d * 4 + d * 4) + 4


def test_config_shapes_are_baselines():
    assert bench.CONFIG_SHAPES["c3"] == (1024, 1024, 1024)  # the metric's workload
    assert bench.CONFIG_SHAPES["c1"][0] == 1                 # the CPU-runnable latency case
    assert bench.CONFIG_SHAPES["c4"] == (1 << 20, 128, 0)    # rows x row length, scoring
    assert bench.CONFIG_SHAPES["c5"] == (16384, 4096, 4096)
    assert sorted(bench.CONFIG_SHAPES) == sorted(synth.CONFIGS)


class _Args:
    config, batch, prompt, gen, seed = "c3", 1024, 1024, 1024, 2026120203


def test_measured_traffic_matches_only_its_workload():
    a = _Args()
    t = bench.measured_traffic(a, "fbs_decode_pair<1, 8>")
    assert isinstance(t, int) and t > 10 ** 11  # the committed C3 summary's figure
    assert bench.measured_traffic(a, "fbs_decode<1, 8>") is None  # another kernel family
    b = _Args()
    b.batch = 512
    assert bench.measured_traffic(b, "fbs_decode_pair<1, 8>") is None  # another workload


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr and r.stdout == ""


def test_extra_configs_parse_to_their_workloads(monkeypatch):
    monkeypatch.setattr(sys, "argv", ["bench.py", "--config", "m1"])
    a = bench.parse()
    assert (a.batch, a.prompt) == (bench.D11_ROWS, 192) == (14287, 192)
    monkeypatch.setattr(sys, "argv", ["bench.py", "--config", "copy"])
    a = bench.parse()
    assert (a.batch, a.prompt) == (4096, 1024)


def test_d11_traffic_summary_has_its_figure():
    import re
    text = open(bench.D11_TRAFFIC_SUMMARY).read()
    m = re.search(r"traffic_bytes_per_launch:\s*(\d+)", text)
    assert m and int(m.group(1)) > 14287 * 656  # at least the records written
    assert bench.D11_PUBLISHED["value"] == 183206
